// Anchored pair sums on gfx950, reference layout: the spatial-hash plan (device build), the pair forward and
// backward over that plan, window counts, the exposure correction and the log-score epilogue.
//
// Plan semantics follow atl/ops/functional.py:132-178 op for op in fp32 (compiled with -ffp-contract=off,
// IEEE division), so slice ranges, slice-centre positions, cell bins, keys and CSR offsets are bit-identical
// to the reference's CPU plan for the same geometry.  The pair tests follow csrc/atl_cpu.cpp:176-200 in the
// same fp32 order, so the set of visited pairs (and so n_i) is identical; the Gaussian uses v_exp_f32 with
// log2(e) folded into the scale (relative error ~|arg| * 2^-24 against expf).
#include "common.h"
#include "../../include/atl_hip.h"

#include <algorithm>
#include <cmath>

using namespace atlhip;

namespace {

// ------------------------------------------------------------------------------------------ statistics
// vmax = max ||v|| as sqrt(fma(vy, vy, vx * vx)) (torch's CPU vector-norm rounding), and the anchor bbox.
// stats (ordered ints): [0] vmax, [1] min x, [2] min y, [3] -max x, [4] -max y  (all reduced with min/max).
__global__ void k_stats_init(int* stats) {
  if (threadIdx.x == 0) {
    stats[0] = float_to_ordered(0.f);
    stats[1] = stats[2] = stats[3] = stats[4] = float_to_ordered(INFINITY);
  }
}

__global__ void __launch_bounds__(kBlock) k_stats(const float2* __restrict__ v, int64_t N,
                                                  const float2* __restrict__ xa, int64_t M, int* stats) {
  __shared__ int red[5][kBlock / kWave];
  int vm = float_to_ordered(0.f);
  int mnx = float_to_ordered(INFINITY), mny = mnx, nmx = mnx, nmy = mnx;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < N; j += stride) {
    const float2 q = v[j];
    vm = max(vm, float_to_ordered(sqrtf(fmaf(q.y, q.y, q.x * q.x))));
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < M; i += stride) {
    const float2 p = xa[i];
    mnx = min(mnx, float_to_ordered(p.x));
    mny = min(mny, float_to_ordered(p.y));
    nmx = min(nmx, float_to_ordered(-p.x));
    nmy = min(nmy, float_to_ordered(-p.y));
  }
  vm = wave_max_i(vm);
  mnx = wave_min_i(mnx);
  mny = wave_min_i(mny);
  nmx = wave_min_i(nmx);
  nmy = wave_min_i(nmy);
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  if (lane == 0) {
    red[0][wid] = vm; red[1][wid] = mnx; red[2][wid] = mny; red[3][wid] = nmx; red[4][wid] = nmy;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kBlock / kWave; ++w) {
      red[0][0] = max(red[0][0], red[0][w]);
      for (int s = 1; s < 5; ++s) red[s][0] = min(red[s][0], red[s][w]);
    }
    atomicMax(stats + 0, red[0][0]);
    for (int s = 1; s < 5; ++s) atomicMin(stats + s, red[s][0]);
  }
}

// ------------------------------------------------------------------------------------------ plan
struct PlanGeo {
  float ox, oy, cell;          // fp32 roundings of the double geometry
  float tau, half_delta, delta;
  int S, GH, GW;
  int64_t B;
};

// Slice range of a source, atl/ops/functional.py:151-152 (same fp32 order).
__device__ __forceinline__ void slice_range(float t, const PlanGeo& g, int& lo, int& hi) {
  const float a = (((t - g.tau) - g.half_delta) / g.delta) - 0.5f;
  const float c = (((t + g.tau) + g.half_delta) / g.delta) - 0.5f;
  const float flo = fminf(fmaxf(ceilf(a), 0.f), (float)(g.S - 1));
  const float fhi = fminf(fmaxf(floorf(c), 0.f), (float)(g.S - 1));
  lo = (int)flo;
  hi = (int)fhi;
}

// Slice centre (s + 0.5) * delta in fp32, functional.py:157.
__device__ __forceinline__ float slice_centre(int s, float delta) { return ((float)s + 0.5f) * delta; }

// Position of source (x, v, t) at slice centre cs and its cell; false if the cell is outside the grid
// (functional.py:158-162).
__device__ __forceinline__ bool source_cell(float2 x, float2 v, float t, float cs, const PlanGeo& g, float2& y,
                                            int& cx, int& cy) {
  const float dt = cs - t;
  y.x = x.x + v.x * dt;
  y.y = x.y + v.y * dt;
  const float fx = floorf((y.x - g.ox) / g.cell);
  const float fy = floorf((y.y - g.oy) / g.cell);
  if (!(fx >= 0.f && fx < (float)g.GW && fy >= 0.f && fy < (float)g.GH)) return false;
  cx = (int)fx;
  cy = (int)fy;
  return true;
}

__global__ void __launch_bounds__(kBlock) k_plan_count(const float2* __restrict__ x, const float* __restrict__ t,
                                                       const float2* __restrict__ v, const int64_t* __restrict__ b,
                                                       int64_t N, PlanGeo g, int* __restrict__ counts) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= N) return;
  const int64_t bj = b[j];
  if (bj < 0 || bj >= g.B) return;
  const float tj = t[j];
  const float2 xj = x[j], vj = v[j];
  int lo, hi;
  slice_range(tj, g, lo, hi);
  for (int s = lo; s <= hi; ++s) {
    float2 y;
    int cx, cy;
    if (!source_cell(xj, vj, tj, slice_centre(s, g.delta), g, y, cx, cy)) continue;
    const int64_t key = ((bj * g.S + s) * g.GH + cy) * (int64_t)g.GW + cx;
    atomicAdd(counts + key, 1);
  }
}

__global__ void __launch_bounds__(kBlock) k_plan_fill(const float2* __restrict__ x, const float* __restrict__ t,
                                                      const float2* __restrict__ v, const int64_t* __restrict__ b,
                                                      int64_t N, PlanGeo g, const int64_t* __restrict__ start,
                                                      int* __restrict__ cursor, float2* __restrict__ src_y,
                                                      float2* __restrict__ src_v, float* __restrict__ src_t,
                                                      int64_t* __restrict__ src_id) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= N) return;
  const int64_t bj = b[j];
  if (bj < 0 || bj >= g.B) return;
  const float tj = t[j];
  const float2 xj = x[j], vj = v[j];
  int lo, hi;
  slice_range(tj, g, lo, hi);
  for (int s = lo; s <= hi; ++s) {
    float2 y;
    int cx, cy;
    if (!source_cell(xj, vj, tj, slice_centre(s, g.delta), g, y, cx, cy)) continue;
    const int64_t key = ((bj * g.S + s) * g.GH + cy) * (int64_t)g.GW + cx;
    const int64_t at = start[key] + atomicAdd(cursor + key, 1);
    src_y[at] = y;
    src_v[at] = vj;
    src_t[at] = tj;
    src_id[at] = j;
  }
}

// Anchors: slice floor(t / delta), cells clamped into the grid, functional.py:170-175.
__global__ void __launch_bounds__(kBlock) k_plan_anchors(const float2* __restrict__ x, const float* __restrict__ t,
                                                         const int64_t* __restrict__ b,
                                                         const int64_t* __restrict__ anchors,
                                                         const float2* __restrict__ anchor_xy, int64_t M, int64_t N,
                                                         PlanGeo g, float2* __restrict__ anc_x,
                                                         float* __restrict__ anc_t, int64_t* __restrict__ anc_cell,
                                                         int64_t* __restrict__ anc_id) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  int64_t a = anchors[i];
  const bool valid = a >= 0 && a < N;
  if (!valid) a = 0;
  const float ta = t[a];
  const float2 xa = anchor_xy ? anchor_xy[i] : x[a];
  const float fs = fminf(fmaxf(floorf(ta / g.delta), 0.f), (float)(g.S - 1));
  const float fx = fminf(fmaxf(floorf((xa.x - g.ox) / g.cell), 0.f), (float)(g.GW - 1));
  const float fy = fminf(fmaxf(floorf((xa.y - g.oy) / g.cell), 0.f), (float)(g.GH - 1));
  anc_x[i] = xa;
  anc_t[i] = ta;
  anc_cell[3 * i + 0] = valid ? b[a] * g.S + (int64_t)fs : -1;
  anc_cell[3 * i + 1] = (int64_t)fx;
  anc_cell[3 * i + 2] = (int64_t)fy;
  anc_id[i] = valid ? a : -1;
}

// ------------------------------------------------------------------------------------------ scan
constexpr int kScanItems = 8;
constexpr int kScanTile = kBlock * kScanItems;

__global__ void __launch_bounds__(kBlock) k_scan_reduce(const int* __restrict__ in, int64_t n,
                                                        int64_t* __restrict__ part) {
  __shared__ int lds[kBlock / kWave + 1];
  const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
  int s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k)
    if (base + k < n) s += in[base + k];
  int total;
  block_exclusive_scan<kBlock>(s, lds, total);
  if (threadIdx.x == 0) part[blockIdx.x] = total;
}

// Exclusive scan of the per-tile totals, in place (one block).
__global__ void __launch_bounds__(kBlock) k_scan_parts(int64_t* __restrict__ part, int64_t nparts) {
  __shared__ int64_t lds[kBlock];
  int64_t carry = 0;
  for (int64_t base = 0; base < nparts; base += kBlock) {
    const int64_t i = base + threadIdx.x;
    const int64_t v = i < nparts ? part[i] : 0;
    lds[threadIdx.x] = v;
    __syncthreads();
    for (int d = 1; d < kBlock; d <<= 1) {
      const int64_t y = threadIdx.x >= (unsigned)d ? lds[threadIdx.x - d] : 0;
      __syncthreads();
      lds[threadIdx.x] += y;
      __syncthreads();
    }
    if (i < nparts) part[i] = carry + lds[threadIdx.x] - v;
    carry += lds[kBlock - 1];
    __syncthreads();
  }
}

template <typename T>
__global__ void __launch_bounds__(kBlock) k_scan_write(const int* __restrict__ in, int64_t n,
                                                       const int64_t* __restrict__ part, T* __restrict__ out) {
  __shared__ int lds[kBlock / kWave + 1];
  const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
  int vals[kScanItems];
  int s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    vals[k] = base + k < n ? in[base + k] : 0;
    s += vals[k];
  }
  int total;
  const int excl = block_exclusive_scan<kBlock>(s, lds, total);
  int64_t run = part[blockIdx.x] + excl;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    run += vals[k];
    if (base + k < n) out[base + k + 1] = (T)run;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) out[0] = 0;
}

__global__ void k_fill_i32(int* __restrict__ p, int64_t n, int v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

// ------------------------------------------------------------------------------------------ pair walk
struct PairRef {
  const float2 *SY, *SV, *AX;
  const float *ST, *AT, *SC;
  const int64_t *SID, *CS, *AC, *AID;
  int64_t S, GH, GW, G, E, N;
  float tau, r2max, kexp;      // kexp = -log2(e) / (2 h^2): exp(-d2 / 2h^2) = exp2(d2 * kexp)
};

__device__ __forceinline__ float gauss(float d2, float kexp) { return __builtin_amdgcn_exp2f(d2 * kexp); }

// Visits the contributing pairs of anchor i over its 3x3 cell neighbourhood; the three cells of a row are
// consecutive keys, so each row is one contiguous CSR range (csrc/atl_cpu.cpp:176-200).
template <typename Visit>
__device__ __forceinline__ void walk_ref(int64_t i, const PairRef& a, Visit&& visit) {
  const int64_t g = a.AC[3 * i], cx = a.AC[3 * i + 1], cy = a.AC[3 * i + 2], id = a.AID[i];
  if (g < 0 || g >= a.G || cx < 0 || cx >= a.GW || cy < 0 || cy >= a.GH) return;
  const float2 xi = a.AX[i];
  const float ti = a.AT[i];
  const float cs = a.SC[g % a.S];
  const float at = ti - cs;
  const int64_t ylo = cy > 0 ? cy - 1 : 0, yhi = cy + 1 < a.GH ? cy + 1 : a.GH - 1;
  const int64_t xlo = cx > 0 ? cx - 1 : 0, xhi = cx + 1 < a.GW ? cx + 1 : a.GW - 1;
  for (int64_t yy = ylo; yy <= yhi; ++yy) {
    const int64_t row = (g * a.GH + yy) * a.GW;
    int64_t k = a.CS[row + xlo];
    int64_t k1 = a.CS[row + xhi + 1];
    k = k < 0 ? 0 : k;
    k1 = k1 > a.E ? a.E : k1;
    for (; k < k1; ++k) {
      if (a.SID[k] == id) continue;
      const float dt = ti - a.ST[k];
      if (fabsf(dt) > a.tau) continue;
      const float2 sy = a.SY[k], sv = a.SV[k];
      const float rx = xi.x - (sy.x + sv.x * at);
      const float ry = xi.y - (sy.y + sv.y * at);
      const float d2 = rx * rx + ry * ry;
      if (d2 > a.r2max) continue;
      visit(k, rx, ry, dt, gauss(d2, a.kexp));
    }
  }
}

__global__ void __launch_bounds__(kBlock) k_pair_fwd_ref(PairRef a, int64_t M, float* __restrict__ out,
                                                         int* __restrict__ count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  double acc = 0.0;
  int n = 0;
  walk_ref(i, a, [&](int64_t, float, float, float, float k) {
    acc += (double)k;
    ++n;
  });
  out[i] = (float)acc;
  if (count) count[i] = n;
}

__global__ void __launch_bounds__(kBlock) k_pair_bwd_ref(PairRef a, int64_t M, const float* __restrict__ gS,
                                                         float invh2, float* __restrict__ gv) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  const float gi = gS[i];
  if (gi == 0.f) return;
  walk_ref(i, a, [&](int64_t k, float rx, float ry, float dt, float kern) {
    const float f = gi * kern * dt * invh2;
    const int64_t j = a.SID[k];
    if (j < 0 || j >= a.N) return;
    atomicAdd(gv + 2 * j, f * rx);
    atomicAdd(gv + 2 * j + 1, f * ry);
  });
}

// ------------------------------------------------------------------------------------------ window counts
// #{j != i, same batch, |t_j - t_i| <= tau} over float64 keys b*4 + t that are ascending in event order
// (EventPacket invariant); lower/upper bounds by binary search, atl/ops/functional.py:210-217.
__device__ __forceinline__ double bt_key(const float* t, const int64_t* b, int64_t j) {
  return (double)b[j] * 4.0 + (double)t[j];
}

__global__ void __launch_bounds__(kBlock) k_window_counts(const float* __restrict__ t,
                                                          const int64_t* __restrict__ b, int64_t N,
                                                          const int64_t* __restrict__ idx, int64_t M, double tau,
                                                          float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  const int64_t a = idx ? idx[i] : i;            // no index array: every event in order
  if (a < 0 || a >= N) { out[i] = 0.f; return; }
  const double ki = bt_key(t, b, a);
  const double lo_v = ki - tau, hi_v = ki + tau;
  int64_t lo = 0, hi = N;                      // first index with key >= lo_v
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (bt_key(t, b, mid) < lo_v) lo = mid + 1; else hi = mid;
  }
  const int64_t first = lo;
  lo = first;
  hi = N;                                      // first index with key > hi_v
  while (lo < hi) {
    const int64_t mid = (lo + hi) >> 1;
    if (bt_key(t, b, mid) <= hi_v) lo = mid + 1; else hi = mid;
  }
  const int64_t c = lo - first - 1;
  out[i] = (float)(c > 0 ? c : 0);
}

// Every event as anchor, in order (idx = null): a block's 1024 consecutive anchors have ascending keys, so their
// bounds lie between those of its first and last anchor.  Four waves find those four bounds with 64-way searches
// (one ballot per round, four rounds for 16M events) instead of 20 dependent probes per thread; the two key
// ranges between them are then read into LDS and every thread searches there.  Ranges wider than kWcCap keys
// fall back to the per-thread search.
constexpr int kWcCap = 2048;
constexpr int kWcPer = 4;                          // anchors per thread: a block covers 1024 consecutive anchors

__device__ __forceinline__ int64_t bound_64way(const float* t, const int64_t* b, int64_t N, double v, bool upper) {
  const int lane = threadIdx.x & 63;
  int64_t lo = 0, hi = N;                          // smallest x in [lo, hi] with x == N or key(x) >= v (> v)
  while (lo < hi) {                                // wave-uniform
    const int64_t span = hi - lo;
    const int64_t p = lo + (span * (lane + 1)) / 64;                      // p in (lo, hi], p_63 = hi
    bool pred = true;
    if (p < N) {
      const double k = bt_key(t, b, p);
      pred = upper ? k > v : k >= v;
    }
    if (lane == 63) pred = true;                   // hi itself satisfies the predicate
    const uint64_t m = __ballot(pred);
    const int f = __ffsll((unsigned long long)m) - 1;                    // first probe that satisfies it
    const int64_t pf = lo + (span * (f + 1)) / 64;
    const int64_t pprev = f == 0 ? lo - 1 : lo + (span * f) / 64;
    // the answer lies in (pprev, pf]: pf satisfies, pprev (if any) does not; lo itself is still unprobed
    if (f == 0) {
      if (lo < N && (upper ? bt_key(t, b, lo) > v : bt_key(t, b, lo) >= v)) return lo;
      lo = lo + 1;
      hi = pf;
    } else {
      lo = pprev + 1;
      hi = pf;
    }
  }
  return lo;
}

__global__ void __launch_bounds__(kBlock) k_window_counts_seq(const float* __restrict__ t,
                                                              const int64_t* __restrict__ b, int64_t N, int64_t M,
                                                              double tau, float* __restrict__ out) {
  __shared__ double A[kWcCap], Bk[kWcCap];
  __shared__ int64_t bound[4];
  const int64_t a0 = (int64_t)blockIdx.x * kBlock * kWcPer;
  const int64_t a1 = min(a0 + kBlock * kWcPer, M) - 1;
  const int g = threadIdx.x >> 6;
  {
    const int64_t ag = (g & 1) ? a1 : a0;
    const double kg = bt_key(t, b, ag);
    const int64_t r = bound_64way(t, b, N, g < 2 ? kg - tau : kg + tau, g >= 2);
    if ((threadIdx.x & 63) == 0) bound[g] = r;
  }
  __syncthreads();
  const int64_t lof = bound[0], lol = bound[1], hif = bound[2], hil = bound[3];
  const int64_t nA = min(lol, N - 1) - lof + 1, nB = min(hil, N - 1) - hif + 1;
  const bool fits = nA <= kWcCap && nB <= kWcCap;
  if (fits) {
    for (int64_t i = threadIdx.x; i < nA; i += kBlock) A[i] = bt_key(t, b, lof + i);
    for (int64_t i = threadIdx.x; i < nB; i += kBlock) Bk[i] = bt_key(t, b, hif + i);
  }
  __syncthreads();
  for (int u = 0; u < kWcPer; ++u) {
    const int64_t a = a0 + u * kBlock + threadIdx.x;
    if (a > a1) return;
    const double ki = bt_key(t, b, a);
    const double lo_v = ki - tau, hi_v = ki + tau;
    int64_t first, last;
    if (fits) {
      int lo = 0, hi = (int)max(nA, (int64_t)0);
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (A[mid] < lo_v) lo = mid + 1; else hi = mid;
      }
      first = lof + lo;
      lo = 0;
      hi = (int)max(nB, (int64_t)0);
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (Bk[mid] <= hi_v) lo = mid + 1; else hi = mid;
      }
      last = hif + lo;
    } else {
      int64_t lo = 0, hi = N;
      while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (bt_key(t, b, mid) < lo_v) lo = mid + 1; else hi = mid;
      }
      first = lo;
      lo = first;
      hi = N;
      while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (bt_key(t, b, mid) <= hi_v) lo = mid + 1; else hi = mid;
      }
      last = lo;
    }
    const int64_t c = last - first - 1;
    out[a] = (float)(c > 0 ? c : 0);
  }
}

__global__ void __launch_bounds__(kBlock) k_check_sorted(const float* __restrict__ t, const int64_t* __restrict__ b,
                                                         int64_t N, int* __restrict__ flag) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j + 1 >= N) return;
  if (bt_key(t, b, j) > bt_key(t, b, j + 1)) atomicOr(flag, 1);
}

// ------------------------------------------------------------------------------------------ exposure
// Per-batch event counts in n_check time bins, atl/objectives/ats.py:39-41 (LDS histogram per block).
constexpr int kBinPer = 16;                        // events per thread (loads issued together)

// Time bin of the exposure check: clamp(trunc(fp32(t * n_check)), 0, n_check - 1) (atl/objectives/ats.py:39).
__device__ __forceinline__ int time_bin(float t, int n_check) {
  const float q = t * (float)n_check;
  int s = (q > -1.f && q < 2147483520.f) ? (int)q : (q >= 2147483520.f ? n_check - 1 : 0);
  return min(max(s, 0), n_check - 1);
}

__global__ void __launch_bounds__(kBlock) k_bin_counts(const float* __restrict__ t, const int64_t* __restrict__ b,
                                                       int64_t N, int64_t B, int n_check, float* __restrict__ counts) {
  extern __shared__ int hist[];
  const int nb = (int)B * n_check;
  for (int k = threadIdx.x; k < nb; k += blockDim.x) hist[k] = 0;
  __syncthreads();
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int lane = threadIdx.x & 63;
  for (int64_t j0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j0 < N; j0 += stride * kBinPer) {
    int64_t bq[kBinPer];
    float tq[kBinPer];
#pragma unroll
    for (int u = 0; u < kBinPer; ++u) {            // all loads of the thread in flight together
      const int64_t j = j0 + u * stride;
      bq[u] = j < N ? b[j] : -1;
      tq[u] = j < N ? t[j] : 0.f;
    }
#pragma unroll
    for (int u = 0; u < kBinPer; ++u) {
      const int64_t bj = bq[u];
      int key = -1;
      if (bj >= 0 && bj < B) key = (int)bj * n_check + time_bin(tq[u], n_check);
      // lanes with equal bins add once: time-ordered events put a whole wave in one or two bins, and 64 LDS
      // atomics on one address would run one after the other
      uint64_t todo = __ballot(1);
      while (todo) {
        const int leader = __ffsll((unsigned long long)todo) - 1;
        const int kl = __shfl(key, leader);
        const uint64_t same = __ballot(key == kl) & todo;
        if (lane == leader && kl >= 0) atomicAdd(hist + kl, __popcll(same));
        todo &= ~same;
      }
    }
  }
  __syncthreads();
  for (int k = threadIdx.x; k < nb; k += blockDim.x)
    if (hist[k]) atomicAdd(counts + k, (float)hist[k]);
}

// The same counts for events sorted by (b, t): the bin of an event does not decrease along a batch, so count k of
// batch b is the distance between the first events of bins k and k + 1.  Wave (b, k) finds both with 64-way
// searches (one ballot per round: four rounds for 16M events) and writes counts[b][k]: no atomics, no fill.
template <typename Pred>
__device__ __forceinline__ int64_t first_true_64way(int64_t lo, int64_t hi, Pred&& pred) {
  const int lane = threadIdx.x & 63;
  while (lo < hi) {                                // wave-uniform; pred monotone (false ... true) on [lo, hi)
    const int64_t span = hi - lo;
    const int64_t q = lo + (span * lane) / 64;     // q_0 = lo, strictly below hi
    const bool pr = (lane == 0 || q != lo + (span * (lane - 1)) / 64) ? pred(q) : false;
    const uint64_t m = __ballot(pr);
    if (m == 0) {                                  // every probe false: the answer lies past the last probe
      lo = lo + (span * 63) / 64 + 1;
      continue;
    }
    const int f = __ffsll((unsigned long long)m) - 1;
    const int64_t qf = lo + (span * f) / 64;
    if (f == 0) return qf;
    lo = lo + (span * (f - 1)) / 64 + 1;
    hi = qf;
  }
  return lo;
}

__global__ void __launch_bounds__(kWave) k_bin_counts_sorted(const float* __restrict__ t,
                                                             const int64_t* __restrict__ b, int64_t N, int n_check,
                                                             float* __restrict__ counts) {
  const int64_t bb = blockIdx.x;
  const int k = blockIdx.y;
  const int64_t s0 = first_true_64way(0, N, [&](int64_t i) { return b[i] >= bb; });
  const int64_t s1 = first_true_64way(s0, N, [&](int64_t i) { return b[i] >= bb + 1; });
  auto edge = [&](int e) -> int64_t {              // first event of the batch with bin >= e
    if (e <= 0) return s0;
    if (e >= n_check) return s1;
    return first_true_64way(s0, s1, [&](int64_t i) { return time_bin(t[i], n_check) >= e; });
  };
  const int64_t e0 = edge(k), e1 = edge(k + 1);
  if (threadIdx.x == 0) counts[bb * n_check + k] = (float)(e1 - e0);
}

// Exposure correction for linear motion (atl/objectives/ats.py:42-50): anchors transported to each bin centre
// with their own velocity, inside test, weighted by count * [|t_a - c| <= tau].
__global__ void __launch_bounds__(kBlock) k_visible(const float2* __restrict__ xa, const float2* __restrict__ va,
                                                    const float* __restrict__ ta, const int64_t* __restrict__ ba,
                                                    int64_t M, const float* __restrict__ counts,
                                                    const float* __restrict__ centres, int64_t B, int n_check,
                                                    float tau, float wmax, float hmax, float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  const int64_t bi = ba[i];
  const float2 x = xa[i], v = va[i];
  const float t = ta[i];
  float vis = 0.f, tot = 0.f;
  if (bi >= 0 && bi < B) {
    const float* cnt = counts + bi * n_check;
    for (int k = 0; k < n_check; ++k) {
      const float c = centres[k];
      const float near = fabsf(t - c) <= tau ? 1.f : 0.f;
      const float dt = c - t;
      const float yx = x.x + v.x * dt, yy = x.y + v.y * dt;
      const float inside = (yx >= 0.f && yx <= wmax && yy >= 0.f && yy <= hmax) ? 1.f : 0.f;
      const float w = cnt[k] * near;
      vis = vis + w * inside;
      tot = tot + w;
    }
  }
  out[i] = fmaxf(vis / fmaxf(tot, 1.f), 1e-3f);
}

// ------------------------------------------------------------------------------------------ epilogue
// log(eps + S / (Wn * 2 * pi * h^2)) with Wn = max(count, 1) * vis (atl/objectives/ats.py:92-96); saves q and D
// for the backward gS = (g / q) / D.
__global__ void __launch_bounds__(kBlock) k_epilogue_fwd(const float* __restrict__ S, const float* __restrict__ wc,
                                                         const float* __restrict__ vis, int64_t M, float pi_f,
                                                         float hh, float eps, float* __restrict__ ls,
                                                         float* __restrict__ q, float* __restrict__ D) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  float wn = fmaxf(wc[i], 1.f);
  if (vis) wn = wn * vis[i];
  const float d = ((wn * 2.f) * pi_f) * hh;
  const float qq = eps + S[i] / d;
  ls[i] = logf(qq);
  q[i] = qq;
  D[i] = d;
}

// The same epilogue fused with the loss: out = (-mean_i ls_i, mean_i ls_i) (atl/objectives/ats.py:102-105), q and D
// saved.  The mean is deterministic: each block adds its terms in double and stores the partial in part[block];
// a second one-block launch adds the partials in block order (a launch boundary orders the two; a ticket in
// one launch would need a device-scope fence per block, which writes back the whole L2 of its XCD).
constexpr int kMeanBlocks = 1024;

__device__ __forceinline__ double block_sum_d(double v, double* red) {
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_down(v, o);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double tot = 0.0;
  if (threadIdx.x == 0)
    for (int w = 0; w < kBlock / 64; ++w) tot += red[w];
  __syncthreads();
  return tot;                                    // valid in thread 0
}

__global__ void __launch_bounds__(kBlock) k_epilogue_mean(const float* __restrict__ S, const float* __restrict__ wc,
                                                          const float* __restrict__ vis, int64_t M, float pi_f,
                                                          float hh, float eps, float* __restrict__ q,
                                                          float* __restrict__ D, double* __restrict__ part) {
  __shared__ double red[kBlock / 64];
  double acc = 0.0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < M; i += stride) {
    float wn = fmaxf(wc[i], 1.f);
    if (vis) wn = wn * vis[i];
    const float d = ((wn * 2.f) * pi_f) * hh;
    const float qq = eps + S[i] / d;
    acc += (double)logf(qq);
    q[i] = qq;
    D[i] = d;
  }
  const double bs = block_sum_d(acc, red);
  if (threadIdx.x == 0) part[blockIdx.x] = bs;
}

__global__ void __launch_bounds__(kBlock) k_epilogue_mean_total(const double* __restrict__ part, int nparts,
                                                                int64_t M, float* __restrict__ out) {
  __shared__ double red[kBlock / 64];
  double t = 0.0;                                // thread k adds partials k, k + 256, ... in order
  for (int k = threadIdx.x; k < nparts; k += kBlock) t += part[k];
  const double tot = block_sum_d(t, red);
  if (threadIdx.x == 0) {
    const float mean = (float)(tot / (double)M);
    out[0] = -mean;
    out[1] = mean;
  }
}

// Backward of the fused loss: d loss / d ls_i = (-g) / M (the gradients of the negation and of the mean), then
// gS = (that / q) / D.
__global__ void __launch_bounds__(kBlock) k_epilogue_mean_bwd(const float* __restrict__ g, const float* __restrict__ q,
                                                              const float* __restrict__ D, int64_t M,
                                                              float* __restrict__ gS) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  const float gl = (-g[0]) / (float)M;
  gS[i] = (gl / q[i]) / D[i];
}

__global__ void __launch_bounds__(kBlock) k_epilogue_bwd(const float* __restrict__ g, const float* __restrict__ q,
                                                         const float* __restrict__ D, int64_t M,
                                                         float* __restrict__ gS) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  gS[i] = (g[i] / q[i]) / D[i];
}

PlanGeo make_geo(double ox, double oy, double cell, double tau, int64_t S, int64_t GH, int64_t GW, int64_t B) {
  PlanGeo g;
  g.ox = (float)ox;
  g.oy = (float)oy;
  g.cell = (float)cell;
  g.tau = (float)tau;
  const double delta = 1.0 / (double)S;
  g.half_delta = (float)(delta / 2);
  g.delta = (float)delta;
  g.S = (int)S;
  g.GH = (int)GH;
  g.GW = (int)GW;
  g.B = B;
  return g;
}

bool geo_ok(int64_t S, int64_t GH, int64_t GW, int64_t B) {
  return S >= 1 && S <= 65536 && GH >= 1 && GW >= 1 && B >= 0 && GH < (1 << 28) && GW < (1 << 28) &&
         (double)B * S * GH * GW < 2.0e9;
}

PairRef make_ref(const float* src_y, const float* src_v, const float* src_t, const int64_t* src_id,
                 const int64_t* cell_start, int64_t E, int64_t ncell, const float* anc_x, const float* anc_t,
                 const int64_t* anc_cell, const int64_t* anc_id, const float* slice_c, int64_t S, int64_t GH,
                 int64_t GW, double h, double tau, double cut, int64_t N) {
  PairRef a;
  a.SY = (const float2*)src_y; a.SV = (const float2*)src_v; a.ST = src_t; a.SID = src_id; a.CS = cell_start;
  a.AX = (const float2*)anc_x; a.AT = anc_t; a.AC = anc_cell; a.AID = anc_id; a.SC = slice_c;
  a.S = S; a.GH = GH; a.GW = GW; a.G = ncell / (GH * GW); a.E = E; a.N = N;
  const float hf = (float)h, cf = (float)cut;
  a.tau = (float)tau;
  a.r2max = cf * cf * hf * hf;
  const float inv2h2 = 1.f / (2.f * hf * hf);
  a.kexp = (float)(-(double)inv2h2 * 1.4426950408889634);
  return a;
}

}  // namespace

// ================================================================================================ C-ABI
extern "C" {

int atl_plan_stats(const float* v, int64_t N, const float* xa, int64_t M, int* stats, hipStream_t stream) {
  if (N < 0 || M < 0 || !stats) { set_error("plan_stats: bad arguments"); return 1; }
  hipLaunchKernelGGL(k_stats_init, dim3(1), dim3(64), 0, stream, stats);
  const int64_t n = N > M ? N : M;
  if (n > 0) {
    unsigned grid = grid_for(n);
    if (grid > 2048) grid = 2048;
    hipLaunchKernelGGL(k_stats, dim3(grid), dim3(kBlock), 0, stream, (const float2*)v, N, (const float2*)xa, M,
                       stats);
  }
  return check_launch("plan_stats");
}

int atl_plan_count(const float* x, const float* t, const float* v, const int64_t* b, int64_t N, int64_t B,
                   double ox, double oy, double cell, double tau, int64_t S, int64_t GH, int64_t GW, int* counts,
                   hipStream_t stream) {
  if (N < 0 || !geo_ok(S, GH, GW, B) || !(cell > 0)) { set_error("plan_count: bad geometry S=%lld GH=%lld GW=%lld", (long long)S, (long long)GH, (long long)GW); return 1; }
  if (N == 0 || B == 0) return 0;
  const PlanGeo g = make_geo(ox, oy, cell, tau, S, GH, GW, B);
  hipLaunchKernelGGL(k_plan_count, dim3(grid_for(N)), dim3(kBlock), 0, stream, (const float2*)x, t,
                     (const float2*)v, b, N, g, counts);
  return check_launch("plan_count");
}

int atl_scan_counts(const int* counts, int64_t n, int64_t* start, int64_t* work, hipStream_t stream) {
  if (n < 0) { set_error("scan_counts: bad size"); return 1; }
  const int64_t tiles = (n + kScanTile - 1) / kScanTile;
  if (tiles == 0) {
    hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(64), 0, stream, (int*)start, 2, 0);
    return check_launch("scan_counts");
  }
  hipLaunchKernelGGL(k_scan_reduce, dim3((unsigned)tiles), dim3(kBlock), 0, stream, counts, n, work);
  hipLaunchKernelGGL(k_scan_parts, dim3(1), dim3(kBlock), 0, stream, work, tiles);
  hipLaunchKernelGGL(k_scan_write<int64_t>, dim3((unsigned)tiles), dim3(kBlock), 0, stream, counts, n,
                     (const int64_t*)work, start);
  return check_launch("scan_counts");
}

int64_t atl_scan_work_size(int64_t n) { return (n + kScanTile - 1) / kScanTile + 1; }

int atl_fill_i32(int* p, int64_t n, int value, hipStream_t stream) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(n)), dim3(kBlock), 0, stream, p, n, value);
  return check_launch("fill_i32");
}

int atl_plan_fill(const float* x, const float* t, const float* v, const int64_t* b, int64_t N, int64_t B,
                  double ox, double oy, double cell, double tau, int64_t S, int64_t GH, int64_t GW,
                  const int64_t* start, int* cursor, float* src_y, float* src_v, float* src_t, int64_t* src_id,
                  hipStream_t stream) {
  if (N < 0 || !geo_ok(S, GH, GW, B) || !(cell > 0)) { set_error("plan_fill: bad geometry"); return 1; }
  if (N == 0 || B == 0) return 0;
  const PlanGeo g = make_geo(ox, oy, cell, tau, S, GH, GW, B);
  hipLaunchKernelGGL(k_plan_fill, dim3(grid_for(N)), dim3(kBlock), 0, stream, (const float2*)x, t,
                     (const float2*)v, b, N, g, start, cursor, (float2*)src_y, (float2*)src_v, src_t, src_id);
  return check_launch("plan_fill");
}

int atl_plan_anchors(const float* x, const float* t, const int64_t* b, const int64_t* anchors,
                     const float* anchor_xy, int64_t M, int64_t N, double ox, double oy, double cell, int64_t S,
                     int64_t GH, int64_t GW, float* anc_x, float* anc_t, int64_t* anc_cell, int64_t* anc_id,
                     hipStream_t stream) {
  if (M < 0 || N < 0 || !geo_ok(S, GH, GW, 1) || !(cell > 0)) { set_error("plan_anchors: bad geometry"); return 1; }
  if (M == 0) return 0;
  if (N == 0) { set_error("plan_anchors: anchors given but no events"); return 1; }
  const PlanGeo g = make_geo(ox, oy, cell, 0.0, S, GH, GW, 1);
  hipLaunchKernelGGL(k_plan_anchors, dim3(grid_for(M)), dim3(kBlock), 0, stream, (const float2*)x, t, b, anchors,
                     (const float2*)anchor_xy, M, N, g, (float2*)anc_x, anc_t, anc_cell, anc_id);
  return check_launch("plan_anchors");
}

int atl_ats_pair_fwd(const float* src_y, const float* src_v, const float* src_t, const int64_t* src_id,
                     const int64_t* cell_start, int64_t E, int64_t ncell, const float* anc_x, const float* anc_t,
                     const int64_t* anc_cell, const int64_t* anc_id, int64_t M, const float* slice_c, int64_t S,
                     int64_t GH, int64_t GW, double h, double tau, double cut, float* out, int* count,
                     hipStream_t stream) {
  if (M < 0 || E < 0 || S < 1 || GH < 1 || GW < 1 || ncell < 0 || ncell % (GH * GW) != 0 || !(h > 0)) {
    set_error("ats_pair_fwd: bad arguments (S=%lld GH=%lld GW=%lld ncell=%lld h=%g)", (long long)S, (long long)GH, (long long)GW, (long long)ncell, h);
    return 1;
  }
  if (M == 0) return 0;
  const PairRef a = make_ref(src_y, src_v, src_t, src_id, cell_start, E, ncell, anc_x, anc_t, anc_cell, anc_id,
                             slice_c, S, GH, GW, h, tau, cut, 0);
  hipLaunchKernelGGL(k_pair_fwd_ref, dim3(grid_for(M)), dim3(kBlock), 0, stream, a, M, out, count);
  return check_launch("ats_pair_fwd");
}

int atl_ats_pair_bwd(const float* gS, const float* src_y, const float* src_v, const float* src_t,
                     const int64_t* src_id, const int64_t* cell_start, int64_t E, int64_t ncell, const float* anc_x,
                     const float* anc_t, const int64_t* anc_cell, const int64_t* anc_id, int64_t M,
                     const float* slice_c, int64_t S, int64_t GH, int64_t GW, double h, double tau, double cut,
                     int64_t N, float* gv, hipStream_t stream) {
  if (M < 0 || E < 0 || N < 0 || S < 1 || GH < 1 || GW < 1 || ncell < 0 || ncell % (GH * GW) != 0 || !(h > 0)) {
    set_error("ats_pair_bwd: bad arguments");
    return 1;
  }
  if (M == 0 || N == 0) return 0;
  const PairRef a = make_ref(src_y, src_v, src_t, src_id, cell_start, E, ncell, anc_x, anc_t, anc_cell, anc_id,
                             slice_c, S, GH, GW, h, tau, cut, N);
  const float invh2 = 1.f / (float)(h * h);
  hipLaunchKernelGGL(k_pair_bwd_ref, dim3(grid_for(M)), dim3(kBlock), 0, stream, a, M, gS, invh2, gv);
  return check_launch("ats_pair_bwd");
}

int atl_window_counts(const float* t, const int64_t* b, int64_t N, const int64_t* idx, int64_t M, double tau,
                      float* out, hipStream_t stream) {
  if (N < 0 || M < 0 || (!idx && M > N)) { set_error("window_counts: bad sizes"); return 1; }
  if (M == 0) return 0;
  if (!idx)
    hipLaunchKernelGGL(k_window_counts_seq, dim3(grid_for(M, kBlock * kWcPer)), dim3(kBlock), 0, stream, t, b, N,
                       M, tau, out);
  else
    hipLaunchKernelGGL(k_window_counts, dim3(grid_for(M)), dim3(kBlock), 0, stream, t, b, N, idx, M, tau, out);
  return check_launch("window_counts");
}

int atl_check_sorted(const float* t, const int64_t* b, int64_t N, int* flag, hipStream_t stream) {
  if (N < 0 || !flag) { set_error("check_sorted: bad arguments"); return 1; }
  hipLaunchKernelGGL(k_fill_i32, dim3(1), dim3(64), 0, stream, flag, 1, 0);
  if (N > 1)
    hipLaunchKernelGGL(k_check_sorted, dim3(grid_for(N)), dim3(kBlock), 0, stream, t, b, N, flag);
  return check_launch("check_sorted");
}

int atl_bin_counts(const float* t, const int64_t* b, int64_t N, int64_t B, int64_t n_check, float* counts,
                   hipStream_t stream) {
  if (N < 0 || B < 0 || n_check < 1 || B * n_check > 8192) { set_error("bin_counts: bad sizes (B*n_check <= 8192)"); return 1; }
  if (N == 0 || B == 0) return 0;
  unsigned grid = grid_for(N, kBlock * kBinPer);
  hipLaunchKernelGGL(k_bin_counts, dim3(grid), dim3(kBlock), (size_t)(B * n_check) * sizeof(int), stream, t, b, N,
                     B, (int)n_check, counts);
  return check_launch("bin_counts");
}

int atl_bin_counts_sorted(const float* t, const int64_t* b, int64_t N, int64_t B, int64_t n_check, float* counts,
                          hipStream_t stream) {
  if (N < 0 || B < 0 || n_check < 1 || n_check > 65535 || B > 2147483647LL) { set_error("bin_counts_sorted: bad sizes"); return 1; }
  if (B == 0) return 0;
  hipLaunchKernelGGL(k_bin_counts_sorted, dim3((unsigned)B, (unsigned)n_check), dim3(kWave), 0, stream, t, b, N,
                     (int)n_check, counts);
  return check_launch("bin_counts_sorted");
}

int atl_visible_fraction(const float* xa, const float* va, const float* ta, const int64_t* ba, int64_t M,
                         const float* counts, const float* centres, int64_t B, int64_t n_check, double tau,
                         int64_t H, int64_t W, float* out, hipStream_t stream) {
  if (M < 0 || B < 0 || n_check < 1) { set_error("visible_fraction: bad sizes"); return 1; }
  if (M == 0) return 0;
  hipLaunchKernelGGL(k_visible, dim3(grid_for(M)), dim3(kBlock), 0, stream, (const float2*)xa, (const float2*)va,
                     ta, ba, M, counts, centres, B, (int)n_check, (float)tau, (float)(W - 1), (float)(H - 1), out);
  return check_launch("visible_fraction");
}

int atl_anchored_epilogue_fwd(const float* S, const float* wc, const float* vis, int64_t M, double h,
                              double eps, float* ls, float* q, float* D, hipStream_t stream) {
  if (M < 0) { set_error("anchored_epilogue_fwd: bad size"); return 1; }
  if (M == 0) return 0;
  hipLaunchKernelGGL(k_epilogue_fwd, dim3(grid_for(M)), dim3(kBlock), 0, stream, S, wc, vis, M, (float)M_PI,
                     (float)(h * h), (float)eps, ls, q, D);
  return check_launch("anchored_epilogue_fwd");
}

int atl_anchored_epilogue_bwd(const float* g, const float* q, const float* D, int64_t M, float* gS,
                              hipStream_t stream) {
  if (M < 0) { set_error("anchored_epilogue_bwd: bad size"); return 1; }
  if (M == 0) return 0;
  hipLaunchKernelGGL(k_epilogue_bwd, dim3(grid_for(M)), dim3(kBlock), 0, stream, g, q, D, M, gS);
  return check_launch("anchored_epilogue_bwd");
}

int64_t atl_anchored_score_mean_scratch_bytes(void) { return (int64_t)kMeanBlocks * 8; }

int atl_anchored_score_mean_fwd(const float* S, const float* wc, const float* vis, int64_t M, double h, double eps,
                                float* q, float* D, void* scratch, float* out, hipStream_t stream) {
  if (M < 0 || !scratch || !out || (M > 0 && (!S || !wc || !q || !D))) {
    set_error("anchored_score_mean_fwd: bad arguments");
    return 1;
  }
  const unsigned grid = M > 0 ? std::min(grid_for(M), (unsigned)kMeanBlocks) : 1u;
  hipLaunchKernelGGL(k_epilogue_mean, dim3(grid), dim3(kBlock), 0, stream, S, wc, vis, M, (float)M_PI,
                     (float)(h * h), (float)eps, q, D, (double*)scratch);
  hipLaunchKernelGGL(k_epilogue_mean_total, dim3(1), dim3(kBlock), 0, stream, (const double*)scratch, (int)grid, M,
                     out);
  return check_launch("anchored_score_mean_fwd");
}

int atl_anchored_score_mean_bwd(const float* g, const float* q, const float* D, int64_t M, float* gS,
                                hipStream_t stream) {
  if (M < 0 || !g) { set_error("anchored_score_mean_bwd: bad arguments"); return 1; }
  if (M == 0) return 0;
  hipLaunchKernelGGL(k_epilogue_mean_bwd, dim3(grid_for(M)), dim3(kBlock), 0, stream, g, q, D, M, gS);
  return check_launch("anchored_score_mean_bwd");
}

}  // extern "C"
