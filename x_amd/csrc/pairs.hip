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
  const int64_t j0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  constexpr int U = 4;                             // loads in flight per thread
  for (int64_t j = j0; j < N; j += U * stride) {
    float2 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) q[u] = v[min(j + u * stride, N - 1)];   // repeats of v[N - 1] change no max
#pragma unroll
    for (int u = 0; u < U; ++u) vm = max(vm, float_to_ordered(sqrtf(fmaf(q[u].y, q[u].y, q[u].x * q[u].x))));
  }
  for (int64_t i = j0; i < M; i += U * stride) {
    float2 p[U];
#pragma unroll
    for (int u = 0; u < U; ++u) p[u] = xa[min(i + u * stride, M - 1)];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      mnx = min(mnx, float_to_ordered(p[u].x));
      mny = min(mny, float_to_ordered(p[u].y));
      nmx = min(nmx, float_to_ordered(-p[u].x));
      nmy = min(nmy, float_to_ordered(-p[u].y));
    }
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

// The same plan by a two-level counting sort instead of one global atomic per entry for the counts and another
// for the cursor (k_plan_count, k_plan_fill: about 25 G scattered atomics/s on this part).  Buckets of 2^shift
// consecutive cell keys.  Pass A (COUNT): every block of kPsPer * kPsBlock sources counts its entries per bucket
// in LDS, writes the row (cnt, block-major) and adds its non-zero counts into the bucket totals; one workgroup
// scans the totals into bucket positions.  Pass A (SCATTER): the block reserves its run of every bucket it feeds
// with one atomic add on the bucket's position (which ends as the bucket's end) and writes one 32-byte record per
// entry, (y, v | key, source, t): y = x + v (c_s - t) as source_cell computes it, so pass B gathers nothing.
// Pass B: one workgroup per bucket counts its records per cell in LDS, scans them into the bucket's part of
// cell_start (the CSR offsets of the old path, bit for bit) and writes every entry at its cell's next slot.
// Entry order within a cell is arrival order, unspecified as before.
constexpr int kPsBlock = 512;
constexpr int kPsPer = 8;                          // sources per thread and pass-A block
constexpr int kPsScanBlock = 1024;
constexpr int kPsMaxBuckets = 16 * kPsScanBlock;
constexpr int kPsMinShift = 7;                     // 128 cells per bucket at least: many pass-B workgroups
constexpr int kPsMaxShift = 12;                    // pass B: at most 4096 cells per bucket (16 KB of LDS)
constexpr int kPsItems = 4;                        // pass B: records per thread in flight together
constexpr int kPsOne = 8;                          // pass B: buckets of up to kPsOne * kPsBlock records are read once

struct PsRec {
  float4 f;                                        // y.x, y.y, v.x, v.y
  int4 i;                                          // key, source, t bits, 0
};

template <bool SCATTER>
__global__ void __launch_bounds__(kPsBlock) k_psort_pass_a(const float2* __restrict__ x, const float* __restrict__ t,
                                                         const float2* __restrict__ v,
                                                         const int64_t* __restrict__ b, int64_t N, PlanGeo g,
                                                         int shift, int nbuckets, int* __restrict__ cnt,
                                                         int* __restrict__ tot_or_pos, PsRec* __restrict__ rec) {
  extern __shared__ int hist[];
  const int blk = blockIdx.x;
  int* mycnt = cnt + (int64_t)blk * nbuckets;
  for (int i = threadIdx.x; i < nbuckets; i += blockDim.x) {
    int h = 0;
    if (SCATTER) {
      const int c = mycnt[i];
      if (c > 0) h = atomicAdd(tot_or_pos + i, c);  // this block's run of bucket i
    }
    hist[i] = h;
  }
  __syncthreads();
  const int64_t j0 = (int64_t)blk * (kPsPer * kPsBlock) + threadIdx.x;
  // the thread's sources are read before any is binned, so that all their loads are in flight together
  int64_t bb[kPsPer];
  float tt[kPsPer];
  float2 xx[kPsPer], vv[kPsPer];
#pragma unroll
  for (int u = 0; u < kPsPer; ++u) {
    const int64_t j = min(j0 + (int64_t)u * kPsBlock, N - 1);
    bb[u] = b[j];
    tt[u] = t[j];
    xx[u] = x[j];
    vv[u] = v[j];
  }
#pragma unroll
  for (int u = 0; u < kPsPer; ++u) {
    const int64_t j = j0 + (int64_t)u * kPsBlock;
    if (j >= N) break;
    const int64_t bj = bb[u];
    if (bj < 0 || bj >= g.B) continue;
    const float tj = tt[u];
    const float2 xj = xx[u], vj = vv[u];
    int lo, hi;
    slice_range(tj, g, lo, hi);
    for (int s = lo; s <= hi; ++s) {
      float2 y;
      int cx, cy;
      if (!source_cell(xj, vj, tj, slice_centre(s, g.delta), g, y, cx, cy)) continue;
      const int key = (int)((((int)bj * g.S + s) * (int64_t)g.GH + cy) * g.GW + cx);
      const int slot = atomicAdd(hist + (key >> shift), 1);
      if (SCATTER) {
        PsRec r;
        r.f = make_float4(y.x, y.y, vj.x, vj.y);
        r.i = make_int4(key, (int)j, __float_as_int(tj), 0);
        rec[slot] = r;
      }
    }
  }
  if (!SCATTER) {
    __syncthreads();
    for (int i = threadIdx.x; i < nbuckets; i += blockDim.x) {
      const int c = hist[i];
      mycnt[i] = c;
      if (c > 0) atomicAdd(tot_or_pos + i, c);
    }
  }
}

__global__ void __launch_bounds__(kPsBlock) k_psort_pass_b(const PsRec* __restrict__ rec, const int* __restrict__ bend,
                                                         const int* __restrict__ tot, int shift, int64_t ncell,
                                                         int nbuckets, int64_t* __restrict__ start,
                                                         float2* __restrict__ src_y, float2* __restrict__ src_v,
                                                         float* __restrict__ src_t, int64_t* __restrict__ src_id) {
  __shared__ int cur[1 << kPsMaxShift];
  __shared__ int wsum[kPsBlock / kWave + 1];
  const int bk = blockIdx.x;
  const int nk = 1 << shift;                       // cells of a bucket
  const int hi = bend[bk], lo = hi - tot[bk];
  const int base = bk << shift;
  const int4* tki = (const int4*)rec;              // int half of record p: tki[2 p + 1]
  for (int i = threadIdx.x; i < nk; i += kPsBlock) cur[i] = 0;
  __syncthreads();
  // a bucket of up to kPsOne * kPsBlock records is read once: the records stay in registers with their rank
  // among the records of their cell (the count's return value), and are written after the scan
  const bool one = hi - lo <= kPsOne * kPsBlock;
  PsRec r1[kPsOne];
  int rk[kPsOne];
  if (one && hi > lo) {                            // positions clamped into the bucket: every load in flight at once
#pragma unroll
    for (int u = 0; u < kPsOne; ++u) r1[u] = rec[min(lo + u * kPsBlock + (int)threadIdx.x, hi - 1)];
#pragma unroll
    for (int u = 0; u < kPsOne; ++u)
      rk[u] = lo + u * kPsBlock + (int)threadIdx.x < hi ? atomicAdd(cur + (r1[u].i.x - base), 1) : 0;
  } else if (!one) {
    for (int k = lo + (int)threadIdx.x; k < hi; k += kPsBlock) atomicAdd(cur + (tki[2 * k + 1].x - base), 1);
  }
  __syncthreads();
  const int per = nk > kPsBlock ? nk / kPsBlock : 1;   // cells per thread in the scan
  const int c0 = threadIdx.x * per;
  int sum = 0;
  for (int q = 0; q < per; ++q) sum += c0 + q < nk ? cur[c0 + q] : 0;
  int total;
  int run = block_exclusive_scan<kPsBlock>(sum, wsum, total);
  for (int q = 0; q < per; ++q) {
    const int c = c0 + q;
    if (c >= nk) break;
    const int n = cur[c];
    cur[c] = lo + run;                             // the cell's next slot
    if ((int64_t)base + c < ncell) start[(int64_t)base + c] = lo + run;
    run += n;
  }
  if (bk == nbuckets - 1 && threadIdx.x == 0) start[ncell] = hi;
  __syncthreads();
  if (one) {
#pragma unroll
    for (int u = 0; u < kPsOne; ++u) {
      if (lo + u * kPsBlock + (int)threadIdx.x >= hi) continue;
      const int at = cur[r1[u].i.x - base] + rk[u];
      src_y[at] = make_float2(r1[u].f.x, r1[u].f.y);
      src_v[at] = make_float2(r1[u].f.z, r1[u].f.w);
      src_t[at] = __int_as_float(r1[u].i.z);
      src_id[at] = r1[u].i.y;
    }
    return;
  }
  for (int k0 = lo; k0 < hi; k0 += kPsItems * kPsBlock) {
    PsRec r[kPsItems];
    int at[kPsItems];
#pragma unroll
    for (int u = 0; u < kPsItems; ++u) {
      const int k = k0 + u * kPsBlock + (int)threadIdx.x;
      if (k < hi) r[u] = rec[k];
    }
#pragma unroll
    for (int u = 0; u < kPsItems; ++u)
      if (k0 + u * kPsBlock + (int)threadIdx.x < hi) at[u] = atomicAdd(cur + (r[u].i.x - base), 1);
#pragma unroll
    for (int u = 0; u < kPsItems; ++u) {
      if (k0 + u * kPsBlock + (int)threadIdx.x >= hi) continue;
      src_y[at[u]] = make_float2(r[u].f.x, r[u].f.y);
      src_v[at[u]] = make_float2(r[u].f.z, r[u].f.w);
      src_t[at[u]] = __int_as_float(r[u].i.z);
      src_id[at[u]] = r[u].i.y;
    }
  }
}

// Exclusive scan of the bucket totals into their positions: one workgroup, 16 totals per thread.
__global__ void __launch_bounds__(kPsScanBlock) k_psort_scan(const int* __restrict__ tot, int n, int* __restrict__ pos) {
  __shared__ int wsum[kPsScanBlock / kWave + 1];
  constexpr int kPer = kPsMaxBuckets / kPsScanBlock;
  int v[kPer];
  int sum = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = threadIdx.x * kPer + k;
    v[k] = i < n ? tot[i] : 0;
    sum += v[k];
  }
  int total;
  int run = block_exclusive_scan<kPsScanBlock>(sum, wsum, total);
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = threadIdx.x * kPer + k;
    if (i < n) pos[i] = run;
    run += v[k];
  }
}

struct PsortLayout {
  int shift, nbuckets, nblk;
  int64_t cnt, tot, pos, item, bytes;
};

// Bucket size and workspace of the sorted plan build; false if the grid or the entry capacity is out of range.
bool psort_layout(int64_t N, int64_t ecap, int64_t ncell, PsortLayout& L) {
  if (N < 0 || ecap < 0 || ncell < 1 || ecap >= ((int64_t)1 << 31) || N >= ((int64_t)1 << 31)) return false;
  int shift = kPsMinShift;
  while (shift <= kPsMaxShift && ((ncell + ((int64_t)1 << shift) - 1) >> shift) > kPsMaxBuckets) ++shift;
  if (shift > kPsMaxShift) return false;
  L.shift = shift;
  L.nbuckets = (int)((ncell + ((int64_t)1 << shift) - 1) >> shift);
  L.nblk = (int)((N + kPsPer * kPsBlock - 1) / (kPsPer * kPsBlock));
  auto a256 = [](int64_t n) { return (n + 255) & ~(int64_t)255; };
  int64_t off = 0;
  L.cnt = off;  off += a256((int64_t)L.nblk * L.nbuckets * 4);
  L.tot = off;  off += a256((int64_t)L.nbuckets * 4);
  L.pos = off;  off += a256((int64_t)L.nbuckets * 4);
  L.item = off; off += a256(ecap * (int64_t)sizeof(PsRec));
  L.bytes = off;
  return true;
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

// PRE: part holds the tile totals themselves, and each block adds up those of the tiles before its own (up to
// kScanPreTiles tiles: cheaper than the launch of k_scan_parts); otherwise part holds their exclusive scan.
constexpr int64_t kScanPreTiles = 2048;

template <typename T, bool PRE>
__global__ void __launch_bounds__(kBlock) k_scan_write(const int* __restrict__ in, int64_t n,
                                                       const int64_t* __restrict__ part, T* __restrict__ out) {
  __shared__ int lds[kBlock / kWave + 1];
  __shared__ int64_t pre_lds[kBlock / kWave];
  int64_t offset = 0;
  if (PRE) {
    int64_t s = 0;
    for (int64_t i = threadIdx.x; i < (int64_t)blockIdx.x; i += kBlock) s += part[i];
#pragma unroll
    for (int d = kWave / 2; d >= 1; d >>= 1) s += __shfl_xor(s, d);
    if ((threadIdx.x & (kWave - 1)) == 0) pre_lds[threadIdx.x / kWave] = s;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kBlock / kWave; ++k) offset += pre_lds[k];
  } else {
    offset = part[blockIdx.x];
  }
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
  int64_t run = offset + excl;
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
constexpr int64_t kMaxRecords = (int64_t)1 << 29;   // records, anchors, events: int indices, 32-bit offsets

struct PairRef {
  const float2 *SY, *SV, *AX;
  const float *ST, *AT, *SC;
  const int64_t *SID, *CS, *AC, *AID;
  int64_t S, GH, GW, G, E, N;
  float tau, r2max, kexp;      // kexp = -log2(e) / (2 h^2): exp(-d2 / 2h^2) = exp2(d2 * kexp)
};

__device__ __forceinline__ float gauss(float d2, float kexp) { return __builtin_amdgcn_exp2f(d2 * kexp); }

// The pair tests of csrc/atl_cpu.cpp:186-195 in their fp32 order: not the anchor's own event, |dt| <= tau,
// |r|^2 <= (cut h)^2, with rx, ry = x_i - (y_k + v_k at).  A NaN passes a test exactly where it does there.
__device__ __forceinline__ bool pair_hit(int sid, int id, float dt, float d2, const PairRef& a) {
  return sid != id && !(fabsf(dt) > a.tau) && !(d2 > a.r2max);
}

// Three CSR row ranges over one plane g: rows ylo..yhi (at most three), columns xlo..xhi of each row as one
// contiguous range (the cells of a row are consecutive keys), clamped to [0, cap).  k0[r] is the first record
// of row r; c1, c2, c3 the running lengths, so position p < c3 of the concatenated list is record
// list_pos(p).  Rows past yhi are empty.  Record and anchor counts are below 2^29 (host-checked), so int.
struct Rows3 {
  int k0[3];
  int c1, c2, c3;
};

__device__ __forceinline__ Rows3 row_ranges(const int64_t* __restrict__ start, int64_t cap, int64_t g, int64_t ylo,
                                            int64_t yhi, int64_t xlo, int64_t xhi, int64_t GH, int64_t GW) {
  Rows3 r;
  int run = 0;
  int c[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    int64_t lo = 0, hi = 0;
    if (ylo + q <= yhi) {
      const int64_t row = (g * GH + ylo + q) * GW;
      lo = start[row + xlo];
      hi = start[row + xhi + 1];
      lo = lo < 0 ? 0 : lo;
      hi = hi > cap ? cap : hi;
      hi = hi < lo ? lo : hi;
    }
    r.k0[q] = (int)lo;
    run += (int)(hi - lo);
    c[q] = run;
  }
  r.c1 = c[0];
  r.c2 = c[1];
  r.c3 = c[2];
  return r;
}

__device__ __forceinline__ int list_pos(int p, const Rows3& r) {
  const int base = p >= r.c2 ? r.k0[2] - r.c2 : (p >= r.c1 ? r.k0[1] - r.c1 : r.k0[0]);
  return base + p;
}

// Load with a 32-bit byte offset from a uniform base (the saddr + voffset addressing form; i * sizeof(T) is
// below 2^32 for records < 2^29).
template <typename T>
__device__ __forceinline__ T ldr(const T* base, uint32_t i) {
  return *(const T*)((const char*)base + i * (uint32_t)sizeof(T));
}

// An anchor as the walk sees it.  id is the low word of the anchor's event id (ids are below 2^31, and -1, an
// anchor without an event, matches no source); g < 0 for an anchor outside the grid, which visits nothing.
struct AnchorView {
  float x, y, t, at;          // position, time, t - slice centre
  int id, g, cx, cy;
};

__device__ __forceinline__ AnchorView no_anchor() {
  AnchorView v;
  v.x = v.y = v.t = v.at = 0.f;
  v.id = -1;
  v.g = -1;
  v.cx = v.cy = 0;
  return v;
}

__device__ __forceinline__ AnchorView anchor_from_plan(int64_t i, bool on, const PairRef& a) {
  AnchorView v = no_anchor();
  if (on) {
    const int64_t g = a.AC[3 * i], cx = a.AC[3 * i + 1], cy = a.AC[3 * i + 2];
    if (g >= 0 && g < a.G && cx >= 0 && cx < a.GW && cy >= 0 && cy < a.GH) {
      const float2 xi = a.AX[i];
      v.x = xi.x;
      v.y = xi.y;
      v.t = a.AT[i];
      v.at = v.t - a.SC[g % a.S];
      v.id = (int)a.AID[i];
      v.g = (int)g;
      v.cx = (int)cx;
      v.cy = (int)cy;
    }
  }
  return v;
}

// Sixteen lanes per anchor, four anchors per wave: the 3x3 cells around the anchor's cell (csrc/atl_cpu.cpp:
// 176-200) are three row ranges, walked as one list in steps of 16 consecutive records, so each group reads
// its records coalesced and the four anchors' dependent loads (cell, row starts, records) overlap.
// Visit(j, rx, ry, dt, kernel) runs on the lanes whose candidate contributes.  The trip count is the wave's
// longest list; E >= 1 (the host handles an empty plan), so a dead lane's clamped record index is valid.
constexpr int kWalkBlock = 256;
constexpr int kGroup = 16;

template <typename Visit>
__device__ __forceinline__ void walk_group(const AnchorView& v, const PairRef& a, Visit&& visit) {
  const int sub = threadIdx.x & (kGroup - 1);
  Rows3 r;
  r.k0[0] = r.k0[1] = r.k0[2] = 0;
  r.c1 = r.c2 = r.c3 = 0;
  if (v.g >= 0)
    r = row_ranges(a.CS, a.E, v.g, v.cy > 0 ? v.cy - 1 : 0, v.cy + 1 < a.GH ? v.cy + 1 : a.GH - 1,
                   v.cx > 0 ? v.cx - 1 : 0, v.cx + 1 < a.GW ? v.cx + 1 : a.GW - 1, a.GH, a.GW);
  const int last = (int)a.E - 1;
  const int trips = wave_max_i((r.c3 + kGroup - 1) / kGroup);
  for (int it = 0; it < trips; ++it) {
    const int p = it * kGroup + sub;
    const bool live = p < r.c3;
    int k = list_pos(live ? p : 0, r);
    k = k < last ? k : last;
    const int sid = ldr((const int*)a.SID, 2u * (uint32_t)k);
    const float st = ldr(a.ST, k);
    const float2 sy = ldr(a.SY, k), sv = ldr(a.SV, k);
    const float dt = v.t - st;
    const float rx = v.x - (sy.x + sv.x * v.at);
    const float ry = v.y - (sy.y + sv.y * v.at);
    const float d2 = rx * rx + ry * ry;
    if (live && pair_hit(sid, v.id, dt, d2, a)) visit(sid, rx, ry, dt, gauss(d2, a.kexp));
  }
}

__device__ __forceinline__ void group_sum(float& acc, int& n) {
#pragma unroll
  for (int d = kGroup / 2; d >= 1; d >>= 1) {
    acc += __shfl_xor(acc, d, kWave);
    n += __shfl_xor(n, d, kWave);
  }
}

// Forward in the plan's anchor order (the workspace-free entry).
__global__ void __launch_bounds__(kWalkBlock) k_pair_fwd_group(PairRef a, int64_t M, float* __restrict__ out,
                                                               int* __restrict__ count) {
  const int64_t i = ((int64_t)blockIdx.x * kWalkBlock + threadIdx.x) / kGroup;
  const bool on = i < M;
  const AnchorView v = anchor_from_plan(i, on, a);
  float acc = 0.f;
  int n = 0;
  walk_group(v, a, [&](int, float, float, float, float k) {
    acc += k;
    ++n;
  });
  group_sum(acc, n);
  if (on && (threadIdx.x & (kGroup - 1)) == 0) {
    out[i] = acc;
    if (count) count[i] = n;
  }
}

// Backward with the reference's per-pair scatter (csrc/atl_cuda.cu:169-180): two global atomics per pair.
// Used only where no workspace is given.  Anchors with gS == 0 are skipped, as there.
__global__ void __launch_bounds__(kWalkBlock) k_pair_bwd_group(PairRef a, int64_t M, const float* __restrict__ gS,
                                                               float invh2, float* __restrict__ gv) {
  const int64_t i = ((int64_t)blockIdx.x * kWalkBlock + threadIdx.x) / kGroup;
  const float gi = i < M ? gS[i] : 0.f;
  const AnchorView v = anchor_from_plan(i, i < M && gi != 0.f, a);
  walk_group(v, a, [&](int j, float rx, float ry, float dt, float kern) {
    const float f = gi * kern * dt * invh2;
    if (j < 0 || j >= a.N) return;
    atomicAdd(gv + 2 * (int64_t)j, f * rx);
    atomicAdd(gv + 2 * (int64_t)j + 1, f * ry);
  });
}

// ---- anchors binned by cell (the workspace entries).  Each anchor inside the grid (and, for the backward,
// with gS != 0, as the reference's backward skips the others) gets a record in its cell's run of the list.
// Within a cell the order follows the atomics; the forward's sums do not depend on it.
struct __align__(16) AnchorRec {
  float x, y, t, g;     // position, time, gS (0 in the forward; the backward reads gS by idx)
  int id, col, row, idx;  // event id (low word), cell column, plane row g * GH + cy, anchor index
};

__device__ __forceinline__ int64_t anchor_key(int64_t i, const PairRef& a) {
  const int64_t g = a.AC[3 * i], cx = a.AC[3 * i + 1], cy = a.AC[3 * i + 2];
  if (g < 0 || g >= a.G || cx < 0 || cx >= a.GW || cy < 0 || cy >= a.GH) return -1;
  return (g * a.GH + cy) * a.GW + cx;
}

__global__ void __launch_bounds__(kBlock) k_anchor_count(PairRef a, int64_t M, const float* __restrict__ gS,
                                                         int* __restrict__ cnt) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M || (gS && gS[i] == 0.f)) return;
  const int64_t key = anchor_key(i, a);
  if (key >= 0) atomicAdd(cnt + key, 1);
}

__device__ __forceinline__ AnchorRec anchor_rec(const PairRef& a, int64_t i, int64_t key, float gi) {
  const float2 xi = a.AX[i];
  AnchorRec rec;
  rec.x = xi.x;
  rec.y = xi.y;
  rec.t = a.AT[i];
  rec.g = gi;
  rec.id = (int)a.AID[i];
  rec.col = (int)a.AC[3 * i + 1];
  rec.row = (int)(key / a.GW);
  rec.idx = (int)i;
  return rec;
}

// Writes each anchor's record into its cell's run, filled from the run's end (the counts run down to zero).
__global__ void __launch_bounds__(kBlock) k_anchor_place(PairRef a, int64_t M, const float* __restrict__ gS,
                                                         const int64_t* __restrict__ astart, int* __restrict__ cnt,
                                                         AnchorRec* __restrict__ arec) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M) return;
  const float gi = gS ? gS[i] : 0.f;
  if (gS && gi == 0.f) return;
  const int64_t key = anchor_key(i, a);
  if (key < 0) return;
  const int slot = atomicSub(cnt + key, 1) - 1;
  arec[astart[key] + slot] = anchor_rec(a, i, key, gi);
}

// The same binning by a two-level counting sort (the plan's scheme: buckets of 2^shift consecutive cells): pass
// A counts the anchors of every block of kAbPer * kAbBlock per bucket in LDS (one block-major row of counts,
// added into the bucket totals), one workgroup scans the totals, and pass A again reserves the block's run of
// each bucket with one atomic add on the bucket's position and writes the anchors' records there; pass B ranks
// each bucket's records by cell in LDS, writes the cells' CSR starts and the records at their final places.
// Within a cell the records follow their arrival in the bucket.  No global atomic per anchor.
constexpr int kAbBlock = 512;
constexpr int kAbPer = 8;                          // anchors per thread of pass A, records per thread of pass B

template <bool SCATTER>
__global__ void __launch_bounds__(kAbBlock) k_abin_a(PairRef a, int64_t M, const float* __restrict__ gS, int shift,
                                                     int nbuckets, int* __restrict__ cnt,
                                                     int* __restrict__ tot_or_pos, AnchorRec* __restrict__ tmp) {
  extern __shared__ int hist[];
  int* mycnt = cnt + (int64_t)blockIdx.x * nbuckets;
  for (int i = threadIdx.x; i < nbuckets; i += kAbBlock) {
    int h = 0;
    if (SCATTER) {
      const int c = mycnt[i];
      if (c > 0) h = atomicAdd(tot_or_pos + i, c);  // this block's run of bucket i
    }
    hist[i] = h;
  }
  __syncthreads();
  const int64_t i0 = (int64_t)blockIdx.x * (kAbPer * kAbBlock) + threadIdx.x;
  int key[kAbPer];
  float gi[kAbPer];
#pragma unroll
  for (int u = 0; u < kAbPer; ++u) {
    const int64_t i = i0 + (int64_t)u * kAbBlock;
    key[u] = -1;
    gi[u] = 0.f;
    if (i < M) {
      gi[u] = gS ? gS[i] : 0.f;
      if (!(gS && gi[u] == 0.f)) key[u] = (int)anchor_key(i, a);   // -1 outside the grid
    }
  }
#pragma unroll
  for (int u = 0; u < kAbPer; ++u) {
    if (key[u] < 0) continue;
    const int slot = atomicAdd(hist + (key[u] >> shift), 1);
    if (SCATTER) tmp[slot] = anchor_rec(a, i0 + (int64_t)u * kAbBlock, key[u], gi[u]);
  }
  if (!SCATTER) {
    __syncthreads();
    for (int i = threadIdx.x; i < nbuckets; i += kAbBlock) {
      const int c = hist[i];
      mycnt[i] = c;
      if (c > 0) atomicAdd(tot_or_pos + i, c);
    }
  }
}

__global__ void __launch_bounds__(kAbBlock) k_abin_b(const AnchorRec* __restrict__ tmp, const int* __restrict__ bend,
                                                     const int* __restrict__ tot, int shift, int64_t ncell,
                                                     int nbuckets, int GW, int64_t* __restrict__ start,
                                                     AnchorRec* __restrict__ arec) {
  __shared__ int cur[1 << kPsMaxShift];
  __shared__ int wsum[kAbBlock / kWave + 1];
  const int bk = blockIdx.x;
  const int nk = 1 << shift;
  const int hi = bend[bk], lo = hi - tot[bk];
  const int base = bk << shift;
  for (int i = threadIdx.x; i < nk; i += kAbBlock) cur[i] = 0;
  __syncthreads();
  const bool one = hi - lo <= kAbPer * kAbBlock;  // the bucket's records stay in registers with their ranks
  AnchorRec r1[kAbPer];
  int rk[kAbPer];
  if (one && hi > lo) {
#pragma unroll
    for (int u = 0; u < kAbPer; ++u) r1[u] = tmp[min(lo + u * kAbBlock + (int)threadIdx.x, hi - 1)];
#pragma unroll
    for (int u = 0; u < kAbPer; ++u)
      rk[u] = lo + u * kAbBlock + (int)threadIdx.x < hi ? atomicAdd(cur + (r1[u].row * GW + r1[u].col - base), 1) : 0;
  } else if (!one) {
    for (int k = lo + (int)threadIdx.x; k < hi; k += kAbBlock) atomicAdd(cur + (tmp[k].row * GW + tmp[k].col - base), 1);
  }
  __syncthreads();
  const int per = nk > kAbBlock ? nk / kAbBlock : 1;   // cells per thread in the scan
  const int c0 = threadIdx.x * per;
  int sum = 0;
  for (int q = 0; q < per; ++q) sum += c0 + q < nk ? cur[c0 + q] : 0;
  int total;
  int run = block_exclusive_scan<kAbBlock>(sum, wsum, total);
  for (int q = 0; q < per; ++q) {
    const int c = c0 + q;
    if (c >= nk) break;
    const int n = cur[c];
    cur[c] = lo + run;                             // the cell's next slot
    if ((int64_t)base + c < ncell) start[(int64_t)base + c] = lo + run;
    run += n;
  }
  if (bk == nbuckets - 1 && threadIdx.x == 0) start[ncell] = hi;
  __syncthreads();
  if (one) {
#pragma unroll
    for (int u = 0; u < kAbPer; ++u)
      if (lo + u * kAbBlock + (int)threadIdx.x < hi) arec[cur[r1[u].row * GW + r1[u].col - base] + rk[u]] = r1[u];
    return;
  }
  for (int k = lo + (int)threadIdx.x; k < hi; k += kAbBlock) {
    const AnchorRec r = tmp[k];
    arec[atomicAdd(cur + (r.row * GW + r.col - base), 1)] = r;
  }
}

// Forward over the binned anchors, one wave per item of up to kCellAnchors anchors of one cell: the anchors of a
// cell share their 3 x 3 neighbourhood, so the wave walks it once, lanes over 64 consecutive records per chunk,
// and every lane evaluates each anchor of the item on its record (the record loads and list arithmetic once per
// NA anchors).  Items per cell ceil(anchors / kCellAnchors), listed by k_cell_items / k_cell_expand.
constexpr int kCellAnchors = 5;

template <int NA>
__device__ __forceinline__ void fwd_cell(const PairRef& a, const AnchorRec* __restrict__ arec, int64_t k0, int g,
                                         int cx, int cy, float* __restrict__ out, int* __restrict__ count) {
  const int lane = threadIdx.x & (kWave - 1);
  const float cs = a.SC[g % a.S];
  float ax[NA], ay[NA], ta[NA], at[NA], acc[NA];
  int id[NA], idx[NA], n[NA];
#pragma unroll
  for (int q = 0; q < NA; ++q) {                 // the same records on every lane
    const AnchorRec r = arec[k0 + q];
    ax[q] = r.x;
    ay[q] = r.y;
    ta[q] = r.t;
    at[q] = r.t - cs;
    id[q] = r.id;
    idx[q] = r.idx;
    acc[q] = 0.f;
    n[q] = 0;
  }
  const Rows3 r = row_ranges(a.CS, a.E, g, cy > 0 ? cy - 1 : 0, cy + 1 < a.GH ? cy + 1 : a.GH - 1,
                             cx > 0 ? cx - 1 : 0, cx + 1 < a.GW ? cx + 1 : a.GW - 1, a.GH, a.GW);
  const int last = (int)a.E - 1;                 // E >= 1 (the host handles an empty plan)
  for (int base = 0; base < r.c3; base += kWave) {
    const int p = base + lane;
    const bool live = p < r.c3;
    int k = list_pos(live ? p : 0, r);
    k = k < last ? k : last;
    const int sid = ldr((const int*)a.SID, 2u * (uint32_t)k);
    const float st = ldr(a.ST, k);
    const float2 sy = ldr(a.SY, k), sv = ldr(a.SV, k);
#pragma unroll
    for (int q = 0; q < NA; ++q) {
      const float dt = ta[q] - st;
      const float rx = ax[q] - (sy.x + sv.x * at[q]);
      const float ry = ay[q] - (sy.y + sv.y * at[q]);
      const float d2 = rx * rx + ry * ry;
      if (live && pair_hit(sid, id[q], dt, d2, a)) {
        acc[q] += gauss(d2, a.kexp);
        ++n[q];
      }
    }
  }
#pragma unroll
  for (int q = 0; q < NA; ++q) {
    acc[q] = wave_sum(acc[q]);
    n[q] = wave_sum(n[q]);
  }
  if (lane == 0) {
#pragma unroll
    for (int q = 0; q < NA; ++q) {
      out[idx[q]] = acc[q];
      if (count) count[idx[q]] = n[q];
    }
  }
}

// Items per cell: ceil(its binned anchors / kCellAnchors).
__global__ void __launch_bounds__(kBlock) k_cell_items(const int64_t* __restrict__ astart, int64_t ncell,
                                                       int* __restrict__ icnt) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= ncell) return;
  icnt[c] = (int)((astart[c + 1] - astart[c] + kCellAnchors - 1) / kCellAnchors);
}

__global__ void __launch_bounds__(kBlock) k_cell_expand(const int* __restrict__ icnt,
                                                        const int64_t* __restrict__ istart, int64_t ncell,
                                                        int2* __restrict__ items) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= ncell) return;
  const int nn = icnt[c];
  const int64_t base = istart[c];
  for (int i = 0; i < nn; ++i) items[base + i] = make_int2((int)c, i * kCellAnchors);
}

// nitems_ptr: the item count (read on the device); the grid covers an upper bound of it.
__global__ void __launch_bounds__(kWalkBlock) k_pair_fwd_cell(PairRef a, const int64_t* __restrict__ astart,
                                                              const AnchorRec* __restrict__ arec,
                                                              const int2* __restrict__ items,
                                                              const int64_t* __restrict__ nitems_ptr,
                                                              float* __restrict__ out, int* __restrict__ count) {
  const int64_t it = ((int64_t)blockIdx.x * kWalkBlock + threadIdx.x) / kWave;
  if (it >= *nitems_ptr) return;                 // per wave: no block barriers
  const int2 item = items[it];
  const int64_t c = item.x;
  const int64_t k0 = astart[c] + item.y;
  const int64_t left = astart[c + 1] - k0;
  const int na = (int)(left < kCellAnchors ? left : kCellAnchors);
  const int64_t rowid = c / a.GW;
  const int cx = (int)(c - rowid * a.GW);
  const int g = (int)(rowid / a.GH), cy = (int)(rowid - (int64_t)g * a.GH);
  switch (na) {
    case 1: fwd_cell<1>(a, arec, k0, g, cx, cy, out, count); break;
    case 2: fwd_cell<2>(a, arec, k0, g, cx, cy, out, count); break;
    case 3: fwd_cell<3>(a, arec, k0, g, cx, cy, out, count); break;
    case 4: fwd_cell<4>(a, arec, k0, g, cx, cy, out, count); break;
    default: fwd_cell<5>(a, arec, k0, g, cx, cy, out, count); break;
  }
}

// ---- source-centric backward.  Work unit: a run of kSegCells source cells of a row; work item: one chunk of
// 64 consecutive records of a unit (so a dense unit spreads over many waves).  One wave per item gathers over
// the binned anchors of the 3 x (kSegCells + 2) cells around the unit and adds each record's sum to gv once
// (two atomics per record instead of two per pair).  A pair (anchor in cell c, record in cell c') is visited
// iff |c - c'| <= 1 in both coordinates of the same plane (the column test is explicit: the unit's anchors
// span kSegCells + 2 columns), the reference's neighbourhood seen from the record's side, and the tests are
// the same, so the visited pairs are the reference's.
constexpr int kSegCells = 6;       // source cells of a row per unit (~6 x 19 records at the 1M-event density)
constexpr int kGatherWaves = 1;    // waves per workgroup, each on its own item
constexpr int kXcds = 8, kXcdRun = 64;
constexpr int kNoCol = -(1 << 29); // column of a padding slot: never within one of a record's column

struct UnitGeo {
  int64_t rowid, g, cy, cx0, cx1;
};

__device__ __forceinline__ UnitGeo unit_geo(int64_t u, int64_t nseg, const PairRef& a) {
  UnitGeo q;
  const int64_t seg = u % nseg;
  q.rowid = u / nseg;
  q.cy = q.rowid % a.GH;
  q.g = q.rowid / a.GH;
  q.cx0 = seg * kSegCells;
  q.cx1 = q.cx0 + kSegCells < a.GW ? q.cx0 + kSegCells : a.GW;
  return q;
}

__device__ __forceinline__ Rows3 unit_anchors(const UnitGeo& q, const int64_t* __restrict__ astart, int64_t Mlist,
                                              const PairRef& a) {
  return row_ranges(astart, Mlist, q.g, q.cy > 0 ? q.cy - 1 : 0, q.cy + 1 < a.GH ? q.cy + 1 : a.GH - 1,
                    q.cx0 > 0 ? q.cx0 - 1 : 0, q.cx1 < a.GW ? q.cx1 : a.GW - 1, a.GH, a.GW);
}

// Items per unit: its 64-record chunks, or none without records or without anchors around it.
__global__ void __launch_bounds__(kBlock) k_unit_chunks(PairRef a, const int64_t* __restrict__ astart, int64_t Mlist,
                                                        int64_t nseg, int64_t units, int* __restrict__ ucnt) {
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= units) return;
  const UnitGeo q = unit_geo(u, nseg, a);
  int64_t e0 = a.CS[q.rowid * a.GW + q.cx0], e1 = a.CS[q.rowid * a.GW + q.cx1];
  e0 = e0 < 0 ? 0 : e0;
  e1 = e1 > a.E ? a.E : e1;
  int n = e1 > e0 ? (int)((e1 - e0 + kWave - 1) / kWave) : 0;
  if (n > 0 && unit_anchors(q, astart, Mlist, a).c3 == 0) n = 0;
  ucnt[u] = n;
}

__global__ void __launch_bounds__(kBlock) k_unit_items(const int* __restrict__ ucnt,
                                                       const int64_t* __restrict__ ustart, int64_t units,
                                                       int2* __restrict__ items) {
  const int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (u >= units) return;
  const int n = ucnt[u];
  const int64_t base = ustart[u];
  for (int c = 0; c < n; ++c) items[base + c] = make_int2((int)u, c);
}

// Workgroup -> logical block such that runs of kXcdRun consecutive blocks (neighbouring cells) share one XCD's
// L2; the hardware places workgroup w on XCD w % 8.  -1 for the padding workgroups of the last group.
__device__ __forceinline__ int64_t xcd_unit(int64_t nblocks) {
  const int64_t w = blockIdx.x;
  const int64_t grp = w / (kXcds * kXcdRun), rem = w - grp * (kXcds * kXcdRun);
  const int64_t u = grp * (kXcds * kXcdRun) + (rem % kXcds) * kXcdRun + rem / kXcds;
  return u < nblocks ? u : -1;
}

// Orders this wave's LDS writes before its later LDS reads (a wave's LDS operations execute in order; this is
// the compiler barrier plus the wait for the writes).
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// max_items bounds the item count (the grid); the count itself is read on the device (nitems_ptr).  SLOTS: each
// record's sum goes to its own slot, slots[k * N + source] with k = slice - the first slice of the source's
// range (a plan holds one record per source and slice of its range, so k < ms; k-major, so that the records of
// one plane write into few N-slot rows; a record outside that range adds its sum with atomics),
// and k_slots_reduce adds every source's slots into gv afterwards; otherwise two atomics per record add it to gv.
template <bool SLOTS>
__global__ void __launch_bounds__(kGatherWaves * kWave)
k_pair_bwd_gather(PairRef a, const int64_t* __restrict__ astart, const AnchorRec* __restrict__ arec, int64_t Mlist,
                  const int2* __restrict__ items, const int64_t* __restrict__ nitems_ptr, int64_t max_items,
                  float invh2, int64_t nseg, float* __restrict__ gv, float2* __restrict__ slots, PlanGeo sg,
                  int ms, const float* __restrict__ gS) {
  __shared__ float4 sa[kGatherWaves][kWave];   // anchor x, y, t, gS
  __shared__ int4 sb[kGatherWaves][kWave];     // at = t - slice centre (bits), anchor id, anchor cell column
  const int lane = threadIdx.x & (kWave - 1), w = threadIdx.x / kWave;
  const int64_t lb = xcd_unit((max_items + kGatherWaves - 1) / kGatherWaves);
  if (lb < 0) return;
  const int64_t it = lb * kGatherWaves + w;
  if (it >= *nitems_ptr) return;               // per wave: the waves of a workgroup never synchronise
  const int2 item = items[it];
  const UnitGeo q = unit_geo(item.x, nseg, a);
  int64_t b0 = a.CS[q.rowid * a.GW + q.cx0], e1 = a.CS[q.rowid * a.GW + q.cx1];
  b0 = b0 < 0 ? 0 : b0;                               // the clamps of k_unit_chunks
  e1 = e1 > a.E ? a.E : e1;
  const int64_t e0 = b0 + (int64_t)item.y * kWave;    // item.y < the unit's chunk count, so e0 < e1
  const float cs = a.SC[q.g % a.S];
  const bool live = e0 + lane < e1;
  const int k = (int)(live ? e0 + lane : e1 - 1);
  const int sid = ldr((const int*)a.SID, 2u * (uint32_t)k);
  const float st = ldr(a.ST, k);
  const float2 sy = ldr(a.SY, k), sv = ldr(a.SV, k);
  int ce = (int)q.cx0;                                 // the record's cell column
  for (int64_t c = q.cx0 + 1; c < q.cx1; ++c) ce = k >= a.CS[q.rowid * a.GW + c] ? (int)c : ce;
  // the chunk's records are in cell order: its first and last lanes bound its columns, and only the anchors of
  // the columns one beside them can pair with it (a dense unit's chunks cover one or two of its cells)
  const int nlive = e1 - e0 < kWave ? (int)(e1 - e0) : kWave;
  const int ca = __shfl(ce, 0), cb = __shfl(ce, nlive - 1);
  UnitGeo qa = q;
  qa.cx0 = ca;
  qa.cx1 = cb + 1;
  const Rows3 r = unit_anchors(qa, astart, Mlist, a);
  float gx = 0.f, gy = 0.f;
  bool any = false;
  for (int pb = 0; pb < r.c3; pb += kWave) {
    const int p = pb + lane;
    if (p < r.c3) {
      const AnchorRec an = arec[list_pos(p, r)];
      sa[w][lane] = make_float4(an.x, an.y, an.t, gS[an.idx]);
      sb[w][lane] = make_int4(__float_as_int(an.t - cs), an.id, an.col, 0);
    } else {
      sa[w][lane] = make_float4(0.f, 0.f, 0.f, 0.f);
      sb[w][lane] = make_int4(0, -1, kNoCol, 0);
    }
    wave_lds_sync();
    const int nj = r.c3 - pb < kWave ? r.c3 - pb : kWave;
    for (int q0 = 0; q0 < nj; q0 += 4) {
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const float4 A = sa[w][q0 + qq];
        const int4 Bq = sb[w][q0 + qq];
        const float at = __int_as_float(Bq.x);
        const float dt = A.z - st;
        const float rx = A.x - (sy.x + sv.x * at);
        const float ry = A.y - (sy.y + sv.y * at);
        const float d2 = rx * rx + ry * ry;
        const bool hit = (unsigned)(Bq.z - ce + 1) <= 2u && pair_hit(sid, Bq.y, dt, d2, a);
        const float f = A.w * gauss(d2, a.kexp) * dt * invh2;
        gx += hit ? f * rx : 0.f;
        gy += hit ? f * ry : 0.f;
        any = any || hit;
      }
    }
    wave_lds_sync();
  }
  if (live && any && sid >= 0 && sid < a.N) {
    int kk = -1;
    if (SLOTS) {
      int lo, hi;
      slice_range(st, sg, lo, hi);
      kk = (int)(q.g % a.S) - lo;
    }
    if (SLOTS && kk >= 0 && kk < ms) {
      slots[(int64_t)kk * a.N + sid] = make_float2(gx, gy);
    } else {
      atomicAdd(gv + 2 * (int64_t)sid, gx);
      atomicAdd(gv + 2 * (int64_t)sid + 1, gy);
    }
  }
}

// gv[j] += the sum of source j's ms slots, in slice order (cleared slots of slices without a record add zero).
__global__ void __launch_bounds__(kBlock) k_slots_reduce(const float2* __restrict__ slots, int64_t N, int S,
                                                         float* __restrict__ gv) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= N) return;
  float sx = 0.f, sy = 0.f;
  for (int s = 0; s < S; ++s) {
    const float2 v = slots[s * N + j];
    sx += v.x;
    sy += v.y;
  }
  float2* g = (float2*)gv + j;
  const float2 old = *g;
  *g = make_float2(old.x + sx, old.y + sy);
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

bool pair_args_ok(int64_t E, int64_t ncell, int64_t M, int64_t S, int64_t GH, int64_t GW, double h, int64_t N) {
  return M >= 0 && E >= 0 && N >= 0 && S >= 1 && GH >= 1 && GW >= 1 && ncell >= 0 && ncell % (GH * GW) == 0 &&
         h > 0 && E < kMaxRecords && M < kMaxRecords && N < kMaxRecords && ncell < ((int64_t)1 << 31);
}

int64_t align256(int64_t n) { return (n + 255) & ~(int64_t)255; }

// Workspace of the binned entries: anchor counts per cell (int), their CSR starts (int64, ncell + 1), the
// scan's tile totals, the anchor records binned by cell (32 bytes, M); the backward adds, per unit of
// kSegCells cells, its item count (int) and CSR starts (int64, units + 1) with their scan totals, and the
// items (int2, at most units + E / 64).
struct PairWs {
  int* cnt;
  int64_t* start;
  int64_t* work;
  AnchorRec* arec;
  int* ucnt;
  int64_t* ustart;
  int64_t* uwork;
  int2* items;
  int64_t* fstart;             // the forward's items per cell: CSR starts (ncell + 1), scan totals, the items
  int64_t* fwork;
  int2* fitems;
  int* abcnt;                  // the anchors' counting sort: block-major bucket counts, bucket totals and
  int* abtot;                  // positions, the records in bucket order (ab_shift < 0: grids of more buckets
  int* abpos;                  // than one workgroup scans take the atomic binning)
  AnchorRec* abtmp;
  float2* slots;               // the backward's per-(source, slice) sums (N * S), when the workspace holds them
  int ab_shift, ab_nbuckets, ab_nblk;
  int64_t units, nseg, max_items, max_fitems, bytes;
};

PairWs pair_ws_layout(void* base, int64_t E, int64_t ncell, int64_t M, int64_t GW, int64_t N = 0, int64_t S = 0) {
  PairWs w;
  w.nseg = (GW + kSegCells - 1) / kSegCells;
  w.units = ncell / GW * w.nseg;
  w.max_items = w.units + E / kWave + 1;
  char* p = (char*)base;
  int64_t off = 0;
  auto take = [&](int64_t nbytes) {
    char* q = p + off;
    off += align256(nbytes > 0 ? nbytes : 1);
    return q;
  };
  w.cnt = (int*)take(4 * ncell);
  w.start = (int64_t*)take(8 * (ncell + 1));
  w.work = (int64_t*)take(8 * atl_scan_work_size(ncell));
  w.arec = (AnchorRec*)take((int64_t)sizeof(AnchorRec) * M);
  w.ucnt = (int*)take(4 * w.units);
  w.ustart = (int64_t*)take(8 * (w.units + 1));
  w.uwork = (int64_t*)take(8 * atl_scan_work_size(w.units));
  w.items = (int2*)take(8 * w.max_items);
  w.max_fitems = M / kCellAnchors + (ncell < M ? ncell : M) + 1;
  w.fstart = (int64_t*)take(8 * (ncell + 1));
  w.fwork = (int64_t*)take(8 * atl_scan_work_size(ncell));
  w.fitems = (int2*)take(8 * w.max_fitems);
  // buckets of about kAbPer * kAbBlock / 2 anchors on average (pass B's workgroups hold up to twice that in
  // registers), at least kPsMinShift and at most kPsMaxShift cells, and few enough for one scan workgroup
  w.ab_shift = -1;
  for (int s = kPsMinShift; s <= kPsMaxShift; ++s)
    if (((ncell + ((int64_t)1 << s) - 1) >> s) <= kPsMaxBuckets &&
        (s == kPsMaxShift || (M << s) >= ncell * (int64_t)(kAbPer * kAbBlock / 2))) {
      w.ab_shift = s;
      break;
    }
  w.ab_nbuckets = w.ab_shift < 0 ? 0 : (int)((ncell + ((int64_t)1 << w.ab_shift) - 1) >> w.ab_shift);
  w.ab_nblk = (int)((M + kAbPer * kAbBlock - 1) / (kAbPer * kAbBlock));
  if (w.ab_shift >= 0) {
    w.abcnt = (int*)take(4 * (int64_t)w.ab_nblk * w.ab_nbuckets);
    w.abtot = (int*)take(4 * (int64_t)w.ab_nbuckets);
    w.abpos = (int*)take(4 * (int64_t)w.ab_nbuckets);
    w.abtmp = (AnchorRec*)take((int64_t)sizeof(AnchorRec) * M);
  }
  w.slots = N > 0 && S > 0 ? (float2*)take(8 * N * S) : nullptr;   // last: the regions above keep their offsets
  w.bytes = off;
  return w;
}

bool pair_ws_ok(const PairWs& w, void* ws, int64_t ws_bytes, const char* what) {
  if (!ws || ws_bytes < w.bytes || ((uintptr_t)ws & 255)) {
    set_error("%s: workspace of %lld bytes (256-aligned) needed, got %lld", what, (long long)w.bytes,
              (long long)ws_bytes);
    return false;
  }
  return true;
}

// Bins the anchors (all inside the grid, or those with gS != 0) into w.arec by cell.
int bin_anchors(const PairRef& a, int64_t M, int64_t ncell, const float* gS, const PairWs& w, hipStream_t stream) {
  if (w.ab_shift >= 0 && M > 0) {
    const size_t lds = (size_t)w.ab_nbuckets * sizeof(int);
    hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(w.ab_nbuckets)), dim3(kBlock), 0, stream, w.abtot,
                       (int64_t)w.ab_nbuckets, 0);
    hipLaunchKernelGGL(k_abin_a<false>, dim3(w.ab_nblk), dim3(kAbBlock), lds, stream, a, M, gS, w.ab_shift,
                       w.ab_nbuckets, w.abcnt, w.abtot, (AnchorRec*)nullptr);
    hipLaunchKernelGGL(k_psort_scan, dim3(1), dim3(kPsScanBlock), 0, stream, (const int*)w.abtot, w.ab_nbuckets,
                       w.abpos);
    hipLaunchKernelGGL(k_abin_a<true>, dim3(w.ab_nblk), dim3(kAbBlock), lds, stream, a, M, gS, w.ab_shift,
                       w.ab_nbuckets, w.abcnt, w.abpos, w.abtmp);
    hipLaunchKernelGGL(k_abin_b, dim3(w.ab_nbuckets), dim3(kAbBlock), 0, stream, (const AnchorRec*)w.abtmp,
                       (const int*)w.abpos, (const int*)w.abtot, w.ab_shift, ncell, w.ab_nbuckets, (int)a.GW,
                       w.start, w.arec);
    return 0;
  }
  hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(ncell)), dim3(kBlock), 0, stream, w.cnt, ncell, 0);
  hipLaunchKernelGGL(k_anchor_count, dim3(grid_for(M)), dim3(kBlock), 0, stream, a, M, gS, w.cnt);
  if (atl_scan_counts(w.cnt, ncell, w.start, w.work, stream)) return 1;
  hipLaunchKernelGGL(k_anchor_place, dim3(grid_for(M)), dim3(kBlock), 0, stream, a, M, gS,
                     (const int64_t*)w.start, w.cnt, w.arec);
  return 0;
}

}  // namespace

// ================================================================================================ C-ABI
extern "C" {

int atl_plan_stats(const float* v, int64_t N, const float* xa, int64_t M, int* stats, hipStream_t stream) {
  if (N < 0 || M < 0 || !stats) { set_error("plan_stats: bad arguments"); return 1; }
  hipLaunchKernelGGL(k_stats_init, dim3(1), dim3(64), 0, stream, stats);
  const int64_t n = N > M ? N : M;
  if (n > 0) {
    unsigned grid = grid_for(n, 4 * kBlock);
    if (grid > 256) grid = 256;                   // few blocks: their same-address atomics serialise
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
  if (tiles <= kScanPreTiles) {
    hipLaunchKernelGGL((k_scan_write<int64_t, true>), dim3((unsigned)tiles), dim3(kBlock), 0, stream, counts, n,
                       (const int64_t*)work, start);
    return check_launch("scan_counts");
  }
  hipLaunchKernelGGL(k_scan_parts, dim3(1), dim3(kBlock), 0, stream, work, tiles);
  hipLaunchKernelGGL((k_scan_write<int64_t, false>), dim3((unsigned)tiles), dim3(kBlock), 0, stream, counts, n,
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

int64_t atl_plan_sort_bytes(int64_t N, int64_t ecap, int64_t ncell) {
  PsortLayout L;
  if (!psort_layout(N, ecap, ncell, L)) return -1;
  return L.bytes;
}

int atl_plan_sort(const float* x, const float* t, const float* v, const int64_t* b, int64_t N, int64_t B, double ox,
                  double oy, double cell, double tau, int64_t S, int64_t GH, int64_t GW, int64_t ecap,
                  int64_t* start, float* src_y, float* src_v, float* src_t, int64_t* src_id, void* ws,
                  int64_t ws_bytes, hipStream_t stream) {
  if (N < 0 || !geo_ok(S, GH, GW, B) || !(cell > 0)) { set_error("plan_sort: bad geometry"); return 1; }
  const int64_t ncell = B * S * GH * GW;
  PsortLayout L;
  if (ncell < 1 || !psort_layout(N, ecap, ncell, L)) { set_error("plan_sort: unsupported sizes (N=%lld ecap=%lld ncell=%lld)", (long long)N, (long long)ecap, (long long)ncell); return 1; }
  if (!ws || ws_bytes < L.bytes) { set_error("plan_sort: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (!start || (N > 0 && (!x || !t || !v || !b))) { set_error("plan_sort: null argument"); return 1; }
  const int64_t ms = std::min<int64_t>((int64_t)std::floor((2.0 * tau + 1.0 / (double)S) * (double)S) + 2, S);
  if (ecap < N * ms) { set_error("plan_sort: ecap %lld below N * max slices (%lld)", (long long)ecap, (long long)(N * ms)); return 1; }
  const PlanGeo g = make_geo(ox, oy, cell, tau, S, GH, GW, B);
  char* w = (char*)ws;
  int* cnt = (int*)(w + L.cnt);
  int* tot = (int*)(w + L.tot);
  int* pos = (int*)(w + L.pos);
  PsRec* rec = (PsRec*)(w + L.item);
  hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(L.nbuckets)), dim3(kBlock), 0, stream, tot, (int64_t)L.nbuckets, 0);
  const size_t lds = (size_t)L.nbuckets * sizeof(int);
  if (L.nblk > 0)
    hipLaunchKernelGGL(k_psort_pass_a<false>, dim3(L.nblk), dim3(kPsBlock), lds, stream, (const float2*)x, t,
                       (const float2*)v, b, N, g, L.shift, L.nbuckets, cnt, tot, (PsRec*)nullptr);
  hipLaunchKernelGGL(k_psort_scan, dim3(1), dim3(kPsScanBlock), 0, stream, (const int*)tot, L.nbuckets, pos);
  if (L.nblk > 0)
    hipLaunchKernelGGL(k_psort_pass_a<true>, dim3(L.nblk), dim3(kPsBlock), lds, stream, (const float2*)x, t,
                       (const float2*)v, b, N, g, L.shift, L.nbuckets, cnt, pos, rec);
  hipLaunchKernelGGL(k_psort_pass_b, dim3(L.nbuckets), dim3(kPsBlock), 0, stream, (const PsRec*)rec,
                     (const int*)pos, (const int*)tot, L.shift, ncell, L.nbuckets, start, (float2*)src_y,
                     (float2*)src_v, src_t, src_id);
  return check_launch("plan_sort");
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
  if (!pair_args_ok(E, ncell, M, S, GH, GW, h, 0)) {
    set_error("ats_pair_fwd: bad arguments (S=%lld GH=%lld GW=%lld ncell=%lld E=%lld M=%lld h=%g)", (long long)S,
              (long long)GH, (long long)GW, (long long)ncell, (long long)E, (long long)M, h);
    return 1;
  }
  if (M == 0) return 0;
  const PairRef a = make_ref(src_y, src_v, src_t, src_id, cell_start, E, ncell, anc_x, anc_t, anc_cell, anc_id,
                             slice_c, S, GH, GW, h, tau, cut, 0);
  if (E == 0) {                                   // no records: every sum and count is zero
    hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(M)), dim3(kBlock), 0, stream, (int*)out, M, 0);
    if (count) hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(M)), dim3(kBlock), 0, stream, count, M, 0);
    return check_launch("ats_pair_fwd");
  }
  hipLaunchKernelGGL(k_pair_fwd_group, dim3(grid_for(M, kWalkBlock / kGroup)), dim3(kWalkBlock), 0, stream, a, M,
                     out, count);
  return check_launch("ats_pair_fwd");
}

int64_t atl_ats_pair_ws_bytes(int64_t E, int64_t ncell, int64_t M, int64_t GW) {
  if (E < 0 || ncell < 0 || M < 0 || GW < 1) return -1;
  return pair_ws_layout(nullptr, E, ncell, M, GW).bytes;
}

int64_t atl_ats_pair_bwd_ws_bytes(int64_t E, int64_t ncell, int64_t M, int64_t GW, int64_t N, int64_t S) {
  if (E < 0 || ncell < 0 || M < 0 || GW < 1 || N < 0 || S < 1 || N >= kMaxRecords || S > 4096) return -1;
  return pair_ws_layout(nullptr, E, ncell, M, GW, N, S).bytes;
}

int atl_ats_pair_fwd_ws(const float* src_y, const float* src_v, const float* src_t, const int64_t* src_id,
                        const int64_t* cell_start, int64_t E, int64_t ncell, const float* anc_x, const float* anc_t,
                        const int64_t* anc_cell, const int64_t* anc_id, int64_t M, const float* slice_c, int64_t S,
                        int64_t GH, int64_t GW, double h, double tau, double cut, float* out, int* count, void* ws,
                        int64_t ws_bytes, hipStream_t stream) {
  if (!pair_args_ok(E, ncell, M, S, GH, GW, h, 0)) {
    set_error("ats_pair_fwd_ws: bad arguments (S=%lld GH=%lld GW=%lld ncell=%lld E=%lld M=%lld h=%g)",
              (long long)S, (long long)GH, (long long)GW, (long long)ncell, (long long)E, (long long)M, h);
    return 1;
  }
  const PairWs w = pair_ws_layout(ws, E, ncell, M, GW);
  if (!pair_ws_ok(w, ws, ws_bytes, "ats_pair_fwd_ws")) return 1;
  if (M == 0) return 0;
  hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(M)), dim3(kBlock), 0, stream, (int*)out, M, 0);
  if (count) hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(M)), dim3(kBlock), 0, stream, count, M, 0);
  if (E == 0 || ncell == 0) return check_launch("ats_pair_fwd_ws");
  const PairRef a = make_ref(src_y, src_v, src_t, src_id, cell_start, E, ncell, anc_x, anc_t, anc_cell, anc_id,
                             slice_c, S, GH, GW, h, tau, cut, 0);
  if (bin_anchors(a, M, ncell, nullptr, w, stream)) return 1;
  // items of up to kCellAnchors anchors of one cell (the per-cell counts reuse cnt, zero after the binning)
  hipLaunchKernelGGL(k_cell_items, dim3(grid_for(ncell)), dim3(kBlock), 0, stream, (const int64_t*)w.start, ncell,
                     w.cnt);
  if (atl_scan_counts(w.cnt, ncell, w.fstart, w.fwork, stream)) return 1;
  hipLaunchKernelGGL(k_cell_expand, dim3(grid_for(ncell)), dim3(kBlock), 0, stream, (const int*)w.cnt,
                     (const int64_t*)w.fstart, ncell, w.fitems);
  const int64_t blocks = (w.max_fitems + kWalkBlock / kWave - 1) / (kWalkBlock / kWave);
  if (blocks > 0x7fffffff) {
    set_error("ats_pair_fwd_ws: %lld anchors too many", (long long)M);
    return 1;
  }
  hipLaunchKernelGGL(k_pair_fwd_cell, dim3((unsigned)blocks), dim3(kWalkBlock), 0, stream, a,
                     (const int64_t*)w.start, (const AnchorRec*)w.arec, (const int2*)w.fitems,
                     (const int64_t*)(w.fstart + ncell), out, count);
  return check_launch("ats_pair_fwd_ws");
}

int atl_ats_pair_bwd(const float* gS, const float* src_y, const float* src_v, const float* src_t,
                     const int64_t* src_id, const int64_t* cell_start, int64_t E, int64_t ncell, const float* anc_x,
                     const float* anc_t, const int64_t* anc_cell, const int64_t* anc_id, int64_t M,
                     const float* slice_c, int64_t S, int64_t GH, int64_t GW, double h, double tau, double cut,
                     int64_t N, float* gv, hipStream_t stream) {
  if (!pair_args_ok(E, ncell, M, S, GH, GW, h, N)) {
    set_error("ats_pair_bwd: bad arguments");
    return 1;
  }
  if (M == 0 || N == 0 || E == 0) return 0;
  const PairRef a = make_ref(src_y, src_v, src_t, src_id, cell_start, E, ncell, anc_x, anc_t, anc_cell, anc_id,
                             slice_c, S, GH, GW, h, tau, cut, N);
  const float invh2 = 1.f / (float)(h * h);
  hipLaunchKernelGGL(k_pair_bwd_group, dim3(grid_for(M, kWalkBlock / kGroup)), dim3(kWalkBlock), 0, stream, a, M,
                     gS, invh2, gv);
  return check_launch("ats_pair_bwd");
}

}  // extern "C"

namespace {
int pair_bwd_ws(const float* gS, const float* src_y, const float* src_v, const float* src_t, const int64_t* src_id,
                const int64_t* cell_start, int64_t E, int64_t ncell, const float* anc_x, const float* anc_t,
                const int64_t* anc_cell, const int64_t* anc_id, int64_t M, const float* slice_c, int64_t S,
                int64_t GH, int64_t GW, double h, double tau, double cut, int64_t N, float* gv, void* ws,
                int64_t ws_bytes, bool binned, hipStream_t stream) {
  if (!pair_args_ok(E, ncell, M, S, GH, GW, h, N)) {
    set_error("ats_pair_bwd_ws: bad arguments");
    return 1;
  }
  // a workspace of atl_ats_pair_bwd_ws_bytes holds the per-(source, slice) sums: no atomics
  const PairWs ws_slots = pair_ws_layout(ws, E, ncell, M, GW, N, S);
  const bool slots = N > 0 && S <= 4096 && ws_bytes >= ws_slots.bytes;
  // slices per source (the plan's bound): the slots of the first ms rows are used
  const int ms = (int)std::min<int64_t>((int64_t)std::floor((2.0 * tau + 1.0 / (double)S) * (double)S) + 2, S);
  const PlanGeo sg = make_geo(0.0, 0.0, 1.0, tau, S, 1, 1, 1);
  const PairWs w = slots ? ws_slots : pair_ws_layout(ws, E, ncell, M, GW);
  if (!pair_ws_ok(w, ws, ws_bytes, "ats_pair_bwd_ws")) return 1;
  if (M == 0 || N == 0 || E == 0 || ncell == 0) return 0;
  const int64_t grp = kXcds * kXcdRun;
  const int64_t blocks = ((w.max_items + kGatherWaves - 1) / kGatherWaves + grp - 1) / grp * grp;
  if (w.units >= kMaxRecords || blocks > 0x7fffffff) {
    set_error("ats_pair_bwd_ws: grid of %lld cells too large", (long long)ncell);
    return 1;
  }
  const PairRef a = make_ref(src_y, src_v, src_t, src_id, cell_start, E, ncell, anc_x, anc_t, anc_cell, anc_id,
                             slice_c, S, GH, GW, h, tau, cut, N);
  const float invh2 = 1.f / (float)(h * h);
  if (slots)
    hipLaunchKernelGGL(k_fill_i32, dim3(grid_for(2 * N * ms)), dim3(kBlock), 0, stream, (int*)w.slots, 2 * N * ms,
                       0);
  // the gather reads each staged anchor's gS by its index: the forward's binning serves as it is
  if (!binned && bin_anchors(a, M, ncell, gS, w, stream)) return 1;
  hipLaunchKernelGGL(k_unit_chunks, dim3(grid_for(w.units)), dim3(kBlock), 0, stream, a, (const int64_t*)w.start, M,
                     w.nseg, w.units, w.ucnt);
  if (atl_scan_counts(w.ucnt, w.units, w.ustart, w.uwork, stream)) return 1;
  hipLaunchKernelGGL(k_unit_items, dim3(grid_for(w.units)), dim3(kBlock), 0, stream, (const int*)w.ucnt,
                     (const int64_t*)w.ustart, w.units, w.items);
  hipLaunchKernelGGL(slots ? k_pair_bwd_gather<true> : k_pair_bwd_gather<false>, dim3((unsigned)blocks),
                     dim3(kGatherWaves * kWave), 0, stream, a, (const int64_t*)w.start, (const AnchorRec*)w.arec, M,
                     (const int2*)w.items, (const int64_t*)(w.ustart + w.units), w.max_items, invh2, w.nseg, gv,
                     w.slots, sg, ms, gS);
  if (slots)
    hipLaunchKernelGGL(k_slots_reduce, dim3(grid_for(N)), dim3(kBlock), 0, stream, (const float2*)w.slots, N, ms,
                       gv);
  return check_launch(binned ? "ats_pair_bwd_ws_binned" : "ats_pair_bwd_ws");
}
}  // namespace

extern "C" {

int atl_ats_pair_bwd_ws(const float* gS, const float* src_y, const float* src_v, const float* src_t,
                        const int64_t* src_id, const int64_t* cell_start, int64_t E, int64_t ncell,
                        const float* anc_x, const float* anc_t, const int64_t* anc_cell, const int64_t* anc_id,
                        int64_t M, const float* slice_c, int64_t S, int64_t GH, int64_t GW, double h, double tau,
                        double cut, int64_t N, float* gv, void* ws, int64_t ws_bytes, hipStream_t stream) {
  return pair_bwd_ws(gS, src_y, src_v, src_t, src_id, cell_start, E, ncell, anc_x, anc_t, anc_cell, anc_id, M,
                     slice_c, S, GH, GW, h, tau, cut, N, gv, ws, ws_bytes, false, stream);
}

int atl_ats_pair_bwd_ws_binned(const float* gS, const float* src_y, const float* src_v, const float* src_t,
                               const int64_t* src_id, const int64_t* cell_start, int64_t E, int64_t ncell,
                               const float* anc_x, const float* anc_t, const int64_t* anc_cell,
                               const int64_t* anc_id, int64_t M, const float* slice_c, int64_t S, int64_t GH,
                               int64_t GW, double h, double tau, double cut, int64_t N, float* gv, void* ws,
                               int64_t ws_bytes, hipStream_t stream) {
  return pair_bwd_ws(gS, src_y, src_v, src_t, src_id, cell_start, E, ncell, anc_x, anc_t, anc_cell, anc_id, M,
                     slice_c, S, GH, GW, h, tau, cut, N, gv, ws, ws_bytes, true, stream);
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
