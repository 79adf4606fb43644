// Fused anchored pair sums on gfx950: the reference's (source, slice) entries and the anchors binned into
// one fixed, clamped fine-cell grid per slice, then a gather-form forward (one lane per anchor) and a
// source-centric backward (one lane per entry), both walking a disc-pruned neighbourhood of fine cells.
//
// What is kept identical to the reference (csrc/atl_cpu.cpp:176-253, atl/ops/functional.py:150-177):
//   * the slice range of every source and its slice-centre position y = x + v (c_s - t), op for op in fp32;
//   * the anchor slice floor(t / delta) clamped to [0, S-1] and at = t - c_s;
//   * the pair tests (id !=, |dt| <= tau, d2 = rx*rx + ry*ry <= (cut*cut)*h*h with
//     rx = x_i - (y + v * at)) in the same fp32 order (this file is built with -ffp-contract=off),
// so the set of contributing pairs, and with it every per-anchor neighbour count, is the reference's.
// What differs is only the spatial index: the reference bins slice-centre positions into cells of
// cut*h + vmax*delta/2 + 1e-3 over the anchors' bounding box and walks 3x3 cells; here positions are first
// clamped into a fixed box around the sensor (clamping never increases a distance) and binned into cells of
// about cut*h/2, and every query walks the rows and column ranges of the cells that meet the disc of radius
// R = cut*h + vmax*max|at| + 0.01 around it.  Any pair that passes the tests lies within R of the query, so
// both walks enumerate a superset of the contributing pairs and apply the same tests to it.  vmax and
// max|at| are reduced on the device, so the whole path runs without a host synchronisation.
#include "common.h"
#include "scan.h"
#include "../../include/atl_hip.h"

#include <cmath>

using namespace atlhip;

namespace {

// Fixed geometry shared by every kernel (host-computed, passed by value).
struct FGeo {
  float gx0, gy0, gx1, gy1;    // clamp box; cell (0, 0) starts at (gx0, gy0)
  float cf;                    // fine cell size
  int GW, GH, S;
  int64_t B;
  int ncell;                   // B * S * GH * GW
  int MS;                      // max slices per source
  float tau, half_delta, delta;
  float r2max, kexp, invh2;    // (cut*cut)*h*h, -log2(e)/(2 h h), 1/(h h)
  float cuth;                  // cut * h
};

// Device scalars written by the plan (ordered-int encodings of non-negative floats).
struct FParams {
  int vmax;                    // max ||v|| over sources
  int atmax;                   // max |t_a - c_s| over anchors
  int pad[6];
};

__device__ __forceinline__ float ordered_to_float(int i) { return __int_as_float(i >= 0 ? i : i ^ 0x7fffffff); }

// Search radius and neighbourhood half-width (in cells) from the device reductions.
__device__ __forceinline__ void search_radius(const FParams* P, const FGeo& G, float& R, float& R2, int& nr) {
  const float vmax = ordered_to_float(P->vmax), atmax = ordered_to_float(P->atmax);
  R = G.cuth * 1.000001f + vmax * atmax * 1.000001f + 0.01f;
  const int lim = max(G.GW, G.GH);
  if (!(R < 1e30f)) {          // inf / NaN velocities: walk the whole slice
    R = 1e30f;
    R2 = 1e30f;
    nr = lim;
    return;
  }
  R2 = R * R;
  const float c = ceilf(R / G.cf);
  nr = c < (float)lim ? (int)c : lim;
}

__device__ __forceinline__ int cell_of(float p, float lo, float hi, float cf, int n) {
  const float c = fminf(fmaxf(p, lo), hi);          // NaN -> lo
  const int i = (int)floorf((c - lo) / cf);
  return min(max(i, 0), n - 1);
}

__device__ __forceinline__ float clampf(float p, float lo, float hi) { return fminf(fmaxf(p, lo), hi); }

// Element i of an array through a 32-bit byte offset from a uniform base (lets the compiler use the
// scalar-base + vector-offset addressing form instead of per-lane 64-bit address arithmetic).
template <typename T>
__device__ __forceinline__ T ld(const T* base, uint32_t i) {
  return *(const T*)((const char*)base + i * (uint32_t)sizeof(T));
}

// Slice range of a source, atl/ops/functional.py:151-152 (same fp32 order as the reference plan).
__device__ __forceinline__ void slice_range(float t, const FGeo& g, int& lo, int& hi) {
  const float a = (((t - g.tau) - g.half_delta) / g.delta) - 0.5f;
  const float c = (((t + g.tau) + g.half_delta) / g.delta) - 0.5f;
  lo = (int)fminf(fmaxf(ceilf(a), 0.f), (float)(g.S - 1));
  hi = (int)fminf(fmaxf(floorf(c), 0.f), (float)(g.S - 1));
}

__device__ __forceinline__ float slice_centre(int s, float delta) { return ((float)s + 0.5f) * delta; }

// Column range [c0, c1] of the cells of row `r` that meet the disc of radius R around (qx, qy); false if
// the row lies entirely outside it.
__device__ __forceinline__ bool row_span(int r, float qx, float qy, float R, float R2, const FGeo& G, int& c0,
                                         int& c1) {
  const float row_lo = G.gy0 + (float)r * G.cf;
  const float row_hi = row_lo + G.cf;
  const float gap = fmaxf(0.f, fmaxf(row_lo - qy, qy - row_hi));
  if (gap > R) return false;
  const float w = sqrtf(fmaxf(R2 - gap * gap, 0.f));
  c0 = cell_of(qx - w, G.gx0, G.gx1, G.cf, G.GW);
  c1 = cell_of(qx + w, G.gx0, G.gx1, G.cf, G.GW);
  return true;
}

// ------------------------------------------------------------------------------------------ plan
__global__ void __launch_bounds__(kBlock) k_fill_zero(int* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// vmax over velocities, max |at| over anchors (atomic max of ordered ints; params zeroed beforehand).
__global__ void __launch_bounds__(kBlock) k_fast_stats(const float2* __restrict__ v, const int64_t* __restrict__ b,
                                                       int64_t N, const float* __restrict__ t,
                                                       const int64_t* __restrict__ anchors, int64_t M, FGeo G,
                                                       FParams* __restrict__ P) {
  int vm = 0, am = 0;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < N; j += stride) {
    const int64_t bj = b[j];
    if (bj < 0 || bj >= G.B) continue;
    const float2 q = v[j];
    vm = max(vm, float_to_ordered(sqrtf(q.x * q.x + q.y * q.y)));
  }
  for (int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; m < M; m += stride) {
    const int64_t a = anchors[m];
    if (a < 0 || a >= N) continue;
    const float ta = t[a];
    const float fs = fminf(fmaxf(floorf(ta / G.delta), 0.f), (float)(G.S - 1));
    am = max(am, float_to_ordered(fabsf(ta - slice_centre((int)fs, G.delta))));
  }
  vm = wave_max_i(vm);
  am = wave_max_i(am);
  if ((threadIdx.x & (kWave - 1)) == 0) {
    if (vm > 0) atomicMax(&P->vmax, vm);
    if (am > 0) atomicMax(&P->atmax, am);
  }
}

// Per (source, slice) entry: fine-cell key of the slice-centre position, counted; the rank within the cell
// is kept for the scatter.  Entry e of source j is slice lo_j + e.
__global__ void __launch_bounds__(kBlock) k_fast_entry_count(const float2* __restrict__ x, const float* __restrict__ t,
                                                             const float2* __restrict__ v,
                                                             const int64_t* __restrict__ b, int64_t N, FGeo G,
                                                             int* __restrict__ cnt, int* __restrict__ rank) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= N) return;
  const int64_t bj = b[j];
  if (bj < 0 || bj >= G.B) return;
  const float tj = t[j];
  const float2 xj = x[j], vj = v[j];
  int lo, hi;
  slice_range(tj, G, lo, hi);
  hi = min(hi, lo + G.MS - 1);
  for (int s = lo; s <= hi; ++s) {
    const float dt = slice_centre(s, G.delta) - tj;
    const float yx = xj.x + vj.x * dt, yy = xj.y + vj.y * dt;
    const int cx = cell_of(yx, G.gx0, G.gx1, G.cf, G.GW), cy = cell_of(yy, G.gy0, G.gy1, G.cf, G.GH);
    const int key = (((int)bj * G.S + s) * G.GH + cy) * G.GW + cx;
    rank[j * G.MS + (s - lo)] = atomicAdd(cnt + key, 1);
  }
}

__global__ void __launch_bounds__(kBlock) k_fast_entry_fill(const float2* __restrict__ x, const float* __restrict__ t,
                                                            const float2* __restrict__ v,
                                                            const int64_t* __restrict__ b, int64_t N, FGeo G,
                                                            const int* __restrict__ start,
                                                            const int* __restrict__ rank,
                                                            float4* __restrict__ esv, int2* __restrict__ eti,
                                                            int* __restrict__ ekey) {
  const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= N) return;
  const int64_t bj = b[j];
  if (bj < 0 || bj >= G.B) return;
  const float tj = t[j];
  const float2 xj = x[j], vj = v[j];
  int lo, hi;
  slice_range(tj, G, lo, hi);
  hi = min(hi, lo + G.MS - 1);
  for (int s = lo; s <= hi; ++s) {
    const float dt = slice_centre(s, G.delta) - tj;
    const float yx = xj.x + vj.x * dt, yy = xj.y + vj.y * dt;
    const int cx = cell_of(yx, G.gx0, G.gx1, G.cf, G.GW), cy = cell_of(yy, G.gy0, G.gy1, G.cf, G.GH);
    const int key = (((int)bj * G.S + s) * G.GH + cy) * G.GW + cx;
    const int at = start[key] + rank[j * G.MS + (s - lo)];
    esv[at] = make_float4(yx, yy, vj.x, vj.y);
    eti[at] = make_int2(__float_as_int(tj), (int)j);
    ekey[at] = key;
  }
}

// Anchor m: slice floor(t / delta) clamped (functional.py:171), fine cell of its clamped position.
__device__ __forceinline__ bool anchor_key(int64_t m, const float2* x, const float* t, const int64_t* b,
                                           const int64_t* anchors, const float2* anchor_xy, int64_t N,
                                           const FGeo& G, int& key, float4& rec, int64_t& a) {
  a = anchors[m];
  if (a < 0 || a >= N) return false;
  const int64_t ba = b[a];
  if (ba < 0 || ba >= G.B) return false;
  const float ta = t[a];
  const float2 xa = anchor_xy ? anchor_xy[m] : x[a];
  const int s = (int)fminf(fmaxf(floorf(ta / G.delta), 0.f), (float)(G.S - 1));
  const int cx = cell_of(xa.x, G.gx0, G.gx1, G.cf, G.GW), cy = cell_of(xa.y, G.gy0, G.gy1, G.cf, G.GH);
  key = (((int)ba * G.S + s) * G.GH + cy) * G.GW + cx;
  rec = make_float4(xa.x, xa.y, ta, ta - slice_centre(s, G.delta));
  return true;
}

__global__ void __launch_bounds__(kBlock) k_fast_anchor_count(const float2* __restrict__ x, const float* __restrict__ t,
                                                              const int64_t* __restrict__ b,
                                                              const int64_t* __restrict__ anchors,
                                                              const float2* __restrict__ anchor_xy, int64_t M,
                                                              int64_t N, FGeo G, int* __restrict__ cnt,
                                                              int* __restrict__ rank) {
  const int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  int key;
  float4 rec;
  int64_t a;
  if (!anchor_key(m, x, t, b, anchors, anchor_xy, N, G, key, rec, a)) return;
  rank[m] = atomicAdd(cnt + key, 1);
}

__global__ void __launch_bounds__(kBlock) k_fast_anchor_fill(const float2* __restrict__ x, const float* __restrict__ t,
                                                             const int64_t* __restrict__ b,
                                                             const int64_t* __restrict__ anchors,
                                                             const float2* __restrict__ anchor_xy, int64_t M,
                                                             int64_t N, FGeo G, const int* __restrict__ start,
                                                             const int* __restrict__ rank, float4* __restrict__ arec,
                                                             int2* __restrict__ aid, int* __restrict__ akey) {
  const int64_t m = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (m >= M) return;
  int key;
  float4 rec;
  int64_t a;
  if (!anchor_key(m, x, t, b, anchors, anchor_xy, N, G, key, rec, a)) return;
  // anchors follow the entries in the shared count/start arrays: their offsets are start[ncell + key] - E
  const int at = start[G.ncell + key] - start[G.ncell] + rank[m];
  arec[at] = rec;
  aid[at] = make_int2((int)a, (int)m);
  akey[at] = key;
}

// ------------------------------------------------------------------------------------------ pair walks
struct FPlan {
  const float4* esv;           // entries: (y.x, y.y, v.x, v.y) at the slice centre
  const int2* eti;             // entries: (t bits, source id)
  const int* ekey;
  const float4* arec;          // anchors: (x, y, t, at)
  const int2* aid;             // anchors: (event id, input position)
  const int* akey;
  const int* start;            // 2*ncell + 1: entry cells, then anchor cells (offset by E)
  const FParams* P;
};

__device__ __forceinline__ void split_key(int key, const FGeo& G, int& g, int& cy, int& cx) {
  const int plane = G.GH * G.GW;
  g = key / plane;
  const int r = key - g * plane;
  cy = r / G.GW;
  cx = r - cy * G.GW;
}

// One candidate pair, predicated: the reference's three tests (csrc/atl_cpu.cpp:187-197) in its fp32 order,
// written as "not rejected" so that NaN distances count as visits exactly as there.
__device__ __forceinline__ bool pair_test(int id_a, int id_s, float ta, float ts, float ax, float ay, float at,
                                          const float4& e, const FGeo& G, float& dt, float& rx, float& ry,
                                          float& d2) {
  dt = ta - ts;
  rx = ax - (e.x + e.z * at);
  ry = ay - (e.y + e.w * at);
  d2 = rx * rx + ry * ry;
  return (id_s != id_a) & !(fabsf(dt) > G.tau) & !(d2 > G.r2max);
}

constexpr int kUnroll = 4;

// Forward: one lane per anchor (in cell order), sum over the entries of its slice within R.
// out[m] = S_m and, with COUNT, count[m] = n_m (number of pairs passing the tests).  The candidate loop
// is unrolled by kUnroll with every load issued before use; per-row partial sums are fp32, the anchor's
// total is accumulated in fp64 (the reference's CPU path sums in fp64).
template <bool COUNT>
__global__ void __launch_bounds__(kBlock) k_fast_fwd(FPlan p, FGeo G, int64_t M, float* __restrict__ out,
                                                     int* __restrict__ count) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int E = p.start[G.ncell];
  const int Mv = p.start[2 * G.ncell] - E;
  if (q >= Mv || q >= M) return;
  float R, R2;
  int nr;
  search_radius(p.P, G, R, R2, nr);
  const float4 A = p.arec[q];
  const int2 ai = p.aid[q];
  int g, cy, cx;
  split_key(p.akey[q], G, g, cy, cx);
  const float qx = clampf(A.x, G.gx0, G.gx1), qy = clampf(A.y, G.gy0, G.gy1);
  const int rlo = max(cy - nr, 0), rhi = min(cy + nr, G.GH - 1);
  double acc = 0.0;
  int n = 0;
  for (int r = rlo; r <= rhi; ++r) {
    int c0, c1;
    if (!row_span(r, qx, qy, R, R2, G, c0, c1)) continue;
    const int row = (g * G.GH + r) * G.GW;
    const int k0 = p.start[row + c0], k1 = p.start[row + c1 + 1];
    float racc = 0.f;
    for (int k = k0; k < k1; k += kUnroll) {
      int2 ti[kUnroll];
      float4 e[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const uint32_t kk = (uint32_t)(k + u);     // up to kUnroll - 1 past the range: padded, masked
        ti[u] = ld(p.eti, kk);
        e[u] = ld(p.esv, kk);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        float dt, rx, ry, d2;
        const bool ok = pair_test(ai.x, ti[u].y, A.z, __int_as_float(ti[u].x), A.x, A.y, A.w, e[u], G, dt, rx, ry,
                                  d2) & (k + u < k1);
        const float kern = __builtin_amdgcn_exp2f(d2 * G.kexp);
        racc += ok ? kern : 0.f;
        if (COUNT) n += ok ? 1 : 0;
      }
    }
    acc += (double)racc;
  }
  out[ai.y] = (float)acc;
  if (COUNT) count[ai.y] = n;
}

// gS in anchor (cell) order.
__global__ void __launch_bounds__(kBlock) k_fast_gather_gs(FPlan p, FGeo G, int64_t M, const float* __restrict__ gS,
                                                           float* __restrict__ gss) {
  const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int Mv = p.start[2 * G.ncell] - p.start[G.ncell];
  if (q >= Mv || q >= M) return;
  gss[q] = gS[p.aid[q].y];
}

// Backward: one lane per entry (source j in slice g), sum over the anchors of slice g within R of it of
// gS_i * k * dt / h^2 * r (csrc/atl_cpu.cpp:240-248), then one atomic add per component into gv[j].
__global__ void __launch_bounds__(kBlock) k_fast_bwd(FPlan p, FGeo G, int64_t ecap, const float* __restrict__ gss,
                                                     float* __restrict__ gv) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int E = p.start[G.ncell];
  if (e >= E || e >= ecap) return;
  float R, R2;
  int nr;
  search_radius(p.P, G, R, R2, nr);
  const float4 sv = p.esv[e];
  const int2 ti = p.eti[e];
  const float tj = __int_as_float(ti.x);
  int g, cy, cx;
  split_key(p.ekey[e], G, g, cy, cx);
  const float qx = clampf(sv.x, G.gx0, G.gx1), qy = clampf(sv.y, G.gy0, G.gy1);
  const int rlo = max(cy - nr, 0), rhi = min(cy + nr, G.GH - 1);
  const int* astart = p.start + G.ncell;
  float gx = 0.f, gy = 0.f;
  for (int r = rlo; r <= rhi; ++r) {
    int c0, c1;
    if (!row_span(r, qx, qy, R, R2, G, c0, c1)) continue;
    const int row = (g * G.GH + r) * G.GW;
    const int k0 = astart[row + c0] - E, k1 = astart[row + c1 + 1] - E;
    for (int k = k0; k < k1; k += kUnroll) {
      int2 ai[kUnroll];
      float4 A[kUnroll];
      float gs[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const uint32_t kk = (uint32_t)(k + u);     // up to kUnroll - 1 past the range: padded, masked
        ai[u] = ld(p.aid, kk);
        A[u] = ld(p.arec, kk);
        gs[u] = ld(gss, kk);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        float dt, rx, ry, d2;
        const bool ok = pair_test(ai[u].x, ti.y, A[u].z, tj, A[u].x, A[u].y, A[u].w, sv, G, dt, rx, ry, d2) &
                        (k + u < k1);
        const float kern = __builtin_amdgcn_exp2f(d2 * G.kexp);
        const float f = gs[u] * kern * dt * G.invh2;
        gx = ok ? fmaf(f, rx, gx) : gx;
        gy = ok ? fmaf(f, ry, gy) : gy;
      }
    }
  }
  if (gx != 0.f || gy != 0.f) {
    const int j = ti.y;
    atomicAdd(gv + 2 * (int64_t)j, gx);
    atomicAdd(gv + 2 * (int64_t)j + 1, gy);
  }
}

// ------------------------------------------------------------------------------------------ host side
int64_t align256(int64_t n) { return (n + 255) & ~(int64_t)255; }

bool make_geo(const atl_fast_geometry* geo, FGeo& G) {
  if (!geo || geo->version != ATL_HIP_ABI_VERSION) return false;
  G.gx0 = geo->gx0; G.gy0 = geo->gy0; G.gx1 = geo->gx1; G.gy1 = geo->gy1; G.cf = geo->cell;
  G.GW = (int)geo->GW; G.GH = (int)geo->GH; G.S = (int)geo->S; G.B = geo->B;
  G.ncell = (int)geo->ncell; G.MS = (int)geo->max_span;
  const double delta = 1.0 / (double)geo->S;
  G.tau = (float)geo->tau;
  G.half_delta = (float)(delta / 2);
  G.delta = (float)delta;
  const float hf = (float)geo->h, cf = (float)geo->cut;
  G.r2max = cf * cf * hf * hf;
  const float inv2h2 = 1.f / (2.f * hf * hf);
  G.kexp = (float)(-(double)inv2h2 * 1.4426950408889634);
  G.invh2 = 1.f / (float)(geo->h * geo->h);
  G.cuth = (float)(geo->cut * geo->h);
  return true;
}

template <typename T>
T* at_off(void* ws, int64_t off) { return (T*)((char*)ws + off); }

FPlan make_plan(void* ws, const atl_fast_geometry* geo) {
  FPlan p;
  p.esv = at_off<float4>(ws, geo->off_esv);
  p.eti = at_off<int2>(ws, geo->off_eti);
  p.ekey = at_off<int>(ws, geo->off_ekey);
  p.arec = at_off<float4>(ws, geo->off_arec);
  p.aid = at_off<int2>(ws, geo->off_aid);
  p.akey = at_off<int>(ws, geo->off_akey);
  p.start = at_off<int>(ws, geo->off_start);
  p.P = at_off<FParams>(ws, geo->off_params);
  return p;
}

}  // namespace

// ================================================================================================ C-ABI
extern "C" {

int atl_fast_geometry_init(int64_t N, int64_t M, int64_t B, int64_t H, int64_t W, int64_t S, double h, double tau,
                           double cut, atl_fast_geometry* geo) {
  if (!geo || N < 0 || M < 0 || B < 1 || H < 1 || W < 1 || S < 1 || S > 65536 || !(h > 0) || !(tau >= 0) ||
      !(cut > 0) || !(h < 1e6) || !(tau < 1e6) || !(cut < 1e6)) {
    set_error("fast_geometry_init: bad arguments (N=%lld M=%lld B=%lld H=%lld W=%lld S=%lld h=%g tau=%g cut=%g)",
              (long long)N, (long long)M, (long long)B, (long long)H, (long long)W, (long long)S, h, tau, cut);
    return 1;
  }
  atl_fast_geometry g{};
  g.version = ATL_HIP_ABI_VERSION;
  g.N = N; g.M = M; g.B = B; g.H = H; g.W = W; g.S = S;
  g.h = h; g.tau = tau; g.cut = cut;
  double cf = 0.5 * cut * h;
  if (cf < 0.5) cf = 0.5;
  const double pad = 16.0;
  g.cell = (float)cf;
  g.gx0 = (float)-pad;
  g.gy0 = (float)-pad;
  g.gx1 = (float)((double)(W - 1) + pad);
  g.gy1 = (float)((double)(H - 1) + pad);
  // cells so that floor((gx1 - gx0) / cell) is the last column, with slack for fp32 rounding
  g.GW = (int64_t)std::floor(((double)g.gx1 - (double)g.gx0) / (double)g.cell) + 2;
  g.GH = (int64_t)std::floor(((double)g.gy1 - (double)g.gy0) / (double)g.cell) + 2;
  const double ncell = (double)B * (double)S * (double)g.GH * (double)g.GW;
  int64_t ms = (int64_t)std::floor((2.0 * tau + 1.0 / (double)S) * (double)S) + 2;
  if (ms > S) ms = S;
  g.max_span = ms;
  const double ecap = (double)N * (double)ms;
  if (ncell * 2 + 1 >= 2.0e9 || ecap >= 2.0e9 || (double)M >= 2.0e9) {
    set_error("fast_geometry_init: problem too large for the 32-bit plan (cells %.0f, entries %.0f)", ncell, ecap);
    return 1;
  }
  g.ncell = (int64_t)ncell;
  g.ecap = (int64_t)ecap;
  const int64_t ncnt = 2 * g.ncell;
  int64_t off = 0;
  g.off_params = off;  off += align256(sizeof(FParams));
  g.off_cnt = off;     off += align256(ncnt * 4);
  g.off_start = off;   off += align256((ncnt + 1) * 4);
  g.off_part = off;    off += align256((scan_tiles(ncnt) + 1) * 4);
  g.off_erank = off;   off += align256(N * ms * 4);
  g.off_arank = off;   off += align256(M * 4);
  // the walks read up to kUnroll - 1 records past a range end: entry and anchor arrays carry that padding
  g.off_esv = off;     off += align256((g.ecap + kUnroll) * 16);
  g.off_eti = off;     off += align256((g.ecap + kUnroll) * 8);
  g.off_ekey = off;    off += align256(g.ecap * 4);
  g.off_arec = off;    off += align256((M + kUnroll) * 16);
  g.off_aid = off;     off += align256((M + kUnroll) * 8);
  g.off_akey = off;    off += align256(M * 4);
  g.off_gss = off;     off += align256((M + kUnroll) * 4);
  g.ws_bytes = off;
  *geo = g;
  return 0;
}

int atl_fast_plan(const atl_fast_geometry* geo, const float* x, const float* t, const float* v, const int64_t* b,
                  const int64_t* anchors, const float* anchor_xy, void* ws, int64_t ws_bytes, hipStream_t stream) {
  FGeo G;
  if (!make_geo(geo, G)) { set_error("fast_plan: geometry not initialised by atl_fast_geometry_init"); return 1; }
  if (!ws || ws_bytes < geo->ws_bytes) { set_error("fast_plan: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)geo->ws_bytes); return 1; }
  const int64_t N = geo->N, M = geo->M;
  if ((N > 0 && (!x || !t || !v || !b)) || (M > 0 && !anchors)) { set_error("fast_plan: null input"); return 1; }
  int* cnt = at_off<int>(ws, geo->off_cnt);
  int* start = at_off<int>(ws, geo->off_start);
  int* part = at_off<int>(ws, geo->off_part);
  int* erank = at_off<int>(ws, geo->off_erank);
  int* arank = at_off<int>(ws, geo->off_arank);
  FParams* P = at_off<FParams>(ws, geo->off_params);
  const int64_t ncnt = 2 * geo->ncell;
  hipLaunchKernelGGL(k_fill_zero, dim3(1), dim3(64), 0, stream, (int*)P, (int64_t)(sizeof(FParams) / 4));
  hipLaunchKernelGGL(k_fill_zero, dim3(grid_for(ncnt)), dim3(kBlock), 0, stream, cnt, ncnt);
  const int64_t n = N > M ? N : M;
  if (n > 0) {
    unsigned grid = grid_for(n);
    if (grid > 1024) grid = 1024;
    hipLaunchKernelGGL(k_fast_stats, dim3(grid), dim3(kBlock), 0, stream, (const float2*)v, b, N, t, anchors, M, G,
                       P);
  }
  if (N > 0)
    hipLaunchKernelGGL(k_fast_entry_count, dim3(grid_for(N)), dim3(kBlock), 0, stream, (const float2*)x, t,
                       (const float2*)v, b, N, G, cnt, erank);
  if (M > 0)
    hipLaunchKernelGGL(k_fast_anchor_count, dim3(grid_for(M)), dim3(kBlock), 0, stream, (const float2*)x, t, b,
                       anchors, (const float2*)anchor_xy, M, N, G, cnt + geo->ncell, arank);
  scan32(cnt, ncnt, part, start, stream);
  if (N > 0)
    hipLaunchKernelGGL(k_fast_entry_fill, dim3(grid_for(N)), dim3(kBlock), 0, stream, (const float2*)x, t,
                       (const float2*)v, b, N, G, (const int*)start, (const int*)erank,
                       at_off<float4>(ws, geo->off_esv), at_off<int2>(ws, geo->off_eti), at_off<int>(ws, geo->off_ekey));
  if (M > 0)
    hipLaunchKernelGGL(k_fast_anchor_fill, dim3(grid_for(M)), dim3(kBlock), 0, stream, (const float2*)x, t, b,
                       anchors, (const float2*)anchor_xy, M, N, G, (const int*)start, (const int*)arank,
                       at_off<float4>(ws, geo->off_arec), at_off<int2>(ws, geo->off_aid),
                       at_off<int>(ws, geo->off_akey));
  return check_launch("fast_plan");
}

int atl_fast_pair_fwd(const atl_fast_geometry* geo, const void* ws, float* out, int* count, hipStream_t stream) {
  FGeo G;
  if (!make_geo(geo, G)) { set_error("fast_pair_fwd: geometry not initialised"); return 1; }
  if (!ws || (geo->M > 0 && !out)) { set_error("fast_pair_fwd: null argument"); return 1; }
  if (geo->M == 0) return 0;
  const FPlan p = make_plan((void*)ws, geo);
  if (count)
    hipLaunchKernelGGL(k_fast_fwd<true>, dim3(grid_for(geo->M)), dim3(kBlock), 0, stream, p, G, geo->M, out, count);
  else
    hipLaunchKernelGGL(k_fast_fwd<false>, dim3(grid_for(geo->M)), dim3(kBlock), 0, stream, p, G, geo->M, out, count);
  return check_launch("fast_pair_fwd");
}

int atl_fast_pair_bwd(const atl_fast_geometry* geo, void* ws, const float* gS, float* gv, hipStream_t stream) {
  FGeo G;
  if (!make_geo(geo, G)) { set_error("fast_pair_bwd: geometry not initialised"); return 1; }
  if (!ws || (geo->M > 0 && (!gS || !gv))) { set_error("fast_pair_bwd: null argument"); return 1; }
  if (geo->M == 0 || geo->N == 0) return 0;
  const FPlan p = make_plan(ws, geo);
  float* gss = at_off<float>(ws, geo->off_gss);
  hipLaunchKernelGGL(k_fast_gather_gs, dim3(grid_for(geo->M)), dim3(kBlock), 0, stream, p, G, geo->M, gS, gss);
  hipLaunchKernelGGL(k_fast_bwd, dim3(grid_for(geo->ecap)), dim3(kBlock), 0, stream, p, G, geo->ecap,
                     (const float*)gss, gv);
  return check_launch("fast_pair_bwd");
}

}  // extern "C"
