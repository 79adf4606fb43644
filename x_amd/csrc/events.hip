// Event <-> image kernels for gfx950: bilinear splat / gather (fwd + bwd), truncated-Gaussian splat
// (fwd + bwd), trilinear voxel grid, and the border-clamped flow-grid sampler of DenseLinearFlow (fwd + bwd).
//
// Semantics follow the reference's CPU loops (csrc/atl_cpu.cpp, cited per kernel); float expressions are
// evaluated in the same order and this file is compiled with -ffp-contract=off, so corner indices and
// weights are bit-identical to the reference's fp32 arithmetic.  Outputs that accumulate (splatted images,
// image gradients, grid gradients) are accumulated into caller-zeroed buffers with hardware float atomics.
#include "common.h"
#include "scan.h"
#include "../../include/atl_hip.h"

#include <cmath>

using namespace atlhip;

namespace {

// In-image corners of floor(x), floor(y): csrc/atl_cpu.cpp:17-33.  f(pixel offset, c, dc/dx, dc/dy).
// The float range test before the integer conversion rejects NaN and coordinates too large for int.
template <typename F>
__device__ __forceinline__ void for_corners(float x, float y, int H, int W, F&& f) {
  const float fx = floorf(x), fy = floorf(y);
  if (!(fx >= -1.f && fx <= (float)(W - 1) && fy >= -1.f && fy <= (float)(H - 1))) return;
  const int x0 = (int)fx, y0 = (int)fy;
  const float ax = x - fx, ay = y - fy;
  const float wx0 = 1.f - ax, wy0 = 1.f - ay;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int yy = y0 + j;
    if (yy < 0 || yy >= H) continue;
    const float wy = j ? ay : wy0;
    const float dwy = j ? 1.f : -1.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int xx = x0 + i;
      if (xx < 0 || xx >= W) continue;
      const float wx = i ? ax : wx0;
      const float dwx = i ? 1.f : -1.f;
      f(yy * W + xx, wx * wy, dwx * wy, wx * dwy);
    }
  }
}

__device__ __forceinline__ bool batch_ok(int64_t b, int64_t B) { return b >= 0 && b < B; }

__global__ void k_fill_i32_ev(int* __restrict__ p, int n) {
  if ((int)threadIdx.x < n) p[threadIdx.x] = 0;
}

// csrc/atl_cpu.cpp:38-56
__global__ void __launch_bounds__(kBlock) k_splat_bilinear_fwd(const float2* __restrict__ pos,
                                                               const float* __restrict__ w,
                                                               const int64_t* __restrict__ bidx, int64_t N, int64_t B,
                                                               int H, int W, float* __restrict__ img) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const float wn = w[n];
  const int64_t b = bidx[n];
  if (wn == 0.f || !batch_ok(b, B)) return;
  float* base = img + b * (int64_t)H * W;
  const float2 p = pos[n];
  for_corners(p.x, p.y, H, W, [&](int off, float c, float, float) { atomicAdd(base + off, wn * c); });
}

// csrc/atl_cpu.cpp:58-76
__global__ void __launch_bounds__(kBlock) k_splat_bilinear_bwd(const float* __restrict__ gimg,
                                                               const float2* __restrict__ pos,
                                                               const float* __restrict__ w,
                                                               const int64_t* __restrict__ bidx, int64_t N, int64_t B,
                                                               int H, int W, float2* __restrict__ gpos,
                                                               float* __restrict__ gw) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t b = bidx[n];
  float sx = 0.f, sy = 0.f, sw = 0.f;
  if (batch_ok(b, B)) {
    const float* base = gimg + b * (int64_t)H * W;
    const float2 p = pos[n];
    for_corners(p.x, p.y, H, W, [&](int off, float c, float dcx, float dcy) {
      const float g = base[off];
      sw += g * c;
      sx += g * dcx;
      sy += g * dcy;
    });
  }
  const float wn = w[n];
  gw[n] = sw;
  gpos[n] = make_float2(wn * sx, wn * sy);
}

// csrc/atl_cpu.cpp:134-149
__global__ void __launch_bounds__(kBlock) k_gather_bilinear_fwd(const float* __restrict__ img,
                                                                const float2* __restrict__ pos,
                                                                const int64_t* __restrict__ bidx, int64_t N,
                                                                int64_t B, int H, int W, float* __restrict__ out) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t b = bidx[n];
  float s = 0.f;
  if (batch_ok(b, B)) {
    const float* base = img + b * (int64_t)H * W;
    const float2 p = pos[n];
    for_corners(p.x, p.y, H, W, [&](int off, float c, float, float) { s += c * base[off]; });
  }
  out[n] = s;
}

// csrc/atl_cpu.cpp:151-172
__global__ void __launch_bounds__(kBlock) k_gather_bilinear_bwd(const float* __restrict__ gval,
                                                                const float* __restrict__ img,
                                                                const float2* __restrict__ pos,
                                                                const int64_t* __restrict__ bidx, int64_t N,
                                                                int64_t B, int H, int W, float* __restrict__ gimg,
                                                                float2* __restrict__ gpos) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t b = bidx[n];
  const float g = gval[n];
  float sx = 0.f, sy = 0.f;
  if (batch_ok(b, B)) {
    const int64_t plane = b * (int64_t)H * W;
    const float2 p = pos[n];
    for_corners(p.x, p.y, H, W, [&](int off, float c, float dcx, float dcy) {
      const float v = img[plane + off];
      sx += dcx * v;
      sy += dcy * v;
      if (g != 0.f) atomicAdd(gimg + plane + off, g * c);
    });
  }
  gpos[n] = make_float2(g * sx, g * sy);
}

// Truncated Gaussian around (lround(x), lround(y)), csrc/atl_cpu.cpp:79-104.
__global__ void __launch_bounds__(kBlock) k_splat_gauss_fwd(const float2* __restrict__ pos,
                                                            const float* __restrict__ w,
                                                            const int64_t* __restrict__ bidx, int64_t N, int64_t B,
                                                            int H, int W, float inv2s2, float norm, int R,
                                                            float* __restrict__ img) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const float wn = w[n] * norm;
  const int64_t b = bidx[n];
  if (wn == 0.f || !batch_ok(b, B)) return;
  const float2 p = pos[n];
  const float rx = roundf(p.x), ry = roundf(p.y);
  if (!(rx >= (float)(-R) && rx <= (float)(W - 1 + R) && ry >= (float)(-R) && ry <= (float)(H - 1 + R))) return;
  const int cx = (int)rx, cy = (int)ry;
  float* base = img + b * (int64_t)H * W;
  const int ylo = max(cy - R, 0), yhi = min(cy + R, H - 1);
  const int xlo = max(cx - R, 0), xhi = min(cx + R, W - 1);
  for (int yy = ylo; yy <= yhi; ++yy) {
    const float dy = (float)yy - p.y;
    for (int xx = xlo; xx <= xhi; ++xx) {
      const float dx = (float)xx - p.x;
      atomicAdd(base + yy * W + xx, wn * expf(-(dx * dx + dy * dy) * inv2s2));
    }
  }
}

// csrc/atl_cpu.cpp:106-131
__global__ void __launch_bounds__(kBlock) k_splat_gauss_bwd(const float* __restrict__ gimg,
                                                            const float2* __restrict__ pos,
                                                            const float* __restrict__ w,
                                                            const int64_t* __restrict__ bidx, int64_t N, int64_t B,
                                                            int H, int W, float inv2s2, float norm, float s2, int R,
                                                            float2* __restrict__ gpos, float* __restrict__ gw) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t b = bidx[n];
  const float2 p = pos[n];
  float sw = 0.f, sx = 0.f, sy = 0.f;
  const float rx = roundf(p.x), ry = roundf(p.y);
  if (batch_ok(b, B) &&
      rx >= (float)(-R) && rx <= (float)(W - 1 + R) && ry >= (float)(-R) && ry <= (float)(H - 1 + R)) {
    const int cx = (int)rx, cy = (int)ry;
    const float* base = gimg + b * (int64_t)H * W;
    const int ylo = max(cy - R, 0), yhi = min(cy + R, H - 1);
    const int xlo = max(cx - R, 0), xhi = min(cx + R, W - 1);
    for (int yy = ylo; yy <= yhi; ++yy) {
      const float dy = (float)yy - p.y;
      for (int xx = xlo; xx <= xhi; ++xx) {
        const float dx = (float)xx - p.x;
        const float gk = norm * expf(-(dx * dx + dy * dy) * inv2s2) * base[yy * W + xx];
        sw += gk;
        sx += gk * dx / s2;
        sy += gk * dy / s2;
      }
    }
  }
  const float wn = w[n];
  gw[n] = sw;
  gpos[n] = make_float2(wn * sx, wn * sy);
}

// Trilinear polarity voting, csrc/atl_cpu.cpp:256-286.
__global__ void __launch_bounds__(kBlock) k_voxel_grid(const float2* __restrict__ pos, const float* __restrict__ t,
                                                       const float* __restrict__ pol,
                                                       const int64_t* __restrict__ bidx, int64_t N, int64_t B, int C,
                                                       int H, int W, float* __restrict__ vox) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t b = bidx[n];
  if (!batch_ok(b, B)) return;
  const float2 p = pos[n];
  const float tn = t[n] * (float)(C - 1);
  const float fx = floorf(p.x), fy = floorf(p.y), ft = floorf(tn);
  if (!(fx >= -1.f && fx <= (float)(W - 1) && fy >= -1.f && fy <= (float)(H - 1) && ft >= -1.f &&
        ft <= (float)(C - 1)))
    return;
  const int x0 = (int)fx, y0 = (int)fy, t0 = (int)ft;
  const float pn = pol[n];
  for (int dt = 0; dt < 2; ++dt) {
    const int tt = t0 + dt;
    if (tt < 0 || tt >= C) continue;
    const float wt = 1.f - fabsf((float)tt - tn);
    for (int dy = 0; dy < 2; ++dy) {
      const int yy = y0 + dy;
      if (yy < 0 || yy >= H) continue;
      const float wy = 1.f - fabsf((float)yy - p.y);
      for (int dx = 0; dx < 2; ++dx) {
        const int xx = x0 + dx;
        if (xx < 0 || xx >= W) continue;
        const float wx = 1.f - fabsf((float)xx - p.x);
        atomicAdd(vox + ((b * C + tt) * (int64_t)H + yy) * W + xx, pn * wt * wy * wx);
      }
    }
  }
}

// ------------------------------------------------------------------------------------------- flow grid
// DenseLinearFlow.field + sample_grid (atl/motion/parametric.py:212-216, 235-251): grid coordinates
// gx = x / sx * (Wg - 1) with sx = max(W - 1, 1) (when `scale` is set; raw grid coordinates otherwise),
// border clamp, corners (y0, x0) .. (y1, x1) with x0 <= Wg - 2, fixed sum order c00 + c01 + c10 + c11.
struct GridCorners {
  int o00, o01, o10, o11;      // offsets inside one (Hg, Wg) plane
  float w00, w01, w10, w11;
};

__device__ __forceinline__ GridCorners grid_corners(float x, float y, int Hg, int Wg, float sxw, float syh,
                                                    bool scale) {
  float gx = x, gy = y;
  if (scale) {
    gx = x / sxw * (float)(Wg - 1);
    gy = y / syh * (float)(Hg - 1);
  }
  gx = fminf(fmaxf(gx, 0.f), (float)(Wg - 1));   // clamp(0, Wg-1); NaN stays NaN as in torch.clamp
  gy = fminf(fmaxf(gy, 0.f), (float)(Hg - 1));
  if (gx != gx) gx = 0.f;
  if (gy != gy) gy = 0.f;
  const float x0 = fminf(floorf(gx), (float)max(Wg - 2, 0));
  const float y0 = fminf(floorf(gy), (float)max(Hg - 2, 0));
  const float ax = gx - x0, ay = gy - y0;
  const int ix0 = (int)x0, iy0 = (int)y0;
  const int ix1 = min(ix0 + 1, Wg - 1), iy1 = min(iy0 + 1, Hg - 1);
  GridCorners c;
  c.o00 = iy0 * Wg + ix0;
  c.o01 = iy0 * Wg + ix1;
  c.o10 = iy1 * Wg + ix0;
  c.o11 = iy1 * Wg + ix1;
  c.w00 = (1.f - ax) * (1.f - ay);
  c.w01 = ax * (1.f - ay);
  c.w10 = (1.f - ax) * ay;
  c.w11 = ax * ay;
  return c;
}

__global__ void __launch_bounds__(kBlock) k_sample_grid_fwd(const float* __restrict__ field, int64_t B, int C,
                                                            int Hg, int Wg, const float2* __restrict__ pos,
                                                            const int64_t* __restrict__ bidx, int64_t N, float sxw,
                                                            float syh, int scale, float* __restrict__ out) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t b = bidx[n];
  float* o = out + n * C;
  if (!batch_ok(b, B)) {
    for (int c = 0; c < C; ++c) o[c] = 0.f;
    return;
  }
  const float2 p = pos[n];
  const GridCorners g = grid_corners(p.x, p.y, Hg, Wg, sxw, syh, scale != 0);
  const int64_t plane = (int64_t)Hg * Wg;
  const float* f = field + b * C * plane;
  for (int c = 0; c < C; ++c) {
    const float* fc = f + c * plane;
    float v = fc[g.o00] * g.w00;
    v = v + fc[g.o01] * g.w01;
    v = v + fc[g.o10] * g.w10;
    v = v + fc[g.o11] * g.w11;
    o[c] = v;
  }
}

__global__ void __launch_bounds__(kBlock) k_sample_grid_bwd(const float* __restrict__ gout, int64_t B, int C,
                                                            int Hg, int Wg, const float2* __restrict__ pos,
                                                            const int64_t* __restrict__ bidx, int64_t N, float sxw,
                                                            float syh, int scale, float* __restrict__ gfield) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t b = bidx[n];
  if (!batch_ok(b, B)) return;
  const float2 p = pos[n];
  const GridCorners g = grid_corners(p.x, p.y, Hg, Wg, sxw, syh, scale != 0);
  const int64_t plane = (int64_t)Hg * Wg;
  float* f = gfield + b * C * plane;
  for (int c = 0; c < C; ++c) {
    const float go = gout[n * C + c];
    if (go == 0.f) continue;
    float* fc = f + c * plane;
    atomicAdd(fc + g.o00, go * g.w00);
    atomicAdd(fc + g.o01, go * g.w01);
    atomicAdd(fc + g.o10, go * g.w10);
    atomicAdd(fc + g.o11, go * g.w11);
  }
}

bool dims_ok(int64_t H, int64_t W) { return H > 0 && W > 0 && H * W < (int64_t)1 << 31; }

// ------------------------------------------------------------------------------------------- flow-grid plan
// The adjoint of the flow lookup as a gather: positions sorted by their base corner (y0, x0) (two-level
// counting sort: LDS bucket histograms per block, then one workgroup per bucket of 8192 corners), then one
// thread per grid node sums the weighted output gradients of the positions in the four cells around it.
// No atomics: scattered float atomics run at ~25 G/s here, and positions on event lines put many
// contributions on the same nodes.
constexpr int kGridShift = 13;
constexpr int kGridKeys = 1 << kGridShift;
constexpr int kGridPerBlock = 4096;
constexpr int kGridSortBlock = 1024;

struct GridPlanGeo {
  int B, Hg, Wg, N, nblk, nb;
  float sxw, syh;
  int scale;
};

__device__ __forceinline__ bool grid_key(const float2* pos, const int64_t* bidx, int n, const GridPlanGeo& g,
                                         int& key, float2& a) {
  const int64_t b = bidx[n];
  if (b < 0 || b >= g.B) return false;
  const float2 p = pos[n];
  const GridCorners c = grid_corners(p.x, p.y, g.Hg, g.Wg, g.sxw, g.syh, g.scale != 0);
  key = (int)b * g.Hg * g.Wg + c.o00;
  a = make_float2(c.w00, c.w01);       // weights are recomputed from (w00, w01, w10, w11) below
  return true;
}

template <bool SCATTER>
__global__ void __launch_bounds__(kBlock) k_grid_pass1(const float2* __restrict__ pos, const int64_t* __restrict__ bidx,
                                                       GridPlanGeo g, int* __restrict__ cnt, int* __restrict__ tkey,
                                                       int* __restrict__ tidx) {
  extern __shared__ int hist[];
  for (int i = threadIdx.x; i < g.nb; i += blockDim.x) hist[i] = 0;
  __syncthreads();
  const int n0 = blockIdx.x * kGridPerBlock, n1 = min(n0 + kGridPerBlock, g.N);
  for (int n = n0 + threadIdx.x; n < n1; n += blockDim.x) {
    int key;
    float2 a;
    if (!grid_key(pos, bidx, n, g, key, a)) continue;
    const int bucket = key >> kGridShift;
    if (!SCATTER) {
      atomicAdd(hist + bucket, 1);
    } else {
      const int at = cnt[bucket * g.nblk + blockIdx.x] + atomicAdd(hist + bucket, 1);
      tkey[at] = key;
      tidx[at] = n;
    }
  }
  if (!SCATTER) {
    __syncthreads();
    for (int i = threadIdx.x; i < g.nb; i += blockDim.x) cnt[i * g.nblk + blockIdx.x] = hist[i];
  }
}

// start (B*Hg*Wg rounded up to buckets, + 1) cell offsets; sidx (position index) in corner order.
__global__ void __launch_bounds__(kGridSortBlock) k_grid_pass2(const int* __restrict__ boff,
                                                               const int* __restrict__ tkey,
                                                               const int* __restrict__ tidx, GridPlanGeo g,
                                                               int* __restrict__ start, int* __restrict__ sidx) {
  __shared__ int cnt[kGridKeys];
  __shared__ int cur[kGridKeys];
  __shared__ int wsum[kGridSortBlock / kWave + 1];
  const int bucket = blockIdx.x;
  const int lo = boff[bucket * g.nblk], hi = boff[(bucket + 1) * g.nblk];
  for (int i = threadIdx.x; i < kGridKeys; i += kGridSortBlock) {
    cnt[i] = 0;
    cur[i] = 0;
  }
  __syncthreads();
  for (int p = lo + threadIdx.x; p < hi; p += kGridSortBlock) atomicAdd(cnt + (tkey[p] & (kGridKeys - 1)), 1);
  __syncthreads();
  constexpr int per = kGridKeys / kGridSortBlock;
  int vals[per];
  int s = 0;
#pragma unroll
  for (int k = 0; k < per; ++k) {
    vals[k] = cnt[threadIdx.x * per + k];
    s += vals[k];
  }
  int total;
  int run = block_exclusive_scan<kGridSortBlock>(s, wsum, total);
#pragma unroll
  for (int k = 0; k < per; ++k) {
    const int i = threadIdx.x * per + k;
    cnt[i] = run;
    start[(bucket << kGridShift) + i] = lo + run;
    run += vals[k];
  }
  if (bucket == g.nb - 1 && threadIdx.x == 0) start[g.nb << kGridShift] = hi;
  __syncthreads();
  for (int p = lo + threadIdx.x; p < hi; p += kGridSortBlock) {
    const int kk = tkey[p] & (kGridKeys - 1);
    sidx[lo + cnt[kk] + atomicAdd(cur + kk, 1)] = tidx[p];
  }
}

// Four lanes per grid node (b, y, x), one for each of the cells (y-1..y, x-1..x) whose positions can have
// the node as a corner: each sums gout[n, c] * weight over its cell (loads issued four positions at a
// time), the quad adds its partial sums and its first lane adds them to gfield (the adjoint of
// k_sample_grid_fwd).
constexpr int kGatherUnroll = 4;
__global__ void __launch_bounds__(kBlock) k_grid_gather(const float* __restrict__ gout, int C,
                                                        const float2* __restrict__ pos, GridPlanGeo g,
                                                        const int* __restrict__ start, const int* __restrict__ sidx,
                                                        float* __restrict__ gfield) {
  const int64_t tid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int plane = g.Hg * g.Wg;
  const int64_t nodes = (int64_t)g.B * plane;
  const bool live = tid < 4 * nodes;                 // every lane of a quad has the same liveness
  const int node = live ? (int)(tid >> 2) : 0;
  const int q = (int)(tid & 3);
  const int b = node / plane, o = node - b * plane;
  const int y = o / g.Wg, x = o - y * g.Wg;
  const int cy = y - 1 + (q >> 1), cx = x - 1 + (q & 1);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const int cmax = C < 4 ? C : 4;
  if (live && cy >= 0 && cx >= 0) {
    const int key = b * plane + cy * g.Wg + cx;
    const int k0 = start[key], k1 = start[key + 1];
    for (int k = k0; k < k1; k += kGatherUnroll) {
      int n[kGatherUnroll];
      float2 p[kGatherUnroll];
#pragma unroll
      for (int u = 0; u < kGatherUnroll; ++u) n[u] = sidx[min(k + u, k1 - 1)];
#pragma unroll
      for (int u = 0; u < kGatherUnroll; ++u) p[u] = pos[n[u]];
#pragma unroll
      for (int u = 0; u < kGatherUnroll; ++u) {
        const GridCorners c = grid_corners(p[u].x, p[u].y, g.Hg, g.Wg, g.sxw, g.syh, g.scale != 0);
        float w = 0.f;
        if (c.o00 == o) w += c.w00;
        if (c.o01 == o) w += c.w01;
        if (c.o10 == o) w += c.w10;
        if (c.o11 == o) w += c.w11;
        if (k + u >= k1) w = 0.f;
        for (int ch = 0; ch < cmax; ++ch) acc[ch] = fmaf(gout[(int64_t)n[u] * C + ch], w, acc[ch]);
      }
    }
  }
  for (int ch = 0; ch < 4; ++ch) {
    acc[ch] += __shfl_xor(acc[ch], 1, kWave);
    acc[ch] += __shfl_xor(acc[ch], 2, kWave);
  }
  if (live && q == 0)
    for (int ch = 0; ch < cmax; ++ch) gfield[((int64_t)b * C + ch) * plane + o] += acc[ch];
}

GridPlanGeo grid_geo(int64_t B, int64_t Hg, int64_t Wg, int64_t N, int64_t img_h, int64_t img_w) {
  GridPlanGeo g;
  g.B = (int)B; g.Hg = (int)Hg; g.Wg = (int)Wg; g.N = (int)N;
  g.nblk = (int)((N + kGridPerBlock - 1) / kGridPerBlock);
  g.nb = (int)((B * Hg * Wg + kGridKeys - 1) / kGridKeys);
  g.scale = img_h > 0 && img_w > 0;
  g.sxw = (float)(img_w - 1 > 1 ? img_w - 1 : 1);
  g.syh = (float)(img_h - 1 > 1 ? img_h - 1 : 1);
  return g;
}

struct GridPlanLayout {
  int64_t cnt, boff, part, start, tkey, tidx, sidx, bytes;
};

int64_t align256(int64_t n) { return (n + 255) & ~(int64_t)255; }

GridPlanLayout grid_layout(const GridPlanGeo& g) {
  GridPlanLayout L;
  const int64_t nbh = (int64_t)g.nb * g.nblk;
  int64_t off = 0;
  L.cnt = off;   off += align256(nbh * 4);
  L.boff = off;  off += align256((nbh + 1) * 4);
  L.part = off;  off += align256((scan_tiles(nbh > 0 ? nbh : 1) + 1) * 4);
  L.start = off; off += align256(((int64_t)g.nb * kGridKeys + 1) * 4);
  L.tkey = off;  off += align256((int64_t)g.N * 4);
  L.tidx = off;  off += align256((int64_t)g.N * 4);
  L.sidx = off;  off += align256((int64_t)g.N * 4);
  L.bytes = off;
  return L;
}

bool grid_plan_ok(int64_t B, int64_t Hg, int64_t Wg, int64_t N) {
  return B >= 1 && Hg >= 1 && Wg >= 1 && N >= 0 && (double)B * Hg * Wg < 1.0e9 && N < ((int64_t)1 << 30) &&
         (B * Hg * Wg + kGridKeys - 1) / kGridKeys <= 16384;
}

}  // namespace

// ================================================================================================ C-ABI
extern "C" {

int atl_splat_bilinear_fwd(const float* pos, const float* w, const int64_t* b, int64_t N, int64_t B, int64_t H,
                           int64_t W, float* img, hipStream_t stream) {
  if (N < 0 || B < 0 || !dims_ok(H, W)) { set_error("splat_bilinear_fwd: bad sizes N=%lld B=%lld H=%lld W=%lld", (long long)N, (long long)B, (long long)H, (long long)W); return 1; }
  if (N == 0 || B == 0) return 0;
  hipLaunchKernelGGL(k_splat_bilinear_fwd, dim3(grid_for(N)), dim3(kBlock), 0, stream, (const float2*)pos, w, b, N,
                     B, (int)H, (int)W, img);
  return check_launch("splat_bilinear_fwd");
}

int atl_splat_bilinear_bwd(const float* gimg, const float* pos, const float* w, const int64_t* b, int64_t N,
                           int64_t B, int64_t H, int64_t W, float* gpos, float* gw, hipStream_t stream) {
  if (N < 0 || B < 0 || !dims_ok(H, W)) { set_error("splat_bilinear_bwd: bad sizes"); return 1; }
  if (N == 0) return 0;
  hipLaunchKernelGGL(k_splat_bilinear_bwd, dim3(grid_for(N)), dim3(kBlock), 0, stream, gimg, (const float2*)pos, w,
                     b, N, B, (int)H, (int)W, (float2*)gpos, gw);
  return check_launch("splat_bilinear_bwd");
}

int atl_splat_gauss_fwd(const float* pos, const float* w, const int64_t* b, int64_t N, int64_t B, int64_t H,
                        int64_t W, double sigma, int64_t R, float* img, hipStream_t stream) {
  if (N < 0 || B < 0 || !dims_ok(H, W) || R < 0 || R > 4096 || !(sigma > 0)) { set_error("splat_gauss_fwd: bad arguments (sigma=%g R=%lld)", sigma, (long long)R); return 1; }
  if (N == 0 || B == 0) return 0;
  const float s2 = (float)(sigma * sigma);
  const float inv2s2 = 1.f / (2.f * s2), norm = 1.f / (2.f * (float)M_PI * s2);
  hipLaunchKernelGGL(k_splat_gauss_fwd, dim3(grid_for(N)), dim3(kBlock), 0, stream, (const float2*)pos, w, b, N, B,
                     (int)H, (int)W, inv2s2, norm, (int)R, img);
  return check_launch("splat_gauss_fwd");
}

int atl_splat_gauss_bwd(const float* gimg, const float* pos, const float* w, const int64_t* b, int64_t N, int64_t B,
                        int64_t H, int64_t W, double sigma, int64_t R, float* gpos, float* gw, hipStream_t stream) {
  if (N < 0 || B < 0 || !dims_ok(H, W) || R < 0 || R > 4096 || !(sigma > 0)) { set_error("splat_gauss_bwd: bad arguments"); return 1; }
  if (N == 0) return 0;
  const float s2 = (float)(sigma * sigma);
  const float inv2s2 = 1.f / (2.f * s2), norm = 1.f / (2.f * (float)M_PI * s2);
  hipLaunchKernelGGL(k_splat_gauss_bwd, dim3(grid_for(N)), dim3(kBlock), 0, stream, gimg, (const float2*)pos, w, b,
                     N, B, (int)H, (int)W, inv2s2, norm, s2, (int)R, (float2*)gpos, gw);
  return check_launch("splat_gauss_bwd");
}

int atl_gather_bilinear_fwd(const float* img, const float* pos, const int64_t* b, int64_t N, int64_t B, int64_t H,
                            int64_t W, float* out, hipStream_t stream) {
  if (N < 0 || B < 0 || !dims_ok(H, W)) { set_error("gather_bilinear_fwd: bad sizes"); return 1; }
  if (N == 0) return 0;
  hipLaunchKernelGGL(k_gather_bilinear_fwd, dim3(grid_for(N)), dim3(kBlock), 0, stream, img, (const float2*)pos, b,
                     N, B, (int)H, (int)W, out);
  return check_launch("gather_bilinear_fwd");
}

int atl_gather_bilinear_bwd(const float* gval, const float* img, const float* pos, const int64_t* b, int64_t N,
                            int64_t B, int64_t H, int64_t W, float* gimg, float* gpos, hipStream_t stream) {
  if (N < 0 || B < 0 || !dims_ok(H, W)) { set_error("gather_bilinear_bwd: bad sizes"); return 1; }
  if (N == 0) return 0;
  hipLaunchKernelGGL(k_gather_bilinear_bwd, dim3(grid_for(N)), dim3(kBlock), 0, stream, gval, img,
                     (const float2*)pos, b, N, B, (int)H, (int)W, gimg, (float2*)gpos);
  return check_launch("gather_bilinear_bwd");
}

int atl_voxel_grid(const float* pos, const float* t, const float* p, const int64_t* b, int64_t N, int64_t B,
                   int64_t C, int64_t H, int64_t W, float* vox, hipStream_t stream) {
  if (N < 0 || B < 0 || C < 1 || !dims_ok(H, W) || C * H * W >= (int64_t)1 << 31) { set_error("voxel_grid: bad sizes"); return 1; }
  if (N == 0 || B == 0) return 0;
  hipLaunchKernelGGL(k_voxel_grid, dim3(grid_for(N)), dim3(kBlock), 0, stream, (const float2*)pos, t, p, b, N, B,
                     (int)C, (int)H, (int)W, vox);
  return check_launch("voxel_grid");
}

int atl_sample_grid_fwd(const float* field, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                        const int64_t* b, int64_t N, int64_t img_h, int64_t img_w, float* out, hipStream_t stream) {
  if (N < 0 || B < 0 || C < 1 || Hg < 1 || Wg < 1 || !dims_ok(Hg, Wg)) { set_error("sample_grid_fwd: bad sizes"); return 1; }
  if (N == 0) return 0;
  const int scale = img_h > 0 && img_w > 0;
  const float sxw = (float)(img_w - 1 > 1 ? img_w - 1 : 1), syh = (float)(img_h - 1 > 1 ? img_h - 1 : 1);
  hipLaunchKernelGGL(k_sample_grid_fwd, dim3(grid_for(N)), dim3(kBlock), 0, stream, field, B, (int)C, (int)Hg,
                     (int)Wg, (const float2*)pos, b, N, sxw, syh, scale, out);
  return check_launch("sample_grid_fwd");
}

int atl_sample_grid_bwd(const float* gout, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                        const int64_t* b, int64_t N, int64_t img_h, int64_t img_w, float* gfield,
                        hipStream_t stream) {
  if (N < 0 || B < 0 || C < 1 || Hg < 1 || Wg < 1 || !dims_ok(Hg, Wg)) { set_error("sample_grid_bwd: bad sizes"); return 1; }
  if (N == 0) return 0;
  const int scale = img_h > 0 && img_w > 0;
  const float sxw = (float)(img_w - 1 > 1 ? img_w - 1 : 1), syh = (float)(img_h - 1 > 1 ? img_h - 1 : 1);
  hipLaunchKernelGGL(k_sample_grid_bwd, dim3(grid_for(N)), dim3(kBlock), 0, stream, gout, B, (int)C, (int)Hg,
                     (int)Wg, (const float2*)pos, b, N, sxw, syh, scale, gfield);
  return check_launch("sample_grid_bwd");
}

int64_t atl_grid_plan_bytes(int64_t B, int64_t Hg, int64_t Wg, int64_t N) {
  if (!grid_plan_ok(B, Hg, Wg, N)) return -1;
  return grid_layout(grid_geo(B, Hg, Wg, N, 0, 0)).bytes;
}

int atl_grid_plan(int64_t B, int64_t Hg, int64_t Wg, const float* pos, const int64_t* b, int64_t N, int64_t img_h,
                  int64_t img_w, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (!grid_plan_ok(B, Hg, Wg, N)) { set_error("grid_plan: bad sizes B=%lld Hg=%lld Wg=%lld N=%lld", (long long)B, (long long)Hg, (long long)Wg, (long long)N); return 1; }
  const GridPlanGeo g = grid_geo(B, Hg, Wg, N, img_h, img_w);
  const GridPlanLayout L = grid_layout(g);
  if (!ws || ws_bytes < L.bytes) { set_error("grid_plan: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (N > 0 && (!pos || !b)) { set_error("grid_plan: null input"); return 1; }
  char* w = (char*)ws;
  int* cnt = (int*)(w + L.cnt);
  int* boff = (int*)(w + L.boff);
  const int64_t nbh = (int64_t)g.nb * g.nblk;
  const size_t lds = (size_t)g.nb * sizeof(int);
  if (g.nblk > 0) {
    hipLaunchKernelGGL(k_grid_pass1<false>, dim3(g.nblk), dim3(kBlock), lds, stream, (const float2*)pos, b, g, cnt,
                       (int*)nullptr, (int*)nullptr);
    scan32(cnt, nbh, (int*)(w + L.part), boff, stream);
    hipLaunchKernelGGL(k_grid_pass1<true>, dim3(g.nblk), dim3(kBlock), lds, stream, (const float2*)pos, b, g, boff,
                       (int*)(w + L.tkey), (int*)(w + L.tidx));
  } else {
    hipLaunchKernelGGL(k_fill_i32_ev, dim3(1), dim3(64), 0, stream, boff, 1);
  }
  hipLaunchKernelGGL(k_grid_pass2, dim3(g.nb), dim3(kGridSortBlock), 0, stream, (const int*)boff,
                     (const int*)(w + L.tkey), (const int*)(w + L.tidx), g, (int*)(w + L.start), (int*)(w + L.sidx));
  return check_launch("grid_plan");
}

int atl_sample_grid_bwd_planned(const float* gout, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                                int64_t N, int64_t img_h, int64_t img_w, const void* ws, float* gfield,
                                hipStream_t stream) {
  if (!grid_plan_ok(B, Hg, Wg, N) || C < 1 || C > 4) { set_error("sample_grid_bwd_planned: bad sizes (C <= 4)"); return 1; }
  if (!ws || !gfield || (N > 0 && (!gout || !pos))) { set_error("sample_grid_bwd_planned: null argument"); return 1; }
  const GridPlanGeo g = grid_geo(B, Hg, Wg, N, img_h, img_w);
  const GridPlanLayout L = grid_layout(g);
  const char* w = (const char*)ws;
  hipLaunchKernelGGL(k_grid_gather, dim3(grid_for(4 * B * Hg * Wg)), dim3(kBlock), 0, stream, gout, (int)C,
                     (const float2*)pos, g, (const int*)(w + L.start), (const int*)(w + L.sidx), gfield);
  return check_launch("sample_grid_bwd_planned");
}

}  // extern "C"
