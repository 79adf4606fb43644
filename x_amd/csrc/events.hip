// Event <-> image kernels for gfx950: bilinear splat / gather (fwd + bwd), truncated-Gaussian splat
// (fwd + bwd), trilinear voxel grid, and the border-clamped flow-grid sampler of DenseLinearFlow (fwd + bwd).
//
// Semantics follow the reference's CPU loops (csrc/atl_cpu.cpp, cited per kernel); float expressions are
// evaluated in the same order and this file is compiled with -ffp-contract=off, so corner indices and
// weights are bit-identical to the reference's fp32 arithmetic.  Outputs that accumulate (splatted images,
// image gradients, grid gradients) are accumulated into caller-zeroed buffers with hardware float atomics.
#include "common.h"
#include "scan.h"
#include "bilinear.h"
#include "traj.h"
#include "../../include/atl_hip.h"

#include <cmath>

using namespace atlhip;

namespace {

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
  if (Wg >= 2) {                                 // o01 = o00 + 1, o11 = o10 + 1: one 8-byte load per grid row
    for (int c = 0; c < C; ++c) {
      const float* fc = f + c * plane;
      float2 r0, r1;
      __builtin_memcpy(&r0, fc + g.o00, sizeof(float2));   // 4-byte aligned: unaligned 8-byte loads are legal
      __builtin_memcpy(&r1, fc + g.o10, sizeof(float2));
      float v = r0.x * g.w00;
      v = v + r0.y * g.w01;
      v = v + r1.x * g.w10;
      v = v + r1.y * g.w11;
      o[c] = v;
    }
    return;
  }
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

// Position gradient of the flow lookup (autograd of atl/motion/parametric.py:235-251 w.r.t. the positions):
// d out / d gx = sum over corners of field * d w / d gx with ax = gx - x0 (x0 a constant), zero where the
// border clamp is active (torch.clamp passes the gradient for min <= gx <= max), times (Wg - 1) / sx for
// image-pixel positions.  gpos (N, 2) written.
__global__ void __launch_bounds__(kBlock) k_sample_grid_bwd_pos(const float* __restrict__ gout,
                                                                const float* __restrict__ field, int64_t B, int C,
                                                                int Hg, int Wg, const float2* __restrict__ pos,
                                                                const int64_t* __restrict__ bidx, int64_t N,
                                                                float sxw, float syh, int scale,
                                                                float2* __restrict__ gpos) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t b = bidx[n];
  const float2 p = pos[n];
  float sx = 0.f, sy = 0.f;
  if (batch_ok(b, B)) {
    float gx = p.x, gy = p.y, kx = 1.f, ky = 1.f;
    if (scale) {
      gx = p.x / sxw * (float)(Wg - 1);
      gy = p.y / syh * (float)(Hg - 1);
      kx = (float)(Wg - 1) / sxw;
      ky = (float)(Hg - 1) / syh;
    }
    const bool inx = gx >= 0.f && gx <= (float)(Wg - 1), iny = gy >= 0.f && gy <= (float)(Hg - 1);
    const GridCorners c = grid_corners(p.x, p.y, Hg, Wg, sxw, syh, scale != 0);
    const float ax = c.ax, ay = c.ay;
    const int64_t plane = (int64_t)Hg * Wg;
    const float* f = field + b * C * plane;
    for (int ch = 0; ch < C; ++ch) {
      const float* fc = f + ch * plane;
      const float f00 = fc[c.o00], f01 = fc[c.o01], f10 = fc[c.o10], f11 = fc[c.o11];
      const float go = gout[n * C + ch];
      sx += go * ((1.f - ay) * (f01 - f00) + ay * (f11 - f10));
      sy += go * ((1.f - ax) * (f10 - f00) + ax * (f11 - f01));
    }
    sx = inx ? sx * kx : 0.f;
    sy = iny ? sy * ky : 0.f;
  }
  gpos[n] = make_float2(sx, sy);
}

// ---------------------------------------------------------------------- many-channel fields (channels last)
// A field of many channels (a coefficient grid) is sampled from a channels-last copy (B, Hg, Wg, Q) of float4,
// Q = ceil(C / 4), channels past C zero: a node's channels are then one contiguous run, so a corner costs Q
// 16-byte loads instead of C loads from C separate planes.  The forward gives each event Q lanes (one channel
// quad each), so the (N, C) output rows are written with consecutive lanes on consecutive quads.  Both kernels
// keep the plane kernels' fp32 operation order, so their results are the same bits.
__global__ void __launch_bounds__(kBlock) k_field_channels_last(const float* __restrict__ field, int C, int Q,
                                                                int64_t plane, int64_t total,
                                                                float4* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t node = i / Q;
  const int q = (int)(i - node * Q);
  const int64_t b = node / plane, o = node - b * plane;
  const float* f = field + b * C * plane + o;
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int c = 4 * q + j;
    v[j] = c < C ? f[c * plane] : 0.f;
  }
  out[i] = make_float4(v[0], v[1], v[2], v[3]);
}

// Two-channel fields (flows) interleaved by node, (B, Hg, Wg, 2): a grid row's two corner nodes with both
// channels are 16 contiguous bytes, so a lookup reads two pieces instead of four; the sums are
// k_sample_grid_fwd's, bit for bit.
__global__ void __launch_bounds__(kBlock) k_flow_interleave(const float* __restrict__ field, int64_t plane,
                                                            int64_t total, float2* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;   // node (b, o)
  if (i >= total) return;
  const int64_t b = i / plane, o = i - b * plane;
  const float* f = field + b * 2 * plane + o;
  out[i] = make_float2(f[0], f[plane]);
}

// Wg >= 2 (a row's corners are adjacent nodes).
__global__ void __launch_bounds__(kBlock) k_sample_flow_il(const float* __restrict__ fil, int64_t B, int Hg, int Wg,
                                                           const float2* __restrict__ pos,
                                                           const int64_t* __restrict__ bidx, int64_t N, float sxw,
                                                           float syh, int scale, float2* __restrict__ out) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t b = bidx[n];
  if (!batch_ok(b, B)) {
    out[n] = make_float2(0.f, 0.f);
    return;
  }
  const float2 p = pos[n];
  const GridCorners g = grid_corners(p.x, p.y, Hg, Wg, sxw, syh, scale != 0);
  const float* f = fil + b * 2 * ((int64_t)Hg * Wg);
  float4 r0, r1;                                 // (c0, c1) of corner x0, then of x0 + 1: 8-byte aligned
  __builtin_memcpy(&r0, f + 2 * (int64_t)g.o00, sizeof(float4));
  __builtin_memcpy(&r1, f + 2 * (int64_t)g.o10, sizeof(float4));
  float v0 = r0.x * g.w00;
  v0 = v0 + r0.z * g.w01;
  v0 = v0 + r1.x * g.w10;
  v0 = v0 + r1.z * g.w11;
  float v1 = r0.y * g.w00;
  v1 = v1 + r0.w * g.w01;
  v1 = v1 + r1.y * g.w10;
  v1 = v1 + r1.w * g.w11;
  out[n] = make_float2(v0, v1);
}

__device__ __forceinline__ float corner_sum(float f00, float f01, float f10, float f11, const GridCorners& g) {
  float v = f00 * g.w00;
  v = v + f01 * g.w01;
  v = v + f10 * g.w10;
  v = v + f11 * g.w11;
  return v;
}

__global__ void __launch_bounds__(kBlock) k_sample_grid_fwd_cl(const float4* __restrict__ fcl, int64_t B, int C,
                                                               int Q, int Hg, int Wg,
                                                               const float2* __restrict__ pos,
                                                               const int64_t* __restrict__ bidx, int N, float sxw,
                                                               float syh, int scale, float* __restrict__ out) {
  const int g = blockIdx.x * blockDim.x + threadIdx.x;   // lane = (event, channel quad); N * Q < 2^31
  const int n = g / Q;
  if (n >= N) return;
  const int q = g - n * Q;
  const int64_t b = bidx[n];
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (batch_ok(b, B)) {
    const float2 p = pos[n];
    const GridCorners c = grid_corners(p.x, p.y, Hg, Wg, sxw, syh, scale != 0);
    const float4* f = fcl + b * ((int64_t)Hg * Wg) * Q + q;
    const float4 a = f[(int64_t)c.o00 * Q], e = f[(int64_t)c.o01 * Q], h = f[(int64_t)c.o10 * Q],
                 k = f[(int64_t)c.o11 * Q];
    v = make_float4(corner_sum(a.x, e.x, h.x, k.x, c), corner_sum(a.y, e.y, h.y, k.y, c),
                    corner_sum(a.z, e.z, h.z, k.z, c), corner_sum(a.w, e.w, h.w, k.w, c));
  }
  float* o = out + (int64_t)n * C + 4 * q;
  if ((C & 3) == 0) {
    *(float4*)o = v;
  } else {
    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (4 * q + j < C) o[j] = vv[j];
  }
}

// Position gradient: one lane per (event, channel quad) as in the forward, so the field and gout reads of an
// event are consecutive 16-byte pieces; each lane forms its four channel terms and the event's first lane adds
// all of them in channel order, as the plane kernel does (same bits).
// With gd set (the trajectory model, B-spline basis, C = 2K): the gradient rows are formed from the displacement's
// gradient gd and the event time tt (k_traj_gout's values) instead of read.
__global__ void __launch_bounds__(kBlock) k_sample_grid_bwd_pos_cl(const float* __restrict__ gout,
                                                                   const float4* __restrict__ fcl, int64_t B, int C,
                                                                   int Q, int Hg, int Wg,
                                                                   const float2* __restrict__ pos,
                                                                   const int64_t* __restrict__ bidx, int64_t N,
                                                                   float sxw, float syh, int scale,
                                                                   float2* __restrict__ gpos,
                                                                   const float2* __restrict__ gd,
                                                                   const float* __restrict__ tt) {
  const int lane = threadIdx.x & (kWave - 1);
  const int epw = kWave / Q;                     // events per wave
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int e = lane / Q, q = lane - e * Q;
  const int64_t n = wave * epw + e;
  const bool live = e < epw && n < N;
  float tx[4] = {0.f, 0.f, 0.f, 0.f}, ty[4] = {0.f, 0.f, 0.f, 0.f};
  bool ok = false, inx = false, iny = false;
  float kx = 1.f, ky = 1.f;
  if (live) {
    const int64_t b = bidx[n];
    ok = batch_ok(b, B);
    if (ok) {
      const float2 p = pos[n];
      float gx = p.x, gy = p.y;
      if (scale) {
        gx = p.x / sxw * (float)(Wg - 1);
        gy = p.y / syh * (float)(Hg - 1);
        kx = (float)(Wg - 1) / sxw;
        ky = (float)(Hg - 1) / syh;
      }
      inx = gx >= 0.f && gx <= (float)(Wg - 1);
      iny = gy >= 0.f && gy <= (float)(Hg - 1);
      const GridCorners c = grid_corners(p.x, p.y, Hg, Wg, sxw, syh, scale != 0);
      const float ax = c.ax, ay = c.ay;
      const float4* f = fcl + b * ((int64_t)Hg * Wg) * Q + q;
      const float4 a = f[(int64_t)c.o00 * Q], h0 = f[(int64_t)c.o01 * Q], h1 = f[(int64_t)c.o10 * Q],
                   k1 = f[(int64_t)c.o11 * Q];
      const float f00[4] = {a.x, a.y, a.z, a.w}, f01[4] = {h0.x, h0.y, h0.z, h0.w},
                  f10[4] = {h1.x, h1.y, h1.z, h1.w}, f11[4] = {k1.x, k1.y, k1.z, k1.w};
      float go[4];
      if (gd) {
        float nb[4];
        const int K = C / 2;
        const int j = bspline_nonzero_rt(tt[n], K, nb);
        const float2 d = gd[n];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) go[jj] = 4 * q + jj < C ? bspline_row(4 * q + jj, K, j, nb, d) : 0.f;
      } else if ((C & 3) == 0) {
        const float* go_row = gout + n * C;
        const float4 g4 = *(const float4*)(go_row + 4 * q);
        go[0] = g4.x;
        go[1] = g4.y;
        go[2] = g4.z;
        go[3] = g4.w;
      } else {
        const float* go_row = gout + n * C;
#pragma unroll
        for (int j = 0; j < 4; ++j) go[j] = 4 * q + j < C ? go_row[4 * q + j] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        tx[j] = go[j] * ((1.f - ay) * (f01[j] - f00[j]) + ay * (f11[j] - f10[j]));
        ty[j] = go[j] * ((1.f - ax) * (f10[j] - f00[j]) + ax * (f11[j] - f01[j]));
      }
    }
  }
  // the event's first lane adds the terms of channels 0 .. C-1 in order (every lane takes part in the shuffles)
  float sx = 0.f, sy = 0.f;
  for (int i = 0; i < Q; ++i) {
    const int src = min(lane + i, kWave - 1);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float ox = __shfl(tx[j], src), oy = __shfl(ty[j], src);
      if (4 * i + j < C) {
        sx += ox;
        sy += oy;
      }
    }
  }
  if (live && q == 0) {
    if (ok) {
      sx = inx ? sx * kx : 0.f;
      sy = iny ? sy * ky : 0.f;
    } else {
      sx = 0.f;
      sy = 0.f;
    }
    gpos[n] = make_float2(sx, sy);
  }
}

// ------------------------------------------------------------------------------ trajectory displacement
// d(p, t) = sum_k c_k(p) g_k(t) of a coefficient grid with channels [y_1..y_K, x_1..x_K] (the displacement of
// atl/motion/trajectories.py: the coefficients are the bilinear border-clamped sample at p, k = 1..K).  Bases:
//   0  polynomial  g_k(t) = t^k
//   1  Bernstein   g_k(t) = binom(K, k) t^k (1 - t)^(K - k)            (degree K, control point 0 pinned to p)
//   2  B-spline    g_k(t) = N_k(t), the clamped uniform B-spline basis of degree P = min(3, K) with K + 1
//                  functions N_0..N_K on [0, 1] (L = K + 1 - P equal spans); N_0 belongs to the pinned start
//                  p, and N_k(0) = 0 for k >= 1, so g_k(t) - g_k(0) = N_k(t).
// One pass per event instead of the (N, 2K) coefficient rows and the products and sums over them.  The powers
// are repeated products (torch's pow rounds differently by a few ulps) and the k sum runs in order.
constexpr int kTrajMaxK = 16;

__host__ __device__ constexpr int binom_int(int n, int k) {   // exact for n <= 16
  int r = 1;
  for (int i = 1; i <= k; ++i) r = r * (n - k + i) / i;
  return r;
}

// The nonzero B-spline functions at t: N_{j..j+P}(t) in nb[0..P] for the span j = clamp(floor(t L), 0, L - 1)
// (outside [0, 1] the end span's polynomial continues), by the triangular Cox-de Boor recursion (Piegl and
// Tiller, The NURBS Book, algorithm A2.2) on the knots u_i = clamp(i - P, 0, L) / L.  Every denominator is at
// least one span wide.
template <int K>
__device__ __forceinline__ int bspline_nonzero(float t, float (&nb)[(K < 3 ? K : 3) + 1]) {
  constexpr int P = K < 3 ? K : 3, L = K + 1 - P;
  const float fl = (float)L;
  const int j = min(max((int)floorf(t * fl), 0), L - 1);
  auto knot = [&](int i) { return (float)min(max(i - P, 0), L) / fl; };
  float left[P + 1], right[P + 1];
  nb[0] = 1.f;
#pragma unroll
  for (int d = 1; d <= P; ++d) {
    left[d] = t - knot(j + P + 1 - d);
    right[d] = knot(j + P + d) - t;
    float saved = 0.f;
#pragma unroll
    for (int r = 0; r < d; ++r) {
      const float tmp = nb[r] / (right[r + 1] + left[d - r]);
      nb[r] = saved + right[r + 1] * tmp;
      saved = left[d - r] * tmp;
    }
    nb[d] = saved;
  }
  return j;
}

template <int K>
__device__ __forceinline__ void traj_basis(float t, int basis, float (&g)[K]) {
  float tk = 1.f;
  if (basis == 0) {
#pragma unroll
    for (int k = 1; k <= K; ++k) {
      tk = tk * t;
      g[k - 1] = tk;
    }
    return;
  }
  if (basis == 2) {
    constexpr int P = K < 3 ? K : 3;
    float nb[P + 1];
    const int j = bspline_nonzero<K>(t, nb);
#pragma unroll
    for (int k = 1; k <= K; ++k) {               // g_k = N_k = nb[k - j] if 0 <= k - j <= P (register selects)
      float v = 0.f;
#pragma unroll
      for (int r = 0; r <= P; ++r) v = k - j == r ? nb[r] : v;
      g[k - 1] = v;
    }
    return;
  }
  const float u = 1.f - t;
  float pw[K];                                   // pw[m] = u^m by repeated products
  pw[0] = 1.f;
#pragma unroll
  for (int m = 1; m < K; ++m) pw[m] = pw[m - 1] * u;
#pragma unroll
  for (int k = 1; k <= K; ++k) {
    tk = tk * t;
    g[k - 1] = (float)binom_int(K, k) * tk * pw[K - k];
  }
}

// One lane per (event, channel quad), the Q = ceil(2K/4) lanes of an event side by side in one wave (64 / Q
// events per wave, the remaining lanes idle): the lanes of an event read the same corner's channels in
// consecutive 16-byte pieces, and the event's first lane adds the Q partial sums.
template <int K>
__global__ void __launch_bounds__(kBlock) k_traj_displacement(const float4* __restrict__ fcl, int64_t B, int Hg,
                                                              int Wg, const float2* __restrict__ gpos,
                                                              const int64_t* __restrict__ bidx,
                                                              const float* __restrict__ t, int basis, int64_t N,
                                                              float2* __restrict__ out) {
  constexpr int C = 2 * K, Q = (C + 3) / 4, EPW = kWave / Q;   // events per wave
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int e = lane / Q, q = lane - e * Q;
  const int64_t n = wave * EPW + e;
  const bool live = e < EPW && n < N;
  float dx = 0.f, dy = 0.f;
  int64_t b = -1;
  if (live) b = bidx[n];
  if (live && batch_ok(b, B)) {
    const float2 p = gpos[n];
    const GridCorners c = grid_corners(p.x, p.y, Hg, Wg, 1.f, 1.f, false);
    float g[K];
    traj_basis<K>(t[n], basis, g);
    const float4* f = fcl + b * ((int64_t)Hg * Wg) * Q + q;
    const float4 a = f[(int64_t)c.o00 * Q], h0 = f[(int64_t)c.o01 * Q], h1 = f[(int64_t)c.o10 * Q],
                 k1 = f[(int64_t)c.o11 * Q];
    const float v[4] = {corner_sum(a.x, h0.x, h1.x, k1.x, c), corner_sum(a.y, h0.y, h1.y, k1.y, c),
                        corner_sum(a.z, h0.z, h1.z, k1.z, c), corner_sum(a.w, h0.w, h1.w, k1.w, c)};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ch = 4 * q + j;
      if (ch >= C) break;
      const int k = ch < K ? ch : ch - K;
      float gk = 0.f;
#pragma unroll
      for (int kk = 0; kk < K; ++kk) gk = kk == k ? g[kk] : gk;   // register select, no indexed private array
      if (ch < K)
        dy = dy + v[j] * gk;
      else
        dx = dx + v[j] * gk;
    }
  }
  // the event's first lane adds its other lanes' sums (every lane takes part in the shuffles)
  float sx = dx, sy = dy;
#pragma unroll
  for (int i = 1; i < Q; ++i) {
    const int src = min(lane + i, kWave - 1);
    const float ox = __shfl(dx, src), oy = __shfl(dy, src);
    if (q + i < Q) {
      sx = sx + ox;
      sy = sy + oy;
    }
  }
  if (live && q == 0) out[n] = make_float2(sx, sy);
}

// The exposure correction of atl/objectives/ats.py:31-50 for PixelTrajectories in one pass: anchor i's trajectory
// start p (n_fp Picard steps p <- xa - d(p, t_a) from p = xa, as PixelTrajectories.origin), its coefficients
// looked up once at p, the trajectory evaluated at the n_check bin centres, y = p + d(p, c_k), and k_visible's
// weighted share of the centres where y is inside the sensor.  Lanes as in k_traj_displacement (Q per anchor, one
// channel quad each) and the same sums in the same order, so every p and y equals the composed ops' bits.  Grid
// coordinates of a pixel position: (p - off) / tile (tile 1: p itself).  The basis at the anchor's time is
// evaluated once, and at the bin centres once per workgroup into LDS (the same function: the same values).
constexpr int kVisMaxCheck = 64;

template <int K>
__global__ void __launch_bounds__(kBlock) k_traj_visible(const float4* __restrict__ fcl, int64_t B, int Hg, int Wg,
                                                         const float2* __restrict__ xa,
                                                         const float* __restrict__ ta,
                                                         const int64_t* __restrict__ bidx, int basis, int64_t M,
                                                         int n_fp, float off, float tile,
                                                         const float* __restrict__ counts,
                                                         const float* __restrict__ centres, int n_check, float tau,
                                                         float wmax, float hmax, float* __restrict__ out) {
  constexpr int C = 2 * K, Q = (C + 3) / 4, EPW = kWave / Q;   // anchors per wave
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int e = lane / Q, q = lane - e * Q;
  const int64_t n = wave * EPW + e;
  const bool live = e < EPW && n < M;
  const int lead = min(e * Q, kWave - 1);        // the anchor's first lane
  int64_t b = -1;
  float2 x0 = make_float2(0.f, 0.f);
  float t = 0.f;
  if (live) {
    b = bidx[n];
    x0 = xa[n];
    t = ta[n];
  }
  const bool ok = live && batch_ok(b, B);
  const float4* f = fcl + (ok ? b : 0) * ((int64_t)Hg * Wg) * Q + q;
  __shared__ float gcs[kVisMaxCheck * K];        // basis at the bin centres, centre-major
  const bool table = n_check <= kVisMaxCheck;
  if (table) {
    for (int i = threadIdx.x; i < n_check; i += blockDim.x) {
      float gc[K];
      traj_basis<K>(centres[i], basis, gc);
#pragma unroll
      for (int k = 0; k < K; ++k) gcs[i * K + k] = gc[k];
    }
  }
  __syncthreads();
  float gt[K];                                   // basis at the anchor's own time
  traj_basis<K>(t, basis, gt);
  // this lane's quad of the coefficients at grid coordinates of pixel position p: v[4]
  auto lookup = [&](float2 p, float (&v)[4]) {
    const float gx = tile == 1.f ? p.x : (p.x - off) / tile, gy = tile == 1.f ? p.y : (p.y - off) / tile;
    const GridCorners c = grid_corners(gx, gy, Hg, Wg, 1.f, 1.f, false);
    const float4 a = f[(int64_t)c.o00 * Q], h0 = f[(int64_t)c.o01 * Q], h1 = f[(int64_t)c.o10 * Q],
                 k1 = f[(int64_t)c.o11 * Q];
    v[0] = corner_sum(a.x, h0.x, h1.x, k1.x, c);
    v[1] = corner_sum(a.y, h0.y, h1.y, k1.y, c);
    v[2] = corner_sum(a.z, h0.z, h1.z, k1.z, c);
    v[3] = corner_sum(a.w, h0.w, h1.w, k1.w, c);
  };
  // d = sum_k c_k g_k(tt) from this lane's quad v, combined over the anchor's lanes in lane order (the event's
  // first lane adds the others' sums, k_traj_displacement's order), returned to every lane of the anchor
  // gsel(k) = g_k at the time in question (k = 0 .. K-1)
  auto disp = [&](const float (&v)[4], auto&& gsel) {
    float dx = 0.f, dy = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int ch = 4 * q + j;
      if (ch >= C) break;
      const int k = ch < K ? ch : ch - K;
      const float gk = gsel(k);
      if (ch < K)
        dy = dy + v[j] * gk;
      else
        dx = dx + v[j] * gk;
    }
    float sx = dx, sy = dy;
#pragma unroll
    for (int i = 1; i < Q; ++i) {
      const int src = min(lane + i, kWave - 1);
      const float ox = __shfl(dx, src), oy = __shfl(dy, src);
      if (q + i < Q) {
        sx = sx + ox;
        sy = sy + oy;
      }
    }
    return make_float2(__shfl(sx, lead), __shfl(sy, lead));
  };
  auto own = [&](int k) {                        // register select, no indexed private array
    float gk = 0.f;
#pragma unroll
    for (int kk = 0; kk < K; ++kk) gk = kk == k ? gt[kk] : gk;
    return gk;
  };
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  float2 p = x0;
  for (int it = 0; it < n_fp; ++it) {            // p <- xa - d(p, t_a)
    if (ok) lookup(p, v);
    const float2 d = disp(v, own);                // every lane takes part in the shuffles
    if (ok) p = make_float2(x0.x - d.x, x0.y - d.y);
  }
  if (ok) lookup(p, v);
  float vis = 0.f, tot = 0.f;
  const float* cnt = counts + (ok ? b : 0) * n_check;
  for (int k = 0; k < n_check; ++k) {
    const float c = centres[k];
    float2 d;                                     // every lane takes part in the shuffles
    if (table) {
      d = disp(v, [&](int kk) { return gcs[k * K + kk]; });
    } else {
      float gc[K];
      traj_basis<K>(c, basis, gc);
      d = disp(v, [&](int kk) {
        float gk = 0.f;
#pragma unroll
        for (int k2 = 0; k2 < K; ++k2) gk = k2 == kk ? gc[k2] : gk;
        return gk;
      });
    }
    if (!ok) continue;
    const float yx = p.x + d.x, yy = p.y + d.y;
    const float near = fabsf(t - c) <= tau ? 1.f : 0.f;
    const float inside = (yx >= 0.f && yx <= wmax && yy >= 0.f && yy <= hmax) ? 1.f : 0.f;
    const float w = cnt[k] * near;
    vis = vis + w * inside;
    tot = tot + w;
  }
  if (live && q == 0) out[n] = fmaxf(vis / fmaxf(tot, 1.f), 1e-3f);
}

// PixelTrajectories.origin's n_fp Picard steps p <- xy - d(p, t) from p = xy in one pass (atl/motion/
// trajectories.py:68-73): lanes as in k_traj_displacement (Q per event, one channel quad each) and its sums in
// its order, so every step equals the composed ops' bits.  P (n_fp x N, may be null) receives the grid
// coordinates (p - off) / tile of each step's p, where the displacement is taken (the backward's positions),
// and row n_fp those of the returned p when P holds n_fp + 1 rows (final = 1).
template <int K>
__global__ void __launch_bounds__(kBlock) k_traj_origin(const float4* __restrict__ fcl, int64_t B, int Hg, int Wg,
                                                        const float2* __restrict__ xy, const float* __restrict__ tt,
                                                        const int64_t* __restrict__ bidx, int basis, int64_t N,
                                                        int n_fp, float off, float tile, float2* __restrict__ P,
                                                        int final, float2* __restrict__ out) {
  constexpr int C = 2 * K, Q = (C + 3) / 4, EPW = kWave / Q;   // events per wave
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int e = lane / Q, q = lane - e * Q;
  const int64_t n = wave * EPW + e;
  const bool live = e < EPW && n < N;
  int64_t b = -1;
  float2 x0 = make_float2(0.f, 0.f);
  float t = 0.f;
  if (live) {
    b = bidx[n];
    x0 = xy[n];
    t = tt[n];
  }
  const bool ok = live && batch_ok(b, B);
  const float4* f = fcl + (ok ? b : 0) * ((int64_t)Hg * Wg) * Q + q;
  float g[K];
  traj_basis<K>(t, basis, g);
  float2 p = x0;
  for (int it = 0; it < n_fp; ++it) {
    const float gx = tile == 1.f ? p.x : (p.x - off) / tile, gy = tile == 1.f ? p.y : (p.y - off) / tile;
    if (P && live && q == 0) P[(int64_t)it * N + n] = make_float2(gx, gy);
    float dx = 0.f, dy = 0.f;
    if (ok) {
      const GridCorners c = grid_corners(gx, gy, Hg, Wg, 1.f, 1.f, false);
      const float4 a = f[(int64_t)c.o00 * Q], h0 = f[(int64_t)c.o01 * Q], h1 = f[(int64_t)c.o10 * Q],
                   k1 = f[(int64_t)c.o11 * Q];
      const float v[4] = {corner_sum(a.x, h0.x, h1.x, k1.x, c), corner_sum(a.y, h0.y, h1.y, k1.y, c),
                          corner_sum(a.z, h0.z, h1.z, k1.z, c), corner_sum(a.w, h0.w, h1.w, k1.w, c)};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ch = 4 * q + j;
        if (ch >= C) break;
        const int k = ch < K ? ch : ch - K;
        float gk = 0.f;
#pragma unroll
        for (int kk = 0; kk < K; ++kk) gk = kk == k ? g[kk] : gk;
        if (ch < K)
          dy = dy + v[j] * gk;
        else
          dx = dx + v[j] * gk;
      }
    }
    float sx = dx, sy = dy;                       // the event's first lane adds the others' sums, in lane order
#pragma unroll
    for (int i = 1; i < Q; ++i) {
      const int src = min(lane + i, kWave - 1);
      const float ox = __shfl(dx, src), oy = __shfl(dy, src);
      if (q + i < Q) {
        sx = sx + ox;
        sy = sy + oy;
      }
    }
    const int lead = min(e * Q, kWave - 1);
    sx = __shfl(sx, lead);
    sy = __shfl(sy, lead);
    p = make_float2(x0.x - sx, x0.y - sy);        // invalid batch: d = 0, p stays xy
  }
  if (live && q == 0) {
    out[n] = p;
    if (P && final)
      P[(int64_t)n_fp * N + n] = make_float2(tile == 1.f ? p.x : (p.x - off) / tile, tile == 1.f ? p.y : (p.y - off) / tile);
  }
}

// The steps' backward of k_traj_origin (B-spline basis) in one pass: for k = n_fp - 1 .. 0, the gradient g of
// p_{k+1} = xy - d(p_k, t) gives the step's displacement gradient gD_k = -g (written to gD, n_fp x N, for the
// coefficient-grid accumulation), gxy += g, and, through d's position derivative at the step's grid coordinates
// P[k] (k_sample_grid_bwd_pos_cl's terms and order, rows formed from gD_k and t), the gradient of p_k divided by
// tile; p_0 = xy adds the last one to gxy.  gxy (N,2) may be null: then the k = 0 position derivative is skipped.
template <int K>
__global__ void __launch_bounds__(kBlock) k_traj_origin_bwd(const float4* __restrict__ fcl, int64_t B, int Hg,
                                                            int Wg, const float2* __restrict__ P,
                                                            const float* __restrict__ tt,
                                                            const int64_t* __restrict__ bidx, int64_t N, int n_fp,
                                                            float tile, const float2* __restrict__ gp,
                                                            float2* __restrict__ gD, float2* __restrict__ gxy) {
  constexpr int C = 2 * K, Q = (C + 3) / 4, EPW = kWave / Q;   // events per wave
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kWave;
  const int e = lane / Q, q = lane - e * Q;
  const int64_t n = wave * EPW + e;
  const bool live = e < EPW && n < N;
  const int lead = min(e * Q, kWave - 1);
  int64_t b = -1;
  float2 g = make_float2(0.f, 0.f);
  float t = 0.f;
  if (live) {
    b = bidx[n];
    g = gp[n];
    t = tt[n];
  }
  const bool ok = live && batch_ok(b, B);
  const float4* f = fcl + (ok ? b : 0) * ((int64_t)Hg * Wg) * Q + q;
  float nb[4];
  const int js = bspline_nonzero_rt(t, K, nb);
  float2 acc = make_float2(0.f, 0.f);
  for (int k = n_fp - 1; k >= 0; --k) {
    const float2 d = make_float2(-g.x, -g.y);
    if (live && q == 0) gD[(int64_t)k * N + n] = d;
    acc = make_float2(acc.x + g.x, acc.y + g.y);
    if (k == 0 && !gxy) break;                     // uniform: gxy is a kernel argument
    float tx[4] = {0.f, 0.f, 0.f, 0.f}, ty[4] = {0.f, 0.f, 0.f, 0.f};
    bool inx = false, iny = false;
    if (ok) {
      const float2 pk = P[(int64_t)k * N + n];
      inx = pk.x >= 0.f && pk.x <= (float)(Wg - 1);
      iny = pk.y >= 0.f && pk.y <= (float)(Hg - 1);
      const GridCorners c = grid_corners(pk.x, pk.y, Hg, Wg, 1.f, 1.f, false);
      const float ax = c.ax, ay = c.ay;
      const float4 a = f[(int64_t)c.o00 * Q], h0 = f[(int64_t)c.o01 * Q], h1 = f[(int64_t)c.o10 * Q],
                   k1 = f[(int64_t)c.o11 * Q];
      const float f00[4] = {a.x, a.y, a.z, a.w}, f01[4] = {h0.x, h0.y, h0.z, h0.w},
                  f10[4] = {h1.x, h1.y, h1.z, h1.w}, f11[4] = {k1.x, k1.y, k1.z, k1.w};
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float go = 4 * q + jj < C ? bspline_row(4 * q + jj, K, js, nb, d) : 0.f;
        tx[jj] = go * ((1.f - ay) * (f01[jj] - f00[jj]) + ay * (f11[jj] - f10[jj]));
        ty[jj] = go * ((1.f - ax) * (f10[jj] - f00[jj]) + ax * (f11[jj] - f01[jj]));
      }
    }
    float sx = 0.f, sy = 0.f;                      // the event's first lane adds channels 0 .. C-1 in order
    for (int i = 0; i < Q; ++i) {
      const int src = min(lane + i, kWave - 1);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float ox = __shfl(tx[jj], src), oy = __shfl(ty[jj], src);
        if (4 * i + jj < C) {
          sx += ox;
          sy += oy;
        }
      }
    }
    sx = ok && inx ? sx : 0.f;
    sy = ok && iny ? sy : 0.f;
    sx = __shfl(sx, lead);
    sy = __shfl(sy, lead);
    g = tile == 1.f ? make_float2(sx, sy) : make_float2(sx / tile, sy / tile);
    if (k == 0) acc = make_float2(acc.x + g.x, acc.y + g.y);   // p_0 = xy
  }
  if (gxy && live && q == 0) gxy[n] = acc;
}

// The displacement's output gradient per coefficient channel: gout[n, c] = g_k(t_n) * gd_n.y for c = k - 1 < K and
// g_k(t_n) * gd_n.x for c = K + k - 1, the rows that the field adjoint and the position gradient of the sampler
// take.  One lane per (event, channel quad), so the rows are written by consecutive lanes.
template <int K>
__global__ void __launch_bounds__(kBlock) k_traj_gout(const float2* __restrict__ gd, const float* __restrict__ t,
                                                      int basis, int N, float* __restrict__ gout) {
  constexpr int C = 2 * K, Q = (C + 3) / 4;
  const int gl = blockIdx.x * blockDim.x + threadIdx.x;   // N * Q < 2^31
  const int n = gl / Q;
  if (n >= N) return;
  const int q = gl - n * Q;
  float g[K];
  traj_basis<K>(t[n], basis, g);
  const float2 d = gd[n];
  float* o = gout + (int64_t)n * C;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int ch = 4 * q + j;
    if (ch >= C) break;
    const int k = ch < K ? ch : ch - K;
    float gk = 0.f;
#pragma unroll
    for (int kk = 0; kk < K; ++kk) gk = kk == k ? g[kk] : gk;   // register select, no indexed private array
    o[ch] = gk * (ch < K ? d.y : d.x);
  }
}

bool dims_ok(int64_t H, int64_t W) { return H > 0 && W > 0 && H * W < (int64_t)1 << 31; }

// ------------------------------------------------------------------------------------------- event noise
// Philox4x32-10 (Salmon, Moraes, Dror, Shaw: "Parallel random numbers: as easy as 1, 2, 3", SC 2011): a
// counter-based generator, so every event draws its own four words from (its index, the call's offset) under
// the seed, in any order and without state.
struct U4 {
  uint32_t x, y, z, w;
};

__device__ __forceinline__ U4 philox4x32_10(U4 c, uint32_t k0, uint32_t k1) {
  constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u, kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t hi0 = __umulhi(kM0, c.x), lo0 = kM0 * c.x;
    const uint32_t hi1 = __umulhi(kM1, c.z), lo1 = kM1 * c.z;
    c = U4{hi1 ^ c.y ^ k0, lo1, hi0 ^ c.w ^ k1, lo0};
    k0 += kW0;
    k1 += kW1;
  }
  return c;
}

// Dequantisation and anchor smoothing noise of the anchored score (atl/objectives/ats.py:79-84 draws them with
// torch.rand / torch.randn): xs = xy + U(-1/2, 1/2)^2 if dequantize, else xy; xa = xs + h N(0, 1)^2 (Box-Muller
// on the other two words) if xa is given.  One pass over the events instead of two fills and two adds.
__global__ void __launch_bounds__(kBlock) k_event_noise(const float2* __restrict__ xy, int64_t N, uint32_t s0,
                                                        uint32_t s1, uint32_t o0, uint32_t o1, float h,
                                                        int dequantize, float2* __restrict__ xs,
                                                        float2* __restrict__ xa) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const U4 r = philox4x32_10(U4{(uint32_t)n, (uint32_t)(n >> 32), o0, o1}, s0, s1);
  constexpr float k24 = 1.f / 16777216.f;          // 24-bit mantissa fractions
  float2 p = xy[n];
  if (dequantize) {
    p.x = p.x + ((float)(r.x >> 8) * k24 - 0.5f);
    p.y = p.y + ((float)(r.y >> 8) * k24 - 0.5f);
  }
  xs[n] = p;
  if (xa) {
    const float u1 = (float)((r.z >> 8) + 1u) * k24;   // (0, 1]: log finite
    const float u2 = (float)(r.w >> 8) * k24;          // [0, 1)
    const float rad = sqrtf(-2.f * logf(u1));
    float sn, cs;
    sincospif(2.f * u2, &sn, &cs);
    xa[n] = make_float2(p.x + h * (rad * cs), p.y + h * (rad * sn));
  }
}


// Per-image mean and unbiased variance of B images of n pixels each: the IWE contrast of
// atl/objectives/cmax.py:23-25, iwe.var(dim=(-2, -1)), whose library reduction over 4 outputs of 307k pixels
// each ran in one workgroup per output.  Pass 1: workgroup (image b, chunk c) sums x and x^2 over its kVarChunk
// pixels in fp64 into part[2 (b nch + c) + {0, 1}]; pass 2: one wave per image adds its chunks' sums in a fixed
// order and writes mean = S1 / n and var = max(S2 - S1 mean, 0) / (n - 1) (NaN for n = 1, as torch.var).
constexpr int kVarItems = 16;
constexpr int kVarChunk = kVarItems * kBlock;   // pixels per workgroup of pass 1

__global__ void __launch_bounds__(kBlock) k_image_var_part(const float* __restrict__ img, int64_t n, int nch,
                                                           double* __restrict__ part) {
  __shared__ double red[2][kBlock / kWave];
  const int b = blockIdx.x / nch, c = blockIdx.x - b * nch;
  const float* __restrict__ x = img + (int64_t)b * n;
  const int64_t p0 = (int64_t)c * kVarChunk + threadIdx.x;
  float v[kVarItems];
#pragma unroll
  for (int k = 0; k < kVarItems; ++k) {            // all loads in flight
    const int64_t p = p0 + (int64_t)k * kBlock;
    v[k] = p < n ? x[p] : 0.f;
  }
  double s1 = 0.0, s2 = 0.0;
#pragma unroll
  for (int k = 0; k < kVarItems; ++k) {
    const double d = v[k];
    s1 += d;
    s2 += d * d;
  }
  s1 = wave_sum(s1);
  s2 = wave_sum(s2);
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) {
    red[0][w] = s1;
    red[1][w] = s2;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double t1 = 0.0, t2 = 0.0;
    for (int i = 0; i < kBlock / kWave; ++i) {
      t1 += red[0][i];
      t2 += red[1][i];
    }
    part[2 * (int64_t)blockIdx.x] = t1;
    part[2 * (int64_t)blockIdx.x + 1] = t2;
  }
}

__global__ void __launch_bounds__(kWave) k_image_var_fin(const double* __restrict__ part, int nch, int64_t n,
                                                         float* __restrict__ mean, float* __restrict__ var) {
  const int64_t base = 2 * (int64_t)blockIdx.x * nch;
  double s1 = 0.0, s2 = 0.0;
  for (int c = threadIdx.x; c < nch; c += kWave) {
    s1 += part[base + 2 * c];
    s2 += part[base + 2 * c + 1];
  }
  s1 = wave_sum(s1);
  s2 = wave_sum(s2);
  if (threadIdx.x == 0) {
    const double m = s1 / (double)n;
    mean[blockIdx.x] = (float)m;
    var[blockIdx.x] = n > 1 ? (float)(fmax(s2 - s1 * m, 0.0) / (double)(n - 1)) : __builtin_nanf("");
  }
}

// Its backward (the autograd of torch.var): gimg[b, p] = gvar[b] * 2 (img[b, p] - mean[b]) / (n - 1).
__global__ void __launch_bounds__(kBlock) k_image_var_bwd(const float* __restrict__ img,
                                                          const float* __restrict__ mean,
                                                          const float* __restrict__ gvar, int64_t n, int64_t total,
                                                          float* __restrict__ gimg) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t b = i / n;
  gimg[i] = gvar[b] * (2.f / (float)(n - 1)) * (img[i] - mean[b]);
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

int atl_sample_grid_bwd_pos(const float* gout, const float* field, int64_t B, int64_t C, int64_t Hg, int64_t Wg,
                            const float* pos, const int64_t* b, int64_t N, int64_t img_h, int64_t img_w, float* gpos,
                            hipStream_t stream) {
  if (N < 0 || B < 0 || C < 1 || Hg < 1 || Wg < 1 || !dims_ok(Hg, Wg)) { set_error("sample_grid_bwd_pos: bad sizes"); return 1; }
  if (N == 0) return 0;
  const int scale = img_h > 0 && img_w > 0;
  const float sxw = (float)(img_w - 1 > 1 ? img_w - 1 : 1), syh = (float)(img_h - 1 > 1 ? img_h - 1 : 1);
  hipLaunchKernelGGL(k_sample_grid_bwd_pos, dim3(grid_for(N)), dim3(kBlock), 0, stream, gout, field, B, (int)C,
                     (int)Hg, (int)Wg, (const float2*)pos, b, N, sxw, syh, scale, (float2*)gpos);
  return check_launch("sample_grid_bwd_pos");
}

int atl_field_channels_last(const float* field, int64_t B, int64_t C, int64_t Hg, int64_t Wg, float* out,
                            hipStream_t stream) {
  if (B < 0 || C < 1 || !dims_ok(Hg, Wg) || C > (int64_t)1 << 20) { set_error("field_channels_last: bad sizes"); return 1; }
  const int64_t Q = (C + 3) / 4, total = B * Hg * Wg * Q;
  if (total == 0) return 0;
  if (!field || !out) { set_error("field_channels_last: null pointer"); return 1; }
  hipLaunchKernelGGL(k_field_channels_last, dim3(grid_for(total)), dim3(kBlock), 0, stream, field, (int)C, (int)Q,
                     Hg * Wg, total, (float4*)out);
  return check_launch("field_channels_last");
}

int atl_flow_interleave(const float* field, int64_t B, int64_t Hg, int64_t Wg, float* out, hipStream_t stream) {
  if (B < 0 || !dims_ok(Hg, Wg)) { set_error("flow_interleave: bad sizes"); return 1; }
  const int64_t total = B * Hg * Wg;
  if (total == 0) return 0;
  if (!field || !out) { set_error("flow_interleave: null pointer"); return 1; }
  hipLaunchKernelGGL(k_flow_interleave, dim3(grid_for(total)), dim3(kBlock), 0, stream, field, Hg * Wg, total,
                     (float2*)out);
  return check_launch("flow_interleave");
}

int atl_sample_flow_il(const float* field_il, int64_t B, int64_t Hg, int64_t Wg, const float* pos, const int64_t* b,
                       int64_t N, int64_t img_h, int64_t img_w, float* out, hipStream_t stream) {
  if (N < 0 || B < 0 || !dims_ok(Hg, Wg) || Wg < 2) { set_error("sample_flow_il: bad sizes (Wg >= 2)"); return 1; }
  if (N == 0) return 0;
  if (!field_il || !pos || !b || !out) { set_error("sample_flow_il: null pointer"); return 1; }
  const int scale = img_h > 0 && img_w > 0;
  const float sxw = (float)(img_w - 1 > 1 ? img_w - 1 : 1), syh = (float)(img_h - 1 > 1 ? img_h - 1 : 1);
  hipLaunchKernelGGL(k_sample_flow_il, dim3(grid_for(N)), dim3(kBlock), 0, stream, field_il, B, (int)Hg, (int)Wg,
                     (const float2*)pos, b, N, sxw, syh, scale, (float2*)out);
  return check_launch("sample_flow_il");
}

int atl_sample_grid_fwd_cl(const float* field_cl, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                           const int64_t* b, int64_t N, int64_t img_h, int64_t img_w, float* out,
                           hipStream_t stream) {
  if (N < 0 || B < 0 || C < 1 || C > (int64_t)1 << 20 || !dims_ok(Hg, Wg)) { set_error("sample_grid_fwd_cl: bad sizes"); return 1; }
  const int64_t Q = (C + 3) / 4;
  if (N * Q >= ((int64_t)1 << 31) - kBlock) { set_error("sample_grid_fwd_cl: N * ceil(C/4) must stay below 2^31"); return 1; }
  if (N == 0) return 0;
  if ((reinterpret_cast<uintptr_t>(field_cl) & 15) || ((C & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 15))) {
    set_error("sample_grid_fwd_cl: field_cl (and out when C % 4 == 0) must be 16-byte aligned");
    return 1;
  }
  const int scale = img_h > 0 && img_w > 0;
  const float sxw = (float)(img_w - 1 > 1 ? img_w - 1 : 1), syh = (float)(img_h - 1 > 1 ? img_h - 1 : 1);
  hipLaunchKernelGGL(k_sample_grid_fwd_cl, dim3(grid_for(N * Q)), dim3(kBlock), 0, stream,
                     (const float4*)field_cl, B, (int)C, (int)Q, (int)Hg, (int)Wg, (const float2*)pos, b, (int)N,
                     sxw, syh, scale, out);
  return check_launch("sample_grid_fwd_cl");
}

int atl_sample_grid_bwd_pos_cl(const float* gout, const float* field_cl, int64_t B, int64_t C, int64_t Hg,
                               int64_t Wg, const float* pos, const int64_t* b, int64_t N, int64_t img_h,
                               int64_t img_w, float* gpos, hipStream_t stream) {
  if (N < 0 || B < 0 || C < 1 || C > (int64_t)1 << 20 || !dims_ok(Hg, Wg)) { set_error("sample_grid_bwd_pos_cl: bad sizes"); return 1; }
  if (N == 0) return 0;
  if ((reinterpret_cast<uintptr_t>(field_cl) & 15) || ((C & 3) == 0 && (reinterpret_cast<uintptr_t>(gout) & 15))) {
    set_error("sample_grid_bwd_pos_cl: field_cl (and gout when C % 4 == 0) must be 16-byte aligned");
    return 1;
  }
  const int scale = img_h > 0 && img_w > 0;
  const float sxw = (float)(img_w - 1 > 1 ? img_w - 1 : 1), syh = (float)(img_h - 1 > 1 ? img_h - 1 : 1);
  const int64_t Q = (C + 3) / 4;
  if (Q > kWave) { set_error("sample_grid_bwd_pos_cl: at most %d channels", 4 * kWave); return 1; }
  const int64_t waves = (N + kWave / Q - 1) / (kWave / Q);
  hipLaunchKernelGGL(k_sample_grid_bwd_pos_cl, dim3(grid_for(waves * kWave)), dim3(kBlock), 0, stream, gout,
                     (const float4*)field_cl, B, (int)C, (int)Q, (int)Hg, (int)Wg, (const float2*)pos, b, N, sxw, syh,
                     scale, (float2*)gpos, (const float2*)nullptr, (const float*)nullptr);
  return check_launch("sample_grid_bwd_pos_cl");
}

int atl_traj_pos_bwd_cl(const float* gd, const float* t, int64_t K, const float* field_cl, int64_t B, int64_t Hg,
                        int64_t Wg, const float* gpos_in, const int64_t* b, int64_t N, float* gpos, hipStream_t stream) {
  if (N < 0 || B < 0 || K < 1 || K > kTrajMaxK || !dims_ok(Hg, Wg)) { set_error("traj_pos_bwd_cl: bad sizes (1 <= K <= %d)", kTrajMaxK); return 1; }
  if (N == 0) return 0;
  if (!gd || !t || !field_cl || !gpos_in || !b || !gpos) { set_error("traj_pos_bwd_cl: null argument"); return 1; }
  if (reinterpret_cast<uintptr_t>(field_cl) & 15) { set_error("traj_pos_bwd_cl: field_cl must be 16-byte aligned"); return 1; }
  const int64_t C = 2 * K, Q = (C + 3) / 4;
  const int64_t waves = (N + kWave / Q - 1) / (kWave / Q);
  hipLaunchKernelGGL(k_sample_grid_bwd_pos_cl, dim3(grid_for(waves * kWave)), dim3(kBlock), 0, stream,
                     (const float*)nullptr, (const float4*)field_cl, B, (int)C, (int)Q, (int)Hg, (int)Wg,
                     (const float2*)gpos_in, b, N, 1.f, 1.f, 0, (float2*)gpos, (const float2*)gd, t);
  return check_launch("traj_pos_bwd_cl");
}

int atl_traj_displacement(const float* field_cl, int64_t B, int64_t C, int64_t K, int64_t Hg, int64_t Wg,
                          const float* gpos, const int64_t* b, const float* t, int64_t N, int64_t basis, float* out,
                          hipStream_t stream) {
  if (N < 0 || B < 0 || K < 1 || K > kTrajMaxK || !dims_ok(Hg, Wg) || basis < 0 || basis > 2) {
    set_error("traj_displacement: bad sizes (1 <= K <= %d, basis 0, 1 or 2)", kTrajMaxK);
    return 1;
  }
  if (C != 2 * K) { set_error("traj_displacement: the coefficient grid has %lld channels, expected 2K = %lld", (long long)C, (long long)(2 * K)); return 1; }
  if (N == 0) return 0;
  if (!field_cl || !gpos || !b || !t || !out) { set_error("traj_displacement: null argument"); return 1; }
  if (reinterpret_cast<uintptr_t>(field_cl) & 15) { set_error("traj_displacement: field_cl must be 16-byte aligned"); return 1; }
  const int64_t Q = (2 * K + 3) / 4, waves = (N + kWave / Q - 1) / (kWave / Q);
  const dim3 grid(grid_for(waves * kWave)), block(kBlock);
  const float4* f = (const float4*)field_cl;
  const float2* p = (const float2*)gpos;
  float2* o = (float2*)out;
  const int bs = (int)basis;
  switch (K) {
#define ATL_TRAJ_CASE(k) \
    case k: hipLaunchKernelGGL(k_traj_displacement<k>, grid, block, 0, stream, f, B, (int)Hg, (int)Wg, p, b, t, bs, N, o); break;
    ATL_TRAJ_CASE(1) ATL_TRAJ_CASE(2) ATL_TRAJ_CASE(3) ATL_TRAJ_CASE(4) ATL_TRAJ_CASE(5) ATL_TRAJ_CASE(6)
    ATL_TRAJ_CASE(7) ATL_TRAJ_CASE(8) ATL_TRAJ_CASE(9) ATL_TRAJ_CASE(10) ATL_TRAJ_CASE(11) ATL_TRAJ_CASE(12)
    ATL_TRAJ_CASE(13) ATL_TRAJ_CASE(14) ATL_TRAJ_CASE(15) ATL_TRAJ_CASE(16)
#undef ATL_TRAJ_CASE
  }
  return check_launch("traj_displacement");
}

int atl_traj_origin(const float* field_cl, int64_t B, int64_t C, int64_t K, int64_t Hg, int64_t Wg, const float* xy,
                    const float* t, const int64_t* b, int64_t N, int64_t n_fp, double offset, int64_t tile,
                    int64_t basis, float* P, int64_t final_row, float* out, hipStream_t stream) {
  if (N < 0 || B < 0 || K < 1 || K > kTrajMaxK || !dims_ok(Hg, Wg) || basis < 0 || basis > 2 || n_fp < 0 ||
      tile < 1) {
    set_error("traj_origin: bad sizes (1 <= K <= %d, basis 0, 1 or 2)", kTrajMaxK);
    return 1;
  }
  if (C != 2 * K) { set_error("traj_origin: the coefficient grid has %lld channels, expected 2K = %lld", (long long)C, (long long)(2 * K)); return 1; }
  if (N == 0) return 0;
  if (!field_cl || !xy || !t || !b || !out) { set_error("traj_origin: null argument"); return 1; }
  if (reinterpret_cast<uintptr_t>(field_cl) & 15) { set_error("traj_origin: field_cl must be 16-byte aligned"); return 1; }
  const int64_t Q = (2 * K + 3) / 4, waves = (N + kWave / Q - 1) / (kWave / Q);
  const dim3 grid(grid_for(waves * kWave)), block(kBlock);
  const float4* f = (const float4*)field_cl;
  const int bs = (int)basis;
  switch (K) {
#define ATL_TRAJ_CASE(k) \
    case k: hipLaunchKernelGGL(k_traj_origin<k>, grid, block, 0, stream, f, B, (int)Hg, (int)Wg, (const float2*)xy, t, \
                               b, bs, N, (int)n_fp, (float)offset, (float)tile, (float2*)P, final_row ? 1 : 0, \
                               (float2*)out); break;
    ATL_TRAJ_CASE(1) ATL_TRAJ_CASE(2) ATL_TRAJ_CASE(3) ATL_TRAJ_CASE(4) ATL_TRAJ_CASE(5) ATL_TRAJ_CASE(6)
    ATL_TRAJ_CASE(7) ATL_TRAJ_CASE(8) ATL_TRAJ_CASE(9) ATL_TRAJ_CASE(10) ATL_TRAJ_CASE(11) ATL_TRAJ_CASE(12)
    ATL_TRAJ_CASE(13) ATL_TRAJ_CASE(14) ATL_TRAJ_CASE(15) ATL_TRAJ_CASE(16)
#undef ATL_TRAJ_CASE
  }
  return check_launch("traj_origin");
}

int atl_traj_origin_bwd(const float* field_cl, int64_t B, int64_t C, int64_t K, int64_t Hg, int64_t Wg,
                        const float* P, const float* t, const int64_t* b, int64_t N, int64_t n_fp, int64_t tile,
                        const float* gp, float* gD, float* gxy, hipStream_t stream) {
  if (N < 0 || B < 0 || K < 3 || K > kTrajMaxK || !dims_ok(Hg, Wg) || n_fp < 1 || tile < 1) {
    set_error("traj_origin_bwd: bad sizes (3 <= K <= %d, n_fp >= 1)", kTrajMaxK);
    return 1;
  }
  if (C != 2 * K) { set_error("traj_origin_bwd: the coefficient grid has %lld channels, expected 2K = %lld", (long long)C, (long long)(2 * K)); return 1; }
  if (N == 0) return 0;
  if (!field_cl || !P || !t || !b || !gp || !gD) { set_error("traj_origin_bwd: null argument"); return 1; }
  if (reinterpret_cast<uintptr_t>(field_cl) & 15) { set_error("traj_origin_bwd: field_cl must be 16-byte aligned"); return 1; }
  const int64_t Q = (2 * K + 3) / 4, waves = (N + kWave / Q - 1) / (kWave / Q);
  const dim3 grid(grid_for(waves * kWave)), block(kBlock);
  const float4* f = (const float4*)field_cl;
  switch (K) {
#define ATL_TRAJ_CASE(k) \
    case k: hipLaunchKernelGGL(k_traj_origin_bwd<k>, grid, block, 0, stream, f, B, (int)Hg, (int)Wg, (const float2*)P, \
                               t, b, N, (int)n_fp, (float)tile, (const float2*)gp, (float2*)gD, (float2*)gxy); break;
    ATL_TRAJ_CASE(3) ATL_TRAJ_CASE(4) ATL_TRAJ_CASE(5) ATL_TRAJ_CASE(6) ATL_TRAJ_CASE(7) ATL_TRAJ_CASE(8)
    ATL_TRAJ_CASE(9) ATL_TRAJ_CASE(10) ATL_TRAJ_CASE(11) ATL_TRAJ_CASE(12) ATL_TRAJ_CASE(13) ATL_TRAJ_CASE(14)
    ATL_TRAJ_CASE(15) ATL_TRAJ_CASE(16)
#undef ATL_TRAJ_CASE
  }
  return check_launch("traj_origin_bwd");
}

int atl_traj_visible(const float* field_cl, int64_t B, int64_t C, int64_t K, int64_t Hg, int64_t Wg, const float* xa,
                     const float* ta, const int64_t* ba, int64_t M, int64_t n_fp, double offset, int64_t tile,
                     int64_t basis, const float* counts, const float* centres, int64_t n_check, double tau,
                     int64_t H, int64_t W, float* out, hipStream_t stream) {
  if (M < 0 || B < 0 || K < 1 || K > kTrajMaxK || !dims_ok(Hg, Wg) || basis < 0 || basis > 2 || n_fp < 0 ||
      n_check < 1 || tile < 1 || H < 1 || W < 1) {
    set_error("traj_visible: bad sizes (1 <= K <= %d, basis 0, 1 or 2)", kTrajMaxK);
    return 1;
  }
  if (C != 2 * K) { set_error("traj_visible: the coefficient grid has %lld channels, expected 2K = %lld", (long long)C, (long long)(2 * K)); return 1; }
  if (M == 0) return 0;
  if (!field_cl || !xa || !ta || !ba || !counts || !centres || !out) { set_error("traj_visible: null argument"); return 1; }
  if (reinterpret_cast<uintptr_t>(field_cl) & 15) { set_error("traj_visible: field_cl must be 16-byte aligned"); return 1; }
  const int64_t Q = (2 * K + 3) / 4, waves = (M + kWave / Q - 1) / (kWave / Q);
  const dim3 grid(grid_for(waves * kWave)), block(kBlock);
  const float4* f = (const float4*)field_cl;
  const float2* p = (const float2*)xa;
  const int bs = (int)basis;
  switch (K) {
#define ATL_TRAJ_CASE(k) \
    case k: hipLaunchKernelGGL(k_traj_visible<k>, grid, block, 0, stream, f, B, (int)Hg, (int)Wg, p, ta, ba, bs, M, \
                               (int)n_fp, (float)offset, (float)tile, counts, centres, (int)n_check, (float)tau, \
                               (float)(W - 1), (float)(H - 1), out); break;
    ATL_TRAJ_CASE(1) ATL_TRAJ_CASE(2) ATL_TRAJ_CASE(3) ATL_TRAJ_CASE(4) ATL_TRAJ_CASE(5) ATL_TRAJ_CASE(6)
    ATL_TRAJ_CASE(7) ATL_TRAJ_CASE(8) ATL_TRAJ_CASE(9) ATL_TRAJ_CASE(10) ATL_TRAJ_CASE(11) ATL_TRAJ_CASE(12)
    ATL_TRAJ_CASE(13) ATL_TRAJ_CASE(14) ATL_TRAJ_CASE(15) ATL_TRAJ_CASE(16)
#undef ATL_TRAJ_CASE
  }
  return check_launch("traj_visible");
}

int atl_traj_gout(const float* gd, const float* t, int64_t N, int64_t K, int64_t basis, float* gout,
                  hipStream_t stream) {
  if (N < 0 || K < 1 || K > kTrajMaxK || basis < 0 || basis > 2) {
    set_error("traj_gout: bad sizes (1 <= K <= %d, basis 0, 1 or 2)", kTrajMaxK);
    return 1;
  }
  const int64_t Q = (2 * K + 3) / 4;
  if (N * Q >= ((int64_t)1 << 31) - kBlock) { set_error("traj_gout: N * ceil(K/2) must stay below 2^31"); return 1; }
  if (N == 0) return 0;
  if (!gd || !t || !gout) { set_error("traj_gout: null argument"); return 1; }
  const dim3 grid(grid_for(N * Q)), block(kBlock);
  const float2* g = (const float2*)gd;
  const int bs = (int)basis, n = (int)N;
  switch (K) {
#define ATL_TRAJ_CASE(k) case k: hipLaunchKernelGGL(k_traj_gout<k>, grid, block, 0, stream, g, t, bs, n, gout); break;
    ATL_TRAJ_CASE(1) ATL_TRAJ_CASE(2) ATL_TRAJ_CASE(3) ATL_TRAJ_CASE(4) ATL_TRAJ_CASE(5) ATL_TRAJ_CASE(6)
    ATL_TRAJ_CASE(7) ATL_TRAJ_CASE(8) ATL_TRAJ_CASE(9) ATL_TRAJ_CASE(10) ATL_TRAJ_CASE(11) ATL_TRAJ_CASE(12)
    ATL_TRAJ_CASE(13) ATL_TRAJ_CASE(14) ATL_TRAJ_CASE(15) ATL_TRAJ_CASE(16)
#undef ATL_TRAJ_CASE
  }
  return check_launch("traj_gout");
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

int atl_event_noise(const float* xy, int64_t N, uint64_t seed, uint64_t offset, double h, int dequantize, float* xs,
                    float* xa, hipStream_t stream) {
  if (N < 0 || (N > 0 && (!xy || !xs)) || !(h >= 0) || !(h < 1e30)) { set_error("event_noise: bad arguments"); return 1; }
  if (N == 0) return 0;
  hipLaunchKernelGGL(k_event_noise, dim3(grid_for(N)), dim3(kBlock), 0, stream, (const float2*)xy, N,
                     (uint32_t)seed, (uint32_t)(seed >> 32), (uint32_t)offset, (uint32_t)(offset >> 32), (float)h,
                     dequantize, (float2*)xs, (float2*)xa);
  return check_launch("event_noise");
}

int64_t atl_image_variance_ws_bytes(int64_t B, int64_t n) {
  if (B < 0 || n < 1) return -1;
  return B * ((n + kVarChunk - 1) / kVarChunk) * 2 * (int64_t)sizeof(double);
}

int atl_image_variance(const float* img, int64_t B, int64_t n, float* mean, float* var, void* ws, int64_t ws_bytes,
                       hipStream_t stream) {
  const int64_t need = atl_image_variance_ws_bytes(B, n);
  if (need < 0 || B * ((n + kVarChunk - 1) / kVarChunk) >= ((int64_t)1 << 31)) { set_error("image_variance: bad sizes B=%lld n=%lld", (long long)B, (long long)n); return 1; }
  if (B == 0) return 0;
  if (!img || !mean || !var || !ws) { set_error("image_variance: null argument"); return 1; }
  if (ws_bytes < need) { set_error("image_variance: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)need); return 1; }
  const int nch = (int)((n + kVarChunk - 1) / kVarChunk);
  hipLaunchKernelGGL(k_image_var_part, dim3((unsigned)(B * nch)), dim3(kBlock), 0, stream, img, n, nch, (double*)ws);
  hipLaunchKernelGGL(k_image_var_fin, dim3((unsigned)B), dim3(kWave), 0, stream, (const double*)ws, nch, n, mean, var);
  return check_launch("image_variance");
}

int atl_image_variance_bwd(const float* img, const float* mean, const float* gvar, int64_t B, int64_t n, float* gimg,
                           hipStream_t stream) {
  if (B < 0 || n < 1) { set_error("image_variance_bwd: bad sizes B=%lld n=%lld", (long long)B, (long long)n); return 1; }
  if (B == 0) return 0;
  if (!img || !mean || !gvar || !gimg) { set_error("image_variance_bwd: null argument"); return 1; }
  hipLaunchKernelGGL(k_image_var_bwd, dim3(grid_for(B * n)), dim3(kBlock), 0, stream, img, mean, gvar, n, B * n, gimg);
  return check_launch("image_variance_bwd");
}

}  // extern "C"
