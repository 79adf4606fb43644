// Bilinear corner helpers shared by the per-event kernels and the tile engine: the in-image corners of the
// splat and gather (csrc/atl_cpu.cpp:17-33) and the border-clamped flow-grid corners of DenseLinearFlow
// (atl/motion/parametric.py:212-216, 235-251).  Every expression keeps the reference's fp32 order; the files
// that include this header are built with -ffp-contract=off.
#pragma once
#include "common.h"

namespace atlhip {

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

// DenseLinearFlow.field + sample_grid (atl/motion/parametric.py:212-216, 235-251): grid coordinates
// gx = x / sx * (Wg - 1) with sx = max(W - 1, 1) (when `scale` is set; raw grid coordinates otherwise),
// border clamp, corners (y0, x0) .. (y1, x1) with x0 <= Wg - 2, fixed sum order c00 + c01 + c10 + c11.
struct GridCorners {
  int o00, o01, o10, o11;      // offsets inside one (Hg, Wg) plane
  float w00, w01, w10, w11;
  float ax, ay;                // gx - x0, gy - y0
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
  c.ax = ax;
  c.ay = ay;
  return c;
}

}  // namespace atlhip
