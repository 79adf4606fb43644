// Clamped uniform B-spline basis of the trajectory model with the number of functions K known at run time
// (the kernels whose channel count is a run-time value use it): the same fp32 operations, in the same order, as
// the compile-time bspline_nonzero<K> of events.hip, so that both give the same bits.  Degree P = min(3, K),
// L = K + 1 - P knot intervals on [0, 1]; nb[0..P] are the non-zero basis values N_j .. N_{j+P} at t and j is
// returned.  The files that include this header are built with -ffp-contract=off.
#pragma once
#include "common.h"

namespace atlhip {

__device__ __forceinline__ int bspline_nonzero_rt(float t, int K, float (&nb)[4]) {
  const int P = K < 3 ? K : 3, L = K + 1 - P;
  const float fl = (float)L;
  const int j = min(max((int)floorf(t * fl), 0), L - 1);
  auto knot = [&](int i) { return (float)min(max(i - P, 0), L) / fl; };
  float left[4], right[4];
  nb[0] = 1.f;
  nb[1] = nb[2] = nb[3] = 0.f;
#pragma unroll
  for (int d = 1; d <= 3; ++d) {
    if (d > P) break;
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

// bspline_nonzero_rt with the knots read from a table: knots[c] = (float)c / (float)L for c = 0..L, the same
// correctly rounded quotients the division gives, so the same bits at six fewer divisions per call.
__device__ __forceinline__ int bspline_nonzero_tab(float t, int K, const float* knots, float (&nb)[4]) {
  const int P = K < 3 ? K : 3, L = K + 1 - P;
  const float fl = (float)L;
  const int j = min(max((int)floorf(t * fl), 0), L - 1);
  auto knot = [&](int i) { return knots[min(max(i - P, 0), L)]; };
  float left[4], right[4];
  nb[0] = 1.f;
  nb[1] = nb[2] = nb[3] = 0.f;
#pragma unroll
  for (int d = 1; d <= 3; ++d) {
    if (d > P) break;
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

// The displacement's gradient row of channel ch (k_traj_gout): g_k(t) * (ch < K ? gd.y : gd.x), k = ch mod K,
// g_k = N_{k+1} = nb[k + 1 - j] when 0 <= k + 1 - j <= P, else 0.
__device__ __forceinline__ float bspline_row(int ch, int K, int j, const float (&nb)[4], float2 gd) {
  const int k = ch < K ? ch : ch - K;
  const int r = k + 1 - j;
  const int P = K < 3 ? K : 3;
  float gk = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) gk = (r == i && i <= P) ? nb[i] : gk;   // register selects
  return gk * (ch < K ? gd.y : gd.x);
}

}  // namespace atlhip
