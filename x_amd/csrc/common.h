// Shared device helpers and error plumbing for the atl HIP library (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

namespace atlhip {

constexpr int kWave = 64;
constexpr int kBlock = 256;

// Last error message of this thread's most recent failing entry point (returned by atl_last_error()).
void set_error(const char* fmt, ...);

inline unsigned grid_for(int64_t n, int per_block = kBlock) {
  const int64_t g = (n + per_block - 1) / per_block;
  return (unsigned)(g < 1 ? 1 : g);
}

// Returns 0, or records the launch error and returns 1.
int check_launch(const char* what);

// ---------------------------------------------------------------------------------------------- device
// Order-preserving map of a float to a signed int (for atomic min/max of floats of any sign).
__device__ __forceinline__ int float_to_ordered(float f) {
  int i = __float_as_int(f);
  return i >= 0 ? i : i ^ 0x7fffffff;
}

template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}

__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = max(v, __shfl_xor(v, d, kWave));
  return v;
}

__device__ __forceinline__ int wave_min_i(int v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = min(v, __shfl_xor(v, d, kWave));
  return v;
}

// Exclusive scan of one int per thread over a block of BS threads.  `lds` holds BS/64 + 1 ints.
template <int BS>
__device__ __forceinline__ int block_exclusive_scan(int v, int* lds, int& total) {
  const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
  int x = v;
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int y = __shfl_up(x, d, kWave);
    if (lane >= d) x += y;
  }
  if (lane == kWave - 1) lds[wid] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < BS / kWave; ++w) {
      const int t = lds[w];
      lds[w] = run;
      run += t;
    }
    lds[BS / kWave] = run;
  }
  __syncthreads();
  const int excl = x - v + lds[wid];
  total = lds[BS / kWave];
  __syncthreads();
  return excl;
}

}  // namespace atlhip
