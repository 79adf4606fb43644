// Device-wide exclusive scans of int32 counts shared by the plan builders: scan32 (two launches: per-tile
// totals, then a per-tile rescan that first sums the totals of the tiles before its own; tiles of
// kScanTile = 2048 counts) and scan_small (up to 16384 counts in one workgroup).
#pragma once
#include "common.h"

namespace atlhip {
namespace {   // one private copy per translation unit that includes this header

constexpr int kScanItems = 8;
constexpr int kScanTile = kBlock * kScanItems;

inline int64_t scan_tiles(int64_t n) { return (n + kScanTile - 1) / kScanTile; }

__global__ void __launch_bounds__(kBlock) k_scan32_reduce(const int* __restrict__ in, int64_t n,
                                                          int* __restrict__ part) {
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

// out[i + 1] = sum(in[0..i]), out[0] = 0.  part holds the tile totals; each block adds up those of the tiles
// before its own (a few thousand at most: cheaper than a launch of its own).
__global__ void __launch_bounds__(kBlock) k_scan32_write(const int* __restrict__ in, int64_t n,
                                                         const int* __restrict__ part, int* __restrict__ out) {
  __shared__ int lds[kBlock / kWave + 1];
  int pre = 0;
  for (int64_t i = threadIdx.x; i < (int64_t)blockIdx.x; i += kBlock) pre += part[i];
  int offset;
  block_exclusive_scan<kBlock>(pre, lds, offset);
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
  int run = offset + excl;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    run += vals[k];
    if (base + k < n) out[base + k + 1] = run;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) out[0] = 0;
}

// Launches the two passes; `part` holds scan_tiles(n) ints (callers reserve one more).  n >= 1.
inline void scan32(const int* in, int64_t n, int* part, int* out, hipStream_t stream) {
  const int64_t tiles = scan_tiles(n);
  hipLaunchKernelGGL(k_scan32_reduce, dim3((unsigned)tiles), dim3(kBlock), 0, stream, in, n, part);
  hipLaunchKernelGGL(k_scan32_write, dim3((unsigned)tiles), dim3(kBlock), 0, stream, in, n, (const int*)part, out);
}

// The same scan of a key-major sequence (element key * nblk + blk) whose counts are stored block-major
// (in[blk * nkeys + key]): histogram blocks write their rows of counts coalesced, and the scan reads them
// transposed (reads of scattered words are cheap next to writes of scattered words).  out is key-major.
__device__ __forceinline__ void scan32t_load(const int* __restrict__ in, int nkeys, int nblk, int64_t base, int64_t n,
                                             int (&vals)[kScanItems]) {
  int key = (int)(base / nblk), blk = (int)(base - (int64_t)key * nblk);
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    vals[k] = base + k < n ? in[(int64_t)blk * nkeys + key] : 0;
    if (++blk == nblk) {
      blk = 0;
      ++key;
    }
  }
}

__global__ void __launch_bounds__(kBlock) k_scan32t_reduce(const int* __restrict__ in, int nkeys, int nblk, int64_t n,
                                                           int* __restrict__ part) {
  __shared__ int lds[kBlock / kWave + 1];
  const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
  int vals[kScanItems];
  scan32t_load(in, nkeys, nblk, base, n, vals);
  int s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) s += vals[k];
  int total;
  block_exclusive_scan<kBlock>(s, lds, total);
  if (threadIdx.x == 0) part[blockIdx.x] = total;
}

__global__ void __launch_bounds__(kBlock) k_scan32t_write(const int* __restrict__ in, int nkeys, int nblk, int64_t n,
                                                          const int* __restrict__ part, int* __restrict__ out) {
  __shared__ int lds[kBlock / kWave + 1];
  int pre = 0;
  for (int64_t i = threadIdx.x; i < (int64_t)blockIdx.x; i += kBlock) pre += part[i];
  int offset;
  block_exclusive_scan<kBlock>(pre, lds, offset);
  const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
  int vals[kScanItems];
  scan32t_load(in, nkeys, nblk, base, n, vals);
  int s = 0;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) s += vals[k];
  int total;
  const int excl = block_exclusive_scan<kBlock>(s, lds, total);
  int run = offset + excl;
#pragma unroll
  for (int k = 0; k < kScanItems; ++k) {
    run += vals[k];
    if (base + k < n) out[base + k + 1] = run;
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) out[0] = 0;
}

inline void scan32t(const int* in, int nkeys, int nblk, int* part, int* out, hipStream_t stream) {
  const int64_t n = (int64_t)nkeys * nblk;
  const int64_t tiles = scan_tiles(n);
  hipLaunchKernelGGL(k_scan32t_reduce, dim3((unsigned)tiles), dim3(kBlock), 0, stream, in, nkeys, nblk, n, part);
  hipLaunchKernelGGL(k_scan32t_write, dim3((unsigned)tiles), dim3(kBlock), 0, stream, in, nkeys, nblk, n,
                     (const int*)part, out);
}

// Exclusive scan of n <= kScanSmallMax counts (bucket or tile totals) into their start positions: one
// workgroup, one launch.
constexpr int kScanSmallBlock = 1024;
constexpr int kScanSmallMax = 16384;

__global__ void __launch_bounds__(kScanSmallBlock) k_scan_small(const int* __restrict__ tot, int n,
                                                                int* __restrict__ pos) {
  __shared__ int wsum[kScanSmallBlock / kWave + 1];
  constexpr int kPer = kScanSmallMax / kScanSmallBlock;
  int v[kPer];
  int s = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = threadIdx.x * kPer + k;
    v[k] = i < n ? tot[i] : 0;
    s += v[k];
  }
  int total;
  int run = block_exclusive_scan<kScanSmallBlock>(s, wsum, total);
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = threadIdx.x * kPer + k;
    if (i < n) pos[i] = run;
    run += v[k];
  }
}

inline void scan_small(const int* tot, int n, int* pos, hipStream_t stream) {
  hipLaunchKernelGGL(k_scan_small, dim3(1), dim3(kScanSmallBlock), 0, stream, tot, n, pos);
}

}  // namespace
}  // namespace atlhip
