// Tile-binned accumulation of per-event contributions into an image or a flow grid, without per-corner
// global atomics: the bilinear splat forward (csrc/atl_cpu.cpp:38-56), the image gradient of the bilinear
// gather (csrc/atl_cpu.cpp:151-172) and the adjoint of the flow-grid lookup (atl/motion/parametric.py:235-251).
//
// Device-wide float atomics are resolved in the memory fabric on this multi-XCD part and run at ~25 G/s when
// scattered, and events concentrated on edges put many of them on the same pixels.  Here every call:
//   1. bins the events by the 16x16 (or 32x32) tile of their base corner: an LDS histogram per block of 4096
//      events, a device scan, and a scatter of 16-byte records (x, y, value, event index) into tile order;
//   2. cuts every tile's records into chunks (a one-workgroup scan over the tiles lists them), one per
//      workgroup, which adds the weighted contributions into an LDS copy of the (T+1) x (T+1) pixels the tile's
//      events reach (corners reach one past the tile): with LDS float atomics (scatter form, chunks of 512), or,
//      for the bilinear modes, by sorting the records by base corner in LDS and summing per corner (gather
//      form, chunks of 512, or of 2048 on crowded tiles);
//   3. flushes every non-zero LDS pixel with one global atomic add (neighbouring tiles share their border row
//      and column, and a crowded tile spans several ranges, so the flush stays atomic; it costs at most
//      (T+1)^2 atomics per tile segment).
// Corner indices and weights are computed exactly as by the per-event kernels (same fp32 expressions), so the
// set of touched pixels is identical; only the order of the float additions differs.
// The coefficient-grid adjoint of the trajectory look-ups (atl_traj_field_bwd) bins its records with their
// gradients and times (no gathers by event index), accumulates in registers per base node (no float atomics
// into LDS, which are slow on this part) and flushes a tile held by one workgroup without global atomics: its
// own nodes in place, its border row and column through a halo buffer added by a second small kernel.
#include "common.h"
#include "scan.h"
#include "bilinear.h"
#include "traj.h"
#include "../../include/atl_hip.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <mutex>

using namespace atlhip;

namespace {

constexpr int kTilePerBlock = 4096;              // binning: events per block
constexpr int kTileBinBlock = 1024;              // binning: threads per block (4 events each)
constexpr int kTileMaxKeys = 16384;              // LDS histogram capacity (tiles over all batches)
constexpr int kAccBlock = 256;                   // accumulation: threads per tile
constexpr int kMaxChannels = 32;                 // field channels of the tile adjoint (LDS: C x 17 x 17 floats)

enum { kImage = 0, kGrid = 1, kGauss = 2, kVoxel = 3, kGridVal = 4, kImageG = 5 };

// Events per binning block by mode: the voxel grid's binning keeps twice as many blocks in flight (1M events:
// 490 blocks of 2048 instead of 245 of 4096; 0.11 against 0.16 ms per voxel grid), which the image and flow
// modes of the IWE pipeline do not gain (their count matrix and scans grow with the block count).
constexpr int kTilePerBlockVoxel = 2048;
__host__ __device__ constexpr int tile_per_block(int mode) { return mode == kVoxel ? kTilePerBlockVoxel : kTilePerBlock; }
// kGridVal: kGrid with the values in the records; kImageG: kImage records (x, y, w, index) accumulating the
// per-event value gout[index] instead of w (the gather's image gradient on the splat's records)
constexpr int kMaxGaussRadius = 8;               // truncated-Gaussian splats of larger radius stay per event

struct TileGeo {
  int B, H, W;               // image (kImage) or grid (kGrid) extent
  int T;                     // tile edge
  int TX, TY, nkeys;         // tiles per row and column, B * TY * TX
  int N, nblk;
  int mode;
  int C;                     // kGrid: channels of the field
  int R;                     // kGauss: splat radius (pixels around round(pos))
  float inv2s2, norm;        // kGauss: 1 / (2 sigma^2), 1 / (2 pi sigma^2)
  int scale;                 // kGrid: positions are image pixels mapped by sxw, syh
  float sxw, syh;
  int vec4;                  // kGrid: C % 4 == 0 and gout 16-byte aligned (rows read as float4)
  int ilv;                   // flush: element 2 p + 1 of out for output element p when ilv = 2 (the odd
                             // slots of an interleaved (value, gradient) image), element p otherwise
};

__device__ __forceinline__ bool batch_ok(int64_t b, int64_t B) { return b >= 0 && b < B; }

// kImage: base corner (floor(x), floor(y)) and the in-image test of csrc/atl_cpu.cpp:17-33 (the corners
// themselves are re-tested one by one when they are added).
__device__ __forceinline__ bool image_base(float x, float y, int H, int W, int& x0, int& y0) {
  const float fx = floorf(x), fy = floorf(y);
  if (!(fx >= -1.f && fx <= (float)(W - 1) && fy >= -1.f && fy <= (float)(H - 1))) return false;
  x0 = (int)fx;
  y0 = (int)fy;
  return true;
}

// kGrid: border-clamped grid corners of atl/motion/parametric.py:235-251 (x0 <= Wg - 2, x1 = min(x0 + 1, Wg - 1)).
struct GridCell {
  int x0, y0, x1, y1;
  float ax, ay;
};

__device__ __forceinline__ GridCell grid_cell(float x, float y, int Hg, int Wg, float sxw, float syh, bool scale) {
  float gx = x, gy = y;
  if (scale) {
    gx = x / sxw * (float)(Wg - 1);
    gy = y / syh * (float)(Hg - 1);
  }
  gx = fminf(fmaxf(gx, 0.f), (float)(Wg - 1));
  gy = fminf(fmaxf(gy, 0.f), (float)(Hg - 1));
  if (gx != gx) gx = 0.f;
  if (gy != gy) gy = 0.f;
  const float fx0 = fminf(floorf(gx), (float)max(Wg - 2, 0));
  const float fy0 = fminf(floorf(gy), (float)max(Hg - 2, 0));
  GridCell c;
  c.ax = gx - fx0;
  c.ay = gy - fy0;
  c.x0 = (int)fx0;
  c.y0 = (int)fy0;
  c.x1 = min(c.x0 + 1, Wg - 1);
  c.y1 = min(c.y0 + 1, Hg - 1);
  return c;
}

// kGauss: centre (round(x), round(y)) of a truncated Gaussian splat and the test of csrc/atl_cpu.cpp:79-104
// (its window of radius R must meet the image).
__device__ __forceinline__ bool gauss_centre(float x, float y, const TileGeo& g, int& cx, int& cy) {
  const float rx = roundf(x), ry = roundf(y);
  if (!(rx >= (float)(-g.R) && rx <= (float)(g.W - 1 + g.R) && ry >= (float)(-g.R) && ry <= (float)(g.H - 1 + g.R)))
    return false;
  cx = (int)rx;
  cy = (int)ry;
  return true;
}

// Tile key of event n (-1: contributes nothing) and its LDS origin.
template <int MODE>
__device__ __forceinline__ int tile_key(float x, float y, int64_t b, const TileGeo& g) {
  if (!batch_ok(b, g.B)) return -1;
  int tx, ty;
  if (MODE == kImage || MODE == kVoxel) {
    int x0, y0;
    if (!image_base(x, y, g.H, g.W, x0, y0)) return -1;
    tx = (x0 + 1) / g.T;
    ty = (y0 + 1) / g.T;
  } else if (MODE == kGauss) {
    int cx, cy;
    if (!gauss_centre(x, y, g, cx, cy)) return -1;
    tx = (cx + g.R) / g.T;
    ty = (cy + g.R) / g.T;
  } else {                                         // kGrid, kGridVal
    const GridCell c = grid_cell(x, y, g.H, g.W, g.sxw, g.syh, g.scale != 0);
    tx = c.x0 / g.T;
    ty = c.y0 / g.T;
  }
  return ((int)b * g.TY + ty) * g.TX + tx;
}

// Chunks of the tile-ordered records: every non-empty tile is cut into chunks of at most `chunk` records, and
// chunk w gets info[w] = (tile, first record, end record, 1 if the tile has more than one chunk); crowded tiles
// (more than 32 * chunk records, where the flushes of many chunks would pile up on the same pixels) take chunks
// of `crowd` records; nchunk[0] = the number of chunks.  One workgroup of NT threads: thread i takes the tiles
// i, i + NT, ... (a run of crowded neighbouring tiles is spread over many threads, each writing its own tile's
// chunks), so the scan of the chunk counts runs in rounds of NT tiles.  It runs as a launch of its own
// (k_tile_chunks) or as one extra workgroup of the pass that places the records (after the scan that fixed the
// tiles' offsets, so the list is ready when the records are).
struct ChunkList {
  int4* info;
  int* nchunk;
  int chunk, crowd;
};

template <int NT>
__device__ __forceinline__ void tile_chunks_body(const int* __restrict__ boff, const TileGeo& g, ChunkList cl) {
  static_assert(kTileMaxKeys % NT == 0, "whole rounds of tiles");
  __shared__ int wsum[NT / kWave + 1];
  constexpr int kPer = kTileMaxKeys / NT;
  const int rounds = (g.nkeys + NT - 1) / NT;
  int r0[kPer], r1[kPer];                         // record range of this thread's tile of every round
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int t = k * NT + threadIdx.x;
    r0[k] = k < rounds ? boff[min(t, g.nkeys) * g.nblk] : 0;
    r1[k] = k < rounds ? boff[min(t + 1, g.nkeys) * g.nblk] : 0;
  }
  int base = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    if (k >= rounds) break;
    const int t = k * NT + threadIdx.x;
    const int len = r1[k] - r0[k];
    const int cs = len > 32 * cl.chunk ? cl.crowd : cl.chunk;
    const int n = t < g.nkeys ? (len + cs - 1) / cs : 0;
    int total;
    const int c = base + block_exclusive_scan<NT>(n, wsum, total);
    const bool crowded = n > kWave / 8;           // a crowded tile's chunks are written by its whole wave
    if (!crowded)
      for (int q = 0; q < n; ++q)
        cl.info[c + q] = make_int4(t, r0[k] + q * cs, min(r0[k] + (q + 1) * cs, r1[k]), n > 1);
    for (uint64_t m = __ballot(crowded); m; m &= m - 1) {
      const int src = __ffsll((unsigned long long)m) - 1;
      const int tt = __shfl(t, src), cc = __shfl(c, src), a0 = __shfl(r0[k], src), a1 = __shfl(r1[k], src);
      const int nn = __shfl(n, src), ss = __shfl(cs, src);
      for (int q = threadIdx.x & (kWave - 1); q < nn; q += kWave)
        cl.info[cc + q] = make_int4(tt, a0 + q * ss, min(a0 + (q + 1) * ss, a1), nn > 1);
    }
    base += total;
  }
  if (threadIdx.x == 0) *cl.nchunk = base;
}

// Binning.  SCATTER = false: per-block tile histogram into cnt[block * nkeys + key] (rows written coalesced; the
// scan reads them transposed, key-major).  SCATTER = true: the block's scanned offsets (boff[key * nblk + block])
// are loaded into LDS and every event writes (x, y, value, index) to its slot; kVoxel
// writes (x, y, polarity, t * (C - 1)) (aux = t) and skips events whose time bins both miss [0, C).  Events of
// value zero are skipped unless SKIP_ZERO is false (records whose index also serves a second accumulation).
// SCATTER with a launch of nblk + 1 workgroups: the last one writes the chunk list `cl` instead.
template <int MODE, bool SCATTER, bool SKIP_ZERO = true>
__global__ void __launch_bounds__(kTileBinBlock) k_tile_bin(const float2* __restrict__ pos,
                                                            const int64_t* __restrict__ bidx,
                                                            const float* __restrict__ val, TileGeo g,
                                                            int* __restrict__ cnt, float4* __restrict__ rec,
                                                            const float* __restrict__ aux = nullptr,
                                                            ChunkList cl = ChunkList{}) {
  extern __shared__ int hist[];
  const int blk = blockIdx.x;
  if (SCATTER && blk == g.nblk) {                 // the extra workgroup: cnt holds the scanned offsets
    tile_chunks_body<kTileBinBlock>(cnt, g, cl);
    return;
  }
  for (int i = threadIdx.x; i < g.nkeys; i += blockDim.x) hist[i] = SCATTER ? cnt[i * g.nblk + blk] : 0;
  __syncthreads();
  constexpr int per = tile_per_block(MODE) / kTileBinBlock;
  const int j0 = blk * tile_per_block(MODE);
  float2 p[per];
  int64_t bj[per];
  float vj[per], v2[per];
#pragma unroll
  for (int u = 0; u < per; ++u) {
    const int j = j0 + u * kTileBinBlock + threadIdx.x;
    bj[u] = j < g.N ? bidx[j] : -1;
    vj[u] = 1.f;
    v2[u] = 0.f;
    if (j < g.N) {
      p[u] = pos[j];
      if (MODE == kGridVal && val) {              // the gradient row (C = 1 or 2): its values ride in the record
        vj[u] = val[(int64_t)j * g.C];
        if (g.C == 2) v2[u] = val[(int64_t)j * 2 + 1];
      } else if (val) {
        vj[u] = val[j];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < per; ++u) {
    const int j = j0 + u * kTileBinBlock + threadIdx.x;
    if (j >= g.N || (SKIP_ZERO && vj[u] == 0.f && v2[u] == 0.f)) continue;   // a zero weight adds nothing
                                                                              // (csrc/atl_cpu.cpp:44)
    float tn = 0.f;
    if (MODE == kVoxel) {                         // csrc/atl_cpu.cpp:265: tn = t * (C - 1)
      tn = aux[j] * (float)(g.C - 1);
      const float ft = floorf(tn);
      if (!(ft >= -1.f && ft <= (float)(g.C - 1))) continue;
    }
    const int key = tile_key<MODE>(p[u].x, p[u].y, bj[u], g);
    if (key < 0) continue;
    const int slot = atomicAdd(hist + key, 1);
    if (SCATTER)
      rec[slot] = make_float4(p[u].x, p[u].y, vj[u],
                              MODE == kVoxel ? tn : MODE == kGridVal ? v2[u] : __int_as_float(j));
  }
  if (!SCATTER) {
    __syncthreads();
    for (int i = threadIdx.x; i < g.nkeys; i += blockDim.x) cnt[(int64_t)blk * g.nkeys + i] = hist[i];
  }
}

constexpr int kAccItems = 2;
constexpr int kAccChunk = kAccBlock * kAccItems;   // records per accumulation workgroup, at most

template <int MODE, int C>
__device__ __forceinline__ void accum_record(const float4& q, const float* __restrict__ gout, const TileGeo& g,
                                             int ox, int oy, int L, float* acc) {
  const int nc = C > 0 ? C : g.C;                  // C = 0: the field's channel count at run time
  if (MODE == kGauss) {
    int cx, cy;
    if (!gauss_centre(q.x, q.y, g, cx, cy)) return;   // never taken: the binning applied this test
    const float wn = q.z * g.norm;
    const int ylo = max(cy - g.R, 0), yhi = min(cy + g.R, g.H - 1);
    const int xlo = max(cx - g.R, 0), xhi = min(cx + g.R, g.W - 1);
    for (int yy = ylo; yy <= yhi; ++yy) {
      const float dy = (float)yy - q.y;
      const int ly = yy - oy;
      for (int xx = xlo; xx <= xhi; ++xx) {
        const float dx = (float)xx - q.x;
        const int lx = xx - ox;
        if ((unsigned)ly < (unsigned)L && (unsigned)lx < (unsigned)L)
          atomicAdd(acc + ly * L + lx, wn * expf(-(dx * dx + dy * dy) * g.inv2s2));
      }
    }
  } else if (MODE == kVoxel) {
    // csrc/atl_cpu.cpp:264-283: corners (t0 + dt, y0 + dy, x0 + dx), each in range, value pol * wt * wy * wx
    int x0, y0;
    if (!image_base(q.x, q.y, g.H, g.W, x0, y0)) return;   // never taken: the binning applied this test
    const float tn = q.w;
    const int t0 = (int)floorf(tn);
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const int tt = t0 + dt;
      if (tt < 0 || tt >= nc) continue;
      const float wt = 1.f - fabsf((float)tt - tn);
#pragma unroll
      for (int dy = 0; dy < 2; ++dy) {
        const int yy = y0 + dy;
        if (yy < 0 || yy >= g.H) continue;
        const float wy = 1.f - fabsf((float)yy - q.y);
#pragma unroll
        for (int dx = 0; dx < 2; ++dx) {
          const int xx = x0 + dx;
          if (xx < 0 || xx >= g.W) continue;
          const float wx = 1.f - fabsf((float)xx - q.x);
          const int ly = yy - oy, lx = xx - ox;
          if ((unsigned)ly < (unsigned)L && (unsigned)lx < (unsigned)L)
            atomicAdd(acc + (tt * L + ly) * L + lx, q.z * wt * wy * wx);
        }
      }
    }
  } else if (MODE == kImage || MODE == kImageG) {
    int x0, y0;
    if (!image_base(q.x, q.y, g.H, g.W, x0, y0)) return;   // never taken: the binning applied this test
    const float val = MODE == kImageG ? gout[__float_as_int(q.w)] : q.z;
    const float fx = (float)x0, fy = (float)y0;
    const float ax = q.x - fx, ay = q.y - fy;
    const float wx0 = 1.f - ax, wy0 = 1.f - ay;
#pragma unroll
    for (int jy = 0; jy < 2; ++jy) {
      const int yy = y0 + jy;
      if (yy < 0 || yy >= g.H) continue;
      const float wy = jy ? ay : wy0;
#pragma unroll
      for (int ix = 0; ix < 2; ++ix) {
        const int xx = x0 + ix;
        if (xx < 0 || xx >= g.W) continue;
        const float wx = ix ? ax : wx0;
        const int ly = yy - oy, lx = xx - ox;
        if ((unsigned)ly < (unsigned)L && (unsigned)lx < (unsigned)L) atomicAdd(acc + ly * L + lx, val * (wx * wy));
      }
    }
  } else if (MODE == kGridVal) {                  // record (x, y, g0, g1): no gather of the gradient rows
    const GridCell c = grid_cell(q.x, q.y, g.H, g.W, g.sxw, g.syh, g.scale != 0);
    const float w00 = (1.f - c.ax) * (1.f - c.ay), w01 = c.ax * (1.f - c.ay);
    const float w10 = (1.f - c.ax) * c.ay, w11 = c.ax * c.ay;
    const int ly0 = c.y0 - oy, ly1 = c.y1 - oy, lx0 = c.x0 - ox, lx1 = c.x1 - ox;
    if ((unsigned)ly0 >= (unsigned)L || (unsigned)ly1 >= (unsigned)L || (unsigned)lx0 >= (unsigned)L ||
        (unsigned)lx1 >= (unsigned)L)
      return;                                                // never taken: the binning chose this tile
    const int i00 = ly0 * L + lx0, i01 = ly0 * L + lx1, i10 = ly1 * L + lx0, i11 = ly1 * L + lx1;
#pragma unroll
    for (int ch = 0; ch < (C > 0 ? C : 1); ++ch) {
      const float go = ch == 0 ? q.z : q.w;
      float* a = acc + ch * L * L;
      atomicAdd(a + i00, go * w00);
      atomicAdd(a + i01, go * w01);
      atomicAdd(a + i10, go * w10);
      atomicAdd(a + i11, go * w11);
    }
  } else {
    const GridCell c = grid_cell(q.x, q.y, g.H, g.W, g.sxw, g.syh, g.scale != 0);
    const int j = __float_as_int(q.w);
    const float w00 = (1.f - c.ax) * (1.f - c.ay), w01 = c.ax * (1.f - c.ay);
    const float w10 = (1.f - c.ax) * c.ay, w11 = c.ax * c.ay;
    const int ly0 = c.y0 - oy, ly1 = c.y1 - oy, lx0 = c.x0 - ox, lx1 = c.x1 - ox;
    if ((unsigned)ly0 >= (unsigned)L || (unsigned)ly1 >= (unsigned)L || (unsigned)lx0 >= (unsigned)L ||
        (unsigned)lx1 >= (unsigned)L)
      return;                                                // never taken: the binning chose this tile
    const int i00 = ly0 * L + lx0, i01 = ly0 * L + lx1, i10 = ly1 * L + lx0, i11 = ly1 * L + lx1;
#pragma unroll
    for (int ch = 0; ch < (C > 0 ? C : kMaxChannels); ++ch) {
      if (C == 0 && ch >= nc) break;
      const float go = gout[(int64_t)j * nc + ch];
      float* a = acc + ch * L * L;
      atomicAdd(a + i00, go * w00);
      atomicAdd(a + i01, go * w01);
      atomicAdd(a + i10, go * w10);
      atomicAdd(a + i11, go * w11);
    }
  }
}

// The chunk list of the tile-ordered records (tile_chunks_body) as a launch of its own: one workgroup.
constexpr int kChunkScanBlock = 1024;
__global__ void __launch_bounds__(kChunkScanBlock) k_tile_chunks(const int* __restrict__ boff, TileGeo g, int chunk,
                                                                 int crowd, int4* __restrict__ info,
                                                                 int* __restrict__ nchunk) {
  tile_chunks_body<kChunkScanBlock>(boff, g, ChunkList{info, nchunk, chunk, crowd});
}

// Accumulation: workgroup w takes chunk w (records of one tile, so a crowded tile is shared by several
// workgroups), adds the weighted contributions of its records into an LDS copy of the pixels that tile's events
// reach, in rounds of kAccChunk records (a chunk list made for the gather form holds up to kBinChunk), and flushes
// the non-zero pixels with one global atomic each.
template <int MODE, int C, int T>
__global__ void __launch_bounds__(kAccBlock) k_tile_accum(const int4* __restrict__ info,
                                                          const int* __restrict__ nchunk,
                                                          const float4* __restrict__ rec,
                                                          const float* __restrict__ gout, TileGeo g,
                                                          float* __restrict__ out) {
  const int L = MODE == kGauss ? T + 2 * g.R : T + 1;   // LDS edge: the pixels one tile's events reach
  extern __shared__ float acc[];                  // nc * L * L floats
  const int nc = C > 0 ? C : g.C;
  if ((int)blockIdx.x >= *nchunk) return;
  const int4 ci = info[blockIdx.x];
  const int key = ci.x, s0 = ci.y, s1 = ci.z;
  float4 q[kAccItems];
#pragma unroll
  for (int u = 0; u < kAccItems; ++u) {           // the records load while the window is cleared
    const int k = s0 + u * kAccBlock + threadIdx.x;
    if (k < s1) q[u] = rec[k];
  }
  for (int a = threadIdx.x; a < nc * L * L; a += kAccBlock) acc[a] = 0.f;
  __syncthreads();
  const int64_t pl = (int64_t)g.H * g.W;
  const int plane = g.TY * g.TX;
  const int b = key / plane, r = key - b * plane;
  const int ty = r / g.TX, tx = r - ty * g.TX;
  const bool img_org = MODE == kImage || MODE == kImageG || MODE == kVoxel;
  const int ox = img_org ? tx * T - 1 : MODE == kGauss ? tx * T - 2 * g.R : tx * T;   // LDS column 0
  const int oy = img_org ? ty * T - 1 : MODE == kGauss ? ty * T - 2 * g.R : ty * T;
  for (int base = s0; base < s1; base += kAccChunk) {
    if (base != s0) {
#pragma unroll
      for (int u = 0; u < kAccItems; ++u) {
        const int k = base + u * kAccBlock + threadIdx.x;
        if (k < s1) q[u] = rec[k];
      }
    }
#pragma unroll
    for (int u = 0; u < kAccItems; ++u)
      if (base + u * kAccBlock + (int)threadIdx.x < s1) accum_record<MODE, C>(q[u], gout, g, ox, oy, L, acc);
  }
  __syncthreads();
  for (int a = threadIdx.x; a < L * L; a += kAccBlock) {
    const int py = oy + a / L, px = ox + a % L;
    if (py < 0 || py >= g.H || px < 0 || px >= g.W) continue;
    for (int ch = 0; ch < nc; ++ch) {
      const float v = acc[ch * L * L + a];
      if (v != 0.f) {
        const int64_t o = ((int64_t)b * nc + ch) * pl + (int64_t)py * g.W + px;
        atomicAdd(out + (g.ilv == 2 ? 2 * o + 1 : o), v);
      }
    }
  }
}

// Gather form of the accumulation for the bilinear modes on 16 x 16 tiles (kImage, kGridVal, and kGrid with at
// most four channels).  An LDS float atomic retires about one lane every three cycles on this part, so the four
// (or 4 C) of them per record bound the scatter form above.  Here a workgroup takes a chunk of one tile (512
// records, or 2048 on a tile of more than 16384) in rounds of 512: it ranks a round's records by base corner with
// one LDS integer atomic each and stores (ax, ay, values) in base-corner order; thread c then adds, per channel,
// the four corner products value * (wx * wy) of the records of base corner c (the scatter form's fp32 products)
// to its register sums.  After the last round every window pixel adds the sums of the base corners that reach it
// and is flushed with one global atomic.  Only the order of the float additions differs from the scatter form.
constexpr int kBinT = 16;
constexpr int kBins = kBinT * kBinT;              // base corners of a tile: thread c sums corner c
constexpr int kBinChunk = 4 * kAccChunk;          // records per workgroup on a crowded tile (four rounds), so
                                                  // it is flushed once per 2048 records rather than per 512
static_assert(kBins == kAccBlock, "one accumulation thread per base corner");

// Base corner (window column bx, row by, both in [0, 16)), fractions and values of record q; false if q adds
// nothing (never for binned records: the binning applied the same tests).
template <int MODE, int C>
__device__ __forceinline__ bool bin_record(const float4& q, const float* __restrict__ gout, const TileGeo& g, int ox,
                                           int oy, int& bx, int& by, float& ax, float& ay, float (&val)[C]) {
  if (MODE == kImage || MODE == kImageG) {
    int x0, y0;
    if (!image_base(q.x, q.y, g.H, g.W, x0, y0)) return false;
    ax = q.x - (float)x0;                         // the scatter form's wx1, wy1 (csrc/atl_cpu.cpp:46-53)
    ay = q.y - (float)y0;
    bx = x0 - ox;
    by = y0 - oy;
    val[0] = MODE == kImageG ? gout[__float_as_int(q.w)] : q.z;
  } else {
    const GridCell c = grid_cell(q.x, q.y, g.H, g.W, g.sxw, g.syh, g.scale != 0);
    ax = c.ax;
    ay = c.ay;
    bx = c.x0 - ox;
    by = c.y0 - oy;
    if (MODE == kGridVal) {
      val[0] = q.z;
      if (C > 1) val[C > 1 ? 1 : 0] = q.w;
    } else {
      const int j = __float_as_int(q.w);
#pragma unroll
      for (int ch = 0; ch < C; ++ch) val[ch] = gout[(int64_t)j * C + ch];
    }
  }
  return (unsigned)bx < (unsigned)kBinT && (unsigned)by < (unsigned)kBinT;
}

template <int MODE, int C>
__global__ void __launch_bounds__(kAccBlock) k_tile_accum_bins(const int4* __restrict__ info,
                                                               const int* __restrict__ nchunk,
                                                               const float4* __restrict__ rec,
                                                               const float* __restrict__ gout, TileGeo g,
                                                               float* __restrict__ out) {
  constexpr int T = kBinT, L = T + 1;
  __shared__ int bcnt[kBins];
  __shared__ int bstart[kBins];
  __shared__ int wsum[kAccBlock / kWave + 1];
  __shared__ float sax[kAccChunk], say[kAccChunk], sval[C][kAccChunk];
  __shared__ float bsum[4 * C][kBins];            // corner k = 2 * iy + ix of base corner c, per channel
  if ((int)blockIdx.x >= *nchunk) return;
  const int4 ci = info[blockIdx.x];
  const int key = ci.x, s0 = ci.y, s1 = ci.z;
  const int tid = threadIdx.x;
  const int64_t pl = (int64_t)g.H * g.W;
  const int plane = g.TY * g.TX;
  const int b = key / plane, r = key - b * plane;
  const int ty = r / g.TX, tx = r - ty * g.TX;
  constexpr bool kImg = MODE == kImage || MODE == kImageG;
  const int ox = kImg ? tx * T - 1 : tx * T;     // window column 0
  const int oy = kImg ? ty * T - 1 : ty * T;
  float s[4][C];                                  // this thread's base corner: corner sums over the rounds
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int ch = 0; ch < C; ++ch) s[k][ch] = 0.f;
  for (int base = s0; base < s1; base += kAccChunk) {   // rounds of kAccChunk records
    float4 q[kAccItems];
#pragma unroll
    for (int u = 0; u < kAccItems; ++u) {
      const int k = base + u * kAccBlock + tid;
      if (k < s1) q[u] = rec[k];
    }
    bcnt[tid] = 0;
    int bin[kAccItems], rank[kAccItems];
    float ax[kAccItems], ay[kAccItems], val[kAccItems][C];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kAccItems; ++u) {
      bin[u] = -1;
      int bx, by;
      if (base + u * kAccBlock + tid < s1 && bin_record<MODE, C>(q[u], gout, g, ox, oy, bx, by, ax[u], ay[u], val[u])) {
        bin[u] = by * T + bx;
        rank[u] = atomicAdd(bcnt + bin[u], 1);
      }
    }
    __syncthreads();
    const int mine = bcnt[tid];
    int total;
    const int first = block_exclusive_scan<kAccBlock>(mine, wsum, total);
    bstart[tid] = first;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kAccItems; ++u) {
      if (bin[u] < 0) continue;
      const int p = bstart[bin[u]] + rank[u];
      sax[p] = ax[u];
      say[p] = ay[u];
#pragma unroll
      for (int ch = 0; ch < C; ++ch) sval[ch][p] = val[u][ch];
    }
    __syncthreads();
    for (int p = first; p < first + mine; ++p) {
      const float fx = sax[p], fy = say[p];
      const float wx0 = 1.f - fx, wy0 = 1.f - fy;
      const float w[4] = {wx0 * wy0, fx * wy0, wx0 * fy, fx * fy};
#pragma unroll
      for (int ch = 0; ch < C; ++ch) {
        const float v = sval[ch][p];
#pragma unroll
        for (int k = 0; k < 4; ++k) s[k][ch] += v * w[k];
      }
    }
    __syncthreads();                              // the next round reuses the counts and the sorted records
  }
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int ch = 0; ch < C; ++ch) bsum[k * C + ch][tid] = s[k][ch];
  __syncthreads();
  // the second corner of an axis is the next pixel, or the same one on a grid of a single column (row)
  const int sx = kImg || g.W > 1 ? 1 : 0, sy = kImg || g.H > 1 ? 1 : 0;
  for (int a = tid; a < L * L; a += kAccBlock) {
    const int ly = a / L, lx = a - ly * L;
    const int py = oy + ly, px = ox + lx;
    if (py < 0 || py >= g.H || px < 0 || px >= g.W) continue;
    float v[C];
#pragma unroll
    for (int ch = 0; ch < C; ++ch) v[ch] = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int cx = lx - (k & 1) * sx, cy = ly - (k >> 1) * sy;
      if ((unsigned)cx >= (unsigned)T || (unsigned)cy >= (unsigned)T) continue;
#pragma unroll
      for (int ch = 0; ch < C; ++ch) v[ch] += bsum[k * C + ch][cy * T + cx];
    }
#pragma unroll
    for (int ch = 0; ch < C; ++ch)
      if (v[ch] != 0.f) {
        const int64_t o = ((int64_t)b * C + ch) * pl + (int64_t)py * g.W + px;
        atomicAdd(out + (g.ilv == 2 ? 2 * o + 1 : o), v[ch]);
      }
  }
}

// Many-channel grid adjoint (kGrid, C > 4 channels, 16 x 16 tiles) in the gather form of k_tile_accum_bins: each
// round of up to 512 records is ranked by base node with one LDS integer atomic each and its fractions are stored
// in base-node order; then, four channels at a time, every thread loads those channels of its own records (16
// bytes of the gradient row each, all in flight together) into LDS in the same order, thread c adds the four
// corner products value * (wx * wy) of its node's records into registers, the sums go through an LDS table, and
// every window node adds the sums of the base nodes that reach it into its own LDS window entry.  The window is flushed once per chunk with one global atomic per
// non-zero node and channel.  The products are the scatter form's; only the order of the additions differs.
// With gd set (the trajectory model, B-spline basis): the gradient rows are not read but formed per record from
// the displacement's gradient gd and the event time tt, K = C / 2 (k_traj_gout's values: bspline_row).
__global__ void __launch_bounds__(kAccBlock) k_tile_accum_rows(const int4* __restrict__ info,
                                                               const int* __restrict__ nchunk,
                                                               const float4* __restrict__ rec,
                                                               const float* __restrict__ gout, TileGeo g,
                                                               float* __restrict__ out,
                                                               const float2* __restrict__ gd,
                                                               const float* __restrict__ tt) {
  constexpr int T = kBinT, L = T + 1;
  extern __shared__ float acc[];                  // nc * L * L window
  __shared__ int bcnt[kBins], bstart[kBins];
  __shared__ int wsum[kAccBlock / kWave + 1];
  __shared__ float sax[kAccChunk], say[kAccChunk];
  __shared__ float4 srow[kAccChunk];              // the group's four channels of every record, in base-node order
  __shared__ float bsum[16][kBins];               // corner k, channel c of the group: row 4 k + c
  if ((int)blockIdx.x >= *nchunk) return;
  const int4 ci = info[blockIdx.x];
  const int key = ci.x, s0 = ci.y, s1 = ci.z;
  const int tid = threadIdx.x;
  const int nc = g.C;
  const int64_t pl = (int64_t)g.H * g.W;
  const int plane = g.TY * g.TX;
  const int b = key / plane, r = key - b * plane;
  const int ty = r / g.TX, tx = r - ty * g.TX;
  const int ox = tx * T, oy = ty * T;
  for (int a = tid; a < nc * L * L; a += kAccBlock) acc[a] = 0.f;
  const int sx = g.W > 1 ? 1 : 0, sy = g.H > 1 ? 1 : 0;   // second corner: the next node, or the same one
  for (int base = s0; base < s1; base += kAccChunk) {
    float4 q[kAccItems];
#pragma unroll
    for (int u = 0; u < kAccItems; ++u) {
      const int k = base + u * kAccBlock + tid;
      if (k < s1) q[u] = rec[k];
    }
    bcnt[tid] = 0;
    __syncthreads();
    int bin[kAccItems], rank[kAccItems];
    float ax[kAccItems], ay[kAccItems];
#pragma unroll
    for (int u = 0; u < kAccItems; ++u) {
      bin[u] = -1;
      if (base + u * kAccBlock + tid >= s1) continue;
      const GridCell c = grid_cell(q[u].x, q[u].y, g.H, g.W, g.sxw, g.syh, g.scale != 0);
      const int bx = c.x0 - ox, by = c.y0 - oy;
      if ((unsigned)bx < (unsigned)T && (unsigned)by < (unsigned)T) {   // always: the binning chose this tile
        ax[u] = c.ax;
        ay[u] = c.ay;
        bin[u] = by * T + bx;
        rank[u] = atomicAdd(bcnt + bin[u], 1);
      }
    }
    __syncthreads();
    const int mine = bcnt[tid];
    int total;
    const int first = block_exclusive_scan<kAccBlock>(mine, wsum, total);
    bstart[tid] = first;
    __syncthreads();
    int pos[kAccItems];
#pragma unroll
    for (int u = 0; u < kAccItems; ++u) {
      pos[u] = -1;
      if (bin[u] < 0) continue;
      pos[u] = bstart[bin[u]] + rank[u];
      sax[pos[u]] = ax[u];
      say[pos[u]] = ay[u];
    }
    const int K = nc / 2;
    float2 dd[kAccItems];                          // gd set: each record's displacement gradient, span, basis
    int jb[kAccItems];
    float nb[kAccItems][4];
    if (gd) {
#pragma unroll
      for (int u = 0; u < kAccItems; ++u) {
        dd[u] = make_float2(0.f, 0.f);
        jb[u] = 0;
        nb[u][0] = nb[u][1] = nb[u][2] = nb[u][3] = 0.f;
        if (pos[u] < 0) continue;
        const int e = __float_as_int(q[u].w);
        dd[u] = gd[e];
        jb[u] = bspline_nonzero_rt(tt[e], K, nb[u]);
      }
    }
    for (int cg = 0; cg < nc; cg += 4) {
      // every thread loads the group's channels of its own records (the loads in flight together) into srow
      float4 v4[kAccItems];
#pragma unroll
      for (int u = 0; u < kAccItems; ++u) {
        v4[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (pos[u] < 0) continue;
        if (gd) {
          v4[u].x = bspline_row(cg, K, jb[u], nb[u], dd[u]);
          if (cg + 1 < nc) v4[u].y = bspline_row(cg + 1, K, jb[u], nb[u], dd[u]);
          if (cg + 2 < nc) v4[u].z = bspline_row(cg + 2, K, jb[u], nb[u], dd[u]);
          if (cg + 3 < nc) v4[u].w = bspline_row(cg + 3, K, jb[u], nb[u], dd[u]);
          continue;
        }
        const float* row = gout + (int64_t)__float_as_int(q[u].w) * nc + cg;
        if (g.vec4) {                               // nc % 4 == 0, 16-byte aligned rows
          v4[u] = *(const float4*)row;
        } else {
          v4[u].x = row[0];
          if (cg + 1 < nc) v4[u].y = row[1];
          if (cg + 2 < nc) v4[u].z = row[2];
          if (cg + 3 < nc) v4[u].w = row[3];
        }
      }
#pragma unroll
      for (int u = 0; u < kAccItems; ++u)
        if (pos[u] >= 0) srow[pos[u]] = v4[u];
      __syncthreads();
      float s[4][4];
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int c = 0; c < 4; ++c) s[k][c] = 0.f;
      for (int p = first; p < first + mine; ++p) {
        const float4 r4 = srow[p];
        const float v[4] = {r4.x, r4.y, r4.z, r4.w};
        const float fx = sax[p], fy = say[p];
        const float wx0 = 1.f - fx, wy0 = 1.f - fy;
        const float w[4] = {wx0 * wy0, fx * wy0, wx0 * fy, fx * fy};
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int c = 0; c < 4; ++c) s[k][c] += v[c] * w[k];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int c = 0; c < 4; ++c) bsum[4 * k + c][tid] = s[k][c];
      __syncthreads();
      for (int a = tid; a < L * L; a += kAccBlock) {   // window node a adds the base nodes that reach it
        const int ly = a / L, lx = a - ly * L;
        float v[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int cx = lx - (k & 1) * sx, cy = ly - (k >> 1) * sy;
          if ((unsigned)cx >= (unsigned)T || (unsigned)cy >= (unsigned)T) continue;
#pragma unroll
          for (int c = 0; c < 4; ++c) v[c] += bsum[4 * k + c][cy * T + cx];
        }
#pragma unroll
        for (int c = 0; c < 4; ++c)
          if (cg + c < nc) acc[(cg + c) * L * L + a] += v[c];
      }
      __syncthreads();                              // bsum and srow are rewritten by the next channel group
    }
  }
  for (int a = tid; a < L * L; a += kAccBlock) {
    const int py = oy + a / L, px = ox + a % L;
    if (py >= g.H || px >= g.W) continue;
    for (int ch = 0; ch < nc; ++ch) {
      const float v = acc[ch * L * L + a];
      if (v != 0.f) atomicAdd(out + ((int64_t)b * nc + ch) * pl + (int64_t)py * g.W + px, v);
    }
  }
}

// ------------------------------------------------------------ coefficient-grid adjoint of trajectory look-ups
// The records of n_look look-ups of N events: look-up r of event e sits at grid position pos[r N + e] with the
// displacement gradient gd[r N + e] and the time t[e] (t_last[e] for the last look-up when t_last is set, the
// transport's look-up at the destination time).  The binning stores (x, y, gd.x, gd.y) and the time of every
// record with a non-zero gradient in tile order, so the accumulation reads its tile's records in sequence (no
// gathers of gradients and times by event index).  A binning block takes `per` records per thread, chosen so
// that a call has about kTrajBinBlocks blocks: the per-block count matrix (nkeys x blocks) and its scan stay
// small on large calls, and each block's run of a tile is longer (14M records on 4800 tiles: the scatter took
// 0.51 ms with 2048 blocks of 512 threads, 0.40 with 512 and 0.38 with 256 blocks of 1024).
constexpr int kTrajBinBlocks = 256;
constexpr int kTrajBinThreads = 1024;

inline int traj_bin_per(int64_t m) {
  const int64_t per = (m + (int64_t)kTrajBinBlocks * kTrajBinThreads - 1) / ((int64_t)kTrajBinBlocks * kTrajBinThreads);
  return (int)std::min<int64_t>(std::max<int64_t>(per, 8), 256);
}

// ROWS: the records of a many-channel sampler adjoint instead (one look-up per event, gd and the times unused):
// (x, y, event index, 0), every record kept (the row is read by the accumulation).  SCATTER also prepares the
// accumulation: its nblk workgroups clear the nh halo floats, and one more workgroup writes the chunk list cl.
template <bool SCATTER, bool ROWS = false>
__global__ void __launch_bounds__(kTrajBinThreads) k_traj_bin(const float2* __restrict__ pos,
                                                            const float2* __restrict__ gd,
                                                            const float* __restrict__ t,
                                                            const float* __restrict__ t_last,
                                                            const int64_t* __restrict__ bidx, int N, int n_look,
                                                            int per, TileGeo g, int* __restrict__ cnt,
                                                            float4* __restrict__ rec, float* __restrict__ tr,
                                                            ChunkList cl, float* __restrict__ halo, int64_t nh) {
  extern __shared__ int hist[];
  const int blk = blockIdx.x;
  if (SCATTER) {
    if (blk == g.nblk) {                         // the extra workgroup: cnt holds the scanned offsets
      tile_chunks_body<kTrajBinThreads>(cnt, g, cl);
      return;
    }
    for (int64_t k = (int64_t)blk * blockDim.x + threadIdx.x; k < nh; k += (int64_t)g.nblk * blockDim.x)
      halo[k] = 0.f;
  }
  for (int i = threadIdx.x; i < g.nkeys; i += blockDim.x) hist[i] = SCATTER ? cnt[i * g.nblk + blk] : 0;
  __syncthreads();
  constexpr int U = 4;                           // records per thread in flight together
  const int64_t j0 = (int64_t)blk * per * kTrajBinThreads;
  for (int u0 = 0; u0 < per; u0 += U) {
    float2 d[U], p[U];
    int e[U], r[U];
    int64_t bj[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = j0 + (int64_t)(u0 + u) * kTrajBinThreads + threadIdx.x;
      const bool in = u0 + u < per && j < g.N;
      r[u] = in ? (int)(j / N) : 0;
      e[u] = in ? (int)(j - (int64_t)r[u] * N) : -1;
      d[u] = in && !ROWS ? gd[j] : make_float2(1.f, 0.f);
      p[u] = in ? pos[j] : make_float2(0.f, 0.f);
      bj[u] = in ? bidx[e[u]] : -1;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (e[u] < 0 || (d[u].x == 0.f && d[u].y == 0.f)) continue;   // a zero gradient adds nothing
      const int key = tile_key<kGrid>(p[u].x, p[u].y, bj[u], g);
      if (key < 0) continue;
      const int slot = atomicAdd(hist + key, 1);
      if (SCATTER && ROWS) {
        rec[slot] = make_float4(p[u].x, p[u].y, __int_as_float(e[u]), 0.f);
      } else if (SCATTER) {
        rec[slot] = make_float4(p[u].x, p[u].y, d[u].x, d[u].y);
        tr[slot] = t_last && r[u] == n_look - 1 ? t_last[e[u]] : t[e[u]];
      }
    }
  }
  if (!SCATTER) {
    __syncthreads();
    for (int i = threadIdx.x; i < g.nkeys; i += blockDim.x) cnt[(int64_t)blk * g.nkeys + i] = hist[i];
  }
}

// Window nodes past a tile's own 16 x 16: its right column (17 nodes, the last one diagonal) and its bottom row
// (16), which belong to the tiles on its right, below and diagonally below.  Halo slot h: right column row h for
// h <= 16, bottom row column h - 17 for h >= 17.
constexpr int kHalo = 2 * kBinT + 1;

// Window sums of channel group entries q at window node (lx, ly): the corner sums (table sb[(c G + q) kBins + base
// node], corner c = 2 iy + ix) of the base nodes that reach the node (the second corner of an axis is the next
// node, or the same one on a grid of a single column or row: sx, sy).
template <int G>
__device__ __forceinline__ void window_sum(const float* sb, int lx, int ly, int sx, int sy, float (&v)[G]) {
#pragma unroll
  for (int q = 0; q < G; ++q) v[q] = 0.f;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int cx = lx - (c & 1) * sx, cy = ly - (c >> 1) * sy;
    if ((unsigned)cx >= (unsigned)kBinT || (unsigned)cy >= (unsigned)kBinT) continue;
#pragma unroll
    for (int q = 0; q < G; ++q) v[q] += sb[(c * G + q) * kBins + cy * kBinT + cx];
  }
}

// Halo slot of window node (lx, ly) past the tile's own 16 x 16 (lx == 16 or ly == 16).
__device__ __forceinline__ int halo_slot(int lx, int ly) { return lx == kBinT ? ly : kBinT + 1 + lx; }

// Accumulation of the trajectory records in the gather form.  Float atomic adds into LDS run at a small fraction
// of the LDS rate on this part (~0.3 lane-adds per CU per cycle against ~8 for a plain read-modify-write), so no
// record is added into shared memory: workgroup w takes chunk w of one tile (info[w] = (tile, first, end,
// shared)) and thread c owns base node c of the tile's 16 x 16.  In rounds of kTrajRound records every thread
// takes three records, forms their base node and fractions (grid_cell) and their B-spline basis
// (bspline_nonzero_tab, the knots from an LDS table), ranks them by base node with one LDS integer atomic each,
// and stores (ax, ay, gd.x, gd.y) and the dense basis row (N_{k+1} in column k, zero elsewhere) in base-node
// order; thread c then adds, for each record of its node, fma(w gd, N, s) into registers for every corner,
// component and column (the scatter form's corner weight times the displacement gradient, times the basis
// value).  After the last round the window nodes sum the four base nodes that reach them (channel groups of
// kTrajGroup through LDS) and flush without global atomics when the tile has a single chunk: its own 16 x 16
// nodes are added in place (no other workgroup writes them in the launch) and its halo goes to the tile's
// slots, which k_traj_halo_add adds to the neighbours afterwards; the chunks of a split tile add both with
// atomics (halo zeroed beforehand).  KM >= K columns are held per component (rows padded with zeros).
constexpr int kTrajRound = 768;                  // records staged per round (three per thread: 50 KB of LDS)
constexpr int kTrajGroup = 8;                    // columns per combination pass

template <int KM>
__global__ void __launch_bounds__(kAccBlock) k_traj_tile_accum(const int4* __restrict__ info,
                                                               const int* __restrict__ nchunk,
                                                               const float4* __restrict__ rec,
                                                               const float* __restrict__ tr, TileGeo g, int K,
                                                               float* __restrict__ out, float* __restrict__ halo) {
  constexpr int T = kBinT, L = T + 1, R = kTrajRound, U = R / kAccBlock;
  constexpr int KP = (KM + 3) & ~3;              // basis row stride (16-byte rows)
  constexpr int kStage = R * KP > 4 * kTrajGroup * kBins ? R * KP : 4 * kTrajGroup * kBins;
  __shared__ int bcnt[kBins], bstart[kBins];
  __shared__ int wsum[kAccBlock / kWave + 1];
  __shared__ float4 sg[R];                       // (ax, ay, gd.x, gd.y) of the round's records, base-node order
  __shared__ __align__(16) float sb[kStage];     // their basis rows; after the rounds: the corner sums
  __shared__ float knots[kMaxChannels / 2 + 1];  // c / L, c = 0..L
  if ((int)blockIdx.x >= *nchunk) return;
  {
    const int P = K < 3 ? K : 3, Lk = K + 1 - P;
    if ((int)threadIdx.x <= Lk) knots[threadIdx.x] = (float)(int)threadIdx.x / (float)Lk;
  }
  const int4 ci = info[blockIdx.x];
  const int key = ci.x, s0 = ci.y, s1 = ci.z;
  const bool shared = ci.w != 0;
  const int tid = threadIdx.x;
  const int nc = 2 * K;
  const int plane = g.TY * g.TX;
  const int b = key / plane, rr = key - b * plane;
  const int ty = rr / g.TX, tx = rr - ty * g.TX;
  const int ox = tx * T, oy = ty * T;
  float s[4][2][KM];                             // corner, component (0: gd.y channels, 1: gd.x), column
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int k = 0; k < KM; ++k) s[c][m][k] = 0.f;
  for (int base = s0; base < s1; base += R) {
    float4 q[U];
    float tq[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = base + u * kAccBlock + tid;
      if (k < s1) {
        q[u] = rec[k];
        tq[u] = tr[k];
      }
    }
    bcnt[tid] = 0;
    __syncthreads();                             // the previous round's readers are done
    int bin[U], rank[U];
    float ax[U], ay[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      bin[u] = -1;
      if (base + u * kAccBlock + tid >= s1) continue;
      const GridCell c = grid_cell(q[u].x, q[u].y, g.H, g.W, g.sxw, g.syh, false);
      const int bx = c.x0 - ox, by = c.y0 - oy;
      if ((unsigned)bx < (unsigned)T && (unsigned)by < (unsigned)T) {   // always: the binning chose this tile
        ax[u] = c.ax;
        ay[u] = c.ay;
        bin[u] = by * T + bx;
        rank[u] = atomicAdd(bcnt + bin[u], 1);
      }
    }
    __syncthreads();
    const int mine = bcnt[tid];
    int total;
    const int first = block_exclusive_scan<kAccBlock>(mine, wsum, total);
    bstart[tid] = first;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (bin[u] < 0) continue;
      const int p = bstart[bin[u]] + rank[u];
      sg[p] = make_float4(ax[u], ay[u], q[u].z, q[u].w);
      float* row = sb + p * KP;
#pragma unroll
      for (int k = 0; k < KP; k += 4) *(float4*)(row + k) = make_float4(0.f, 0.f, 0.f, 0.f);
      float nb[4];
      const int j = bspline_nonzero_tab(tq[u], K, knots, nb);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int k = j - 1 + r;                 // column of nb[r] (g_k = N_{k+1})
        if (k >= 0 && k < K) row[k] = nb[r];
      }
    }
    __syncthreads();
    for (int p = first; p < first + mine; ++p) {
      const float4 a = sg[p];
      const float wx0 = 1.f - a.x, wy0 = 1.f - a.y;
      const float w[4] = {wx0 * wy0, a.x * wy0, wx0 * a.y, a.x * a.y};
      float v[4][2];                             // corner weight times gd (channel k: gd.y, channel K + k: gd.x)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        v[c][0] = w[c] * a.w;
        v[c][1] = w[c] * a.z;
      }
      const float* row = sb + p * KP;
#pragma unroll
      for (int k = 0; k < KM; ++k) {
        const float bk = row[k];
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int m = 0; m < 2; ++m) s[c][m][k] = __fmaf_rn(v[c][m], bk, s[c][m][k]);
      }
    }
  }
  // thread c adds the sums reaching its own node c (the node of base node c); threads 0..32 write the halo.
  // A single-chunk tile reads its own nodes' previous values first, all channels in flight together.
  const int oly = tid / T, olx = tid - oly * T;
  const int opy = oy + oly, opx = ox + olx;
  const bool oin = opy < g.H && opx < g.W;
  const int64_t pl = (int64_t)g.H * g.W;
  float* const obase = out + (int64_t)b * nc * pl + (int64_t)opy * g.W + opx;
  float prev[2][KM];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int k = 0; k < KM; ++k) prev[m][k] = !shared && oin && k < K ? obase[(int64_t)(m * K + k) * pl] : 0.f;
  __syncthreads();                               // the staging area becomes the corner-sum table
  const int sx = g.W > 1 ? 1 : 0, sy = g.H > 1 ? 1 : 0;
  constexpr int G = kTrajGroup;
#pragma unroll
  for (int m = 0; m < 2; ++m) {
#pragma unroll
    for (int k0 = 0; k0 < KM; k0 += G) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int q = 0; q < G; ++q)
          if (k0 + q < KM) sb[(c * G + q) * kBins + tid] = s[c][m][k0 + q];
      __syncthreads();
      {
        float v[G];
        window_sum<G>(sb, olx, oly, sx, sy, v);
#pragma unroll
        for (int q = 0; q < G; ++q) {
          const int k = k0 + q;
          if (k >= KM || k >= K || !oin || v[q] == 0.f) continue;
          float* o = obase + (int64_t)(m * K + k) * pl;
          if (shared)
            atomicAdd(o, v[q]);
          else
            *o = prev[m][k] + v[q];
        }
      }
      if (tid < kHalo) {
        const int lx = tid <= T ? T : tid - (T + 1), ly = tid <= T ? tid : T;
        float v[G];
        window_sum<G>(sb, lx, ly, sx, sy, v);
#pragma unroll
        for (int q = 0; q < G; ++q) {
          const int k = k0 + q;
          if (k >= KM || k >= K || v[q] == 0.f) continue;
          float* h = halo + ((int64_t)key * nc + m * K + k) * kHalo + halo_slot(lx, ly);
          if (shared)
            atomicAdd(h, v[q]);
          else
            *h = v[q];
        }
      }
      __syncthreads();                           // the table is rewritten by the next group
    }
  }
}

// The many-channel sampler adjoint (C in 5..32 channels, gout (N, C) rows) in the same form: thread c owns base
// node c; per round of kRowsRound records the loading threads stage (ax, ay) and the record's gradient row
// gout[j] in base-node order, and thread c adds fma(row, w, s) for every corner and channel of its node's records
// (the scatter form's products go * w, fused); the window sums and the flush are k_traj_tile_accum's.
constexpr int kRowsRound = 512;                  // records staged per round (two per thread)

template <int CM>
__global__ void __launch_bounds__(kAccBlock) k_rows_tile_accum(const int4* __restrict__ info,
                                                               const int* __restrict__ nchunk,
                                                               const float4* __restrict__ rec,
                                                               const float* __restrict__ gout, TileGeo g,
                                                               float* __restrict__ out, float* __restrict__ halo) {
  constexpr int T = kBinT, L = T + 1, R = kRowsRound, U = R / kAccBlock;
  constexpr int CP = (CM + 3) & ~3;              // row stride (16-byte rows)
  constexpr int kStage = R * CP > 4 * kTrajGroup * kBins ? R * CP : 4 * kTrajGroup * kBins;
  __shared__ int bcnt[kBins], bstart[kBins];
  __shared__ int wsum[kAccBlock / kWave + 1];
  __shared__ float2 sa[R];                       // (ax, ay) of the round's records, base-node order
  __shared__ __align__(16) float sb[kStage];     // their gradient rows; after the rounds: the corner sums
  if ((int)blockIdx.x >= *nchunk) return;
  const int4 ci = info[blockIdx.x];
  const int key = ci.x, s0 = ci.y, s1 = ci.z;
  const bool shared = ci.w != 0;
  const int tid = threadIdx.x;
  const int nc = g.C;
  const int plane = g.TY * g.TX;
  const int b = key / plane, rr = key - b * plane;
  const int ty = rr / g.TX, tx = rr - ty * g.TX;
  const int ox = tx * T, oy = ty * T;
  // a single-chunk tile's own node of this thread: its previous values, read now (in flight during the rounds)
  const int oly = tid / T, olx = tid - oly * T;
  const int opy = oy + oly, opx = ox + olx;
  const bool oin = opy < g.H && opx < g.W;
  const int64_t pl = (int64_t)g.H * g.W;
  float* const obase = out + (int64_t)b * nc * pl + (int64_t)opy * g.W + opx;
  float prev[CM];
#pragma unroll
  for (int k = 0; k < CM; ++k) prev[k] = !shared && oin && k < nc ? obase[(int64_t)k * pl] : 0.f;
  float s[4][CM];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int k = 0; k < CM; ++k) s[c][k] = 0.f;
  for (int base = s0; base < s1; base += R) {
    float4 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = base + u * kAccBlock + tid;
      if (k < s1) q[u] = rec[k];
    }
    bcnt[tid] = 0;
    __syncthreads();                             // the previous round's readers are done
    int bin[U], rank[U];
    float ax[U], ay[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      bin[u] = -1;
      if (base + u * kAccBlock + tid >= s1) continue;
      const GridCell c = grid_cell(q[u].x, q[u].y, g.H, g.W, g.sxw, g.syh, g.scale != 0);
      const int bx = c.x0 - ox, by = c.y0 - oy;
      if ((unsigned)bx < (unsigned)T && (unsigned)by < (unsigned)T) {   // always: the binning chose this tile
        ax[u] = c.ax;
        ay[u] = c.ay;
        bin[u] = by * T + bx;
        rank[u] = atomicAdd(bcnt + bin[u], 1);
      }
    }
    __syncthreads();
    const int mine = bcnt[tid];
    int total;
    const int first = block_exclusive_scan<kAccBlock>(mine, wsum, total);
    bstart[tid] = first;
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (bin[u] < 0) continue;
      const int p = bstart[bin[u]] + rank[u];
      sa[p] = make_float2(ax[u], ay[u]);
      const float* src = gout + (int64_t)__float_as_int(q[u].z) * nc;
      float* row = sb + p * CP;
      if (g.vec4) {                              // nc % 4 == 0, 16-byte aligned rows
#pragma unroll
        for (int k = 0; k < CP; k += 4)
          *(float4*)(row + k) = k < nc ? *(const float4*)(src + k) : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
#pragma unroll
        for (int k = 0; k < CP; ++k) row[k] = k < nc ? src[k] : 0.f;
      }
    }
    __syncthreads();
    for (int p = first; p < first + mine; ++p) {
      const float2 a = sa[p];
      const float wx0 = 1.f - a.x, wy0 = 1.f - a.y;
      const float w[4] = {wx0 * wy0, a.x * wy0, wx0 * a.y, a.x * a.y};
      const float* row = sb + p * CP;
#pragma unroll
      for (int k = 0; k < CM; ++k) {
        const float go = row[k];
#pragma unroll
        for (int c = 0; c < 4; ++c) s[c][k] = __fmaf_rn(go, w[c], s[c][k]);
      }
    }
  }
  __syncthreads();                               // the staging area becomes the corner-sum table
  const int sx = g.W > 1 ? 1 : 0, sy = g.H > 1 ? 1 : 0;
  constexpr int G = kTrajGroup;
#pragma unroll
  for (int k0 = 0; k0 < CM; k0 += G) {
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
      for (int q = 0; q < G; ++q)
        if (k0 + q < CM) sb[(c * G + q) * kBins + tid] = s[c][k0 + q];
    __syncthreads();
    {
      float v[G];
      window_sum<G>(sb, olx, oly, sx, sy, v);
#pragma unroll
      for (int q = 0; q < G; ++q) {
        const int ch = k0 + q;
        if (ch >= CM || ch >= nc || !oin || v[q] == 0.f) continue;
        float* o = obase + (int64_t)ch * pl;
        if (shared)
          atomicAdd(o, v[q]);
        else
          *o = prev[ch] + v[q];
      }
    }
    if (tid < kHalo) {
      const int lx = tid <= T ? T : tid - (T + 1), ly = tid <= T ? tid : T;
      float v[G];
      window_sum<G>(sb, lx, ly, sx, sy, v);
#pragma unroll
      for (int q = 0; q < G; ++q) {
        const int ch = k0 + q;
        if (ch >= CM || ch >= nc || v[q] == 0.f) continue;
        float* h = halo + ((int64_t)key * nc + ch) * kHalo + halo_slot(lx, ly);
        if (shared)
          atomicAdd(h, v[q]);
        else
          *h = v[q];
      }
    }
    __syncthreads();
  }
}

__global__ void __launch_bounds__(kBlock) k_fill_zero_f(float* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// Adds the halos to the nodes they belong to: thread (tile, channel, i) owns node (0, i) of the tile's left
// column (i < 16) or node (i - 15, 0) of its top row (16 <= i < 31) and adds the halo slots that land there (the
// left tile's right column, the upper tile's bottom row, the upper-left tile's diagonal node), one thread per node.
__global__ void __launch_bounds__(kBlock) k_traj_halo_add(const float* __restrict__ halo, TileGeo g, int nc,
                                                          float* __restrict__ out) {
  constexpr int T = kBinT;
  constexpr int kOwn = 2 * T - 1;                 // left column and top row nodes of a tile
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= (int64_t)g.nkeys * nc * kOwn) return;
  const int i = (int)(id % kOwn);
  const int64_t kc = id / kOwn;
  const int ch = (int)(kc % nc), key = (int)(kc / nc);
  const int plane = g.TY * g.TX;
  const int b = key / plane, rr = key - b * plane;
  const int ty = rr / g.TX, tx = rr - ty * g.TX;
  auto slot = [&](int k, int h) { return halo[((int64_t)k * nc + ch) * kHalo + h]; };
  int lx, ly;
  float v = 0.f;
  if (i < T) {
    lx = 0;
    ly = i;
    if (tx > 0) v += slot(key - 1, i);
    if (i == 0 && ty > 0) {
      v += slot(key - g.TX, T + 1);
      if (tx > 0) v += slot(key - g.TX - 1, T);
    }
  } else {
    lx = i - T + 1;
    ly = 0;
    if (ty > 0) v += slot(key - g.TX, T + 1 + lx);
  }
  const int py = ty * T + ly, px = tx * T + lx;
  if (v == 0.f || py >= g.H || px >= g.W) return;
  out[((int64_t)b * nc + ch) * g.H * g.W + (int64_t)py * g.W + px] += v;
}

// gpos of the bilinear gather backward (csrc/atl_cpu.cpp:151-172, the position half): per event, no atomics.
__global__ void __launch_bounds__(kBlock) k_gather_bwd_pos(const float* __restrict__ gval,
                                                           const float* __restrict__ img,
                                                           const float2* __restrict__ pos,
                                                           const int64_t* __restrict__ bidx, int64_t N, int64_t B,
                                                           int H, int W, float2* __restrict__ gpos) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t b = bidx[n];
  const float gn = gval[n];
  float sx = 0.f, sy = 0.f;
  int x0, y0;
  const float2 p = pos[n];
  if (batch_ok(b, B) && image_base(p.x, p.y, H, W, x0, y0)) {
    const float* base = img + b * (int64_t)H * W;
    const float ax = p.x - (float)x0, ay = p.y - (float)y0;
    const float wx0 = 1.f - ax, wy0 = 1.f - ay;
#pragma unroll
    for (int jy = 0; jy < 2; ++jy) {
      const int yy = y0 + jy;
      if (yy < 0 || yy >= H) continue;
      const float wy = jy ? ay : wy0;
      const float dwy = jy ? 1.f : -1.f;
#pragma unroll
      for (int ix = 0; ix < 2; ++ix) {
        const int xx = x0 + ix;
        if (xx < 0 || xx >= W) continue;
        const float wx = ix ? ax : wx0;
        const float dwx = ix ? 1.f : -1.f;
        const float v = base[yy * W + xx];
        sx += (dwx * wy) * v;
        sy += (wx * dwy) * v;
      }
    }
  }
  gpos[n] = make_float2(gn * sx, gn * sy);
}

int64_t align256(int64_t n) { return (n + 255) & ~(int64_t)255; }

// Geometry: the smallest tile edge (16 or 32) whose tile count fits the LDS histogram; false if none does.
bool tile_geo(int mode, int64_t B, int64_t H, int64_t W, int64_t N, int64_t img_h, int64_t img_w, TileGeo& g,
              int R = 0) {
  if (B < 1 || H < 1 || W < 1 || N < 0 || N >= ((int64_t)1 << 30) || (double)B * H * W >= 2.0e9) return false;
  if (mode == kGauss && (R < 0 || R > kMaxGaussRadius)) return false;
  g.vec4 = 0;
  g.ilv = 1;
  const int64_t ext = mode == kGauss ? 2 * R : 1;   // base corners / centres span W + ext positions per row
  for (int T : {16, 32}) {
    const int64_t tx = (W + ext + T - 1) / T, ty = (H + ext + T - 1) / T;
    if (B * tx * ty <= kTileMaxKeys) {
      g.B = (int)B; g.H = (int)H; g.W = (int)W; g.T = T;
      g.TX = (int)tx; g.TY = (int)ty; g.nkeys = (int)(B * tx * ty);
      g.N = (int)N;
      g.nblk = (int)((N + tile_per_block(mode) - 1) / tile_per_block(mode));
      g.mode = mode;
      g.C = 1;
      g.R = R;
      g.inv2s2 = g.norm = 0.f;
      g.scale = img_h > 0 && img_w > 0;
      g.sxw = (float)(img_w - 1 > 1 ? img_w - 1 : 1);
      g.syh = (float)(img_h - 1 > 1 ? img_h - 1 : 1);
      return (double)g.nkeys * g.nblk + 1 < 2.0e9;
    }
  }
  return false;
}

struct TileLayout {
  int64_t cnt, boff, part, rec, info, nchunk, bytes;
};

// Chunks of one call, at most: one per non-empty tile plus one per kAccChunk records.
inline int64_t max_chunks(const TileGeo& g) { return (int64_t)g.nkeys + ((int64_t)g.N + kAccChunk - 1) / kAccChunk; }

TileLayout tile_layout(const TileGeo& g) {
  TileLayout L;
  const int64_t nbh = (int64_t)g.nkeys * g.nblk;
  int64_t off = 0;
  L.cnt = off;    off += align256(nbh * 4);
  L.boff = off;   off += align256((nbh + 1) * 4);
  L.part = off;   off += align256((scan_tiles(nbh > 0 ? nbh : 1) + 1) * 4);
  L.rec = off;    off += align256((int64_t)g.N * 16);
  L.info = off;   off += align256(max_chunks(g) * 16);
  L.nchunk = off; off += 256;
  L.bytes = off;
  return L;
}

__global__ void k_tile_zero1(int* p) { p[0] = 0; }

// ATL_TILE_SCATTER=1 in the environment selects the scatter form of the accumulation for every mode (read at
// every call, so that a test can compare both forms in one process).  A backward that reuses its forward's chunk
// list may therefore run the other form on it: the scatter form takes chunks of any length, in rounds.
bool tile_scatter_form() {
  const char* e = std::getenv("ATL_TILE_SCATTER");
  return e && e[0] == '1';
}

// The accumulation form of tile_accum<MODE, C> on geometry g (gather: one thread per pixel of a 16 x 16 tile)
// and the chunk list it runs on: chunks of kAccChunk records, crowded tiles in chunks of kBinChunk for the gather
// form.
template <int MODE, int C>
bool tile_gather(const TileGeo& g) {
  constexpr bool kGatherForm =
      MODE == kImage || MODE == kImageG || MODE == kGridVal || (MODE == kGrid && C >= 1 && C <= 4);
  return kGatherForm && g.T == kBinT && !tile_scatter_form();
}

template <int MODE, int C>
ChunkList tile_chunk_list(const TileGeo& g, const TileLayout& L, void* ws) {
  char* w = (char*)ws;
  return ChunkList{(int4*)(w + L.info), (int*)(w + L.nchunk), kAccChunk,
                   tile_gather<MODE, C>(g) ? kBinChunk : kAccChunk};
}

// Histogram, scan and scatter of the records; with cl, the scatter launch's extra workgroup writes that chunk
// list (then the accumulation runs with listed = true).
template <int MODE>
void tile_bin(const TileGeo& g, const TileLayout& L, void* ws, const float* pos, const int64_t* b, const float* val,
              hipStream_t stream, const float* aux = nullptr, const ChunkList* cl = nullptr) {
  char* w = (char*)ws;
  int* cnt = (int*)(w + L.cnt);
  int* boff = (int*)(w + L.boff);
  if (g.nblk == 0) {
    hipLaunchKernelGGL(k_tile_zero1, dim3(1), dim3(1), 0, stream, boff);
    return;
  }
  const size_t lds = (size_t)g.nkeys * sizeof(int);
  hipLaunchKernelGGL((k_tile_bin<MODE, false>), dim3(g.nblk), dim3(kTileBinBlock), lds, stream, (const float2*)pos,
                     b, val, g, cnt, (float4*)nullptr, aux, ChunkList{});
  scan32t(cnt, g.nkeys, g.nblk, (int*)(w + L.part), boff, stream);
  hipLaunchKernelGGL((k_tile_bin<MODE, true>), dim3(g.nblk + (cl ? 1 : 0)), dim3(kTileBinBlock), lds, stream,
                     (const float2*)pos, b, val, g, boff, (float4*)(w + L.rec), aux, cl ? *cl : ChunkList{});
}

// listed: the chunk list in ws is already that of this form (an earlier accumulation on the same records).
template <int MODE, int C>
void tile_accum(const TileGeo& g, const TileLayout& L, const void* ws, const float* gout, float* out,
                hipStream_t stream, bool listed = false) {
  if (g.nblk == 0) return;
  char* w = (char*)ws;                             // the chunk list is written here (a part of the plan)
  int4* info = (int4*)(w + L.info);
  int* nchunk = (int*)(w + L.nchunk);
  constexpr bool kGatherForm =
      MODE == kImage || MODE == kImageG || MODE == kGridVal || (MODE == kGrid && C >= 1 && C <= 4);
  const bool gather = tile_gather<MODE, C>(g);
  if (!listed) {
    const ChunkList cl = tile_chunk_list<MODE, C>(g, L, w);
    hipLaunchKernelGGL(k_tile_chunks, dim3(1), dim3(kChunkScanBlock), 0, stream, (const int*)(w + L.boff), g,
                       cl.chunk, cl.crowd, info, nchunk);
  }
  const unsigned grid = (unsigned)max_chunks(g);  // workgroups past the chunk count return at once
  const int nc = C > 0 ? C : g.C;
  const size_t edge = MODE == kGauss ? (size_t)(g.T + 2 * g.R) : (size_t)(g.T + 1);
  const size_t lds = (size_t)nc * edge * edge * sizeof(float);
  if (gather)
    hipLaunchKernelGGL((k_tile_accum_bins<MODE, kGatherForm ? (C > 0 ? C : 1) : 1>), dim3(grid), dim3(kAccBlock), 0,
                       stream, (const int4*)info, (const int*)nchunk, (const float4*)(w + L.rec), gout, g, out);
  else if (g.T == 16)
    hipLaunchKernelGGL((k_tile_accum<MODE, C, 16>), dim3(grid), dim3(kAccBlock), lds, stream, (const int4*)info,
                       (const int*)nchunk, (const float4*)(w + L.rec), gout, g, out);
  else
    hipLaunchKernelGGL((k_tile_accum<MODE, C, 32>), dim3(grid), dim3(kAccBlock), lds, stream, (const int4*)info,
                       (const int*)nchunk, (const float4*)(w + L.rec), gout, g, out);
}

// Binning and accumulation of one set of records, the chunk list written by the binning's scatter launch.
template <int MODE, int C>
void tile_bin_accum(const TileGeo& g, const TileLayout& L, void* ws, const float* pos, const int64_t* b,
                    const float* val, float* out, hipStream_t stream, const float* aux = nullptr) {
  const ChunkList cl = tile_chunk_list<MODE, C>(g, L, ws);
  tile_bin<MODE>(g, L, ws, pos, b, val, stream, aux, &cl);
  tile_accum<MODE, C>(g, L, ws, nullptr, out, stream, true);
}

// Scratch of atl_splat_bilinear_fwd_noalloc: the tile engine's workspace (counts, offsets, records) for callers
// that cannot allocate device memory.  Every GPU the library runs on holds its own copy until the process ends.
// Host code never passes the array's name to a kernel (on the host it is a stand-in, not a device address): the
// address of each device's copy is looked up with hipGetSymbolAddress, with that device current, by atl_init (the
// library's set-up, for every visible device) or else by the entry point's first call on a device, and kept in
// g_scratch_ptr.
// Each call rewrites every byte of it that its kernels read (counts by the histogram pass, offsets by the scan,
// records by the scatter), so nothing needs clearing; calls that overlap on one GPU share it and race.
constexpr int64_t kNoAllocScratchBytes = 64ll << 20;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
void* g_scratch_ptr[kMaxDevices] = {};
std::mutex g_scratch_mu;

// The scratch address on the current device `dev`, looked up on first use (caller holds g_scratch_mu).
int noalloc_lookup(int dev, const char* what) {
  if (g_scratch_ptr[dev]) return 0;
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    set_error("%s: hipGetSymbolAddress of the scratch array failed on device %d: %s", what, dev, hipGetErrorString(e));
    return 1;
  }
  g_scratch_ptr[dev] = p;
  return 0;
}

int noalloc_scratch(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    set_error("splat_bilinear_fwd_noalloc: no current device");
    return 1;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (noalloc_lookup(dev, "splat_bilinear_fwd_noalloc") != 0) return 1;
  *out = g_scratch_ptr[dev];
  return 0;
}

// ------------------------------------------------------------------------------------ warp -> splat -> gather
// The image of warped events sampled back at the events, forward and backward to a dense flow grid, in one
// sequence of launches (the composition atl/motion/parametric.py:53-56 -> atl/objectives/base.py:40-60 ->
// atl/ops/functional.py:67-87 with the flow of parametric.py:212-216):
//   v_j = sample(grid, x_j), y_j = x_j + v_j (t_ref - t_j), w_j = [y_j inside the sensor] (or 1),
//   img = splat(y, w), vals_j = gather(img, y_j).
// The forward bins the warped events by image tile (the histogram is taken by the warp kernel itself, with the
// flow-grid tile histogram of the events' own positions beside it) and keeps y, w and the records for the
// backward, which splats the value gradient on those records, forms each event's flow gradient in one per-event
// kernel that writes it straight into its flow-grid tile slot, and accumulates the flow-grid adjoint on the tile
// engine.  The image (forward) and the flow-grid gradient (backward) are written, not accumulated: the first
// kernel of each clears them.  Every per-event expression is the composed path's, in its fp32 order.
// The per-event kernels of the pipeline (k_wsg_warp, k_wsg_grad) take k_tile_bin's 4096 events per block in
// 1024 threads of 4 events: 16 waves per CU hide their gathers' latency better than 8 waves of 8 events.
constexpr int kWsgBlock = 1024;
static_assert(kTilePerBlock % kWsgBlock == 0, "whole events per thread");

// One-node grids (Hg = Wg = 1, a translation) of at most kOneNodeMaxB windows: the adjoint is a sum per window.
constexpr int kOneNodeMaxB = 64;
constexpr int kOneNodeBlocks = 256;

bool wsg_one_node(int64_t B, int64_t Hg, int64_t Wg) { return Hg == 1 && Wg == 1 && B <= kOneNodeMaxB; }

// Where the flow-grid adjoint's tile counts are made: in the forward's k_wsg_warp when both histograms fit its
// LDS (kCountWarp: one count matrix over both key spaces, one scan), else by a counting pass and a scan of their
// own in the backward (kCountBwd); none for one-node grids.
enum WsgCount { kCountNone, kCountWarp, kCountBwd };

struct WsgLayout {
  TileGeo gi, gg;              // image tiles (kImage / kImageG), flow-grid tiles (kGridVal, 2 channels)
  TileLayout Li, Lg;           // views (offsets from the workspace base) into one count matrix, one offset array
                               // and one record array, with a chunk list each
  WsgCount count;
  int nkc;                     // count matrix columns (keys): gi.nkeys + gg.nkeys with kCountWarp, else gi.nkeys
  int64_t y, w, gv, G, fil;    // warped positions (N float2), weights (N), flow gradients (N float2, one-node
                               // grids only), the (image, image gradient) pairs (B H W float2), the flow's
                               // node-interleaved copy (B Hg Wg float2)
  int64_t bytes;
};

// With kCountWarp the joint scan puts the image records at [0, Ni) and the flow-grid records at [Ni, Ni + Ng) of
// the record array (the grid's offsets follow the image's); otherwise the grid's records have their own scan and
// the array's second half.
bool wsg_layout(int64_t N, int64_t B, int64_t H, int64_t W, int64_t Hg, int64_t Wg, WsgLayout& L) {
  if (N < 1 || B < 1 || H < 1 || W < 1 || Hg < 1 || Wg < 1) return false;
  if (!tile_geo(kImage, B, H, W, N, 0, 0, L.gi) || !tile_geo(kGridVal, B, Hg, Wg, N, H, W, L.gg)) return false;
  if (B * H * W >= ((int64_t)1 << 31) || B * 2 * Hg * Wg >= ((int64_t)1 << 31)) return false;
  if (L.gi.nblk != L.gg.nblk) return false;       // one block partition for both histograms
  L.gg.C = 2;
  L.count = wsg_one_node(B, Hg, Wg) ? kCountNone : L.gi.nkeys + L.gg.nkeys <= kTileMaxKeys ? kCountWarp : kCountBwd;
  L.nkc = L.count == kCountWarp ? L.gi.nkeys + L.gg.nkeys : L.gi.nkeys;
  const int64_t nblk = L.gi.nblk, nbh = (int64_t)(L.gi.nkeys + L.gg.nkeys) * nblk;
  int64_t off = 0;
  const int64_t cnt = off;  off += align256(nbh * 4);
  const int64_t boff = off; off += align256((nbh + 1) * 4);
  const int64_t part = off; off += align256((scan_tiles(nbh) + 1) * 4);
  const int64_t rec = off;  off += align256(2 * N * 16);
  L.Li.info = off;   off += align256(max_chunks(L.gi) * 16);
  L.Li.nchunk = off; off += 256;
  L.Lg.info = off;   off += align256(max_chunks(L.gg) * 16);
  L.Lg.nchunk = off; off += 256;
  L.Li.cnt = L.Lg.cnt = cnt;
  L.Li.part = L.Lg.part = part;
  L.Li.boff = boff;
  L.Lg.boff = boff + (int64_t)L.gi.nkeys * nblk * 4;
  L.Li.rec = rec;
  L.Lg.rec = L.count == kCountWarp ? rec : rec + N * 16;
  L.y = off;  off += align256(N * 8);
  L.w = off;  off += align256(N * 4);
  L.gv = off; off += align256(N * 8);
  L.G = off;  off += align256(B * H * W * 8);
  L.fil = off; off += align256(B * Hg * Wg * 8);
  L.bytes = L.Li.bytes = L.Lg.bytes = off;
  return true;
}

// Warp, weight and the image-tile histogram, with the block partition of k_tile_bin (4096 events per block) so
// that its scatter pass finds the same per-block counts.  Every event with an in-image base corner is counted,
// masked ones (w = 0) included: the value gradient of the gather reaches them.  Counts go to cnt[block * cstride
// + key]; with countg, the flow-grid tile histogram of the events' own positions too, at columns g.nkeys + key
// (every event of a valid window: the backward's k_wsg_grad places its gradient rows by it, over the same
// partition).  The threads also clear the nz floats of `zero` (the image,
// which the splat then accumulates).  WIDE (Wg >= 2): the flow is read from its node-interleaved copy fil
// (B, Hg, Wg, 2; atl_flow_interleave), where a row's two corners with both channels are 16 contiguous bytes, so an
// event reads two pieces instead of four (the sums are the planar ones, bit for bit); a single kernel with both
// forms compiled to separate 4-byte loads.
template <bool WIDE>
__global__ void __launch_bounds__(kWsgBlock) k_wsg_warp(const float* __restrict__ grid,
                                                        const float* __restrict__ fil, int Hg, int Wg,
                                                            float sxw, float syh, const float2* __restrict__ xy,
                                                            const float* __restrict__ t,
                                                            const int64_t* __restrict__ bidx, float t_ref, int mask,
                                                            TileGeo g, float2* __restrict__ y, float* __restrict__ w,
                                                            int* __restrict__ cnt, int cstride, TileGeo gg,
                                                            bool countg, float* __restrict__ zero, int64_t nz) {
  extern __shared__ int hist[];
  int* histg = hist + g.nkeys;
  const int blk = blockIdx.x;
  for (int i = threadIdx.x; i < g.nkeys; i += blockDim.x) hist[i] = 0;
  if (countg)
    for (int i = threadIdx.x; i < gg.nkeys; i += blockDim.x) histg[i] = 0;
  for (int64_t k = (int64_t)blk * blockDim.x + threadIdx.x; k < nz; k += (int64_t)gridDim.x * blockDim.x) zero[k] = 0.f;
  constexpr int per = kTilePerBlock / kWsgBlock;
  const int j0 = blk * kTilePerBlock;
  const int64_t plane = (int64_t)Hg * Wg;
  const float wmax = (float)(g.W - 1), hmax = (float)(g.H - 1);
  float2 p[per];
  float tj[per];
  int64_t bj[per];
#pragma unroll
  for (int u = 0; u < per; ++u) {                 // every event's inputs first, then every flow row
    const int j = j0 + u * kWsgBlock + threadIdx.x;
    bj[u] = j < g.N ? bidx[j] : -1;
    p[u] = j < g.N ? xy[j] : make_float2(0.f, 0.f);
    tj[u] = j < g.N ? t[j] : 0.f;
  }
  float4 ra[per], rb[per];                        // (row 0, row 1) corner pairs of the two flow channels
  GridCorners c[per];
#pragma unroll
  for (int u = 0; u < per; ++u) {
    c[u] = grid_corners(p[u].x, p[u].y, Hg, Wg, sxw, syh, true);
    ra[u] = rb[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (!batch_ok(bj[u], g.B)) continue;          // sample_grid of an event outside the batch: zero
    const float* f = grid + bj[u] * 2 * plane;
    if (WIDE) {                                   // o01 = o00 + 1, o11 = o10 + 1: one 16-byte piece per row
      const float* fi = fil + bj[u] * 2 * plane;
      float4 r0, r1;                              // (c0, c1) of corner x0, then of x0 + 1: 8-byte aligned
      __builtin_memcpy(&r0, fi + 2 * (int64_t)c[u].o00, sizeof(float4));
      __builtin_memcpy(&r1, fi + 2 * (int64_t)c[u].o10, sizeof(float4));
      ra[u] = make_float4(r0.x, r0.z, r1.x, r1.z);
      rb[u] = make_float4(r0.y, r0.w, r1.y, r1.w);
    } else {
      ra[u] = make_float4(f[c[u].o00], f[c[u].o01], f[c[u].o10], f[c[u].o11]);
      rb[u] = make_float4(f[plane + c[u].o00], f[plane + c[u].o01], f[plane + c[u].o10], f[plane + c[u].o11]);
    }
  }
  __syncthreads();                                // the histogram is cleared
#pragma unroll
  for (int u = 0; u < per; ++u) {
    const int j = j0 + u * kWsgBlock + threadIdx.x;
    if (j >= g.N) continue;
    float vx = ra[u].x * c[u].w00;                // atl/motion/parametric.py:235-251, the device sampler's order
    vx = vx + ra[u].y * c[u].w01;
    vx = vx + ra[u].z * c[u].w10;
    vx = vx + ra[u].w * c[u].w11;
    float vy = rb[u].x * c[u].w00;
    vy = vy + rb[u].y * c[u].w01;
    vy = vy + rb[u].z * c[u].w10;
    vy = vy + rb[u].w * c[u].w11;
    if (!batch_ok(bj[u], g.B)) vx = vy = 0.f;
    const float step = t_ref - tj[u];             // parametric.py:53-56: x + v * (t_ref - t)
    const float yx = p[u].x + vx * step, yy = p[u].y + vy * step;
    const float wj = !mask || (yx >= 0.f && yx <= wmax && yy >= 0.f && yy <= hmax) ? 1.f : 0.f;
    y[j] = make_float2(yx, yy);
    w[j] = wj;
    const int key = tile_key<kImage>(yx, yy, bj[u], g);
    if (key >= 0) atomicAdd(hist + key, 1);
    if (countg) {
      const int kg = tile_key<kGridVal>(p[u].x, p[u].y, bj[u], gg);
      if (kg >= 0) atomicAdd(histg + kg, 1);
    }
  }
  __syncthreads();
  int* __restrict__ row = cnt + (int64_t)blk * cstride;
  for (int i = threadIdx.x; i < g.nkeys; i += blockDim.x) row[i] = hist[i];
  if (countg)
    for (int i = threadIdx.x; i < gg.nkeys; i += blockDim.x) row[g.nkeys + i] = histg[i];
}

// vals_j = gather(img, y_j): csrc/atl_cpu.cpp:134-149.
__global__ void __launch_bounds__(kBlock) k_wsg_gather(const float* __restrict__ img, const float2* __restrict__ y,
                                                       const int64_t* __restrict__ bidx, int64_t N, int64_t B, int H,
                                                       int W, float* __restrict__ vals) {
  const int64_t n = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const int64_t b = bidx[n];
  float s = 0.f;
  const float2 p = y[n];
  const float fx = floorf(p.x), fy = floorf(p.y);
  if (batch_ok(b, B) && fx >= -1.f && fx <= (float)(W - 1) && fy >= -1.f && fy <= (float)(H - 1)) {
    const float* base = img + b * (int64_t)H * W;  // for_corners' corners and order, one 8-byte load per row
    const int x0 = (int)fx, y0 = (int)fy;
    const float ax = p.x - fx, ay = p.y - fy;
    const float wx0 = 1.f - ax, wy0 = 1.f - ay;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int yy = y0 + j;
      if (yy < 0 || yy >= H) continue;
      const float wy = j ? ay : wy0;
      const float* row = base + (int64_t)yy * W;
      if (x0 >= 0 && x0 + 1 < W) {
        float2 r;
        __builtin_memcpy(&r, row + x0, sizeof(float2));
        s += (wx0 * wy) * r.x;
        s += (ax * wy) * r.y;
      } else {
        if (x0 >= 0) s += (wx0 * wy) * row[x0];
        if (x0 + 1 < W) s += (ax * wy) * row[x0 + 1];
      }
    }
  }
  vals[n] = s;
}

// Flow-grid adjoint of a one-node grid (Hg = Wg = 1, a translation): every event's sample is the node with weight
// 1, so the node's gradient is the sum of its batch's per-event rows gv (N, 2); B <= kOneNodeMaxB windows.  Per
// block: a wave whose lanes share one window adds its rows across the wave first; partial sums per window in LDS,
// then one global atomic per window and channel (ggrid accumulated, as the tile adjoint accumulates).

__global__ void __launch_bounds__(kBlock) k_one_node_adjoint(const float2* __restrict__ gv,
                                                             const int64_t* __restrict__ bidx, int64_t N, int B,
                                                             float* __restrict__ ggrid) {
  __shared__ float part[2 * kOneNodeMaxB];
  for (int i = threadIdx.x; i < 2 * B; i += blockDim.x) part[i] = 0.f;
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t base = (int64_t)blockIdx.x * blockDim.x; base < N; base += stride) {   // uniform trip count
    const int64_t n = base + threadIdx.x;
    int64_t bb = -1;
    float2 g = make_float2(0.f, 0.f);
    if (n < N) {
      bb = bidx[n];
      g = gv[n];
    }
    const bool ok = bb >= 0 && bb < B;
    const int bw = __shfl((int)bb, 0);
    if (__all(!(n < N) || (int)bb == bw) && bw >= 0 && bw < B) {        // one window across the wave
      const float sx = wave_sum(ok ? g.x : 0.f), sy = wave_sum(ok ? g.y : 0.f);
      if (lane == 0) {
        atomicAdd(part + 2 * bw, sx);
        atomicAdd(part + 2 * bw + 1, sy);
      }
    } else if (ok) {
      atomicAdd(part + 2 * bb, g.x);
      atomicAdd(part + 2 * bb + 1, g.y);
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < 2 * B; i += blockDim.x)
    if (part[i] != 0.f) atomicAdd(ggrid + i, part[i]);   // ggrid (B, 2, 1, 1): element 2 b + c
}

// The backward's image pair: ig[p] = (img[p], gimg[p] or 0); the value gradient's splat is then added into the
// second slots, and the per-event gradient reads both images of a corner row with one 16-byte load.  The same
// threads clear the nz floats of `zero` (the flow-grid gradient, which the adjoint then accumulates).
__global__ void __launch_bounds__(kBlock) k_wsg_pack(const float* __restrict__ img, const float* __restrict__ gimg,
                                                     int64_t n, float2* __restrict__ ig, float* __restrict__ zero,
                                                     int64_t nz) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) ig[i] = make_float2(img[i], gimg ? gimg[i] : 0.f);
  for (int64_t k = i; k < nz; k += (int64_t)gridDim.x * blockDim.x) zero[k] = 0.f;
}

// Per-event gradient: the position gradient of the gather (gvals_j * grad img(y_j), csrc/atl_cpu.cpp:151-172) plus
// that of the splat (w_j * grad G(y_j), csrc/atl_cpu.cpp:58-76, G the image gradient), times (t_ref - t_j) for the
// flow sampled at x_j.  RECS: every row goes straight to its slot in the flow-grid tile order as the record
// (x, y, gv.x, gv.y), the slots counted by the forward's k_wsg_warp over the same block partition and scanned
// (boff; a zero row adds nothing and keeps its slot); otherwise the rows are written to gv (one-node grids).
// RECS with nblk + 1 workgroups: the last one writes the chunk list `cl` of the records.
template <bool RECS>
__global__ void __launch_bounds__(kWsgBlock) k_wsg_grad(const float2* __restrict__ ig,
                                                            const float* __restrict__ gvals,
                                                            const float2* __restrict__ y, const float* __restrict__ w,
                                                            const float2* __restrict__ xy,
                                                            const float* __restrict__ t,
                                                            const int64_t* __restrict__ bidx, float t_ref,
                                                            int H, int W, TileGeo gg, float2* __restrict__ gv,
                                                            const int* __restrict__ boff, float4* __restrict__ rec,
                                                            ChunkList cl) {
  extern __shared__ int hist[];
  const int blk = blockIdx.x;
  if (RECS && blk == gg.nblk) {
    tile_chunks_body<kWsgBlock>(boff, gg, cl);
    return;
  }
  if (RECS)
    for (int i = threadIdx.x; i < gg.nkeys; i += blockDim.x) hist[i] = boff[i * gg.nblk + blk];
  constexpr int per = kTilePerBlock / kWsgBlock;
  const int j0 = blk * kTilePerBlock;
  const int64_t pl = (int64_t)H * W;
  float2 p[per];
  int64_t bj[per];
#pragma unroll
  for (int u = 0; u < per; ++u) {                 // positions first, then every corner row of every event
    const int j = j0 + u * kWsgBlock + threadIdx.x;
    bj[u] = j < gg.N ? bidx[j] : -1;
    p[u] = j < gg.N ? y[j] : make_float2(0.f, 0.f);
  }
  float4 row[per][2];                             // per corner row: (img, G) at x0 and at x0 + 1
#pragma unroll
  for (int u = 0; u < per; ++u) {
    const float fx = floorf(p[u].x), fy = floorf(p[u].y);
    const bool ok = batch_ok(bj[u], gg.B) && fx >= -1.f && fx <= (float)(W - 1) && fy >= -1.f &&
                    fy <= (float)(H - 1);
    const int x0 = ok ? (int)fx : 0, y0 = ok ? (int)fy : 0;
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      row[u][r] = make_float4(0.f, 0.f, 0.f, 0.f);
      const int yy = y0 + r;
      if (!ok || yy < 0 || yy >= H) continue;
      const float2* q = ig + bj[u] * pl + (int64_t)yy * W;
      if (x0 >= 0 && x0 + 1 < W) {
        __builtin_memcpy(&row[u][r], q + x0, sizeof(float4));   // both corners: one 16-byte load
      } else {
        if (x0 >= 0) { const float2 c = q[x0]; row[u][r].x = c.x; row[u][r].y = c.y; }
        if (x0 + 1 < W) { const float2 c = q[x0 + 1]; row[u][r].z = c.x; row[u][r].w = c.y; }
      }
    }
  }
  __syncthreads();                                // the run starts are loaded
#pragma unroll
  for (int u = 0; u < per; ++u) {
    const int j = j0 + u * kWsgBlock + threadIdx.x;
    if (j >= gg.N) continue;
    float s1x = 0.f, s1y = 0.f, s2x = 0.f, s2y = 0.f;
    const float fx = floorf(p[u].x), fy = floorf(p[u].y);
    if (batch_ok(bj[u], gg.B) && fx >= -1.f && fx <= (float)(W - 1) && fy >= -1.f && fy <= (float)(H - 1)) {
      const int x0 = (int)fx, y0 = (int)fy;       // for_corners' corners, weights and order
      const float ax = p[u].x - fx, ay = p[u].y - fy;
      const float wx0 = 1.f - ax, wy0 = 1.f - ay;
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int yy = y0 + r;
        if (yy < 0 || yy >= H) continue;
        const float wy = r ? ay : wy0;
        const float dwy = r ? 1.f : -1.f;
        if (x0 >= 0) {                             // corner (x0, yy): wx = 1 - ax, dwx = -1
          const float dcx = -1.f * wy, dcy = wx0 * dwy, v = row[u][r].x, q = row[u][r].y;
          s1x += dcx * v;
          s1y += dcy * v;
          s2x += q * dcx;
          s2y += q * dcy;
        }
        if (x0 + 1 < W) {                          // corner (x0 + 1, yy): wx = ax, dwx = 1
          const float dcx = 1.f * wy, dcy = ax * dwy, v = row[u][r].z, q = row[u][r].w;
          s1x += dcx * v;
          s1y += dcy * v;
          s2x += q * dcx;
          s2y += q * dcy;
        }
      }
    }
    const float g = gvals ? gvals[j] : 0.f;
    const float wj = w[j];
    const float gx = g * s1x + wj * s2x, gy = g * s1y + wj * s2y;
    const float step = t_ref - t[j];
    const float vx = gx * step, vy = gy * step;
    if (!RECS) {
      gv[j] = make_float2(vx, vy);
      continue;
    }
    const float2 x = xy[j];
    const int key = tile_key<kGridVal>(x.x, x.y, bj[u], gg);
    if (key >= 0) rec[atomicAdd(hist + key, 1)] = make_float4(x.x, x.y, vx, vy);
  }
}

// Trajectory adjoint: geometry of m records on a (B, 2K, Hg, Wg) grid (16 x 16 tiles only), the block count of
// its binning, and its workspace: the tile layout, the records' times and the halo slots.
constexpr int kTrajChunk = 8192;                  // records per accumulation workgroup: most tiles take one

bool traj_geo(int64_t K, int64_t B, int64_t Hg, int64_t Wg, int64_t m, TileGeo& g) {
  if (K < 3 || 2 * K > kMaxChannels || !tile_geo(kGrid, B, Hg, Wg, m, 0, 0, g) || g.T != kBinT) return false;
  g.C = (int)(2 * K);
  const int64_t rpb = (int64_t)traj_bin_per(m) * kTrajBinThreads;
  g.nblk = (int)((m + rpb - 1) / rpb);
  return true;
}

struct TrajLayout {
  TileLayout t;
  int64_t tr, halo, bytes;
};

TrajLayout traj_layout(const TileGeo& g) {
  TrajLayout L;
  L.t = tile_layout(g);
  int64_t off = L.t.bytes;
  L.tr = off;   off += align256((int64_t)g.N * 4);
  L.halo = off; off += align256((int64_t)g.nkeys * g.C * kHalo * 4);
  L.bytes = off;
  return L;
}

// Many-channel sampler adjoint: geometry of N look-ups on a (B, C, Hg, Wg) grid, 5 <= C <= 32, 16 x 16 tiles.
bool rows_geo(int64_t C, int64_t B, int64_t Hg, int64_t Wg, int64_t N, int64_t img_h, int64_t img_w, TileGeo& g) {
  if (C < 5 || C > kMaxChannels || !tile_geo(kGrid, B, Hg, Wg, N, img_h, img_w, g) || g.T != kBinT) return false;
  g.C = (int)C;
  const int64_t rpb = (int64_t)traj_bin_per(N) * kTrajBinThreads;
  g.nblk = (int)((N + rpb - 1) / rpb);
  return true;
}

// The scatter launch of the trajectory and many-channel adjoints' records (k_traj_bin<true, ROWS>), which also
// clears the halo slots and writes the chunk list; then tile_halo_accumulate runs the accumulation and the halo
// flush.
template <bool ROWS>
void traj_scatter(const TileGeo& g, const TrajLayout& L, char* w, const float* pos, const float* gd, const float* t,
                  const float* t_last, const int64_t* b, int64_t N, int n_look, int per, hipStream_t stream) {
  const ChunkList cl{(int4*)(w + L.t.info), (int*)(w + L.t.nchunk), kTrajChunk, kTrajChunk};
  hipLaunchKernelGGL((k_traj_bin<true, ROWS>), dim3(g.nblk + 1), dim3(kTrajBinThreads),
                     (size_t)g.nkeys * sizeof(int), stream, (const float2*)pos, (const float2*)gd, t, t_last, b,
                     (int)N, n_look, per, g, (int*)(w + L.t.boff), (float4*)(w + L.t.rec),
                     ROWS ? (float*)nullptr : (float*)(w + L.tr), cl,
                     (float*)(w + L.halo), (int64_t)g.nkeys * g.C * kHalo);
}

template <typename Accum>
void tile_halo_accumulate(const TileGeo& g, const TrajLayout& L, char* w, int64_t m, float* gfield,
                          hipStream_t stream, Accum accum) {
  int4* info = (int4*)(w + L.t.info);
  int* nchunk = (int*)(w + L.t.nchunk);
  float* halo = (float*)(w + L.halo);
  const int64_t nchunks = (int64_t)g.nkeys + (m + kTrajChunk - 1) / kTrajChunk;   // ceil(len / chunk) per tile
  accum((unsigned)nchunks, (const int4*)info, (const int*)nchunk, halo);
  const int64_t nfix = (int64_t)g.nkeys * g.C * (2 * kBinT - 1);
  hipLaunchKernelGGL(k_traj_halo_add, dim3(grid_for(nfix)), dim3(kBlock), 0, stream, (const float*)halo, g, g.C,
                     gfield);
}

}  // namespace

// ================================================================================================ C-ABI
extern "C" {

int64_t atl_tile_ws_bytes(int64_t N, int64_t B, int64_t H, int64_t W) {
  TileGeo g;
  if (!tile_geo(kImage, B, H, W, N, 0, 0, g)) return -1;
  return tile_layout(g).bytes;
}

int atl_splat_bilinear_fwd_ws(const float* pos, const float* w, const int64_t* b, int64_t N, int64_t B, int64_t H,
                              int64_t W, float* img, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (N == 0 || B == 0) return 0;
  TileGeo g;
  if (!tile_geo(kImage, B, H, W, N, 0, 0, g)) { set_error("splat_bilinear_fwd_ws: unsupported sizes N=%lld B=%lld H=%lld W=%lld", (long long)N, (long long)B, (long long)H, (long long)W); return 1; }
  const TileLayout L = tile_layout(g);
  if (!ws || ws_bytes < L.bytes) { set_error("splat_bilinear_fwd_ws: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (!pos || !w || !b || !img) { set_error("splat_bilinear_fwd_ws: null argument"); return 1; }
  tile_bin_accum<kImage, 1>(g, L, ws, pos, b, w, img, stream);
  return check_launch("splat_bilinear_fwd_ws");
}

int atl_init(void) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
    (void)hipGetLastError();                       // no device: nothing to set up
    return 0;
  }
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) { set_error("atl_init: hipGetDevice failed"); return 1; }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  int rc = 0;
  for (int d = 0; d < count && d < kMaxDevices && rc == 0; ++d) {
    if (hipSetDevice(d) != hipSuccess) { set_error("atl_init: hipSetDevice(%d) failed", d); rc = 1; break; }
    rc = noalloc_lookup(d, "atl_init");
  }
  if (hipSetDevice(cur) != hipSuccess && rc == 0) { set_error("atl_init: could not restore device %d", cur); rc = 1; }
  return rc;
}

int atl_splat_bilinear_fwd_noalloc(const float* pos, const float* w, const int64_t* b, int64_t N, int64_t B,
                                   int64_t H, int64_t W, float* img, hipStream_t stream) {
  if (N < 0 || B < 0 || H < 0 || W < 0) { set_error("splat_bilinear_fwd_noalloc: bad sizes"); return 1; }
  if (N == 0 || B == 0) return 0;
  TileGeo g;
  if (!tile_geo(kImage, B, H, W, N, 0, 0, g)) { set_error("splat_bilinear_fwd_noalloc: unsupported sizes N=%lld B=%lld H=%lld W=%lld", (long long)N, (long long)B, (long long)H, (long long)W); return 1; }
  const TileLayout L = tile_layout(g);
  if (L.bytes > kNoAllocScratchBytes) {
    set_error("splat_bilinear_fwd_noalloc: N=%lld B=%lld H=%lld W=%lld needs %lld bytes of scratch, more than the "
              "library's %lld (use atl_splat_bilinear_fwd_ws with a workspace)", (long long)N, (long long)B,
              (long long)H, (long long)W, (long long)L.bytes, (long long)kNoAllocScratchBytes);
    return 1;
  }
  if (!pos || !w || !b || !img) { set_error("splat_bilinear_fwd_noalloc: null argument"); return 1; }
  void* ws = nullptr;
  if (noalloc_scratch(&ws) != 0) return 1;
  tile_bin_accum<kImage, 1>(g, L, ws, pos, b, w, img, stream);
  return check_launch("splat_bilinear_fwd_noalloc");
}

// voxel_grid on the tile engine: the C time bins are the channels of a (T+1)^2 LDS window per tile segment.
constexpr int kMaxVoxelLds = 65536;              // bytes of LDS for one window

static bool voxel_geo(int64_t N, int64_t B, int64_t C, int64_t H, int64_t W, TileGeo& g) {
  if (C < 1 || C > 1024 || !tile_geo(kVoxel, B, H, W, N, 0, 0, g)) return false;
  g.C = (int)C;
  return C * (g.T + 1) * (g.T + 1) * 4 <= kMaxVoxelLds && B * C * H * W < ((int64_t)1 << 31);
}

int64_t atl_voxel_ws_bytes(int64_t N, int64_t B, int64_t C, int64_t H, int64_t W) {
  TileGeo g;
  if (!voxel_geo(N, B, C, H, W, g)) return -1;
  return tile_layout(g).bytes;
}

int atl_voxel_grid_ws(const float* pos, const float* t, const float* p, const int64_t* b, int64_t N, int64_t B,
                      int64_t C, int64_t H, int64_t W, float* vox, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (N < 0 || B < 0 || C < 1 || H < 1 || W < 1) { set_error("voxel_grid_ws: bad sizes"); return 1; }
  if (N == 0 || B == 0) return 0;
  TileGeo g;
  if (!voxel_geo(N, B, C, H, W, g)) { set_error("voxel_grid_ws: unsupported sizes N=%lld B=%lld C=%lld H=%lld W=%lld (use atl_voxel_grid)", (long long)N, (long long)B, (long long)C, (long long)H, (long long)W); return 1; }
  const TileLayout L = tile_layout(g);
  if (!ws || ws_bytes < L.bytes) { set_error("voxel_grid_ws: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (!pos || !t || !p || !b || !vox) { set_error("voxel_grid_ws: null argument"); return 1; }
  tile_bin_accum<kVoxel, 0>(g, L, ws, pos, b, p, vox, stream, t);
  return check_launch("voxel_grid_ws");
}

int atl_gather_bilinear_bwd_ws(const float* gval, const float* img, const float* pos, const int64_t* b, int64_t N,
                               int64_t B, int64_t H, int64_t W, float* gimg, float* gpos, void* ws, int64_t ws_bytes,
                               hipStream_t stream) {
  if (N == 0) return 0;
  TileGeo g;
  if (!tile_geo(kImage, B, H, W, N, 0, 0, g)) { set_error("gather_bilinear_bwd_ws: unsupported sizes"); return 1; }
  const TileLayout L = tile_layout(g);
  if (!ws || ws_bytes < L.bytes) { set_error("gather_bilinear_bwd_ws: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (!gval || !img || !pos || !b || !gimg || !gpos) { set_error("gather_bilinear_bwd_ws: null argument"); return 1; }
  hipLaunchKernelGGL(k_gather_bwd_pos, dim3(grid_for(N)), dim3(kBlock), 0, stream, gval, img, (const float2*)pos, b,
                     N, B, (int)H, (int)W, (float2*)gpos);
  tile_bin_accum<kImage, 1>(g, L, ws, pos, b, gval, gimg, stream);
  return check_launch("gather_bilinear_bwd_ws");
}

int64_t atl_splat_gauss_ws_bytes(int64_t N, int64_t B, int64_t H, int64_t W, int64_t R) {
  TileGeo g;
  if (!tile_geo(kGauss, B, H, W, N, 0, 0, g, (int)R)) return -1;
  return tile_layout(g).bytes;
}

int atl_splat_gauss_fwd_ws(const float* pos, const float* w, const int64_t* b, int64_t N, int64_t B, int64_t H,
                           int64_t W, double sigma, int64_t R, float* img, void* ws, int64_t ws_bytes,
                           hipStream_t stream) {
  if (N == 0 || B == 0) return 0;
  TileGeo g;
  if (!(sigma > 0) || !tile_geo(kGauss, B, H, W, N, 0, 0, g, (int)R)) { set_error("splat_gauss_fwd_ws: unsupported arguments (sigma=%g R=%lld)", sigma, (long long)R); return 1; }
  const TileLayout L = tile_layout(g);
  if (!ws || ws_bytes < L.bytes) { set_error("splat_gauss_fwd_ws: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (!pos || !w || !b || !img) { set_error("splat_gauss_fwd_ws: null argument"); return 1; }
  const float s2 = (float)(sigma * sigma);        // the per-event kernel's constants, same fp32 expressions
  g.inv2s2 = 1.f / (2.f * s2);
  g.norm = 1.f / (2.f * (float)M_PI * s2);
  tile_bin_accum<kGauss, 1>(g, L, ws, pos, b, w, img, stream);
  return check_launch("splat_gauss_fwd_ws");
}

// Flow-grid adjoint through a tile plan: atl_grid_plan bins the positions once (in the forward), and
// atl_sample_grid_bwd_planned accumulates gout into gfield tile by tile.
int64_t atl_grid_plan_bytes(int64_t B, int64_t Hg, int64_t Wg, int64_t N) {
  TileGeo g;
  if (!tile_geo(kGrid, B, Hg, Wg, N, 0, 0, g)) return -1;
  return tile_layout(g).bytes;
}

int atl_grid_plan(int64_t B, int64_t Hg, int64_t Wg, const float* pos, const int64_t* b, int64_t N, int64_t img_h,
                  int64_t img_w, void* ws, int64_t ws_bytes, hipStream_t stream) {
  TileGeo g;
  if (!tile_geo(kGrid, B, Hg, Wg, N, img_h, img_w, g)) { set_error("grid_plan: bad sizes B=%lld Hg=%lld Wg=%lld N=%lld", (long long)B, (long long)Hg, (long long)Wg, (long long)N); return 1; }
  const TileLayout L = tile_layout(g);
  if (!ws || ws_bytes < L.bytes) { set_error("grid_plan: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (N > 0 && (!pos || !b)) { set_error("grid_plan: null input"); return 1; }
  tile_bin<kGrid>(g, L, ws, pos, b, nullptr, stream);
  return check_launch("grid_plan");
}

int atl_sample_grid_bwd_binned(const float* gout, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                               const int64_t* b, int64_t N, int64_t img_h, int64_t img_w, float* gfield, void* ws,
                               int64_t ws_bytes, hipStream_t stream) {
  TileGeo g;
  if (!tile_geo(kGridVal, B, Hg, Wg, N, img_h, img_w, g) || C < 1 || C > 2) { set_error("sample_grid_bwd_binned: bad sizes (C <= 2, at most 16384 tiles)"); return 1; }
  g.C = (int)C;
  const TileLayout L = tile_layout(g);
  if (!ws || ws_bytes < L.bytes) { set_error("sample_grid_bwd_binned: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (N == 0) return 0;
  if (!gout || !pos || !b || !gfield) { set_error("sample_grid_bwd_binned: null argument"); return 1; }
  if (C == 1)
    tile_bin_accum<kGridVal, 1>(g, L, ws, pos, b, gout, gfield, stream);
  else
    tile_bin_accum<kGridVal, 2>(g, L, ws, pos, b, gout, gfield, stream);
  return check_launch("sample_grid_bwd_binned");
}

int atl_sample_grid_bwd_planned(const float* gout, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                                int64_t N, int64_t img_h, int64_t img_w, void* ws, float* gfield,
                                hipStream_t stream) {
  TileGeo g;
  if (!tile_geo(kGrid, B, Hg, Wg, N, img_h, img_w, g) || C < 1 || C > kMaxChannels || (C > 4 && g.T != 16)) { set_error("sample_grid_bwd_planned: bad sizes (C <= 4, or C <= 32 on grids of at most 16384 16x16 tiles)"); return 1; }
  g.C = (int)C;
  g.vec4 = (C & 3) == 0 && (reinterpret_cast<uintptr_t>(gout) & 15) == 0;
  if (!ws || !gfield || (N > 0 && !gout)) { set_error("sample_grid_bwd_planned: null argument"); return 1; }
  (void)pos;                                     // the plan's records carry the positions
  const TileLayout L = tile_layout(g);
  switch (C) {
    case 1: tile_accum<kGrid, 1>(g, L, ws, gout, gfield, stream); break;
    case 2: tile_accum<kGrid, 2>(g, L, ws, gout, gfield, stream); break;
    case 3: tile_accum<kGrid, 3>(g, L, ws, gout, gfield, stream); break;
    case 4: tile_accum<kGrid, 4>(g, L, ws, gout, gfield, stream); break;
    default:
      if (g.T == kBinT && !tile_scatter_form()) {   // gather form (C > 4 is only planned with 16 x 16 tiles)
        if (g.nblk == 0) break;
        char* w = (char*)ws;
        int4* info = (int4*)(w + L.info);
        int* nchunk = (int*)(w + L.nchunk);
        hipLaunchKernelGGL(k_tile_chunks, dim3(1), dim3(kChunkScanBlock), 0, stream, (const int*)(w + L.boff), g,
                           kAccChunk, kBinChunk, info, nchunk);
        hipLaunchKernelGGL(k_tile_accum_rows, dim3((unsigned)max_chunks(g)), dim3(kAccBlock),
                           (size_t)C * (kBinT + 1) * (kBinT + 1) * sizeof(float), stream, (const int4*)info,
                           (const int*)nchunk, (const float4*)(w + L.rec), gout, g, gfield, (const float2*)nullptr,
                           (const float*)nullptr);
      } else {
        tile_accum<kGrid, 0>(g, L, ws, gout, gfield, stream);
      }
      break;
  }
  return check_launch("sample_grid_bwd_planned");
}

int atl_traj_field_bwd_planned(const float* gd, const float* t, int64_t K, int64_t B, int64_t Hg, int64_t Wg,
                               int64_t N, void* ws, float* gfield, hipStream_t stream) {
  TileGeo g;
  if (K < 3 || 2 * K > kMaxChannels || !tile_geo(kGrid, B, Hg, Wg, N, 0, 0, g) || g.T != kBinT) {
    set_error("traj_field_bwd_planned: bad sizes (3 <= K <= %d on grids of at most 16384 16x16 tiles)", kMaxChannels / 2);
    return 1;
  }
  g.C = (int)(2 * K);
  g.vec4 = false;
  if (!ws || !gfield || (N > 0 && (!gd || !t))) { set_error("traj_field_bwd_planned: null argument"); return 1; }
  if (N == 0 || g.nblk == 0) return 0;
  const TileLayout L = tile_layout(g);
  char* w = (char*)ws;
  int4* info = (int4*)(w + L.info);
  int* nchunk = (int*)(w + L.nchunk);
  // with more than kBinChunk / 2 records per tile on average (the many-step origin adjoints), chunks of kBinChunk
  // records (four accumulation rounds per workgroup): a window is cleared and flushed once per 2048 records, not
  // per 512; sparser planes keep the 512-record chunks, which spread a dense tile over more workgroups
  const int chunk = N > (int64_t)g.nkeys * (kBinChunk / 2) ? kBinChunk : kAccChunk;
  hipLaunchKernelGGL(k_tile_chunks, dim3(1), dim3(kChunkScanBlock), 0, stream, (const int*)(w + L.boff), g, chunk,
                     kBinChunk, info, nchunk);
  hipLaunchKernelGGL(k_tile_accum_rows, dim3((unsigned)max_chunks(g)), dim3(kAccBlock),
                     (size_t)g.C * (kBinT + 1) * (kBinT + 1) * sizeof(float), stream, (const int4*)info,
                     (const int*)nchunk, (const float4*)(w + L.rec), (const float*)nullptr, g, gfield,
                     (const float2*)gd, t);
  return check_launch("traj_field_bwd_planned");
}

int64_t atl_traj_field_bwd_bytes(int64_t K, int64_t B, int64_t Hg, int64_t Wg, int64_t n_rec) {
  TileGeo g;
  if (!traj_geo(K, B, Hg, Wg, n_rec, g)) return -1;
  return traj_layout(g).bytes;
}

int atl_traj_field_bwd(const float* gd, const float* pos, const float* t, const float* t_last, const int64_t* b,
                       int64_t N, int64_t n_look, int64_t K, int64_t B, int64_t Hg, int64_t Wg, void* ws,
                       int64_t ws_bytes, float* gfield, hipStream_t stream) {
  if (N < 0 || n_look < 1 || (double)N * (double)n_look >= (double)(1 << 30)) {
    set_error("traj_field_bwd: bad record count N=%lld n_look=%lld", (long long)N, (long long)n_look);
    return 1;
  }
  const int64_t m = N * n_look;
  TileGeo g;
  if (!traj_geo(K, B, Hg, Wg, m, g)) {
    set_error("traj_field_bwd: bad sizes (3 <= K <= %d on grids of at most 16384 16x16 tiles)", kMaxChannels / 2);
    return 1;
  }
  const TrajLayout L = traj_layout(g);
  if (!ws || ws_bytes < L.bytes) { set_error("traj_field_bwd: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (m == 0) return 0;
  if (!gd || !pos || !t || !b || !gfield) { set_error("traj_field_bwd: null argument"); return 1; }
  char* w = (char*)ws;
  int* cnt = (int*)(w + L.t.cnt);
  int* boff = (int*)(w + L.t.boff);
  float4* rec = (float4*)(w + L.t.rec);
  float* tr = (float*)(w + L.tr);
  const int per = traj_bin_per(m);
  const size_t lds = (size_t)g.nkeys * sizeof(int);
  hipLaunchKernelGGL(k_traj_bin<false>, dim3(g.nblk), dim3(kTrajBinThreads), lds, stream, (const float2*)pos,
                     (const float2*)gd, t, t_last, b, (int)N, (int)n_look, per, g, cnt, (float4*)nullptr,
                     (float*)nullptr, ChunkList{}, (float*)nullptr, (int64_t)0);
  scan32t(cnt, g.nkeys, g.nblk, (int*)(w + L.t.part), boff, stream);
  traj_scatter<false>(g, L, w, pos, gd, t, t_last, b, N, (int)n_look, per, stream);
  tile_halo_accumulate(g, L, w, m, gfield, stream, [&](unsigned grid, const int4* info, const int* nchunk, float* halo) {
    auto launch = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(grid), dim3(kAccBlock), 0, stream, info, nchunk, (const float4*)rec,
                         (const float*)tr, g, (int)K, gfield, halo);
    };
    if (K <= 4)
      launch(k_traj_tile_accum<4>);
    else if (K <= 8)
      launch(k_traj_tile_accum<8>);
    else if (K <= 10)
      launch(k_traj_tile_accum<10>);
    else if (K <= 12)
      launch(k_traj_tile_accum<12>);
    else
      launch(k_traj_tile_accum<16>);
  });
  return check_launch("traj_field_bwd");
}

int64_t atl_sample_grid_bwd_rows_bytes(int64_t B, int64_t C, int64_t Hg, int64_t Wg, int64_t N) {
  TileGeo g;
  if (!rows_geo(C, B, Hg, Wg, N, 0, 0, g)) return -1;
  return traj_layout(g).bytes;
}

int atl_sample_grid_bwd_rows(const float* gout, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                             const int64_t* b, int64_t N, int64_t img_h, int64_t img_w, float* gfield, void* ws,
                             int64_t ws_bytes, hipStream_t stream) {
  TileGeo g;
  if (!rows_geo(C, B, Hg, Wg, N, img_h, img_w, g)) {
    set_error("sample_grid_bwd_rows: bad sizes (5 <= C <= %d on grids of at most 16384 16x16 tiles)", kMaxChannels);
    return 1;
  }
  const TrajLayout L = traj_layout(g);
  if (!ws || ws_bytes < L.bytes) { set_error("sample_grid_bwd_rows: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (N == 0) return 0;
  if (!gout || !pos || !b || !gfield) { set_error("sample_grid_bwd_rows: null argument"); return 1; }
  g.vec4 = (C & 3) == 0 && (reinterpret_cast<uintptr_t>(gout) & 15) == 0;
  char* w = (char*)ws;
  int* cnt = (int*)(w + L.t.cnt);
  int* boff = (int*)(w + L.t.boff);
  float4* rec = (float4*)(w + L.t.rec);
  const int per = traj_bin_per(N);
  const size_t lds = (size_t)g.nkeys * sizeof(int);
  hipLaunchKernelGGL((k_traj_bin<false, true>), dim3(g.nblk), dim3(kTrajBinThreads), lds, stream, (const float2*)pos,
                     (const float2*)nullptr, (const float*)nullptr, (const float*)nullptr, b, (int)N, 1, per, g, cnt,
                     (float4*)nullptr, (float*)nullptr, ChunkList{}, (float*)nullptr, (int64_t)0);
  scan32t(cnt, g.nkeys, g.nblk, (int*)(w + L.t.part), boff, stream);
  traj_scatter<true>(g, L, w, pos, nullptr, nullptr, nullptr, b, N, 1, per, stream);
  tile_halo_accumulate(g, L, w, N, gfield, stream, [&](unsigned grid, const int4* info, const int* nchunk, float* halo) {
    auto launch = [&](auto kern) {
      hipLaunchKernelGGL(kern, dim3(grid), dim3(kAccBlock), 0, stream, info, nchunk, (const float4*)rec, gout, g,
                         gfield, halo);
    };
    if (C <= 8)
      launch(k_rows_tile_accum<8>);
    else if (C <= 12)
      launch(k_rows_tile_accum<12>);
    else if (C <= 16)
      launch(k_rows_tile_accum<16>);
    else if (C <= 20)
      launch(k_rows_tile_accum<20>);
    else if (C <= 24)
      launch(k_rows_tile_accum<24>);
    else
      launch(k_rows_tile_accum<32>);
  });
  return check_launch("sample_grid_bwd_rows");
}

// Warp -> splat -> gather (the fused pipeline above).  Workspace bytes, or -1 for unsupported sizes.
int64_t atl_warp_splat_gather_ws_bytes(int64_t N, int64_t B, int64_t H, int64_t W, int64_t Hg, int64_t Wg) {
  WsgLayout L;
  if (N == 0)                                     // no events: the outputs are zeros, no workspace is read
    return B >= 1 && H >= 1 && W >= 1 && Hg >= 1 && Wg >= 1 && wsg_layout(1, B, H, W, Hg, Wg, L) ? 0 : -1;
  return wsg_layout(N, B, H, W, Hg, Wg, L) ? L.bytes : -1;
}

int atl_warp_splat_gather_fwd(const float* grid, int64_t B, int64_t Hg, int64_t Wg, const float* xy, const float* t,
                              const int64_t* b, int64_t N, int64_t H, int64_t W, double t_ref, int64_t mask_border,
                              float* img, float* vals, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (N == 0) {                                   // img is written: all zero
    if (!img) { set_error("warp_splat_gather_fwd: null argument"); return 1; }
    if (B * H * W > 0)
      hipLaunchKernelGGL(k_fill_zero_f, dim3(grid_for(B * H * W)), dim3(kBlock), 0, stream, img, B * H * W);
    return check_launch("warp_splat_gather_fwd");
  }
  WsgLayout L;
  if (!wsg_layout(N, B, H, W, Hg, Wg, L)) { set_error("warp_splat_gather_fwd: unsupported sizes N=%lld B=%lld H=%lld W=%lld Hg=%lld Wg=%lld", (long long)N, (long long)B, (long long)H, (long long)W, (long long)Hg, (long long)Wg); return 1; }
  if (!ws || ws_bytes < L.bytes) { set_error("warp_splat_gather_fwd: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (!grid || !xy || !t || !b || !img) { set_error("warp_splat_gather_fwd: null argument"); return 1; }
  char* w = (char*)ws;
  const TileGeo& g = L.gi;
  float2* y = (float2*)(w + L.y);
  float* wt = (float*)(w + L.w);
  const float sxw = (float)(W - 1 > 1 ? W - 1 : 1), syh = (float)(H - 1 > 1 ? H - 1 : 1);
  const size_t lds = (size_t)g.nkeys * sizeof(int);
  // with kCountWarp, the flow-grid adjoint's counts too, and one scan over both key spaces
  const bool joint = L.count == kCountWarp;
  const size_t wlds = lds + (joint ? (size_t)L.gg.nkeys * sizeof(int) : 0);
  float* fil = (float*)(w + L.fil);
  if (Wg >= 2 && atl_flow_interleave(grid, B, Hg, Wg, fil, stream) != 0) return 1;
  hipLaunchKernelGGL(Wg >= 2 ? k_wsg_warp<true> : k_wsg_warp<false>, dim3(g.nblk), dim3(kWsgBlock), wlds,
                     stream, grid, (const float*)fil, (int)Hg, (int)Wg, sxw, syh, (const float2*)xy, t, b, (float)t_ref,
                     (int)(mask_border != 0), g, y, wt, (int*)(w + L.Li.cnt), L.nkc, L.gg, joint, img, B * H * W);
  scan32t((int*)(w + L.Li.cnt), L.nkc, g.nblk, (int*)(w + L.Li.part), (int*)(w + L.Li.boff), stream);
  hipLaunchKernelGGL((k_tile_bin<kImage, true, false>), dim3(g.nblk + 1), dim3(kTileBinBlock), lds, stream,
                     (const float2*)y, b, (const float*)wt, g, (int*)(w + L.Li.boff), (float4*)(w + L.Li.rec),
                     (const float*)nullptr, tile_chunk_list<kImage, 1>(g, L.Li, w));
  tile_accum<kImage, 1>(g, L.Li, w, nullptr, img, stream, true);
  if (vals)
    hipLaunchKernelGGL(k_wsg_gather, dim3(grid_for(N)), dim3(kBlock), 0, stream, (const float*)img,
                       (const float2*)y, b, N, B, (int)H, (int)W, vals);
  return check_launch("warp_splat_gather_fwd");
}

int atl_warp_splat_gather_bwd(const float* img, const float* gvals, const float* gimg, const float* xy,
                              const float* t, const int64_t* b, int64_t N, int64_t B, int64_t H, int64_t W,
                              int64_t Hg, int64_t Wg, double t_ref, float* ggrid, void* ws, int64_t ws_bytes,
                              hipStream_t stream) {
  if (N == 0) {                                   // ggrid is written: all zero
    if (!ggrid) { set_error("warp_splat_gather_bwd: null argument"); return 1; }
    if (B * 2 * Hg * Wg > 0)
      hipLaunchKernelGGL(k_fill_zero_f, dim3(grid_for(B * 2 * Hg * Wg)), dim3(kBlock), 0, stream, ggrid,
                         B * 2 * Hg * Wg);
    return check_launch("warp_splat_gather_bwd");
  }
  WsgLayout L;
  if (!wsg_layout(N, B, H, W, Hg, Wg, L)) { set_error("warp_splat_gather_bwd: unsupported sizes"); return 1; }
  if (!ws || ws_bytes < L.bytes) { set_error("warp_splat_gather_bwd: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (!img || !xy || !t || !b || !ggrid) { set_error("warp_splat_gather_bwd: null argument"); return 1; }
  char* w = (char*)ws;
  float2* ig = (float2*)(w + L.G);
  const int64_t npix = B * H * W;
  // (img, G) with G = gimg + splat(y, gvals), the image gradient, accumulated on the forward's records
  hipLaunchKernelGGL(k_wsg_pack, dim3(grid_for(npix)), dim3(kBlock), 0, stream, img, gimg, npix, ig, ggrid,
                     B * 2 * Hg * Wg);
  if (gvals) {
    TileGeo gi = L.gi;
    gi.ilv = 2;
    tile_accum<kImageG, 1>(gi, L.Li, w, gvals, (float*)ig, stream, true);
  }
  const TileGeo& gg = L.gg;
  if (L.count == kCountNone) {                    // a translation: the adjoint is a sum per window
    hipLaunchKernelGGL(k_wsg_grad<false>, dim3(gg.nblk), dim3(kWsgBlock), 0, stream, (const float2*)ig, gvals,
                       (const float2*)(w + L.y), (const float*)(w + L.w), (const float2*)xy, t, b, (float)t_ref,
                       (int)H, (int)W, gg, (float2*)(w + L.gv), (const int*)nullptr, (float4*)nullptr, ChunkList{});
    const unsigned nb = std::min<unsigned>(grid_for(N), kOneNodeBlocks);
    hipLaunchKernelGGL(k_one_node_adjoint, dim3(nb), dim3(kBlock), 0, stream, (const float2*)(w + L.gv), b, N,
                       (int)B, ggrid);
    return check_launch("warp_splat_gather_bwd");
  }
  // the rows' flow-grid tiles were counted and scanned by the forward (kCountWarp) or are here (kCountBwd), and
  // k_wsg_grad writes the records in place
  if (L.count == kCountBwd) {
    hipLaunchKernelGGL((k_tile_bin<kGridVal, false, false>), dim3(gg.nblk), dim3(kTileBinBlock),
                       (size_t)gg.nkeys * sizeof(int), stream, (const float2*)xy, b, (const float*)nullptr, gg,
                       (int*)(w + L.Lg.cnt), (float4*)nullptr, (const float*)nullptr, ChunkList{});
    scan32t((int*)(w + L.Lg.cnt), gg.nkeys, gg.nblk, (int*)(w + L.Lg.part), (int*)(w + L.Lg.boff), stream);
  }
  hipLaunchKernelGGL(k_wsg_grad<true>, dim3(gg.nblk + 1), dim3(kWsgBlock), (size_t)gg.nkeys * sizeof(int),
                     stream, (const float2*)ig, gvals, (const float2*)(w + L.y), (const float*)(w + L.w),
                     (const float2*)xy, t, b, (float)t_ref, (int)H, (int)W, gg, (float2*)nullptr,
                     (const int*)(w + L.Lg.boff), (float4*)(w + L.Lg.rec), tile_chunk_list<kGridVal, 2>(gg, L.Lg, w));
  tile_accum<kGridVal, 2>(gg, L.Lg, w, nullptr, ggrid, stream, true);
  return check_launch("warp_splat_gather_bwd");
}

}  // extern "C"
