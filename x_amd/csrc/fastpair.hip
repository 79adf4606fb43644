// Fused anchored pair sums on gfx950: the reference's (source, slice) entries and the anchors binned into
// one fixed, clamped fine-cell grid per slice, then a gather-form forward (the anchors of one cell share a
// wave, whose lanes take the candidate entries of their neighbourhood) and a source-centric backward (one
// lane per source, walking the anchors around all of its slices), both over disc-pruned rows of fine cells.
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
//
// The plan is a two-level counting sort with no per-item global atomics (scattered global atomics run at
// ~25 G/s on MI355X, against ~450 G/s for coalesced traffic): pass 1 histograms buckets of 1024 keys (more
// for very fine grids) in LDS per block and scatters full records into bucket order; pass 2 gives every
// bucket one workgroup that sorts it by cell with an LDS histogram and writes the cell offsets and the final
// records.  Entries and anchors
// share one key space (anchor keys offset by the padded cell count), so both sorts run in the same
// launches.  The same sort also orders the sources by the cell of their own-slice position (in tiles of
// 8 x 8 cells, so that a wave's sources form a compact patch), and the
// backward gives each source one lane that walks the anchors of all its slices: the gradient of a source
// is complete in registers and written once, without atomics.
#include <algorithm>
#include <type_traits>

#include "common.h"
#include "scan.h"
#include "bilinear.h"
#include "../../include/atl_hip.h"

#include <cmath>

using namespace atlhip;

namespace {

// Buckets hold 2^bshift keys, bshift the smallest of kMinBucketShift.. that keeps the bucket count within
// kMaxBuckets (the pass-1 LDS histogram).  Small buckets keep pass 2 balanced (two LDS arrays of 4 KB each).
constexpr int kMinBucketShift = 10;
constexpr int kMaxBucketShift = 13;
constexpr int kMaxBuckets = 16384;
static_assert(kMaxBuckets <= kScanSmallMax, "bucket totals are scanned by one workgroup");
constexpr int kSortBlock = 512;                    // pass-2 workgroup
constexpr int kP1Block = 1024;                     // pass-1 workgroup
constexpr int kSrcPerBlock = 4096;                 // pass-1 sources per block (4 per thread)
constexpr int kAncPerBlock = 8192;                 // pass-1 anchors per block (8 per thread)
constexpr int kUnroll = 8;                         // record arrays padded by the longest walk step
constexpr int kStep = 4;                           // candidates per walk step
constexpr int kStepLong = 8;                       // the step of a wave whose walks are long (dense neighbourhoods)
constexpr int kLongWalk = 256;                     // a lane's slice candidates above which its wave steps long
constexpr int kSliceBatch = 4;                     // pass 1: slices of one source keyed and placed together

constexpr int kXcd = 8;                            // XCDs: consecutive workgroups go round-robin over them
constexpr int kTrajPairMaxK = 12;                  // trajectory model: coefficients per axis (K) the kernels take

// Fixed geometry shared by every kernel (host-computed, passed by value).
struct FGeo {
  float gx0, gy0, gx1, gy1;    // clamp box; cell (0, 0) starts at (gx0, gy0)
  float cf;                    // fine cell size
  float icf;                   // 1 / cf (fp32), for the walks' conservative cell lookups
  int GW, GH, S;
  int64_t B;
  int ncell;                   // B * S * GH * GW
  int ncell_pad;               // ncell rounded up to whole buckets: anchor keys start here, source keys at 2x
  int MS;                      // max slices per source
  int nblk_e, nblk_a;          // pass-1 blocks over sources, over anchors
  int nbuckets;                // 3 * ncell_pad >> bshift
  int bshift;                  // log2 of the keys per bucket
  float tau, half_delta, delta;
  float r2max, kexp, invh2;    // (cut*cut)*h*h, -log2(e)/(2 h h), 1/(h h)
  float cuth;                  // cut * h
  int gcells;                  // forward groups: cells of one row per group
  int stile;                   // source order: tiles of stile x stile cells (about kSrcTilePx px)
  int vplanes;                 // B * S <= kMaxPlanes: the plan keeps every (batch, slice) plane's max ||v||
};

// Planes (batch, slice) whose largest entry velocity the plan keeps (after FParams in the workspace): the
// forward's walks around anchors of plane (b, s) then use that plane's bound instead of the global one.
constexpr int kMaxPlanes = 1024;

// Device scalars written by the plan (ordered-int encodings of non-negative floats).
struct FParams {
  int vmax;                    // max ||v|| over sources
  int atmax;                   // max |t_a - c_s| over anchors
  int dup;                     // non-zero if an event occurs more than once among the anchors
  int unique;                  // non-zero if the anchors are every event in order (no index array): no repeats
  int nonfinite;               // non-zero if a backward record (anchor position, time or gS) is not finite
  int planes;                  // non-zero if the per-plane maxima below were written (trajectory plans)
  int pad[2];
};                             // followed by B * S ints (ordered): each plane's max ||v|| when `planes`

__device__ __forceinline__ int* plane_vmax(const FParams* P) { return (int*)(P + 1) ; }

// One 32-byte record per sorted item, written with a single scattered line (separate arrays would cost one
// scattered cache line each, and scattered lines are what the sort pays for):
//   entries  f = (y.x, y.y, v.x, v.y) at the slice centre, i = (t bits, source id, key, 0)
//   anchors  f = (x, y, t, at),                            i = (event id, input position, key, cy << 16 | cx)
//   sources  f = (x, y, v.x, v.y),                         i = (t bits, source id, key, 0)
// key is the cell key within the item's own key space (the tmp records carry the combined key).
struct Rec {
  float4 f;
  int4 i;
};

__device__ __forceinline__ float ordered_to_float(int i) { return __int_as_float(i >= 0 ? i : i ^ 0x7fffffff); }

// Search radius from the device reductions: every contributing pair lies within R of its query (cut*h and
// the largest displacement v*at, each with relative slack, plus 0.01 px for fp32 rounding of positions).
__device__ __forceinline__ void search_radius(const FParams* P, const FGeo& G, float& R, float& R2) {
  const float vmax = ordered_to_float(P->vmax), atmax = ordered_to_float(P->atmax);
  R = G.cuth * 1.000001f + vmax * atmax * 1.000001f + 0.01f;
  if (!(R < 1e30f)) {          // inf / NaN velocities: walk the whole slice
    R = 1e30f;
    R2 = 1e30f;
    return;
  }
  R2 = R * R;
}

__device__ __forceinline__ float clampf(float p, float lo, float hi) { return fminf(fmaxf(p, lo), hi); }

// Cell of a position: floor((clamp(p) - lo) / cf) by a multiplication with 1/cf.  The binning and the walk
// bounds use this same monotone function, so an item at p with lo_q <= p <= hi_q lies in a cell between
// cell(lo_q) and cell(hi_q); the 0.01 px slack in R covers the rounding of the walk bounds themselves.
__device__ __forceinline__ int cell_walk(float p, float lo, float hi, float icf, int n) {
  const float c = fminf(fmaxf(p, lo), hi);          // NaN -> lo
  const int i = (int)floorf((c - lo) * icf);
  return min(max(i, 0), n - 1);
}

// Element i of an array through a 32-bit byte offset from a uniform base (lets the compiler use the
// scalar-base + vector-offset addressing form instead of per-lane 64-bit address arithmetic).
template <typename T>
__device__ __forceinline__ T ld(const T* base, uint32_t i) {
  return *(const T*)((const char*)base + i * (uint32_t)sizeof(T));
}

// Workgroup index such that runs of kXcdRun consecutive logical blocks (neighbouring cells) execute on one
// XCD and share its L2, while the runs still alternate over the XCDs (the hardware places workgroup w on
// XCD w % 8) so that every XCD sees every part of the problem.  -1 for the padding blocks of the last group.
constexpr int kXcdRun = 64;
__device__ __forceinline__ int xcd_block(int nblocks) {
  const int w = blockIdx.x;
  const int grp = w / (kXcd * kXcdRun), rem = w - grp * (kXcd * kXcdRun);
  const int logical = grp * (kXcd * kXcdRun) + (rem % kXcd) * kXcdRun + rem / kXcd;
  return logical < nblocks ? logical : -1;
}

// Slice range of a source, atl/ops/functional.py:151-152 (same fp32 order as the reference plan).
__device__ __forceinline__ void slice_range(float t, const FGeo& g, int& lo, int& hi) {
  const float a = (((t - g.tau) - g.half_delta) / g.delta) - 0.5f;
  const float c = (((t + g.tau) + g.half_delta) / g.delta) - 0.5f;
  lo = (int)fminf(fmaxf(ceilf(a), 0.f), (float)(g.S - 1));
  hi = (int)fminf(fmaxf(floorf(c), 0.f), (float)(g.S - 1));
  hi = min(hi, lo + g.MS - 1);
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
  const float w = __builtin_amdgcn_sqrtf(fmaxf(R2 - gap * gap, 0.f));   // ~1 ulp: far inside the slack
  c0 = cell_walk(qx - w, G.gx0, G.gx1, G.icf, G.GW);
  c1 = cell_walk(qx + w, G.gx0, G.gx1, G.icf, G.GW);
  return true;
}

// Cell key of an entry of slice s at slice-centre position (yx, yy).
__device__ __forceinline__ int entry_key_at(float yx, float yy, int bj, int s, const FGeo& G) {
  const int cx = cell_walk(yx, G.gx0, G.gx1, G.icf, G.GW), cy = cell_walk(yy, G.gy0, G.gy1, G.icf, G.GH);
  return ((bj * G.S + s) * G.GH + cy) * G.GW + cx;
}

// Entry (j, s) of the linear model: slice-centre position (functional.py:157-158) and cell key.
__device__ __forceinline__ int entry_key(float2 xj, float2 vj, float tj, int bj, int s, const FGeo& G, float& yx,
                                         float& yy) {
  const float dt = slice_centre(s, G.delta) - tj;
  yx = xj.x + vj.x * dt;
  yy = xj.y + vj.y * dt;
  return entry_key_at(yx, yy, bj, s, G);
}

// Entry (j, s) of the trajectory model: source j carries its trajectory start p and its 2K coefficients
// cf = [y_1..y_K, x_1..x_K]; tab row s = [g_1..g_K(c_s), g_1'..g_K'(c_s)].  The slice-centre position is
// y = p + sum_k cf_k g_k(c_s) and the velocity v = sum_k cf_k g_k'(c_s), each sum in k order in fp32.
template <int K>
__device__ __forceinline__ void traj_entry(const float (&cf)[2 * K], float px, float py,
                                           const float* __restrict__ tab, int s, float& yx, float& yy, float& vx,
                                           float& vy) {
  const float* row = tab + s * 2 * K;
  float dx = 0.f, dy = 0.f, ux = 0.f, uy = 0.f;
#pragma unroll
  for (int k = 0; k < K; ++k) {
    const float g = row[k], gd = row[K + k];
    dy = dy + cf[k] * g;
    dx = dx + cf[K + k] * g;
    uy = uy + cf[k] * gd;
    ux = ux + cf[K + k] * gd;
  }
  yx = px + dx;
  yy = py + dy;
  vx = ux;
  vy = uy;
}

// Sources are ordered by their own-slice cell in tile order: bands of G.stile cell rows, within a band tiles
// of G.stile columns, within a tile row by row.  This is a bijection of the cells of a plane onto
// [0, GH * GW) (partial tiles at the right and bottom edges included), so the key space is the entries' and
// the plane index is still key / (GH * GW); 64 consecutive sources then cover a compact patch rather than a
// strip of a row, which keeps a wave's neighbourhoods (and its staged anchors) small.
// The tiles are about kSrcTilePx px on a side whatever the cell size: the flow adjoint accumulates a tile's
// records in a window of 16 x 16 grid nodes, and a tile of 8 cells of 3 px (h = 2) overflowed it.
constexpr double kSrcTilePx = 12.0;
__device__ __forceinline__ int source_key(int key, const FGeo& G) {
  const int pc = G.GH * G.GW, T = G.stile;
  const int plane = key / pc, rem = key - plane * pc;
  const int cy = rem / G.GW, cx = rem - cy * G.GW;
  const int band = cy / T, ly = cy - band * T, tx = cx / T, lx = cx - tx * T;
  const int hb = min(T, G.GH - band * T), wt = min(T, G.GW - tx * T);
  return plane * pc + band * T * G.GW + tx * T * hb + ly * wt + lx;
}

// Anchor m: slice floor(t / delta) clamped (functional.py:171), fine cell of its clamped position; the key
// is offset by ncell_pad into the anchors' half of the key space.
__device__ __forceinline__ bool anchor_rec(int64_t m, const float2* x, const float* t, const int64_t* b,
                                           const int64_t* anchors, const float2* anchor_xy, int64_t N,
                                           const FGeo& G, int& key, Rec& rec) {
  const int64_t a = anchors ? anchors[m] : m;     // no index array: every event is its own anchor
  if (a < 0 || a >= N) return false;
  const int64_t ba = b[a];
  if (ba < 0 || ba >= G.B) return false;
  const float ta = t[a];
  const float2 xa = anchor_xy ? anchor_xy[m] : x[a];
  const int s = (int)fminf(fmaxf(floorf(ta / G.delta), 0.f), (float)(G.S - 1));   // = anchor_slice(ta, G)
  const int cx = cell_walk(xa.x, G.gx0, G.gx1, G.icf, G.GW), cy = cell_walk(xa.y, G.gy0, G.gy1, G.icf, G.GH);
  key = G.ncell_pad + ((((int)ba * G.S + s) * G.GH + cy) * G.GW + cx);
  rec.f = make_float4(xa.x, xa.y, ta, ta - slice_centre(s, G.delta));
  rec.i = make_int4((int)a, (int)m, key, (cy << 16) | cx);
  return true;
}

// ------------------------------------------------------------------------------------------ plan
__global__ void __launch_bounds__(kBlock) k_fill_zero(int* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}



// Pass 1.  Blocks [0, nblk_a) cover kAncPerBlock anchors each, blocks [nblk_a, nblk_a + nblk_e) kSrcPerBlock
// sources each (their entries and one source record keyed by the cell of the own-slice entry).
// SCATTER = false: per-block bucket histogram into cnt[block * nbuckets + bucket] (block-major: written and read
// back coalesced), its non-zero counts added into the bucket totals tot[bucket], and the reductions behind the
// search radius: vmax over the sources' velocities and max |at| over the anchors (block maxima, one atomic max
// per block into P, zeroed beforehand; ordered-int encodings of non-negative floats).  SCATTER = true: the block
// reserves its run of every bucket it feeds with one atomic add on the bucket's position bpos[bucket] (the
// exclusive scan of the totals; after this pass it holds the bucket's end), keeps the run starts in LDS, and
// each record takes its slot.  The runs of one bucket follow in no fixed block order; pass 2 orders the bucket.
// The source model: K = 0 linear (x, v per source: y = x + v (c_s - t), the reference's), K > 0 trajectories
// (x = the trajectory start p, `coef` the (N, 2K) coefficient rows, `tab` the (S, 2K) slice-centre basis table).
// ENT = false (linear model, SCATTER only): the entries are counted (the totals fix every bucket's place) but not
// written: the block reserves runs of the anchor and source buckets only, and k_entry_pass writes the entries
// later from the sorted source records.
template <bool SCATTER, int K, bool ENT = true>
__global__ void __launch_bounds__(kP1Block) k_sort_pass1(const float2* __restrict__ x, const float* __restrict__ t,
                                                       const float2* __restrict__ v, const int64_t* __restrict__ b,
                                                       int64_t N, const int64_t* __restrict__ anchors,
                                                       const float2* __restrict__ anchor_xy, int64_t M, FGeo G,
                                                       int* __restrict__ cnt, int* __restrict__ bsum,
                                                       Rec* __restrict__ trec, FParams* __restrict__ P,
                                                       int* __restrict__ self, int* __restrict__ eself,
                                                       const float* __restrict__ coef,
                                                       const float* __restrict__ tab) {
  extern __shared__ int hist[];
  __shared__ int red[kP1Block / kWave];
  __shared__ int vpl[kMaxPlanes];                // the block's max ||v|| per (batch, slice) plane (count pass)
  int vm = 0;                                    // this thread's max ||v|| (sources) or max |at| (anchors)
  const int blk = blockIdx.x;
  // the trajectory model's velocities differ by slice and trajectory (the fastest few set the global bound); the
  // linear model's per-plane maxima bought nothing measurable and cost the count pass contended LDS atomics
  const int nplanes = !SCATTER && K > 0 && G.vplanes ? (int)G.B * G.S : 0;
  for (int i = threadIdx.x; i < nplanes; i += blockDim.x) vpl[i] = 0;
  if (nplanes && blk == 0 && threadIdx.x == 0) P->planes = 1;
  int* __restrict__ mycnt = cnt + (int64_t)blk * G.nbuckets;
  const int bpk = G.ncell_pad >> G.bshift;       // buckets per key space (the entries' buckets come first)
  for (int i = threadIdx.x; i < G.nbuckets; i += blockDim.x) {
    int h = 0;
    if (SCATTER && (ENT || i >= bpk)) {
      const int c = mycnt[i];
      if (c > 0) h = atomicAdd(bsum + i, c);   // bsum = bpos: this block's run of bucket i
    }
    hist[i] = h;
  }
  if (!SCATTER && blk == 0 && threadIdx.x == 0 && !anchors) P->unique = 1;
  __syncthreads();
  // anchor blocks first: they are about a quarter of a source block's work, and dispatched last they would
  // queue on the few CUs left free by the source blocks
  const bool src_blk = blk >= G.nblk_a;
  if (src_blk && K > 0) {
    // trajectory sources, one at a time: the 2K coefficients stay in registers across the source's slices
    constexpr int KK = K > 0 ? K : 1;
    const int64_t j0 = (int64_t)(blk - G.nblk_a) * kSrcPerBlock;
    for (int u = 0; u < kSrcPerBlock / kP1Block; ++u) {
      const int64_t j = j0 + u * kP1Block + threadIdx.x;
      if (j >= N) break;
      if (!SCATTER) {
        self[j] = -1;
        eself[j] = -1;
      }
      const int64_t bj = b[j];
      if (bj < 0 || bj >= G.B) continue;
      const float tj = t[j];
      const float2 pj = x[j];
      float cf[2 * KK];
#pragma unroll
      for (int c = 0; c < 2 * KK; ++c) cf[c] = coef[j * (2 * KK) + c];
      int lo, hi;
      slice_range(tj, G, lo, hi);
      const int own = min(max((int)fminf(fmaxf(floorf(tj / G.delta), 0.f), (float)(G.S - 1)), lo), hi);
      for (int s = lo; s <= hi; ++s) {
        float yx, yy, vx, vy;
        traj_entry<KK>(cf, pj.x, pj.y, tab, s, yx, yy, vx, vy);
        if (!SCATTER) {
          const int vo = float_to_ordered(sqrtf(vx * vx + vy * vy));
          vm = max(vm, vo);
          // the lanes of a wave mostly share a plane: the atomic only where the running maximum is exceeded
          if (nplanes && vo > vpl[(int)bj * G.S + s]) atomicMax(vpl + (int)bj * G.S + s, vo);
        }
        const int key = entry_key_at(yx, yy, (int)bj, s, G);
        const int slot = atomicAdd(hist + (key >> G.bshift), 1);
        int sslot = -1, skey = -1;
        if (s == own) {                          // the source record goes with its own slice
          skey = 2 * G.ncell_pad + source_key(key, G);
          sslot = atomicAdd(hist + (skey >> G.bshift), 1);
        }
        if (SCATTER) {
          Rec r;
          r.f = make_float4(yx, yy, vx, vy);
          r.i = make_int4(__float_as_int(tj), (int)j, key, 0);
          trec[slot] = r;
          if (sslot >= 0) {
            r.f = make_float4(pj.x, pj.y, 0.f, 0.f);
            r.i = make_int4(__float_as_int(tj), (int)j, skey, 0);
            trec[sslot] = r;
          }
        }
      }
    }
  } else if (src_blk && SCATTER && !ENT) {
    // the source record only: keyed by the cell of the own-slice entry, in the entries' fp32 operations.  All
    // loads first (indices clamped to the last source), so that they are in flight together.
    constexpr int per = kSrcPerBlock / kP1Block;
    const int64_t j0 = (int64_t)(blk - G.nblk_a) * kSrcPerBlock + threadIdx.x;
    int64_t bs[per];
    float ts[per];
    float2 xs[per], vs[per];
#pragma unroll
    for (int u = 0; u < per; ++u) {
      const int64_t j = min(j0 + u * kP1Block, N - 1);
      bs[u] = b[j];
      ts[u] = t[j];
      xs[u] = x[j];
      vs[u] = v[j];
    }
#pragma unroll
    for (int u = 0; u < per; ++u) {
      const int64_t j = j0 + u * kP1Block;
      const int64_t bj = bs[u];
      if (j >= N || bj < 0 || bj >= G.B) continue;
      const float tj = ts[u];
      const float2 xj = xs[u], vj = vs[u];
      int lo, hi;
      slice_range(tj, G, lo, hi);
      if (lo > hi) continue;                     // no entries, no record (as in the batched loop below)
      const int own = min(max((int)fminf(fmaxf(floorf(tj / G.delta), 0.f), (float)(G.S - 1)), lo), hi);
      float yx, yy;
      const int skey = 2 * G.ncell_pad + source_key(entry_key(xj, vj, tj, (int)bj, own, G, yx, yy), G);
      Rec r;
      r.f = make_float4(xj.x, xj.y, vj.x, vj.y);
      r.i = make_int4(__float_as_int(tj), (int)j, skey, 0);
      trec[atomicAdd(hist + (skey >> G.bshift), 1)] = r;
    }
  } else if (src_blk) {
    constexpr int per = kSrcPerBlock / kP1Block;
    const int64_t j0 = (int64_t)(blk - G.nblk_a) * kSrcPerBlock;
    float2 xj[per], vj[per];
    float tj[per];
    int64_t bj[per];
#pragma unroll
    for (int u = 0; u < per; ++u) {              // all loads of the thread's sources first
      const int64_t j = j0 + u * kP1Block + threadIdx.x;
      bj[u] = j < N ? b[j] : -1;
      if (j < N) {
        tj[u] = t[j];
        xj[u] = x[j];
        vj[u] = v[j];
        if (!SCATTER) {                            // "no anchor record" / "no own-slice entry" until pass 2
          self[j] = -1;
          eself[j] = -1;
        }
      }
    }
#pragma unroll
    for (int u = 0; u < per; ++u) {
      const int64_t j = j0 + u * kP1Block + threadIdx.x;
      if (bj[u] < 0 || bj[u] >= G.B) continue;
      if (!SCATTER) vm = max(vm, float_to_ordered(sqrtf(vj[u].x * vj[u].x + vj[u].y * vj[u].y)));
      int lo, hi;
      slice_range(tj[u], G, lo, hi);
      const int own = min(max((int)fminf(fmaxf(floorf(tj[u] / G.delta), 0.f), (float)(G.S - 1)), lo), hi);
      // kSliceBatch slices at a time: keys, then all LDS slot atomics, then all stores (no atomic -> store
      // round trip per record)
      for (int s0 = lo; s0 <= hi; s0 += kSliceBatch) {
        int key[kSliceBatch + 1], slot[kSliceBatch + 1];
        float yx[kSliceBatch], yy[kSliceBatch];
#pragma unroll
        for (int q = 0; q < kSliceBatch; ++q) key[q] = entry_key(xj[u], vj[u], tj[u], (int)bj[u], min(s0 + q, hi), G,
                                                                yx[q], yy[q]);
        const int oq = own - s0;                   // the source record goes with its own slice
        key[kSliceBatch] = -1;
#pragma unroll
        for (int q = 0; q < kSliceBatch; ++q)
          if (q == oq) key[kSliceBatch] = 2 * G.ncell_pad + source_key(key[q], G);
#pragma unroll
        for (int q = 0; q <= kSliceBatch; ++q) {
          const bool live = q < kSliceBatch ? s0 + q <= hi : key[kSliceBatch] >= 0;
          if (live) slot[q] = atomicAdd(hist + (key[q] >> G.bshift), 1);
        }
        if (SCATTER) {
#pragma unroll
          for (int q = 0; q < kSliceBatch; ++q) {
            if (s0 + q > hi) continue;
            Rec r;
            r.f = make_float4(yx[q], yy[q], vj[u].x, vj[u].y);
            r.i = make_int4(__float_as_int(tj[u]), (int)j, key[q], 0);
            trec[slot[q]] = r;
          }
          if (key[kSliceBatch] >= 0) {
            Rec r;
            r.f = make_float4(xj[u].x, xj[u].y, vj[u].x, vj[u].y);
            r.i = make_int4(__float_as_int(tj[u]), (int)j, key[kSliceBatch], 0);
            trec[slot[kSliceBatch]] = r;
          }
        }
      }
    }
  } else {
    const int64_t m0 = (int64_t)blk * kAncPerBlock;
    const int64_t m1 = m0 + kAncPerBlock < M ? m0 + kAncPerBlock : M;
    constexpr int kAB = 4;                       // anchors per batch: loads, slot atomics and stores grouped
    for (int64_t mb = m0 + threadIdx.x; mb < m1; mb += kAB * blockDim.x) {
      int key[kAB], slot[kAB];
      bool ok[kAB];
      Rec r[kAB];
#pragma unroll
      for (int q = 0; q < kAB; ++q) {
        const int64_t m = mb + q * blockDim.x;
        ok[q] = m < m1 && anchor_rec(m, x, t, b, anchors, anchor_xy, N, G, key[q], r[q]);
      }
#pragma unroll
      for (int q = 0; q < kAB; ++q)
        if (ok[q]) {
          slot[q] = atomicAdd(hist + (key[q] >> G.bshift), 1);
          if (!SCATTER) vm = max(vm, float_to_ordered(fabsf(r[q].f.w)));
        }
      if (SCATTER) {
#pragma unroll
        for (int q = 0; q < kAB; ++q)
          if (ok[q]) trec[slot[q]] = r[q];
      }
    }
  }
  if (!SCATTER) {
    vm = wave_max_i(vm);
    if ((threadIdx.x & (kWave - 1)) == 0) red[threadIdx.x / kWave] = vm;
    __syncthreads();
    for (int i = threadIdx.x; i < G.nbuckets; i += blockDim.x) {   // bsum = tot
      const int c = hist[i];
      mycnt[i] = c;
      if (c > 0) atomicAdd(bsum + i, c);
    }
    if (threadIdx.x == 0) {
      for (int w = 1; w < kP1Block / kWave; ++w) vm = max(vm, red[w]);
      if (vm > 0) atomicMax(src_blk ? &P->vmax : &P->atmax, vm);
    }
    if (src_blk)
      for (int i = threadIdx.x; i < nplanes; i += blockDim.x)
        if (vpl[i] > 0) atomicMax(plane_vmax(P) + i, vpl[i]);
  }
}

// Pass 2: workgroup `bucket` sorts its records by cell.  start[key] (combined key space, 3 * ncell_pad + 1
// offsets) receives the CSR; entry records land at [0, E), anchor records at [0, Mv) and source records at
// [0, Nv) of their own arrays.  Every thread handles kSortItems records per round, all loads issued first.
constexpr int kSortItems = 8;

// Where pass 2 puts the sorted items.  Entries are split into their positions and velocities (16 B) and
// times (4 B), which is all the forward reads; the leave-one-out test there compares record positions, with
// eself[j] the position of event j's entry in its own anchor slice.
struct SortOut {
  int* start;
  float4* epos;                // entries: (y.x, y.y, v.x, v.y)
  float* etim;                 // entries: t
  int* eself;                  // per event: its entry in slice floor(t / delta), -1 if none
  Rec* arec;                   // anchors
  Rec* srec;                   // sources
  int* self;                   // per event: its anchor record, -1 if none
};

__device__ __forceinline__ int anchor_slice(float t, const FGeo& G) {
  return (int)fminf(fmaxf(floorf(t / G.delta), 0.f), (float)(G.S - 1));
}

// Key spaces [space0, space0 + gridDim.x / gps), gps = ceil(bpk / GROUP) workgroups per space: workgroup g of a
// space sorts its buckets [g * GROUP, (g + 1) * GROUP) together (one CSR over their keys): the anchor and source
// buckets hold a few hundred records each, and a workgroup per bucket would spend most of its time on the
// per-bucket scan and barriers.  bend: the end of every bucket (bpos after pass 1), tot: the bucket totals; a
// bucket starts at its end minus its total, so that the anchor and source buckets can be sorted before the
// entry buckets are filled.
template <int SHIFT, int GROUP>
__global__ void __launch_bounds__(kSortBlock) k_sort_pass2(const int* __restrict__ bend, const int* __restrict__ tot,
                                                           int space0, const Rec* __restrict__ trec, FGeo G,
                                                           SortOut o) {
  int* __restrict__ start = o.start;
  constexpr int kKeys = GROUP << SHIFT;            // keys of one workgroup
  __shared__ int cnt[kKeys];
  __shared__ int cur[kKeys];
  __shared__ int wsum[kSortBlock / kWave + 1];
  const int bpk = G.ncell_pad >> SHIFT;            // buckets per key space
  const int gps = (bpk + GROUP - 1) / GROUP;
  const int space = space0 + (int)blockIdx.x / gps;   // 0 entries, 1 anchors, 2 sources
  const int b0 = space * bpk + ((int)blockIdx.x % gps) * GROUP;
  const int b1 = min(b0 + GROUP, (space + 1) * bpk);
  const int hi = bend[b1 - 1];
  const int lo = bend[b0] - tot[b0];
  const int base_key = b0 << SHIFT;
  const int nkeys = (b1 - b0) << SHIFT;
  const int E = bend[bpk] - tot[bpk], EA = bend[2 * bpk] - tot[2 * bpk];
  const int4* tki = (const int4*)trec;             // int half of record p: tki[2 * p + 1]
  for (int i = threadIdx.x; i < kKeys; i += kSortBlock) {
    cnt[i] = 0;
    cur[i] = 0;
  }
  __syncthreads();
  // A group of at most kSortBlock * kSortItems records (the common case) is read once and kept in registers
  // from the count to the scatter, and the count's atomic returns each record's rank within its cell; larger
  // groups count from the keys, read the records again and rank them with a second atomic at the scatter.
  const bool one = hi - lo <= kSortBlock * kSortItems;
  Rec r1[kSortItems];
  int rank[kSortItems];                            // one-read path: the record's rank within its cell
  if (one) {
#pragma unroll
    for (int u = 0; u < kSortItems; ++u) {
      const int p = lo + u * kSortBlock + threadIdx.x;
      if (p < hi) r1[u] = trec[p];
    }
#pragma unroll
    for (int u = 0; u < kSortItems; ++u)
      if (lo + u * kSortBlock + (int)threadIdx.x < hi) rank[u] = atomicAdd(cnt + (r1[u].i.z - base_key), 1);
  } else {
    for (int base = lo; base < hi; base += kSortBlock * kSortItems) {
      int key[kSortItems];
#pragma unroll
      for (int u = 0; u < kSortItems; ++u) {
        const int p = base + u * kSortBlock + threadIdx.x;
        key[u] = p < hi ? tki[2 * p + 1].z : -1;
      }
#pragma unroll
      for (int u = 0; u < kSortItems; ++u)
        if (key[u] >= 0) atomicAdd(cnt + (key[u] - base_key), 1);
    }
  }
  __syncthreads();
  constexpr int per = kKeys / kSortBlock;
  int vals[per];
  int s = 0;
#pragma unroll
  for (int k = 0; k < per; ++k) {
    vals[k] = cnt[threadIdx.x * per + k];
    s += vals[k];
  }
  int total;
  int run = block_exclusive_scan<kSortBlock>(s, wsum, total);
#pragma unroll
  for (int k = 0; k < per; ++k) {
    const int i = threadIdx.x * per + k;
    cnt[i] = run;
    if (i < nkeys) start[base_key + i] = lo + run;
    run += vals[k];
  }
  if (b1 == G.nbuckets && threadIdx.x == 0) start[3 * G.ncell_pad] = hi;
  __syncthreads();
  const int off = space == 0 ? 0 : (space == 1 ? E : EA);
  Rec* out = space == 1 ? o.arec : o.srec;
  const int kbase = space * G.ncell_pad;
  const int plane_cells = G.GH * G.GW;
  auto place = [&](Rec r, int rk) {               // rk: the record's rank within its cell
    const int kk = r.i.z - base_key;
    const int pos = lo + cnt[kk] + rk - off;
    r.i.z -= kbase;
    if (space == 0) {
      o.epos[pos] = r.f;
      const float tj = __int_as_float(r.i.x);
      o.etim[pos] = tj;
      if ((r.i.z / plane_cells) % G.S == anchor_slice(tj, G)) o.eself[r.i.y] = pos;
    } else {
      out[pos] = r;
      if (space == 1) o.self[r.i.x] = pos;       // the anchor's event id -> its record
    }
  };
  if (one) {
#pragma unroll
    for (int u = 0; u < kSortItems; ++u)
      if (lo + u * kSortBlock + (int)threadIdx.x < hi) place(r1[u], rank[u]);
    return;
  }
  for (int base = lo; base < hi; base += kSortBlock * kSortItems) {
    Rec r[kSortItems];
    bool live[kSortItems];
#pragma unroll
    for (int u = 0; u < kSortItems; ++u) {
      const int p = base + u * kSortBlock + threadIdx.x;
      live[u] = p < hi;
      if (live[u]) r[u] = trec[p];
    }
#pragma unroll
    for (int u = 0; u < kSortItems; ++u)
      if (live[u]) place(r[u], atomicAdd(cur + (r[u].i.z - base_key), 1));
  }
}

// Entries of the linear model from the sorted source records.  A source lies near its own-slice position in
// every slice, so the source records (in own-slice tile order) are a spatially coherent order of the entries'
// sources: pass E1 (SCATTER = false) counts, per block of kEntSrcPerBlock source records, the entries that each
// entry bucket receives (cnt, block-major); pass E2 (SCATTER = true) reserves the block's run of every entry
// bucket it feeds and writes one 8-byte item per entry, (source record, cell key), instead of a 32-byte record:
// the slice-centre position is computed again from the source record by k_entry_write, in the same fp32
// operations, after k_entry_rank has put the items in cell order.
constexpr int kEntBlock = 512;                     // entry passes: workgroup
constexpr int kEntSrcPerBlock = 2048;              // entry passes: source records per block (4 per thread)
template <bool SCATTER>
__global__ void __launch_bounds__(kEntBlock) k_entry_pass(const Rec* __restrict__ srec, const int* __restrict__ start,
                                                       FGeo G, int* __restrict__ cnt, int* __restrict__ bpos,
                                                       int2* __restrict__ item) {
  extern __shared__ int hist[];
  const int nb0 = G.ncell_pad >> G.bshift;       // the entries' buckets
  const int EA = start[2 * G.ncell_pad];
  const int Nv = start[3 * G.ncell_pad] - EA;
  const int q0 = blockIdx.x * kEntSrcPerBlock;
  if (q0 >= Nv) return;                          // the same blocks return in both passes
  int* __restrict__ mycnt = cnt + (int64_t)blockIdx.x * nb0;
  for (int i = threadIdx.x; i < nb0; i += blockDim.x) {
    int h = 0;
    if (SCATTER) {
      const int c = mycnt[i];
      if (c > 0) h = atomicAdd(bpos + i, c);
    }
    hist[i] = h;
  }
  __syncthreads();
  const int scells = G.S * G.GH * G.GW;
  constexpr int per = kEntSrcPerBlock / kEntBlock;
  Rec r[per];
#pragma unroll
  for (int u = 0; u < per; ++u) r[u] = srec[min(q0 + u * kEntBlock + (int)threadIdx.x, Nv - 1)];   // all in flight
#pragma unroll
  for (int u = 0; u < per; ++u) {
    const int q = q0 + u * kEntBlock + threadIdx.x;
    if (q >= Nv) continue;
    const float tj = __int_as_float(r[u].i.x);
    const float2 xj = make_float2(r[u].f.x, r[u].f.y), vj = make_float2(r[u].f.z, r[u].f.w);
    const int bj = r[u].i.z / scells;
    int lo, hi;
    slice_range(tj, G, lo, hi);
    for (int s0 = lo; s0 <= hi; s0 += kSliceBatch) {
      int key[kSliceBatch], slot[kSliceBatch];
#pragma unroll
      for (int k = 0; k < kSliceBatch; ++k) {
        float yx, yy;
        key[k] = entry_key(xj, vj, tj, bj, min(s0 + k, hi), G, yx, yy);
      }
#pragma unroll
      for (int k = 0; k < kSliceBatch; ++k)
        if (s0 + k <= hi) slot[k] = atomicAdd(hist + (key[k] >> G.bshift), 1);
      if (SCATTER) {
#pragma unroll
        for (int k = 0; k < kSliceBatch; ++k)
          if (s0 + k <= hi) item[slot[k]] = make_int2(q, key[k]);
      }
    }
  }
  if (!SCATTER) {
    __syncthreads();
    for (int i = threadIdx.x; i < nb0; i += blockDim.x) mycnt[i] = hist[i];
  }
}

// Passes E1 and E2 in one launch, for sources of at most MAXE slices: each entry's key and its rank in the
// block's run of its bucket (a returning LDS atomic) stay in registers, the block then reserves its runs with one
// global atomic per bucket it feeds, and every entry is written at run start + rank.  No count matrix, and the
// source records and keys are read and formed once.
template <int MAXE>
__global__ void __launch_bounds__(kEntBlock) k_entry_scatter(const Rec* __restrict__ srec,
                                                          const int* __restrict__ start, FGeo G,
                                                          int* __restrict__ bpos, int2* __restrict__ item) {
  extern __shared__ int hist[];
  const int nb0 = G.ncell_pad >> G.bshift;
  const int EA = start[2 * G.ncell_pad];
  const int Nv = start[3 * G.ncell_pad] - EA;
  const int q0 = blockIdx.x * kEntSrcPerBlock;
  if (q0 >= Nv) return;
  for (int i = threadIdx.x; i < nb0; i += blockDim.x) hist[i] = 0;
  const int scells = G.S * G.GH * G.GW;
  constexpr int per = kEntSrcPerBlock / kEntBlock;
  Rec r[per];
#pragma unroll
  for (int u = 0; u < per; ++u) r[u] = srec[min(q0 + u * kEntBlock + (int)threadIdx.x, Nv - 1)];
  __syncthreads();                               // the histogram is cleared
  int key[per][MAXE], rank[per][MAXE];
#pragma unroll
  for (int u = 0; u < per; ++u) {
    const int q = q0 + u * kEntBlock + threadIdx.x;
    const float tj = __int_as_float(r[u].i.x);
    const float2 xj = make_float2(r[u].f.x, r[u].f.y), vj = make_float2(r[u].f.z, r[u].f.w);
    const int bj = r[u].i.z / scells;
    int lo, hi;
    slice_range(tj, G, lo, hi);
    if (q >= Nv) hi = lo - 1;                    // no entries
#pragma unroll
    for (int k = 0; k < MAXE; ++k) {
      key[u][k] = -1;
      rank[u][k] = 0;
      if (lo + k <= hi) {                        // never past G.MS slices: whole waves skip the tail
        float yx, yy;
        key[u][k] = entry_key(xj, vj, tj, bj, lo + k, G, yx, yy);
        rank[u][k] = atomicAdd(hist + (key[u][k] >> G.bshift), 1);
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nb0; i += blockDim.x) {
    const int c = hist[i];
    hist[i] = c > 0 ? atomicAdd(bpos + i, c) : 0;
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < per; ++u) {
    const int q = q0 + u * kEntBlock + threadIdx.x;
#pragma unroll
    for (int k = 0; k < MAXE; ++k)
      if (key[u][k] >= 0) item[hist[key[u][k] >> G.bshift] + rank[u][k]] = make_int2(q, key[u][k]);
  }
}

// Pass E3: workgroup `bucket` (an entry bucket) orders its items by cell, as k_sort_pass2 orders records, into
// `sorted` (items at their final positions) and writes the CSR of its keys.  bend: the bucket ends after pass E2,
// tot: the bucket totals.  Up to kSortBlock * kEntItems items are read once and ranked as they arrive; larger
// buckets count first and read their items again to place them.  Pass E4 (k_entry_write) then turns every
// sorted item into its entry.
constexpr int kEntItems = 16;
template <int SHIFT>
__global__ void __launch_bounds__(kSortBlock) k_entry_rank(const int* __restrict__ bend, const int* __restrict__ tot,
                                                           const int2* __restrict__ item, int2* __restrict__ sorted,
                                                           int* __restrict__ start, FGeo G) {
  constexpr int kBucketKeys = 1 << SHIFT;
  __shared__ int cnt[kBucketKeys];
  __shared__ int cur[kBucketKeys];
  __shared__ int wsum[kSortBlock / kWave + 1];
  const int bucket = blockIdx.x;
  const int hi = bend[bucket];
  const int lo = hi - tot[bucket];
  for (int i = threadIdx.x; i < kBucketKeys; i += kSortBlock) {
    cnt[i] = 0;
    cur[i] = 0;
  }
  __syncthreads();
  const bool one = hi - lo <= kSortBlock * kEntItems;
  int2 it[kEntItems];                              // (source record, key); key -1: no item
  int rank[kEntItems];
#pragma unroll
  for (int u = 0; u < kEntItems; ++u) {
    it[u] = make_int2(0, -1);
    rank[u] = 0;
  }
  if (one && hi > lo) {
    // unconditional loads (positions clamped into the bucket), so that all of them are in flight at once
#pragma unroll
    for (int u = 0; u < kEntItems; ++u) it[u] = item[min(lo + u * kSortBlock + (int)threadIdx.x, hi - 1)];
#pragma unroll
    for (int u = 0; u < kEntItems; ++u) {
      if (lo + u * kSortBlock + (int)threadIdx.x >= hi) it[u].y = -1;
      if (it[u].y >= 0) rank[u] = atomicAdd(cnt + (it[u].y & (kBucketKeys - 1)), 1);
    }
  } else if (!one) {
    for (int base = lo; base < hi; base += kSortBlock * kSortItems) {
      int key[kSortItems];
#pragma unroll
      for (int u = 0; u < kSortItems; ++u) key[u] = item[min(base + u * kSortBlock + (int)threadIdx.x, hi - 1)].y;
#pragma unroll
      for (int u = 0; u < kSortItems; ++u)
        if (base + u * kSortBlock + (int)threadIdx.x < hi) atomicAdd(cnt + (key[u] & (kBucketKeys - 1)), 1);
    }
  }
  __syncthreads();
  constexpr int per = kBucketKeys / kSortBlock;
  int vals[per];
  int sum = 0;
#pragma unroll
  for (int k = 0; k < per; ++k) {
    vals[k] = cnt[threadIdx.x * per + k];
    sum += vals[k];
  }
  int total;
  int run = block_exclusive_scan<kSortBlock>(sum, wsum, total);
  const int base_key = bucket << SHIFT;
#pragma unroll
  for (int k = 0; k < per; ++k) {
    const int i = threadIdx.x * per + k;
    cnt[i] = run;
    start[base_key + i] = lo + run;
    run += vals[k];
  }
  __syncthreads();
  if (one) {                                       // an empty bucket has no live item (key -1 throughout)
#pragma unroll
    for (int u = 0; u < kEntItems; ++u)
      if (it[u].y >= 0) sorted[lo + cnt[it[u].y & (kBucketKeys - 1)] + rank[u]] = it[u];
    return;
  }
  for (int base = lo; base < hi; base += kSortBlock * kSortItems) {
    int2 jt[kSortItems];
#pragma unroll
    for (int u = 0; u < kSortItems; ++u) jt[u] = item[min(base + u * kSortBlock + (int)threadIdx.x, hi - 1)];
#pragma unroll
    for (int u = 0; u < kSortItems; ++u)
      if (base + u * kSortBlock + (int)threadIdx.x < hi) {
        const int kk = jt[u].y & (kBucketKeys - 1);
        sorted[lo + cnt[kk] + atomicAdd(cur + kk, 1)] = jt[u];
      }
  }
}

// Pass E4: entry p from sorted item p = (source record q, key): slice s of the key's plane, position
// y = x + v (c_s - t) in entry_key's fp32 operations; eself names the entry of the event's anchor slice.
// Entries [0, E), E = start[ncell_pad] (the anchors' first position); kEntWrite per thread, the writes in entry
// order.
constexpr int kEntWrite = 8;
__global__ void __launch_bounds__(kBlock) k_entry_write(const int2* __restrict__ sorted, const Rec* __restrict__ srec,
                                                        FGeo G, SortOut o, int nblocks) {
  const int lb = xcd_block(nblocks);
  if (lb < 0) return;
  const int E = o.start[G.ncell_pad];
  const int p0 = lb * (kBlock * kEntWrite) + threadIdx.x;
  if (p0 >= E) return;
  const int Nv = o.start[3 * G.ncell_pad] - o.start[2 * G.ncell_pad];
  const int plane_cells = G.GH * G.GW;
  int2 it[kEntWrite];
  Rec r[kEntWrite];
#pragma unroll
  for (int u = 0; u < kEntWrite; ++u) it[u] = sorted[min(p0 + u * kBlock, E - 1)];
#pragma unroll
  for (int u = 0; u < kEntWrite; ++u) r[u] = srec[min(max(it[u].x, 0), Nv - 1)];   // q < Nv by construction
#pragma unroll
  for (int u = 0; u < kEntWrite; ++u) {
    const int pos = p0 + u * kBlock;
    if (pos >= E) break;
    const float tj = __int_as_float(r[u].i.x);
    const int sl = (it[u].y / plane_cells) % G.S;
    const float dt = slice_centre(sl, G.delta) - tj;
    o.epos[pos] = make_float4(r[u].f.x + r[u].f.z * dt, r[u].f.y + r[u].f.w * dt, r[u].f.z, r[u].f.w);
    o.etim[pos] = tj;
    if (sl == anchor_slice(tj, G)) o.eself[r[u].i.y] = pos;
  }
}

// ------------------------------------------------------------------------------------------ pair walks
struct FPlan {
  const float4* epos;          // entries in cell order: (y.x, y.y, v.x, v.y)
  const float* etim;           // entries in cell order: t
  const int* eself;            // per event: position of its own-slice entry, -1 if none
  const Rec* arec;             // anchors in cell order
  const Rec* srec;             // sources in own-slice cell order, tile by tile (source_key)
  float4* brec;                // anchors in cell order for the backward: (x, y, t, gS / h^2)
  int* self;                   // per event: position of its own anchor record, -1 if it is no anchor
  const int* start;            // 3*ncell_pad + 1: entry cells, anchor cells (offset by E), source cells
  FParams* P;
};

// One candidate pair, predicated: the reference's three tests (csrc/atl_cpu.cpp:187-197) in its fp32 order,
// written as "not rejected" so that NaN distances count as visits exactly as there.  The leave-one-out test
// compares id_a and id_s: the anchor event's own entry position and the candidate's position (one entry per
// source and slice, so this is the reference's id test).
__device__ __forceinline__ bool pair_test(int id_a, int id_s, float ta, float ts, float ax, float ay, float at,
                                          const float4& e, const FGeo& G, float& dt, float& rx, float& ry,
                                          float& d2) {
  dt = ta - ts;
  rx = ax - (e.x + e.z * at);
  ry = ay - (e.y + e.w * at);
  d2 = rx * rx + ry * ry;
  return (id_s != id_a) & !(fabsf(dt) > G.tau) & !(d2 > G.r2max);
}

// ------------------------------------------------------------------------------------------ walks
// Queries come in cell order, kAnchorsPerWave (forward) or 64 (backward) to a wave.  Forward: the anchors of up
// to G.gcells consecutive cells of one row (about kGroupWidth px) form a group; the group's anchors are
// wave-uniform and the lanes take 64 candidates of the group's common neighbourhood at a time (coalesced loads, each candidate read once
// for the whole group); every anchor's sum is reduced across the wave after its last chunk.  A walk with one lane per anchor reads a different cache line in every
// lane, and that is what bounds it.  Backward: one lane per source walks its own neighbourhoods (sources'
// per-slice positions differ, so a group shares less there than it costs to set up).

constexpr int kPairBlock = 64;                     // workgroup of the pair walks
constexpr int kBwdParts = 2;                       // backward lanes per source (each walks part of its slices)
static_assert(kBwdParts == 1 || kBwdParts == 2 || kBwdParts == 4, "a source's parts are combined by a butterfly");
constexpr int kGroup = 8;                          // queries evaluated per pass over a group's candidates
constexpr double kGroupWidth = 9.0;                // a forward group spans cells of one row over about this many px

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float unif(float v) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v))); }

// Cross-lane helpers on DPP (gfx9 row operations: quad_perm, row_mirror, row_shr, row_bcast) instead of
// LDS permutes.
template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ float dppf(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false));
}

// Sum over the 64 lanes, returned wave-uniform.
__device__ __forceinline__ float wave_sum_f(float v) {
  v += dppf<0xB1, 0xF>(v);                       // quad_perm [1, 0, 3, 2]
  v += dppf<0x4E, 0xF>(v);                       // quad_perm [2, 3, 0, 1]
  v += dppf<0x141, 0xF>(v);                      // row_half_mirror
  v += dppf<0x140, 0xF>(v);                      // row_mirror: every lane holds its row's sum
  v += dppf<0x142, 0xA>(v);                      // row_bcast:15 into rows 1, 3
  v += dppf<0x143, 0xC>(v);                      // row_bcast:31 into rows 2, 3: lane 63 holds the total
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ int wave_sum_i(int v) {
  v += dpp<0xB1, 0xF>(v);
  v += dpp<0x4E, 0xF>(v);
  v += dpp<0x141, 0xF>(v);
  v += dpp<0x140, 0xF>(v);
  v += dpp<0x142, 0xA>(v);
  v += dpp<0x143, 0xC>(v);
  return __builtin_amdgcn_readlane(v, 63);
}

// Sums over the 64 lanes of WD values at once, returned wave-uniform.  gfx950's lane swaps fold pairs of values
// together: permlane32_swap(a, b) + its partner gives a's 32-lane partial sums in lanes 0-31 and b's in 32-63;
// permlane16_swap then folds two such vectors into four 16-lane rows (a, c, b, d for the pairs (a, b), (c, d)),
// and four DPP steps sum each row.  Eight values cost 20 VALU operations instead of 8 tree reductions of 6.
__device__ __forceinline__ float fold32(float a, float b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(a), __float_as_int(b), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}
__device__ __forceinline__ float fold16(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(a), __float_as_int(b), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}
__device__ __forceinline__ float row_sum16(float v) {
  v += dppf<0xB1, 0xF>(v);                       // quad_perm [1, 0, 3, 2]
  v += dppf<0x4E, 0xF>(v);                       // quad_perm [2, 3, 0, 1]
  v += dppf<0x141, 0xF>(v);                      // row_half_mirror
  v += dppf<0x140, 0xF>(v);                      // row_mirror: every lane holds its row's sum
  return v;
}
template <int WD>
__device__ __forceinline__ void multi_sum_f(const float (&v)[WD], float (&out)[WD]) {
  if (WD == 1) {
    out[0] = wave_sum_f(v[0]);
    return;
  }
  constexpr int kQ = (WD + 3) / 4;               // vectors of four values after the two folds
#pragma unroll
  for (int q = 0; q < kQ; ++q) {
    auto at = [&](int k) { return 4 * q + k < WD ? v[4 * q + k] : 0.f; };
    const float w0 = fold32(at(0), at(1));
    const float w1 = 4 * q + 2 < WD ? fold32(at(2), at(3)) : 0.f;
    const float x = row_sum16(fold16(w0, w1));   // rows: values 4q, 4q + 2, 4q + 1, 4q + 3
    constexpr int kLane[4] = {0, 32, 16, 48};
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (4 * q + k < WD) out[4 * q + k] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), kLane[k]));
  }
}

// Inclusive prefix sum over the 64 lanes.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += dpp<0x111, 0xF>(v);                       // row_shr:1
  v += dpp<0x112, 0xF>(v);                       // row_shr:2
  v += dpp<0x114, 0xF>(v);                       // row_shr:4
  v += dpp<0x118, 0xF>(v);                       // row_shr:8: scans within rows of 16
  v += dpp<0x142, 0xA>(v);                       // row_bcast:15
  v += dpp<0x143, 0xC>(v);                       // row_bcast:31
  return v;
}

__device__ __forceinline__ int rdlane(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float rdlanef(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Per-lane walk of the R-neighbourhood of (qx, qy) in plane `plane`: visit(k, e, Step<U>) for U consecutive
// candidates [k, k + U) of a row ending at e (positions past e are padded records, masked by the caller; U is at
// most kUnroll).  cstart offsets minus `base`.
template <int U>
using Step = std::integral_constant<int, U>;

template <typename Visit>
__device__ __forceinline__ void walk(const int* __restrict__ cstart, int base, int plane, float qx, float qy, float R,
                                     float R2, const FGeo& G, Visit&& visit) {
  const int rlo = cell_walk(qy - R, G.gy0, G.gy1, G.icf, G.GH), rhi = cell_walk(qy + R, G.gy0, G.gy1, G.icf, G.GH);
  for (int r = rlo; r <= rhi; ++r) {
    int c0, c1;
    if (!row_span(r, qx, qy, R, R2, G, c0, c1)) continue;
    const int rowk = plane + r * G.GW;
    const int e = cstart[rowk + c1 + 1] - base;
    for (int k = cstart[rowk + c0] - base; k < e; k += kStep) visit(k, e, Step<kStep>{});
  }
}

// The same walk with the rows of the neighbourhood flattened: the spans of up to kRowTab rows are fetched at
// once into this lane's column of an LDS table (tab[r * kBlock]), then the lane steps through them without
// waiting for the other lanes at row ends (a wave's lanes have rows of different lengths; stepping row by row
// in lockstep leaves most lanes idle).  Taller neighbourhoods take the row-by-row walk.
constexpr int kRowTab = 8;

// ADAPT: a wave in which some lane's neighbourhood holds more than kLongWalk candidates takes steps of kStepLong
// (more loads in flight per lane on long walks; short walks keep kStep, which leaves fewer lanes masked).
template <bool ADAPT = false, typename Visit>
__device__ __forceinline__ void walk_flat(const int* __restrict__ cstart, int base, int plane, float qx, float qy,
                                          float R, float R2, const FGeo& G, int2* tab, Visit&& visit) {
  const int rlo = cell_walk(qy - R, G.gy0, G.gy1, G.icf, G.GH), rhi = cell_walk(qy + R, G.gy0, G.gy1, G.icf, G.GH);
  const int nrows = rhi - rlo + 1;
  if (nrows > kRowTab) {
    walk(cstart, base, plane, qx, qy, R, R2, G, visit);
    return;
  }
  int kk[kRowTab], ee[kRowTab];
#pragma unroll
  for (int i = 0; i < kRowTab; ++i) {              // all span loads in flight together
    kk[i] = base;
    ee[i] = base;
    int c0, c1;
    if (i < nrows && row_span(rlo + i, qx, qy, R, R2, G, c0, c1)) {
      const int rowk = plane + (rlo + i) * G.GW;
      kk[i] = cstart[rowk + c0];
      ee[i] = cstart[rowk + c1 + 1];
    }
  }
#pragma unroll
  for (int i = 0; i < kRowTab; ++i) tab[i * kPairBlock] = make_int2(kk[i] - base, ee[i] - base);
  auto steps = [&](auto step) {
    constexpr int U = decltype(step)::value;
    int ri = 0;                                    // row of cur; nxt holds row ri + 1 (read one row ahead)
    int2 cur = make_int2(kk[0] - base, ee[0] - base);
    int2 nxt = make_int2(kk[1] - base, ee[1] - base);
    while (true) {
      if (cur.x >= cur.y) {
        do {
          cur = nxt;
          ++ri;
          nxt = ri + 1 < nrows ? tab[(ri + 1) * kPairBlock] : make_int2(0, 0);
        } while (cur.x >= cur.y && ri < nrows - 1);
        if (cur.x >= cur.y) break;
      }
      visit(cur.x, cur.y, step);
      cur.x += U;
    }
  };
  bool lng = false;
  if (ADAPT) {
    int tot = 0;
#pragma unroll
    for (int i = 0; i < kRowTab; ++i) tot += ee[i] - kk[i];
    lng = __any(tot > kLongWalk);                  // uniform over the wave's walking lanes
  }
  if (lng)
    steps(Step<kStepLong>{});
  else
    steps(Step<kStep>{});
}

// Group walk: the candidates of the cells of plane `plane` that meet the R-neighbourhood of the box
// [x0, x1] x [y0, y1], 64 per chunk: use(load(pos), pos) with pos the lane's candidate index (-1 if idle).  Row
// spans are fetched one row per lane and prefix-summed across the wave.  All arguments wave-uniform.
// Up to kRowTable rows (the usual case: R / cf < 3) the row starts and offsets are read into scalars once
// and every chunk maps its lanes with one compare and select per row; taller neighbourhoods take the
// general loop.
constexpr int kRowTable = 8;

// Candidate position of chunk index idx: idx plus the offset of the last row starting at or before idx
// (e_k: row starts in the chunk numbering, o_k: row offsets); -1 past the last candidate.  All operands are
// passed by value, so the select chain stays in registers.
__device__ __forceinline__ int row_map(int idx, int total, int e1, int e2, int e3, int e4, int e5, int e6, int e7,
                                       int o0, int o1, int o2, int o3, int o4, int o5, int o6, int o7) {
  int off = o0;
  off = idx >= e1 ? o1 : off;
  off = idx >= e2 ? o2 : off;
  off = idx >= e3 ? o3 : off;
  off = idx >= e4 ? o4 : off;
  off = idx >= e5 ? o5 : off;
  off = idx >= e6 ? o6 : off;
  off = idx >= e7 ? o7 : off;
  return idx < total ? idx + off : -1;
}

template <typename Load, typename Use>
__device__ __forceinline__ void group_walk(const int* __restrict__ cstart, int base, int plane, float x0, float x1,
                                           float y0, float y1, float R, float R2, const FGeo& G, Load&& load,
                                           Use&& use) {
  const int lane = threadIdx.x & (kWave - 1);
  const int rlo = uni(cell_walk(y0 - R, G.gy0, G.gy1, G.icf, G.GH));
  const int rhi = uni(cell_walk(y1 + R, G.gy0, G.gy1, G.icf, G.GH));
  for (int rb = rlo; rb <= rhi; rb += kWave) {
    const int r = rb + lane;
    int s0 = 0, len = 0;
    if (r <= rhi) {
      const float row_lo = G.gy0 + (float)r * G.cf, row_hi = row_lo + G.cf;
      const float gap = fmaxf(0.f, fmaxf(row_lo - y1, y0 - row_hi));
      if (gap <= R) {
        const float w = __builtin_amdgcn_sqrtf(fmaxf(R2 - gap * gap, 0.f));   // ~1 ulp: far inside the slack
        const int c0 = cell_walk(x0 - w, G.gx0, G.gx1, G.icf, G.GW);
        const int c1 = cell_walk(x1 + w, G.gx0, G.gx1, G.icf, G.GW);
        const int rowk = plane + r * G.GW;
        s0 = cstart[rowk + c0] - base;
        len = cstart[rowk + c1 + 1] - base - s0;
      }
    }
    const int nrb = min(kWave, rhi - rb + 1);   // rows of this batch
    const int incl = wave_incl_scan(len);
    const int excl = incl - len;
    const int total = rdlane(incl, kWave - 1);
    if (nrb <= kRowTable) {
      // lanes >= nrb hold len 0 and excl = total, so their entries never match a valid index.  Row starts
      // are scalars; row offsets are copied once into vector registers, so that each row of the select chain
      // is one compare and one VCC select.  They are separate variables, not an array: a select chain over
      // an array is folded into an indexed load from a table in private memory.
      static_assert(kRowTable == 8, "the row table below has eight rows");
#define ATL_ROW(k) const int e##k = rdlane(excl, k); int o##k; \
      asm("v_mov_b32 %0, %1" : "=v"(o##k) : "s"(rdlane(s0 - excl, k)));
      ATL_ROW(0) ATL_ROW(1) ATL_ROW(2) ATL_ROW(3) ATL_ROW(4) ATL_ROW(5) ATL_ROW(6) ATL_ROW(7)
#undef ATL_ROW
      (void)e0;
      auto map = [=](int c0) {
        return row_map(c0 + lane, total, e1, e2, e3, e4, e5, e6, e7, o0, o1, o2, o3, o4, o5, o6, o7);
      };
      int pos = map(0);
      auto cur = load(pos);
      for (int c0 = 0; c0 < total; c0 += kWave) {  // the next chunk's candidates load while this one computes
        const int pn = map(c0 + kWave);
        auto nxt = load(pn);
        use(cur, pos);
        cur = nxt;
        pos = pn;
      }
      continue;
    }
    int j = 0;                                  // first row that the current chunk may touch
    for (int c0 = 0; c0 < total; c0 += kWave) {
      const int idx = c0 + lane;
      int pos = -1;
      while (j < nrb) {
        const int ej = rdlane(excl, j);
        if (ej >= c0 + kWave) break;
        const int lj = rdlane(len, j);
        const int sj = rdlane(s0, j);
        if (idx >= ej && idx < ej + lj) pos = sj + (idx - ej);
        if (ej + lj > c0 + kWave) break;        // row continues into the next chunk
        ++j;
      }
      use(load(pos), pos);
    }
  }
}

// One pass of a group walk for WD wave-uniform anchors read from lanes src0 .. src0 + na - 1 (slots past na
// repeat the last anchor and are discarded): lane src0 + a receives anchor a's sum (and count) in mine
// (mine_n).  es is each anchor lane's own entry position: the leave-one-out test skips that candidate.
template <int WD, bool COUNT>
__device__ __forceinline__ void fwd_pass(const FPlan& p, const FGeo& G, int plane, float R, float R2, float vmax,
                                         const float4& A, int es, int src0, int na, int lane, float& mine,
                                         int& mine_n) {
  float ax[WD], ay[WD], ta[WD], at[WD], acc[WD];
  int id[WD], cnt[WD];
#pragma unroll
  for (int a = 0; a < WD; ++a) {
    const int src = src0 + min(a, na - 1);
    ax[a] = rdlanef(A.x, src);
    ay[a] = rdlanef(A.y, src);
    ta[a] = rdlanef(A.z, src);
    at[a] = rdlanef(A.w, src);
    id[a] = rdlane(es, src);
    acc[a] = 0.f;
    cnt[a] = 0;
  }
  {                                                // these anchors' own radius: vmax * max |at| over the pass
    float atg = 0.f;
#pragma unroll
    for (int a = 0; a < WD; ++a) atg = fmaxf(atg, fabsf(at[a]));
    const float rg = G.cuth * 1.000001f + vmax * atg * 1.000001f + 0.01f;
    if (rg < R) {                                  // false for NaN / inf: keep the whole-slice walk
      R = rg;
      R2 = rg * rg;
    }
  }
  struct Cand {
    float4 e;
    float t;
  };
  auto load = [&](int pos) {
    const uint32_t k = (uint32_t)max(pos, 0);
    return Cand{ld(p.epos, k), ld(p.etim, k)};
  };
  // The walk covers the R-neighbourhood of the box of these anchors' clamped positions (tighter than their
  // cells' box: every contributing candidate lies within R of its anchor, and clamping never increases a
  // distance).  Slots past na repeat the last anchor, so they do not widen it.
  float bx0 = clampf(ax[0], G.gx0, G.gx1), bx1 = bx0, by0 = clampf(ay[0], G.gy0, G.gy1), by1 = by0;
#pragma unroll
  for (int a = 1; a < WD; ++a) {
    const float cx = clampf(ax[a], G.gx0, G.gx1), cy = clampf(ay[a], G.gy0, G.gy1);
    bx0 = fminf(bx0, cx);
    bx1 = fmaxf(bx1, cx);
    by0 = fminf(by0, cy);
    by1 = fmaxf(by1, cy);
  }
  group_walk(p.start, 0, plane, bx0, bx1, by0, by1, R, R2, G, load, [&](const Cand& c, int pos) {
    const float4 e = c.e;
    const float ts = c.t;
#pragma unroll
    for (int a = 0; a < WD; ++a) {
      float dt, rx, ry, d2;
      const bool ok = pair_test(id[a], pos, ta[a], ts, ax[a], ay[a], at[a], e, G, dt, rx, ry, d2) & (pos >= 0);
      const float kern = __builtin_amdgcn_exp2f(d2 * G.kexp);
      acc[a] += ok ? kern : 0.f;
      if (COUNT) cnt[a] += ok ? 1 : 0;
    }
  });
  float sum[WD];
  multi_sum_f<WD>(acc, sum);
#pragma unroll
  for (int a = 0; a < WD; ++a) {
    if (a < na) {
      if (lane == src0 + a) mine = sum[a];
      if (COUNT) {
        const int ca = wave_sum_i(cnt[a]);
        if (lane == src0 + a) mine_n = ca;
      }
    }
  }
}

// Forward: out[m] = S_m and, with COUNT, count[m] = n_m (number of pairs passing the tests).  Every lane
// sums one candidate per chunk, the 64 lane partials are added in a tree (the reference's CPU path sums
// sequentially in fp64; both stay well inside 1e-5 of the exact sum).
// A wave takes kAnchorsPerWave consecutive anchors (lanes past them hold copies and idle through the group loop;
// every lane takes candidates in the walks).  The wave's time follows the density around its anchors, and
// smaller units let the hardware's wave queue even out dense and sparse regions: 16 anchors per wave run the
// C3 forward in 365 us against 410 us with 64 (32: 379 us; 8 or 12: as 16; 4: 390 us).
constexpr int kAnchorsPerWave = 16;
constexpr int kAnchorsPerBlock = kPairBlock / kWave * kAnchorsPerWave;

// Register budgets (amdgpu_waves_per_eu: the compiler keeps the kernel within the registers of that many waves
// per SIMD): the forward fits 8 waves without spills (53 VGPRs, 69 unconstrained), the backward 6 (80 VGPRs, three
// spills outside its walk loop; 88 unconstrained), the trajectory backward 4 at K = 10 (128 VGPRs, 135
// unconstrained).  Same code, more waves to hide the candidate loads: C3 forward 0.329 -> 0.322 ms, backward
// 0.446 -> 0.435 ms, C4 trajectory backward 1.89 -> 1.67 ms (alternating runs on one box).  Tighter budgets spill
// inside the walks (backward at 7 waves: 13 spills; trajectory backward at 5: 42).
template <bool COUNT>
__global__ void __launch_bounds__(kPairBlock) __attribute__((amdgpu_waves_per_eu(8))) k_fast_fwd(FPlan p, FGeo G, int M, float* __restrict__ out,
                                                     int* __restrict__ count) {
  const int lb = xcd_block((M + kAnchorsPerBlock - 1) / kAnchorsPerBlock);
  if (lb < 0) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int wbase = (lb * (kPairBlock / kWave) + (int)(threadIdx.x / kWave)) * kAnchorsPerWave;
  const int E = uni(p.start[G.ncell_pad]);
  const int Mv = uni(p.start[2 * G.ncell_pad]) - E;
  if (wbase >= Mv) return;
  const int n = min(kAnchorsPerWave, Mv - wbase);
  float R, R2;
  search_radius(p.P, G, R, R2);
  R = unif(R);
  R2 = unif(R2);
  const float vmax = unif(ordered_to_float(p.P->vmax));
  const int* vpl = plane_vmax(p.P);
  const bool planes = G.vplanes && uni(p.P->planes) != 0;
  const bool have = lane < n;
  const int q = wbase + min(lane, n - 1);
  const Rec AR = p.arec[q];
  const float4 A = AR.f;
  const int4 ai = AR.i;
  const int key = ai.z;
  const int es = p.eself[ai.x];                  // the anchor event's own entry in this slice, -1 if none
  const int plane_cells = G.GH * G.GW;
  float mine = 0.f;
  int mine_n = 0;
  uint64_t todo = __ballot(have);
  while (todo) {
    const int i = __ffsll((unsigned long long)todo) - 1;
    const int gkey = rdlane(key, i);
    const int cyx = rdlane(ai.w, i);               // the group's cell, packed by the plan (no divisions)
    const int cy = cyx >> 16, cx = cyx & 0xffff;
    const int plane = gkey - (cy * G.GW + cx);
    // the plane's own velocity bound (its entries only are candidates); NaN keeps the global one
    const float vg = planes ? fminf(vmax, ordered_to_float(vpl[plane / plane_cells])) : vmax;
    // the group: anchors of up to G.gcells consecutive cells of one row (lanes i .. i + gsize - 1)
    const int span = min(G.gcells, G.GW - cx);
    const uint64_t gmask = __ballot(have && key >= gkey && key - gkey < span) & todo;
    todo &= ~gmask;
    const int gsize = __popcll(gmask);
    for (int a0 = 0; a0 < gsize; a0 += kGroup) {
      const int na = min(kGroup, gsize - a0);
      if (na == 1)
        fwd_pass<1, COUNT>(p, G, plane, R, R2, vg, A, es, i + a0, na, lane, mine, mine_n);
      else if (na == 2)
        fwd_pass<2, COUNT>(p, G, plane, R, R2, vg, A, es, i + a0, na, lane, mine, mine_n);
      else if (na == 3)
        fwd_pass<3, COUNT>(p, G, plane, R, R2, vg, A, es, i + a0, na, lane, mine, mine_n);
      else if (na == 4)
        fwd_pass<4, COUNT>(p, G, plane, R, R2, vg, A, es, i + a0, na, lane, mine, mine_n);
      else if (na <= 6)
        fwd_pass<6, COUNT>(p, G, plane, R, R2, vg, A, es, i + a0, na, lane, mine, mine_n);
      else
        fwd_pass<kGroup, COUNT>(p, G, plane, R, R2, vg, A, es, i + a0, na, lane, mine, mine_n);
    }
  }
  if (have) {
    out[ai.y] = mine;
    if (COUNT) count[ai.y] = mine_n;
  }
}

// Finite and small enough that products of two such values stay finite.
__device__ __forceinline__ bool bounded(float v) { return fabsf(v) < 1e30f; }

// Record range of slice s of (batch b, tile (tb, tx)) in the source records.
__device__ __forceinline__ int2 src_tile_range(const FPlan& p, const FGeo& G, int b, int s, int tb, int tx, int EA) {
  const int T = G.stile;
  const int hb = min(T, G.GH - tb * T), wt = min(T, G.GW - tx * T);
  const int k0 = (b * G.S + s) * (G.GH * G.GW) + tb * T * G.GW + tx * T * hb;
  const int* sstart = p.start + 2 * G.ncell_pad;
  return make_int2(sstart[k0] - EA, sstart[k0 + hb * wt] - EA);
}

// Backward records of the anchors in cell order, brec[q] = (x, y, t, gS / h^2): one 16-byte load per candidate in
// the backward's per-lane walks (the anchor's at = t - c_s is recomputed there with the same fp32 operation).
// Also checks that no event occurs twice among the anchors (self[id] then names only one of the records); an
// index-free plan (every event once) skips that check.  Threads q < N clear gv[q] for the backward, which then
// writes each source's total (sources without a record keep the zero).
__global__ void __launch_bounds__(kBlock) k_fast_gather_gs(FPlan p, FGeo G, int M, const float* __restrict__ gS,
                                                           int N, float2* __restrict__ gv) {
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (gv && q < N) gv[q] = make_float2(0.f, 0.f);
  const int Mv = p.start[2 * G.ncell_pad] - p.start[G.ncell_pad];
  // the walks' padding past the last record (Mv <= M: inside the M + kUnroll records): zeros
  if (q < kUnroll) p.brec[Mv + q] = make_float4(0.f, 0.f, 0.f, 0.f);
  if (q >= Mv || q >= M) return;
  const Rec r = p.arec[q];
  const float4 br = make_float4(r.f.x, r.f.y, r.f.z, gS[r.i.y] * G.invh2);
  p.brec[q] = br;
  if (!p.P->unique && p.self[r.i.x] != q) p.P->dup = 1;
  if (!(bounded(br.x) && bounded(br.y) && bounded(br.z) && bounded(br.w))) p.P->nonfinite = 1;
}

// One source's walk over the anchors of every slice of its range (csrc/atl_cpu.cpp:240-248): returns
// sum_i gS_i * k * dt / h^2 * r.  Leave-one-out (LOO): the pair of an event with its own anchor record has
// dt = t_j - t_j = 0, so with finite records and source data its term is exactly zero and the test is skipped
// (kLooNone); otherwise (kLooPos) the candidate's record position is compared with the position of the source's
// own anchor record (sp), and with an event repeated among the anchors (kLooId) the event ids are compared, as
// the reference does.
enum { kLooNone = 0, kLooPos = 1, kLooId = 2 };
template <int LOO>
__device__ __forceinline__ float2 bwd_source(const FPlan& p, const FGeo& G, float R, float R2, float4 sr, int sid,
                                             float tj, int key, int sp, int part, int2* tab) {
  const int plane_cells = G.GH * G.GW;
  const int* astart = p.start + G.ncell_pad;
  const int E = uni(p.start[G.ncell_pad]);
  const int* aid = (const int*)p.arec + 4;         // event id of record k: aid[8 * k]
  int lo_l, hi_l;
  slice_range(tj, G, lo_l, hi_l);
  if (kBwdParts > 1) {                             // part p of kBwdParts: its share of the slices, in order
    const int L = max(hi_l - lo_l + 1, 0);
    const int a = lo_l + (part * L) / kBwdParts, b = lo_l + ((part + 1) * L) / kBwdParts - 1;
    lo_l = a;
    hi_l = b;
  }
  const int bj = key / (G.S * plane_cells);
  float mgx = 0.f, mgy = 0.f;
  float4 sv;                                       // the current slice's entry (y, v) and centre
  float cs;
  auto visit = [&](int k, int e, auto step) {
    constexpr int U = decltype(step)::value;
    float4 A[U];
    int id[U];
    // one lane offset for the U loads, the step within the record run folded into the (scalar) base
#pragma unroll
    for (int u = 0; u < U; ++u) {
      A[u] = ld((const float4*)p.brec + u, (uint32_t)k);
      if (LOO == kLooId) id[u] = ld(aid + 8 * u, 8u * (uint32_t)k);
    }
    const int rem = e - k, self_u = sp - k;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float at = A[u].z - cs;
      const float dt = A[u].z - tj;
      const float rx = A[u].x - (sv.x + sv.z * at);
      const float ry = A[u].y - (sv.y + sv.w * at);
      const float d2 = rx * rx + ry * ry;
      const bool other = LOO == kLooId ? id[u] != sid : LOO == kLooPos ? u != self_u : true;
      const bool ok = other & !(fabsf(dt) > G.tau) & !(d2 > G.r2max) & (u < rem);
      const float kern = __builtin_amdgcn_exp2f(d2 * G.kexp);
      const float f = A[u].w * kern * dt;           // A.w = gS / h^2
      if (LOO == kLooNone) {                         // every record and the source are finite and below
        float fo = ok ? f : 0.f;                     // 1e30 (checked), so a zero factor adds exactly nothing
        asm volatile("" : "+v"(fo));                 // keep one select (not folded into two after the FMAs)
        mgx = fmaf(fo, rx, mgx);
        mgy = fmaf(fo, ry, mgy);
      } else {                                       // selects: a record may hold anything, NaN included
        mgx = ok ? fmaf(f, rx, mgx) : mgx;
        mgy = ok ? fmaf(f, ry, mgy) : mgy;
      }
    }
  };
  auto entry = [&](int s, float4& e4, float& c) {
    entry_key(make_float2(sr.x, sr.y), make_float2(sr.z, sr.w), tj, bj, s, G, e4.x, e4.y);
    e4.z = sr.z;
    e4.w = sr.w;
    c = slice_centre(s, G.delta);
  };
  for (int s = lo_l; s <= hi_l; ++s) {
    entry(s, sv, cs);
    const float qx = clampf(sv.x, G.gx0, G.gx1), qy = clampf(sv.y, G.gy0, G.gy1);
    walk_flat<true>(astart, E, (bj * G.S + s) * plane_cells, qx, qy, R, R2, G, tab, visit);
  }
  return make_float2(mgx, mgy);
}

// Backward: every source (one lane each, own-slice tile order) sums, over the anchors of each slice of its
// range within R of its slice-centre position, gS_i * k * dt / h^2 * r (csrc/atl_cpu.cpp:240-248);
// gv[j] = the total (each source has one record: no atomics).
__global__ void __launch_bounds__(kPairBlock) __attribute__((amdgpu_waves_per_eu(6))) k_fast_bwd(FPlan p, FGeo G, int N, float2* __restrict__ gv,
                                                      float2* __restrict__ gvr) {
  __shared__ int2 tab[kRowTab * kPairBlock];           // per-lane row spans of the current slice (column threadIdx.x)
  constexpr int kSrcPerWave = kWave / kBwdParts;
  const int lb = xcd_block((N + kPairBlock / kBwdParts - 1) / (kPairBlock / kBwdParts));
  if (lb < 0) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int part = lane / kSrcPerWave, ls = lane - part * kSrcPerWave;
  const int wbase = (lb * (kPairBlock / kWave) + (int)(threadIdx.x / kWave)) * kSrcPerWave;
  const int EA = uni(p.start[2 * G.ncell_pad]);
  const int Nv = uni(p.start[3 * G.ncell_pad]) - EA;
  if (wbase >= Nv) return;
  const int n = min(kSrcPerWave, Nv - wbase);
  float R, R2;
  search_radius(p.P, G, R, R2);
  R = unif(R);
  R2 = unif(R2);
  const bool have = ls < n;
  const Rec SR = p.srec[wbase + min(ls, n - 1)];
  const int4 si = SR.i;
  const float tj = __int_as_float(si.x);
  // this source's own search radius: its entries all move with its own velocity, |v_j| * max|at| <= vmax * max|at|
  {
    const float vj = sqrtf(SR.f.z * SR.f.z + SR.f.w * SR.f.w);
    const float rj = G.cuth * 1.000001f + vj * ordered_to_float(p.P->atmax) * 1.000001f + 0.01f;
    if (rj < R) {                                  // false for NaN / inf velocities: keep the whole-slice walk
      R = rj;
      R2 = rj * rj;
    }
  }
  const int sp = p.self[si.y];
  int2* mytab = tab + threadIdx.x;
  float2 m = make_float2(0.f, 0.f);
  // the leave-one-out test can be skipped when every term of a source with its own anchor is exactly zero
  const bool src_finite = bounded(SR.f.x) && bounded(SR.f.y) && bounded(SR.f.z) && bounded(SR.f.w) && bounded(tj);
  const int loo = uni(p.P->dup) ? kLooId : (uni(p.P->nonfinite) || __ballot(have && !src_finite)) ? kLooPos
                                                                                                    : kLooNone;
  if (have) {
    if (loo == kLooId)
      m = bwd_source<kLooId>(p, G, R, R2, SR.f, si.y, tj, si.z, sp, part, mytab);
    else if (loo == kLooPos)
      m = bwd_source<kLooPos>(p, G, R, R2, SR.f, si.y, tj, si.z, sp, part, mytab);
    else
      m = bwd_source<kLooNone>(p, G, R, R2, SR.f, si.y, tj, si.z, sp, part, mytab);
  }
#pragma unroll
  for (int o = kSrcPerWave; o < kWave; o <<= 1) {  // the parts of a source sit kSrcPerWave lanes apart
    m.x += __shfl_xor(m.x, o);
    m.y += __shfl_xor(m.y, o);
  }
  if (have && part == 0) {                         // by event (gv), or by source record (gvr, coalesced)
    if (gv) gv[si.y] = m;
    if (gvr) gvr[wbase + ls] = m;
  }
}

// Flow-grid adjoint of the velocities v_j = sample(grid, x_j) (atl/motion/parametric.py:235-251 under autograd)
// over the source records.  The sources are sorted by own-slice cell in 8 x 8-cell tiles, and a source lies within
// |v| delta / 2 of its own-slice position, so the records of one tile (of all S slices) sit in a compact patch of
// the grid and need no binning.  k_src_adj_list cuts every (batch, tile)'s records into chunks of at most 1024;
// k_src_flow_adjoint gives each chunk one workgroup, which accumulates it in the tile engine's gather form: the
// records are ranked by base node with one LDS integer atomic each, thread c adds value * (wx * wy) of its node's
// records for the four corners and two channels (the scatter's fp32 products), and every window node adds the
// sums of the base nodes that reach it and is flushed with one global atomic.  The 16 x 16 window of base nodes
// starts at the chunk's smallest base node; a record outside it (a position clamped from far outside the box)
// adds its four corners with global atomics.
struct FlowGeo {
  int Hg, Wg;
  float sxw, syh;              // pixel -> grid scaling of DenseLinearFlow.field (scale on), parametric.py:214-215
  int scale;
};

constexpr int kAdjBlock = 256;
constexpr int kAdjT = 16;                        // window of base nodes
constexpr int kAdjItems = 2;
constexpr int kAdjChunk = kAdjBlock * kAdjItems; // records per chunk (one workgroup)
constexpr int kAdjListBlock = 1024;
constexpr int kAdjMaxSlices = 64;

// Source records of every (batch, tile) over its S slices: one thread per (tile, slice), the slices of a tile in
// SP consecutive lanes (SP: S rounded up to a power of two, at most 64), summed across them.  The same threads
// clear the flow-grid gradient (ng floats), which k_src_flow_adjoint then accumulates.
__global__ void __launch_bounds__(kBlock) k_src_tile_counts(FPlan p, FGeo G, int ntiles, int SP,
                                                            int* __restrict__ tilecnt, float* __restrict__ ggrid,
                                                            int64_t ng) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t g = i; g < ng; g += (int64_t)gridDim.x * blockDim.x) ggrid[g] = 0.f;
  const int q = i / SP, s = i - q * SP;
  int n = 0;
  if (q < ntiles && s < G.S) {
    const int TXb = (G.GW + G.stile - 1) / G.stile, TYb = (G.GH + G.stile - 1) / G.stile;
    const int b = q / (TXb * TYb), tr = q - b * TXb * TYb;
    const int tb = tr / TXb, tx = tr - tb * TXb;
    const int2 r = src_tile_range(p, G, b, s, tb, tx, p.start[2 * G.ncell_pad]);
    n = r.y - r.x;
  }
  for (int d = SP >> 1; d >= 1; d >>= 1) n += __shfl_xor(n, d, kWave);
  if (s == 0 && q < ntiles) tilecnt[q] = n;
}

// Chunk list: info[w] = (batch-tile index, first record of the tile's concatenated slice ranges) from the tiles'
// record counts; one workgroup, thread i takes the tiles i, i + 1024, ... in rounds.
__global__ void __launch_bounds__(kAdjListBlock) k_src_adj_list(const int* __restrict__ tilecnt, int ntiles,
                                                                int2* __restrict__ info, int* __restrict__ nchunk) {
  __shared__ int wsum[kAdjListBlock / kWave + 1];
  int base = 0;
  for (int t0 = 0; t0 < ntiles; t0 += kAdjListBlock) {
    const int t = t0 + threadIdx.x;
    const int n = t < ntiles ? tilecnt[t] : 0;
    const int nc = (n + kAdjChunk - 1) / kAdjChunk;
    int total;
    const int c = base + block_exclusive_scan<kAdjListBlock>(nc, wsum, total);
    for (int k = 0; k < nc; ++k) info[c + k] = make_int2(t, k * kAdjChunk);
    base += total;
  }
  if (threadIdx.x == 0) *nchunk = base;
}

__global__ void __launch_bounds__(kAdjBlock) k_src_flow_adjoint(FPlan p, FGeo G, FlowGeo F,
                                                             const int2* __restrict__ info,
                                                             const int* __restrict__ nchunk,
                                                             const float2* __restrict__ gvr,
                                                             float* __restrict__ ggrid) {
  constexpr int T = kAdjT, L = T + 1;
  __shared__ int seg[kAdjMaxSlices + 1];          // prefix of the S slice ranges' lengths
  __shared__ int sbase[kAdjMaxSlices];
  __shared__ int bcnt[T * T], bstart[T * T];
  __shared__ int wsum[kAdjBlock / kWave + 1];
  __shared__ float sax[kAdjChunk], say[kAdjChunk], sv0[kAdjChunk], sv1[kAdjChunk];
  __shared__ float bsum[8][T * T];                // corner k = 2 * iy + ix, channel c: row 2 k + c
  __shared__ int org[2];
  if ((int)blockIdx.x >= *nchunk) return;
  const int2 ci = info[blockIdx.x];
  const int tid = threadIdx.x;
  const int TXb = (G.GW + G.stile - 1) / G.stile, TYb = (G.GH + G.stile - 1) / G.stile;
  const int b = ci.x / (TXb * TYb), tr = ci.x - b * TXb * TYb;
  const int tb = tr / TXb, tx = tr - tb * TXb;
  if (tid < kWave) {                               // slices s < S <= 64 of batch b: one wave
    int lo = 0, len = 0;
    if (tid < G.S) {
      const int2 r = src_tile_range(p, G, b, tid, tb, tx, p.start[2 * G.ncell_pad]);
      lo = r.x;
      len = r.y - r.x;
    }
    int incl = len;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
      const int y = __shfl_up(incl, d, kWave);
      if (tid >= d) incl += y;
    }
    seg[tid + 1] = incl;
    sbase[tid] = lo;
    if (tid == 0) {
      seg[0] = 0;
      org[0] = 0x7fffffff;
      org[1] = 0x7fffffff;
    }
  }
  bcnt[tid] = 0;
  __syncthreads();
  const int r0 = ci.y, r1 = min(seg[G.S], ci.y + kAdjChunk);
  GridCorners c[kAdjItems];
  float2 g[kAdjItems];
  bool live[kAdjItems];
  int mx = 0x7fffffff, my = 0x7fffffff;
#pragma unroll
  for (int u = 0; u < kAdjItems; ++u) {           // the chunk's records and gradients, then their corners
    const int r = r0 + u * kAdjBlock + tid;
    live[u] = r < r1;
    int q = 0;
    if (live[u]) {
      int s = 0;
      while (seg[s + 1] <= r) ++s;
      q = sbase[s] + (r - seg[s]);
    }
    const float4 f = live[u] ? p.srec[q].f : make_float4(0.f, 0.f, 0.f, 0.f);
    g[u] = live[u] ? gvr[q] : make_float2(0.f, 0.f);
    c[u] = grid_corners(f.x, f.y, F.Hg, F.Wg, F.sxw, F.syh, F.scale != 0);
    live[u] = live[u] && !(g[u].x == 0.f && g[u].y == 0.f);   // a zero row adds nothing
    if (live[u]) {
      const int y0 = c[u].o00 / F.Wg;
      mx = min(mx, c[u].o00 - y0 * F.Wg);
      my = min(my, y0);
    }
  }
  mx = wave_min_i(mx);
  my = wave_min_i(my);
  if ((tid & (kWave - 1)) == 0) {
    atomicMin(org, mx);
    atomicMin(org + 1, my);
  }
  __syncthreads();
  const int ox = org[0], oy = org[1];
  if (ox == 0x7fffffff) return;                   // every row of the chunk is zero
  const int64_t plane = (int64_t)F.Hg * F.Wg;
  float* gb = ggrid + (int64_t)b * 2 * plane;
  int bin[kAdjItems], rank[kAdjItems];
#pragma unroll
  for (int u = 0; u < kAdjItems; ++u) {
    bin[u] = -1;
    if (!live[u]) continue;
    const int y0 = c[u].o00 / F.Wg, x0 = c[u].o00 - y0 * F.Wg;
    const int bx = x0 - ox, by = y0 - oy;
    if ((unsigned)bx < (unsigned)T && (unsigned)by < (unsigned)T) {
      bin[u] = by * T + bx;
      rank[u] = atomicAdd(bcnt + bin[u], 1);
    } else {                                      // outside the window: the four corners directly
      atomicAdd(gb + c[u].o00, g[u].x * c[u].w00);
      atomicAdd(gb + c[u].o01, g[u].x * c[u].w01);
      atomicAdd(gb + c[u].o10, g[u].x * c[u].w10);
      atomicAdd(gb + c[u].o11, g[u].x * c[u].w11);
      atomicAdd(gb + plane + c[u].o00, g[u].y * c[u].w00);
      atomicAdd(gb + plane + c[u].o01, g[u].y * c[u].w01);
      atomicAdd(gb + plane + c[u].o10, g[u].y * c[u].w10);
      atomicAdd(gb + plane + c[u].o11, g[u].y * c[u].w11);
    }
  }
  __syncthreads();
  const int mine = bcnt[tid];
  int total;
  const int first = block_exclusive_scan<kAdjBlock>(mine, wsum, total);
  bstart[tid] = first;
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kAdjItems; ++u) {
    if (bin[u] < 0) continue;
    const int q = bstart[bin[u]] + rank[u];
    sax[q] = c[u].ax;
    say[q] = c[u].ay;
    sv0[q] = g[u].x;
    sv1[q] = g[u].y;
  }
  __syncthreads();
  float sum[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) sum[k] = 0.f;
  for (int q = first; q < first + mine; ++q) {
    const float fx = sax[q], fy = say[q];
    const float wx0 = 1.f - fx, wy0 = 1.f - fy;
    const float w[4] = {wx0 * wy0, fx * wy0, wx0 * fy, fx * fy};
    const float v0 = sv0[q], v1 = sv1[q];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      sum[2 * k] += v0 * w[k];
      sum[2 * k + 1] += v1 * w[k];
    }
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) bsum[k][tid] = sum[k];
  __syncthreads();
  // the second corner of an axis is the next node, or the same one on a grid of a single column (row)
  const int sx = F.Wg > 1 ? 1 : 0, sy = F.Hg > 1 ? 1 : 0;
  for (int a = tid; a < L * L; a += kAdjBlock) {
    const int ly = a / L, lx = a - ly * L;
    const int py = oy + ly, px = ox + lx;
    if (py >= F.Hg || px >= F.Wg) continue;
    float v0 = 0.f, v1 = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int cx = lx - (k & 1) * sx, cy = ly - (k >> 1) * sy;
      if ((unsigned)cx >= (unsigned)T || (unsigned)cy >= (unsigned)T) continue;
      v0 += bsum[2 * k][cy * T + cx];
      v1 += bsum[2 * k + 1][cy * T + cx];
    }
    const int64_t o = (int64_t)py * F.Wg + px;
    if (v0 != 0.f) atomicAdd(gb + o, v0);
    if (v1 != 0.f) atomicAdd(gb + plane + o, v1);
  }
}

// Backward of the trajectory model: every source (one lane per part of its slices, own-slice tile order) sums
// over the anchors of each slice s of its range, within R of its slice-centre position y_s, the gradients of the
// entry's position and velocity, Gy_s = sum_i gS_i k r / h^2 and Gv_s = sum_i gS_i k r at_i / h^2
// (r = x_i - (y_s + v_s at_i), the pair terms of the forward), and chains them in registers through
// y_s = p + sum_k cf_k g_k(c_s), v_s = sum_k cf_k g_k'(c_s): gp[j] = sum_s Gy_s and
// gcoef[j, k] = sum_s (Gy_s g_k(c_s) + Gv_s g_k'(c_s)) per axis (channels [y_1..y_K, x_1..x_K]).  Each source's
// gradients are complete in its lanes and written once, without atomics.
template <int K, bool DUP>
__device__ __forceinline__ void bwd_traj_source(const FPlan& p, const FGeo& G, float R, float R2, float atmax, float px,
                                                float py, const float (&cf)[2 * K], const float* __restrict__ tab,
                                                int sid, float tj, int key, int sp, int part, int2* rowtab,
                                                float (&gc)[2 * K], float& gpx, float& gpy) {
  const int plane_cells = G.GH * G.GW;
  const int* astart = p.start + G.ncell_pad;
  const int E = uni(p.start[G.ncell_pad]);
  const int* aid = (const int*)p.arec + 4;         // event id of record k: aid[8 * k]
  int lo_l, hi_l;
  slice_range(tj, G, lo_l, hi_l);
  if (kBwdParts > 1) {
    const int L = max(hi_l - lo_l + 1, 0);
    const int a = lo_l + (part * L) / kBwdParts, b = lo_l + ((part + 1) * L) / kBwdParts - 1;
    lo_l = a;
    hi_l = b;
  }
  const int bj = key / (G.S * plane_cells);
  for (int s = lo_l; s <= hi_l; ++s) {
    float yx, yy, vx, vy;
    traj_entry<K>(cf, px, py, tab, s, yx, yy, vx, vy);
    const float cs = slice_centre(s, G.delta);
    const float qx = clampf(yx, G.gx0, G.gx1), qy = clampf(yy, G.gy0, G.gy1);
    // this entry's own search radius: its pairs lie within cut h + |v_s| max|at| of y_s (the global R takes the
    // largest velocity of all entries); the same slack as search_radius
    float Rs = R, R2s = R2;
    {
      const float rs = G.cuth * 1.000001f + sqrtf(vx * vx + vy * vy) * atmax * 1.000001f + 0.01f;
      if (rs < R) {                                // false for NaN / inf velocities: keep the global walk
        Rs = rs;
        R2s = rs * rs;
      }
    }
    float gyx = 0.f, gyy = 0.f, gvx = 0.f, gvy = 0.f;
    walk_flat(astart, E, (bj * G.S + s) * plane_cells, qx, qy, Rs, R2s, G, rowtab, [&](int k, int e, auto step) {
      constexpr int U = decltype(step)::value;
      float4 A[U];
      int id[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        A[u] = ld((const float4*)p.brec + u, (uint32_t)k);
        if (DUP) id[u] = ld(aid + 8 * u, 8u * (uint32_t)k);
      }
      const int rem = e - k, self_u = sp - k;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float at = A[u].z - cs;
        const float dt = A[u].z - tj;
        const float rx = A[u].x - (yx + vx * at);
        const float ry = A[u].y - (yy + vy * at);
        const float d2 = rx * rx + ry * ry;
        const bool other = DUP ? id[u] != sid : u != self_u;
        const bool ok = other & !(fabsf(dt) > G.tau) & !(d2 > G.r2max) & (u < rem);
        // selects, not products with zero: records past the range end may hold anything, NaN included
        const float f = A[u].w * __builtin_amdgcn_exp2f(d2 * G.kexp);   // A.w = gS / h^2
        const float fx = f * rx, fy = f * ry;
        gyx = ok ? gyx + fx : gyx;
        gyy = ok ? gyy + fy : gyy;
        gvx = ok ? fmaf(fx, at, gvx) : gvx;
        gvy = ok ? fmaf(fy, at, gvy) : gvy;
      }
    });
    gpx += gyx;
    gpy += gyy;
    const float* row = tab + s * 2 * K;
#pragma unroll
    for (int k = 0; k < K; ++k) {
      const float g = row[k], gd = row[K + k];
      gc[k] = fmaf(gyy, g, fmaf(gvy, gd, gc[k]));
      gc[K + k] = fmaf(gyx, g, fmaf(gvx, gd, gc[K + k]));
    }
  }
}

template <int K>
__global__ void __launch_bounds__(kPairBlock) __attribute__((amdgpu_waves_per_eu(4))) k_fast_bwd_traj(FPlan p, FGeo G, int N, const float* __restrict__ coef,
                                                             const float* __restrict__ tab, float2* __restrict__ gp,
                                                             float* __restrict__ gcoef) {
  __shared__ int2 rowtab[kRowTab * kPairBlock];
  constexpr int kSrcPerWave = kWave / kBwdParts;
  const int lb = xcd_block((N + kPairBlock / kBwdParts - 1) / (kPairBlock / kBwdParts));
  if (lb < 0) return;
  const int lane = threadIdx.x & (kWave - 1);
  const int part = lane / kSrcPerWave, ls = lane - part * kSrcPerWave;
  const int wbase = (lb * (kPairBlock / kWave) + (int)(threadIdx.x / kWave)) * kSrcPerWave;
  const int EA = uni(p.start[2 * G.ncell_pad]);
  const int Nv = uni(p.start[3 * G.ncell_pad]) - EA;
  if (wbase >= Nv) return;
  const int n = min(kSrcPerWave, Nv - wbase);
  float R, R2;
  search_radius(p.P, G, R, R2);
  R = unif(R);
  R2 = unif(R2);
  const bool have = ls < n;
  const Rec SR = p.srec[wbase + min(ls, n - 1)];
  const int4 si = SR.i;
  const float tj = __int_as_float(si.x);
  float cf[2 * K], gc[2 * K];
#pragma unroll
  for (int c = 0; c < 2 * K; ++c) {
    cf[c] = coef[(int64_t)si.y * (2 * K) + c];
    gc[c] = 0.f;
  }
  const int sp = p.self[si.y];
  float gpx = 0.f, gpy = 0.f;
  if (have) {
    const float atmax = unif(ordered_to_float(p.P->atmax));
    if (uni(p.P->dup))
      bwd_traj_source<K, true>(p, G, R, R2, atmax, SR.f.x, SR.f.y, cf, tab, si.y, tj, si.z, sp, part,
                               rowtab + threadIdx.x, gc, gpx, gpy);
    else
      bwd_traj_source<K, false>(p, G, R, R2, atmax, SR.f.x, SR.f.y, cf, tab, si.y, tj, si.z, sp, part,
                                rowtab + threadIdx.x, gc, gpx, gpy);
  }
#pragma unroll
  for (int o = kSrcPerWave; o < kWave; o <<= 1) {  // the parts of a source sit kSrcPerWave lanes apart
    gpx += __shfl_xor(gpx, o);
    gpy += __shfl_xor(gpy, o);
#pragma unroll
    for (int c = 0; c < 2 * K; ++c) gc[c] += __shfl_xor(gc[c], o);
  }
  if (have && part == 0) {
    gp[si.y] = make_float2(gpx, gpy);
#pragma unroll
    for (int c = 0; c < 2 * K; ++c) gcoef[(int64_t)si.y * (2 * K) + c] = gc[c];
  }
}

// ------------------------------------------------------------------------------------------ host side
int64_t align256(int64_t n) { return (n + 255) & ~(int64_t)255; }

// Source tile edge in cells (about kSrcTilePx px) of a fine-cell size.
inline int src_tile_cells(float cell) { return std::min(16, std::max(2, (int)std::lround(kSrcTilePx / (double)cell))); }

// Bytes the flow adjoint keeps in the sort-record region: the per-source gradients, then its chunk list, chunk
// count and tile record counts.
inline int64_t adj_scratch_bytes(int64_t B, int64_t N, int64_t GW, int64_t GH, float cell) {
  const int64_t st = src_tile_cells(cell);
  const int64_t tiles = B * ((GW + st - 1) / st) * ((GH + st - 1) / st);
  const int64_t maxc = tiles + (N + kAdjChunk - 1) / kAdjChunk;
  return align256(N * 8) + maxc * (int64_t)sizeof(int2) + 64 * 4 + tiles * 4;
}

bool make_geo(const atl_fast_geometry* geo, FGeo& G) {
  if (!geo || geo->version != ATL_HIP_ABI_VERSION) return false;
  G.gx0 = geo->gx0; G.gy0 = geo->gy0; G.gx1 = geo->gx1; G.gy1 = geo->gy1; G.cf = geo->cell;
  G.icf = 1.f / G.cf;
  G.GW = (int)geo->GW; G.GH = (int)geo->GH; G.S = (int)geo->S; G.B = geo->B;
  G.ncell = (int)geo->ncell; G.ncell_pad = (int)geo->ncell_pad; G.MS = (int)geo->max_span;
  G.nblk_e = (int)((geo->N + kSrcPerBlock - 1) / kSrcPerBlock);
  G.nblk_a = (int)((geo->M + kAncPerBlock - 1) / kAncPerBlock);
  G.bshift = geo->bucket_shift;
  if (G.bshift < kMinBucketShift || G.bshift > kMaxBucketShift) return false;
  G.nbuckets = (int)((3 * geo->ncell_pad) >> G.bshift);
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
  // groups about kGroupWidth px wide whatever the cell size: a fixed cell count made groups of 3 px at h = 0.5,
  // where the per-pass set-up then dominates, and of 12 px at h = 2, where the box does
  G.gcells = std::min(16, std::max(1, (int)std::lround(kGroupWidth / (double)G.cf)));
  G.stile = src_tile_cells(G.cf);
  G.vplanes = geo->B * geo->S <= kMaxPlanes;
  return true;
}

template <typename T>
T* at_off(void* ws, int64_t off) { return (T*)((char*)ws + off); }

FPlan make_plan(void* ws, const atl_fast_geometry* geo) {
  FPlan p;
  p.epos = at_off<float4>(ws, geo->off_epos);
  p.etim = at_off<float>(ws, geo->off_etim);
  p.eself = at_off<int>(ws, geo->off_eself);
  p.arec = at_off<Rec>(ws, geo->off_arec);
  p.srec = at_off<Rec>(ws, geo->off_srec);
  p.brec = at_off<float4>(ws, geo->off_brec);
  p.self = at_off<int>(ws, geo->off_self);
  p.start = at_off<int>(ws, geo->off_start);
  p.P = at_off<FParams>(ws, geo->off_params);
  return p;
}

unsigned xcd_grid(int64_t nblocks) {
  const int64_t g = kXcd * kXcdRun;
  return (unsigned)(((nblocks + g - 1) / g) * g);
}

}  // namespace

// ================================================================================================ C-ABI
extern "C" {

int atl_fast_geometry_init(int64_t N, int64_t M, int64_t B, int64_t H, int64_t W, int64_t S, double h, double tau,
                           double cut, atl_fast_geometry* geo) {
  if (!geo || N < 0 || M < 0 || B < 1 || H < 1 || W < 1 || S < 1 || S > 65536 || !(h > 0) || !(tau >= 0) ||
      !(cut > 0) || !(h < 1e6) || !(tau < 1e6) || !(cut < 1e6) || H > (1 << 20) || W > (1 << 20)) {
    set_error("fast_geometry_init: bad arguments (N=%lld M=%lld B=%lld H=%lld W=%lld S=%lld h=%g tau=%g cut=%g)",
              (long long)N, (long long)M, (long long)B, (long long)H, (long long)W, (long long)S, h, tau, cut);
    return 1;
  }
  atl_fast_geometry g{};
  g.version = ATL_HIP_ABI_VERSION;
  g.N = N; g.M = M; g.B = B; g.H = H; g.W = W; g.S = S;
  g.h = h; g.tau = tau; g.cut = cut;
  // Cells of about 0.6 cut h: smaller cells cut fewer candidates per walk but add rows, passes and plan cells.
  // Measured on the 1M-event window (step time): 1.2 px beat 0.75 and 0.9 at h = 0.5, 1.8 beat 1.5 and 2.0 at
  // h = 1, 2.1 beat 1.8, 2.4 and 3.0 at h = 2.  Denser entries (rho per px^2 and slice on average) shift the
  // balance to the candidates: the 4M-event blobs ran 177 ms with 1.2 or 1.5 px cells and 194 ms with 1.8, so
  // above 2 entries per px^2 the size shrinks as rho^-1/4.  At most max(2.1, 2 R / 7) with R ~ cut h + 0.7, so
  // that a walk's rows still fit the forward's 8-row table.
  const double rho = (double)N * std::min(1.0, 2.0 * tau + 1.0 / (double)S) / ((double)B * (double)H * (double)W);
  const double dens = rho > 2.0 ? std::pow(2.0 / rho, 0.25) : 1.0;
  const double cmax = std::max(2.1, 2.0 * (cut * h + 0.7) / 7.0);
  const double cf = std::min(std::max(0.6 * cut * h * dens, 1.2), cmax);
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
  int shift = kMinBucketShift;
  double ncell_pad = 0, nbuckets = 0;
  for (; shift <= kMaxBucketShift; ++shift) {
    const double keys = std::ldexp(1.0, shift);
    ncell_pad = std::ceil(ncell / keys) * keys;
    nbuckets = 3 * ncell_pad / keys;
    if (nbuckets <= kMaxBuckets) break;
  }
  const double nblk = std::ceil((double)N / kSrcPerBlock) + std::ceil((double)M / kAncPerBlock);
  // GW, GH < 32768: anchor records pack (cy, cx) into 16-bit halves
  if (3 * ncell_pad + 1 >= 2.0e9 || ecap + M + N >= 2.0e9 || nbuckets > kMaxBuckets || nbuckets * nblk + 1 >= 2.0e9 ||
      g.GW >= 32768 || g.GH >= 32768) {
    set_error("fast_geometry_init: problem too large for the 32-bit plan (cells %.0f, entries %.0f)", ncell, ecap);
    return 1;
  }
  g.bucket_shift = shift;
  g.ncell = (int64_t)ncell;
  g.ncell_pad = (int64_t)ncell_pad;
  g.ecap = (int64_t)ecap;
  const int64_t nbh = (int64_t)(nbuckets * nblk);
  int64_t off = 0;
  // params and the bucket totals are adjacent: one fill clears both
  g.off_params = off;  off += align256(sizeof(FParams) + (B * S <= kMaxPlanes ? B * S * 4 : 0));
  g.off_part = off;    off += align256((int64_t)nbuckets * 4);        // bucket totals
  g.off_boff = off;    off += align256((int64_t)nbuckets * 4);        // bucket positions, then bucket ends
  g.off_cnt = off;     off += align256(nbh * 4);                      // per-block histograms, block-major
  g.off_start = off;   off += align256((3 * g.ncell_pad + 1) * 4);
  // the sort's records sit at their bucket positions in all three key spaces (the linear model's anchor and
  // source records after the entries' counted places), so the region holds ecap + M + N records; after the plan
  // it also serves the flow adjoint's scratch (per-source gradients, chunk list, tile counts)
  g.off_trec = off;    off += align256(std::max((g.ecap + M + N) * (int64_t)sizeof(Rec),
                                                adj_scratch_bytes(B, N, g.GW, g.GH, g.cell)));
  // the walks read up to kUnroll - 1 records past a range end: entry and anchor arrays carry that padding
  g.off_epos = off;    off += align256((g.ecap + kUnroll) * (int64_t)sizeof(float4));
  g.off_etim = off;    off += align256((g.ecap + kUnroll) * (int64_t)sizeof(float));
  g.off_eself = off;   off += align256(N * (int64_t)sizeof(int));
  g.off_arec = off;    off += align256((M + kUnroll) * (int64_t)sizeof(Rec));
  g.off_srec = off;    off += align256(N * (int64_t)sizeof(Rec));
  g.off_brec = off;    off += align256((M + kUnroll) * (int64_t)sizeof(float4));
  g.off_self = off;    off += align256(N * (int64_t)sizeof(int));
  g.ws_bytes = off;
  *geo = g;
  return 0;
}

}  // extern "C"

namespace {

// The plan's launches for source model K (0: linear, x / v per source; K > 0: trajectories, x = starts p,
// coef rows and the slice table tab).
template <int K>
int fast_plan_impl(const atl_fast_geometry* geo, const FGeo& G, const float* x, const float* t, const float* v,
                   const int64_t* b, const int64_t* anchors, const float* anchor_xy, const float* coef,
                   const float* tab, void* ws, hipStream_t stream) {
  const int64_t N = geo->N, M = geo->M;
  FParams* P = at_off<FParams>(ws, geo->off_params);
  int* cnt = at_off<int>(ws, geo->off_cnt);
  int* bpos = at_off<int>(ws, geo->off_boff);
  int* tot = at_off<int>(ws, geo->off_part);
  Rec* trec = at_off<Rec>(ws, geo->off_trec);
  const int nblk = G.nblk_e + G.nblk_a;
  const int64_t nclear = (geo->off_part - geo->off_params) / 4 + G.nbuckets;   // params and bucket totals
  hipLaunchKernelGGL(k_fill_zero, dim3(grid_for(nclear)), dim3(kBlock), 0, stream, (int*)P, nclear);
  const size_t lds = (size_t)G.nbuckets * sizeof(int);
  if (nblk > 0)
    hipLaunchKernelGGL((k_sort_pass1<false, K>), dim3(nblk), dim3(kP1Block), lds, stream, (const float2*)x, t,
                       (const float2*)v, b, N, anchors, (const float2*)anchor_xy, M, G, cnt, tot, (Rec*)nullptr, P,
                       at_off<int>(ws, geo->off_self), at_off<int>(ws, geo->off_eself), coef, tab);
  scan_small(tot, G.nbuckets, bpos, stream);
  // the linear model defers its entries: pass 1 places the anchor and source records, pass 2 sorts them, and
  // k_entry_pass / k_entry_rank / k_entry_write build the entries from the sorted source records (8-byte items)
  constexpr bool kSplit = K == 0;
  if (nblk > 0)
    hipLaunchKernelGGL((k_sort_pass1<true, K, !kSplit>), dim3(nblk), dim3(kP1Block), lds, stream,
                       (const float2*)x, t, (const float2*)v, b, N, anchors, (const float2*)anchor_xy, M, G, cnt,
                       bpos, trec, (FParams*)nullptr, (int*)nullptr, (int*)nullptr, coef, tab);
  const SortOut out{at_off<int>(ws, geo->off_start), at_off<float4>(ws, geo->off_epos),
                    at_off<float>(ws, geo->off_etim), at_off<int>(ws, geo->off_eself),
                    at_off<Rec>(ws, geo->off_arec), at_off<Rec>(ws, geo->off_srec), at_off<int>(ws, geo->off_self)};
  // the anchor and source spaces in groups of kSortGroupKeys keys; the entries' space (trajectory model) one
  // bucket per workgroup
  constexpr int kSortGroupKeys = 4096;
  auto pass2g = G.bshift == 10 ? k_sort_pass2<10, kSortGroupKeys / 1024> : G.bshift == 11 ? k_sort_pass2<11, kSortGroupKeys / 2048>
              : G.bshift == 12 ? k_sort_pass2<12, 1> : k_sort_pass2<13, 1>;
  const int bpk = G.ncell_pad >> G.bshift;
  const int grp = std::max(1, kSortGroupKeys >> G.bshift);
  const int gps = (bpk + grp - 1) / grp;
  hipLaunchKernelGGL(pass2g, dim3(2 * gps), dim3(kSortBlock), 0, stream, (const int*)bpos, (const int*)tot, 1,
                     (const Rec*)trec, G, out);
  if (!kSplit) {
    auto pass2 = G.bshift == 10 ? k_sort_pass2<10, 1> : G.bshift == 11 ? k_sort_pass2<11, 1>
               : G.bshift == 12 ? k_sort_pass2<12, 1> : k_sort_pass2<13, 1>;
    hipLaunchKernelGGL(pass2, dim3(bpk), dim3(kSortBlock), 0, stream, (const int*)bpos, (const int*)tot, 0,
                       (const Rec*)trec, G, out);
  }
  if (kSplit) {
    int2* item = (int2*)trec;                    // [0, E) of the items; pass 2 has read the records
    const Rec* srec = at_off<Rec>(ws, geo->off_srec);
    const int* start = at_off<int>(ws, geo->off_start);
    const size_t elds = (size_t)bpk * sizeof(int);
    // per-block counts: (N / kEntSrcPerBlock) * bpk <= nblk * nbuckets ints (kEntSrcPerBlock = kSrcPerBlock / 2)
    static_assert(2 * kEntSrcPerBlock >= kSrcPerBlock, "the entry passes' counts fit the plan's count array");
    const unsigned eblk = (unsigned)((N + kEntSrcPerBlock - 1) / kEntSrcPerBlock);
    if (eblk > 0 && G.MS <= 12) {                // keys and ranks in registers
      auto scatter = G.MS <= 8 ? k_entry_scatter<8> : k_entry_scatter<12>;
      hipLaunchKernelGGL(scatter, dim3(eblk), dim3(kEntBlock), elds, stream, srec, start, G, bpos, item);
    } else if (eblk > 0) {
      hipLaunchKernelGGL(k_entry_pass<false>, dim3(eblk), dim3(kEntBlock), elds, stream, srec, start, G, cnt,
                         bpos, item);
      hipLaunchKernelGGL(k_entry_pass<true>, dim3(eblk), dim3(kEntBlock), elds, stream, srec, start, G, cnt,
                         bpos, item);
    }
    auto erank = G.bshift == 10 ? k_entry_rank<10> : G.bshift == 11 ? k_entry_rank<11>
               : G.bshift == 12 ? k_entry_rank<12> : k_entry_rank<13>;
    int2* sorted = item + geo->ecap;             // [ecap, ecap + E) of the items' space: 16 ecap <= 32 (ecap + M + N) bytes
    hipLaunchKernelGGL(erank, dim3(bpk), dim3(kSortBlock), 0, stream, (const int*)bpos, (const int*)tot,
                       (const int2*)item, sorted, out.start, G);
    const int64_t wblk = (geo->ecap + kBlock * kEntWrite - 1) / (kBlock * kEntWrite);
    if (wblk > 0)                                // runs of consecutive entries on one XCD (see xcd_block)
      hipLaunchKernelGGL(k_entry_write, dim3(xcd_grid(wblk)), dim3(kBlock), 0, stream, (const int2*)sorted, srec,
                         G, out, (int)wblk);
  }
  return 0;
}

bool plan_args_ok(const atl_fast_geometry* geo, FGeo& G, void* ws, int64_t ws_bytes, const char* what) {
  if (!make_geo(geo, G)) { set_error("%s: geometry not initialised by atl_fast_geometry_init", what); return false; }
  if (!ws || ws_bytes < geo->ws_bytes) { set_error("%s: workspace of %lld bytes, need %lld", what, (long long)ws_bytes, (long long)geo->ws_bytes); return false; }
  return true;
}

}  // namespace

extern "C" {

int atl_fast_plan(const atl_fast_geometry* geo, const float* x, const float* t, const float* v, const int64_t* b,
                  const int64_t* anchors, const float* anchor_xy, void* ws, int64_t ws_bytes, hipStream_t stream) {
  FGeo G;
  if (!plan_args_ok(geo, G, ws, ws_bytes, "fast_plan")) return 1;
  const int64_t N = geo->N, M = geo->M;
  if ((N > 0 && (!x || !t || !v || !b)) || (M > 0 && !anchors && M != N)) { set_error("fast_plan: null input"); return 1; }
  fast_plan_impl<0>(geo, G, x, t, v, b, anchors, anchor_xy, nullptr, nullptr, ws, stream);
  return check_launch("fast_plan");
}

int atl_fast_plan_traj(const atl_fast_geometry* geo, const float* p, const float* coef, int64_t K, const float* tab,
                       const float* t, const int64_t* b, const int64_t* anchors, const float* anchor_xy, void* ws,
                       int64_t ws_bytes, hipStream_t stream) {
  FGeo G;
  if (!plan_args_ok(geo, G, ws, ws_bytes, "fast_plan_traj")) return 1;
  const int64_t N = geo->N, M = geo->M;
  if (K < 1 || K > kTrajPairMaxK) { set_error("fast_plan_traj: K = %lld outside 1..%d", (long long)K, kTrajPairMaxK); return 1; }
  if ((N > 0 && (!p || !coef || !tab || !t || !b)) || (M > 0 && !anchors && M != N)) { set_error("fast_plan_traj: null input"); return 1; }
  switch (K) {
#define ATL_K(k) case k: fast_plan_impl<k>(geo, G, p, t, nullptr, b, anchors, anchor_xy, coef, tab, ws, stream); break;
    ATL_K(1) ATL_K(2) ATL_K(3) ATL_K(4) ATL_K(5) ATL_K(6) ATL_K(7) ATL_K(8) ATL_K(9) ATL_K(10) ATL_K(11) ATL_K(12)
#undef ATL_K
  }
  return check_launch("fast_plan_traj");
}

int atl_fast_pair_fwd(const atl_fast_geometry* geo, const void* ws, float* out, int* count, hipStream_t stream) {
  FGeo G;
  if (!make_geo(geo, G)) { set_error("fast_pair_fwd: geometry not initialised"); return 1; }
  if (!ws || (geo->M > 0 && !out)) { set_error("fast_pair_fwd: null argument"); return 1; }
  if (geo->M == 0) return 0;
  const FPlan p = make_plan((void*)ws, geo);
  const unsigned grid = xcd_grid((geo->M + kAnchorsPerBlock - 1) / kAnchorsPerBlock);
  if (count)
    hipLaunchKernelGGL(k_fast_fwd<true>, dim3(grid), dim3(kPairBlock), 0, stream, p, G, (int)geo->M, out, count);
  else
    hipLaunchKernelGGL(k_fast_fwd<false>, dim3(grid), dim3(kPairBlock), 0, stream, p, G, (int)geo->M, out, count);
  return check_launch("fast_pair_fwd");
}

int atl_fast_pair_bwd(const atl_fast_geometry* geo, void* ws, const float* gS, float* gv, hipStream_t stream) {
  FGeo G;
  if (!make_geo(geo, G)) { set_error("fast_pair_bwd: geometry not initialised"); return 1; }
  if (!ws || (geo->N > 0 && !gv) || (geo->M > 0 && !gS)) { set_error("fast_pair_bwd: null argument"); return 1; }
  if (geo->N == 0) return 0;
  const FPlan p = make_plan(ws, geo);
  hipLaunchKernelGGL(k_fast_gather_gs, dim3(grid_for(std::max(geo->M, geo->N))), dim3(kBlock), 0, stream, p, G,
                     (int)geo->M, gS, (int)geo->N, (float2*)gv);
  if (geo->M > 0)
    hipLaunchKernelGGL(k_fast_bwd, dim3(xcd_grid((geo->N + kPairBlock / kBwdParts - 1) / (kPairBlock / kBwdParts))),
                       dim3(kPairBlock), 0, stream, p, G, (int)geo->N, (float2*)gv, (float2*)nullptr);
  return check_launch("fast_pair_bwd");
}

// The flow path's backward in two steps: the pair backward writes each source's velocity gradient by source
// record into the plan's temporary sort records (dead after the plan), and the adjoint accumulates them into the
// flow grid.  atl_fast_pair_bwd_flow runs both.
int atl_fast_pair_bwd_src(const atl_fast_geometry* geo, void* ws, const float* gS, hipStream_t stream) {
  FGeo G;
  if (!make_geo(geo, G)) { set_error("fast_pair_bwd_src: geometry not initialised"); return 1; }
  if (!ws || (geo->M > 0 && !gS)) { set_error("fast_pair_bwd_src: null argument"); return 1; }
  if (geo->N == 0 || geo->M == 0) return 0;
  const FPlan p = make_plan(ws, geo);
  float2* gvr = at_off<float2>(ws, geo->off_trec);
  hipLaunchKernelGGL(k_fast_gather_gs, dim3(grid_for(std::max(geo->M, geo->N))), dim3(kBlock), 0, stream, p, G,
                     (int)geo->M, gS, (int)geo->N, (float2*)nullptr);
  hipLaunchKernelGGL(k_fast_bwd, dim3(xcd_grid((geo->N + kPairBlock / kBwdParts - 1) / (kPairBlock / kBwdParts))),
                     dim3(kPairBlock), 0, stream, p, G, (int)geo->N, (float2*)nullptr, gvr);
  return check_launch("fast_pair_bwd_src");
}

int atl_fast_flow_adjoint(const atl_fast_geometry* geo, void* ws, int64_t Hg, int64_t Wg, int64_t img_h,
                          int64_t img_w, float* ggrid, hipStream_t stream) {
  FGeo G;
  if (!make_geo(geo, G)) { set_error("fast_flow_adjoint: geometry not initialised"); return 1; }
  if (Hg < 1 || Wg < 1 || (double)geo->B * 2 * Hg * Wg >= 2.0e9 || G.S > kAdjMaxSlices) { set_error("fast_flow_adjoint: bad sizes (Hg=%lld Wg=%lld, S=%d <= %d)", (long long)Hg, (long long)Wg, G.S, kAdjMaxSlices); return 1; }
  if (!ws || !ggrid) { set_error("fast_flow_adjoint: null argument"); return 1; }
  if (geo->N == 0 || geo->M == 0) {              // no pairs: a zero gradient (0.0f is all-zero bits)
    const int64_t ng = geo->B * 2 * Hg * Wg;
    hipLaunchKernelGGL(k_fill_zero, dim3(grid_for(ng)), dim3(kBlock), 0, stream, (int*)ggrid, ng);
    return check_launch("fast_flow_adjoint");
  }
  const FPlan p = make_plan(ws, geo);
  const float2* gvr = at_off<float2>(ws, geo->off_trec);
  FlowGeo F;
  F.Hg = (int)Hg;
  F.Wg = (int)Wg;
  F.scale = img_h > 0 && img_w > 0;
  F.sxw = (float)(img_w - 1 > 1 ? img_w - 1 : 1);
  F.syh = (float)(img_h - 1 > 1 ? img_h - 1 : 1);
  const int64_t tiles = geo->B * ((G.GW + G.stile - 1) / G.stile) * ((G.GH + G.stile - 1) / G.stile);
  const int64_t maxc = tiles + (geo->N + kAdjChunk - 1) / kAdjChunk;   // chunks, at most (adj_scratch_bytes)
  int2* info = (int2*)(at_off<char>(ws, geo->off_trec) + align256(geo->N * 8));   // after the gradients
  int* nchunk = (int*)(info + maxc);
  int* tilecnt = nchunk + 64;
  int SP = 1;
  while (SP < G.S) SP <<= 1;
  const int64_t ng = geo->B * 2 * Hg * Wg;      // the gradient is written, not added to: cleared here first
  hipLaunchKernelGGL(k_src_tile_counts, dim3(grid_for(std::max<int64_t>(tiles * SP, ng / 4))), dim3(kBlock), 0, stream,
                     p, G, (int)tiles, SP, tilecnt, ggrid, ng);
  hipLaunchKernelGGL(k_src_adj_list, dim3(1), dim3(kAdjListBlock), 0, stream, (const int*)tilecnt, (int)tiles, info,
                     nchunk);
  hipLaunchKernelGGL(k_src_flow_adjoint, dim3((unsigned)maxc), dim3(kAdjBlock), 0, stream, p, G, F,
                     (const int2*)info, (const int*)nchunk, gvr, ggrid);
  return check_launch("fast_flow_adjoint");
}

int atl_fast_pair_bwd_flow(const atl_fast_geometry* geo, void* ws, const float* gS, int64_t Hg, int64_t Wg,
                           int64_t img_h, int64_t img_w, float* ggrid, hipStream_t stream) {
  if (atl_fast_pair_bwd_src(geo, ws, gS, stream) != 0) return 1;
  return atl_fast_flow_adjoint(geo, ws, Hg, Wg, img_h, img_w, ggrid, stream);
}

int atl_fast_pair_bwd_traj(const atl_fast_geometry* geo, void* ws, const float* gS, const float* coef, int64_t K,
                           const float* tab, float* gp, float* gcoef, hipStream_t stream) {
  FGeo G;
  if (!make_geo(geo, G)) { set_error("fast_pair_bwd_traj: geometry not initialised"); return 1; }
  if (K < 1 || K > kTrajPairMaxK) { set_error("fast_pair_bwd_traj: K = %lld outside 1..%d", (long long)K, kTrajPairMaxK); return 1; }
  if (!ws || (geo->N > 0 && (!gp || !gcoef || !coef || !tab)) || (geo->M > 0 && !gS)) { set_error("fast_pair_bwd_traj: null argument"); return 1; }
  if (geo->N == 0) return 0;
  const FPlan p = make_plan(ws, geo);
  // gp cleared by the record pass, gcoef here: sources outside the plan keep zero gradients
  hipLaunchKernelGGL(k_fill_zero, dim3(grid_for(geo->N * 2 * K)), dim3(kBlock), 0, stream, (int*)gcoef, geo->N * 2 * K);
  hipLaunchKernelGGL(k_fast_gather_gs, dim3(grid_for(std::max(geo->M, geo->N))), dim3(kBlock), 0, stream, p, G,
                     (int)geo->M, gS, (int)geo->N, (float2*)gp);
  if (geo->M > 0) {
    const dim3 grid(xcd_grid((geo->N + kPairBlock / kBwdParts - 1) / (kPairBlock / kBwdParts))), block(kPairBlock);
    switch (K) {
#define ATL_K(k) case k: hipLaunchKernelGGL(k_fast_bwd_traj<k>, grid, block, 0, stream, p, G, (int)geo->N, coef, tab, (float2*)gp, gcoef); break;
      ATL_K(1) ATL_K(2) ATL_K(3) ATL_K(4) ATL_K(5) ATL_K(6) ATL_K(7) ATL_K(8) ATL_K(9) ATL_K(10) ATL_K(11) ATL_K(12)
#undef ATL_K
    }
  }
  return check_launch("fast_pair_bwd_traj");
}

}  // extern "C"
