// k-nearest-neighbour look-up of MotionPriorCMax's displacement table (atl/objectives/mpcm.py:30-42,56-78): for
// every plane p (batch x time bin) and query q (a look-up-table cell centre), the k nearest of the plane's n points
// (tile-trajectory positions).  The reference computes a dense (Q x n) distance matrix per plane (torch.cdist) and
// a top-k over it; here the points are binned once into a uniform grid of about one point per cell and every query
// searches rings of cells around its own cell, keeping a sorted top-k in registers, until no unvisited cell can
// hold a closer point.
//
// Order: squared distance (qx - px)^2 + (qy - py)^2 with each product and the sum rounded in fp32 (the file is built
// with -ffp-contract=off), ties by the lower point index; the indices are written in that order.  This is the
// exact-distance order of the reference's GPU path (pykeops argKmin on (x_i - y_j)^2); its CPU path (cdist's
// matrix-product form, then topk) selects the same set wherever the k-th and (k+1)-th distances are apart, and
// leaves the order of exact ties open.  Points whose distance is not finite are never selected (their slots,
// possible only if fewer than k finite points exist, hold -1).
#include "common.h"
#include "scan.h"
#include "../../include/atl_hip.h"

#include <cmath>

using namespace atlhip;

namespace {

constexpr int kKnnMaxK = 32;
constexpr int kGeomBlock = 1024;

// Grid of one plane (shared by all planes: the queries define it).  Cell (cx, cy) covers
// [ox + cx * csx, ox + (cx + 1) * csx) x [oy + cy * csy, ...); positions outside the grid are clamped into the border
// cells, whose extent is therefore unbounded on their outer sides.
struct KnnGeom {
  float ox, oy, csx, csy, icx, icy;
  int GX, GY;
};

struct KnnLayout {
  int64_t geom, cnt, start, part, pts, bytes;
};

inline int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }

KnnLayout knn_layout(int64_t P, int64_t n) {
  const int64_t ncap = n + 1;                      // cells per plane, at most
  const int64_t ncell = P * ncap;
  KnnLayout L;
  int64_t off = 0;
  L.geom = off;  off += align256(sizeof(KnnGeom));
  L.cnt = off;   off += align256(ncell * 4);
  L.start = off; off += align256((ncell + 1) * 4);
  L.part = off;  off += align256((scan_tiles(ncell) + 1) * 4);
  L.pts = off;   off += align256(P * n * 16);
  L.bytes = off;
  return L;
}

__device__ __forceinline__ int cell_of(float p, float o, float ic, int G) {
  const float c = floorf((p - o) * ic);
  return (int)fminf(fmaxf(c, 0.f), (float)(G - 1));   // NaN -> 0
}

// The queries' bounding box, split into about n cells (at most n + 1) of aspect close to 1.
__global__ void __launch_bounds__(kGeomBlock) k_knn_geom(const float2* __restrict__ q, int64_t Q, int64_t n,
                                                         KnnGeom* __restrict__ geo) {
  __shared__ float red[4][kGeomBlock / kWave];
  float x0 = INFINITY, y0 = INFINITY, x1 = -INFINITY, y1 = -INFINITY;
  for (int64_t i = threadIdx.x; i < Q; i += kGeomBlock) {
    const float2 p = q[i];
    if (isfinite(p.x) && isfinite(p.y)) {
      x0 = fminf(x0, p.x); x1 = fmaxf(x1, p.x);
      y0 = fminf(y0, p.y); y1 = fmaxf(y1, p.y);
    }
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    x0 = fminf(x0, __shfl_xor(x0, d, kWave)); x1 = fmaxf(x1, __shfl_xor(x1, d, kWave));
    y0 = fminf(y0, __shfl_xor(y0, d, kWave)); y1 = fmaxf(y1, __shfl_xor(y1, d, kWave));
  }
  const int w = threadIdx.x / kWave;
  if ((threadIdx.x & (kWave - 1)) == 0) { red[0][w] = x0; red[1][w] = x1; red[2][w] = y0; red[3][w] = y1; }
  __syncthreads();
  if (threadIdx.x != 0) return;
  for (int k = 1; k < kGeomBlock / kWave; ++k) {
    x0 = fminf(x0, red[0][k]); x1 = fmaxf(x1, red[1][k]); y0 = fminf(y0, red[2][k]); y1 = fmaxf(y1, red[3][k]);
  }
  if (!(x0 <= x1)) { x0 = 0.f; x1 = 0.f; }       // no finite query: any grid will do
  if (!(y0 <= y1)) { y0 = 0.f; y1 = 0.f; }
  const float w_ = fmaxf(x1 - x0, 1.f), h_ = fmaxf(y1 - y0, 1.f);
  const double ncap = (double)n + 1.0;
  const double cs = sqrt((double)w_ * (double)h_ / (double)(n > 0 ? n : 1));
  int GX = (int)fmin(fmax(ceil((double)w_ / cs), 1.0), ncap);
  int GY = (int)fmin(fmax(ceil((double)h_ / cs), 1.0), floor(ncap / GX));
  GY = GY < 1 ? 1 : GY;
  KnnGeom g;
  g.ox = x0; g.oy = y0;
  g.csx = w_ / (float)GX; g.csy = h_ / (float)GY;
  g.icx = (float)GX / w_; g.icy = (float)GY / h_;
  g.GX = GX; g.GY = GY;
  *geo = g;
}

__global__ void __launch_bounds__(kBlock) k_knn_zero(int* __restrict__ p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i < n) p[i] = 0;
}

// Point counts per cell (plane-major, ncap cells per plane); SCATTER: each point takes a slot of its cell (filled
// from the cell's end: the counts run back to zero) and writes (x, y, index) there.
template <bool SCATTER>
__global__ void __launch_bounds__(kBlock) k_knn_bin(const float2* __restrict__ pts, int64_t P, int64_t n,
                                                    const KnnGeom* __restrict__ geo, int* __restrict__ cnt,
                                                    const int* __restrict__ start, float4* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (i >= P * n) return;
  const KnnGeom g = *geo;
  const int64_t plane = i / n;
  const int j = (int)(i - plane * n);
  const float2 p = pts[i];
  const int64_t c = plane * (n + 1) + (int64_t)cell_of(p.y, g.oy, g.icy, g.GY) * g.GX + cell_of(p.x, g.ox, g.icx, g.GX);
  if (!SCATTER) {
    atomicAdd(cnt + c, 1);
  } else {
    const int slot = start[c] + atomicSub(cnt + c, 1) - 1;
    out[slot] = make_float4(p.x, p.y, __int_as_float(j), 0.f);
  }
}

// (d, j) before (D, J) in the output order
__device__ __forceinline__ bool before(float d, int j, float D, int J) { return d < D || (d == D && j < J); }

// One query per thread: rings of cells around its own cell, each ring's rows read as contiguous cell ranges; the
// search ends when the k-th best distance is below the squared distance to every unvisited cell (with a slack
// that covers the rounding of the binning), or when every cell has been visited.
template <int KC>
__global__ void __launch_bounds__(kBlock) k_knn_query(const float2* __restrict__ qs, int64_t Q, int64_t n, int k,
                                                      const KnnGeom* __restrict__ geo, const int* __restrict__ start,
                                                      const float4* __restrict__ pts, int64_t* __restrict__ out) {
  const int64_t plane = blockIdx.y;
  const int64_t qi = (int64_t)blockIdx.x * kBlock + threadIdx.x;
  if (qi >= Q) return;
  const KnnGeom g = *geo;
  const float2 q = qs[qi];
  const int* __restrict__ cs = start + plane * (n + 1);
  const int qcx = cell_of(q.x, g.ox, g.icx, g.GX), qcy = cell_of(q.y, g.oy, g.icy, g.GY);
  float D[KC];
  int J[KC];
#pragma unroll
  for (int s = 0; s < KC; ++s) { D[s] = INFINITY; J[s] = 0x7fffffff; }
  float dk = INFINITY;                             // the k-th entry (slot k - 1)
  int jk = 0x7fffffff;
  // slack of the unvisited-cell bounds: a point can be binned one rounding away from its cell's edge
  const float slack = 1e-4f * (g.csx + g.csy) + 1e-5f * (fabsf(g.ox) + fabsf(g.oy) + fabsf(q.x) + fabsf(q.y));
  const int rmax = max(g.GX, g.GY);
  for (int r = 0; r <= rmax; ++r) {
    const int y0 = max(qcy - r, 0), y1 = min(qcy + r, g.GY - 1);
    for (int y = y0; y <= y1; ++y) {
      const bool edge_row = (y == qcy - r) || (y == qcy + r);
      // the ring's cells of row y: the whole span on its top and bottom rows, else its two end cells
      for (int part = 0; part < (edge_row ? 1 : 2); ++part) {
        int x0, x1;
        if (edge_row) { x0 = qcx - r; x1 = qcx + r; }
        else { x0 = part == 0 ? qcx - r : qcx + r; x1 = x0; }
        x0 = max(x0, 0); x1 = min(x1, g.GX - 1);
        if (x0 > x1) continue;
        const int b = cs[y * g.GX + x0], e = cs[y * g.GX + x1 + 1];
        for (int t = b; t < e; ++t) {
          const float4 p = pts[t];
          const float dx = q.x - p.x, dy = q.y - p.y;
          const float d = dx * dx + dy * dy;
          const int j = __float_as_int(p.z);
          if (!before(d, j, dk, jk)) continue;
          float cd = d;
          int cj = j;
#pragma unroll
          for (int s = 0; s < KC; ++s) {           // insertion: the array stays sorted by (d, j)
            const bool lt = before(cd, cj, D[s], J[s]);
            const float td = D[s];
            const int tj = J[s];
            D[s] = lt ? cd : td;
            J[s] = lt ? cj : tj;
            cd = lt ? td : cd;
            cj = lt ? tj : cj;
          }
          dk = D[0];
          jk = J[0];
#pragma unroll
          for (int s = 1; s < KC; ++s) {
            dk = s == k - 1 ? D[s] : dk;
            jk = s == k - 1 ? J[s] : jk;
          }
        }
      }
    }
    // distance from q to the nearest unvisited cell: beyond each side of the (2r + 1)^2 block that is not at the
    // grid's edge (border cells extend to infinity, so a block side at the edge leaves nothing beyond it)
    float lb = INFINITY;
    if (qcx - r > 0) lb = fminf(lb, q.x - (g.ox + (float)(qcx - r) * g.csx));
    if (qcx + r < g.GX - 1) lb = fminf(lb, (g.ox + (float)(qcx + r + 1) * g.csx) - q.x);
    if (qcy - r > 0) lb = fminf(lb, q.y - (g.oy + (float)(qcy - r) * g.csy));
    if (qcy + r < g.GY - 1) lb = fminf(lb, (g.oy + (float)(qcy + r + 1) * g.csy) - q.y);
    if (lb == INFINITY) break;                     // every cell visited
    lb = fmaxf(lb - slack, 0.f);
    if (dk < lb * lb) break;                       // finite and closer than anything unvisited
  }
  int64_t* o = out + (plane * Q + qi) * k;
#pragma unroll
  for (int s = 0; s < KC; ++s)
    if (s < k) o[s] = D[s] < INFINITY ? (int64_t)J[s] : (int64_t)-1;
}

}  // namespace

extern "C" {

int64_t atl_knn_ws_bytes(int64_t P, int64_t n) {
  if (P < 0 || n < 0 || P * (n + 1) >= (int64_t)1 << 31) return -1;
  return knn_layout(P, n).bytes;
}

int atl_knn_indices(const float* queries, int64_t Q, const float* points, int64_t P, int64_t n, int64_t k,
                    int64_t* idx, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (Q < 0 || P < 0 || n < 0 || k < 1 || k > kKnnMaxK || k > n || P * (n + 1) >= (int64_t)1 << 31 ||
      Q > (int64_t)1 << 30 || P > 65535) {
    set_error("knn_indices: bad sizes Q=%lld P=%lld n=%lld k=%lld (1 <= k <= min(n, %d))", (long long)Q, (long long)P,
              (long long)n, (long long)k, kKnnMaxK);
    return 1;
  }
  if (Q == 0 || P == 0) return 0;
  const KnnLayout L = knn_layout(P, n);
  if (!ws || ws_bytes < L.bytes) { set_error("knn_indices: workspace of %lld bytes, need %lld", (long long)ws_bytes, (long long)L.bytes); return 1; }
  if (!queries || !points || !idx) { set_error("knn_indices: null argument"); return 1; }
  char* w = (char*)ws;
  KnnGeom* geo = (KnnGeom*)(w + L.geom);
  int* cnt = (int*)(w + L.cnt);
  int* start = (int*)(w + L.start);
  float4* pts = (float4*)(w + L.pts);
  const int64_t ncell = P * (n + 1), np = P * n;
  hipLaunchKernelGGL(k_knn_geom, dim3(1), dim3(kGeomBlock), 0, stream, (const float2*)queries, Q, n, geo);
  hipLaunchKernelGGL(k_knn_zero, dim3(grid_for(ncell)), dim3(kBlock), 0, stream, cnt, ncell);
  hipLaunchKernelGGL((k_knn_bin<false>), dim3(grid_for(np)), dim3(kBlock), 0, stream, (const float2*)points, P, n,
                     (const KnnGeom*)geo, cnt, (const int*)nullptr, (float4*)nullptr);
  scan32(cnt, ncell, (int*)(w + L.part), start, stream);
  hipLaunchKernelGGL((k_knn_bin<true>), dim3(grid_for(np)), dim3(kBlock), 0, stream, (const float2*)points, P, n,
                     (const KnnGeom*)geo, cnt, (const int*)start, pts);
  const dim3 grid(grid_for(Q), (unsigned)P);
  if (k <= 8)
    hipLaunchKernelGGL((k_knn_query<8>), grid, dim3(kBlock), 0, stream, (const float2*)queries, Q, n, (int)k,
                       (const KnnGeom*)geo, (const int*)start, (const float4*)pts, idx);
  else if (k <= 16)
    hipLaunchKernelGGL((k_knn_query<16>), grid, dim3(kBlock), 0, stream, (const float2*)queries, Q, n, (int)k,
                       (const KnnGeom*)geo, (const int*)start, (const float4*)pts, idx);
  else
    hipLaunchKernelGGL((k_knn_query<32>), grid, dim3(kBlock), 0, stream, (const float2*)queries, Q, n, (int)k,
                       (const KnnGeom*)geo, (const int*)start, (const float4*)pts, idx);
  return check_launch("knn_indices");
}

}  // extern "C"
