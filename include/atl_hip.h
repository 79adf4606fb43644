/* C-ABI of libatl_hip.so: the MI355X (gfx950) event-transport hot path of atl.
 *
 * Replaces the reference's pybind module (csrc/atl_cpu.cpp:299-329, declarations csrc/atl_ops.h:18-75) as the
 * boundary under atl/ops/functional.py.  Conventions for every entry point:
 *   - plain device pointers, sizes and a hipStream_t; kernels are launched asynchronously on that stream;
 *   - layouts as csrc/atl_ops.h:3-14: pos (N,2) f32 [x, y], w (N) f32, b (N) int64, img (B,H,W) f32,
 *     all contiguous;
 *   - outputs are caller-allocated; outputs documented as "accumulated" must be zero-filled by the caller
 *     (the reference allocates them with torch::zeros, csrc/atl_cpu.cpp:41,154,229);
 *   - return 0 on success, non-zero on a rejected argument or launch error; atl_last_error() returns the
 *     message (per host thread).
 * Nothing here allocates device memory; scratch buffers are passed in by the caller.
 */
#ifndef ATL_HIP_H_
#define ATL_HIP_H_

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#define ATL_HIP_ABI_VERSION 1

#ifdef __cplusplus
extern "C" {
#endif

const char* atl_last_error(void);
int atl_abi_version(void);

/* ---------------------------------------------------------------- splat / gather (csrc/atl_ops.h:20-29) */

/* splat_bilinear_fwd (csrc/atl_ops.h:20, csrc/atl_cpu.cpp:38-56): img[b,y,x] += w * bilinear(pos).
 * img (B,H,W) accumulated. */
int atl_splat_bilinear_fwd(const float* pos, const float* w, const int64_t* b, int64_t N, int64_t B, int64_t H,
                           int64_t W, float* img, hipStream_t stream);
/* splat_bilinear_bwd (csrc/atl_ops.h:21, csrc/atl_cpu.cpp:58-76): gpos (N,2), gw (N) written. */
int atl_splat_bilinear_bwd(const float* gimg, const float* pos, const float* w, const int64_t* b, int64_t N,
                           int64_t B, int64_t H, int64_t W, float* gpos, float* gw, hipStream_t stream);
/* splat_gauss_fwd (csrc/atl_ops.h:23-24, csrc/atl_cpu.cpp:79-104): truncated Gaussian of radius R around
 * round(pos), normalised by 2 pi sigma^2.  img accumulated. */
int atl_splat_gauss_fwd(const float* pos, const float* w, const int64_t* b, int64_t N, int64_t B, int64_t H,
                        int64_t W, double sigma, int64_t R, float* img, hipStream_t stream);
/* splat_gauss_bwd (csrc/atl_ops.h:25-26, csrc/atl_cpu.cpp:106-131): gpos, gw written. */
int atl_splat_gauss_bwd(const float* gimg, const float* pos, const float* w, const int64_t* b, int64_t N, int64_t B,
                        int64_t H, int64_t W, double sigma, int64_t R, float* gpos, float* gw, hipStream_t stream);
/* gather_bilinear_fwd (csrc/atl_ops.h:28, csrc/atl_cpu.cpp:134-149): out (N) written, zero padding. */
int atl_gather_bilinear_fwd(const float* img, const float* pos, const int64_t* b, int64_t N, int64_t B, int64_t H,
                            int64_t W, float* out, hipStream_t stream);
/* gather_bilinear_bwd (csrc/atl_ops.h:29, csrc/atl_cpu.cpp:151-172): gimg (B,H,W) accumulated, gpos written. */
int atl_gather_bilinear_bwd(const float* gval, const float* img, const float* pos, const int64_t* b, int64_t N,
                            int64_t B, int64_t H, int64_t W, float* gimg, float* gpos, hipStream_t stream);
/* The same splat forward and gather backward with tile-binned LDS accumulation instead of one global atomic
 * per corner (identical corner indices and weights; float sums in another order).  ws: a workspace of
 * atl_tile_ws_bytes(N, B, H, W) bytes (-1: sizes unsupported, use the entry points above). */
int64_t atl_tile_ws_bytes(int64_t N, int64_t B, int64_t H, int64_t W);
int atl_splat_bilinear_fwd_ws(const float* pos, const float* w, const int64_t* b, int64_t N, int64_t B, int64_t H,
                              int64_t W, float* img, void* ws, int64_t ws_bytes, hipStream_t stream);
int atl_gather_bilinear_bwd_ws(const float* gval, const float* img, const float* pos, const int64_t* b, int64_t N,
                               int64_t B, int64_t H, int64_t W, float* gimg, float* gpos, void* ws, int64_t ws_bytes,
                               hipStream_t stream);
/* No counterpart in the reference: the tile-binned splat forward of atl_splat_bilinear_fwd_ws for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It allocates nothing: its workspace is a 64 MiB array held by the library on every GPU it runs on
 * (until the process ends), which fits atl_tile_ws_bytes(N, B, H, W) <= 64 MiB (about 3.6M events at 640x480,
 * B = 1); larger calls fail with status 1 and a message.  img (B,H,W) is accumulated, as by the _ws form.
 * The array's address on each device is resolved by atl_init (call it once after loading the library, before
 * any capture), or else by the first call on that device.  Calls that overlap on one GPU share the array and
 * race. */
int atl_splat_bilinear_fwd_noalloc(const float* pos, const float* w, const int64_t* b, int64_t N, int64_t B,
                                   int64_t H, int64_t W, float* img, hipStream_t stream);
/* Library set-up (no counterpart in the reference): resolves per-device state, the no-allocation entry point's
 * scratch address on every visible device, with that device current; the current device is restored.  Returns 0
 * (also with no device present) or 1 with a message.  The ctypes binding calls it once at load on a GPU host. */
int atl_init(void);
/* The Gaussian splat forward with the same tile engine (tiles of the rounded centres, an LDS window of
 * T + 2R pixels per tile); R <= 8.  ws: atl_splat_gauss_ws_bytes(N, B, H, W, R) bytes (-1: unsupported). */
int64_t atl_splat_gauss_ws_bytes(int64_t N, int64_t B, int64_t H, int64_t W, int64_t R);
int atl_splat_gauss_fwd_ws(const float* pos, const float* w, const int64_t* b, int64_t N, int64_t B, int64_t H,
                           int64_t W, double sigma, int64_t R, float* img, void* ws, int64_t ws_bytes,
                           hipStream_t stream);
/* voxel_grid (csrc/atl_ops.h:49-50, csrc/atl_cpu.cpp:256-286): vox (B,C,H,W) accumulated. */
int atl_voxel_grid(const float* pos, const float* t, const float* p, const int64_t* b, int64_t N, int64_t B,
                   int64_t C, int64_t H, int64_t W, float* vox, hipStream_t stream);
/* The same voxel grid on the tile-binned LDS engine (the C time bins are the channels of each tile's window;
 * identical corner indices and weights, float sums in another order).  ws: atl_voxel_ws_bytes(N, B, C, H, W)
 * bytes (-1: sizes unsupported, use atl_voxel_grid). */
int64_t atl_voxel_ws_bytes(int64_t N, int64_t B, int64_t C, int64_t H, int64_t W);
int atl_voxel_grid_ws(const float* pos, const float* t, const float* p, const int64_t* b, int64_t N, int64_t B,
                      int64_t C, int64_t H, int64_t W, float* vox, void* ws, int64_t ws_bytes, hipStream_t stream);

/* Warp -> splat -> gather in one launch sequence: the composition of DenseLinearFlow.transport
 * (atl/motion/parametric.py:53-56, 212-216, 235-251), make_iwe with a bilinear splat and pooled polarity
 * (atl/objectives/base.py:40-60, csrc/atl_cpu.cpp:38-56) and gather (csrc/atl_cpu.cpp:134-149), which the
 * reference runs as separate ops.  Forward: y = x + v(x) (t_ref - t) with v the border-clamped sample of the flow
 * grid (B,2,Hg,Wg) at pixel x, w = [y inside the sensor] if mask_border else 1, img (B,H,W) = splat(y, w)
 * (written), vals (N) = gather(img, y) (written; may be null).  Backward: ggrid (B,2,Hg,Wg) written with the
 * flow-grid gradient of <gvals, vals> + <gimg, img> (either may be null), from the forward's ws.  ws: atl_warp_splat_gather_ws_bytes bytes (-1: sizes unsupported; 0 for N = 0, whose outputs are zeros). */
int64_t atl_warp_splat_gather_ws_bytes(int64_t N, int64_t B, int64_t H, int64_t W, int64_t Hg, int64_t Wg);
int atl_warp_splat_gather_fwd(const float* grid, int64_t B, int64_t Hg, int64_t Wg, const float* xy, const float* t,
                              const int64_t* b, int64_t N, int64_t H, int64_t W, double t_ref, int64_t mask_border,
                              float* img, float* vals, void* ws, int64_t ws_bytes, hipStream_t stream);
int atl_warp_splat_gather_bwd(const float* img, const float* gvals, const float* gimg, const float* xy,
                              const float* t, const int64_t* b, int64_t N, int64_t B, int64_t H, int64_t W,
                              int64_t Hg, int64_t Wg, double t_ref, float* ggrid, void* ws, int64_t ws_bytes,
                              hipStream_t stream);

/* ---------------------------------------------------------------- flow-grid sampling */

/* DenseLinearFlow.field + sample_grid (atl/motion/parametric.py:212-216, 235-251): out (N,C) written, bilinear
 * border-clamped sample of field (B,C,Hg,Wg).  With img_h, img_w > 0 the positions are image pixels mapped by
 * g = x / max(W-1, 1) * (Wg-1); with img_h = img_w = 0 they are grid coordinates. */
int atl_sample_grid_fwd(const float* field, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                        const int64_t* b, int64_t N, int64_t img_h, int64_t img_w, float* out, hipStream_t stream);
/* Adjoint of atl_sample_grid_fwd w.r.t. the field (the index_put accumulate of parametric.py:247-251 under
 * autograd): gfield (B,C,Hg,Wg) accumulated. */
int atl_sample_grid_bwd(const float* gout, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                        const int64_t* b, int64_t N, int64_t img_h, int64_t img_w, float* gfield,
                        hipStream_t stream);

/* Gradient of atl_sample_grid_fwd w.r.t. the positions (the autograd of parametric.py:235-251 through its
 * weights; zero where the border clamp is active): gpos (N,2) written. */
int atl_sample_grid_bwd_pos(const float* gout, const float* field, int64_t B, int64_t C, int64_t Hg, int64_t Wg,
                            const float* pos, const int64_t* b, int64_t N, int64_t img_h, int64_t img_w, float* gpos,
                            hipStream_t stream);
/* Two-channel fields (flows): atl_flow_interleave copies a (B,2,Hg,Wg) field into out (B,Hg,Wg,2), node by node;
 * atl_sample_flow_il then samples it as atl_sample_grid_fwd samples the planar field with C = 2 (the same bits)
 * from two 16-byte reads per event instead of four 8-byte reads; needs Wg >= 2.  No counterpart in the
 * reference (a layout of its sample_grid, atl/motion/parametric.py:235-251). */
int atl_flow_interleave(const float* field, int64_t B, int64_t Hg, int64_t Wg, float* out, hipStream_t stream);
int atl_sample_flow_il(const float* field_il, int64_t B, int64_t Hg, int64_t Wg, const float* pos, const int64_t* b,
                       int64_t N, int64_t img_h, int64_t img_w, float* out, hipStream_t stream);
/* Many-channel fields (a trajectory coefficient grid: C = 2K channels sampled at every event), no counterpart
 * in the reference's extension: they replace the same sample_grid (atl/motion/parametric.py:235-251) where the
 * plane layout would cost C loads per corner.  atl_field_channels_last writes the channels-last copy
 * field_cl (B, Hg, Wg, 4*ceil(C/4)) float, channels past C zero.  atl_sample_grid_fwd_cl and
 * atl_sample_grid_bwd_pos_cl then return the same bits as atl_sample_grid_fwd and atl_sample_grid_bwd_pos on
 * the plane field.  field_cl 16-byte aligned (out and gout too when C % 4 == 0); N * ceil(C/4) < 2^31 for the
 * forward; C <= 256 for the position gradient. */
int atl_field_channels_last(const float* field, int64_t B, int64_t C, int64_t Hg, int64_t Wg, float* field_cl,
                            hipStream_t stream);
int atl_sample_grid_fwd_cl(const float* field_cl, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                           const int64_t* b, int64_t N, int64_t img_h, int64_t img_w, float* out,
                           hipStream_t stream);
int atl_sample_grid_bwd_pos_cl(const float* gout, const float* field_cl, int64_t B, int64_t C, int64_t Hg,
                               int64_t Wg, const float* pos, const int64_t* b, int64_t N, int64_t img_h,
                               int64_t img_w, float* gpos, hipStream_t stream);
/* PixelTrajectories.displacement (atl/motion/trajectories.py:26-37 basis, the coefficient look-up and the sum
 * over k), fused, no counterpart in the reference's extension: out (N,2) written, d = (sum_k c_{K+k} g_k,
 * sum_k c_k g_k) of the channels-last coefficient grid field_cl (B, Hg, Wg, 4*ceil(C/4), channels
 * [y_1..y_K, x_1..x_K], C = 2K: any other C is rejected) sampled at grid coordinates gpos, with
 * g_k(t) = t^k (basis 0), binom(K,k) t^k (1-t)^(K-k) (basis 1) or N_k(t) (basis 2: the clamped uniform
 * B-spline of degree min(3, K) with K + 1 functions N_0..N_K on [0, 1], N_0 pinned to the start); 1 <= K <= 16.
 * atl_traj_gout writes the (N, 2K) output gradient per channel, gout[n, k-1] = g_k gd.y and
 * gout[n, K+k-1] = g_k gd.x, which atl_sample_grid_bwd_planned (field) and atl_sample_grid_bwd_pos_cl
 * (positions) take. */
int atl_traj_displacement(const float* field_cl, int64_t B, int64_t C, int64_t K, int64_t Hg, int64_t Wg,
                          const float* gpos, const int64_t* b, const float* t, int64_t N, int64_t basis, float* out,
                          hipStream_t stream);
/* PixelTrajectories.origin (atl/motion/trajectories.py:68-73) in one pass: n_fp Picard steps p <- xy - d(p, t) from
 * p = xy, out (N,2) written, bit-identical to n_fp composed atl_traj_displacement calls with the subtraction between
 * them.  P (n_fp, N, 2), may be null, receives the grid coordinates (p - offset) / tile (tile 1: p) of every step's
 * p, where its displacement is taken: the positions of the steps' backward; with final_row != 0, P has n_fp + 1
 * rows and the last receives those of the returned p (where PixelTrajectories.transport's last look-up is). */
int atl_traj_origin(const float* field_cl, int64_t B, int64_t C, int64_t K, int64_t Hg, int64_t Wg, const float* xy,
                    const float* t, const int64_t* b, int64_t N, int64_t n_fp, double offset, int64_t tile,
                    int64_t basis, float* P, int64_t final_row, float* out, hipStream_t stream);
/* The backward of atl_traj_origin's steps for the B-spline basis (K >= 3), in one pass: from gp (N,2), the gradient
 * of the returned p, for k = n_fp - 1 .. 0 the step's displacement gradient gD_k = -g (gD (n_fp, N, 2) written,
 * for atl_grid_plan + atl_traj_field_bwd_planned over all n_fp N records) and g <- the displacement's position
 * derivative at P[k] applied to gD_k, divided by tile (atl_traj_pos_bwd_cl's terms and order).  gxy (N,2), may
 * be null, receives the gradient of xy (sum of every step's g plus the last position derivative). */
int atl_traj_origin_bwd(const float* field_cl, int64_t B, int64_t C, int64_t K, int64_t Hg, int64_t Wg,
                        const float* P, const float* t, const int64_t* b, int64_t N, int64_t n_fp, int64_t tile,
                        const float* gp, float* gD, float* gxy, hipStream_t stream);
/* The exposure correction of atl/objectives/ats.py:31-50 (visible_fraction) for PixelTrajectories in one pass:
 * each anchor's trajectory start (n_fp Picard steps from xa, as PixelTrajectories.origin), its coefficients looked
 * up once there, the trajectory evaluated at the n_check bin centres, and the weighted share of centres inside the
 * sensor (counts (B, n_check), centres (n_check)), out (M) written; bit-identical to the composed
 * atl_traj_displacement calls and atl_visible_fraction's sums.  Grid coordinates of a pixel position p:
 * (p - offset) / tile (tile 1: p).  No counterpart in the reference (its visible_fraction transports the anchors
 * once per centre). */
int atl_traj_visible(const float* field_cl, int64_t B, int64_t C, int64_t K, int64_t Hg, int64_t Wg, const float* xa,
                     const float* ta, const int64_t* ba, int64_t M, int64_t n_fp, double offset, int64_t tile,
                     int64_t basis, const float* counts, const float* centres, int64_t n_check, double tau,
                     int64_t H, int64_t W, float* out, hipStream_t stream);
/* The backward of atl_traj_displacement for the B-spline basis (basis 2) without the (N, 2K) gradient rows of
 * atl_traj_gout: each kernel forms an event's row from the displacement's gradient gd (N,2) and its time t.
 * atl_traj_field_bwd_planned accumulates the coefficient grid's gradient (B, 2K, Hg, Wg; accumulated: zero it
 * first) on the positions' tile plan (atl_grid_plan with img 0, 0), K >= 3; atl_traj_pos_bwd_cl writes the positions'
 * gradient gpos (N,2) as atl_sample_grid_bwd_pos_cl does (the same bits).  No counterpart in the reference (the
 * adjoint of its per-channel lookup under autograd). */
int atl_traj_field_bwd_planned(const float* gd, const float* t, int64_t K, int64_t B, int64_t Hg, int64_t Wg,
                               int64_t N, void* ws, float* gfield, hipStream_t stream);
/* The same coefficient-grid gradient for n_look look-ups of N events in one call, binned here (no plan): look-up
 * r of event e at grid position pos[r N + e] (n_look, N, 2) with displacement gradient gd[r N + e] and time t[e]
 * (t_last[e] for the last look-up when t_last is not null: PixelTrajectories.transport's look-up at the
 * destination time), batch b[e]; gfield (B, 2K, Hg, Wg) accumulated (zero it first), 3 <= K <= 16, 16x16 tiles
 * (at most 16384 over the batch).  Workspace: atl_traj_field_bwd_bytes(K, B, Hg, Wg, N n_look) bytes (-1 if the
 * sizes are unsupported); calls that share a workspace must not overlap.  The products are those of
 * atl_traj_field_bwd_planned; only the order of the float additions differs.  No counterpart in the reference
 * (autograd's adjoint of every look-up of atl/motion/trajectories.py:68-77). */
int64_t atl_traj_field_bwd_bytes(int64_t K, int64_t B, int64_t Hg, int64_t Wg, int64_t n_rec);
int atl_traj_field_bwd(const float* gd, const float* pos, const float* t, const float* t_last, const int64_t* b,
                       int64_t N, int64_t n_look, int64_t K, int64_t B, int64_t Hg, int64_t Wg, void* ws,
                       int64_t ws_bytes, float* gfield, hipStream_t stream);
int atl_traj_pos_bwd_cl(const float* gd, const float* t, int64_t K, const float* field_cl, int64_t B, int64_t Hg,
                        int64_t Wg, const float* gpos_in, const int64_t* b, int64_t N, float* gpos, hipStream_t stream);
int atl_traj_gout(const float* gd, const float* t, int64_t N, int64_t K, int64_t basis, float* gout,
                  hipStream_t stream);
/* The same adjoint through a tile plan: atl_grid_plan bins the positions by the 16x16 tile of their base
 * grid node into a workspace of atl_grid_plan_bytes(B, Hg, Wg, N) bytes (-1 if the sizes are unsupported);
 * atl_sample_grid_bwd_planned then accumulates gout tile by tile in LDS and flushes each tile's touched nodes.
 * gfield accumulated; C <= 32 (C > 4 only where 16x16 tiles fit the binning).  The positions and img_h, img_w
 * must be the ones the plan was built from (the plan keeps its own copy of the positions; `pos` is not read).
 * Each call also writes its list of record chunks into the plan's workspace: one call per plan at a time. */
int64_t atl_grid_plan_bytes(int64_t B, int64_t Hg, int64_t Wg, int64_t N);
int atl_grid_plan(int64_t B, int64_t Hg, int64_t Wg, const float* pos, const int64_t* b, int64_t N, int64_t img_h,
                  int64_t img_w, void* ws, int64_t ws_bytes, hipStream_t stream);
/* The same adjoint for fields of C <= 2 channels with the binning done here, in the backward: the records carry
 * the gradient rows (x, y, gout[j, 0], gout[j, 1]), so the accumulation reads no row by event index (a random
 * 8-byte read that every XCD's L2 fetched separately).  ws: atl_grid_plan_bytes(B, Hg, Wg, N) bytes, no plan
 * needed; gfield accumulated. */
int atl_sample_grid_bwd_binned(const float* gout, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                               const int64_t* b, int64_t N, int64_t img_h, int64_t img_w, float* gfield, void* ws,
                               int64_t ws_bytes, hipStream_t stream);
int atl_sample_grid_bwd_planned(const float* gout, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                                int64_t N, int64_t img_h, int64_t img_w, void* ws, float* gfield,
                                hipStream_t stream);
/* The field adjoint of a many-channel lookup (5 <= C <= 32, 16x16 tiles; gfield accumulated: zero it first),
 * binned here (no plan): the records are sorted by tile, every workgroup sums its tile's records per base node in
 * registers and writes its own nodes without global atomics (border row and column through a halo buffer in ws).
 * ws: atl_sample_grid_bwd_rows_bytes(B, C, Hg, Wg, N) bytes (-1: unsupported).  The same corner products as
 * atl_sample_grid_bwd (the adjoint of atl/motion/parametric.py:235-251), fused into the sums; other order. */
int64_t atl_sample_grid_bwd_rows_bytes(int64_t B, int64_t C, int64_t Hg, int64_t Wg, int64_t N);
int atl_sample_grid_bwd_rows(const float* gout, int64_t B, int64_t C, int64_t Hg, int64_t Wg, const float* pos,
                             const int64_t* b, int64_t N, int64_t img_h, int64_t img_w, float* gfield, void* ws,
                             int64_t ws_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- event noise */

/* Per-image mean and unbiased variance of B images of n pixels each (the IWE contrast of
 * atl/objectives/cmax.py:23-25, iwe.var(dim=(-2, -1))): mean (B) and var (B) written, var = NaN for n = 1.  Sums in
 * fp64 over fixed chunks of pixels, added in a fixed order.  ws: atl_image_variance_ws_bytes(B, n) bytes (-1: bad
 * sizes).  The backward writes gimg (B, n) = gvar[b] * 2 (img - mean[b]) / (n - 1), torch.var's gradient. */
int64_t atl_image_variance_ws_bytes(int64_t B, int64_t n);
int atl_image_variance(const float* img, int64_t B, int64_t n, float* mean, float* var, void* ws, int64_t ws_bytes,
                       hipStream_t stream);
int atl_image_variance_bwd(const float* img, const float* mean, const float* gvar, int64_t B, int64_t n, float* gimg,
                           hipStream_t stream);

/* Dequantisation and smoothing noise of AnchoredExact (atl/objectives/ats.py:79-84, where torch.rand - 0.5 and
 * h * torch.randn are drawn on a CPU generator and added): xs (N,2) = xy + U(-1/2, 1/2) per coordinate when
 * dequantize != 0 (else a copy of xy); xa (N,2) = xs + h N(0, 1) per coordinate when xa is not null.  Philox4x32-10
 * keyed by seed, counter (event index, offset): the same (seed, offset) gives the same draws, a new offset new
 * ones.  Not the reference's random numbers (those come from torch's CPU generator). */
int atl_event_noise(const float* xy, int64_t N, uint64_t seed, uint64_t offset, double h, int dequantize, float* xs,
                    float* xa, hipStream_t stream);

/* ---------------------------------------------------------------- pair plan (atl/ops/functional.py:132-178) */

/* Reductions behind the plan geometry (functional.py:139,144-145): stats (5 ints, ordered-int encoding of
 * floats: i >= 0 ? bits = i : bits = i ^ 0x7fffffff) = [max ||v|| as sqrt(fma(vy,vy,vx*vx)), min xa.x,
 * min xa.y, min -xa.x, min -xa.y]. */
int atl_plan_stats(const float* v, int64_t N, const float* xa, int64_t M, int* stats, hipStream_t stream);
/* Per-cell entry counts of the (source, slice) pairs, functional.py:150-167: counts (B*S*GH*GW) int32
 * accumulated.  ox, oy, cell, tau are the host doubles of functional.py:139-149 (rounded to fp32 inside). */
int atl_plan_count(const float* x, const float* t, const float* v, const int64_t* b, int64_t N, int64_t B,
                   double ox, double oy, double cell, double tau, int64_t S, int64_t GH, int64_t GW, int* counts,
                   hipStream_t stream);
/* start (n+1) int64 = [0, cumsum(counts)] (functional.py:168); work holds atl_scan_work_size(n) int64. */
int atl_scan_counts(const int* counts, int64_t n, int64_t* start, int64_t* work, hipStream_t stream);
int64_t atl_scan_work_size(int64_t n);
int atl_fill_i32(int* p, int64_t n, int value, hipStream_t stream);
/* Scatter of the plan entries into CSR order (functional.py:163-165, 176): cursor (ncell) zero-filled.
 * Entry order inside one cell is unspecified, as with the reference's torch.argsort. */
int atl_plan_fill(const float* x, const float* t, const float* v, const int64_t* b, int64_t N, int64_t B,
                  double ox, double oy, double cell, double tau, int64_t S, int64_t GH, int64_t GW,
                  const int64_t* start, int* cursor, float* src_y, float* src_v, float* src_t, int64_t* src_id,
                  hipStream_t stream);
/* The plan's entries and CSR offsets (functional.py:149-168) in one call, by a two-level counting sort (no
 * per-entry global atomics): start (ncell+1) int64 and the entries src_y (,2), src_v (,2), src_t, src_id written at
 * [0, E), E = start[ncell]; the entry arrays hold ecap >= N * (floor((2 tau + 1/S) S) + 2, at most S) entries.
 * The same keys, slice positions and offsets as atl_plan_count + atl_scan_counts + atl_plan_fill; entry order
 * inside one cell unspecified.  ws: atl_plan_sort_bytes(N, ecap, ncell) bytes (-1: unsupported sizes). */
int64_t atl_plan_sort_bytes(int64_t N, int64_t ecap, int64_t ncell);
int atl_plan_sort(const float* x, const float* t, const float* v, const int64_t* b, int64_t N, int64_t B, double ox,
                  double oy, double cell, double tau, int64_t S, int64_t GH, int64_t GW, int64_t ecap,
                  int64_t* start, float* src_y, float* src_v, float* src_t, int64_t* src_id, void* ws,
                  int64_t ws_bytes, hipStream_t stream);
/* Anchor fields of the plan (functional.py:169-177): anc_x (M,2), anc_t (M), anc_cell (M,3), anc_id (M).
 * anchor_xy may be null (positions x[anchors]). */
int atl_plan_anchors(const float* x, const float* t, const int64_t* b, const int64_t* anchors,
                     const float* anchor_xy, int64_t M, int64_t N, double ox, double oy, double cell, int64_t S,
                     int64_t GH, int64_t GW, float* anc_x, float* anc_t, int64_t* anc_cell, int64_t* anc_id,
                     hipStream_t stream);

/* ---------------------------------------------------------------- pair sums over a reference-layout plan */

/* ats_pair_fwd (csrc/atl_ops.h:31-42, csrc/atl_cpu.cpp:203-222): out (M) written.  E = number of plan
 * entries, ncell = B*S*GH*GW (cell_start has ncell+1 entries).  count (M) int32 receives n_i, the number of
 * visited pairs of each anchor, when non-null (not output by the reference).  Sixteen lanes per anchor read
 * the anchor's three CSR row ranges coalesced, in the plan's anchor order.  E, M, N < 2^29, ncell < 2^31. */
int atl_ats_pair_fwd(const float* src_y, const float* src_v, const float* src_t, const int64_t* src_id,
                     const int64_t* cell_start, int64_t E, int64_t ncell, const float* anc_x, const float* anc_t,
                     const int64_t* anc_cell, const int64_t* anc_id, int64_t M, const float* slice_c, int64_t S,
                     int64_t GH, int64_t GW, double h, double tau, double cut, float* out, int* count,
                     hipStream_t stream);
/* ats_pair_bwd (csrc/atl_ops.h:43-47, csrc/atl_cpu.cpp:224-253): gv (N,2) accumulated, with the reference's
 * two global atomics per pair (csrc/atl_cuda.cu:169-180); for a caller that cannot pass a workspace.
 * E, M, N < 2^29. */
int atl_ats_pair_bwd(const float* gS, const float* src_y, const float* src_v, const float* src_t,
                     const int64_t* src_id, const int64_t* cell_start, int64_t E, int64_t ncell, const float* anc_x,
                     const float* anc_t, const int64_t* anc_cell, const int64_t* anc_id, int64_t M,
                     const float* slice_c, int64_t S, int64_t GH, int64_t GW, double h, double tau, double cut,
                     int64_t N, float* gv, hipStream_t stream);
/* Workspace entries of the same two ops (csrc/atl_ops.h:31-47), for a binding that allocates a workspace
 * with its outputs: ws is atl_ats_pair_ws_bytes(E, ncell, M, GW) bytes of device memory, 256-byte aligned,
 * contents on entry ignored, and serves either call.  Both bin the anchors by cell first.
 * atl_ats_pair_fwd_ws: the same out and count as atl_ats_pair_fwd, one wave per item of up to five anchors of
 * one cell, which walks the cell's 3 x 3 neighbourhood once for all of them.  atl_ats_pair_bwd_ws, source-centric: each chunk of 64 plan entries
 * of a run of six cells of a row gathers over the binned anchors (gS != 0) around it and adds every entry's
 * sum to gv once (two atomics per entry instead of two per pair); the same visited pairs and terms as
 * atl_ats_pair_bwd, gv (N,2) accumulated.  A workspace of atl_ats_pair_bwd_ws_bytes(E, ncell, M, GW, N, S)
 * bytes (the same regions, then N * S float2) lets the backward write each entry's sum to its own
 * (source, slice) slot instead, a plan holding one entry per source and slice, and add every source's slots in
 * slice order: no atomics.  Either size serves either call; -1 for unsupported sizes (S > 4096). */
int64_t atl_ats_pair_ws_bytes(int64_t E, int64_t ncell, int64_t M, int64_t GW);
int64_t atl_ats_pair_bwd_ws_bytes(int64_t E, int64_t ncell, int64_t M, int64_t GW, int64_t N, int64_t S);
int atl_ats_pair_fwd_ws(const float* src_y, const float* src_v, const float* src_t, const int64_t* src_id,
                        const int64_t* cell_start, int64_t E, int64_t ncell, const float* anc_x, const float* anc_t,
                        const int64_t* anc_cell, const int64_t* anc_id, int64_t M, const float* slice_c, int64_t S,
                        int64_t GH, int64_t GW, double h, double tau, double cut, float* out, int* count, void* ws,
                        int64_t ws_bytes, hipStream_t stream);
int atl_ats_pair_bwd_ws(const float* gS, const float* src_y, const float* src_v, const float* src_t,
                        const int64_t* src_id, const int64_t* cell_start, int64_t E, int64_t ncell,
                        const float* anc_x, const float* anc_t, const int64_t* anc_cell, const int64_t* anc_id,
                        int64_t M, const float* slice_c, int64_t S, int64_t GH, int64_t GW, double h, double tau,
                        double cut, int64_t N, float* gv, void* ws, int64_t ws_bytes, hipStream_t stream);
/* atl_ats_pair_bwd_ws over the anchors binned by the atl_ats_pair_fwd_ws call that ran in this ws on the same plan
 * and anchors (ws untouched since): the binning is not repeated, every binned anchor takes its gS (anchors of
 * gS = 0 included, adding zero terms as the reference's loop does).  No counterpart in the reference, whose
 * forward and backward are separate calls (csrc/atl_ops.h:31-47). */
int atl_ats_pair_bwd_ws_binned(const float* gS, const float* src_y, const float* src_v, const float* src_t,
                               const int64_t* src_id, const int64_t* cell_start, int64_t E, int64_t ncell,
                               const float* anc_x, const float* anc_t, const int64_t* anc_cell,
                               const int64_t* anc_id, int64_t M, const float* slice_c, int64_t S, int64_t GH,
                               int64_t GW, double h, double tau, double cut, int64_t N, float* gv, void* ws,
                               int64_t ws_bytes, hipStream_t stream);

/* ---------------------------------------------------------------- fused pair sums (no host synchronisation)
 *
 * The same S_i and dS/dv as atl_ats_pair_fwd/bwd over the reference plan (functional.py:181-207:
 * build_pair_plan + ats_pair_fwd / ats_pair_bwd), built and evaluated without a host round trip:
 * the reference's (source, slice) entries and the anchors are binned into a fixed fine-cell grid clamped
 * around the sensor, the forward gathers per anchor and the backward gathers per entry (no per-pair
 * atomics).  The contributing pairs, and so every per-anchor neighbour count, are the reference's.
 *
 * Usage: atl_fast_geometry_init (host only, fills the struct, including ws_bytes) -> allocate ws_bytes
 * of device memory -> atl_fast_plan -> atl_fast_pair_fwd -> atl_fast_pair_bwd (any number of times while
 * the workspace is kept).  Inputs: x (N,2) raw source positions, t (N), v (N,2) velocities, b (N) int64;
 * anchors (M) int64 event indices, anchor_xy (M,2) anchor positions or null (x[anchors]). */
typedef struct atl_fast_geometry {
  int32_t version;                      /* ATL_HIP_ABI_VERSION once initialised */
  int32_t bucket_shift;                 /* log2 of the cell keys per sort bucket */
  int64_t N, M, B, H, W, S;
  double h, tau, cut;
  float gx0, gy0, gx1, gy1, cell;       /* clamp box and fine cell size (pixels) */
  float reserved_f;
  int64_t GW, GH, ncell, ncell_pad, max_span, ecap;
  int64_t ws_bytes;                     /* workspace layout (byte offsets) */
  int64_t off_params, off_cnt, off_boff, off_part, off_start, off_trec, off_epos, off_etim, off_eself, off_arec,
      off_srec, off_brec, off_self;
} atl_fast_geometry;

int atl_fast_geometry_init(int64_t N, int64_t M, int64_t B, int64_t H, int64_t W, int64_t S, double h, double tau,
                           double cut, atl_fast_geometry* geo);
/* Plan: entries and anchors binned and sorted by (batch, slice, cell) in ws.  anchors may be null when M == N:
 * every event is then its own anchor, in event order (the reference's anchors = arange(N)). */
int atl_fast_plan(const atl_fast_geometry* geo, const float* x, const float* t, const float* v, const int64_t* b,
                  const int64_t* anchors, const float* anchor_xy, void* ws, int64_t ws_bytes, hipStream_t stream);
/* out (M) written for every valid anchor (zero-fill it first); count (M) int32 receives n_i when non-null. */
int atl_fast_pair_fwd(const atl_fast_geometry* geo, const void* ws, float* out, int* count, hipStream_t stream);
/* gv (N,2) written: each source's gradient, zero for sources outside the plan (no fill needed). */
int atl_fast_pair_bwd(const atl_fast_geometry* geo, void* ws, const float* gS, float* gv, hipStream_t stream);
/* The same backward when the velocities were DenseLinearFlow.field(x) (atl/motion/parametric.py:212-216,
 * 235-251): the gradient goes to the flow grid (B,2,Hg,Wg), written to ggrid (no fill needed), as
 * atl_fast_pair_bwd followed by sample_grid's adjoint at x would give it (float sums in another order), with no
 * per-event gradient array.  img_h, img_w: the pixel -> grid scaling of atl_sample_grid_fwd (0, 0: x are grid
 * coordinates).  The plan's temporary sort records (dead after the plan) hold the per-source gradients. */
int atl_fast_pair_bwd_flow(const atl_fast_geometry* geo, void* ws, const float* gS, int64_t Hg, int64_t Wg,
                           int64_t img_h, int64_t img_w, float* ggrid, hipStream_t stream);
/* atl_fast_pair_bwd_flow in its two steps: the pair backward (the source gradients, kept in ws), then the
 * adjoint into ggrid.  Run them in this order on one stream, with nothing in between that rebuilds the plan. */
int atl_fast_pair_bwd_src(const atl_fast_geometry* geo, void* ws, const float* gS, hipStream_t stream);
int atl_fast_flow_adjoint(const atl_fast_geometry* geo, void* ws, int64_t Hg, int64_t Wg, int64_t img_h,
                          int64_t img_w, float* ggrid, hipStream_t stream);

/* The same fused pair sums for trajectory motion (the anchored score with PixelTrajectories, which the
 * reference's exact kernel does not take: atl/objectives/ats.py:77-78 requires motion linear at the event).
 * No counterpart in the reference's extension; it replaces atl_fast_plan / atl_fast_pair_bwd where each
 * source's slice-centre position and velocity come from its trajectory instead of x + v (c_s - t):
 * source j has the trajectory start p[j] (N,2) and coefficients coef[j] (N, 2K, channels [y_1..y_K,
 * x_1..x_K]); tab (S, 2K) holds the basis at the slice centres, row s = [g_1..g_K(c_s), g_1'..g_K'(c_s)].
 * Entry (j, s): y = p + sum_k coef_k g_k(c_s), v = sum_k coef_k g_k'(c_s) (fp32, sums in k order); the pairs,
 * tests and sums are then those of atl_fast_pair_fwd, which evaluates the forward unchanged.
 * atl_fast_pair_bwd_traj writes, for every source, gp (N,2) = dL/dp and gcoef (N, 2K) = dL/dcoef (zero for
 * sources outside the plan).  1 <= K <= 12. */
int atl_fast_plan_traj(const atl_fast_geometry* geo, const float* p, const float* coef, int64_t K, const float* tab,
                       const float* t, const int64_t* b, const int64_t* anchors, const float* anchor_xy, void* ws,
                       int64_t ws_bytes, hipStream_t stream);
int atl_fast_pair_bwd_traj(const atl_fast_geometry* geo, void* ws, const float* gS, const float* coef, int64_t K,
                           const float* tab, float* gp, float* gcoef, hipStream_t stream);

/* ---------------------------------------------------------------- anchored-score pieces */

/* window_counts (atl/ops/functional.py:210-217): out (M) written.  Requires keys b*4 + t ascending in event
 * order (the EventPacket invariant, atl/core/events.py:11-12); atl_check_sorted tests it (flag = 1 if not).
 * idx may be null (M <= N): the first M events, in order. */
int atl_window_counts(const float* t, const int64_t* b, int64_t N, const int64_t* idx, int64_t M, double tau,
                      float* out, hipStream_t stream);
int atl_check_sorted(const float* t, const int64_t* b, int64_t N, int* flag, hipStream_t stream);
/* Per-batch event counts in n_check time bins (atl/objectives/ats.py:39-41): counts (B, n_check) f32
 * accumulated. */
int atl_bin_counts(const float* t, const int64_t* b, int64_t N, int64_t B, int64_t n_check, float* counts,
                   hipStream_t stream);
/* The same counts for events sorted by (b, t) (the EventPacket order): counts (B, n_check) written (no fill
 * needed), by binary searches for the bin edges of every batch instead of a pass with atomics. */
int atl_bin_counts_sorted(const float* t, const int64_t* b, int64_t N, int64_t B, int64_t n_check, float* counts,
                          hipStream_t stream);
/* visible_fraction for linear motion (atl/objectives/ats.py:31-50): anchors xa (M,2) with velocities va (M,2)
 * transported to the bin centres (n_check floats), out (M) written. */
int atl_visible_fraction(const float* xa, const float* va, const float* ta, const int64_t* ba, int64_t M,
                         const float* counts, const float* centres, int64_t B, int64_t n_check, double tau,
                         int64_t H, int64_t W, float* out, hipStream_t stream);
/* Log-score epilogue (atl/objectives/ats.py:92-96): ls = log(eps + S / D), D = max(wc,1) * vis * 2 pi h^2
 * (vis may be null); q = eps + S/D and D are saved for atl_anchored_epilogue_bwd: gS = (g / q) / D. */
int atl_anchored_epilogue_fwd(const float* S, const float* wc, const float* vis, int64_t M, double h,
                              double eps, float* ls, float* q, float* D, hipStream_t stream);
int atl_anchored_epilogue_bwd(const float* g, const float* q, const float* D, int64_t M, float* gS,
                              hipStream_t stream);
/* The epilogue fused with the loss of atl/objectives/ats.py:102-105: out[0] = -mean_i ls_i (the loss),
 * out[1] = mean_i ls_i (the score), q and D saved as above; the mean is summed in double in a fixed order
 * (deterministic, two launches).  scratch: atl_anchored_score_mean_scratch_bytes() bytes of device memory for the
 * per-block partial sums (no initial contents needed).  The backward takes the loss
 * gradient g (1 float on the device): gS = (((-g) / M) / q) / D, the chain of the negation, the mean and the
 * epilogue. */
int64_t atl_anchored_score_mean_scratch_bytes(void);
int atl_anchored_score_mean_fwd(const float* S, const float* wc, const float* vis, int64_t M, double h, double eps,
                                float* q, float* D, void* scratch, float* out, hipStream_t stream);
int atl_anchored_score_mean_bwd(const float* g, const float* q, const float* D, int64_t M, float* gS,
                                hipStream_t stream);

/* ---------------------------------------------------------------- MotionPriorCMax look-up table
 * knn_indices (atl/objectives/mpcm.py:30-42): for every plane p < P and query q < Q, the k nearest of the plane's n
 * points (points (P, n, 2), queries (Q, 2) shared by the planes); idx (P, Q, k) int64 written, in the order
 * (squared distance (qx - px)^2 + (qy - py)^2 with each fp32 operation rounded, then lower index).  1 <= k <=
 * min(n, 32).  Points with a non-finite distance are never selected (a slot without a point holds -1).  The
 * reference's dense cdist + topk is replaced by a grid-binned ring search.  ws: atl_knn_ws_bytes(P, n) bytes (-1:
 * too many cells for 32-bit indices). */
int64_t atl_knn_ws_bytes(int64_t P, int64_t n);
int atl_knn_indices(const float* queries, int64_t Q, const float* points, int64_t P, int64_t n, int64_t k,
                    int64_t* idx, void* ws, int64_t ws_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ATL_HIP_H_ */
