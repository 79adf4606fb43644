"""Differentiable event-transport ops on MI355X HIP kernels (same API as atl/ops/functional.py).

* :func:`splat`          events -> image (bilinear vote or truncated Gaussian); grads to positions and weights
* :func:`gather`         bilinear sample of an image at event positions; grads to image and positions
* :func:`ats_pair_sums`  exact anchored leave-one-out Gaussian sums for per-event velocities; grad to v
* :func:`build_pair_plan`, :class:`PairPlan`  the spatial hash behind the pair sums (built on the device)
* :func:`window_counts`  per-anchor number of same-batch events within +-tau
* :func:`voxel_grid`     trilinear polarity voting (no grad)
* :func:`sample_grid`    bilinear border-clamped lookup in a (B, C, Hg, Wg) field; grad to the field

Device tensors run on the HIP library (libatl_hip.so) through the C-ABI; CPU tensors use the pure-torch
semantics of :mod:`x_amd.ops.reference`, as the reference does without its extension.
"""
from __future__ import annotations

import contextlib
import ctypes
import math
import threading
from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch

from . import reference as ref
from ._ext import F32, I64, FastGeometry, HipLibraryError, call, ext_supports, get_ext, load_library, ptr, stream_of


def _f32(t):
    return t.contiguous().float()


# ------------------------------------------------------------------------------------------- splat
class _SplatBilinear(torch.autograd.Function):
    """atl/ops/functional.py:24-35."""

    @staticmethod
    def forward(ctx, pos, w, b, B, H, W):
        pos, w, b = _f32(pos), _f32(w), b.contiguous().long()
        ctx.save_for_backward(pos, w, b)
        return get_ext().splat_bilinear_fwd(pos, w, b, B, H, W)

    @staticmethod
    def backward(ctx, g):
        pos, w, b = ctx.saved_tensors
        gp, gw = get_ext().splat_bilinear_bwd(g.contiguous().float(), pos, w, b)
        return gp, gw, None, None, None, None


class _SplatGauss(torch.autograd.Function):
    """atl/ops/functional.py:38-50."""

    @staticmethod
    def forward(ctx, pos, w, b, B, H, W, sigma, radius):
        pos, w, b = _f32(pos), _f32(w), b.contiguous().long()
        ctx.save_for_backward(pos, w, b)
        ctx.sigma, ctx.radius = sigma, radius
        return get_ext().splat_gauss_fwd(pos, w, b, B, H, W, sigma, radius)

    @staticmethod
    def backward(ctx, g):
        pos, w, b = ctx.saved_tensors
        gp, gw = get_ext().splat_gauss_bwd(g.contiguous().float(), pos, w, b, ctx.sigma, ctx.radius)
        return gp, gw, None, None, None, None, None, None


def splat(pos: torch.Tensor, w: torch.Tensor, b: torch.Tensor, B: int, H: int, W: int,
          kernel: str = "bilinear", sigma: float = 1.0, radius: int | None = None) -> torch.Tensor:
    """Accumulate weighted events into a (B, H, W) image (atl/ops/functional.py:53-65)."""
    if kernel == "bilinear":
        if ext_supports(pos):
            return _SplatBilinear.apply(pos, w, b, B, H, W)
        return ref.splat_bilinear(pos, w, b, B, H, W)
    if kernel == "gauss":
        radius = int(math.ceil(3 * sigma)) if radius is None else radius
        if ext_supports(pos):
            return _SplatGauss.apply(pos, w, b, B, H, W, float(sigma), int(radius))
        return ref.splat_gauss(pos, w, b, B, H, W, sigma, radius)
    raise ValueError(kernel)


# ------------------------------------------------------------------------------------------- gather
class _Gather(torch.autograd.Function):
    """atl/ops/functional.py:69-80."""

    @staticmethod
    def forward(ctx, img, pos, b):
        img, pos, b = _f32(img), _f32(pos), b.contiguous().long()
        ctx.save_for_backward(img, pos, b)
        return get_ext().gather_bilinear_fwd(img, pos, b)

    @staticmethod
    def backward(ctx, g):
        img, pos, b = ctx.saved_tensors
        gi, gp = get_ext().gather_bilinear_bwd(g.contiguous().float(), img, pos, b)
        return gi, gp, None


def gather(img: torch.Tensor, pos: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Bilinear sample of a (B, H, W) image at event positions (zero outside); differentiable in both."""
    if ext_supports(pos):
        return _Gather.apply(img, pos, b)
    return ref.gather_bilinear(img, pos, b)


# ------------------------------------------------------------------------------------------- blur
def gaussian_kernel1d(sigma: float, device, dtype=torch.float32):
    """Normalised Gaussian taps exp(-x^2 / 2 sigma^2) at x = -r..r, r = max(ceil(3 sigma), 1)
    (atl/ops/functional.py:91-96)."""
    r = max(int(math.ceil(3 * sigma)), 1)
    x = torch.linspace(-r, r, 2 * r + 1, device=device, dtype=dtype)
    taps = torch.exp(-(x * x) / (2 * sigma * sigma))
    return taps / taps.sum()


def blur(img: torch.Tensor, sigma: float) -> torch.Tensor:
    """Separable Gaussian blur of a (B, H, W) or (B, C, H, W) image with zero padding (atl/ops/functional.py:
    99-110): one 1-D pass along the rows, one along the columns, each a conv1d over every image line."""
    if sigma <= 0:
        return img
    taps = gaussian_kernel1d(sigma, img.device, img.dtype).view(1, 1, -1)
    r = (taps.shape[-1] - 1) // 2
    H, W = img.shape[-2:]
    lead = img.shape[:-2]
    along_w = torch.nn.functional.conv1d(img.reshape(-1, 1, W), taps, padding=r).view(*lead, H, W)
    cols = along_w.transpose(-1, -2).reshape(-1, 1, H)
    along_h = torch.nn.functional.conv1d(cols, taps, padding=r).view(*lead, W, H)
    return along_h.transpose(-1, -2).contiguous()


# ------------------------------------------------------------------------------------------- flow grid
def _tile_plan_ok(B, C, Hg, Wg):
    """The tile adjoint takes C <= 4 channels, or up to 32 where 16x16 tiles fit its 16384-bin binning."""
    return C <= 4 or (C <= 32 and B * ((Wg + 16) // 16) * ((Hg + 16) // 16) <= 16384)


class _LayoutScope(threading.local):
    copies: Optional[list] = None         # [(field, its version, layout, stream, the copy)] while a scope is open


_SCOPE = _LayoutScope()


@contextlib.contextmanager
def layout_scope():
    """Reuse layout copies of a field within one evaluation.  The device samplers read a field from a layout copy
    (channels-last for wide coefficient grids, node-interleaved for two-channel flows).  Inside this scope the copy
    made by a field's first look-up serves its later look-ups on the same stream (the trajectory model samples its
    coefficient grid at every fixed-point step, and a flow is sampled at the sources and at the anchors), as long
    as the field's storage, shape and in-place version are unchanged.  Outside any scope every look-up makes its own
    copy.  The objectives open a scope around one evaluation; a caller may open one around a whole step.  Within a
    scope, writes that leave the version counter unchanged (through ``.data``, or raw device pointers) are not
    seen: do not update a field that way inside a scope.  Scopes nest (the outermost one holds the copies) and
    are per thread; the copies are released when the outermost scope ends, or when the autograd graph that saved
    them for its backward is freed."""
    if _SCOPE.copies is not None:
        yield
        return
    _SCOPE.copies = []
    try:
        yield
    finally:
        _SCOPE.copies = None


def _cached_copy(fld: torch.Tensor, layout: str, make) -> torch.Tensor:
    """A layout copy of ``fld``: the open scope's copy of the same field (storage, shape, stride, dtype, version
    and stream alike), else a new one, recorded in the scope if one is open."""
    copies = _SCOPE.copies
    if copies is None:
        return make()
    ver, st = fld._version, torch.cuda.current_stream(fld.device).cuda_stream
    for src, v, lay, s, cp in copies:
        if (lay == layout and v == ver and s == st and src.data_ptr() == fld.data_ptr() and src.shape == fld.shape
                and src.stride() == fld.stride() and src.dtype == fld.dtype and src._version == ver):
            return cp
    cp = make()
    copies.append((fld, ver, layout, st, cp))
    return cp


def _channels_last(fld: torch.Tensor) -> torch.Tensor:
    """(B, Hg, Wg, 4 ceil(C / 4)) channels-last copy of a (B, C, Hg, Wg) field (reused within a layout_scope)."""
    def make():
        B, C, Hg, Wg = fld.shape
        fcl = torch.empty(B, Hg, Wg, 4 * ((C + 3) // 4), device=fld.device, dtype=F32)
        with torch.cuda.device(fld.device):
            call("atl_field_channels_last", ptr(fld), B, C, Hg, Wg, ptr(fcl), stream_of(fld))
        return fcl
    return _cached_copy(fld, "cl", make)


def _interleaved(fld: torch.Tensor) -> torch.Tensor:
    """(B, Hg, Wg, 2) node-interleaved copy of a (B, 2, Hg, Wg) flow (reused within a layout_scope)."""
    def make():
        B, _, Hg, Wg = fld.shape
        fil = torch.empty(B, Hg, Wg, 2, device=fld.device, dtype=F32)
        with torch.cuda.device(fld.device):
            call("atl_flow_interleave", ptr(fld), B, Hg, Wg, ptr(fil), stream_of(fld))
        return fil
    return _cached_copy(fld, "il", make)


class _SampleGrid(torch.autograd.Function):
    """Bilinear border-clamped lookup of a (B, C, Hg, Wg) field (atl/motion/parametric.py:235-251).

    The field's gradient accumulates tile by tile in LDS instead of scattered atomic adds.  Fields of one or two
    channels (flows) bin the positions together with their gradient rows in the backward, so the accumulation
    reads no row by event index; wider fields bin the positions in the forward (a device plan) and gather their
    rows in the backward.  The positions' gradient (through the interpolation weights) is a per-event gather.
    Fields of CL_MIN_CHANNELS channels or more are sampled from a channels-last copy (same bits, a node's channels
    in one run), two-channel fields (flows) from a node-interleaved copy (same bits, a grid row's two corners in
    one 16-byte read)."""

    CL_MIN_CHANNELS = 4

    @staticmethod
    def forward(ctx, fld, pos, b, img_h, img_w, plan):
        fld_in = fld if fld.dtype == F32 and fld.is_contiguous() else _f32(fld)
        fld, pos, b = fld_in, _f32(pos), b.contiguous().long()
        B, C, Hg, Wg = fld.shape
        N = pos.shape[0]
        out = torch.empty(N, C, device=pos.device, dtype=F32)
        ctx.plan = None
        Q = (C + 3) // 4
        cl = _SampleGrid.CL_MIN_CHANNELS <= C <= 256 and N * Q < 2 ** 31 - 1024
        with torch.cuda.device(pos.device):
            st = stream_of(pos)
            if cl:
                fcl = _channels_last(fld_in)
                call("atl_sample_grid_fwd_cl", ptr(fcl), B, C, Hg, Wg, ptr(pos), ptr(b), N, int(img_h), int(img_w),
                     ptr(out), st)
                fld = fcl                          # the backward's position gradient reads the same copy
            elif C == 2 and Wg >= 2:               # a flow: two 16-byte reads per lookup (the backward: planar)
                call("atl_sample_flow_il", ptr(_interleaved(fld_in)), B, Hg, Wg, ptr(pos), ptr(b), N, int(img_h),
                     int(img_w), ptr(out), st)
            else:
                call("atl_sample_grid_fwd", ptr(fld), B, C, Hg, Wg, ptr(pos), ptr(b), N, int(img_h), int(img_w),
                     ptr(out), st)
            ctx.cl = cl
            ctx.binned = bool(plan) and C <= 2 and int(load_library().atl_grid_plan_bytes(B, Hg, Wg, N)) >= 0
            # many channels: binned in the backward (records sorted by tile, per-node sums, halo flush)
            ctx.rows = bool(plan) and C > 4 and int(load_library().atl_sample_grid_bwd_rows_bytes(B, C, Hg, Wg, N)) >= 0
            if plan and not ctx.binned and not ctx.rows and _tile_plan_ok(B, C, Hg, Wg):
                nbytes = int(load_library().atl_grid_plan_bytes(B, Hg, Wg, N))
                if nbytes >= 0:
                    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=pos.device)
                    call("atl_grid_plan", B, Hg, Wg, ptr(pos), ptr(b), N, int(img_h), int(img_w), ptr(ws), nbytes, st)
                    ctx.plan = ws
        ctx.save_for_backward(pos, b, fld)
        ctx.shape, ctx.img = (B, C, Hg, Wg), (int(img_h), int(img_w))
        return out

    @staticmethod
    def backward(ctx, g):
        pos, b, fld = ctx.saved_tensors
        B, C, Hg, Wg = ctx.shape
        g = g.contiguous().float()
        gf = gp = None
        with torch.cuda.device(pos.device):
            if ctx.needs_input_grad[0]:
                gf = torch.zeros(B, C, Hg, Wg, device=pos.device, dtype=F32)
                if ctx.rows:
                    N = pos.shape[0]
                    nbytes = int(load_library().atl_sample_grid_bwd_rows_bytes(B, C, Hg, Wg, N))
                    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=pos.device)
                    call("atl_sample_grid_bwd_rows", ptr(g), B, C, Hg, Wg, ptr(pos), ptr(b), N, ctx.img[0],
                         ctx.img[1], ptr(gf), ptr(ws), nbytes, stream_of(pos))
                elif ctx.binned:
                    N = pos.shape[0]
                    nbytes = int(load_library().atl_grid_plan_bytes(B, Hg, Wg, N))
                    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=pos.device)
                    call("atl_sample_grid_bwd_binned", ptr(g), B, C, Hg, Wg, ptr(pos), ptr(b), N, ctx.img[0],
                         ctx.img[1], ptr(gf), ptr(ws), nbytes, stream_of(pos))
                elif ctx.plan is not None:
                    call("atl_sample_grid_bwd_planned", ptr(g), B, C, Hg, Wg, ptr(pos), pos.shape[0], ctx.img[0],
                         ctx.img[1], ptr(ctx.plan), ptr(gf), stream_of(pos))
                else:
                    call("atl_sample_grid_bwd", ptr(g), B, C, Hg, Wg, ptr(pos), ptr(b), pos.shape[0], ctx.img[0],
                         ctx.img[1], ptr(gf), stream_of(pos))
            if ctx.needs_input_grad[1]:
                gp = torch.empty_like(pos)
                call("atl_sample_grid_bwd_pos_cl" if ctx.cl else "atl_sample_grid_bwd_pos", ptr(g), ptr(fld), B, C,
                     Hg, Wg, ptr(pos), ptr(b), pos.shape[0], ctx.img[0], ctx.img[1], ptr(gp), stream_of(pos))
        return gf, gp, None, None, None, None


class _WarpSplatGather(torch.autograd.Function):
    """DenseLinearFlow warp -> bilinear splat -> gather in one launch sequence (the composition of
    atl/motion/parametric.py:53-56, atl/objectives/base.py:40-60 and atl/ops/functional.py:67-87): returns the
    image of warped events and its values at the warped events; the backward gives the flow grid's gradient.
    The forward's workspace (warped positions, weights, the binned records) is kept for the backward."""

    @staticmethod
    def forward(ctx, grid, xy, t, b, t_ref, H, W, mask_border):
        grid, xy, t, b = _f32(grid), _f32(xy), _f32(t), b.contiguous().long()
        B, _, Hg, Wg = grid.shape
        N = xy.shape[0]
        lib = load_library()
        nbytes = int(lib.atl_warp_splat_gather_ws_bytes(N, B, H, W, Hg, Wg))
        if nbytes < 0:
            raise ValueError(f"warp_splat_gather: unsupported sizes N={N} B={B} {H}x{W}, grid {Hg}x{Wg}")
        img = torch.empty(B, H, W, device=xy.device, dtype=F32)          # written by the launch
        vals = torch.empty(N, device=xy.device, dtype=F32)
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=xy.device)
        with torch.cuda.device(xy.device):
            call("atl_warp_splat_gather_fwd", ptr(grid), B, Hg, Wg, ptr(xy), ptr(t), ptr(b), N, H, W, float(t_ref),
                 int(bool(mask_border)), ptr(img), ptr(vals), ptr(ws), nbytes, stream_of(xy))
        ctx.save_for_backward(img, xy, t, b, ws)
        ctx.shape, ctx.t_ref = (B, H, W, Hg, Wg), float(t_ref)
        ctx.set_materialize_grads(False)
        return img, vals

    @staticmethod
    def backward(ctx, gimg, gvals):
        img, xy, t, b, ws = ctx.saved_tensors
        B, H, W, Hg, Wg = ctx.shape
        if not ctx.needs_input_grad[0] or (gimg is None and gvals is None):
            return (None,) * 8
        ggrid = torch.empty(B, 2, Hg, Wg, device=xy.device, dtype=F32)   # written by the launch
        gimg = None if gimg is None else gimg.contiguous().float()
        gvals = None if gvals is None else gvals.contiguous().float()
        with torch.cuda.device(xy.device):
            call("atl_warp_splat_gather_bwd", ptr(img), ptr(gvals), ptr(gimg), ptr(xy), ptr(t), ptr(b), xy.shape[0],
                 B, H, W, Hg, Wg, ctx.t_ref, ptr(ggrid), ptr(ws), ws.numel(), stream_of(xy))
        return ggrid, None, None, None, None, None, None, None


def warp_splat_gather(grid: torch.Tensor, xy: torch.Tensor, t: torch.Tensor, b: torch.Tensor, t_ref: float, H: int,
                      W: int, mask_border: bool = True):
    """Image of events warped by the dense flow ``grid`` (B, 2, Hg, Wg) to ``t_ref`` and its bilinear values at the
    warped events: ``(img (B, H, W), vals (N))``, with ``vals.sum()`` (or any loss of img and vals)
    differentiable with respect to the grid.  The same numbers as ``DenseLinearFlow.transport`` -> ``splat`` ->
    ``gather`` with the weight ``inside(y)`` (or 1), on the device in one sequence of launches."""
    if not xy.is_cuda:
        raise ValueError("warp_splat_gather runs on the GPU (use transport, splat and gather on the CPU)")
    _check_events(xy, b, t, what="warp_splat_gather")
    if grid.dim() != 4 or grid.shape[1] != 2:
        raise ValueError(f"warp_splat_gather: the flow grid must be (B, 2, Hg, Wg), got {tuple(grid.shape)}")
    return _WarpSplatGather.apply(grid, xy, t, b, float(t_ref), int(H), int(W), bool(mask_border))


class _ImageVariance(torch.autograd.Function):
    """Per-image unbiased variance over the last two dimensions (atl/objectives/cmax.py:23-25, the IWE contrast
    iwe.var(dim=(-2, -1))) on the device: fp64 sums over fixed pixel chunks in two launches, and torch.var's
    gradient in one."""

    @staticmethod
    def forward(ctx, img):
        x = _f32(img)
        lead, n = x.shape[:-2], x.shape[-2] * x.shape[-1]
        B = x.numel() // max(n, 1)
        mean = torch.empty(B, device=x.device, dtype=F32)
        var = torch.empty(B, device=x.device, dtype=F32)
        lib = load_library()
        nbytes = int(lib.atl_image_variance_ws_bytes(B, n))
        if nbytes < 0:
            raise ValueError(f"image_variance: unsupported sizes {tuple(x.shape)}")
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
        with torch.cuda.device(x.device):
            call("atl_image_variance", ptr(x), B, n, ptr(mean), ptr(var), ptr(ws), nbytes, stream_of(x))
        ctx.save_for_backward(x, mean)
        ctx.shape = (B, n)
        return var.view(lead)

    @staticmethod
    def backward(ctx, gvar):
        x, mean = ctx.saved_tensors
        B, n = ctx.shape
        g = gvar.contiguous().float().view(B)
        gimg = torch.empty_like(x)
        with torch.cuda.device(x.device):
            call("atl_image_variance_bwd", ptr(x), ptr(mean), ptr(g), B, n, ptr(gimg), stream_of(x))
        return gimg


def image_variance(img: torch.Tensor) -> torch.Tensor:
    """``img.var(dim=(-2, -1))`` (unbiased, over each image's pixels), differentiable; device tensors run the HIP
    kernels, host tensors torch's reduction."""
    if img.dim() < 2 or img.shape[-2] * img.shape[-1] < 1:
        raise ValueError(f"image_variance needs images of at least one pixel, got {tuple(img.shape)}")
    if not img.is_cuda:
        return img.var(dim=(-2, -1))
    return _ImageVariance.apply(img)


class _TrajDisplacement(torch.autograd.Function):
    """PixelTrajectories.displacement in one kernel (atl/motion/trajectories.py: d = sum_k c_k(p) g_k(t), the
    coefficients c_k the border-clamped bilinear sample of a (B, 2K, Hg, Wg) grid at grid coordinates p).
    Differentiable w.r.t. the grid and the positions; the times carry no gradient.  The backward writes the
    per-channel output gradient (g_k times the displacement's gradient) and hands it to the flow sampler's
    field adjoint and position gradient."""

    @staticmethod
    def forward(ctx, fld, gpos, b, t, K, basis, plan):
        fld, gpos, b, t = _f32(fld), _f32(gpos), b.contiguous().long(), _f32(t)
        B, C, Hg, Wg = fld.shape
        N = gpos.shape[0]
        out = torch.empty(N, 2, device=gpos.device, dtype=F32)
        ctx.plan = None
        with torch.cuda.device(gpos.device):
            st = stream_of(gpos)
            fcl = _channels_last(fld)
            call("atl_traj_displacement", ptr(fcl), B, C, K, Hg, Wg, ptr(gpos), ptr(b), ptr(t), N, basis, ptr(out),
                 st)
            bspline = basis == TRAJ_BASES["bspline"] and K >= 3 and _traj_field_ok(K, B, Hg, Wg, N) >= 0
            ctx.bspline = bspline
            if plan and not bspline and _tile_plan_ok(B, C, Hg, Wg):
                nbytes = int(load_library().atl_grid_plan_bytes(B, Hg, Wg, N))
                if nbytes >= 0:
                    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=gpos.device)
                    call("atl_grid_plan", B, Hg, Wg, ptr(gpos), ptr(b), N, 0, 0, ptr(ws), nbytes, st)
                    ctx.plan = ws
        ctx.save_for_backward(gpos, b, t, fcl)
        ctx.shape, ctx.K, ctx.basis = (B, C, Hg, Wg), K, basis
        return out

    @staticmethod
    def backward(ctx, gd):
        gpos, b, t, fcl = ctx.saved_tensors
        B, C, Hg, Wg = ctx.shape
        N = gpos.shape[0]
        gd = gd.contiguous().float()
        gf = gp = None
        with torch.cuda.device(gpos.device):
            st = stream_of(gpos)
            if ctx.bspline:
                # the gradient rows are formed from gd and t inside both kernels (no (N, 2K) rows in memory)
                if ctx.needs_input_grad[0]:
                    gf = _traj_field_grad(gd.view(1, N, 2), gpos.view(1, N, 2), t, None, b, ctx.K, B, Hg, Wg)
                if ctx.needs_input_grad[1]:
                    gp = torch.empty_like(gpos)
                    call("atl_traj_pos_bwd_cl", ptr(gd), ptr(t), ctx.K, ptr(fcl), B, Hg, Wg, ptr(gpos), ptr(b), N,
                         ptr(gp), st)
                return gf, gp, None, None, None, None, None
            g = torch.empty(N, C, device=gpos.device, dtype=F32)
            call("atl_traj_gout", ptr(gd), ptr(t), N, ctx.K, ctx.basis, ptr(g), st)
            if ctx.needs_input_grad[0]:
                gf = torch.zeros(B, C, Hg, Wg, device=gpos.device, dtype=F32)
                if ctx.plan is not None:
                    call("atl_sample_grid_bwd_planned", ptr(g), B, C, Hg, Wg, ptr(gpos), N, 0, 0, ptr(ctx.plan),
                         ptr(gf), st)
                else:
                    call("atl_sample_grid_bwd", ptr(g), B, C, Hg, Wg, ptr(gpos), ptr(b), N, 0, 0, ptr(gf), st)
            if ctx.needs_input_grad[1]:
                gp = torch.empty_like(gpos)
                call("atl_sample_grid_bwd_pos_cl", ptr(g), ptr(fcl), B, C, Hg, Wg, ptr(gpos), ptr(b), N, 0, 0,
                     ptr(gp), st)
        return gf, gp, None, None, None, None, None


TRAJ_MAX_K = 16
TRAJ_BASES = {"polynomial": 0, "bezier": 1, "bspline": 2}


def _check_events(pos, b, *per_event, what):
    """Shape checks of a device op's event arrays, before any launch: pos (N, 2), b and every per-event
    array (N,)."""
    if pos.dim() != 2 or pos.shape[1] != 2:
        raise ValueError(f"{what}: positions must be (N, 2), got {tuple(pos.shape)}")
    n = pos.shape[0]
    if b.shape != (n,):
        raise ValueError(f"{what}: batch index must be ({n},), got {tuple(b.shape)}")
    for a in per_event:
        if a.shape != (n,):
            raise ValueError(f"{what}: per-event array must be ({n},), got {tuple(a.shape)}")


def traj_displacement(fld: torch.Tensor, gpos: torch.Tensor, b: torch.Tensor, t: torch.Tensor, K: int,
                      basis: str) -> torch.Tensor:
    """Displacement (N, 2) in (x, y) of trajectories with coefficient grid ``fld`` (B, 2K, Hg, Wg), channels
    [y_1..y_K, x_1..x_K], at grid coordinates ``gpos``; ``basis`` "polynomial", "bezier" or "bspline" (the
    clamped uniform B-spline of degree min(3, K) with K + 1 functions, the first pinned to the start).  Device
    tensors, K <= TRAJ_MAX_K."""
    get_ext()
    if basis not in TRAJ_BASES:
        raise ValueError(f"unknown basis {basis!r}")
    if t.requires_grad:
        raise ValueError("traj_displacement: event times carry no gradient")
    if not 1 <= int(K) <= TRAJ_MAX_K:
        raise ValueError(f"traj_displacement: K = {K} outside 1..{TRAJ_MAX_K}")
    if fld.dim() != 4 or fld.shape[1] != 2 * int(K):
        raise ValueError(f"traj_displacement: coefficient grid must be (B, 2K = {2 * int(K)}, Hg, Wg), got "
                         f"{tuple(fld.shape)}")
    _check_events(gpos, b, t, what="traj_displacement")
    plan = fld.requires_grad and torch.is_grad_enabled()
    return _TrajDisplacement.apply(fld, gpos, b, t, int(K), TRAJ_BASES[basis], plan)


def _traj_field_ok(K, B, Hg, Wg, n_rec):
    """atl_traj_field_bwd's workspace bytes for n_rec look-ups, or -1 where it does not take the sizes."""
    return int(load_library().atl_traj_field_bwd_bytes(int(K), B, Hg, Wg, n_rec))


def _traj_field_grad(gD, P, t, t_last, b, K, B, Hg, Wg):
    """Coefficient-grid gradient (B, 2K, Hg, Wg) of n look-ups of N events: look-up r of event e at grid position
    P[r, e] with displacement gradient gD[r, e] (both (n, N, 2)) and time t[e] (t_last[e] for the last look-up
    when t_last is given), binned and accumulated in one atl_traj_field_bwd call."""
    n, N = P.shape[0], P.shape[1]
    nbytes = _traj_field_ok(K, B, Hg, Wg, n * N)
    if nbytes < 0:
        raise HipLibraryError(f"traj field gradient: unsupported sizes K={K} B={B} {Hg}x{Wg} records={n * N}")
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=gD.device)
    gf = torch.zeros(B, 2 * int(K), Hg, Wg, device=gD.device, dtype=F32)
    call("atl_traj_field_bwd", ptr(gD), ptr(P), ptr(t), ptr(t_last), ptr(b), N, n, int(K), B, Hg, Wg, ptr(ws), nbytes,
         ptr(gf), stream_of(gD))
    return gf


class _TrajOrigin(torch.autograd.Function):
    """PixelTrajectories.origin's n Picard steps p_{k+1} = xy - d(p_k, t), p_0 = xy, as one autograd node
    (atl/motion/trajectories.py:68-73 differentiated step by step, as autograd does there), and with ``t_dst``
    PixelTrajectories.transport's last look-up y = p + d(p, t_dst) (trajectories.py:75-77) in the same node.  The
    forward runs the steps in one kernel (atl_traj_origin, the composed ops' bits) and keeps the positions the
    displacements are taken at; the backward runs the steps' position gradients in reverse order in one kernel
    (atl_traj_origin_bwd) and then adds the coefficient-grid gradient of every look-up in one accumulation over
    their records (one tile plan instead of one per look-up), each record's row formed from its displacement
    gradient and time.  B-spline basis with K >= 3 on a grid the tile adjoint takes (the caller checks); grid
    coordinates g = (p - offset) / tile."""

    @staticmethod
    def forward(ctx, fld, xy, b, t, K, basis, n, offset, tile, t_dst):
        fld, xy, b, t = _f32(fld), _f32(xy), b.contiguous().long(), _f32(t)
        B, C, Hg, Wg = fld.shape
        N = xy.shape[0]
        fin = t_dst is not None
        P = torch.empty(n + int(fin), N, 2, device=xy.device, dtype=F32)   # grid coordinates of every look-up
        p = torch.empty(N, 2, device=xy.device, dtype=F32)
        with torch.cuda.device(xy.device):
            st = stream_of(xy)
            fcl = _channels_last(fld)
            call("atl_traj_origin", ptr(fcl), B, C, K, Hg, Wg, ptr(xy), ptr(t), ptr(b), N, n, float(offset), int(tile),
                 basis, ptr(P), int(fin), ptr(p), st)
            if fin:
                t_dst = _f32(t_dst)
                d = torch.empty(N, 2, device=xy.device, dtype=F32)
                call("atl_traj_displacement", ptr(fcl), B, C, K, Hg, Wg, ptr(P[n]), ptr(b), ptr(t_dst), N, basis,
                     ptr(d), st)
                p = p + d
        ctx.save_for_backward(P, b, t, fcl, t_dst if fin else None)
        ctx.shape, ctx.K, ctx.tile, ctx.n, ctx.fin = (B, C, Hg, Wg), K, tile, n, fin
        return p

    @staticmethod
    def backward(ctx, gy):
        P, b, t, fcl, t_dst = ctx.saved_tensors
        B, C, Hg, Wg = ctx.shape
        n, fin = ctx.n, ctx.fin
        N = P.shape[1]
        gy = gy.contiguous().float()
        gD = torch.empty(n + int(fin), N, 2, device=gy.device, dtype=F32)   # gradient of every look-up
        gxy = torch.empty_like(gy) if ctx.needs_input_grad[1] else None
        gf = None
        with torch.cuda.device(gy.device):
            st = stream_of(gy)
            g = gy
            if fin:                                                  # y = p + d(p, t_dst)
                gD[n] = gy
                gk = torch.empty_like(gy)
                call("atl_traj_pos_bwd_cl", ptr(gy), ptr(t_dst), ctx.K, ptr(fcl), B, Hg, Wg, ptr(P[n]), ptr(b), N,
                     ptr(gk), st)
                g = gy + (gk if ctx.tile == 1 else gk / ctx.tile)
            # the steps in reverse order: gD_k = -g, g <- d's position derivative at P[k] applied to gD_k / tile
            call("atl_traj_origin_bwd", ptr(fcl), B, C, ctx.K, Hg, Wg, ptr(P), ptr(t), ptr(b), N, n, ctx.tile,
                 ptr(g), ptr(gD), ptr(gxy), st)
            if ctx.needs_input_grad[0]:
                gf = _traj_field_grad(gD, P, t, t_dst, b, ctx.K, B, Hg, Wg)
        return gf, gxy, None, None, None, None, None, None, None, None


def traj_origin(fld: torch.Tensor, xy: torch.Tensor, b: torch.Tensor, t: torch.Tensor, K: int, basis: str,
                n_steps: int, offset: float = 0.0, tile: int = 1, t_dst: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Trajectory starts p with p = xy - d(p, t) after ``n_steps`` Picard steps from p = xy, on the device, with
    the fixed-point steps as one autograd node (the same values and gradients as composing traj_displacement
    n_steps times; the coefficient-grid gradient of all steps is added in one accumulation).  With ``t_dst`` (N,)
    the node returns the transported positions p + d(p, t_dst) instead (PixelTrajectories.transport).  B-spline
    basis, 3 <= K <= TRAJ_MAX_K, ``fld`` (B, 2K, Hg, Wg) taken by the tile adjoint; grid coordinates
    (p - offset) / tile."""
    get_ext()
    if basis != "bspline" or not 3 <= int(K) <= TRAJ_MAX_K:
        raise ValueError("traj_origin: B-spline basis with 3 <= K <= TRAJ_MAX_K")
    if t.requires_grad or (t_dst is not None and t_dst.requires_grad):
        raise ValueError("traj_origin: event times carry no gradient")
    if fld.dim() != 4 or fld.shape[1] != 2 * int(K):
        raise ValueError(f"traj_origin: coefficient grid must be (B, 2K = {2 * int(K)}, Hg, Wg), got "
                         f"{tuple(fld.shape)}")
    B, C, Hg, Wg = fld.shape
    if not _tile_plan_ok(B, C, Hg, Wg):
        raise ValueError("traj_origin: grid too large for the tile adjoint")
    _check_events(xy, b, t, *(() if t_dst is None else (t_dst,)), what="traj_origin")
    if int(n_steps) < 1:
        raise ValueError("traj_origin: at least one step")
    return _TrajOrigin.apply(fld, xy, b, t, int(K), TRAJ_BASES[basis], int(n_steps), float(offset), int(tile), t_dst)


def sample_grid_hip(fld: torch.Tensor, pos: torch.Tensor, b: torch.Tensor, img_hw=(0, 0)) -> torch.Tensor:
    """HIP flow lookup: ``pos`` are grid coordinates, or image pixels mapped by x / max(W-1, 1) * (Wg-1)
    when ``img_hw`` = (H, W) is given (DenseLinearFlow.field).  Differentiable w.r.t. the field and the
    positions."""
    get_ext()
    if fld.dim() != 4:
        raise ValueError(f"sample_grid: field must be (B, C, Hg, Wg), got {tuple(fld.shape)}")
    _check_events(pos, b, what="sample_grid")
    plan = fld.requires_grad and torch.is_grad_enabled()     # sort the positions for a gather backward
    return _SampleGrid.apply(fld, pos, b, img_hw[0], img_hw[1], plan)


# ------------------------------------------------------------------------------------------- anchored pairs
@dataclass
class PairPlan:
    """Spatial hash for :func:`ats_pair_sums`: (source, slice) entries sorted by (batch, slice, cell)
    (atl/ops/functional.py:114-130)."""
    src_y: torch.Tensor
    src_v: torch.Tensor
    src_t: torch.Tensor
    src_id: torch.Tensor
    cell_start: torch.Tensor
    anc_x: torch.Tensor
    anc_t: torch.Tensor
    anc_cell: torch.Tensor
    anc_id: torch.Tensor
    slice_c: torch.Tensor
    S: int
    GH: int
    GW: int
    geometry: dict = field(default_factory=dict)


def decode_ordered(st: np.ndarray) -> np.ndarray:
    """Floats from the order-preserving int encoding used by the device reductions."""
    st = st.astype(np.int32)
    return np.where(st >= 0, st, st ^ np.int32(0x7FFFFFFF)).astype(np.int32).view(np.float32)


def plan_stats(v: torch.Tensor, xa: torch.Tensor):
    """(vmax, min x, min y, max x, max y) of the plan geometry from one device reduction (one host sync)."""
    dev = v.device
    stats = torch.empty(5, dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        call("atl_plan_stats", ptr(v), v.shape[0], ptr(xa), xa.shape[0], ptr(stats), stream_of(v))
    f = decode_ordered(stats.cpu().numpy())
    return float(f[0]), float(f[1]), float(f[2]), -float(f[3]), -float(f[4])


def plan_geometry(vmax: float, bbox, M: int, h, tau, cut, S, W, H):
    """Grid geometry in Python doubles exactly as atl/ops/functional.py:135-149."""
    delta = 1.0 / S
    cell = max(cut * h + vmax * delta / 2 + 1e-3, 1.0)
    if M:
        ox, oy = bbox[0] - cell, bbox[1] - cell
        ex, ey = bbox[2] + cell, bbox[3] + cell
    else:
        ox, oy, ex, ey = -cell, -cell, W + cell, H + cell
    GW = int(math.ceil((ex - ox) / cell)) + 1
    GH = int(math.ceil((ey - oy) / cell)) + 1
    return dict(delta=delta, cell=cell, ox=ox, oy=oy, ex=ex, ey=ey, GW=GW, GH=GH, vmax=vmax)


def _scan(counts: torch.Tensor) -> torch.Tensor:
    n = counts.shape[0]
    lib_work = int(load_library().atl_scan_work_size(n))
    start = torch.empty(n + 1, dtype=I64, device=counts.device)
    work = torch.empty(max(lib_work, 1), dtype=I64, device=counts.device)
    call("atl_scan_counts", ptr(counts), n, ptr(start), ptr(work), stream_of(counts))
    return start


def _build_pair_plan_hip(x, t, v, b, B, H, W, anchors, h, tau, cut, n_slices, anchor_xy):
    dev = x.device
    S = int(n_slices)
    delta = 1.0 / S
    x, t, vd = _f32(x), _f32(t), _f32(v.detach())
    b, anchors = b.contiguous().long(), anchors.contiguous().long()
    N, M = t.shape[0], anchors.shape[0]
    xa_all = _f32(x[anchors] if anchor_xy is None else anchor_xy.detach())
    with torch.cuda.device(dev):
        vmax, *bbox = plan_stats(vd, xa_all)
        geo = plan_geometry(vmax if N else 0.0, bbox, M, h, tau, cut, S, W, H)
        GW, GH, cell, ox, oy = geo["GW"], geo["GH"], geo["cell"], geo["ox"], geo["oy"]
        ncell = B * S * GH * GW
        if ncell >= 2 ** 31:
            raise ValueError(f"pair plan grid too large ({ncell} cells)")
        st = stream_of(x)
        lib = load_library()
        ecap = N * min(int(math.floor((2.0 * float(tau) + 1.0 / S) * S)) + 2, S)   # entries per source, at most
        nbytes = int(lib.atl_plan_sort_bytes(N, ecap, ncell))
        if nbytes >= 0:                            # counting sort: no per-entry atomics, one synchronisation
            ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
            cell_start = torch.empty(ncell + 1, dtype=I64, device=dev)
            src_y = torch.empty(ecap, 2, dtype=F32, device=dev)
            src_v = torch.empty(ecap, 2, dtype=F32, device=dev)
            src_t = torch.empty(ecap, dtype=F32, device=dev)
            src_id = torch.empty(ecap, dtype=I64, device=dev)
            call("atl_plan_sort", ptr(x), ptr(t), ptr(vd), ptr(b), N, B, ox, oy, cell, float(tau), S, GH, GW, ecap,
                 ptr(cell_start), ptr(src_y), ptr(src_v), ptr(src_t), ptr(src_id), ptr(ws), nbytes, st)
            E = int(cell_start[-1])
            src_y, src_v, src_t, src_id = src_y[:E], src_v[:E], src_t[:E], src_id[:E]
        else:
            counts = torch.zeros(ncell, dtype=torch.int32, device=dev)
            call("atl_plan_count", ptr(x), ptr(t), ptr(vd), ptr(b), N, B, ox, oy, cell, float(tau), S, GH, GW,
                 ptr(counts), st)
            cell_start = _scan(counts)
            E = int(cell_start[-1])
            src_y = torch.empty(E, 2, dtype=F32, device=dev)
            src_v = torch.empty(E, 2, dtype=F32, device=dev)
            src_t = torch.empty(E, dtype=F32, device=dev)
            src_id = torch.empty(E, dtype=I64, device=dev)
            counts.zero_()
            call("atl_plan_fill", ptr(x), ptr(t), ptr(vd), ptr(b), N, B, ox, oy, cell, float(tau), S, GH, GW,
                 ptr(cell_start), ptr(counts), ptr(src_y), ptr(src_v), ptr(src_t), ptr(src_id), st)
        anc_x = torch.empty(M, 2, dtype=F32, device=dev)
        anc_t = torch.empty(M, dtype=F32, device=dev)
        anc_cell = torch.empty(M, 3, dtype=I64, device=dev)
        anc_id = torch.empty(M, dtype=I64, device=dev)
        call("atl_plan_anchors", ptr(x), ptr(t), ptr(b), ptr(anchors),
             ptr(None if anchor_xy is None else xa_all), M, N, ox, oy, cell, S, GH, GW, ptr(anc_x), ptr(anc_t),
             ptr(anc_cell), ptr(anc_id), st)
        slice_c = (torch.arange(S, device=dev, dtype=F32) + 0.5) * delta
    return PairPlan(src_y, src_v, src_t, src_id, cell_start, anc_x, anc_t, anc_cell, anc_id, slice_c, S, GH, GW,
                    geo)


def _slice_span(t: torch.Tensor, tau: float, S: int):
    """First and last slice whose centre lies within tau + delta/2 of each event time (delta = 1/S), clamped to
    [0, S-1]: fp32 in the order (t -/+ tau -/+ delta/2) / delta - 1/2 (atl/ops/functional.py:151-152)."""
    d = 1.0 / S
    lo = torch.ceil((t - tau - d / 2) / d - 0.5)
    hi = torch.floor((t + tau + d / 2) / d - 0.5)
    return lo.clamp(0, S - 1).long(), hi.clamp(0, S - 1).long()


def _cell_index(p: torch.Tensor, ox: float, oy: float, cell: float):
    """Integer cell column and row of positions p (N, 2): floor((p - o) / cell) in fp32."""
    return torch.floor((p[:, 0] - ox) / cell).long(), torch.floor((p[:, 1] - oy) / cell).long()


def _build_pair_plan_torch(x, t, v, b, B, H, W, anchors, h, tau, cut, n_slices, anchor_xy):
    """CPU tensors: the plan of atl/ops/functional.py:132-178 built one slice at a time.  For slice s the
    sources whose slice span holds s are transported to the slice centre c_s, y = x + v (c_s - t) (fp32: one
    subtraction, one product, one sum, the reference's rounding), binned, and keyed by (batch, slice, row,
    column).  The slices' entries are then put in key order by one stable sort, which leaves the entries of a
    cell in source order, the order the reference's stable sort of its (source, slice) list gives.  Cell offsets
    are the positions of the cell numbers in the sorted keys."""
    S = int(n_slices)
    with torch.no_grad():
        t = t.float()
        vel = v.detach().float()
        anc_xy = (x[anchors] if anchor_xy is None else anchor_xy).float()
        nrm = vel.norm(dim=1)
        vmax = float(nrm.max()) if nrm.numel() else 0.0
        box = ((float(anc_xy[:, 0].min()), float(anc_xy[:, 1].min()), float(anc_xy[:, 0].max()),
                float(anc_xy[:, 1].max())) if anc_xy.numel() else (0.0, 0.0, 0.0, 0.0))
        geo = plan_geometry(vmax, box, anc_xy.shape[0], h, tau, cut, S, W, H)
        gw, gh, side, ox, oy = geo["GW"], geo["GH"], geo["cell"], geo["ox"], geo["oy"]
        centres = (torch.arange(S, dtype=torch.float32) + 0.5) * (1.0 / S)
        first, last = _slice_span(t, tau, S)
        ids, keys = [], []
        for s in range(S):
            src = torch.nonzero((first <= s) & (s <= last)).flatten()
            ys = x[src].float() + vel[src] * (centres[s] - t[src])[:, None]
            col, row = _cell_index(ys, ox, oy, side)
            inside = (col >= 0) & (col < gw) & (row >= 0) & (row < gh)
            src, col, row = src[inside], col[inside], row[inside]
            ids.append(src)
            keys.append(((b[src] * S + s) * gh + row) * gw + col)
        key_all = torch.cat(keys) if keys else torch.zeros(0, dtype=I64)
        id_all = torch.cat(ids) if ids else torch.zeros(0, dtype=I64)
        key_all, perm = torch.sort(key_all, stable=True)
        sid = id_all[perm]
        slc = (key_all // (gh * gw)) % S
        y = x[sid].float() + vel[sid] * (centres[slc] - t[sid])[:, None]
        cell_start = torch.searchsorted(key_all, torch.arange(B * S * gh * gw + 1, dtype=I64))
        ta = t[anchors]
        a_slice = torch.floor(ta / (1.0 / S)).clamp(0, S - 1).long()
        a_col, a_row = _cell_index(anc_xy, ox, oy, side)
        anc_cell = torch.stack([b[anchors] * S + a_slice, a_col.clamp(0, gw - 1), a_row.clamp(0, gh - 1)], 1)
    return PairPlan(y.contiguous(), vel[sid].contiguous(), t[sid].contiguous(), sid.contiguous(), cell_start,
                    anc_xy.contiguous(), ta.contiguous(), anc_cell.contiguous(), anchors.long().contiguous(),
                    centres, S, gh, gw, geo)


def build_pair_plan(x, t, v, b, B, H, W, anchors, h, tau, cut=3.0, n_slices=16, anchor_xy=None) -> PairPlan:
    """Spatial hash of (source, slice) pairs sorted by (batch, slice, cell) (atl/ops/functional.py:132-178).

    On device tensors the plan is built by HIP kernels (count, scan, scatter) with the reference's fp32
    arithmetic, so slice ranges, cell bins, keys and ``cell_start`` are bit-identical to the reference's CPU
    plan.  ``vmax`` is max ||v|| evaluated as sqrt(fma(vy, vy, vx * vx)), the rounding of torch's CPU vector
    norm on AVX2/AVX-512 hosts.  Entry order within one cell is unspecified, as with ``torch.argsort``."""
    with torch.no_grad():
        if x.is_cuda:
            get_ext()
            return _build_pair_plan_hip(x, t, v, b, B, H, W, anchors, h, tau, cut, n_slices, anchor_xy)
        return _build_pair_plan_torch(x, t, v, b, B, H, W, anchors, h, tau, cut, n_slices, anchor_xy)


class _ATSPair(torch.autograd.Function):
    """atl/ops/functional.py:181-196: forward over a plan; gradient to the per-event velocities only."""

    @staticmethod
    def forward(ctx, v, plan: PairPlan, h, tau, cut):
        e = get_ext()
        ctx.plan, ctx.args, ctx.n = plan, (float(h), float(tau), float(cut)), v.shape[0]
        p = plan
        # the workspace keeps the anchors binned by the forward for the backward (one binning per step)
        out, ctx.ws = e.ats_pair_fwd(p.src_y, p.src_v, p.src_t, p.src_id, p.cell_start, p.anc_x, p.anc_t,
                                     p.anc_cell, p.anc_id, p.slice_c, p.S, p.GH, p.GW, *ctx.args, keep_ws=True,
                                     n_src=ctx.n)
        return out

    @staticmethod
    def backward(ctx, g):
        p = ctx.plan
        gv = get_ext().ats_pair_bwd(g.contiguous().float(), p.src_y, p.src_v, p.src_t, p.src_id, p.cell_start,
                                    p.anc_x, p.anc_t, p.anc_cell, p.anc_id, p.slice_c, p.S, p.GH, p.GW,
                                    *ctx.args, ctx.n, ws=ctx.ws)
        return gv, None, None, None, None


class FastPairPlan:
    """Device workspace of the fused pair-sum path (include/atl_hip.h, atl_fast_*): the reference's (source,
    slice) entries and the anchors binned on a fixed fine-cell grid, built without a host synchronisation.
    Holds its inputs alive for as long as it is used.

    ``traj=(coef, K, table)`` selects the trajectory source model: ``x`` are then the trajectory starts p (N, 2),
    ``coef`` the (N, 2K) coefficient rows and ``table`` the (S, 2K) basis at the slice centres; ``v`` is unused
    (pass None) and ``anchor_xy`` is required (the anchors are not at the starts)."""

    def __init__(self, x, t, v, b, B, H, W, anchors, h, tau, cut=3.0, n_slices=16, anchor_xy=None, traj=None):
        dev = x.device
        self.x, self.t = _f32(x), _f32(t)
        self.b = b.contiguous().long()
        self.anchors = None if anchors is None else anchors.contiguous().long()   # None: every event, in order
        self.anchor_xy = None if anchor_xy is None else _f32(anchor_xy.detach())
        N = self.t.shape[0]
        M = N if self.anchors is None else self.anchors.shape[0]
        self.traj = traj is not None
        if self.traj:
            coef, K, table = traj
            self.K = int(K)
            self.coef, self.table = _f32(coef.detach()), _f32(table)
            if self.coef.shape != (N, 2 * self.K) or self.table.shape != (int(n_slices), 2 * self.K):
                raise ValueError(f"trajectory pair sums: coef must be ({N}, {2 * self.K}) and table "
                                 f"({int(n_slices)}, {2 * self.K})")
            if self.anchor_xy is None:
                raise ValueError("trajectory pair sums need anchor_xy (the anchors are not at the trajectory starts)")
            self.v = None
        else:
            self.v = _f32(v.detach())
            if self.v.shape != (N, 2):
                raise ValueError("x, v must be (N, 2) and t, b (N,)")
        if self.x.shape != (N, 2) or self.b.shape != (N,):
            raise ValueError("x must be (N, 2) and t, b (N,)")
        if self.anchor_xy is not None and self.anchor_xy.shape != (M, 2):
            raise ValueError("anchor_xy must be (M, 2)")
        self.N, self.M, self.device = N, M, dev
        self.geo = FastGeometry()
        lib = load_library()
        if lib.atl_fast_geometry_init(N, M, int(B), int(H), int(W), int(n_slices), float(h), float(tau), float(cut),
                                      ctypes.byref(self.geo)) != 0:
            raise HipLibraryError("atl_fast_geometry_init: " + lib.atl_last_error().decode(errors="replace"))
        self.ws = torch.empty(int(self.geo.ws_bytes), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            if self.traj:
                call("atl_fast_plan_traj", ctypes.byref(self.geo), ptr(self.x), ptr(self.coef), self.K,
                     ptr(self.table), ptr(self.t), ptr(self.b), ptr(self.anchors), ptr(self.anchor_xy), ptr(self.ws),
                     int(self.geo.ws_bytes), stream_of(self.x))
            else:
                call("atl_fast_plan", ctypes.byref(self.geo), ptr(self.x), ptr(self.t), ptr(self.v), ptr(self.b),
                     ptr(self.anchors), ptr(self.anchor_xy), ptr(self.ws), int(self.geo.ws_bytes), stream_of(self.x))

    def forward(self, count: Optional[torch.Tensor] = None) -> torch.Tensor:
        out = torch.zeros(self.M, dtype=F32, device=self.device)
        with torch.cuda.device(self.device):
            call("atl_fast_pair_fwd", ctypes.byref(self.geo), ptr(self.ws), ptr(out), ptr(count), stream_of(out))
        return out

    def _check_gs(self, gS):
        gS = _f32(gS)
        if gS.shape != (self.M,):
            raise ValueError(f"gS has shape {tuple(gS.shape)}, expected ({self.M},)")
        return gS

    def backward(self, gS: torch.Tensor) -> torch.Tensor:
        """Linear model: dL/dv (N, 2)."""
        if self.traj:
            raise ValueError("a trajectory plan has backward_traj")
        gS = self._check_gs(gS)
        gv = torch.empty(self.N, 2, dtype=F32, device=self.device)
        with torch.cuda.device(self.device):
            call("atl_fast_pair_bwd", ctypes.byref(self.geo), ptr(self.ws), ptr(gS), ptr(gv), stream_of(gv))
        return gv

    def backward_flow(self, gS: torch.Tensor, B: int, Hg: int, Wg: int, img_h: int, img_w: int) -> torch.Tensor:
        """Linear model whose velocities are the dense flow sampled at x (DenseLinearFlow.field): dL/dgrid
        (B, 2, Hg, Wg), the pair backward's source gradients accumulated into the grid tile by tile over the
        source records (no per-event gradient array, no binning)."""
        if self.traj:
            raise ValueError("a trajectory plan has backward_traj")
        gS = self._check_gs(gS)
        gg = torch.empty(int(B), 2, int(Hg), int(Wg), dtype=F32, device=self.device)   # written by the adjoint
        with torch.cuda.device(self.device):
            st = stream_of(gg)
            call("atl_fast_pair_bwd_src", ctypes.byref(self.geo), ptr(self.ws), ptr(gS), st)
            call("atl_fast_flow_adjoint", ctypes.byref(self.geo), ptr(self.ws), int(Hg), int(Wg), int(img_h),
                 int(img_w), ptr(gg), st)
        return gg

    def backward_traj(self, gS: torch.Tensor):
        """Trajectory model: (dL/dp (N, 2), dL/dcoef (N, 2K))."""
        if not self.traj:
            raise ValueError("a linear plan has backward")
        gS = self._check_gs(gS)
        gp = torch.empty(self.N, 2, dtype=F32, device=self.device)
        gc = torch.empty(self.N, 2 * self.K, dtype=F32, device=self.device)
        with torch.cuda.device(self.device):
            call("atl_fast_pair_bwd_traj", ctypes.byref(self.geo), ptr(self.ws), ptr(gS), ptr(self.coef), self.K,
                 ptr(self.table), ptr(gp), ptr(gc), stream_of(gp))
        return gp, gc

    def counts(self) -> torch.Tensor:
        """n_i: number of contributing pairs of every anchor (bit-identical to the reference's visits)."""
        cnt = torch.zeros(self.M, dtype=torch.int32, device=self.device)
        self.forward(count=cnt)
        return cnt


class _ATSPairFast(torch.autograd.Function):
    """atl/ops/functional.py:181-196 on the fused path: plan and forward in one go, gradient to v only."""

    @staticmethod
    def forward(ctx, v, x, t, b, anchors, anchor_xy, B, H, W, h, tau, cut, n_slices):
        plan = FastPairPlan(x, t, v, b, B, H, W, anchors, h, tau, cut, n_slices, anchor_xy)
        ctx.plan = plan
        return plan.forward()

    @staticmethod
    def backward(ctx, g):
        gv = ctx.plan.backward(g)
        return gv, None, None, None, None, None, None, None, None, None, None, None, None


class _ATSPairFlow(torch.autograd.Function):
    """ats_pair_sums with v = DenseLinearFlow.field(x) (atl/motion/parametric.py:212-216, 235-251) folded in:
    the flow is sampled at x, the pairs summed as by _ATSPairFast, and the backward hands the pair gradients of
    the velocities straight to the flow grid (one pass over the plan's source records) instead of returning them
    per event for sample_grid's adjoint."""

    @staticmethod
    def forward(ctx, grid, x, t, b, anchors, anchor_xy, B, H, W, h, tau, cut, n_slices):
        with torch.no_grad():
            v = sample_grid_hip(grid.detach(), x, b, img_hw=(H, W))
        plan = FastPairPlan(x, t, v, b, B, H, W, anchors, h, tau, cut, n_slices, anchor_xy)
        ctx.plan, ctx.shape, ctx.img = plan, tuple(grid.shape), (int(H), int(W))
        return plan.forward()

    @staticmethod
    def backward(ctx, g):
        Bg, _, Hg, Wg = ctx.shape
        gg = ctx.plan.backward_flow(g, Bg, Hg, Wg, ctx.img[0], ctx.img[1])
        return gg, None, None, None, None, None, None, None, None, None, None, None, None


def ats_pair_sums_flow(grid, x, t, b, B, H, W, anchors, h, tau, cut=3.0, n_slices=16, anchor_xy=None):
    """ats_pair_sums(x, t, DenseLinearFlow.field(x), ...) on the device with the gradient going to the dense flow
    grid (B, 2, Hg, Wg) directly: the same sums and the same grid gradient as sampling the flow and calling
    ats_pair_sums (float sums of the adjoint in another order)."""
    if not x.is_cuda:
        raise ValueError("ats_pair_sums_flow runs on the GPU (sample the flow and call ats_pair_sums on the CPU)")
    if grid.dim() != 4 or grid.shape[1] != 2 or grid.shape[0] != int(B):
        raise ValueError(f"ats_pair_sums_flow: the flow grid must be ({int(B)}, 2, Hg, Wg), got {tuple(grid.shape)}")
    get_ext()
    return _ATSPairFlow.apply(grid, x.detach(), t.detach(), b, anchors, anchor_xy, int(B), int(H), int(W),
                              float(h), float(tau), float(cut), int(n_slices))


def ats_pair_sums(x, t, v, b, B, H, W, anchors, h, tau, cut=3.0, n_slices=16, force_ref=False, anchor_xy=None):
    """S_i = sum_{j != i} 1[|t_i - t_j| <= tau] exp(-|x_i - x_j - v_j (t_i - t_j)|^2 / 2h^2) for anchors i
    (atl/ops/functional.py:199-207).  ``x`` are raw event positions, ``v`` per-event velocities in px per
    window; the gradient flows to ``v`` only.  ``anchors=None`` means every event, in order.  Device tensors run the fused HIP path (same contributing pairs
    as the reference's plan + kernel, no host synchronisation)."""
    if force_ref or not ext_supports(x):
        if anchors is None:
            anchors = torch.arange(x.shape[0], device=x.device)
        return ref.ats_pair_sums(x.float(), t.float(), v.float(), b, anchors, h, tau, cut, anchor_xy=anchor_xy)
    get_ext()
    return _ATSPairFast.apply(v.float(), x.detach(), t.detach(), b, anchors, anchor_xy, int(B), int(H), int(W),
                              float(h), float(tau), float(cut), int(n_slices))


def ats_pair_sums_reference_layout(x, t, v, b, B, H, W, anchors, h, tau, cut=3.0, n_slices=16, anchor_xy=None):
    """The call pattern of the reference's unchanged ats_pair_sums (atl/ops/functional.py:199-207) on this
    library: the reference's plan layout built on the device (build_pair_plan, bit-exact with the reference's),
    then the pybind-surface ops ats_pair_fwd / ats_pair_bwd through their workspace entries (anchors binned by
    cell; the forward one wave per cell item, the backward source-centric without per-pair atomics).  Same values
    as ats_pair_sums; kept to measure what a caller gets without switching to the fused path."""
    if anchors is None:
        anchors = torch.arange(x.shape[0], device=x.device)
    plan = build_pair_plan(x.detach(), t, v.detach(), b, B, H, W, anchors, h, tau, cut, n_slices,
                           anchor_xy=None if anchor_xy is None else anchor_xy.detach())
    return _ATSPair.apply(v.float(), plan, h, tau, cut)


class _ATSPairTraj(torch.autograd.Function):
    """Pair sums of the trajectory model: gradients to the trajectory starts p and the coefficient rows."""

    @staticmethod
    def forward(ctx, p, coef, t, b, anchors, anchor_xy, B, H, W, h, tau, cut, n_slices, K, table):
        plan = FastPairPlan(p.detach(), t, None, b, B, H, W, anchors, h, tau, cut, n_slices, anchor_xy,
                            traj=(coef, K, table))
        ctx.plan = plan
        return plan.forward()

    @staticmethod
    def backward(ctx, g):
        gp, gc = ctx.plan.backward_traj(g)
        return (gp, gc) + (None,) * 13


TRAJ_PAIR_MAX_K = 12


def ats_pair_sums_traj(p, coef, t, b, B, H, W, anchors, h, tau, cut=3.0, n_slices=16, anchor_xy=None, K=None,
                       table=None):
    """Anchored pair sums for trajectory motion (no counterpart in the reference, whose exact pair sums need
    motion linear at the event, atl/objectives/ats.py:77-78).  Source j moves on its trajectory
    q_j(c) = p_j + sum_k coef_jk g_k(c); seen from an anchor i of slice s (c_s its centre, at_i = t_i - c_s) it
    sits at q_j(c_s) + q_j'(c_s) at_i, the trajectory linearised at the slice centre (exact for straight
    trajectories, where the sum is the reference's).  S_i sums exp(-|x_i - that|^2 / 2h^2) over j != i of the
    same batch with |t_i - t_j| <= tau and distance <= cut h (the reference's tests, fp32 order).
    ``coef`` (N, 2K) rows [y_1..y_K, x_1..x_K], ``table`` (S, 2K) = [g_k(c_s), g_k'(c_s)], ``anchor_xy``
    (M, 2) the anchor positions (required).  Gradients flow to ``p`` and ``coef``.  CPU tensors: the O(MN)
    torch reference."""
    if anchor_xy is None:
        raise ValueError("ats_pair_sums_traj needs anchor_xy")
    K = int(K if K is not None else coef.shape[1] // 2)
    if not ext_supports(p):
        if anchors is None:
            anchors = torch.arange(p.shape[0], device=p.device)
        return ref.ats_pair_sums_traj(p.float(), coef.float(), t.float(), b, anchors, anchor_xy.float(), h, tau,
                                      cut, int(n_slices), table.float())
    if not 1 <= K <= TRAJ_PAIR_MAX_K:
        raise ValueError(f"ats_pair_sums_traj: K = {K} outside 1..{TRAJ_PAIR_MAX_K}")
    get_ext()
    return _ATSPairTraj.apply(p.float(), coef.float(), t.detach(), b, anchors, anchor_xy, int(B), int(H), int(W),
                              float(h), float(tau), float(cut), int(n_slices), K, table)


def pair_counts(plan: PairPlan, h, tau, cut) -> torch.Tensor:
    """n_i: number of contributing pairs of every anchor of a device plan (instrumented forward)."""
    p = plan
    cnt = torch.zeros(p.anc_x.shape[0], dtype=torch.int32, device=p.anc_x.device)
    get_ext().ats_pair_fwd(p.src_y, p.src_v, p.src_t, p.src_id, p.cell_start, p.anc_x, p.anc_t, p.anc_cell,
                           p.anc_id, p.slice_c, p.S, p.GH, p.GW, h, tau, cut, count=cnt)
    return cnt


# ------------------------------------------------------------------------------------------- window counts
def events_sorted(t: torch.Tensor, b: torch.Tensor) -> bool:
    """True if the keys b*4 + t ascend in event order (device check, one host sync)."""
    t, b = _f32(t), b.contiguous().long()
    flag = torch.empty(1, dtype=torch.int32, device=t.device)
    with torch.cuda.device(t.device):
        call("atl_check_sorted", ptr(t), ptr(b), t.shape[0], ptr(flag), stream_of(t))
    return int(flag.item()) == 0


def window_counts(t: torch.Tensor, b: torch.Tensor, idx: torch.Tensor, tau: float,
                  assume_sorted: Optional[bool] = None) -> torch.Tensor:
    """#{j != i, same batch, |t_j - t_i| <= tau} for i in idx (atl/ops/functional.py:210-217); ``idx=None``
    means every event, in order.

    Device path: binary searches over the float64 keys b*4 + t in event order, which the EventPacket
    invariant (sorted by (b, t)) keeps ascending; ``assume_sorted=None`` verifies that first, an unsorted
    input is sorted (by key) before the search."""
    if not t.is_cuda:
        key = b.double() * 4.0 + t.double()
        ks, _ = torch.sort(key)
        ki = key if idx is None else key[idx]
        lo = torch.searchsorted(ks, ki - tau, right=False)
        hi = torch.searchsorted(ks, ki + tau, right=True)
        return (hi - lo - 1).clamp(min=0).to(t.dtype)
    get_ext()
    t, b = _f32(t), b.contiguous().long()
    if assume_sorted is None:
        assume_sorted = events_sorted(t, b)
    if idx is None and not assume_sorted:
        idx = torch.arange(t.shape[0], device=t.device)
    idx = None if idx is None else idx.contiguous().long()
    if not assume_sorted:
        key = b.double() * 4.0 + t.double()
        order = torch.argsort(key, stable=True)
        inv = torch.empty_like(order)
        inv[order] = torch.arange(order.numel(), device=order.device)
        t, b, idx = t[order].contiguous(), b[order].contiguous(), inv[idx].contiguous()
    M = t.shape[0] if idx is None else idx.shape[0]
    out = torch.empty(M, dtype=F32, device=t.device)
    with torch.cuda.device(t.device):
        call("atl_window_counts", ptr(t), ptr(b), t.shape[0], ptr(idx), M, float(tau), ptr(out), stream_of(t))
    return out


# ------------------------------------------------------------------------------------------- exposure
_CENTRES = {}


def bin_centres(n_check: int, device) -> torch.Tensor:
    """0.5 (e_k + e_{k+1}) of linspace(0, 1, n_check + 1) in fp32 (atl/objectives/ats.py:37-38)."""
    key = (int(n_check), str(device))
    c = _CENTRES.get(key)
    if c is None:
        edges = torch.linspace(0, 1, n_check + 1)
        c = (0.5 * (edges[:-1] + edges[1:])).to(device)
        _CENTRES[key] = c
    return c


def event_noise(xy: torch.Tensor, seed: int, offset: int, h: float, dequantize: bool = True,
                smooth: bool = True):
    """Dequantised positions xs = xy + U(-1/2, 1/2) and smoothed anchor positions xa = xs + h N(0, 1), per
    coordinate, drawn in one device pass (Philox4x32-10 keyed by ``seed``, counter (event, ``offset``); the
    noise of atl/objectives/ats.py:79-84, not its random numbers).  Returns (xs, xa), xa None without
    ``smooth``.  No gradient flows to ``xy``."""
    get_ext()
    xy = _f32(xy.detach())
    if xy.dim() != 2 or xy.shape[1] != 2:
        raise ValueError("xy must be (N, 2)")
    xs = torch.empty_like(xy)
    xa = torch.empty_like(xy) if smooth else None
    with torch.cuda.device(xy.device):
        call("atl_event_noise", ptr(xy), xy.shape[0], int(seed) & (2 ** 64 - 1), int(offset) & (2 ** 64 - 1),
             float(h), int(bool(dequantize)), ptr(xs), ptr(xa), stream_of(xy))
    return xs, xa


def bin_counts(t_all, b_all, B, n_check=16, assume_sorted: bool = False) -> torch.Tensor:
    """Events per (batch, time bin) (atl/objectives/ats.py:37-41): a (B, n_check) float tensor.  With events
    sorted by (b, t) the counts come from binary searches for the bin edges; otherwise from a pass with
    atomics."""
    t_all, b_all = _f32(t_all), b_all.contiguous().long()
    dev = t_all.device
    with torch.cuda.device(dev):
        if assume_sorted:
            counts = torch.empty(B, n_check, dtype=F32, device=dev)
            call("atl_bin_counts_sorted", ptr(t_all), ptr(b_all), t_all.shape[0], B, n_check, ptr(counts),
                 stream_of(t_all))
        else:
            counts = torch.zeros(B, n_check, dtype=F32, device=dev)
            call("atl_bin_counts", ptr(t_all), ptr(b_all), t_all.shape[0], B, n_check, ptr(counts), stream_of(t_all))
    return counts


def visible_fraction_linear(xa, va, ta, ba, t_all, b_all, B, H, W, tau, n_check=16, assume_sorted: bool = False):
    """Exposure correction of atl/objectives/ats.py:31-50 for motion linear at the event: anchors (xa, ta, ba)
    with velocities ``va`` transported to the n_check bin centres.  ``assume_sorted``: the events (t_all,
    b_all) are sorted by (b, t).  No grad."""
    dev = xa.device
    xa, va, ta, ba = _f32(xa), _f32(va), _f32(ta), ba.contiguous().long()
    counts = bin_counts(t_all, b_all, B, n_check, assume_sorted)
    out = torch.empty(ta.shape[0], dtype=F32, device=dev)
    centres = bin_centres(n_check, dev)
    with torch.cuda.device(dev):
        st = stream_of(xa)
        call("atl_visible_fraction", ptr(xa), ptr(va), ptr(ta), ptr(ba), ta.shape[0], ptr(counts), ptr(centres), B,
             n_check, float(tau), int(H), int(W), ptr(out), st)
    return out


def traj_visible_fraction(fld, K: int, basis: str, n_fp: int, offset: float, tile: int, xa, ta, ba, t_all, b_all, B,
                          H, W, tau, n_check=16, assume_sorted: bool = False):
    """Exposure correction for PixelTrajectories (atl/objectives/ats.py:31-50) in one pass: each anchor's
    trajectory start (n_fp Picard steps), its coefficients from ``fld`` (B, 2K, Hg, Wg; the model's tile-centre
    grid) looked up once, the trajectory at the n_check bin centres; bit-identical to origin, then displacement per
    centre.  No grad."""
    dev = xa.device
    fld = _f32(fld.detach())
    B_, C, Hg, Wg = fld.shape
    if C != 2 * int(K) or K > TRAJ_MAX_K or basis not in TRAJ_BASES:
        raise ValueError(f"traj_visible_fraction: coefficient grid of {C} channels, K = {K}, basis {basis!r}")
    xa, ta, ba = _f32(xa.detach()), _f32(ta), ba.contiguous().long()
    counts = bin_counts(t_all, b_all, B, n_check, assume_sorted)
    edges = torch.linspace(0, 1, n_check + 1, device=dev)
    centres = (0.5 * (edges[:-1] + edges[1:])).contiguous()
    out = torch.empty(ta.shape[0], dtype=F32, device=dev)
    with torch.cuda.device(dev):
        call("atl_traj_visible", ptr(_channels_last(fld)), B_, C, int(K), Hg, Wg, ptr(xa), ptr(ta), ptr(ba),
             ta.shape[0], int(n_fp), float(offset), int(tile), TRAJ_BASES[basis], ptr(counts), ptr(centres), n_check,
             float(tau), int(H), int(W), ptr(out), stream_of(xa))
    return out


class _AnchoredEpilogue(torch.autograd.Function):
    """log(eps + S / (Wn 2 pi h^2)) with Wn = max(count, 1) * vis (atl/objectives/ats.py:92-96)."""

    @staticmethod
    def forward(ctx, S, wc, vis, h, eps):
        S, wc = _f32(S), _f32(wc)
        vis = None if vis is None else _f32(vis)
        M = S.shape[0]
        ls, q, D = (torch.empty(M, dtype=F32, device=S.device) for _ in range(3))
        with torch.cuda.device(S.device):
            call("atl_anchored_epilogue_fwd", ptr(S), ptr(wc), ptr(vis), M, float(h), float(eps), ptr(ls), ptr(q),
                 ptr(D), stream_of(S))
        ctx.save_for_backward(q, D)
        return ls

    @staticmethod
    def backward(ctx, g):
        q, D = ctx.saved_tensors
        gS = torch.empty_like(q)
        g = g.contiguous().float()
        with torch.cuda.device(q.device):
            call("atl_anchored_epilogue_bwd", ptr(g), ptr(q), ptr(D), q.shape[0], ptr(gS), stream_of(q))
        return gS, None, None, None, None


def anchored_log_scores(S, wc, vis, h, eps):
    """Device log-score epilogue (gradient to S only)."""
    get_ext()
    return _AnchoredEpilogue.apply(S, wc, vis, h, eps)


def _mean_scratch(dev):
    """Per-block partial sums of the fused loss (8 KB, allocated per call from torch's caching allocator)."""
    return torch.empty(int(load_library().atl_anchored_score_mean_scratch_bytes()), dtype=torch.uint8, device=dev)


class _AnchoredScoreMean(torch.autograd.Function):
    """loss = -mean_i log(eps + S_i / (Wn_i 2 pi h^2)) and the score = -loss in one launch
    (atl/objectives/ats.py:92-105); gradient to S only."""

    @staticmethod
    def forward(ctx, S, wc, vis, h, eps):
        S, wc = _f32(S), _f32(wc)
        vis = None if vis is None else _f32(vis)
        M = S.shape[0]
        q, D = (torch.empty(M, dtype=F32, device=S.device) for _ in range(2))
        out = torch.empty(2, dtype=F32, device=S.device)
        st = stream_of(S)
        with torch.cuda.device(S.device):
            call("atl_anchored_score_mean_fwd", ptr(S), ptr(wc), ptr(vis), M, float(h), float(eps), ptr(q), ptr(D),
                 ptr(_mean_scratch(S.device)), ptr(out), st)
        ctx.save_for_backward(q, D)
        ctx.set_materialize_grads(False)
        loss, score = out[0], out[1]
        ctx.mark_non_differentiable(score)
        return loss, score

    @staticmethod
    def backward(ctx, g, _gscore):
        if g is None:
            return None, None, None, None, None
        q, D = ctx.saved_tensors
        gS = torch.empty_like(q)
        g = g.contiguous().float()
        with torch.cuda.device(q.device):
            call("atl_anchored_score_mean_bwd", ptr(g), ptr(q), ptr(D), q.shape[0], ptr(gS), stream_of(q))
        return gS, None, None, None, None


def anchored_score_mean(S, wc, vis, h, eps):
    """Device loss of the anchored score: (loss, score) with loss = -mean log-score (differentiable w.r.t. S)
    and score = -loss (detached)."""
    get_ext()
    return _AnchoredScoreMean.apply(S, wc, vis, h, eps)


# ------------------------------------------------------------------------------------------- voxel grid
def _standardise_nonzero(rows: torch.Tensor) -> None:
    """In place, per row: the non-zero entries minus their mean, divided by their sample standard deviation
    (n - 1 in the denominator) when it is positive; zero entries stay zero."""
    nz = rows != 0
    n = nz.sum(1, keepdim=True)
    mean = torch.where(nz, rows, 0.0).sum(1, keepdim=True) / n.clamp(min=1)
    dev = torch.where(nz, rows - mean, 0.0)
    sd = ((dev * dev).sum(1, keepdim=True) / (n - 1)).sqrt()      # NaN for a single non-zero entry
    rows.copy_(torch.where(nz, dev / torch.where(sd > 0, sd, 1.0), rows))


def voxel_grid(pos, t, p, b, B, C, H, W, normalize: str | None = "mean_std") -> torch.Tensor:
    """Trilinear polarity voxel grid (B, C, H, W), optionally normalised (atl/ops/functional.py:221-238)."""
    with torch.no_grad():
        if ext_supports(pos):
            vox = get_ext().voxel_grid(_f32(pos), _f32(t), _f32(p), b.contiguous().long(), B, C, H, W)
        else:
            vox = ref.voxel_grid(pos.float(), t.float(), p.float(), b, B, C, H, W)
        if normalize == "mean_std":
            _standardise_nonzero(vox.view(B, -1))
        elif normalize == "max":
            vox = vox / vox.abs().amax(dim=(1, 2, 3), keepdim=True).clamp(min=1e-9)
    return vox


# ------------------------------------------------------------------------------ k nearest neighbours
KNN_MAX_K = 32


def _knn_torch(queries: torch.Tensor, pts: torch.Tensor, k: int, chunk: int) -> torch.Tensor:
    """CPU form of knn_indices: (P, n, 2) points -> (P, Q, k), same order as the HIP kernel (fp32 squared distance
    with every operation rounded, ties by the lower index through a stable sort)."""
    P = pts.shape[0]
    out = torch.empty(P, queries.shape[0], k, dtype=torch.int64)
    for s in range(0, queries.shape[0], chunk):
        q = queries[s:s + chunk]
        dx = q[None, :, None, 0] - pts[:, None, :, 0]
        dy = q[None, :, None, 1] - pts[:, None, :, 1]
        d = dx * dx + dy * dy
        out[:, s:s + chunk] = torch.sort(d, dim=-1, stable=True).indices[..., :k]
    return out


def knn_indices(queries: torch.Tensor, points: torch.Tensor, k: int, chunk: int = 4096) -> torch.Tensor:
    """queries (Q, 2), points (B, T, n, 2) -> (B, T, Q, k) int64 indices of the k nearest points per (b, t) plane
    (atl/objectives/mpcm.py:30-42).  Order: squared distance (qx - px)^2 + (qy - py)^2 in fp32, ties by the lower
    index.  On the device one HIP pass (grid-binned ring search); no gradient (the indices select, they do not
    weigh)."""
    if points.dim() != 4 or points.shape[-1] != 2 or queries.dim() != 2 or queries.shape[-1] != 2:
        raise ValueError(f"queries must be (Q, 2) and points (B, T, n, 2), got {tuple(queries.shape)} and "
                         f"{tuple(points.shape)}")
    B, T, n, _ = points.shape
    k = int(k)
    if not 1 <= k <= min(n, KNN_MAX_K):
        raise ValueError(f"k must be in [1, min(n, {KNN_MAX_K})], got k={k} with n={n}")
    q = queries.detach().to(torch.float32).contiguous()
    pts = points.detach().to(torch.float32).reshape(B * T, n, 2).contiguous()
    if not pts.is_cuda:
        return _knn_torch(q.cpu(), pts, k, chunk).view(B, T, -1, k)
    if q.device != pts.device:
        raise ValueError("queries and points must be on the same device")
    Q = q.shape[0]
    out = torch.empty(B, T, Q, k, dtype=torch.int64, device=pts.device)
    nbytes = load_library().atl_knn_ws_bytes(B * T, n)
    if nbytes < 0:
        raise ValueError(f"knn_indices: {B * T} planes of {n} points are too many for 32-bit cell indices")
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=pts.device)
    with torch.cuda.device(pts.device):
        call("atl_knn_indices", ptr(q), Q, ptr(pts), B * T, n, k, ptr(out), ptr(ws), nbytes, stream_of(pts))
    return out
