"""ORACLE — test infrastructure only.

CPU restatement of the reference's event-transport hot path, used to check the HIP library (x_amd) and, in
bench.py, as the timed CPU baseline.  Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline``
leg may import this package; the product path never does and fails loudly without its HIP library.

Two halves:

* ``liboracle.so`` (atl_oracle.cpp): the OpenMP loops of the reference's csrc/atl_cpu.cpp (splat, gather,
  pair sums, voxel grid) on raw pointers, plus an instrumented per-anchor neighbour count.
* NumPy fp32 restatements (this file) of the host-side pieces the reference builds from torch ops:
  ``build_pair_plan`` (atl/ops/functional.py:132-178), ``window_counts`` (:210-217), ``sample_grid`` and
  ``DenseLinearFlow.field`` (atl/motion/parametric.py:212-216, 235-251), ``visible_fraction``
  (atl/objectives/ats.py:31-50) and the anchored-score epilogue and its gradient (ats.py:95-96, 102-105).
* The trajectory pair sums (no reference implementation: the reference's exact pair sums refuse trajectory
  motion): a basis table from library routines (scipy's BSpline), the plan's fp32 entries and an fp64 brute
  force with gradients.
* MotionPriorCMax's look-up table (atl/objectives/mpcm.py:30-42,73-77): brute-force k nearest neighbours by a
  stable sort of fp32 squared distances, and the table's mean.
  NumPy evaluates every fp32 operation separately with IEEE rounding and never fuses, which reproduces
  torch's CPU op-by-op rounding; Python scalars are rounded to fp32 first, as torch does when it combines
  them with fp32 tensors.

Parity pins for every function live in tests/test_oracle.py (fp64 brute force, closed forms, invariants,
the reference's known-answer tests).
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
F32 = np.float32
_LIB = None


def lib():
    """Load (building on first use if needed) the oracle's OpenMP library."""
    global _LIB
    if _LIB is None:
        so = HERE / "liboracle.so"
        if not so.exists():
            subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
        _LIB = ctypes.CDLL(str(so))
        _LIB.oracle_vmax.restype = ctypes.c_float
    return _LIB


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _i(v):
    return ctypes.c_int64(int(v))


def _d(v):
    return ctypes.c_double(float(v))


def _f32c(a):
    return np.ascontiguousarray(a, dtype=F32)


def _i64c(a):
    return np.ascontiguousarray(a, dtype=np.int64)


def num_threads() -> int:
    return int(lib().oracle_num_threads())


# ----------------------------------------------------------------------------------------- splat / gather
def splat_bilinear_fwd(pos, w, b, B, H, W):
    pos, w, b = _f32c(pos), _f32c(w), _i64c(b)
    img = np.zeros((B, H, W), F32)
    lib().oracle_splat_bilinear_fwd(_p(pos), _p(w), _p(b), _i(len(w)), _i(B), _i(H), _i(W), _p(img))
    return img


def splat_bilinear_bwd(gimg, pos, w, b):
    gimg, pos, w, b = _f32c(gimg), _f32c(pos), _f32c(w), _i64c(b)
    gp, gw = np.zeros_like(pos), np.zeros_like(w)
    lib().oracle_splat_bilinear_bwd(_p(gimg), _p(pos), _p(w), _p(b), _i(len(w)), _i(gimg.shape[1]),
                                    _i(gimg.shape[2]), _p(gp), _p(gw))
    return gp, gw


def splat_gauss_fwd(pos, w, b, B, H, W, sigma, R):
    pos, w, b = _f32c(pos), _f32c(w), _i64c(b)
    img = np.zeros((B, H, W), F32)
    lib().oracle_splat_gauss_fwd(_p(pos), _p(w), _p(b), _i(len(w)), _i(H), _i(W), _d(sigma), _i(R), _p(img))
    return img


def splat_gauss_bwd(gimg, pos, w, b, sigma, R):
    gimg, pos, w, b = _f32c(gimg), _f32c(pos), _f32c(w), _i64c(b)
    gp, gw = np.zeros_like(pos), np.zeros_like(w)
    lib().oracle_splat_gauss_bwd(_p(gimg), _p(pos), _p(w), _p(b), _i(len(w)), _i(gimg.shape[1]), _i(gimg.shape[2]),
                                 _d(sigma), _i(R), _p(gp), _p(gw))
    return gp, gw


def gather_bilinear_fwd(img, pos, b):
    img, pos, b = _f32c(img), _f32c(pos), _i64c(b)
    out = np.zeros(pos.shape[0], F32)
    lib().oracle_gather_bilinear_fwd(_p(img), _p(pos), _p(b), _i(pos.shape[0]), _i(img.shape[1]), _i(img.shape[2]),
                                     _p(out))
    return out


def gather_bilinear_bwd(gval, img, pos, b):
    gval, img, pos, b = _f32c(gval), _f32c(img), _f32c(pos), _i64c(b)
    gimg, gp = np.zeros_like(img), np.zeros_like(pos)
    lib().oracle_gather_bilinear_bwd(_p(gval), _p(img), _p(pos), _p(b), _i(pos.shape[0]), _i(img.shape[1]),
                                     _i(img.shape[2]), _p(gimg), _p(gp))
    return gimg, gp


def voxel_grid(pos, t, p, b, B, C, H, W):
    pos, t, p, b = _f32c(pos), _f32c(t), _f32c(p), _i64c(b)
    vox = np.zeros((B, C, H, W), F32)
    lib().oracle_voxel_grid(_p(pos), _p(t), _p(p), _p(b), _i(len(t)), _i(C), _i(H), _i(W), _p(vox))
    return vox


# ----------------------------------------------------------------------------------------- pair plan
def vmax(v) -> float:
    """max_j ||v_j|| with torch's CPU rounding, sqrt(fma(vy, vy, vx*vx)) (atl/ops/functional.py:139)."""
    v = _f32c(v).reshape(-1, 2)
    return float(lib().oracle_vmax(_p(v), _i(v.shape[0]))) if v.shape[0] else 0.0


def plan_geometry(vmax_f: float, xa, h, tau, cut, S, W, H):
    """Grid geometry in Python doubles, atl/ops/functional.py:135-149."""
    delta = 1.0 / S
    cell = max(cut * h + vmax_f * delta / 2 + 1e-3, 1.0)
    if xa.shape[0]:
        ox, oy = float(xa[:, 0].min()) - cell, float(xa[:, 1].min()) - cell
        ex, ey = float(xa[:, 0].max()) + cell, float(xa[:, 1].max()) + cell
    else:
        ox, oy, ex, ey = -cell, -cell, W + cell, H + cell
    GW = int(math.ceil((ex - ox) / cell)) + 1
    GH = int(math.ceil((ey - oy) / cell)) + 1
    return dict(delta=delta, cell=cell, ox=ox, oy=oy, GW=GW, GH=GH)


def slice_range(t, tau, S):
    """Per-source slice range [s_lo, s_hi] with |t - c_s| <= tau + delta/2, atl/ops/functional.py:151-152."""
    delta = 1.0 / S
    t = _f32c(t)
    a = ((t - F32(tau)) - F32(delta / 2)) / F32(delta) - F32(0.5)
    c = ((t + F32(tau)) + F32(delta / 2)) / F32(delta) - F32(0.5)
    s_lo = np.clip(np.ceil(a), 0, S - 1).astype(np.int64)
    s_hi = np.clip(np.floor(c), 0, S - 1).astype(np.int64)
    return s_lo, s_hi


def slice_centres(S):
    """(s + 0.5) * delta in fp32, atl/ops/functional.py:157."""
    return (np.arange(S, dtype=F32) + F32(0.5)) * F32(1.0 / S)


def build_pair_plan(x, t, v, b, B, H, W, anchors, h, tau, cut=3.0, n_slices=16, anchor_xy=None):
    """NumPy restatement of atl/ops/functional.py:132-178.  Returns a dict with the PairPlan fields.

    Entries inside one cell come out in ascending source order (a stable sort); the reference's
    ``torch.argsort`` leaves that order unspecified, so plans are compared per cell as multisets."""
    x, t, v, b = _f32c(x), _f32c(t), _f32c(v).reshape(-1, 2), _i64c(b)
    anchors = _i64c(anchors)
    S = int(n_slices)
    delta = 1.0 / S
    xa = x[anchors] if anchor_xy is None else _f32c(anchor_xy)
    geo = plan_geometry(vmax(v), xa, h, tau, cut, S, W, H)
    cell, ox, oy, GW, GH = geo["cell"], geo["ox"], geo["oy"], geo["GW"], geo["GH"]
    s_lo, s_hi = slice_range(t, tau, S)
    cnt = np.clip(s_hi - s_lo + 1, 0, None)
    rep = np.repeat(np.arange(t.shape[0], dtype=np.int64), cnt)
    start = np.cumsum(cnt) - cnt
    s = s_lo[rep] + (np.arange(rep.shape[0], dtype=np.int64) - start[rep])
    cs_all = slice_centres(S)
    y = x[rep] + v[rep] * (cs_all[s] - t[rep])[:, None]
    cx = np.floor((y[:, 0] - F32(ox)) / F32(cell)).astype(np.int64)
    cy = np.floor((y[:, 1] - F32(oy)) / F32(cell)).astype(np.int64)
    keep = (cx >= 0) & (cx < GW) & (cy >= 0) & (cy < GH)
    rep, s, y, cx, cy = rep[keep], s[keep], y[keep], cx[keep], cy[keep]
    key = ((b[rep] * S + s) * GH + cy) * GW + cx
    order = np.argsort(key, kind="stable")
    key, rep, y = key[order], rep[order], y[order]
    ncell = B * S * GH * GW
    counts = np.bincount(key, minlength=ncell)
    cell_start = np.concatenate([np.zeros(1, np.int64), np.cumsum(counts)]).astype(np.int64)
    ta = t[anchors]
    sa = np.clip(np.floor(ta / F32(delta)), 0, S - 1).astype(np.int64)
    acx = np.clip(np.floor((xa[:, 0] - F32(ox)) / F32(cell)).astype(np.int64), 0, GW - 1)
    acy = np.clip(np.floor((xa[:, 1] - F32(oy)) / F32(cell)).astype(np.int64), 0, GH - 1)
    anc_cell = np.stack([b[anchors] * S + sa, acx, acy], 1).astype(np.int64)
    return dict(src_y=np.ascontiguousarray(y), src_v=np.ascontiguousarray(v[rep]),
                src_t=np.ascontiguousarray(t[rep]), src_id=np.ascontiguousarray(rep), cell_start=cell_start,
                anc_x=np.ascontiguousarray(xa), anc_t=np.ascontiguousarray(ta), anc_cell=np.ascontiguousarray(anc_cell),
                anc_id=anchors.copy(), slice_c=cs_all, S=S, GH=GH, GW=GW, key=key, geometry=geo)


def build_pair_plan_torch(x, t, v, b, B, H, W, anchors, h, tau, cut=3.0, n_slices=16, anchor_xy=None):
    """The same plan built with torch CPU ops in the reference's sequence (atl/ops/functional.py:132-178:
    repeat_interleave, floor, argsort, bincount, cumsum), as the reference builds it on CPU tensors; returned as
    build_pair_plan's dict of NumPy arrays (zero-copy views) for the OpenMP pair loops.  Used to time the CPU
    baseline; keys and cell offsets equal build_pair_plan's."""
    import torch
    x, t, v = (torch.from_numpy(_f32c(a)) for a in (x, t, v))
    v = v.reshape(-1, 2)
    b, anchors = torch.from_numpy(_i64c(b)), torch.from_numpy(_i64c(anchors))
    S = int(n_slices)
    delta = 1.0 / S
    xa = x[anchors] if anchor_xy is None else torch.from_numpy(_f32c(anchor_xy))
    vmax_f = float(torch.linalg.vector_norm(v, dim=1).max()) if v.shape[0] else 0.0
    geo = plan_geometry(vmax_f, xa.numpy(), h, tau, cut, S, W, H)
    cell, ox, oy, GW, GH = geo["cell"], geo["ox"], geo["oy"], geo["GW"], geo["GH"]
    s_lo = torch.ceil((t - tau - delta / 2) / delta - 0.5).clamp(0, S - 1).long()
    s_hi = torch.floor((t + tau + delta / 2) / delta - 0.5).clamp(0, S - 1).long()
    cnt = (s_hi - s_lo + 1).clamp(min=0)
    rep = torch.repeat_interleave(torch.arange(t.numel()), cnt)
    first = torch.cumsum(cnt, 0) - cnt
    s = s_lo[rep] + (torch.arange(rep.numel()) - first[rep])
    cs = (torch.arange(S, dtype=torch.float32) + 0.5) * delta
    y = x[rep] + v[rep] * (cs[s] - t[rep])[:, None]
    cx = torch.floor((y[:, 0] - ox) / cell).long()
    cy = torch.floor((y[:, 1] - oy) / cell).long()
    keep = (cx >= 0) & (cx < GW) & (cy >= 0) & (cy < GH)
    rep, s, y, cx, cy = rep[keep], s[keep], y[keep], cx[keep], cy[keep]
    key = ((b[rep] * S + s) * GH + cy) * GW + cx
    order = torch.argsort(key, stable=True)
    key, rep, y = key[order], rep[order], y[order]
    counts = torch.bincount(key, minlength=B * S * GH * GW)
    cell_start = torch.cat([counts.new_zeros(1), torch.cumsum(counts, 0)])
    ta = t[anchors]
    sa = torch.clamp(torch.floor(ta / delta), 0, S - 1).long()
    acx = torch.floor((xa[:, 0] - ox) / cell).long().clamp(0, GW - 1)
    acy = torch.floor((xa[:, 1] - oy) / cell).long().clamp(0, GH - 1)
    anc_cell = torch.stack([b[anchors] * S + sa, acx, acy], 1)
    n = lambda a: np.ascontiguousarray(a.numpy())
    return dict(src_y=n(y), src_v=n(v[rep]), src_t=n(t[rep]), src_id=n(rep), cell_start=n(cell_start),
                anc_x=n(xa), anc_t=n(ta), anc_cell=n(anc_cell), anc_id=n(anchors), slice_c=n(cs), S=S, GH=GH, GW=GW,
                key=n(key), geometry=geo)


def ats_pair_fwd(plan, h, tau, cut, with_counts=False):
    p = plan
    M = p["anc_x"].shape[0]
    out = np.zeros(M, F32)
    cnt = np.zeros(M, np.int64) if with_counts else None
    lib().oracle_ats_pair_fwd(_p(p["src_y"]), _p(p["src_v"]), _p(p["src_t"]), _p(p["src_id"]), _p(p["cell_start"]),
                              _p(p["anc_x"]), _p(p["anc_t"]), _p(p["anc_cell"]), _p(p["anc_id"]), _p(p["slice_c"]),
                              _i(M), _i(p["S"]), _i(p["GH"]), _i(p["GW"]), _d(h), _d(tau), _d(cut), _p(out),
                              _p(cnt) if with_counts else ctypes.c_void_p(0))
    return (out, cnt) if with_counts else out


def ats_pair_bwd(gS, plan, h, tau, cut, N):
    p = plan
    gS = _f32c(gS)
    M = p["anc_x"].shape[0]
    gv = np.zeros((N, 2), F32)
    lib().oracle_ats_pair_bwd(_p(gS), _p(p["src_y"]), _p(p["src_v"]), _p(p["src_t"]), _p(p["src_id"]),
                              _p(p["cell_start"]), _p(p["anc_x"]), _p(p["anc_t"]), _p(p["anc_cell"]), _p(p["anc_id"]),
                              _p(p["slice_c"]), _i(M), _i(p["S"]), _i(p["GH"]), _i(p["GW"]), _d(h), _d(tau), _d(cut),
                              _p(gv))
    return gv


def window_counts(t, b, idx, tau):
    """#{j != i, same batch, |t_j - t_i| <= tau}: float64 keys b*4 + t, atl/ops/functional.py:210-217."""
    key = _i64c(b).astype(np.float64) * 4.0 + _f32c(t).astype(np.float64)
    ks = np.sort(key)
    ki = key[_i64c(idx)]
    lo = np.searchsorted(ks, ki - tau, side="left")
    hi = np.searchsorted(ks, ki + tau, side="right")
    return np.clip(hi - lo - 1, 0, None).astype(F32)


# ----------------------------------------------------------------------------------------- motion pieces
def sample_grid(field, gpos, b):
    """Bilinear, border-clamped sample of a (B, C, Hg, Wg) field, atl/motion/parametric.py:235-251.
    Returns (values (N, C), corner indices (N, 4) into the flattened (B*Hg*Wg) plane, weights (N, 4))."""
    field, gpos, b = _f32c(field), _f32c(gpos), _i64c(b)
    B, C, Hg, Wg = field.shape
    gx = np.clip(gpos[:, 0], F32(0), F32(Wg - 1))
    gy = np.clip(gpos[:, 1], F32(0), F32(Hg - 1))
    x0 = np.minimum(np.floor(gx), F32(max(Wg - 2, 0)))
    y0 = np.minimum(np.floor(gy), F32(max(Hg - 2, 0)))
    ax, ay = gx - x0, gy - y0
    x0, y0 = x0.astype(np.int64), y0.astype(np.int64)
    x1, y1 = np.minimum(x0 + 1, Wg - 1), np.minimum(y0 + 1, Hg - 1)
    f = np.ascontiguousarray(field.transpose(0, 2, 3, 1).reshape(-1, C))
    base = b * (Hg * Wg)
    idx = np.stack([base + y0 * Wg + x0, base + y0 * Wg + x1, base + y1 * Wg + x0, base + y1 * Wg + x1], 1)
    one = F32(1)
    wts = np.stack([(one - ax) * (one - ay), ax * (one - ay), (one - ax) * ay, ax * ay], 1)
    out = f[idx[:, 0]] * wts[:, 0:1]
    out = out + f[idx[:, 1]] * wts[:, 1:2]
    out = out + f[idx[:, 2]] * wts[:, 2:3]
    out = out + f[idx[:, 3]] * wts[:, 3:4]
    return out, idx, wts


def dense_grid_pos(xy, H, W, Hg, Wg):
    """Grid coordinates of DenseLinearFlow.field, atl/motion/parametric.py:214-215."""
    xy = _f32c(xy)
    gx = xy[:, 0] / F32(max(W - 1, 1)) * F32(Wg - 1)
    gy = xy[:, 1] / F32(max(H - 1, 1)) * F32(Hg - 1)
    return np.stack([gx, gy], 1)


def dense_velocity(grid, xy, b, H, W):
    """DenseLinearFlow.field(xy, b) (atl/motion/parametric.py:212-216)."""
    Hg, Wg = grid.shape[-2:]
    return sample_grid(grid, dense_grid_pos(xy, H, W, Hg, Wg), b)


def sample_grid_bwd(gout, idx, wts, shape):
    """Adjoint of sample_grid w.r.t. the field: index_put accumulate of g * w into each corner (fp64 sum)."""
    B, C, Hg, Wg = shape
    acc = np.zeros((B * Hg * Wg, C), np.float64)
    for k in range(4):
        np.add.at(acc, idx[:, k], gout.astype(np.float64) * wts[:, k:k + 1].astype(np.float64))
    return acc.reshape(B, Hg, Wg, C).transpose(0, 3, 1, 2).astype(F32)


def visible_fraction_dense(grid, xa, ta, ba, t_all, b_all, B, H, W, tau, n_check=16):
    """Exposure correction for a linear dense-flow motion, atl/objectives/ats.py:31-50."""
    xa, ta, ba = _f32c(xa), _f32c(ta), _i64c(ba)
    t_all, b_all = _f32c(t_all), _i64c(b_all)
    edges = np.linspace(0, 1, n_check + 1).astype(F32)
    centres = F32(0.5) * (edges[:-1] + edges[1:])
    sl = np.clip((t_all * F32(n_check)).astype(np.int64), 0, n_check - 1)
    counts = np.zeros((B, n_check), F32)
    np.add.at(counts, (b_all, sl), F32(1))
    va, _, _ = dense_velocity(grid, xa, ba, H, W)
    vis = np.zeros_like(ta)
    tot = np.zeros_like(ta)
    for k in range(n_check):
        c = F32(float(centres[k]))
        near = (np.abs(ta - c) <= F32(tau)).astype(F32)
        dt = c - ta
        y = xa + va * dt[:, None]
        inside = ((y[:, 0] >= 0) & (y[:, 0] <= W - 1) & (y[:, 1] >= 0) & (y[:, 1] <= H - 1)).astype(F32)
        w = counts[ba, k] * near
        vis = vis + w * inside
        tot = tot + w
    return np.maximum(vis / np.maximum(tot, F32(1)), F32(1e-3))


def anchored_epilogue(S, wc, h, H, W, eps_frac=1e-2, vis=None):
    """log(eps + S / (Wn * 2 pi h^2)) with Wn = max(wc, 1) [* vis] (atl/objectives/ats.py:92-96) and
    d(-mean)/dS (ats.py:102-105)."""
    S = _f32c(S)
    Wn = np.maximum(_f32c(wc), F32(1))
    if vis is not None:
        Wn = Wn * _f32c(vis)
    eps = F32(eps_frac / (H * W))
    D = ((Wn * F32(2)) * F32(math.pi)) * F32(h ** 2)
    q = eps + S / D
    ls = np.log(q)
    g = F32(-1.0) / F32(S.shape[0])
    gS = (g / q) / D
    return ls, gS, D


# ----------------------------------------------------------------------------------------- brute force
def pair_sums_fp64(x, t, v, b, anchors, h, tau, cut, anchor_xy=None, chunk=512):
    """fp64 brute force of the defining sum (atl/ops/reference.py:58-71) and its gradient kernel:
    returns S (M,), count (M,), and a function gS -> gv (N, 2)."""
    x, t, v = (np.asarray(a, np.float64) for a in (x, t, v))
    b = np.asarray(b)
    anchors = np.asarray(anchors, np.int64)
    xa_all = x[anchors] if anchor_xy is None else np.asarray(anchor_xy, np.float64)
    M, N = anchors.shape[0], t.shape[0]
    S = np.zeros(M)
    cnt = np.zeros(M, np.int64)
    blocks = []
    for s0 in range(0, M, chunk):
        a = anchors[s0:s0 + chunk]
        xa = xa_all[s0:s0 + chunk]
        dt = t[a][:, None] - t[None, :]
        r = xa[:, None, :] - x[None] - v[None] * dt[..., None]
        d2 = (r * r).sum(-1)
        ok = (b[a][:, None] == b[None]) & (np.abs(dt) <= tau) & (d2 <= (cut * h) ** 2)
        ok &= a[:, None] != np.arange(N)[None]
        k = np.where(ok, np.exp(-d2 / (2 * h * h)), 0.0)
        S[s0:s0 + chunk] = k.sum(1)
        cnt[s0:s0 + chunk] = ok.sum(1)
        blocks.append((s0, k, r, dt))

    def grad(gS):
        gS = np.asarray(gS, np.float64)
        gv = np.zeros((N, 2))
        for s0, k, r, dt in blocks:
            f = gS[s0:s0 + k.shape[0], None] * k * dt / (h * h)
            gv[:, 0] += (f * r[..., 0]).sum(0)
            gv[:, 1] += (f * r[..., 1]).sum(0)
        return gv

    return S, cnt, grad


def near_boundary_pairs(x, t, v, b, anchors, h, tau, cut, anchor_xy=None, rel=1e-5):
    """Per-anchor count of pairs whose fp64 d^2 or |dt| lies within ``rel`` of a cut-off: fp32 evaluation order
    may legitimately decide those either way, so exact counts are compared modulo them."""
    x, t, v = (np.asarray(a, np.float64) for a in (x, t, v))
    b = np.asarray(b)
    anchors = np.asarray(anchors, np.int64)
    xa = x[anchors] if anchor_xy is None else np.asarray(anchor_xy, np.float64)
    dt = t[anchors][:, None] - t[None, :]
    r = xa[:, None, :] - x[None] - v[None] * dt[..., None]
    d2 = (r * r).sum(-1)
    r2 = (cut * h) ** 2
    same = b[anchors][:, None] == b[None]
    amb = same & ((np.abs(d2 - r2) <= rel * r2) | (np.abs(np.abs(dt) - tau) <= rel * max(tau, 1e-6)))
    return amb.sum(1)


# ----------------------------------------------------------------------------------------- trajectories
# The trajectory pair sums have no reference implementation: atl/objectives/ats.py:77-78 refuses motion that
# is not linear at the event.  Their definition (the reference's pair sum with each source's transport to the
# anchor time replaced by its trajectory linearised at the anchor's slice centre) is restated here twice: in
# fp32 with the plan's operation order (for bit-exact neighbour counts through the C++ pair loops above) and
# in float64 by brute force (values and gradients).
def traj_basis_table(times, K, kind):
    """Float64 g_1..g_K and their time derivatives at ``times`` (two (n, K) arrays), from library routines:
    scipy's BSpline for the clamped uniform B-spline (degree min(3, K), K + 1 functions, the first pinned to the
    start), closed forms for the polynomial and Bernstein bases (atl/motion/trajectories.py:26-37)."""
    t = np.asarray(times, np.float64)
    if kind == "polynomial":
        k = np.arange(1, K + 1)
        return t[:, None] ** k, k * t[:, None] ** (k - 1)
    if kind == "bezier":
        from scipy.special import comb
        def bern(n, i):
            return comb(n, i) * t ** i * (1 - t) ** (n - i) if 0 <= i <= n else np.zeros_like(t)
        val = np.stack([bern(K, i) for i in range(1, K + 1)], 1)
        der = np.stack([K * (bern(K - 1, i - 1) - bern(K - 1, i)) for i in range(1, K + 1)], 1)
        return val, der
    from scipy.interpolate import BSpline
    P = min(3, K)
    L = K + 1 - P
    knots = np.concatenate([np.zeros(P), np.linspace(0, 1, L + 1), np.ones(P)])
    val, der = np.zeros((t.size, K)), np.zeros((t.size, K))
    for i in range(1, K + 1):
        c = np.zeros(K + 1)
        c[i] = 1.0
        spl = BSpline(knots, c, P, extrapolate=True)
        val[:, i - 1] = spl(t)
        der[:, i - 1] = spl.derivative()(t)
    return val, der


def traj_slice_table(K, kind, S):
    """(S, 2K) float32 table [g_k(c_s), g_k'(c_s)] at the fp32 slice centres (atl/ops/functional.py:157)."""
    val, der = traj_basis_table(slice_centres(S).astype(np.float64), K, kind)
    return np.concatenate([val, der], 1).astype(F32)


def traj_entries(p, coef, tab, t, tau, S):
    """The trajectory plan's (source, slice) entries in fp32 with the kernels' operation order: for s in the
    source's slice range, y = p + sum_k coef_k g_k(c_s) and v = sum_k coef_k g_k'(c_s), each sum in k order
    (channels [y_1..y_K, x_1..x_K]).  Returns (rep, s, y (E, 2), v (E, 2))."""
    p, coef, tab, t = _f32c(p), _f32c(coef), _f32c(tab), _f32c(t)
    K = coef.shape[1] // 2
    s_lo, s_hi = slice_range(t, tau, S)
    cnt = np.clip(s_hi - s_lo + 1, 0, None)
    rep = np.repeat(np.arange(t.shape[0], dtype=np.int64), cnt)
    start = np.cumsum(cnt) - cnt
    s = s_lo[rep] + (np.arange(rep.shape[0], dtype=np.int64) - start[rep])
    cf, row = coef[rep], tab[s]
    dx = np.zeros(rep.shape[0], F32)
    dy, ux, uy = dx.copy(), dx.copy(), dx.copy()
    for k in range(K):
        dy = dy + cf[:, k] * row[:, k]
        dx = dx + cf[:, K + k] * row[:, k]
        uy = uy + cf[:, k] * row[:, K + k]
        ux = ux + cf[:, K + k] * row[:, K + k]
    y = np.stack([p[rep, 0] + dx, p[rep, 1] + dy], 1)
    return rep, s, y, np.stack([ux, uy], 1)


def build_pair_plan_traj(p, coef, tab, t, b, B, H, W, anchors, anchor_xy, h, tau, cut=3.0, n_slices=16):
    """The reference plan (atl/ops/functional.py:132-178, as build_pair_plan) over the trajectory entries: the
    cell size takes vmax over the entries' velocities (so every contributing pair stays within the 3 x 3 cells
    of its anchor).  Its dict runs through ats_pair_fwd (values, counts); the backward of the trajectory model
    is traj_pair_sums_fp64's."""
    t, b = _f32c(t), _i64c(b)
    anchors = _i64c(anchors)
    S = int(n_slices)
    delta = 1.0 / S
    xa = _f32c(anchor_xy)
    rep, s, y, v = traj_entries(p, coef, tab, t, tau, S)
    geo = plan_geometry(vmax(v), xa, h, tau, cut, S, W, H)
    cell, ox, oy, GW, GH = geo["cell"], geo["ox"], geo["oy"], geo["GW"], geo["GH"]
    cx = np.floor((y[:, 0] - F32(ox)) / F32(cell)).astype(np.int64)
    cy = np.floor((y[:, 1] - F32(oy)) / F32(cell)).astype(np.int64)
    keep = (cx >= 0) & (cx < GW) & (cy >= 0) & (cy < GH)
    rep, s, y, v, cx, cy = rep[keep], s[keep], y[keep], v[keep], cx[keep], cy[keep]
    key = ((b[rep] * S + s) * GH + cy) * GW + cx
    order = np.argsort(key, kind="stable")
    key, rep, y, v = key[order], rep[order], y[order], v[order]
    counts = np.bincount(key, minlength=B * S * GH * GW)
    cell_start = np.concatenate([np.zeros(1, np.int64), np.cumsum(counts)]).astype(np.int64)
    ta = t[anchors]
    sa = np.clip(np.floor(ta / F32(delta)), 0, S - 1).astype(np.int64)
    acx = np.clip(np.floor((xa[:, 0] - F32(ox)) / F32(cell)).astype(np.int64), 0, GW - 1)
    acy = np.clip(np.floor((xa[:, 1] - F32(oy)) / F32(cell)).astype(np.int64), 0, GH - 1)
    anc_cell = np.stack([b[anchors] * S + sa, acx, acy], 1).astype(np.int64)
    return dict(src_y=np.ascontiguousarray(y), src_v=np.ascontiguousarray(v), src_t=np.ascontiguousarray(t[rep]),
                src_id=np.ascontiguousarray(rep), cell_start=cell_start, anc_x=np.ascontiguousarray(xa),
                anc_t=np.ascontiguousarray(ta), anc_cell=np.ascontiguousarray(anc_cell), anc_id=anchors.copy(),
                slice_c=slice_centres(S), S=S, GH=GH, GW=GW, key=key, geometry=geo)


def ats_pair_bwd_traj(gS, plan, tab, K, h, tau, cut, N):
    """Gradients (gp (N, 2), gcoef (N, 2K)) of the trajectory pair sums over a build_pair_plan_traj plan, from the
    OpenMP pair loop (float64 accumulation)."""
    p = plan
    gS, tab = _f32c(gS), _f32c(tab)
    M = p["anc_x"].shape[0]
    gp, gc = np.zeros((N, 2)), np.zeros((N, 2 * K))
    lib().oracle_ats_pair_bwd_traj(_p(gS), _p(p["src_y"]), _p(p["src_v"]), _p(p["src_t"]), _p(p["src_id"]),
                                   _p(p["cell_start"]), _p(p["anc_x"]), _p(p["anc_t"]), _p(p["anc_cell"]),
                                   _p(p["anc_id"]), _p(p["slice_c"]), _i(M), _i(p["S"]), _i(p["GH"]), _i(p["GW"]),
                                   _d(h), _d(tau), _d(cut), _p(tab), _i(K), _p(gp), _p(gc))
    return gp, gc


def traj_pair_sums_fp64(p, coef, t, b, anchors, anchor_xy, h, tau, cut, S, K, kind, chunk=256):
    """Float64 brute force of the trajectory pair sums by their definition (basis from traj_basis_table):
    S (M,), count (M,), and a function gS -> (gp (N, 2), gcoef (N, 2K)) of their gradients,
    dS_i/dy = k r / h^2 and dS_i/dv = k r at_i / h^2 chained through y = p + sum coef g, v = sum coef g'."""
    p, coef, t = (np.asarray(a, np.float64) for a in (p, coef, t))
    b = np.asarray(b)
    anchors = np.asarray(anchors, np.int64)
    xa_all = np.asarray(anchor_xy, np.float64)
    N, M = t.shape[0], anchors.shape[0]
    cs = slice_centres(S).astype(np.float64)
    g, gd = traj_basis_table(cs, K, kind)                       # (S, K)
    ys = p[None] + np.stack([g @ coef[:, K:].T, g @ coef[:, :K].T], -1)      # (S, N, 2) in (x, y)
    vs = np.stack([gd @ coef[:, K:].T, gd @ coef[:, :K].T], -1)
    s_lo, s_hi = slice_range(t.astype(F32), tau, S)
    out, cnt = np.zeros(M), np.zeros(M, np.int64)
    blocks = []
    for c0 in range(0, M, chunk):
        a = anchors[c0:c0 + chunk]
        ta = t[a]
        s = np.clip(np.floor(ta * S), 0, S - 1).astype(np.int64)
        at = ta - cs[s]
        r = xa_all[c0:c0 + chunk, None, :] - (ys[s] + vs[s] * at[:, None, None])
        d2 = (r * r).sum(-1)
        dt = ta[:, None] - t[None, :]
        ok = (b[a][:, None] == b[None]) & (np.abs(dt) <= tau) & (d2 <= (cut * h) ** 2)
        ok &= (a[:, None] != np.arange(N)[None]) & (s_lo[None] <= s[:, None]) & (s[:, None] <= s_hi[None])
        k = np.where(ok, np.exp(-d2 / (2 * h * h)), 0.0)
        out[c0:c0 + chunk], cnt[c0:c0 + chunk] = k.sum(1), ok.sum(1)
        blocks.append((c0, s, at, k, r))

    def grad(gS):
        gS = np.asarray(gS, np.float64)
        gp, gc = np.zeros((N, 2)), np.zeros((N, 2 * K))
        for c0, s, at, k, r in blocks:
            f = gS[c0:c0 + k.shape[0], None] * k / (h * h)       # (m, N)
            fy, fv = f[..., None] * r, (f * at[:, None])[..., None] * r     # (m, N, 2): dL/dy, dL/dv per pair
            gp += fy.sum(0)
            # chain: y_x uses the x channels (K..2K), y_y the y channels (0..K)
            gc[:, K:] += np.einsum("mn,mk->nk", fy[..., 0], g[s]) + np.einsum("mn,mk->nk", fv[..., 0], gd[s])
            gc[:, :K] += np.einsum("mn,mk->nk", fy[..., 1], g[s]) + np.einsum("mn,mk->nk", fv[..., 1], gd[s])
        return gp, gc

    return out, cnt, grad


def traj_displacement(coeffs, p, t, b, K, kind):
    """PixelTrajectories.displacement with one trajectory per pixel (atl/motion/trajectories.py:62-66): the 2K
    coefficients sampled at p (sample_grid, fp32) times the float64 basis at t, summed over k; (N, 2) in (x, y),
    and the (N, 2K) rows, corner indices and weights of the look-up."""
    rows, idx, wts = sample_grid(coeffs, p, b)
    g, _ = traj_basis_table(np.asarray(t, np.float64), K, kind)
    r = rows.astype(np.float64)
    d = np.stack([(r[:, K:] * g).sum(1), (r[:, :K] * g).sum(1)], 1).astype(F32)
    return d, rows, idx, wts


def traj_origin(coeffs, xy, t, b, K, kind, n_fixed_point=6):
    """Trajectory start through (xy, t): n_fixed_point steps p <- xy - d(p, t) from p = xy
    (atl/motion/trajectories.py:68-73)."""
    xy = _f32c(xy)
    p = xy
    for _ in range(n_fixed_point):
        p = xy - traj_displacement(coeffs, p, t, b, K, kind)[0]
    return p


def traj_visible_fraction(coeffs, xa, ta, ba, t_all, b_all, B, H, W, tau, K, kind, n_check=16):
    """Exposure correction (atl/objectives/ats.py:31-50) for per-pixel trajectories: each anchor's trajectory
    start found once, the trajectory evaluated at the n_check bin centres."""
    xa, ta, ba = _f32c(xa), _f32c(ta), _i64c(ba)
    t_all, b_all = _f32c(t_all), _i64c(b_all)
    edges = np.linspace(0, 1, n_check + 1).astype(F32)
    centres = F32(0.5) * (edges[:-1] + edges[1:])
    sl = np.clip((t_all * F32(n_check)).astype(np.int64), 0, n_check - 1)
    counts = np.zeros((B, n_check), F32)
    np.add.at(counts, (b_all, sl), F32(1))
    p = traj_origin(coeffs, xa, ta, ba, K, kind)
    vis, tot = np.zeros_like(ta), np.zeros_like(ta)
    for k in range(n_check):
        c = F32(float(centres[k]))
        y = p + traj_displacement(coeffs, p, np.full(ta.shape, c), ba, K, kind)[0]
        inside = ((y[:, 0] >= 0) & (y[:, 0] <= W - 1) & (y[:, 1] >= 0) & (y[:, 1] <= H - 1)).astype(F32)
        w = counts[ba, k] * (np.abs(ta - c) <= F32(tau)).astype(F32)
        vis = vis + w * inside
        tot = tot + w
    return np.maximum(vis / np.maximum(tot, F32(1)), F32(1e-3))


# ----------------------------------------------------------------------------------------- IWE
def blur(img, sigma):
    """Separable Gaussian blur with zero padding (atl/ops/functional.py:91-110): taps exp(-x^2 / 2 sigma^2),
    x = -r..r, r = max(ceil(3 sigma), 1), normalised; scipy.ndimage.correlate1d along each axis in float64."""
    from scipy.ndimage import correlate1d
    if sigma <= 0:
        return np.asarray(img, F32)
    r = max(int(math.ceil(3 * sigma)), 1)
    x = np.arange(-r, r + 1, dtype=np.float64)
    k = np.exp(-x * x / (2 * sigma * sigma))
    k /= k.sum()
    out = correlate1d(np.asarray(img, np.float64), k, axis=-1, mode="constant", cval=0.0)
    return correlate1d(out, k, axis=-2, mode="constant", cval=0.0).astype(F32)


def make_iwe(xy_ref, t, p, b, B, H, W, t_ref, kernel="bilinear", sigma=1.0, polarity="pooled", mask_border=True,
             scale_by_dt=False):
    """Image of warped events (atl/objectives/base.py:40-60): weights 1 [* (1 - |t - t_ref| clamped to [0, 1])]
    [* inside(xy_ref)], split polarity -> batch entries 2b + (p < 0), then the bilinear splat (+ blur) or the
    Gaussian splat of radius ceil(3 sigma)."""
    xy_ref, t, p, b = _f32c(xy_ref), _f32c(t), _f32c(p), _i64c(b)
    w = np.ones(t.shape[0], F32)
    if scale_by_dt:
        w = w * (F32(1) - np.clip(np.abs(t - F32(t_ref)), 0, 1)).astype(F32)
    if mask_border:
        w = w * ((xy_ref[:, 0] >= 0) & (xy_ref[:, 0] <= W - 1) & (xy_ref[:, 1] >= 0)
                 & (xy_ref[:, 1] <= H - 1)).astype(F32)
    nb = B
    if polarity == "split":
        b, nb = 2 * b + (p < 0).astype(np.int64), 2 * B
    if kernel == "gauss":
        return splat_gauss_fwd(xy_ref, w, b, nb, H, W, sigma, int(math.ceil(3 * sigma)))
    return blur(splat_bilinear_fwd(xy_ref, w, b, nb, H, W), sigma)


# ----------------------------------------------------------------------------------- MotionPriorCMax KNN
def knn_indices(queries, points, k):
    """knn_indices (atl/objectives/mpcm.py:30-42): queries (Q, 2), points (P, n, 2) -> (P, Q, k) int64, the k
    nearest points of each plane in the order (squared distance, index): d = (qx - px)^2 + (qy - py)^2 with every
    fp32 operation rounded separately; ties by the lower index (a stable sort of d over the points' order)."""
    q = _f32c(queries).reshape(-1, 2)
    pts = _f32c(points)
    P, n = pts.shape[0], pts.shape[1]
    out = np.empty((P, q.shape[0], k), np.int64)
    for s in range(P):
        dx = q[:, None, 0] - pts[s][None, :, 0]
        dy = q[:, None, 1] - pts[s][None, :, 1]
        d = dx * dx + dy * dy                                  # float32 throughout
        out[s] = np.argsort(d, axis=1, kind="stable")[:, :k]
    return out


def lut_mean(flow_to_ref, idx):
    """The look-up table of MotionPriorCMaxLoss.lut_flow (atl/objectives/mpcm.py:73-77): the mean over the k
    neighbours of their displacement to t_ref.  flow_to_ref (P, n, 2), idx (P, Q, k) -> (P, Q, 2) float32 (fp32
    sum in neighbour order, then the division by k)."""
    f = _f32c(flow_to_ref)
    g = np.stack([f[s][idx[s]] for s in range(f.shape[0])])        # (P, Q, k, 2)
    acc = np.zeros(g.shape[:2] + (2,), np.float32)
    for j in range(g.shape[2]):
        acc = acc + g[:, :, j]
    return acc / np.float32(g.shape[2])
