"""Pure-torch semantics of every op, differentiable through autograd, for CPU tensors.

This plays the part of the reference's atl/ops/reference.py (its fallback without the extension): device
tensors never come here, they always run on the HIP library.  Each op is written from its defining formula,
vectorised over a small stacked axis (the four bilinear corners, the (2R+1)^2 Gaussian taps) so that one
``index_add`` or one masked gather does the whole scatter or lookup:

* bilinear weights (1 - a, a) per axis at the corners of floor(pos), zero padding   (reference.py:10-28, 46-55)
* truncated Gaussian around round(pos), normalised by 2 pi sigma^2                  (reference.py:31-43)
* brute-force anchored leave-one-out Gaussian sums, O(M N) in anchor chunks         (reference.py:58-71)
* trilinear polarity voxel grid                                                     (reference.py:74-86)
* the trajectory pair sums (slice-linearised transport), O(M N)                     (no counterpart)
"""
from __future__ import annotations

import math

import torch


def _corners(pos: torch.Tensor):
    """(N, 4) column, row and weight of the four corners around floor(pos), ordered (0,0), (1,0), (0,1), (1,1)
    in (dx, dy)."""
    base = torch.floor(pos)
    frac = pos - base
    dx = pos.new_tensor([0.0, 1.0, 0.0, 1.0])
    dy = pos.new_tensor([0.0, 0.0, 1.0, 1.0])
    wx = torch.where(dx.bool(), frac[:, :1], 1 - frac[:, :1])
    wy = torch.where(dy.bool(), frac[:, 1:], 1 - frac[:, 1:])
    col = (base[:, :1] + dx).long()
    row = (base[:, 1:] + dy).long()
    return col, row, wx * wy


def _inside(col, row, H, W):
    return (col >= 0) & (col < W) & (row >= 0) & (row < H)


def splat_bilinear(pos, w, b, B, H, W):
    """img[b, y, x] += w * weight over the in-image corners."""
    col, row, cw = _corners(pos)
    ok = _inside(col, row, H, W)
    flat = (b[:, None] * H + row) * W + col
    vals = w[:, None] * cw
    return pos.new_zeros(B * H * W).index_add(0, flat[ok], vals[ok]).view(B, H, W)


def splat_gauss(pos, w, b, B, H, W, sigma, radius):
    """img += w * exp(-d^2 / 2 sigma^2) / (2 pi sigma^2) over the (2R+1)^2 pixels around round(pos)."""
    r = torch.arange(-radius, radius + 1, device=pos.device)
    oy, ox = torch.meshgrid(r, r, indexing="ij")
    col = torch.round(pos[:, :1]).long() + ox.reshape(1, -1)
    row = torch.round(pos[:, 1:]).long() + oy.reshape(1, -1)
    d2 = (col.to(pos.dtype) - pos[:, :1]) ** 2 + (row.to(pos.dtype) - pos[:, 1:]) ** 2
    vals = w[:, None] * torch.exp(-d2 / (2 * sigma * sigma)) / (2 * math.pi * sigma * sigma)
    ok = _inside(col, row, H, W)
    flat = (b[:, None] * H + row) * W + col
    return pos.new_zeros(B * H * W).index_add(0, flat[ok], vals[ok]).view(B, H, W)


def gather_bilinear(img, pos, b):
    """sum over the in-image corners of weight * img[b, y, x] (zero outside)."""
    B, H, W = img.shape
    col, row, cw = _corners(pos)
    ok = _inside(col, row, H, W)
    flat = (b[:, None] * H + row.clamp(0, H - 1)) * W + col.clamp(0, W - 1)
    return torch.where(ok, cw * img.reshape(-1)[flat], torch.zeros_like(cw)).sum(1)


def _pair_mask(dt, d2, same_batch, not_self, h, tau, cut):
    return same_batch & not_self & (dt.abs() <= tau) & (d2 <= (cut * h) ** 2)


def ats_pair_sums(x, t, v, b, anchors, h, tau, cut=3.0, chunk=2048, anchor_xy=None):
    """S_i = sum_{j != i, same batch, |t_i - t_j| <= tau, |r| <= cut h} exp(-|r|^2 / 2h^2),
    r = x_i - (x_j + v_j (t_i - t_j)); differentiable w.r.t. v (and anchor_xy)."""
    n = t.shape[0]
    ids = torch.arange(n, device=t.device)
    parts = []
    for lo in range(0, anchors.shape[0], chunk):
        a = anchors[lo:lo + chunk]
        xa = x[a] if anchor_xy is None else anchor_xy[lo:lo + chunk]
        dt = t[a][:, None] - t[None, :]                              # (m, n)
        moved = x[None, :, :] + v[None, :, :] * dt[:, :, None]      # sources transported to the anchor times
        r = xa[:, None, :] - moved
        d2 = (r * r).sum(-1)
        keep = _pair_mask(dt, d2, b[a][:, None] == b[None, :], a[:, None] != ids[None, :], h, tau, cut)
        parts.append((torch.exp(-d2 / (2 * h * h)) * keep).sum(1))
    return torch.cat(parts) if parts else x.new_zeros(0)


def ats_pair_sums_traj(p, coef, t, b, anchors, anchor_xy, h, tau, cut, n_slices, table, chunk=1024):
    """The trajectory pair sums by their definition: anchor i of slice s (floor(t_i S) clamped, centre c_s,
    at_i = t_i - c_s) sees source j at y_j(c_s) + v_j(c_s) at_i, with y_j(c) = p_j + sum_k coef_jk g_k(c) and
    v_j(c) = sum_k coef_jk g_k'(c) from the (S, 2K) table; the pair tests are the reference's, and the source
    must have slice s in its range (|t_j - c_s| <= tau + 1 / 2S), as in the plan.  Differentiable w.r.t. p and
    coef."""
    S = int(n_slices)
    K = coef.shape[1] // 2
    delta = 1.0 / S
    n = t.shape[0]
    ids = torch.arange(n, device=t.device)
    cy, cx = coef[:, :K], coef[:, K:]
    # every source's position and velocity at every slice centre: (S, n, 2)
    g, gd = table[:, :K], table[:, K:]
    ys = p[None] + torch.stack([g @ cx.T, g @ cy.T], -1)
    vs = torch.stack([gd @ cx.T, gd @ cy.T], -1)
    lo = torch.ceil((t - tau - delta / 2) / delta - 0.5).clamp(0, S - 1).long()
    hi = torch.floor((t + tau + delta / 2) / delta - 0.5).clamp(0, S - 1).long()
    parts = []
    for c0 in range(0, anchors.shape[0], chunk):
        a = anchors[c0:c0 + chunk]
        ta = t[a]
        s = torch.clamp(torch.floor(ta / delta), 0, S - 1).long()
        at = ta - (s.to(t.dtype) + 0.5) * delta
        r = anchor_xy[c0:c0 + chunk][:, None, :] - (ys[s] + vs[s] * at[:, None, None])
        d2 = (r * r).sum(-1)
        dt = ta[:, None] - t[None, :]
        keep = _pair_mask(dt, d2, b[a][:, None] == b[None, :], a[:, None] != ids[None, :], h, tau, cut)
        keep = keep & (lo[None, :] <= s[:, None]) & (s[:, None] <= hi[None, :])
        parts.append((torch.exp(-d2 / (2 * h * h)) * keep).sum(1))
    return torch.cat(parts) if parts else p.new_zeros(0)


def voxel_grid(pos, t, p, b, B, C, H, W):
    """vox[b, c, y, x] += p * (1 - |c - t (C - 1)|) * bilinear weight, over the two nearest time bins."""
    col, row, cw = _corners(pos)
    tn = t * (C - 1)
    t0 = torch.floor(tn)
    vox = pos.new_zeros(B * C * H * W)
    for step in (0.0, 1.0):
        tb = t0 + step
        wt = 1 - (tb - tn).abs()
        tbl = tb.long()[:, None]
        ok = _inside(col, row, H, W) & (tbl >= 0) & (tbl < C)
        flat = ((b[:, None] * C + tbl) * H + row) * W + col
        vox = vox.index_add(0, flat[ok], ((p * wt)[:, None] * cw)[ok])
    return vox.view(B, C, H, W)
