"""Pure-torch semantics of every op (differentiable through autograd), used for CPU tensors.

Same role as the reference's atl/ops/reference.py (its CPU fallback without the extension); device tensors
never come here, they always run on the HIP library.  Written from the defining formulas:

* bilinear corners of floor(pos) with weights (1-a, a), zero padding        (reference.py:10-28, 46-55)
* truncated Gaussian around round(pos), normalised by 2 pi sigma^2           (reference.py:31-43)
* brute-force anchored leave-one-out Gaussian sums, O(M N)                   (reference.py:58-71)
* trilinear polarity voxel grid                                              (reference.py:74-86)
"""
from __future__ import annotations

import math

import torch


def _bilinear_terms(pos):
    x, y = pos[:, 0], pos[:, 1]
    fx, fy = torch.floor(x), torch.floor(y)
    ax, ay = x - fx, y - fy
    terms = []
    for dy, wy in ((0, 1 - ay), (1, ay)):
        for dx, wx in ((0, 1 - ax), (1, ax)):
            terms.append(((fx + dx).long(), (fy + dy).long(), wx * wy))
    return terms


def splat_bilinear(pos, w, b, B, H, W):
    img = pos.new_zeros(B * H * W)
    for xx, yy, c in _bilinear_terms(pos):
        ok = (xx >= 0) & (xx < W) & (yy >= 0) & (yy < H)
        img = img.index_add(0, (b[ok] * H + yy[ok]) * W + xx[ok], (w * c)[ok])
    return img.view(B, H, W)


def splat_gauss(pos, w, b, B, H, W, sigma, radius):
    img = pos.new_zeros(B * H * W)
    cx, cy = torch.round(pos[:, 0]).long(), torch.round(pos[:, 1]).long()
    scale = 1.0 / (2 * math.pi * sigma * sigma)
    for oy in range(-radius, radius + 1):
        for ox in range(-radius, radius + 1):
            xx, yy = cx + ox, cy + oy
            ok = (xx >= 0) & (xx < W) & (yy >= 0) & (yy < H)
            d2 = (xx.to(pos.dtype) - pos[:, 0]) ** 2 + (yy.to(pos.dtype) - pos[:, 1]) ** 2
            val = w * scale * torch.exp(-d2 / (2 * sigma * sigma))
            img = img.index_add(0, (b[ok] * H + yy[ok]) * W + xx[ok], val[ok])
    return img.view(B, H, W)


def gather_bilinear(img, pos, b):
    B, H, W = img.shape
    flat = img.reshape(-1)
    out = pos.new_zeros(pos.shape[0])
    for xx, yy, c in _bilinear_terms(pos):
        ok = (xx >= 0) & (xx < W) & (yy >= 0) & (yy < H)
        idx = (b * H + yy.clamp(0, H - 1)) * W + xx.clamp(0, W - 1)
        out = out + torch.where(ok, c * flat[idx], torch.zeros_like(c))
    return out


def ats_pair_sums(x, t, v, b, anchors, h, tau, cut=3.0, chunk=2048, anchor_xy=None):
    """S_i = sum_{j != i, same batch, |t_i - t_j| <= tau, |r| <= cut h} exp(-|r|^2 / 2h^2),
    r = x_i - x_j - v_j (t_i - t_j); differentiable w.r.t. v."""
    outs = []
    ids = torch.arange(t.numel(), device=t.device)
    for s in range(0, anchors.numel(), chunk):
        a = anchors[s:s + chunk]
        xa = x[a] if anchor_xy is None else anchor_xy[s:s + chunk]
        dt = t[a][:, None] - t[None, :]
        r = xa[:, None, :] - x[None] - v[None] * dt[..., None]
        d2 = (r * r).sum(-1)
        ok = (b[a][:, None] == b[None]) & (dt.abs() <= tau) & (d2 <= (cut * h) ** 2) & (a[:, None] != ids[None])
        outs.append(torch.where(ok, torch.exp(-d2 / (2 * h * h)), torch.zeros_like(d2)).sum(1))
    return torch.cat(outs) if outs else x.new_zeros(0)


def voxel_grid(pos, t, p, b, B, C, H, W):
    vox = pos.new_zeros(B * C * H * W)
    tn = t * (C - 1)
    t0 = torch.floor(tn)
    for dt in (0, 1):
        tt = (t0 + dt).long()
        wt = 1 - (tt.to(pos.dtype) - tn).abs()
        for xx, yy, c in _bilinear_terms(pos):
            ok = (xx >= 0) & (xx < W) & (yy >= 0) & (yy < H) & (tt >= 0) & (tt < C)
            vox = vox.index_add(0, (((b * C + tt) * H + yy) * W + xx)[ok], (p * wt * c)[ok])
    return vox.view(B, C, H, W)
