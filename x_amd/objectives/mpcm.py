"""MotionPriorCMax's loss (atl/objectives/mpcm.py:45-107): the focus of a polarity-split IWE whose events are
displaced by a look-up table, plus a Charbonnier smoothness of that table.

The table (``lut_flow``, mpcm.py:56-78) holds, for every cell of a ``lut`` x ``lut`` pixel grid and every time bin,
the mean displacement to t_ref of the K trajectories nearest to the cell centre at the bin's mid time.  The
nearest-neighbour search is the loss's dominant cost in the reference (a dense distance matrix and a top-k per
plane); here it is one HIP pass over grid-binned points (``x_amd.ops.knn_indices``), and the table's gather and mean
stay torch ops so that the gradient reaches the trajectory coefficients as in the reference.
"""
from __future__ import annotations

import torch

from ..core.events import EventPacket
from ..ops import knn_indices
from .base import IWEConfig, Objective, make_iwe, sobel

__all__ = ["MotionPriorCMaxLoss", "knn_indices", "charbonnier_tv"]


def charbonnier_tv(field: torch.Tensor, eps: float = 1e-3) -> torch.Tensor:
    """Smoothness of a (B, C, H, W) field: the mean Charbonnier penalty sqrt(g^2 + eps^2) of its Sobel gradients,
    averaged over the two directions (atl/objectives/cmax.py:141-145)."""
    B, C, H, W = field.shape
    gx, gy = sobel(field.reshape(B * C, H, W))
    e2 = eps * eps
    return 0.5 * ((gx * gx + e2).sqrt().mean() + (gy * gy + e2).sqrt().mean())


class MotionPriorCMaxLoss(Objective):
    """Focus of the look-up-table IWE (1 / mean of |Sobel_x| + |Sobel_y|, or of the squared gradient magnitude)
    plus ``smooth_weight`` times the Charbonnier smoothness of the table; constructor of the reference."""
    name = "mpcm_focus"

    def __init__(self, num_bins: int = 15, num_knn: int = 32, smooth_weight: float = 0.003, lut: int = 4,
                 t_ref="random", scale_by_dt: bool = True, polarity_split: bool = True, sigma: float = 1.0,
                 focus_norm: str = "l1"):
        if focus_norm not in ("l1", "l2"):
            raise ValueError(f"focus_norm must be 'l1' or 'l2', got {focus_norm!r}")
        self.num_bins, self.num_knn, self.smooth_weight, self.lut = int(num_bins), int(num_knn), smooth_weight, int(lut)
        self.t_ref, self.scale_by_dt, self.polarity_split = t_ref, scale_by_dt, polarity_split
        self.sigma, self.focus_norm = sigma, focus_norm

    def cell_centres(self, H: int, W: int, device) -> torch.Tensor:
        """(Hl * Wl, 2) centres (x, y) of the table's cells, row-major: lut * i + lut / 2 - 1/2."""
        half = self.lut / 2.0 - 0.5
        cy = torch.arange(0, H, self.lut, device=device, dtype=torch.float32) + half
        cx = torch.arange(0, W, self.lut, device=device, dtype=torch.float32) + half
        return torch.cartesian_prod(cy, cx).flip(-1).contiguous()

    def lut_flow(self, motion, H: int, W: int, t_ref: torch.Tensor):
        """Look-up table (B, bins, Hl, Wl, 2) and the bin edges (bins + 1): per cell and bin, the mean of
        q(t_ref) - q(t_mid) over the num_knn trajectories nearest to the cell centre at the bin's mid time t_mid."""
        dev = motion.tile_c.device
        edges = torch.linspace(0, 1, self.num_bins + 1, device=dev)
        mids = (edges[:-1] + edges[1:]) * 0.5
        tr = motion.tile_trajectories(torch.cat([t_ref.reshape(1).to(mids), mids]))   # (B, 1 + bins, n, 2)
        at_ref, at_mid = tr[:, :1], tr[:, 1:]
        centres = self.cell_centres(H, W, dev)
        k = min(self.num_knn, at_mid.shape[2])
        idx = knn_indices(centres, at_mid.detach(), k)                                 # (B, bins, Q, k)
        disp = at_ref - at_mid                                                         # (B, bins, n, 2)
        B, nb, n, _ = disp.shape
        picked = torch.gather(disp.reshape(B * nb, n, 2), 1,
                              idx.reshape(B * nb, -1, 1).expand(-1, -1, 2))            # (B * bins, Q * k, 2)
        table = picked.view(B, nb, -1, k, 2).mean(3)
        Hl, Wl = -(-H // self.lut), -(-W // self.lut)
        return table.view(B, nb, Hl, Wl, 2), edges

    def __call__(self, ev: EventPacket, motion):
        H, W = ev.height, ev.width
        if self.t_ref == "random":
            t_ref = torch.rand((), device=ev.device)
        else:
            t_ref = torch.tensor(float(self.t_ref), device=ev.device)
        table, edges = self.lut_flow(motion, H, W, t_ref)
        nb, Hl, Wl = self.num_bins, table.shape[2], table.shape[3]
        tbin = (torch.searchsorted(edges, ev.t.contiguous()) - 1).clamp(0, nb - 1)
        cy = torch.div(ev.xy[:, 1], self.lut, rounding_mode="floor").long().clamp(0, Hl - 1)
        cx = torch.div(ev.xy[:, 0], self.lut, rounding_mode="floor").long().clamp(0, Wl - 1)
        warped = ev.xy + table[ev.b, tbin, cy, cx]
        cfg = IWEConfig(kernel="bilinear", sigma=self.sigma, polarity="split" if self.polarity_split else "pooled",
                        mask_border=True, scale_by_dt=self.scale_by_dt)
        gx, gy = sobel(make_iwe(ev, warped, t_ref, cfg))
        sharp = (gx.abs() + gy.abs()).mean() if self.focus_norm == "l1" else (gx * gx + gy * gy).mean()
        focus = 1.0 / (sharp + 1e-12)
        if self.smooth_weight > 0:
            field = table.permute(0, 1, 4, 2, 3).reshape(-1, 2, Hl, Wl)
            smooth = self.smooth_weight * charbonnier_tv(field)
        else:
            smooth = focus.new_zeros(())
        return {"loss": focus + smooth, "focus": focus.detach(), "smooth": smooth.detach(), "sharpness": sharp.detach()}
