"""The HIP k-nearest-neighbour pass of MotionPriorCMax's look-up table against the oracle (bit-exact indices, in
order), and the look-up table and loss on the device against the package's CPU path."""
import numpy as np
import pytest
import torch

import oracle as O
from x_amd.ops import functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32 = np.float32


def _knn(q, pts, k):
    """pts (P, n, 2) numpy -> (P, Q, k) from the HIP pass."""
    qt = torch.as_tensor(q, device=DEV)
    pt = torch.as_tensor(pts, device=DEV)[None]
    out = F.knn_indices(qt, pt, k)
    torch.cuda.synchronize()
    return out[0].cpu().numpy()


@pytest.mark.parametrize("k", [1, 5, 8, 9, 16, 17, 32])
def test_knn_random_planes_match_oracle(k):
    print(f"knn random planes k={k}", flush=True)
    rng = np.random.default_rng(k)
    q = (rng.random((1500, 2)) * [160, 120]).astype(F32)
    pts = (rng.random((3, 700, 2)) * [170, 130] - 5).astype(F32)
    assert np.array_equal(_knn(q, pts, k), O.knn_indices(q, pts, k))


def test_knn_ties_on_a_lattice_in_index_order():
    print("knn lattice ties", flush=True)
    gy, gx = np.meshgrid(np.arange(12) * 4.0 + 2, np.arange(16) * 4.0 + 2, indexing="ij")
    pts = np.stack([gx.ravel(), gy.ravel()], 1).astype(F32)[None].repeat(2, 0)
    pts[1] = pts[1][::-1]                                       # same points, reversed indices
    hy, hx = np.meshgrid(np.arange(0, 48, 4) + 1.5, np.arange(0, 64, 4) + 1.5, indexing="ij")
    q = np.stack([hx.ravel(), hy.ravel()], 1).astype(F32)
    for k in (4, 8, 32):
        assert np.array_equal(_knn(q, pts, k), O.knn_indices(q, pts, k))


def test_knn_edge_cases():
    rng = np.random.default_rng(7)
    print("knn: points far outside the query box, coincident points, k = n", flush=True)
    q = (rng.random((300, 2)) * 30).astype(F32)
    pts = np.concatenate([(rng.random((1, 40, 2)) * 30).astype(F32),
                          np.array([[[1e4, 1e4], [-5e3, 7.0], [3.0, -2e4]]], F32),
                          np.full((1, 5, 2), 12.25, F32)], 1)
    for k in (1, 7, 32):
        assert np.array_equal(_knn(q, pts, k), O.knn_indices(q, pts, k))
    small = pts[:, :6]
    assert np.array_equal(_knn(q, small, 6), O.knn_indices(q, small, 6))
    print("knn: a single query, a single point", flush=True)
    assert np.array_equal(_knn(q[:1], pts[:, :1], 1), np.zeros((1, 1, 1), np.int64))
    with pytest.raises(ValueError):
        F.knn_indices(torch.as_tensor(q, device=DEV), torch.as_tensor(pts, device=DEV)[None], 33)


def _smooth_coeffs(B, C, H, W, seed, scale):
    g = torch.Generator().manual_seed(seed)
    c = torch.randn(B, C, H, W, generator=g)
    c = torch.nn.functional.avg_pool2d(c, 31, 1, 15, count_include_pad=False)
    return (c / c.abs().amax() * scale).float()


def test_knn_look_up_table_shape_against_oracle():
    # MotionPriorCMax's DSEC configuration: 480x640, 4 px cells (19200 queries), tile-4 trajectories (19200 points
    # per plane), 15 time bins, 32 neighbours; the oracle checks 2 planes on 1500 queries
    from x_amd.motion import PixelTrajectories
    from x_amd.objectives import MotionPriorCMaxLoss
    print("knn look-up table shape: 15 planes x 19200 points, 19200 queries, k = 32", flush=True)
    coef = _smooth_coeffs(1, 20, 480, 640, 0, 25.0).to(DEV)
    m = PixelTrajectories(coef, 10, "bspline", tile=4)
    loss = MotionPriorCMaxLoss()
    edges = torch.linspace(0, 1, 16, device=DEV)
    mids = (edges[:-1] + edges[1:]) * 0.5
    pts = m.tile_trajectories(mids)[0].contiguous()             # (15, 19200, 2)
    q = loss.cell_centres(480, 640, DEV)
    got = F.knn_indices(q, pts[None], 32)[0]
    torch.cuda.synchronize()
    rng = np.random.default_rng(0)
    sel = rng.choice(q.shape[0], 1500, replace=False)
    for plane in (0, 14):
        want = O.knn_indices(q.cpu().numpy()[sel], pts[plane:plane + 1].cpu().numpy(), 32)[0]
        assert np.array_equal(got[plane].cpu().numpy()[sel], want)


def test_mpcm_loss_device_matches_cpu():
    from x_amd import synth
    from x_amd.core import EventPacket
    from x_amd.motion import PixelTrajectories
    from x_amd.objectives import MotionPriorCMaxLoss
    print("mpcm loss device vs cpu", flush=True)
    win = synth.small_window(seed=4, n=6000, B=2)
    coef = _smooth_coeffs(2, 6, win.height, win.width, 1, 3.0)
    res = {}
    for dev in ("cpu", DEV):
        ev = EventPacket.from_window(win, dev)
        g = coef.clone().to(dev).requires_grad_(True)
        out = MotionPriorCMaxLoss(num_knn=16, t_ref=0.35)(ev, PixelTrajectories(g, 3, "bspline", tile=4))
        out["loss"].backward()
        res[dev] = (float(out["loss"].detach()), g.grad.detach().cpu().numpy())
    (l0, g0), (l1, g1) = res["cpu"], res[DEV]
    assert abs(l1 - l0) <= 1e-5 * abs(l0)
    assert np.abs(g1 - g0).max() <= 1e-4 * np.abs(g0).max()
