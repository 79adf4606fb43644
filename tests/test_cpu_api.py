"""The ops API on CPU tensors (pure-torch semantics, as the reference without its extension) agrees with the
oracle; device tensors never take this path."""
import math

import numpy as np
import pytest
import torch

import oracle as O
from tests.conftest import rand_events
from x_amd.ops import functional as F
from x_amd.ops import reference as R

F32 = np.float32


def test_cpu_splat_gather_match_oracle():
    pos, w, b, _ = rand_events(n=600, seed=0)
    img = F.splat(torch.from_numpy(pos), torch.from_numpy(w), torch.from_numpy(b), 2, 20, 24)
    assert np.allclose(img.numpy(), O.splat_bilinear_fwd(pos, w, b, 2, 20, 24), atol=1e-5)
    G = np.random.default_rng(1).standard_normal((2, 20, 24)).astype(F32)
    val = F.gather(torch.from_numpy(G), torch.from_numpy(pos), torch.from_numpy(b))
    assert np.allclose(val.numpy(), O.gather_bilinear_fwd(G, pos, b), atol=1e-5)
    gi = F.splat(torch.from_numpy(pos), torch.from_numpy(w), torch.from_numpy(b), 2, 20, 24, kernel="gauss",
                 sigma=1.3)
    assert np.allclose(gi.numpy(), O.splat_gauss_fwd(pos, w, b, 2, 20, 24, 1.3, int(math.ceil(3.9))), atol=1e-5)


def test_cpu_pair_sums_and_window_counts():
    pos, _, b, t = rand_events(n=500, seed=2)
    v = (np.random.default_rng(3).standard_normal((500, 2)) * 5).astype(F32)
    anchors = np.arange(0, 500, 2)
    S = F.ats_pair_sums(torch.from_numpy(pos), torch.from_numpy(t), torch.from_numpy(v), torch.from_numpy(b), 2, 20,
                        24, torch.from_numpy(anchors), 1.2, 0.3)
    Sb, _, _ = O.pair_sums_fp64(pos, t, v, b, anchors, 1.2, 0.3, 3.0)
    assert np.allclose(S.numpy(), Sb, atol=1e-4, rtol=1e-4)
    wc = F.window_counts(torch.from_numpy(t), torch.from_numpy(b), torch.from_numpy(anchors), 0.1)
    assert np.array_equal(wc.numpy(), O.window_counts(t, b, anchors, 0.1))


def test_reference_module_is_differentiable():
    pos, w, b, _ = rand_events(n=200, seed=4)
    p = torch.from_numpy(pos).requires_grad_(True)
    R.splat_bilinear(p, torch.from_numpy(w), torch.from_numpy(b), 2, 20, 24).pow(2).sum().backward()
    assert p.grad is not None and torch.isfinite(p.grad).all()


def test_cpu_trajectory_pair_sums_match_oracle():
    """The CPU (pure torch) trajectory pair sums against the oracle's float64 brute force: values and the
    gradients to the starts and the coefficient rows."""
    rng = np.random.default_rng(4)
    pos, _, b, t = rand_events(n=500, seed=6)
    K = 4
    coef = (rng.standard_normal((500, 2 * K)) * 2).astype(F32)
    p = (pos - rng.uniform(-1, 1, pos.shape)).astype(F32)
    anchors = np.arange(0, 500, 2)
    xa = (pos[anchors] + rng.standard_normal((250, 2)) * 0.5).astype(F32)
    tab = O.traj_slice_table(K, "bspline", 16)
    tp, tc = torch.from_numpy(p).requires_grad_(True), torch.from_numpy(coef).requires_grad_(True)
    S = F.ats_pair_sums_traj(tp, tc, torch.from_numpy(t), torch.from_numpy(b), 2, 20, 24, torch.from_numpy(anchors),
                             1.2, 0.3, 3.0, 16, anchor_xy=torch.from_numpy(xa), K=K, table=torch.from_numpy(tab))
    S64, _, grad = O.traj_pair_sums_fp64(p, coef, t, b, anchors, xa, 1.2, 0.3, 3.0, 16, K, "bspline")
    assert np.allclose(S.detach().numpy(), S64, rtol=1e-5, atol=1e-5)
    gS = rng.standard_normal(250).astype(F32)
    S.backward(torch.from_numpy(gS))
    gp, gc = grad(gS)
    assert np.allclose(tp.grad.numpy(), gp, rtol=1e-3, atol=1e-4 * np.abs(gp).max())
    assert np.allclose(tc.grad.numpy(), gc, rtol=1e-3, atol=1e-4 * np.abs(gc).max())


def test_cpu_anchored_trajectories_straight_equals_exact():
    """On CPU tensors: straight B-spline trajectories (control points v xi_k) score as AnchoredExact with the
    translation v (same noise)."""
    from x_amd import synth
    from x_amd.core import EventPacket
    from x_amd.motion import PixelTrajectories, Translation
    from x_amd.motion.trajectories import greville
    from x_amd.objectives import AnchoredExact, AnchoredTrajectories
    win = synth.small_window(seed=5, n=1200, B=1)
    ev = EventPacket.from_window(win, "cpu")
    K, v = 6, (-1.5, 2.0)
    xi = torch.tensor(greville(K), dtype=torch.float32)
    c = torch.cat([v[1] * xi, v[0] * xi]).view(1, 2 * K, 1, 1).expand(1, 2 * K, win.height, win.width).contiguous()
    ls_t, _ = AnchoredTrajectories(h=1.0, tau=0.3, n_anchors=None, seed=0).log_scores(
        ev, PixelTrajectories(c, K, "bspline", tile=1))
    ls_e, _ = AnchoredExact(h=1.0, tau=0.3, n_anchors=None, seed=0).log_scores(
        ev, Translation(1, win.height, win.width, init=torch.tensor([v])))
    assert np.allclose(ls_t.detach().numpy(), ls_e.detach().numpy(), rtol=1e-5, atol=1e-5)


def test_cpu_objectives_refuse_the_wrong_motion():
    from x_amd import synth
    from x_amd.core import EventPacket
    from x_amd.motion import PixelTrajectories, Translation
    from x_amd.objectives import AnchoredExact, AnchoredTrajectories
    win = synth.small_window(seed=5, n=300, B=1)
    ev = EventPacket.from_window(win, "cpu")
    traj = PixelTrajectories(torch.zeros(1, 6, win.height, win.width), 3, "bspline")
    with pytest.raises(ValueError):
        AnchoredExact(n_anchors=None)(ev, traj)
    with pytest.raises(ValueError):
        AnchoredTrajectories(n_anchors=None)(ev, Translation(1, win.height, win.width))
    with pytest.raises(ValueError):
        AnchoredExact(rng="gpu")


def test_cpu_knn_indices_match_oracle_and_reject_bad_k():
    rng = np.random.default_rng(3)
    q = torch.as_tensor((rng.random((200, 2)) * 40).astype(np.float32))
    pts = torch.as_tensor((rng.random((2, 3, 90, 2)) * 44 - 2).astype(np.float32))
    got = F.knn_indices(q, pts, 10, chunk=64)
    want = O.knn_indices(q.numpy(), pts.reshape(6, 90, 2).numpy(), 10).reshape(2, 3, 200, 10)
    assert np.array_equal(got.numpy(), want)
    for bad in (0, 33, 91):
        with pytest.raises(ValueError):
            F.knn_indices(q, pts, bad)


def test_cpu_mpcm_loss_runs_and_backprops():
    # the reference's test_objectives.py:86-90 on a synthetic window: K = 1 trajectories from a zero grid
    from x_amd import synth
    from x_amd.core import EventPacket
    from x_amd.motion import PixelTrajectories
    from x_amd.objectives import MotionPriorCMaxLoss
    win = synth.small_window(seed=2, n=3000, B=1)
    ev = EventPacket.from_window(win, "cpu")
    g = torch.zeros(1, 2, ev.height, ev.width, requires_grad=True)
    out = MotionPriorCMaxLoss(num_knn=8, t_ref=0.3)(ev, PixelTrajectories(g, K=1))
    out["loss"].backward()
    assert torch.isfinite(out["loss"]) and g.grad is not None and float(g.grad.abs().sum()) > 0


def test_cpu_voxel_grid_normalisations():
    """voxel_grid's normalisations (atl/ops/functional.py:229-237): "mean_std" gives each batch entry's non-zero
    voxels mean 0 and sample standard deviation 1 (float64 check) and leaves zeros at zero; an entry with one
    non-zero voxel keeps it minus its mean (0); "max" divides each entry by its largest magnitude."""
    pos, _, b, t = rand_events(n=800, B=3, seed=11)
    p = np.where(np.random.default_rng(12).random(800) < 0.5, 1.0, -1.0).astype(F32)
    b[b == 2] = 1                                            # entry 2: empty but for one event
    b[-1] = 2
    pos[-1] = (5.0, 6.0)
    t[-1] = 0.0
    args = [torch.from_numpy(a) for a in (pos, t, p, b)]
    raw = F.voxel_grid(*args, 3, 5, 20, 24, normalize=None).numpy().astype(np.float64)
    got = F.voxel_grid(*args, 3, 5, 20, 24).numpy()
    for k in range(2):
        nz = raw[k] != 0
        want = (raw[k][nz] - raw[k][nz].mean()) / raw[k][nz].std(ddof=1)
        assert np.allclose(got[k][nz], want, atol=1e-5) and np.all(got[k][~nz] == 0)
    assert (raw[2] != 0).sum() == 1 and np.all(got[2] == 0)
    mx = F.voxel_grid(*args, 3, 5, 20, 24, normalize="max").numpy()
    for k in range(3):
        assert np.allclose(mx[k], raw[k] / np.abs(raw[k]).max(), atol=1e-6)
