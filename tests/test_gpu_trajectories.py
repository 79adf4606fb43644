"""Pixel trajectories and the sliced anchored score on the HIP path (the continuous-time workload).

The trajectory model and the sliced score are host compositions (torch) of the fused displacement kernel, the
HIP flow sampler (forward, field adjoint through the tile plan, position gradient), the Gaussian splat and the
bilinear gather.  They run here on the device against the same composition on CPU tensors, where every op is
plain PyTorch (x_amd/ops/reference.py); the fused displacement is also pinned to float64 here, the other
kernels to the oracle in test_gpu_ops.py.  Bars: values
within 1e-5 relative, gradients within 1e-4 relative to the largest magnitude."""
import math

import numpy as np
import pytest
import torch

import oracle as O
from x_amd import synth
from x_amd.core import EventPacket
from x_amd.motion import PixelTrajectories, sample_grid
from x_amd.objectives import AnchoredSliced

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32 = np.float32


def N(t):
    return t.detach().cpu().numpy()


def close_rel(got, want, rel):
    scale = max(float(np.abs(want).max()), 1e-30)
    err = float(np.abs(got.astype(np.float64) - want.astype(np.float64)).max())
    assert err <= rel * scale, f"max err {err:.3e} vs scale {scale:.3e} (rel {err / scale:.2e})"


@pytest.mark.parametrize("C,scale", [(2, False), (3, True), (20, False)])
def test_sample_grid_position_and_field_gradients(C, scale):
    """Flow sampler forward bit-exact vs the oracle; gradients w.r.t. the field (tile plan, C up to 32) and the
    positions (zero where the border clamp is active) vs torch autograd of the same lookup on the CPU."""
    print(f"sample_grid grads C={C} scale={scale}", flush=True)
    rng = np.random.default_rng(C)
    B, Hg, Wg, n = 2, 30, 40, 20000
    H, W = (120, 160) if scale else (Hg, Wg)
    pos = np.stack([rng.uniform(-3, W + 2, n), rng.uniform(-3, H + 2, n)], 1).astype(F32)
    pos[:50] = np.round(pos[:50])                                       # integer corners
    b = rng.integers(0, B, n).astype(np.int64)
    fld = rng.standard_normal((B, C, Hg, Wg)).astype(F32)
    g = rng.standard_normal((n, C)).astype(F32)
    res = {}
    for dev in ("cpu", DEV):
        tf = torch.tensor(fld, device=dev, requires_grad=True)
        tp = torch.tensor(pos, device=dev, requires_grad=True)
        tb = torch.tensor(b, device=dev)
        if scale:
            gp = torch.stack([tp[:, 0] / max(W - 1, 1) * (Wg - 1), tp[:, 1] / max(H - 1, 1) * (Hg - 1)], 1)
            out = sample_grid(tf, gp, tb) if dev == "cpu" else __import__("x_amd").ops.sample_grid_hip(
                tf, tp, tb, img_hw=(H, W))
        else:
            out = sample_grid(tf, tp, tb)
        (out * torch.tensor(g, device=dev)).sum().backward()
        res[dev] = (N(out), N(tf.grad), N(tp.grad))
    if not scale:
        assert np.array_equal(res[DEV][0], O.sample_grid(fld, pos, b)[0])
    close_rel(res[DEV][0], res["cpu"][0], 1e-5)
    close_rel(res[DEV][1], res["cpu"][1], 1e-4)
    close_rel(res[DEV][2], res["cpu"][2], 1e-4)


@pytest.mark.parametrize("K,kind", [(1, "polynomial"), (2, "bezier"), (7, "bezier"), (10, "bezier"),
                                    (16, "polynomial")])
def test_traj_displacement_matches_fp64_and_torch_gradients(K, kind):
    """The fused displacement against the oracle's exact coefficient samples times the basis in float64; its
    field gradient against the float64 adjoint, its position gradient against the CPU torch composition (sample
    the 2K channels, multiply by the basis, sum over k) under autograd; absent batches give zero rows."""
    print(f"traj_displacement K={K} {kind}", flush=True)
    from x_amd.ops import functional as F
    rng = np.random.default_rng(K * 7 + len(kind))
    n, B, Hg, Wg = 5000, 2, 19, 27
    fld = (rng.standard_normal((B, 2 * K, Hg, Wg)) * 2).astype(F32)
    gpos = np.stack([rng.uniform(-2, Wg + 1, n), rng.uniform(-2, Hg + 1, n)], 1).astype(F32)
    b = rng.integers(0, B, n).astype(np.int64)
    b[::89] = B
    t = rng.uniform(0, 1, n).astype(F32)
    t[:4] = [0.0, 1.0, 0.5, 1e-3]
    ok = b < B
    tf = torch.tensor(fld, device=DEV, requires_grad=True)
    tp = torch.tensor(gpos, device=DEV, requires_grad=True)
    d = F.traj_displacement(tf, tp, torch.tensor(b, device=DEV), torch.tensor(t, device=DEV), K, kind)
    coef, idx, wts = O.sample_grid(fld, gpos[ok], b[ok])
    tt = t[ok].astype(np.float64)[:, None]
    k = np.arange(1, K + 1)
    if kind == "bezier":
        g = np.array([math.comb(K, j) for j in k], np.float64) * tt ** k * (1 - tt) ** (K - k)
    else:
        g = tt ** k
    c64 = coef.astype(np.float64)
    want = np.stack([(c64[:, K:] * g).sum(1), (c64[:, :K] * g).sum(1)], 1)
    got = N(d)
    close_rel(got[ok], want, 1e-5)
    assert not got[~ok].any()
    gd = rng.standard_normal((n, 2)).astype(F32)
    d.backward(torch.tensor(gd, device=DEV))
    gout = np.concatenate([g * gd[ok, 1:2], g * gd[ok, 0:1]], 1)
    close_rel(N(tf.grad), O.sample_grid_bwd(gout, idx, wts, fld.shape), 1e-4)
    cf = torch.tensor(fld)
    cp = torch.tensor(gpos[ok], requires_grad=True)
    cc = sample_grid(cf, cp, torch.tensor(b[ok]))
    gk = torch.tensor(g.astype(F32))
    cd = torch.stack([(cc[:, K:] * gk).sum(1), (cc[:, :K] * gk).sum(1)], 1)
    cd.backward(torch.tensor(gd[ok]))
    close_rel(N(tp.grad)[ok], N(cp.grad), 1e-4)
    assert not N(tp.grad)[~ok].any()


def test_traj_displacement_empty_and_rejected_inputs():
    """No events: an empty (0, 2) result and zero gradients; a basis the kernel does not know and times that
    carry a gradient are refused on the host."""
    print("traj_displacement empty", flush=True)
    from x_amd.ops import functional as F
    tf = torch.randn(2, 8, 9, 11, device=DEV, requires_grad=True)
    tp = torch.zeros(0, 2, device=DEV, requires_grad=True)
    tb = torch.zeros(0, dtype=torch.long, device=DEV)
    tt = torch.zeros(0, device=DEV)
    d = F.traj_displacement(tf, tp, tb, tt, 4, "bezier")
    assert d.shape == (0, 2)
    d.sum().backward()
    assert not N(tf.grad).any() and tp.grad.shape == (0, 2)
    with pytest.raises(ValueError):
        F.traj_displacement(tf, tp, tb, tt, 4, "spline")
    with pytest.raises(ValueError):
        F.traj_displacement(tf, tp, tb, tt.clone().requires_grad_(True), 4, "bezier")


@pytest.mark.parametrize("K,kind", [(1, "polynomial"), (3, "bezier"), (4, "polynomial"), (10, "bezier")])
def test_pixel_trajectories_device_matches_cpu(K, kind):
    """Transport (fixed-point origin + displacement) values and coefficient gradients, device vs CPU."""
    print(f"trajectories K={K} {kind}", flush=True)
    win = synth.small_window(seed=K, n=3000, B=2)
    rng = np.random.default_rng(K)
    coeffs = synth.trajectory_coeffs(rng, 2, K, win.height, win.width, sigma_px=8.0, dmax=3.0)
    w = rng.standard_normal((win.n, 2)).astype(F32)
    res = {}
    for dev in ("cpu", DEV):
        ev = EventPacket.from_window(win, dev)
        c = torch.tensor(coeffs, device=dev, requires_grad=True)
        m = PixelTrajectories(c, K, kind)
        y = m.transport(ev.xy, ev.t, 0.7, ev.b)
        (y * torch.tensor(w, device=dev)).sum().backward()
        res[dev] = (N(y), N(c.grad))
    close_rel(res[DEV][0], res["cpu"][0], 1e-5)
    close_rel(res[DEV][1], res["cpu"][1], 1e-4)


def test_pixel_trajectories_linear_closed_form():
    """Degree-1 polynomial trajectories with a constant coefficient field are the linear warp:
    transport(x, t, t') = x + c (t' - t), velocity = c."""
    win = synth.small_window(seed=3, n=2000, B=1)
    ev = EventPacket.from_window(win, DEV)
    c = torch.zeros(1, 2, win.height, win.width, device=DEV)
    c[:, 0] = 1.5                                          # y coefficient
    c[:, 1] = -2.25                                        # x coefficient
    m = PixelTrajectories(c, 1)
    y = N(m.transport(ev.xy, ev.t, 0.25, ev.b))
    want = win.xy + np.array([-2.25, 1.5], F32) * (F32(0.25) - win.t)[:, None]
    assert np.allclose(y, want, atol=1e-5)
    assert np.allclose(N(m.velocity(ev.xy, ev.t, ev.b)), np.array([[-2.25, 1.5]], F32))


@pytest.mark.parametrize("smooth", [True, False])
def test_anchored_sliced_device_matches_cpu(smooth):
    """The sliced anchored score (Gaussian splats, gathers, finite-difference log-det, leave-one-out terms,
    exposure correction) on degree-3 Bezier trajectories: loss and coefficient gradient, device vs CPU, with the
    same CPU-generated noise."""
    print(f"anchored sliced smooth={smooth}", flush=True)
    win = synth.small_window(seed=9, n=4000, B=2)
    rng = np.random.default_rng(9)
    coeffs = synth.trajectory_coeffs(rng, 2, 3, win.height, win.width, sigma_px=8.0, dmax=3.0)
    res = {}
    for dev in ("cpu", DEV):
        ev = EventPacket.from_window(win, dev)
        c = torch.tensor(coeffs, device=dev, requires_grad=True)
        obj = AnchoredSliced(n_slices=6, sigma=1.0, tau=0.3, seed=0, smooth_anchors=smooth)
        out = obj(ev, PixelTrajectories(c, 3, "bezier"))
        out["loss"].backward()
        res[dev] = (float(out["loss"].detach()), N(c.grad))
    assert abs(res[DEV][0] - res["cpu"][0]) <= 1e-5 * abs(res["cpu"][0])
    close_rel(res[DEV][1], res["cpu"][1], 1e-4)
