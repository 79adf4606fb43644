"""Pixel trajectories and the anchored score for trajectories on the HIP path (the continuous-time workload:
per-pixel cubic B-spline trajectories with 10 control points, 4 windows x 500k events).

* the fused displacement (polynomial, Bernstein and B-spline bases) against float64 (basis from scipy's BSpline
  in the oracle) and the flow sampler's adjoints;
* the trajectory pair sums (atl_fast_plan_traj, atl_fast_pair_fwd, atl_fast_pair_bwd_traj) against the oracle:
  per-anchor neighbour counts bit-exact with the oracle's fp32 plan and pair loops, sums within 1e-5, gradients
  to the starts and coefficients within 1e-4 of the float64 brute force (small) or the oracle's pair loops
  (full size);
* AnchoredTrajectories end to end against the same chain on CPU tensors, and straight trajectories against
  AnchoredExact.
Bars: values within 1e-5 relative, gradients within 1e-4 relative to the largest magnitude."""
import numpy as np
import pytest
import torch

import oracle as O
from tests.conftest import assert_logs_close, assert_sums_close, rand_events
from x_amd import synth
from x_amd.core import EventPacket
from x_amd.motion import PixelTrajectories, sample_grid
from x_amd.objectives import AnchoredExact, AnchoredTrajectories
from x_amd.ops import functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32 = np.float32


def T(a):
    return torch.as_tensor(np.ascontiguousarray(a), device=DEV)


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
                                    (16, "polynomial"), (1, "bspline"), (3, "bspline"), (10, "bspline"),
                                    (16, "bspline")])
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
    g, _ = O.traj_basis_table(t[ok].astype(np.float64), K, kind)     # float64, scipy's BSpline for the spline
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


@pytest.mark.parametrize("K", [3, 10, 16])
def test_traj_bspline_backward_forms_rows_in_kernel(K):
    """The B-spline backward that forms each event's gradient row from gd and t inside the kernels equals the one
    that writes the rows first (atl_traj_gout): position gradient bit for bit, field gradient to the order of
    the flush atomics."""
    print(f"traj bspline backward K={K}", flush=True)
    from x_amd.ops import functional as F
    rng = np.random.default_rng(K)
    n, B, Hg, Wg = 6000, 2, 21, 34
    C = 2 * K
    fld = T((rng.standard_normal((B, C, Hg, Wg)) * 2).astype(F32))
    gpos = T(np.stack([rng.uniform(-2, Wg + 1, n), rng.uniform(-2, Hg + 1, n)], 1).astype(F32))
    b = T(rng.integers(0, B, n).astype(np.int64))
    t = T(rng.uniform(-0.1, 1.1, n).astype(F32))                 # the end spans continue outside [0, 1]
    gd = T(rng.standard_normal((n, 2)).astype(F32))
    fcl = F._channels_last(fld)
    nbytes = int(F.load_library().atl_grid_plan_bytes(B, Hg, Wg, n))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=DEV)
    st = F.stream_of(gpos)
    F.call("atl_grid_plan", B, Hg, Wg, F.ptr(gpos), F.ptr(b), n, 0, 0, F.ptr(ws), nbytes, st)
    rows = torch.empty(n, C, device=DEV)
    F.call("atl_traj_gout", F.ptr(gd), F.ptr(t), n, K, 2, F.ptr(rows), st)
    gf_old, gf_new = torch.zeros_like(fld), torch.zeros_like(fld)
    F.call("atl_sample_grid_bwd_planned", F.ptr(rows), B, C, Hg, Wg, F.ptr(gpos), n, 0, 0, F.ptr(ws), F.ptr(gf_old), st)
    F.call("atl_traj_field_bwd_planned", F.ptr(gd), F.ptr(t), K, B, Hg, Wg, n, F.ptr(ws), F.ptr(gf_new), st)
    gp_old, gp_new = torch.empty_like(gpos), torch.empty_like(gpos)
    F.call("atl_sample_grid_bwd_pos_cl", F.ptr(rows), F.ptr(fcl), B, C, Hg, Wg, F.ptr(gpos), F.ptr(b), n, 0, 0,
           F.ptr(gp_old), st)
    F.call("atl_traj_pos_bwd_cl", F.ptr(gd), F.ptr(t), K, F.ptr(fcl), B, Hg, Wg, F.ptr(gpos), F.ptr(b), n,
           F.ptr(gp_new), st)
    assert torch.equal(gp_new, gp_old)
    close_rel(N(gf_new), N(gf_old), 1e-6)


@pytest.mark.parametrize("K,n_look,last,crowd", [(3, 1, False, 0), (10, 3, True, 0), (16, 2, False, 0),
                                                 (10, 2, True, 20000)])
def test_traj_field_bwd_equals_the_row_adjoint(K, n_look, last, crowd):
    """atl_traj_field_bwd (its own binning, one accumulation over n_look look-ups per event, halo flush) against
    the rows of atl_traj_gout (the last look-up at t_last) accumulated by the per-event sampler adjoint: equal to
    the order of the float additions.  Positions spill past every grid edge (border clamp), some gradients are
    zero, and with crowd a single tile holds that many records (split over several workgroups)."""
    print(f"traj field bwd K={K} n_look={n_look} last={last} crowd={crowd}", flush=True)
    rng = np.random.default_rng(100 + K + crowd)
    n, B, Hg, Wg = 7000 + crowd // 2, 2, 37, 53
    C = 2 * K
    pos = np.stack([rng.uniform(-2, Wg + 1, (n_look, n)), rng.uniform(-2, Hg + 1, (n_look, n))], -1)
    if crowd:                                      # one tile (nodes 16..31 x 16..31 of window 1) takes crowd records
        sel = rng.choice(n, crowd // n_look, replace=False)
        pos[:, sel] = rng.uniform(16.0, 31.9, (n_look, len(sel), 2))
    b = rng.integers(0, B, n).astype(np.int64)
    if crowd:
        b[sel] = 1
    t = rng.uniform(-0.1, 1.1, n).astype(F32)
    tl = rng.uniform(0.0, 1.0, n).astype(F32) if last else None
    gd = rng.standard_normal((n_look, n, 2)).astype(F32)
    gd[:, rng.random(n) < 0.1] = 0.0
    tp, tgd, tb, tt = T(pos.astype(F32)), T(gd), T(b), T(t)
    ttl = T(tl) if last else None
    st = F.stream_of(tp)
    nbytes = int(F.load_library().atl_traj_field_bwd_bytes(K, B, Hg, Wg, n_look * n))
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    got = torch.zeros(B, C, Hg, Wg, device=DEV)
    F.call("atl_traj_field_bwd", F.ptr(tgd), F.ptr(tp), F.ptr(tt), F.ptr(ttl), F.ptr(tb), n, n_look, K, B, Hg, Wg,
           F.ptr(ws), nbytes, F.ptr(got), st)
    want = torch.zeros_like(got)
    for r in range(n_look):
        tr = ttl if last and r == n_look - 1 else tt
        rows = torch.empty(n, C, device=DEV)
        F.call("atl_traj_gout", F.ptr(tgd[r]), F.ptr(tr), n, K, 2, F.ptr(rows), st)
        F.call("atl_sample_grid_bwd", F.ptr(rows), B, C, Hg, Wg, F.ptr(tp[r]), F.ptr(tb), n, 0, 0, F.ptr(want), st)
    close_rel(N(got), N(want), 1e-6)
    assert torch.equal(got == 0, want == 0)
    # a second call on the same workspace (its halo and chunk list rewritten) accumulates the same sum again
    F.call("atl_traj_field_bwd", F.ptr(tgd), F.ptr(tp), F.ptr(tt), F.ptr(ttl), F.ptr(tb), n, n_look, K, B, Hg, Wg,
           F.ptr(ws), nbytes, F.ptr(got), st)
    close_rel(N(got), 2 * N(want), 1e-6)


@pytest.mark.parametrize("C,scale,crowd", [(5, False, 0), (12, True, 0), (20, False, 12000), (32, False, 0)])
def test_sample_grid_bwd_rows_equals_the_per_event_adjoint(C, scale, crowd):
    """atl_sample_grid_bwd_rows (binned in the call, per-node register sums, halo flush) against the per-event
    atomic adjoint atl_sample_grid_bwd on the same rows: equal to the order of the float additions; positions past
    every edge, pixel-to-grid scaling, and with crowd one tile holding that many records (several workgroups)."""
    print(f"sample_grid_bwd_rows C={C} scale={scale} crowd={crowd}", flush=True)
    rng = np.random.default_rng(200 + C + crowd)
    n, B, Hg, Wg = 6000 + crowd, 2, 37, 53
    H, W = (150, 212) if scale else (Hg, Wg)
    pos = np.stack([rng.uniform(-3, W + 2, n), rng.uniform(-3, H + 2, n)], 1).astype(F32)
    b = rng.integers(0, B, n).astype(np.int64)
    if crowd:
        pos[:crowd] = rng.uniform(16.0, 31.9, (crowd, 2))
        b[:crowd] = 0
    g = rng.standard_normal((n, C)).astype(F32)
    g[rng.random(n) < 0.05] = 0.0
    tg, tp, tb = T(g), T(pos), T(b)
    ih, iw = (H, W) if scale else (0, 0)
    st = F.stream_of(tp)
    nbytes = int(F.load_library().atl_sample_grid_bwd_rows_bytes(B, C, Hg, Wg, n))
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    got = torch.zeros(B, C, Hg, Wg, device=DEV)
    F.call("atl_sample_grid_bwd_rows", F.ptr(tg), B, C, Hg, Wg, F.ptr(tp), F.ptr(tb), n, ih, iw, F.ptr(got),
           F.ptr(ws), nbytes, st)
    want = torch.zeros_like(got)
    F.call("atl_sample_grid_bwd", F.ptr(tg), B, C, Hg, Wg, F.ptr(tp), F.ptr(tb), n, ih, iw, F.ptr(want), st)
    close_rel(N(got), N(want), 1e-6)
    assert F.load_library().atl_sample_grid_bwd_rows_bytes(B, 4, Hg, Wg, n) == -1      # C <= 4: other paths
    assert F.load_library().atl_sample_grid_bwd_rows_bytes(B, 33, Hg, Wg, n) == -1


def test_traj_field_bwd_rejects_bad_sizes():
    """Sizes atl_traj_field_bwd does not take are refused before any launch (workspace query -1, call status 1)."""
    lib = F.load_library()
    assert lib.atl_traj_field_bwd_bytes(2, 1, 16, 16, 10) == -1          # K < 3
    assert lib.atl_traj_field_bwd_bytes(17, 1, 16, 16, 10) == -1         # 2K > 32
    assert lib.atl_traj_field_bwd_bytes(4, 1, 16, 16, 0) > 0
    p = torch.zeros(1, 5, 2, device=DEV)
    t = torch.zeros(5, device=DEV)
    b = torch.zeros(5, dtype=torch.long, device=DEV)
    gf = torch.zeros(1, 8, 16, 16, device=DEV)
    nbytes = int(lib.atl_traj_field_bwd_bytes(4, 1, 16, 16, 5))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    st = F.stream_of(p)
    assert lib.atl_traj_field_bwd(F.ptr(p), F.ptr(p), F.ptr(t), None, F.ptr(b), 5, 1, 4, 1, 16, 16, F.ptr(ws),
                                  nbytes - 256, F.ptr(gf), st) == 1
    assert b"workspace" in lib.atl_last_error()
    assert lib.atl_traj_field_bwd(F.ptr(p), F.ptr(p), F.ptr(t), None, F.ptr(b), 5, 0, 4, 1, 16, 16, F.ptr(ws),
                                  nbytes, F.ptr(gf), st) == 1
    assert not gf.any()


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
    # shapes the kernel would read past: all refused on the host before any launch
    p5 = torch.zeros(5, 2, device=DEV)
    b5 = torch.zeros(5, dtype=torch.long, device=DEV)
    t5 = torch.zeros(5, device=DEV)
    for args in ((tf, p5, b5, t5, 3), (tf, p5, b5, t5, 5),                     # C != 2K
                 (tf, torch.zeros(5, 3, device=DEV), b5, t5, 4),                # positions not (N, 2)
                 (tf, p5, b5[:4], t5, 4), (tf, p5, b5, t5[:3], 4),              # short b, short t
                 (tf[0], p5, b5, t5, 4), (tf, p5, b5, t5, 17)):                 # not 4-D, K > 16
        with pytest.raises(ValueError):
            F.traj_displacement(*args, "bspline")
    with pytest.raises(ValueError):
        F.sample_grid_hip(tf, torch.zeros(5, 3, device=DEV), b5)
    with pytest.raises(ValueError):
        F.sample_grid_hip(tf, p5, b5[:2])
    # the C entry point itself rejects a channel count that is not 2K
    from x_amd.ops import _ext
    fcl = torch.zeros(2, 9, 11, 8, device=DEV)
    rc = _ext.load_library().atl_traj_displacement(_ext.ptr(fcl), 2, 6, 4, 9, 11, _ext.ptr(p5), _ext.ptr(b5),
                                                     _ext.ptr(t5), 5, 2, _ext.ptr(p5), None)
    assert rc == 1 and b"expected 2K" in _ext.load_library().atl_last_error()


@pytest.mark.parametrize("K,tile,steps,dst", [(3, 1, 6, False), (10, 1, 6, False), (10, 4, 6, False),
                                              (4, 4, 1, False), (10, 1, 6, True), (3, 4, 2, True)])
def test_traj_origin_node_matches_composed_steps(K, tile, steps, dst):
    """The fixed-point origin as one autograd node (one field accumulation over every step's records), and with
    dst the transport's last look-up in the same node, against the same steps composed from traj_displacement:
    the same positions bit for bit, and the same coefficient-grid and position gradients to the order of the
    accumulation's additions."""
    print(f"traj origin node K={K} tile={tile} steps={steps} dst={dst}", flush=True)
    from x_amd.ops import functional as F
    rng = np.random.default_rng(10 * K + tile)
    win = synth.small_window(seed=K + tile, n=4000, B=2)
    coeffs = synth.trajectory_coeffs(rng, 2, K, win.height, win.width, sigma_px=8.0, dmax=3.0)
    w = T(rng.standard_normal((win.n, 2)).astype(F32))
    ev = EventPacket.from_window(win, DEV)
    off = float(tile // 2)
    td = T(rng.uniform(0, 1, win.n).astype(F32)) if dst else None
    res = []
    for fused in (True, False):
        c = torch.tensor(coeffs, device=DEV, requires_grad=True)
        fld = c if tile == 1 else c[:, :, tile // 2::tile, tile // 2::tile]
        xy = ev.xy.clone().requires_grad_(True)
        if fused:
            p = F.traj_origin(fld, xy, ev.b, ev.t, K, "bspline", steps, off, tile, t_dst=td)
        else:
            p = xy
            for _ in range(steps):
                g = p if tile == 1 else (p - off) / tile
                p = xy - F.traj_displacement(fld, g, ev.b, ev.t, K, "bspline")
            if dst:
                p = p + F.traj_displacement(fld, p if tile == 1 else (p - off) / tile, ev.b, td, K, "bspline")
        (p * w).sum().backward()
        res.append((p.detach(), c.grad, xy.grad))
    assert torch.equal(res[0][0], res[1][0])
    close_rel(N(res[0][1]), N(res[1][1]), 1e-5)
    close_rel(N(res[0][2]), N(res[1][2]), 1e-5)


@pytest.mark.parametrize("K,kind,tile", [(1, "polynomial", 4), (3, "bezier", 4), (4, "polynomial", 4),
                                         (10, "bezier", 4), (3, "bspline", 1), (10, "bspline", 1),
                                         (10, "bspline", 4)])
def test_pixel_trajectories_device_matches_cpu(K, kind, tile):
    """Transport (fixed-point origin + displacement) values and coefficient gradients, device vs CPU."""
    print(f"trajectories K={K} {kind} tile={tile}", flush=True)
    win = synth.small_window(seed=K, n=3000, B=2)
    rng = np.random.default_rng(K)
    coeffs = synth.trajectory_coeffs(rng, 2, K, win.height, win.width, sigma_px=8.0, dmax=3.0)
    w = rng.standard_normal((win.n, 2)).astype(F32)
    res = {}
    for dev in ("cpu", DEV):
        ev = EventPacket.from_window(win, dev)
        c = torch.tensor(coeffs, device=dev, requires_grad=True)
        m = PixelTrajectories(c, K, kind, tile=tile)
        y = m.transport(ev.xy, ev.t, 0.7, ev.b)
        (y * torch.tensor(w, device=dev)).sum().backward()
        res[dev] = (N(y), N(c.grad))
    close_rel(res[DEV][0], res["cpu"][0], 1e-5)
    close_rel(res[DEV][1], res["cpu"][1], 1e-4)


@pytest.mark.parametrize("K,kind,tile,n_check", [(10, "bspline", 1, 16), (3, "bezier", 4, 16),
                                                 (1, "polynomial", 1, 16), (10, "bspline", 4, 16),
                                                 (10, "bspline", 1, 70)])
def test_traj_visible_fraction_same_bits(K, kind, tile, n_check):
    """The one-pass exposure correction for trajectories against the composed device ops (origin, then the
    displacement at every bin centre, then the weighted share), bit for bit; the bin-centre basis from the
    kernel's LDS table (n_check <= 64) and computed per centre (more bins)."""
    print(f"trajectory visible fraction K={K} {kind} tile={tile} n_check={n_check}", flush=True)
    win = synth.small_window(seed=K + tile, n=4000, B=2)
    rng = np.random.default_rng(K * 3 + tile)
    coeffs = synth.trajectory_coeffs(rng, 2, K, win.height, win.width, sigma_px=8.0, dmax=6.0)
    ev = EventPacket.from_window(win, DEV)
    m = PixelTrajectories(T(coeffs), K, kind, tile=tile)
    xa = ev.xy + T(rng.standard_normal((win.n, 2)).astype(F32))
    tau = 0.3
    got = F.traj_visible_fraction(m.tile_c, K, kind, m.n_fp, m.offset, m.tile, xa, ev.t, ev.b, ev.t, ev.b, 2,
                                  win.height, win.width, tau, n_check)
    with torch.no_grad():
        counts = F.bin_counts(ev.t, ev.b, 2, n_check)
        edges = torch.linspace(0, 1, n_check + 1, device=DEV)
        start = m.origin(xa, ev.t, ev.b)
        vis, tot = torch.zeros_like(ev.t), torch.zeros_like(ev.t)
        for k, c in enumerate((0.5 * (edges[:-1] + edges[1:])).tolist()):
            y = start + m.displacement(start, ev.b, torch.full_like(ev.t, c))
            seen = (y[:, 0] >= 0) & (y[:, 0] <= win.width - 1) & (y[:, 1] >= 0) & (y[:, 1] <= win.height - 1)
            w = counts[ev.b, k] * ((ev.t - c).abs() <= tau).float()
            vis += w * seen.float()
            tot += w
        want = (vis / tot.clamp(min=1)).clamp(min=1e-3)
    assert torch.equal(got, want)
    assert 0.01 < float((want < 0.999).float().mean()) < 0.99      # trajectories leave the sensor and stay


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


def test_pixel_trajectories_straight_bspline_closed_form():
    """Cubic B-spline control points c_k = v xi_k at the Greville abscissae are the straight trajectory p + v t:
    transport(x, t, t') = x + v (t' - t) (linear precision of the basis)."""
    from x_amd.motion.trajectories import greville
    win = synth.small_window(seed=4, n=2000, B=1)
    ev = EventPacket.from_window(win, DEV)
    K = 10
    xi = torch.tensor(greville(K), dtype=torch.float32, device=DEV)
    v = (1.75, -3.5)                                       # (x, y) px per window
    c = torch.cat([v[1] * xi, v[0] * xi]).view(1, 2 * K, 1, 1).expand(1, 2 * K, win.height, win.width)
    m = PixelTrajectories(c.contiguous(), K, "bspline", tile=1)
    y = N(m.transport(ev.xy, ev.t, 0.6, ev.b))
    want = win.xy + np.array(v, F32) * (F32(0.6) - win.t)[:, None]
    assert np.allclose(y, want, atol=2e-5)


def _traj_case(seed, n, B, H, W, K, kind, h, tau, S):
    """Events of a small window, trajectory starts p near the events, smooth coefficient rows, smoothed anchors,
    the slice table (oracle: scipy's BSpline)."""
    win = synth.small_window(seed=seed, n=n // B, H=H, W=W, B=B)
    rng = np.random.default_rng(seed + 50)
    xs = (win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(F32)
    fld = synth.trajectory_coeffs(rng, B, K, H, W, sigma_px=6.0, dmax=4.0)
    coef, _, _ = O.sample_grid(fld, xs, win.b)
    p = (xs - rng.uniform(-1, 1, xs.shape)).astype(F32)
    xa = (xs + h * rng.standard_normal(xs.shape)).astype(F32)
    return win, p, coef.astype(F32), xa, O.traj_slice_table(K, kind, S)


def check_traj_against_oracle(p, coef, tab, t, b, B, H, W, anchors, xa, h, tau, S, K, kind, fp64=True,
                              index_free=False):
    """Device trajectory pair sums vs the oracle: counts bit-exact with the fp32 plan and pair loops, sums within
    1e-5 of them, gradients within 1e-4 of the float64 brute force (or, without fp64, of the pair loops)."""
    print(f"traj pair case N={len(t)} M={len(anchors)} K={K} {kind} h={h} tau={tau} S={S}", flush=True)
    plan_o = O.build_pair_plan_traj(p, coef, tab, t, b, B, H, W, anchors, xa, h, tau, 3.0, S)
    want, wcnt = O.ats_pair_fwd(plan_o, h, tau, 3.0, with_counts=True)
    plan = F.FastPairPlan(T(p), T(t), None, T(b), B, H, W, None if index_free else T(anchors), h, tau, 3.0, S, T(xa),
                          traj=(T(coef), K, T(tab)))
    assert np.array_equal(N(plan.counts()), wcnt)
    assert_sums_close(N(plan.forward()), want)
    gS = np.random.default_rng(7).standard_normal(len(anchors)).astype(F32)
    gp, gc = plan.backward_traj(T(gS))
    if fp64:
        S64, c64, grad = O.traj_pair_sums_fp64(p, coef, t, b, anchors, xa, h, tau, 3.0, S, K, kind)
        close_rel(N(plan.forward()), S64, 1e-5)
        wp, wc = grad(gS)
    else:
        wp, wc = O.ats_pair_bwd_traj(gS, plan_o, tab, K, h, tau, 3.0, len(t))
    close_rel(N(gp), wp, 1e-4)
    close_rel(N(gc), wc, 1e-4)
    return wcnt


@pytest.mark.parametrize("K,kind,tau,S,h", [(10, "bspline", 0.8, 16, 1.0), (3, "bspline", 0.2, 16, 1.0),
                                            (1, "bspline", 0.3, 8, 1.5), (4, "bezier", 0.5, 16, 0.5),
                                            (2, "polynomial", 1.0, 4, 1.0)])
def test_traj_pair_sums_match_oracle(K, kind, tau, S, h):
    win, p, coef, xa, tab = _traj_case(21 + K, 4000, 2, 40, 48, K, kind, h, tau, S)
    cnt = check_traj_against_oracle(p, coef, tab, win.t, win.b, 2, 40, 48, np.arange(win.n), xa, h, tau, S, K, kind)
    assert cnt.sum() > win.n


def test_traj_pair_sums_anchor_subsets_duplicates_and_edges():
    """Unsorted anchor subsets, an event listed twice among the anchors (leave-one-out by id), starts far
    outside the sensor (clamped bins), and no events at all."""
    K, kind = 10, "bspline"
    win, p, coef, xa, tab = _traj_case(31, 3000, 2, 40, 48, K, kind, 1.0, 0.4, 16)
    rng = np.random.default_rng(3)
    sub = rng.permutation(win.n)[: win.n // 3]
    check_traj_against_oracle(p, coef, tab, win.t, win.b, 2, 40, 48, sub, xa[sub], 1.0, 0.4, 16, K, kind)
    dup = np.concatenate([np.arange(0, win.n, 2), np.arange(0, win.n, 6)])
    check_traj_against_oracle(p, coef, tab, win.t, win.b, 2, 40, 48, dup, xa[dup], 1.0, 0.4, 16, K, kind)
    p2 = p.copy()
    p2[::9] += F32(200.0)
    check_traj_against_oracle(p2, coef, tab, win.t, win.b, 2, 40, 48, np.arange(win.n), xa, 1.0, 0.4, 16, K, kind,
                              index_free=True)
    z2, z1 = torch.zeros(0, 2, device=DEV), torch.zeros(0, device=DEV)
    zb = torch.zeros(0, dtype=torch.long, device=DEV)
    plan = F.FastPairPlan(z2, z1, None, zb, 1, 40, 48, None, 1.0, 0.4, 3.0, 16, z2,
                          traj=(torch.zeros(0, 2 * K, device=DEV), K, T(tab)))
    gp, gc = plan.backward_traj(z1)
    assert plan.forward().shape == (0,) and gp.shape == (0, 2) and gc.shape == (0, 2 * K)


def test_traj_pair_sums_straight_trajectories_are_the_linear_sums():
    """Straight trajectories (starts p = x - v t, control points v xi_k) give the reference's linear pair sums:
    device values within 1e-5 and the velocity gradient recovered from the start and coefficient gradients,
    -t gp + sum_k xi_k gcoef_k, within 1e-4 of the reference's dS/dv (float64 brute force)."""
    from x_amd.motion.trajectories import greville
    pos, _, b, t = rand_events(n=800, seed=9)
    rng = np.random.default_rng(2)
    v = (rng.standard_normal((800, 2)) * 5).astype(F32)
    K = 10
    xi = greville(K)
    p = (pos - v * t[:, None]).astype(F32)
    coef = np.concatenate([v[:, 1:2] * xi, v[:, 0:1] * xi], 1).astype(F32)
    tab = O.traj_slice_table(K, "bspline", 16)
    anchors = np.arange(0, 800, 2)
    xa = (pos[anchors] + rng.standard_normal((400, 2)) * 0.5).astype(F32)
    plan = F.FastPairPlan(T(p), T(t), None, T(b), 2, 20, 24, T(anchors), 1.5, 0.3, 3.0, 16, T(xa),
                          traj=(T(coef), K, T(tab)))
    Sl, _, grad = O.pair_sums_fp64(pos, t, v, b, anchors, 1.5, 0.3, 3.0, anchor_xy=xa)
    close_rel(N(plan.forward()), Sl, 1e-5)
    gS = rng.standard_normal(400).astype(F32)
    gp, gc = (N(a).astype(np.float64) for a in plan.backward_traj(T(gS)))
    gv = -t[:, None] * gp + np.stack([(gc[:, K:] * xi).sum(1), (gc[:, :K] * xi).sum(1)], 1)
    close_rel(gv, grad(gS), 1e-4)


def test_traj_pair_sums_full_size():
    """The continuous-time workload at full size: 4 windows x 500k events at 640x480 on per-pixel cubic B-spline
    trajectories (10 control points), starts and coefficients from the model on the device, tau = 0.8, h = 1, 16
    slices, every event an anchor: counts bit-exact with the oracle's fp32 plan and pair loops, sums within
    1e-5, start and coefficient gradients within 1e-4 of the oracle's pair loops."""
    print("traj pair sums full size 4 x 500k", flush=True)
    win = synth.bspline_windows(seed=0)
    K = win.motion["K"]
    ev = EventPacket.from_window(win, DEV)
    m = PixelTrajectories(torch.as_tensor(win.motion["coeffs"], device=DEV), K, "bspline", tile=1)
    xs_d, xa_d = F.event_noise(ev.xy, 0, 0, 1.0)
    with torch.no_grad():
        p_d = m.origin(xs_d, ev.t, ev.b)
        coef_d = m.coeff_rows(p_d, ev.b)
    tab = O.traj_slice_table(K, "bspline", 16)
    assert np.array_equal(N(m.slice_tables(16, DEV)), tab)
    cnt = check_traj_against_oracle(N(p_d), N(coef_d), tab, win.t, win.b, 4, 480, 640, np.arange(win.n), N(xa_d),
                                    1.0, 0.8, 16, K, "bspline", fp64=False, index_free=True)
    assert cnt.sum() > 20 * win.n


def test_anchored_trajectories_device_matches_cpu():
    """AnchoredTrajectories (B-spline, K = 10, per-pixel) end to end: log scores and coefficient gradient, device
    vs the same chain on CPU tensors (CPU-generated noise on both)."""
    print("anchored trajectories device vs cpu", flush=True)
    win = synth.small_window(seed=12, n=2500, B=2)
    rng = np.random.default_rng(12)
    K = 10
    coeffs = synth.trajectory_coeffs(rng, 2, K, win.height, win.width, sigma_px=8.0, dmax=3.0)
    res = {}
    for dev in ("cpu", DEV):
        ev = EventPacket.from_window(win, dev)
        c = torch.tensor(coeffs, device=dev, requires_grad=True)
        obj = AnchoredTrajectories(h=1.0, tau=0.5, n_anchors=None, seed=0)
        ls, _ = obj.log_scores(ev, PixelTrajectories(c, K, "bspline", tile=1))
        (-ls.mean()).backward()
        res[dev] = (N(ls), N(c.grad))
    close_rel(res[DEV][0], res["cpu"][0], 1e-5)
    close_rel(res[DEV][1], res["cpu"][1], 1e-4)


def test_anchored_trajectories_straight_equals_exact():
    """Constant straight B-spline trajectories (control points v xi_k everywhere) and the translation v: the
    trajectory score equals AnchoredExact's (same noise), log scores within 1e-5."""
    from x_amd.motion import Translation
    from x_amd.motion.trajectories import greville
    win = synth.small_window(seed=13, n=3000, B=1)
    ev = EventPacket.from_window(win, DEV)
    K = 10
    v = (2.5, -1.25)
    xi = torch.tensor(greville(K), dtype=torch.float32, device=DEV)
    c = torch.cat([v[1] * xi, v[0] * xi]).view(1, 2 * K, 1, 1).expand(1, 2 * K, win.height, win.width).contiguous()
    ls_t, _ = AnchoredTrajectories(h=1.0, tau=0.3, n_anchors=None, seed=0).log_scores(
        ev, PixelTrajectories(c, K, "bspline", tile=1))
    mt = Translation(1, win.height, win.width, init=torch.tensor([v])).to(DEV)
    ls_e, _ = AnchoredExact(h=1.0, tau=0.3, n_anchors=None, seed=0).log_scores(ev, mt)
    close_rel(N(ls_t), N(ls_e), 1e-5)


# ------------------------------------------------------------------------ the continuous-time objective end to end
def _crop_c4(x0=0, y0=0, w=200, h=150):
    """The continuous-time workload (4 windows x 500k events, 640x480, per-pixel cubic B-splines with 10 control
    points) restricted to the events inside one 200 x 150 px box at the sensor corner: the workload's event
    density and trajectories at about a tenth of its events, with trajectories that leave the sensor."""
    win = synth.bspline_windows(seed=0)
    keep = (win.xy[:, 0] >= x0) & (win.xy[:, 0] < x0 + w) & (win.xy[:, 1] >= y0) & (win.xy[:, 1] < y0 + h)
    sub = synth.Window(xy=np.ascontiguousarray(win.xy[keep]), t=np.ascontiguousarray(win.t[keep]), p=win.p[keep],
                       b=np.ascontiguousarray(win.b[keep]), height=win.height, width=win.width,
                       batch_size=win.batch_size, duration=win.duration, motion=win.motion)
    return sub


def _bilinear64(fld, p):
    """Border-clamped bilinear sample (float64) of a (C, Hg, Wg) field at grid positions p (n, 2): (n, C)."""
    C, Hg, Wg = fld.shape
    gx, gy = np.clip(p[:, 0], 0, Wg - 1), np.clip(p[:, 1], 0, Hg - 1)
    x0, y0 = np.minimum(np.floor(gx), Wg - 2).astype(np.int64), np.minimum(np.floor(gy), Hg - 2).astype(np.int64)
    ax, ay = (gx - x0)[:, None], (gy - y0)[:, None]
    f = fld.transpose(1, 2, 0)
    return (f[y0, x0] * (1 - ax) * (1 - ay) + f[y0, x0 + 1] * ax * (1 - ay) + f[y0 + 1, x0] * (1 - ax) * ay
            + f[y0 + 1, x0 + 1] * ax * ay)


def _disp64(fld, p, t, K):
    g, _ = O.traj_basis_table(t, K, "bspline")
    r = _bilinear64(fld, p)
    return np.stack([(r[:, K:] * g).sum(1), (r[:, :K] * g).sum(1)], 1), r


def _origin64(fld, xy, t, K, steps=6):
    p = xy.copy()
    for _ in range(steps):
        p = xy - _disp64(fld, p, t, K)[0]
    return p


def _pair_terms64(p, rows, tj, ids, xa, ta, aid, K, h, tau, S):
    """float64 kernel values of every (anchor, source) pair of the given sources under the trajectory pair sums'
    definition (slice-centre linearisation, the three tests, leave-one-out): (values, count)."""
    cs = O.slice_centres(S).astype(np.float64)
    g, gd = O.traj_basis_table(cs, K, "bspline")
    s_lo, s_hi = O.slice_range(tj.astype(F32), tau, S)
    s = np.clip(np.floor(ta * S), 0, S - 1).astype(np.int64)
    at = ta - cs[s]
    y = p[None] + np.stack([g[s] @ rows[:, K:].T, g[s] @ rows[:, :K].T], -1)          # (m, n, 2)
    v = np.stack([gd[s] @ rows[:, K:].T, gd[s] @ rows[:, :K].T], -1)
    r = xa[:, None, :] - (y + v * at[:, None, None])
    d2 = (r * r).sum(-1)
    ok = (np.abs(ta[:, None] - tj[None]) <= tau) & (d2 <= 9 * h * h) & (aid[:, None] != ids[None])
    ok &= (s_lo[None] <= s[:, None]) & (s[:, None] <= s_hi[None])
    return np.where(ok, np.exp(-d2 / (2 * h * h)), 0.0).sum(1), ok.sum()


def test_anchored_trajectories_end_to_end_against_the_oracle():
    """AnchoredTrajectories(rng="device") and the IWE-variance leg on the continuous-time workload (a 200 x 150 px
    crop of the 4 windows) against the oracle chain:
    * trajectory starts of the device's fixed-point node within 2e-4 px of the oracle's (fp32, float64 basis);
    * on those starts: per-anchor neighbour counts bit-exact (oracle plan and pair loops), window counts and
      exposure bit-exact (anchors whose positions at a bin centre come within 1e-3 px of the sensor edge
      excepted), log scores within 1e-5 of the oracle epilogue;
    * the coefficient-grid gradient of -mean(log score) and of the IWE variance against float64 central
      differences of the chain (six fixed-point steps, coefficient rows, pair sums, epilogue; transport to 0.5,
      splat, variance) on the largest-gradient coefficients, within 2e-4;
    * the device IWE against O.splat_bilinear_fwd at the device's transported positions, which are within 2e-4
      px of the oracle's transport."""
    from x_amd.objectives import iwe_variance
    from x_amd.objectives.base import IWEConfig, make_iwe
    print("anchored trajectories end to end vs oracle (C4 crop)", flush=True)
    win = _crop_c4()
    K, h, tau, S, seed = win.motion["K"], 1.0, 0.8, 16, 5
    H, W, B = win.height, win.width, win.batch_size
    coeffs = win.motion["coeffs"]
    n = win.n
    ev = EventPacket.from_window(win, DEV)
    c = torch.tensor(coeffs, device=DEV, requires_grad=True)
    m = PixelTrajectories(c, K, "bspline", tile=1)
    obj = AnchoredTrajectories(h=h, tau=tau, cut=3.0, n_slices=S, n_anchors=None, seed=seed, rng="device")
    ls_d, _ = obj.log_scores(ev, m)
    (-ls_d.mean()).backward()
    g_score = N(c.grad).astype(np.float64)
    xs_d, xa_d = F.event_noise(ev.xy, seed, 0, h)                 # the objective's own first draw
    xs, xa = N(xs_d), N(xa_d)
    with torch.no_grad():
        p_d = N(m.origin(xs_d, ev.t, ev.b))
    p_o = O.traj_origin(coeffs, xs, win.t, win.b, K, "bspline")
    assert np.abs(p_d - p_o).max() <= 2e-4
    rows, _, _ = O.sample_grid(coeffs, p_d, win.b)
    tab = O.traj_slice_table(K, "bspline", S)
    anchors = np.arange(n)
    plan = O.build_pair_plan_traj(p_d, rows, tab, win.t, win.b, B, H, W, anchors, xa, h, tau, 3.0, S)
    S_o, cnt_o = O.ats_pair_fwd(plan, h, tau, 3.0, with_counts=True)
    dplan = F.FastPairPlan(T(p_d), ev.t, None, ev.b, B, H, W, None, h, tau, 3.0, S, xa_d,
                           traj=(T(rows), K, T(tab)))
    assert np.array_equal(N(dplan.counts()), cnt_o) and cnt_o.sum() > 50 * n
    wc = O.window_counts(win.t, win.b, anchors, tau)
    assert np.array_equal(N(F.window_counts(ev.t, ev.b, None, tau, assume_sorted=True)), wc)
    vis = O.traj_visible_fraction(coeffs, xa, win.t, win.b, win.t, win.b, B, H, W, tau, K, "bspline")
    assert (vis < 1).sum() > 100                                  # the crop's trajectories leave the sensor
    ls_o, _, D = O.anchored_epilogue(S_o, wc, h, H, W, 1e-2, vis)
    # anchors whose trajectory position at some bin centre lies within 1e-3 px of the sensor edge: fp32 may count
    # them inside or outside
    pa = np.zeros((n, 2))
    clear = np.ones(n, bool)
    for b in range(B):
        sel = win.b == b
        pa[sel] = _origin64(coeffs[b].astype(np.float64), xa[sel].astype(np.float64), win.t[sel].astype(np.float64), K)
        for k in range(16):
            ck = (k + 0.5) / 16
            yk = pa[sel] + _disp64(coeffs[b].astype(np.float64), pa[sel], np.full(sel.sum(), ck), K)[0]
            near = np.zeros(sel.sum(), bool)
            for col, hi in ((0, W - 1), (1, H - 1)):
                near |= (np.abs(yk[:, col]) <= 1e-3) | (np.abs(yk[:, col] - hi) <= 1e-3)
            clear[np.nonzero(sel)[0][near]] = False
    assert clear.mean() > 0.99
    assert_logs_close(N(ls_d)[clear], ls_o[clear])

    # ---- gradient of -mean(log score): float64 central differences of the chain on the largest-gradient
    # coefficients (a perturbation moves only the sources whose fixed-point iterates touch the node)
    Dd = D.astype(np.float64)
    eps = 1e-2 / (H * W)
    checked = 0
    for flat in np.argsort(-np.abs(g_score).ravel())[:8]:
        b, ch, yy, xx = np.unravel_index(flat, g_score.shape)
        sel = np.nonzero(win.b == b)[0]
        fld = coeffs[b].astype(np.float64)
        e = 1e-3
        xs64, t64 = xs[sel].astype(np.float64), win.t[sel].astype(np.float64)
        sums, counts = [], []
        for sgn in (1, -1, 0):
            f2 = fld.copy()
            f2[ch, yy, xx] += sgn * e
            p2 = _origin64(f2, xs64, t64, K)
            sums.append((p2, _bilinear64(f2, p2)))
        moved = np.nonzero(np.any(sums[0][0] != sums[1][0], 1) | np.any(sums[0][1] != sums[1][1], 1))[0]
        assert 0 < moved.size < 400
        ids = sel[moved]
        vals = []
        for p2, r2 in sums:
            v, cnt = _pair_terms64(p2[moved], r2[moved], t64[moved], ids, xa[sel].astype(np.float64), t64,
                                   sel, K, h, tau, S)
            vals.append(v)
            counts.append(cnt)
        if len(set(counts)) != 1:
            continue                                   # a pair crosses a cut-off: no derivative there
        # the sums without the moved sources' terms (the oracle's sums hold them at the unperturbed coefficients)
        base = S_o[sel].astype(np.float64) - vals[2]
        lp = np.log(eps + (base + vals[0]) / Dd[sel])
        lm = np.log(eps + (base + vals[1]) / Dd[sel])
        fd = -(lp - lm).sum() / n / (2 * e)
        assert abs(g_score[b, ch, yy, xx] - fd) <= 2e-4 * abs(fd), (b, ch, yy, xx, g_score[b, ch, yy, xx], fd)
        checked += 1
    assert checked >= 3

    # ---- the IWE leg: transport to 0.5, bilinear splat with the inside mask, variance over pixels
    c.grad = None
    cfg = IWEConfig(kernel="bilinear", sigma=0.0)
    y_d = m.transport(ev.xy, ev.t, 0.5, ev.b)
    img_d = make_iwe(ev, y_d, 0.5, cfg)
    var = img_d.var(dim=(-2, -1)).mean()
    var.backward()
    g_iwe = N(c.grad).astype(np.float64)
    assert abs(float(var.detach()) - float(N(iwe_variance(ev, m, 0.5)))) <= 1e-6 * abs(float(var.detach()))
    y = N(y_d)
    q_o = O.traj_origin(coeffs, win.xy, win.t, win.b, K, "bspline")
    y_o = q_o + O.traj_displacement(coeffs, q_o, np.full(n, 0.5, F32), win.b, K, "bspline")[0]
    assert np.abs(y - y_o).max() <= 2e-4
    w = ((y[:, 0] >= 0) & (y[:, 0] <= W - 1) & (y[:, 1] >= 0) & (y[:, 1] <= H - 1)).astype(F32)
    img_o = O.splat_bilinear_fwd(y, w, win.b, B, H, W)
    close_rel(N(img_d), img_o, 1e-5)
    img64 = img_o.astype(np.float64)
    checked = 0
    for flat in np.argsort(-np.abs(g_iwe).ravel())[:8]:
        b, ch, yy, xx = np.unravel_index(flat, g_iwe.shape)
        sel = np.nonzero(win.b == b)[0]
        fld = coeffs[b].astype(np.float64)
        e = 1e-3
        xy64, t64 = win.xy[sel].astype(np.float64), win.t[sel].astype(np.float64)
        ys = []
        for sgn in (1, -1):
            f2 = fld.copy()
            f2[ch, yy, xx] += sgn * e
            q2 = _origin64(f2, xy64, t64, K)
            ys.append(q2 + _disp64(f2, q2, np.full(sel.size, 0.5), K)[0])
        moved = np.nonzero(np.any(ys[0] != ys[1], 1))[0]
        inside = [((yk[moved, 0] >= 0) & (yk[moved, 0] <= W - 1) & (yk[moved, 1] >= 0) & (yk[moved, 1] <= H - 1))
                  for yk in ys]
        cells = [np.floor(yk[moved]) for yk in ys]
        if not (np.array_equal(inside[0], inside[1]) and np.array_equal(cells[0], cells[1])):
            continue                                   # a mask flip or a pixel crossing between the two sides
        base = img64[b].copy()
        y_base = y[sel[moved]].astype(np.float64)
        w_base = w[sel[moved]].astype(np.float64)
        for j in range(moved.size):                    # take the moved events out of the oracle image (fp64)
            base -= _splat64_one(y_base[j], w_base[j], H, W)
        vs = []
        for k, yk in enumerate(ys):
            im = base.copy()
            for j in range(moved.size):
                im += _splat64_one(yk[moved[j]], float(inside[k][j]), H, W)
            vs.append(im.var(ddof=1))
        fd = (vs[0] - vs[1]) / B / (2 * e)
        assert abs(g_iwe[b, ch, yy, xx] - fd) <= 2e-4 * abs(fd), (b, ch, yy, xx, g_iwe[b, ch, yy, xx], fd)
        checked += 1
    assert checked >= 3


def _splat64_one(y, w, H, W):
    """float64 bilinear splat of one event (zero padding)."""
    img = np.zeros((H, W))
    x0, y0 = int(np.floor(y[0])), int(np.floor(y[1]))
    ax, ay = y[0] - x0, y[1] - y0
    for dx, wx in ((0, 1 - ax), (1, ax)):
        for dy, wy in ((0, 1 - ay), (1, ay)):
            if 0 <= x0 + dx < W and 0 <= y0 + dy < H:
                img[y0 + dy, x0 + dx] += w * wx * wy
    return img
