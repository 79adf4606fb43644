"""Fused pair-sum path (atl_fast_*) against the oracle: per-anchor neighbour counts bit-exact, sums within
1e-5 relative, velocity gradients within 1e-4 (relative to the largest magnitude, as gradient sums cancel).

The fused path bins positions on its own fine grid; these tests check that it finds exactly the reference's
contributing pairs (counts) and sums them to the reference's values, on the reference test shapes, on the
edge cases of the plan (empty inputs, clamped positions far outside the sensor, coincident events, anchor
subsets in any order) and at the full 1M-event size against the reference-layout kernels."""
import numpy as np
import pytest
import torch

import oracle as O
from tests.conftest import assert_sums_close, rand_events
from x_amd import synth
from x_amd.ops import functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32 = np.float32


def T(a):
    return torch.as_tensor(np.ascontiguousarray(a), device=DEV)


def N(t):
    return t.detach().cpu().numpy()


def close_rel(got, want, rel):
    scale = max(float(np.abs(want).max()), 1e-30) if want.size else 1.0
    err = float(np.abs(got.astype(np.float64) - want.astype(np.float64)).max()) if want.size else 0.0
    assert err <= rel * scale, f"max err {err:.3e} vs scale {scale:.3e} (rel {err / scale:.2e})"


def _case(seed=0, n=6000, B=2, H=40, W=48, h=1.0):
    win = synth.small_window(seed=seed, n=n // B, H=H, W=W, B=B)
    v, _, _ = O.dense_velocity(win.motion["grid"], win.xy, win.b, H, W)
    rng = np.random.default_rng(seed + 100)
    xs = (win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(F32)
    xa = (xs + h * rng.standard_normal(xs.shape)).astype(F32)
    return win, xs, v, xa


def check_against_oracle(xs, t, v, b, B, H, W, anchors, xa, h, tau, S, seed=0, index_free=False):
    """Counts, sums and gradients of the fused path vs the oracle on the reference plan.  ``index_free``: the
    anchors are every event in order and the fused plan gets no index array (the benchmarked form)."""
    print(f"fast pair case N={len(t)} M={len(anchors)} B={B} HxW={H}x{W} h={h} tau={tau} S={S}", flush=True)
    p = O.build_pair_plan(xs, t, v, b, B, H, W, anchors, h, tau, 3.0, S, anchor_xy=xa)
    want, wcnt = O.ats_pair_fwd(p, h, tau, 3.0, with_counts=True)
    if index_free:
        assert np.array_equal(anchors, np.arange(len(t)))
    plan = F.FastPairPlan(T(xs), T(t), T(v), T(b), B, H, W, None if index_free else T(anchors), h, tau, 3.0, S,
                          None if xa is None else T(xa))
    assert np.array_equal(N(plan.counts()), wcnt)
    assert_sums_close(N(plan.forward()), want)
    gS = np.random.default_rng(seed + 3).standard_normal(len(anchors)).astype(F32)
    close_rel(N(plan.backward(T(gS))), O.ats_pair_bwd(gS, p, h, tau, 3.0, len(t)), 1e-4)
    return wcnt


# at most 8, 9, 12 and 16 slices per source (the entry passes keep up to 12 in registers, more take two passes)
@pytest.mark.parametrize("tau,S,h", [(0.2, 16, 1.0), (1.0, 8, 1.5), (0.05, 4, 0.5), (0.2, 16, 2.0), (0.3, 16, 1.0),
                                     (0.6, 16, 1.0)])
def test_fast_matches_oracle(tau, S, h):
    win, xs, v, xa = _case(seed=11, h=h)
    cnt = check_against_oracle(xs, win.t, v, win.b, 2, 40, 48, np.arange(win.n), xa, h, tau, S)
    assert cnt.sum() > win.n                 # the case has real neighbourhoods


def test_fast_anchor_subsets_and_raw_positions():
    win, xs, v, xa = _case(seed=12)
    rng = np.random.default_rng(0)
    perm = rng.permutation(win.n)[: win.n // 3]              # unsorted subset, smoothed positions
    check_against_oracle(xs, win.t, v, win.b, 2, 40, 48, perm, xa[perm], 1.0, 0.2, 16)
    every3 = np.arange(0, win.n, 3)                          # x[anchors] (anchor_xy None)
    check_against_oracle(xs, win.t, v, win.b, 2, 40, 48, every3, None, 1.0, 0.2, 16)


def test_fast_duplicate_anchors():
    """An event listed twice among the anchors: both records skip exactly their own event (leave-one-out by id,
    the backward's fallback from the own-record position test)."""
    win, xs, v, xa = _case(seed=15)
    anchors = np.concatenate([np.arange(0, win.n, 2), np.arange(0, win.n, 6)])
    check_against_oracle(xs, win.t, v, win.b, 2, 40, 48, anchors, None, 1.0, 0.2, 16)
    check_against_oracle(xs, win.t, v, win.b, 2, 40, 48, anchors, xa[anchors], 1.0, 0.2, 16)


def test_fast_reference_test_shape():
    """tests/test_ops.py:62-77 shape: n=600, B=2, 20x24, positions in [-2, W+2), v = 6 N(0,1), h=1.5."""
    pos, _, b, t = rand_events(n=600, seed=3)
    v = (np.random.default_rng(1).standard_normal((600, 2)) * 6).astype(F32)
    anchors = np.arange(0, 600, 3)
    for tau, S in [(1.0, 8), (0.2, 16), (0.05, 4)]:
        check_against_oracle(pos, t, v, b, 2, 20, 24, anchors, None, 1.5, tau, S)


def test_fast_edge_cases():
    rng = np.random.default_rng(5)
    # coincident events: many at the same position and time (ties in t, d2 = 0, leave-one-out by id)
    n = 400
    xs = np.repeat(np.array([[10.0, 7.0], [30.0, 20.0]], F32), n // 2, axis=0)
    t = np.sort(np.repeat(rng.random(n // 8).astype(F32), 8))
    v = np.zeros((n, 2), F32)
    b = np.zeros(n, np.int64)
    check_against_oracle(xs, t, v, b, 1, 40, 48, np.arange(n), None, 1.0, 0.2, 16)
    # positions and slice-centre positions far outside the sensor (clamped bins), large velocities
    win, xs, v, xa = _case(seed=13)
    xs2 = xs.copy()
    xs2[::7] += F32(300.0)
    xs2[1::7] -= F32(250.0)
    v2 = (v * F32(8.0)).astype(F32)
    check_against_oracle(xs2, win.t, v2, win.b, 2, 40, 48, np.arange(win.n), xa, 1.0, 0.2, 16)
    # times exactly on slice boundaries and at 0 / 1
    t3 = np.sort(np.concatenate([np.arange(17, dtype=F32) / F32(16), rng.random(583).astype(F32)]))
    xs3 = (rng.random((600, 2)) * [48, 40]).astype(F32)
    v3 = (rng.standard_normal((600, 2)) * 3).astype(F32)
    check_against_oracle(xs3, t3, v3, np.zeros(600, np.int64), 1, 40, 48, np.arange(600), None, 1.0, 0.2, 16)


def test_fast_empty_inputs():
    x = torch.zeros(0, 2, device=DEV)
    t = torch.zeros(0, device=DEV)
    b = torch.zeros(0, dtype=torch.int64, device=DEV)
    plan = F.FastPairPlan(x, t, x, b, 1, 40, 48, b, 1.0, 0.2)
    assert plan.forward().shape == (0,) and plan.backward(t).shape == (0, 2)
    # events but no anchors
    win, xs, v, xa = _case(seed=14)
    plan = F.FastPairPlan(T(xs), T(win.t), T(v), T(win.b), 2, 40, 48, torch.zeros(0, dtype=torch.int64, device=DEV),
                          1.0, 0.2)
    assert plan.forward().shape == (0,)
    assert float(plan.backward(torch.zeros(0, device=DEV)).abs().sum()) == 0.0


def test_fast_api_autograd_matches_bruteforce():
    """ats_pair_sums on device (the fused path) vs the O(MN) fp64 brute force, values and gradients."""
    pos, _, b, t = rand_events(n=600, seed=3)
    rng = np.random.default_rng(1)
    v = (rng.standard_normal((600, 2)) * 6).astype(F32)
    anchors = np.arange(0, 600, 3)
    for tau, S in [(1.0, 8), (0.2, 16), (0.05, 4)]:
        tv = T(v).requires_grad_(True)
        s_ext = F.ats_pair_sums(T(pos), T(t), tv, T(b), 2, 20, 24, T(anchors), 1.5, tau, cut=3.0, n_slices=S)
        Sb, _, grad = O.pair_sums_fp64(pos, t, v, b, anchors, 1.5, tau, 3.0)
        assert np.allclose(N(s_ext), Sb, atol=1e-4, rtol=1e-4)
        gS = rng.standard_normal(len(anchors)).astype(F32)
        s_ext.backward(T(gS))
        assert np.allclose(N(tv.grad), grad(gS), atol=1e-4, rtol=1e-3)


def test_fast_plumbing_size_matches_oracle():
    """100k events on 240x180 (translation 2.0, -1.25 px per window): every event an anchor, vs the oracle."""
    win = synth.plumbing_translation(seed=0)
    rng = np.random.default_rng(21)
    xs = (win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(F32)
    xa = (xs + rng.standard_normal(xs.shape)).astype(F32)
    v = np.broadcast_to(np.asarray(win.motion["theta"][:2], F32), xs.shape).copy()
    check_against_oracle(xs, win.t, v, win.b, 1, win.height, win.width, np.arange(win.n), xa, 1.0, 0.2, 16)


@pytest.mark.parametrize("h", [1.0, 0.5, 2.0])
def test_fast_full_size_matches_oracle(h):
    """The headline window at full size, directly against the oracle: 1M events at 640x480 (dense flow,
    dequantised sources, smoothed anchors, every event an anchor without an index array, as benchmarked), tau =
    0.2, 16 slices: every per-anchor count bit-exact, sums within 1e-5, velocity gradients within 1e-4."""
    win = synth.dense_flow_window(seed=0)
    rng = np.random.default_rng(0)
    xs = (win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(F32)
    xa = (xs + h * rng.standard_normal(xs.shape)).astype(F32)
    v, _, _ = O.dense_velocity(win.motion["grid"], xs, win.b, 480, 640)
    cnt = check_against_oracle(xs, win.t, v, win.b, 1, 480, 640, np.arange(win.n), xa, h, 0.2, 16, index_free=True)
    assert cnt.sum() > 10 * win.n


def test_fast_blob_contention_matches_oracle():
    """Contention shape against the oracle: 4M events, 90% in 5 Gaussian blobs (sigma 8 px), Sim2 flow
    (0, 0, 0.1, 0.1), h = 1, a random 40k-anchor subset (thousands of neighbours each): counts bit-exact, sums
    within 1e-5, gradients within 1e-4."""
    win = synth.blob_window(seed=0)
    rng = np.random.default_rng(1)
    xs = (win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(F32)
    th = win.motion["theta"].astype(F32)
    c = np.array([(640 - 1) / 2.0, (480 - 1) / 2.0], F32)
    d = (xs - c).astype(F32)
    v = np.stack([th[0] + (th[2] * d[:, 0] - th[3] * d[:, 1]), th[1] + (th[3] * d[:, 0] + th[2] * d[:, 1])],
                 1).astype(F32)
    anchors = np.sort(rng.choice(win.n, 40_000, replace=False))
    xa = (xs[anchors] + rng.standard_normal((len(anchors), 2))).astype(F32)
    cnt = check_against_oracle(xs, win.t, v, win.b, 1, 480, 640, anchors, xa, 1.0, 0.2, 16)
    assert cnt.mean() > 1000


@pytest.mark.parametrize("h", [1.0, 0.5, 2.0])
def test_fast_full_size_matches_reference_layout(h):
    """1M events at 640x480 (dense flow, dequantised sources, smoothed anchors, all anchors): the fused path
    against the reference-layout device plan + kernels (themselves pinned to the oracle above): counts
    bit-exact, sums within 1e-5, gradients within 1e-4."""
    print(f"full size h={h}", flush=True)
    win = synth.dense_flow_window(seed=0)
    rng = np.random.default_rng(0)
    xs = (win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(F32)
    xa = (xs + h * rng.standard_normal(xs.shape)).astype(F32)
    v, _, _ = O.dense_velocity(win.motion["grid"], xs, win.b, 480, 640)
    anchors = T(np.arange(win.n))
    tx, tt, tv, tb, txa = T(xs), T(win.t), T(v), T(win.b), T(xa)
    ref_plan = F.build_pair_plan(tx, tt, tv, tb, 1, 480, 640, anchors, h, 0.2, 3.0, 16, anchor_xy=txa)
    want_cnt = N(F.pair_counts(ref_plan, h, 0.2, 3.0))
    e = F.get_ext()
    p = ref_plan
    want = N(e.ats_pair_fwd(p.src_y, p.src_v, p.src_t, p.src_id, p.cell_start, p.anc_x, p.anc_t, p.anc_cell,
                            p.anc_id, p.slice_c, p.S, p.GH, p.GW, h, 0.2, 3.0))
    plan = F.FastPairPlan(tx, tt, tv, tb, 1, 480, 640, anchors, h, 0.2, 3.0, 16, txa)
    assert np.array_equal(N(plan.counts()), want_cnt)
    assert_sums_close(N(plan.forward()), want)
    gS = torch.randn(win.n, device=DEV, generator=torch.Generator(device=DEV).manual_seed(4))
    gv_ref = N(e.ats_pair_bwd(gS, p.src_y, p.src_v, p.src_t, p.src_id, p.cell_start, p.anc_x, p.anc_t, p.anc_cell,
                              p.anc_id, p.slice_c, p.S, p.GH, p.GW, h, 0.2, 3.0, win.n))
    close_rel(N(plan.backward(gS)), gv_ref, 1e-4)


def test_fast_blob_contention_matches_reference_layout():
    """Contention stress shape: 4M events, 90% in 5 Gaussian blobs (sigma 8 px), Sim2 flow (0, 0, 0.1, 0.1),
    h = 1, a random 40k-anchor subset: fused path against the reference-layout device plan and kernels
    (counts bit-exact, sums within 1e-5, gradients within 1e-4)."""
    print("blob contention, 4M events", flush=True)
    win = synth.blob_window(seed=0)
    rng = np.random.default_rng(0)
    xs = (win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(F32)
    th = win.motion["theta"].astype(F32)
    c = np.array([(640 - 1) / 2.0, (480 - 1) / 2.0], F32)
    d = (xs - c).astype(F32)
    v = np.stack([th[0] + (th[2] * d[:, 0] - th[3] * d[:, 1]), th[1] + (th[3] * d[:, 0] + th[2] * d[:, 1])],
                 1).astype(F32)
    anchors = np.sort(rng.choice(win.n, 40_000, replace=False))
    xa = (xs[anchors] + rng.standard_normal((len(anchors), 2))).astype(F32)
    tx, tt, tv, tb, ta, txa = T(xs), T(win.t), T(v), T(win.b), T(anchors), T(xa)
    ref_plan = F.build_pair_plan(tx, tt, tv, tb, 1, 480, 640, ta, 1.0, 0.2, 3.0, 16, anchor_xy=txa)
    want_cnt = N(F.pair_counts(ref_plan, 1.0, 0.2, 3.0))
    assert want_cnt.mean() > 1000                       # dense neighbourhoods
    e = F.get_ext()
    p = ref_plan
    args = (p.src_y, p.src_v, p.src_t, p.src_id, p.cell_start, p.anc_x, p.anc_t, p.anc_cell, p.anc_id, p.slice_c,
            p.S, p.GH, p.GW, 1.0, 0.2, 3.0)
    want = N(e.ats_pair_fwd(*args))
    plan = F.FastPairPlan(tx, tt, tv, tb, 1, 480, 640, ta, 1.0, 0.2, 3.0, 16, txa)
    assert np.array_equal(N(plan.counts()), want_cnt)
    assert_sums_close(N(plan.forward()), want)
    gS = torch.randn(len(anchors), device=DEV, generator=torch.Generator(device=DEV).manual_seed(5))
    close_rel(N(plan.backward(gS)), N(e.ats_pair_bwd(gS, *args, win.n)), 1e-4)


@pytest.mark.parametrize("B,H,W,Hg,Wg,h", [(2, 40, 48, 40, 48, 1.0), (2, 37, 53, 9, 14, 0.5), (1, 30, 36, 30, 1, 2.0),
                                            (3, 24, 20, 2, 2, 1.0)])
def test_pair_sums_flow_matches_oracle(B, H, W, Hg, Wg, h):
    """ats_pair_sums_flow (the flow sampled inside, its gradient accumulated over the plan's source records) against
    the oracle: sums within 1e-5, and the flow-grid gradient (pair backward, then sample_grid's adjoint) within
    1e-4, on full-resolution, coarse and degenerate grids, with sources far outside the sensor (clamped into the
    border nodes and the plan's box, so that their records fall outside the tile's window)."""
    print(f"pair sums flow B={B} {H}x{W} grid {Hg}x{Wg} h={h}", flush=True)
    rng = np.random.default_rng(B * 100 + Hg)
    n = 2500 * B
    win = synth.small_window(seed=Hg + Wg, n=n // B, H=H, W=W, B=B)
    grid = (rng.standard_normal((B, 2, Hg, Wg)) * 4.0).astype(F32)
    xs = (win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(F32)
    xs[::97] = np.array([-40.0, 7.5], F32)                       # far outside: clamped in the grid and the box
    xs[1::101] = np.array([W + 30.0, H + 25.0], F32)
    xa = (xs + h * rng.standard_normal(xs.shape)).astype(F32)
    v, idx, wts = O.dense_velocity(grid, xs, win.b, H, W)
    anchors = np.arange(win.n)
    p = O.build_pair_plan(xs, win.t, v, win.b, B, H, W, anchors, h, 0.2, 3.0, 16, anchor_xy=xa)
    want = O.ats_pair_fwd(p, h, 0.2, 3.0)
    gS = rng.standard_normal(win.n).astype(F32)
    want_g = O.sample_grid_bwd(O.ats_pair_bwd(gS, p, h, 0.2, 3.0, win.n), idx, wts, grid.shape)
    tg = T(grid).requires_grad_(True)
    S = F.ats_pair_sums_flow(tg, T(xs), T(win.t), T(win.b), B, H, W, None, h, 0.2, 3.0, 16, anchor_xy=T(xa))
    assert_sums_close(N(S), want)
    (S * T(gS)).sum().backward()
    close_rel(N(tg.grad), want_g, 1e-4)


def test_pair_sums_flow_full_size_matches_composed():
    """1M events, 640x480, dense flow: the flow path's sums and grid gradient against sampling the flow and calling
    ats_pair_sums (whose own backward goes through sample_grid's binned adjoint)."""
    print("pair sums flow vs composed, 1M events", flush=True)
    win = synth.dense_flow_window(seed=0)
    H, W = win.height, win.width
    rng = np.random.default_rng(5)
    xs = T((win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(F32))
    xa = T((N(xs) + rng.standard_normal(win.xy.shape)).astype(F32))
    t, b = T(win.t), T(win.b)
    gS = torch.randn(win.n, device=DEV)
    res = []
    for fused in (True, False):
        tg = T(win.motion["grid"]).requires_grad_(True)
        if fused:
            S = F.ats_pair_sums_flow(tg, xs, t, b, 1, H, W, None, 1.0, 0.2, 3.0, 16, anchor_xy=xa)
        else:
            v = F.sample_grid_hip(tg, xs, b, img_hw=(H, W))
            S = F.ats_pair_sums(xs, t, v, b, 1, H, W, None, 1.0, 0.2, 3.0, 16, anchor_xy=xa)
        (S * gS).sum().backward()
        res.append((N(S), N(tg.grad)))
    # the same pairs; the within-cell record order follows the plan's LDS atomics, so sums differ in the last bits
    assert_sums_close(res[0][0], res[1][0])
    close_rel(res[0][1], res[1][1], 1e-4)
