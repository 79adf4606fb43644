"""Pins of the oracle (CPU): every oracle function is checked against the reference's own known-answer tests,
fp64 brute force of the defining sums, closed forms and invariants, chosen so that a dropped term, a wrong
sign or index, or a transposed operand fails at least one of them."""
import math

import numpy as np
import pytest
import torch

import oracle as O
from tests.conftest import rand_events
from x_amd import synth

F32 = np.float32


# ------------------------------------------------------------------------------------------- fp64 helpers
def splat_fp64(pos, w, b, B, H, W):
    img = np.zeros((B, H, W))
    for n in range(len(w)):
        x, y = float(pos[n, 0]), float(pos[n, 1])
        x0, y0 = math.floor(x), math.floor(y)
        ax, ay = x - x0, y - y0
        for dx, wx in ((0, 1 - ax), (1, ax)):
            for dy, wy in ((0, 1 - ay), (1, ay)):
                xx, yy = x0 + dx, y0 + dy
                if 0 <= xx < W and 0 <= yy < H:
                    img[b[n], yy, xx] += float(w[n]) * wx * wy
    return img


def gather_fp64(img, pos, b):
    B, H, W = img.shape
    out = np.zeros(len(pos))
    for n in range(len(pos)):
        x, y = float(pos[n, 0]), float(pos[n, 1])
        x0, y0 = math.floor(x), math.floor(y)
        ax, ay = x - x0, y - y0
        for dx, wx in ((0, 1 - ax), (1, ax)):
            for dy, wy in ((0, 1 - ay), (1, ay)):
                xx, yy = x0 + dx, y0 + dy
                if 0 <= xx < W and 0 <= yy < H:
                    out[n] += wx * wy * float(img[b[n], yy, xx])
    return out


# ------------------------------------------------------------------------------------------- splat / gather
def test_splat_matches_fp64_brute_force():
    pos, w, b, _ = rand_events(n=400, seed=1)
    got = O.splat_bilinear_fwd(pos, w, b, 2, 20, 24)
    assert np.allclose(got, splat_fp64(pos, w, b, 2, 20, 24), atol=2e-6, rtol=1e-6)


def test_splat_mass_conservation_and_integer_positions():
    rng = np.random.default_rng(2)
    pos = np.stack([rng.uniform(1, 22, 300), rng.uniform(1, 18, 300)], 1).astype(F32)
    w = rng.uniform(0.5, 2, 300).astype(F32)
    b = np.zeros(300, np.int64)
    img = O.splat_bilinear_fwd(pos, w, b, 1, 20, 24)
    assert abs(float(img.sum(dtype=np.float64)) - float(w.sum(dtype=np.float64))) < 1e-3
    ip = np.round(pos).astype(F32)
    img = O.splat_bilinear_fwd(ip, w, b, 1, 20, 24)
    for n in range(20):   # an integer position deposits its whole weight into exactly one pixel
        one = O.splat_bilinear_fwd(ip[n:n + 1], w[n:n + 1], b[n:n + 1], 1, 20, 24)
        assert (one != 0).sum() == 1 and one[0, int(ip[n, 1]), int(ip[n, 0])] == w[n]


def test_gather_matches_fp64_and_adjoint_identities():
    pos, w, b, _ = rand_events(n=400, seed=3)
    rng = np.random.default_rng(4)
    G = rng.standard_normal((2, 20, 24)).astype(F32)
    val = O.gather_bilinear_fwd(G, pos, b)
    assert np.allclose(val, gather_fp64(G, pos, b), atol=1e-5)
    # <splat(w), G> = <w, gather(G)>
    lhs = float((O.splat_bilinear_fwd(pos, w, b, 2, 20, 24).astype(np.float64) * G).sum())
    rhs = float((w.astype(np.float64) * val).sum())
    assert abs(lhs - rhs) < 1e-3 * max(1.0, abs(lhs))
    # splat_bwd.gw == gather_fwd(gimg) at the same positions (same corner order: bit-identical)
    gp, gw = O.splat_bilinear_bwd(G, pos, w, b)
    assert np.array_equal(gw, val)
    # gather_bwd.gimg with gval = w is the splat of w
    gimg, _ = O.gather_bilinear_bwd(w, G, pos, b)
    assert np.allclose(gimg, O.splat_bilinear_fwd(pos, w, b, 2, 20, 24), atol=1e-5)


def test_splat_and_gather_position_gradients_by_finite_differences():
    rng = np.random.default_rng(5)
    n = 60
    pos = np.stack([rng.uniform(2.1, 20.9, n), rng.uniform(2.1, 16.9, n)], 1)
    frac = pos - np.floor(pos)
    pos[(frac < 0.05) | (frac > 0.95)] += 0.3          # stay away from integer crossings
    pos = pos.astype(F32)
    w = rng.uniform(0.5, 1.5, n).astype(F32)
    b = np.zeros(n, np.int64)
    G = rng.standard_normal((1, 20, 24)).astype(F32)
    gp, _ = O.splat_bilinear_bwd(G, pos, w, b)
    gval = rng.standard_normal(n).astype(F32)
    _, gp2 = O.gather_bilinear_bwd(gval, G, pos, b)
    eps = 1e-3
    for k in range(2):
        d = np.zeros_like(pos, dtype=np.float64)
        d[:, k] = eps
        p1, p0 = pos.astype(np.float64) + d, pos.astype(np.float64) - d
        fd = (gather_fp64(G, p1, b) - gather_fp64(G, p0, b)) / (2 * eps)   # d<splat(w), G>/dpos = w * dgather
        assert np.allclose(gp[:, k], w * fd, atol=1e-3, rtol=1e-3)
        assert np.allclose(gp2[:, k], gval * fd, atol=1e-3, rtol=1e-3)


def test_gauss_splat_mass_is_normalised():
    # known-answer test of the reference, tests/test_ops.py:97-100
    img = O.splat_gauss_fwd(np.array([[10.3, 7.6]], F32), np.ones(1, F32), np.zeros(1, np.int64), 1, 20, 24, 1.0, 3)
    assert abs(float(img.sum()) - 1.0) < 3e-3


def test_gauss_splat_matches_fp64_and_gradient():
    pos, w, b, _ = rand_events(n=200, seed=6)
    sigma, R = 1.3, 4
    img = O.splat_gauss_fwd(pos, w, b, 2, 20, 24, sigma, R)
    ref = np.zeros((2, 20, 24))
    for n in range(len(w)):
        cx, cy = int(math.floor(pos[n, 0] + 0.5)), int(math.floor(pos[n, 1] + 0.5))
        for yy in range(max(cy - R, 0), min(cy + R, 19) + 1):
            for xx in range(max(cx - R, 0), min(cx + R, 23) + 1):
                d2 = (xx - float(pos[n, 0])) ** 2 + (yy - float(pos[n, 1])) ** 2
                ref[b[n], yy, xx] += float(w[n]) * math.exp(-d2 / (2 * sigma ** 2)) / (2 * math.pi * sigma ** 2)
    assert np.allclose(img, ref, atol=1e-5)
    G = np.random.default_rng(7).standard_normal((2, 20, 24)).astype(F32)
    _, gw = O.splat_gauss_bwd(G, pos, w, b, sigma, R)
    lhs = float((ref * G).sum())
    assert abs(lhs - float((gw.astype(np.float64) * w).sum())) < 1e-3 * max(1, abs(lhs))


def test_voxel_grid_mass_and_placement():
    rng = np.random.default_rng(8)
    n = 200
    pos = np.stack([rng.uniform(1, 22, n), rng.uniform(1, 18, n)], 1).astype(F32)
    t = rng.uniform(0, 1, n).astype(F32)
    p = np.where(rng.uniform(size=n) < 0.5, 1.0, -1.0).astype(F32)
    b = rng.integers(0, 2, n).astype(np.int64)
    vox = O.voxel_grid(pos, t, p, b, 2, 5, 20, 24)
    for k in range(2):   # trilinear weights of an interior event sum to one
        assert abs(float(vox[k].sum()) - float(p[b == k].sum())) < 1e-3
    one = O.voxel_grid(np.array([[3.0, 4.0]], F32), np.array([0.5], F32), np.ones(1, F32), np.zeros(1, np.int64),
                       1, 5, 20, 24)
    assert one[0, 2, 4, 3] == 1.0 and (one != 0).sum() == 1


# ------------------------------------------------------------------------------------------- window counts
def test_window_counts_known_answer():
    # tests/test_ops.py:90-95 of the reference
    c = O.window_counts(np.array([0.0, 0.1, 0.2, 0.9, 0.0, 0.5], F32), np.array([0, 0, 0, 0, 1, 1]), np.arange(6), 0.15)
    assert c.tolist() == [1, 2, 1, 0, 0, 0]


def test_window_counts_brute_force():
    _, _, b, t = rand_events(n=700, B=3, seed=9)
    idx = np.arange(0, 700, 3)
    got = O.window_counts(t, b, idx, 0.07)
    td = t.astype(np.float64)
    want = [(((b == b[i]) & (np.abs(td - td[i]) <= 0.07)).sum() - 1) for i in idx]
    assert got.tolist() == want


# ------------------------------------------------------------------------------------------- pair plan + sums
def test_vmax_matches_torch_cpu_norm():
    if torch.backends.cpu.get_cpu_capability() == "DEFAULT":
        pytest.skip("torch CPU kernels without FMA: a different rounding of the norm")
    v = np.random.default_rng(10).standard_normal((200_000, 2)).astype(F32) * 7
    vt = torch.from_numpy(v)
    assert O.vmax(v) == float(vt.norm(dim=1).max())
    for k in range(0, 200_000, 20_000):          # per-vector agreement, not only the maximum
        assert O.vmax(v[k:k + 1]) == float(vt[k].norm())


def _dense_case(seed=0, n=2500, B=2, H=40, W=48):
    win = synth.small_window(seed=seed, n=n // B, H=H, W=W, B=B)
    v, _, _ = O.dense_velocity(win.motion["grid"], win.xy, win.b, H, W)
    return win, v


def test_plan_invariants():
    win, v = _dense_case(seed=1)
    anchors = np.arange(0, win.n, 2)
    p = O.build_pair_plan(win.xy, win.t, v, win.b, 2, 40, 48, anchors, 1.2, 0.2, 3.0, 16)
    key, cs = p["key"], p["cell_start"]
    assert np.all(np.diff(key) >= 0)
    assert cs[0] == 0 and cs[-1] == key.shape[0] and np.all(np.diff(cs) >= 0)
    assert np.array_equal(np.diff(cs), np.bincount(key, minlength=cs.shape[0] - 1))
    s_lo, s_hi = O.slice_range(win.t, 0.2, 16)
    ids, cnt = np.unique(p["src_id"], return_counts=True)
    full = cnt == (s_hi - s_lo + 1)[ids]            # sources with no entry dropped by the grid
    assert full.mean() > 0.9
    assert np.all(cnt <= (s_hi - s_lo + 1)[ids])
    # each entry's position lies in its cell
    geo = p["geometry"]
    cx = key % p["GW"]
    cy = (key // p["GW"]) % p["GH"]
    assert np.all(np.floor((p["src_y"][:, 0] - F32(geo["ox"])) / F32(geo["cell"])) == cx)
    assert np.all(np.floor((p["src_y"][:, 1] - F32(geo["oy"])) / F32(geo["cell"])) == cy)


def test_numpy_plan_matches_torch_op_rounding():
    """The NumPy restatement rounds like torch's CPU ops (the reference builds its plan with them)."""
    from x_amd.ops.functional import _build_pair_plan_torch
    win, v = _dense_case(seed=2)
    anchors = np.arange(0, win.n, 3)
    xa = win.xy[anchors] + np.random.default_rng(3).standard_normal((len(anchors), 2)).astype(F32)
    p = O.build_pair_plan(win.xy, win.t, v, win.b, 2, 40, 48, anchors, 1.0, 0.2, 3.0, 16, anchor_xy=xa)
    T = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    q = _build_pair_plan_torch(T(win.xy), T(win.t), T(v), T(win.b), 2, 40, 48, T(anchors), 1.0, 0.2, 3.0, 16,
                               T(xa))
    assert (q.GH, q.GW) == (p["GH"], p["GW"])
    assert np.array_equal(q.cell_start.numpy(), p["cell_start"])
    assert np.array_equal(q.src_id.numpy(), p["src_id"])          # both stable sorts
    assert np.array_equal(q.src_y.numpy(), p["src_y"])
    assert np.array_equal(q.anc_cell.numpy(), p["anc_cell"])


@pytest.mark.parametrize("tau,S,h", [(0.2, 16, 1.0), (1.0, 8, 1.5), (0.05, 4, 0.7)])
def test_pair_sums_match_fp64_brute_force(tau, S, h):
    win, v = _dense_case(seed=4, n=2000)
    anchors = np.arange(0, win.n, 2)
    rng = np.random.default_rng(5)
    xs = (win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(F32)
    xa = (xs[anchors] + h * rng.standard_normal((len(anchors), 2))).astype(F32)
    p = O.build_pair_plan(xs, win.t, v, win.b, 2, 40, 48, anchors, h, tau, 3.0, S, anchor_xy=xa)
    Sv, cnt = O.ats_pair_fwd(p, h, tau, 3.0, with_counts=True)
    Sb, cb, grad = O.pair_sums_fp64(xs, win.t, v, win.b, anchors, h, tau, 3.0, anchor_xy=xa)
    amb = O.near_boundary_pairs(xs, win.t, v, win.b, anchors, h, tau, 3.0, anchor_xy=xa)
    ok = amb == 0
    assert ok.mean() > 0.95
    assert np.array_equal(cnt[ok], cb[ok])
    assert np.allclose(Sv[ok], Sb[ok], rtol=1e-5, atol=1e-6)
    gS = (rng.standard_normal(len(anchors)) * ok).astype(F32)
    gv = O.ats_pair_bwd(gS, p, h, tau, 3.0, win.n)
    want = grad(gS)
    scale = np.abs(want).max()
    assert np.allclose(gv, want, rtol=1e-4, atol=1e-5 * scale)


def test_pair_sums_closed_forms():
    # a single pair, static: S = exp(-d^2 / 2h^2); the anchor itself is left out
    x = np.array([[10.0, 10.0], [11.2, 10.5]], F32)
    t = np.array([0.5, 0.5], F32)
    v = np.zeros((2, 2), F32)
    b = np.zeros(2, np.int64)
    p = O.build_pair_plan(x, t, v, b, 1, 20, 20, np.array([0]), 1.0, 0.2, 3.0, 16)
    Sv, cnt = O.ats_pair_fwd(p, 1.0, 0.2, 3.0, with_counts=True)
    assert cnt[0] == 1 and abs(Sv[0] - math.exp(-(1.2 ** 2 + 0.5 ** 2) / 2)) < 1e-6
    # moving source: its position is transported to the anchor time, x_j + v_j (t_i - t_j)
    t2 = np.array([0.5, 0.4], F32)
    v2 = np.array([[0, 0], [-12.0, -5.0]], F32)       # at t=0.5 the source sits at (10.0, 10.0)
    p = O.build_pair_plan(x, t2, v2, b, 1, 20, 20, np.array([0]), 1.0, 0.2, 3.0, 16)
    Sv = O.ats_pair_fwd(p, 1.0, 0.2, 3.0)
    assert abs(Sv[0] - 1.0) < 1e-5
    gv = O.ats_pair_bwd(np.ones(1, F32), p, 1.0, 0.2, 3.0, 2)
    assert np.allclose(gv, 0.0, atol=1e-5)                  # r = 0: zero gradient
    # tau -> 0: only simultaneous events count; an isolated anchor scores 0
    x3 = np.array([[5, 5], [5.5, 5], [6, 5], [15, 15]], F32)
    t3 = np.array([0.3, 0.3, 0.31, 0.3], F32)
    p = O.build_pair_plan(x3, t3, np.zeros((4, 2), F32), np.zeros(4, np.int64), 1, 20, 20, np.arange(4), 1.0, 1e-6,
                          3.0, 16)
    Sv, cnt = O.ats_pair_fwd(p, 1.0, 1e-6, 3.0, with_counts=True)
    assert cnt.tolist() == [1, 1, 0, 0] and Sv[3] == 0.0
    assert abs(Sv[0] - math.exp(-0.125)) < 1e-6


# ------------------------------------------------------------------------------------------- motion pieces
def test_sample_grid_is_exact_on_linear_fields_and_clamps_at_the_border():
    Hg, Wg = 7, 9
    yy, xx = np.meshgrid(np.arange(Hg), np.arange(Wg), indexing="ij")
    field = np.stack([1.5 + 0.25 * xx - 0.5 * yy, -2.0 + 0.125 * xx + 0.75 * yy])[None].astype(F32)
    rng = np.random.default_rng(11)
    g = np.stack([rng.uniform(0, Wg - 1, 500), rng.uniform(0, Hg - 1, 500)], 1).astype(F32)
    out, _, _ = O.sample_grid(field, g, np.zeros(500, np.int64))
    gd = g.astype(np.float64)
    want = np.stack([1.5 + 0.25 * gd[:, 0] - 0.5 * gd[:, 1], -2.0 + 0.125 * gd[:, 0] + 0.75 * gd[:, 1]], 1)
    assert np.allclose(out, want, atol=1e-5)
    far = np.array([[-3.0, -1.0], [20.0, 30.0], [Wg - 1.0, Hg - 1.0]], F32)
    out, _, _ = O.sample_grid(field, far, np.zeros(3, np.int64))
    assert np.allclose(out[0], field[0, :, 0, 0]) and np.allclose(out[1], field[0, :, -1, -1])
    assert np.allclose(out[2], field[0, :, -1, -1])


def test_sample_grid_backward_is_the_adjoint():
    rng = np.random.default_rng(12)
    field = rng.standard_normal((2, 2, 6, 8)).astype(F32)
    g = np.stack([rng.uniform(-1, 8, 300), rng.uniform(-1, 6, 300)], 1).astype(F32)
    b = rng.integers(0, 2, 300)
    out, idx, wts = O.sample_grid(field, g, b)
    go = rng.standard_normal(out.shape).astype(F32)
    gf = O.sample_grid_bwd(go, idx, wts, field.shape)
    assert abs(float((gf.astype(np.float64) * field).sum()) - float((go.astype(np.float64) * out).sum())) < 1e-3


def test_visible_fraction_closed_form_translation():
    rng = np.random.default_rng(13)
    H, W, M = 30, 40, 400
    xa = np.stack([rng.uniform(-5, 45, M), rng.uniform(-3, 33, M)], 1).astype(F32)
    ta = rng.uniform(0, 1, M).astype(F32)
    vx = 12.0
    grid = np.zeros((1, 2, 2, 2), F32)
    grid[0, 0] = vx                                              # uniform velocity (vx, 0)
    t_all = np.sort(rng.uniform(0, 1, 5000)).astype(F32)
    vis = O.visible_fraction_dense(grid, xa, ta, np.zeros(M, np.int64), t_all, np.zeros(5000, np.int64), 1, H, W, 0.3)
    counts = np.bincount(np.clip((t_all * 16).astype(int), 0, 15), minlength=16).astype(np.float64)
    c = (np.arange(16) + 0.5) / 16
    want = np.empty(M)
    for i in range(M):
        wgt = counts * (np.abs(ta[i] - c) <= 0.3)
        y = xa[i, 0] + vx * (c - ta[i])
        ins = (y >= 0) & (y <= W - 1) & (xa[i, 1] >= 0) & (xa[i, 1] <= H - 1)
        want[i] = max((wgt * ins).sum() / max(wgt.sum(), 1), 1e-3)
    assert np.allclose(vis, want, atol=1e-6)
    inside = (xa[:, 1] >= 0) & (xa[:, 1] <= H - 1) & (xa[:, 0] >= 12) & (xa[:, 0] <= W - 13)
    assert np.all(vis[inside] == 1.0)


def test_anchored_epilogue_closed_form():
    rng = np.random.default_rng(14)
    S = rng.uniform(0, 50, 100).astype(F32)
    wc = rng.integers(0, 200, 100).astype(F32)
    ls, gS, D = O.anchored_epilogue(S, wc, 1.3, 48, 64)
    Dd = np.maximum(wc, 1) * 2 * math.pi * 1.3 ** 2
    qd = 1e-2 / (48 * 64) + S / Dd
    assert np.allclose(ls, np.log(qd), rtol=1e-6, atol=1e-6)
    assert np.allclose(gS, -1.0 / 100 / qd / Dd, rtol=1e-5)


def test_dense_grid_pos_aligns_the_corners():
    """DenseLinearFlow's pixel -> grid map (atl/motion/parametric.py:214-215) with Hg != H, Wg != W: pixel 0 lands
    on node 0 and pixel W-1 (H-1) on node Wg-1 (Hg-1), so a field linear in the node index is sampled as the same
    linear function of the pixel, scaled by (Wg-1)/(W-1)."""
    H, W, Hg, Wg = 48, 64, 7, 11
    corners = np.array([[0, 0], [W - 1, 0], [0, H - 1], [W - 1, H - 1]], F32)
    g = O.dense_grid_pos(corners, H, W, Hg, Wg)
    assert np.array_equal(g, np.array([[0, 0], [Wg - 1, 0], [0, Hg - 1], [Wg - 1, Hg - 1]], F32))
    yy, xx = np.meshgrid(np.arange(Hg), np.arange(Wg), indexing="ij")
    grid = np.stack([0.5 * xx + 2.0, -0.25 * yy + 1.0])[None].astype(F32)
    rng = np.random.default_rng(15)
    xy = np.stack([rng.uniform(0, W - 1, 300), rng.uniform(0, H - 1, 300)], 1).astype(F32)
    v, _, _ = O.dense_velocity(grid, xy, np.zeros(300, np.int64), H, W)
    want = np.stack([0.5 * xy[:, 0] * (Wg - 1) / (W - 1) + 2.0, -0.25 * xy[:, 1] * (Hg - 1) / (H - 1) + 1.0], 1)
    assert np.allclose(v, want, atol=1e-5)


# ------------------------------------------------------------------------------------------- trajectories
@pytest.mark.parametrize("K", [1, 2, 3, 4, 10, 12])
def test_traj_basis_bspline_identities(K):
    """The B-spline table (scipy's BSpline): with N_0 = 1 - sum_k g_k, the K + 1 functions are a partition of
    unity, non-negative, reproduce t at the Greville abscissae (linear precision), vanish at t = 0 for k >= 1;
    K = 1 is t and K = 2 the quadratic Bernstein basis; derivatives match central differences."""
    t = np.linspace(0, 1, 101)[:-1]
    g, gd = O.traj_basis_table(t, K, "bspline")
    P, L = min(3, K), K + 1 - min(3, K)
    knots = np.concatenate([np.zeros(P), np.linspace(0, 1, L + 1), np.ones(P)])
    xi = np.array([knots[k + 1:k + P + 1].mean() for k in range(1, K + 1)])
    assert np.all(g >= -1e-15) and np.all(g.sum(1) <= 1 + 1e-12)
    assert np.allclose(g @ xi, t, atol=1e-12)
    g0, _ = O.traj_basis_table(np.zeros(1), K, "bspline")
    assert np.allclose(g0, 0)
    if K == 1:
        assert np.allclose(g[:, 0], t)
    if K == 2:
        assert np.allclose(g, np.stack([2 * t * (1 - t), t * t], 1))
    e = 1e-6
    tt = np.linspace(0.01, 0.99, 37)
    gp, _ = O.traj_basis_table(tt + e, K, "bspline")
    gm, _ = O.traj_basis_table(tt - e, K, "bspline")
    _, d = O.traj_basis_table(tt, K, "bspline")
    assert np.allclose((gp - gm) / (2 * e), d, atol=1e-5 * max(1, np.abs(d).max()))


def test_traj_basis_polynomial_and_bezier():
    t = np.linspace(0, 1, 23)
    g, gd = O.traj_basis_table(t, 4, "polynomial")
    assert np.allclose(g, np.stack([t, t ** 2, t ** 3, t ** 4], 1)) and np.allclose(gd[:, 2], 3 * t ** 2)
    g, gd = O.traj_basis_table(t, 3, "bezier")
    assert np.allclose(g, np.stack([3 * t * (1 - t) ** 2, 3 * t ** 2 * (1 - t), t ** 3], 1))
    assert np.allclose(gd[:, 2], 3 * t ** 2)


def test_traj_pair_sums_straight_trajectories_are_the_reference_sums():
    """Closed form: starts p = x - v t and control points v xi_k (straight B-spline trajectories) give the
    reference's pair sums (fp64 brute force of atl/ops/reference.py:58-71), the same counts, and
    -t gp + sum_k xi_k gcoef_k = dS/dv."""
    rng = np.random.default_rng(16)
    n, K = 400, 10
    x = np.stack([rng.uniform(0, 30, n), rng.uniform(0, 20, n)], 1)
    t = np.sort(rng.random(n))
    b = np.sort(rng.integers(0, 2, n))
    v = rng.standard_normal((n, 2)) * 4
    P, L = 3, K - 2
    knots = np.concatenate([np.zeros(P), np.linspace(0, 1, L + 1), np.ones(P)])
    xi = np.array([knots[k + 1:k + P + 1].mean() for k in range(1, K + 1)])
    coef = np.concatenate([v[:, 1:2] * xi, v[:, 0:1] * xi], 1)
    anchors = np.arange(n)
    xa = x + rng.standard_normal((n, 2)) * 0.5
    S1, c1, g1 = O.traj_pair_sums_fp64(x - v * t[:, None], coef, t, b, anchors, xa, 1.0, 0.25, 3.0, 16, K, "bspline")
    S0, c0, g0 = O.pair_sums_fp64(x, t, v, b, anchors, 1.0, 0.25, 3.0, anchor_xy=xa)
    assert np.allclose(S1, S0, atol=1e-12) and np.array_equal(c1, c0) and c0.sum() > n
    gS = rng.standard_normal(n)
    gp, gc = g1(gS)
    gv = -t[:, None] * gp + np.stack([(gc[:, K:] * xi).sum(1), (gc[:, :K] * xi).sum(1)], 1)
    assert np.allclose(gv, g0(gS), atol=1e-10)


def test_traj_pair_sums_gradients_match_finite_differences():
    rng = np.random.default_rng(17)
    n, K = 250, 5
    x = np.stack([rng.uniform(0, 12, n), rng.uniform(0, 9, n)], 1)
    t = np.sort(rng.random(n))
    b = np.zeros(n, np.int64)
    coef = rng.standard_normal((n, 2 * K)) * 2
    xa = x + rng.standard_normal((n, 2)) * 0.5
    gS = rng.standard_normal(n)
    args = (t, b, np.arange(n), xa, 1.0, 0.3, 3.0, 16, K, "bspline")
    _, _, grad = O.traj_pair_sums_fp64(x, coef, *args)
    gp, gc = grad(gS)
    e = 1e-6
    j, k = np.unravel_index(np.abs(gc).argmax(), gc.shape)
    c2 = coef.copy(); c2[j, k] += e
    sp = O.traj_pair_sums_fp64(x, c2, *args)[0] @ gS
    c2[j, k] -= 2 * e
    sm = O.traj_pair_sums_fp64(x, c2, *args)[0] @ gS
    assert abs((sp - sm) / (2 * e) - gc[j, k]) <= 1e-6 * max(1.0, abs(gc[j, k]))
    i = int(np.abs(gp[:, 1]).argmax())
    x2 = x.copy(); x2[i, 1] += e
    sp = O.traj_pair_sums_fp64(x2, coef, *args)[0] @ gS
    x2[i, 1] -= 2 * e
    sm = O.traj_pair_sums_fp64(x2, coef, *args)[0] @ gS
    assert abs((sp - sm) / (2 * e) - gp[i, 1]) <= 1e-6 * max(1.0, abs(gp[i, 1]))


def test_traj_fp32_plan_and_pair_loops_match_fp64():
    """The oracle's fp32 trajectory plan through its OpenMP pair loops against the float64 brute force: counts equal
    except for pairs within 1e-5 of a cut-off, sums within 1e-5, the loops' gradients within 1e-4."""
    rng = np.random.default_rng(18)
    n, K, H, W = 3000, 10, 30, 40
    x = np.stack([rng.uniform(0, W, n), rng.uniform(0, H, n)], 1).astype(F32)
    t = np.sort(rng.random(n)).astype(F32)
    b = np.zeros(n, np.int64)
    coef = (rng.standard_normal((n, 2 * K)) * 2).astype(F32)
    xa = (x + rng.standard_normal((n, 2)) * 0.5).astype(F32)
    tab = O.traj_slice_table(K, "bspline", 16)
    plan = O.build_pair_plan_traj(x, coef, tab, t, b, 1, H, W, np.arange(n), xa, 1.0, 0.3, 3.0, 16)
    S32, c32 = O.ats_pair_fwd(plan, 1.0, 0.3, 3.0, with_counts=True)
    S64, c64, grad = O.traj_pair_sums_fp64(x, coef, t, b, np.arange(n), xa, 1.0, 0.3, 3.0, 16, K, "bspline")
    assert np.abs(c32 - c64).sum() <= 3 and c64.sum() > 10 * n
    assert np.allclose(S32, S64, rtol=1e-5, atol=1e-5 * S64.max())
    gS = rng.standard_normal(n).astype(F32)
    gp, gc = O.ats_pair_bwd_traj(gS, plan, tab, K, 1.0, 0.3, 3.0, n)
    wp, wc = grad(gS)
    assert np.abs(gp - wp).max() <= 1e-4 * np.abs(wp).max() and np.abs(gc - wc).max() <= 1e-4 * np.abs(wc).max()


@pytest.mark.parametrize("tau,S,h", [(0.2, 16, 1.0), (1.0, 8, 1.5), (0.05, 4, 0.7)])
def test_torch_plan_equals_numpy_plan(tau, S, h):
    """build_pair_plan_torch (the reference's torch CPU op sequence, which the CPU baseline times) and the NumPy
    restatement give the same plan bit for bit: geometry, keys, cell offsets, entries (id, position, velocity,
    time) and anchor cells."""
    if torch.backends.cpu.get_cpu_capability() == "DEFAULT":
        pytest.skip("torch CPU kernels without FMA: a different rounding of the norm")
    win, v = _dense_case(seed=20 + S)
    rng = np.random.default_rng(S)
    anchors = np.sort(rng.permutation(win.n)[: win.n // 2])
    xa = (win.xy[anchors] + h * rng.standard_normal((len(anchors), 2))).astype(F32)
    for axy in (None, xa):
        p = O.build_pair_plan(win.xy, win.t, v, win.b, 2, 40, 48, anchors, h, tau, 3.0, S, anchor_xy=axy)
        q = O.build_pair_plan_torch(win.xy, win.t, v, win.b, 2, 40, 48, anchors, h, tau, 3.0, S, anchor_xy=axy)
        assert p["geometry"] == q["geometry"] and (p["GH"], p["GW"], p["S"]) == (q["GH"], q["GW"], q["S"])
        for f in ("key", "cell_start", "src_id", "src_y", "src_v", "src_t", "anc_x", "anc_t", "anc_cell", "anc_id",
                  "slice_c"):
            assert p[f].dtype == q[f].dtype and np.array_equal(p[f], q[f]), f
        assert p["key"].shape[0] > len(win.t)


def _linear_coeff_field(rng, K, Hg, Wg, slope):
    """A (1, 2K, Hg, Wg) coefficient field linear in the node position, c(p) = a + Bx px + By py per channel
    (bilinear interpolation reproduces it exactly inside the grid), and its float64 parameters."""
    a = rng.standard_normal(2 * K) * 2.0
    bx, by = rng.standard_normal(2 * K) * slope, rng.standard_normal(2 * K) * slope
    yy, xx = np.meshgrid(np.arange(Hg, dtype=np.float64), np.arange(Wg, dtype=np.float64), indexing="ij")
    fld = (a[:, None, None] + bx[:, None, None] * xx + by[:, None, None] * yy)[None].astype(F32)
    return fld, a, bx, by


def test_traj_displacement_closed_forms():
    """traj_displacement: (1) K = 2 B-splines are the quadratic Bernstein pair 2t(1 - t), t^2, so on a field linear
    in the position d_x = c_x1(p) 2t(1 - t) + c_x2(p) t^2 (x channels after the y channels); (2) control points
    v xi_k at the Greville abscissae give d = v t for K = 10 (linear precision); (3) positions outside the grid
    take the border node's coefficients."""
    rng = np.random.default_rng(40)
    Hg, Wg, n = 12, 16, 400
    fld, a, bx, by = _linear_coeff_field(rng, 2, Hg, Wg, 0.3)
    p = np.stack([rng.uniform(0, Wg - 1, n), rng.uniform(0, Hg - 1, n)], 1).astype(F32)
    t = rng.uniform(0, 1, n).astype(F32)
    b = np.zeros(n, np.int64)
    d, _, _, _ = O.traj_displacement(fld, p, t, b, 2, "bspline")
    pd, td = p.astype(np.float64), t.astype(np.float64)
    c = a[None] + bx[None] * pd[:, :1] + by[None] * pd[:, 1:]         # (n, 4): y1, y2, x1, x2
    g1, g2 = 2 * td * (1 - td), td * td
    want = np.stack([c[:, 2] * g1 + c[:, 3] * g2, c[:, 0] * g1 + c[:, 1] * g2], 1)
    assert np.abs(d - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
    from x_amd.motion.trajectories import greville
    K = 10
    v = np.array([3.5, -2.25])
    xi = greville(K)
    uni = np.concatenate([v[1] * xi, v[0] * xi]).astype(F32)[None, :, None, None] * np.ones((1, 1, Hg, Wg), F32)
    d, rows, _, _ = O.traj_displacement(uni, p, t, b, K, "bspline")
    assert np.abs(d - td[:, None] * v[None]).max() <= 2e-6 * np.abs(v).max()
    far = np.array([[-5.0, -3.0], [Wg + 7.0, Hg + 2.0]], F32)
    _, rows, _, _ = O.traj_displacement(fld, far, np.full(2, 0.5, F32), np.zeros(2, np.int64), 2, "bspline")
    assert np.array_equal(rows[0], fld[0, :, 0, 0]) and np.array_equal(rows[1], fld[0, :, -1, -1])


def test_traj_origin_solves_the_inversion():
    """traj_origin: on uniform straight trajectories p = xy - v t; on a coefficient field linear in the position
    d(p, t) = a(t) + M(t) p, so the start solves (I + M(t)) p = xy - a(t), a 2 x 2 system per event solved in
    float64 (the Picard steps contract by |M| <= 0.05, six of them leave < 1e-7 px)."""
    from x_amd.motion.trajectories import greville
    rng = np.random.default_rng(41)
    Hg, Wg, n, K = 40, 48, 500, 10
    xy = np.stack([rng.uniform(8, Wg - 9, n), rng.uniform(8, Hg - 9, n)], 1).astype(F32)
    t = rng.uniform(0, 1, n).astype(F32)
    b = np.zeros(n, np.int64)
    v = np.array([-2.0, 4.5])
    xi = greville(K)
    uni = np.concatenate([v[1] * xi, v[0] * xi]).astype(F32)[None, :, None, None] * np.ones((1, 1, Hg, Wg), F32)
    p = O.traj_origin(uni, xy, t, b, K, "bspline")
    assert np.abs(p - (xy - t[:, None].astype(np.float64) * v)).max() <= 1e-5
    fld, a, bx, by = _linear_coeff_field(rng, K, Hg, Wg, 0.004)
    p = O.traj_origin(fld, xy, t, b, K, "bspline")
    g, _ = O.traj_basis_table(t.astype(np.float64), K, "bspline")      # (n, K)
    ax, ay = g @ a[K:], g @ a[:K]                                         # a(t): x from the x channels
    mxx, mxy, myx, myy = g @ bx[K:], g @ by[K:], g @ bx[:K], g @ by[:K]
    assert max(np.abs(mxx).max(), np.abs(mxy).max(), np.abs(myx).max(), np.abs(myy).max()) < 0.05
    rx, ry = xy[:, 0] - ax, xy[:, 1] - ay
    det = (1 + mxx) * (1 + myy) - mxy * myx
    want = np.stack([((1 + myy) * rx - mxy * ry) / det, ((1 + mxx) * ry - myx * rx) / det], 1)
    assert np.abs(p - want).max() <= 2e-5


def test_traj_visible_fraction_closed_forms():
    """traj_visible_fraction: (1) straight uniform trajectories of velocity v give the translation's closed form
    (the anchor seen at xa + v (c_k - ta)); (2) on a field linear in the position, the starts from the float64
    2 x 2 solve and the positions p + a(c_k) + M(c_k) p in float64 give the same weighted shares (anchors whose
    positions come within 1e-3 px of the sensor edge are left out: fp32 may put them either side)."""
    from x_amd.motion.trajectories import greville
    rng = np.random.default_rng(42)
    H, W, M, K, tau = 30, 40, 500, 10, 0.3
    xa = np.stack([rng.uniform(-5, W + 5, M), rng.uniform(-3, H + 3, M)], 1).astype(F32)
    ta = rng.uniform(0, 1, M).astype(F32)
    ba = np.zeros(M, np.int64)
    t_all = np.sort(rng.uniform(0, 1, 5000)).astype(F32)
    b_all = np.zeros(5000, np.int64)
    counts = np.bincount(np.clip((t_all * 16).astype(int), 0, 15), minlength=16).astype(np.float64)
    c = (np.arange(16) + 0.5) / 16

    def shares(pos_at):                       # pos_at(k) -> (M, 2) float64 positions at centre k
        vis, tot = np.zeros(M), np.zeros(M)
        for k in range(16):
            y = pos_at(k)
            ins = (y[:, 0] >= 0) & (y[:, 0] <= W - 1) & (y[:, 1] >= 0) & (y[:, 1] <= H - 1)
            wgt = counts[k] * (np.abs(ta.astype(np.float64) - c[k]) <= tau)
            vis += wgt * ins
            tot += wgt
        return np.maximum(vis / np.maximum(tot, 1), 1e-3)

    def edge_clear(pos_at):
        ok = np.ones(M, bool)
        for k in range(16):
            y = pos_at(k)
            for col, hi in ((0, W - 1), (1, H - 1)):
                ok &= (np.abs(y[:, col]) > 1e-3) & (np.abs(y[:, col] - hi) > 1e-3)
        return ok

    v = np.array([9.0, -4.0])
    xi = greville(K)
    uni = np.concatenate([v[1] * xi, v[0] * xi]).astype(F32)[None, :, None, None] * np.ones((1, 1, H, W), F32)
    got = O.traj_visible_fraction(uni, xa, ta, ba, t_all, b_all, 1, H, W, tau, K, "bspline")
    at = lambda k: xa.astype(np.float64) + v * (c[k] - ta.astype(np.float64))[:, None]
    ok = edge_clear(at)
    assert ok.mean() > 0.95 and np.allclose(got[ok], shares(at)[ok], atol=1e-6)
    # a coefficient grid twice the sensor's size, so that starts stay inside it while anchors cross the sensor edge
    fld, a, bx, by = _linear_coeff_field(rng, K, 2 * H, 2 * W, 0.004)
    xa = np.stack([rng.uniform(8, 2 * W - 9, M), rng.uniform(8, 2 * H - 9, M)], 1).astype(F32)
    g, _ = O.traj_basis_table(ta.astype(np.float64), K, "bspline")
    rx, ry = xa[:, 0] - g @ a[K:], xa[:, 1] - g @ a[:K]
    mxx, mxy, myx, myy = g @ bx[K:], g @ by[K:], g @ bx[:K], g @ by[:K]
    det = (1 + mxx) * (1 + myy) - mxy * myx
    p = np.stack([((1 + myy) * rx - mxy * ry) / det, ((1 + mxx) * ry - myx * rx) / det], 1)
    gc, _ = O.traj_basis_table(c, K, "bspline")

    def at_lin(k):
        gk = gc[k]
        cx = gk @ a[K:] + (gk @ bx[K:]) * p[:, 0] + (gk @ by[K:]) * p[:, 1]
        cy = gk @ a[:K] + (gk @ bx[:K]) * p[:, 0] + (gk @ by[:K]) * p[:, 1]
        return p + np.stack([cx, cy], 1)

    got = O.traj_visible_fraction(fld, xa, ta, ba, t_all, b_all, 1, H, W, tau, K, "bspline")
    ok = edge_clear(at_lin)
    want = shares(at_lin)
    assert ok.sum() > 100 and np.allclose(got[ok], want[ok], atol=1e-6)
    assert (want[ok] < 1).sum() > 20                   # the case has anchors that leave the sensor


def test_blur_impulse_response_and_mass():
    """The oracle's blur: an impulse far from the border becomes the outer product of the normalised taps (mass
    1); an image at the border loses exactly the mass that falls outside (zero padding)."""
    img = np.zeros((1, 31, 33), F32)
    img[0, 15, 16] = 1.0
    out = O.blur(img, 1.3)
    r = int(math.ceil(3 * 1.3))
    x = np.arange(-r, r + 1)
    k = np.exp(-x * x / (2 * 1.3 ** 2))
    k /= k.sum()
    assert np.allclose(out[0, 15 - r:16 + r, 16 - r:17 + r], np.outer(k, k), atol=1e-7)
    assert abs(float(out.sum()) - 1.0) < 1e-6
    edge = np.zeros((1, 20, 20), F32)
    edge[0, 0, 10] = 1.0                         # on the top row: the taps at rows -3..-1 fall outside
    k1 = np.exp(-np.arange(-3, 4) ** 2 / 2.0)
    k1 /= k1.sum()
    assert abs(float(O.blur(edge, 1.0).sum()) - k1[3:].sum()) < 1e-6


def test_make_iwe_weights_and_polarity_split():
    """The oracle's IWE: integer positions deposit their weights in one pixel; the border mask drops events
    outside; scale_by_dt weights 1 - |t - t_ref|; split polarity puts positive events in entry 2b, negative
    ones in 2b + 1."""
    xy = np.array([[2, 3], [2, 3], [5, 1], [-1, 2], [4, 4]], F32)
    t = np.array([0.5, 0.1, 0.9, 0.5, 1.7], F32)
    p = np.array([1, -1, 1, 1, -1], F32)
    b = np.array([0, 0, 1, 1, 1])
    img = O.make_iwe(xy, t, p, b, 2, 6, 7, 0.5, sigma=0.0)
    assert img[0, 3, 2] == 2 and img[1, 1, 5] == 1 and img[1, 4, 4] == 1 and img.sum() == 4
    img = O.make_iwe(xy, t, p, b, 2, 6, 7, 0.5, sigma=0.0, scale_by_dt=True)
    assert np.isclose(img[0, 3, 2], 1.0 + 0.6) and np.isclose(img[1, 1, 5], 0.6) and img[1, 4, 4] == 0
    img = O.make_iwe(xy, t, p, b, 2, 6, 7, 0.5, sigma=0.0, polarity="split")
    assert img.shape == (4, 6, 7) and img[0, 3, 2] == 1 and img[1, 3, 2] == 1 and img[2, 1, 5] == 1
    assert img[3, 4, 4] == 1


# --------------------------------------------------------------------------- MotionPriorCMax KNN (oracle)
def _separated(d64, k, rel=1e-5):
    """Rows whose k-th and (k+1)-th float64 distances are apart (the neighbour set is then unambiguous)."""
    s = np.sort(d64, axis=1)
    return (s[:, k] - s[:, k - 1]) > rel * np.maximum(s[:, k], 1e-12)


def test_knn_oracle_matches_kd_tree_in_float64():
    from scipy.spatial import cKDTree
    rng = np.random.default_rng(5)
    q = (rng.random((300, 2)) * [64, 48]).astype(F32)
    pts = (rng.random((2, 400, 2)) * [70, 50] - 3).astype(F32)
    k = 12
    got = O.knn_indices(q, pts, k)
    for s in range(2):
        dist, ref = cKDTree(pts[s].astype(np.float64)).query(q.astype(np.float64), k=k + 1)
        d64 = ((q[:, None, :].astype(np.float64) - pts[s][None].astype(np.float64)) ** 2).sum(-1)
        ok = _separated(d64, k)
        assert ok.mean() > 0.95
        for i in np.nonzero(ok)[0]:
            assert set(got[s, i]) == set(ref[i, :k])
            # ascending distance (ties in fp32 only where float64 cannot tell them apart)
            dd = d64[i, got[s, i]]
            assert np.all(np.diff(dd) >= -1e-9 * dd.max())


def test_knn_oracle_ties_by_index_on_a_regular_grid():
    # points on a 4 px lattice, queries half a pixel off the lattice: many exactly equal distances
    gy, gx = np.meshgrid(np.arange(6) * 4.0 + 2, np.arange(7) * 4.0 + 2, indexing="ij")
    pts = np.stack([gx.ravel(), gy.ravel()], 1).astype(F32)[None]
    q = np.array([[1.5, 1.5], [9.5, 5.5], [13.5, 13.5], [26.0, 22.0]], F32)
    k = 9
    got = O.knn_indices(q, pts, k)
    for i, (qx, qy) in enumerate(q):
        cand = []
        for j, (px, py) in enumerate(pts[0]):
            dx, dy = F32(qx) - F32(px), F32(qy) - F32(py)
            cand.append((float(F32(F32(dx * dx) + F32(dy * dy))), j))
        want = [j for _, j in sorted(cand)[:k]]                 # (distance, index) lexicographic
        assert list(got[0, i]) == want


def test_knn_oracle_agrees_with_the_reference_cpu_path():
    # the reference's CPU path: torch.cdist + topk(largest=False) (atl/objectives/mpcm.py:37-41); same sets
    # wherever the k-th and (k+1)-th distances are apart
    rng = np.random.default_rng(9)
    q = (rng.random((500, 2)) * 80).astype(F32)
    pts = (rng.random((1, 3, 300, 2)) * 80).astype(F32)
    k = 8
    d = torch.cdist(torch.as_tensor(q)[None].expand(3, -1, -1), torch.as_tensor(pts[0]))
    ref = torch.topk(d, k, dim=-1, largest=False).indices.numpy()
    got = O.knn_indices(q, pts[0], k)
    for s in range(3):
        d64 = ((q[:, None, :].astype(np.float64) - pts[0, s][None].astype(np.float64)) ** 2).sum(-1)
        ok = _separated(d64, k, rel=1e-4)
        for i in np.nonzero(ok)[0]:
            assert set(got[s, i]) == set(ref[s, i])


def test_lut_mean_matches_float64_mean():
    rng = np.random.default_rng(2)
    f = rng.standard_normal((2, 50, 2)).astype(F32)
    idx = rng.integers(0, 50, (2, 30, 7))
    want = f.astype(np.float64)[np.arange(2)[:, None, None], idx].mean(2)
    got = O.lut_mean(f, idx)
    assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()
