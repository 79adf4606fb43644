"""HIP kernels against the oracle on identical seeded inputs (the reference's tests/test_ops.py, on the GPU).

Bars: integer outputs (cell bins, keys, CSR offsets, neighbour counts, window counts) bit-exact; values
computed in the same fp32 order bit-exact where no atomics reorder sums; forward values within 1e-5
relative; gradients within 1e-4 relative (to the largest magnitude, as gradient sums cancel)."""
import math

import numpy as np
import pytest
import torch

import oracle as O
from tests.conftest import assert_logs_close, assert_sums_close, rand_events
from x_amd import synth
from x_amd.ops import functional as F

pytestmark = pytest.mark.gpu
DEV = "cuda"
F32 = np.float32


def T(a, dev=DEV):
    return torch.as_tensor(np.ascontiguousarray(a), device=dev)


def N(t):
    return t.detach().cpu().numpy()


def close_rel(got, want, rel, floor=0.0):
    """|got - want| <= rel * max(|want|) elementwise (plus an absolute floor)."""
    scale = max(float(np.abs(want).max()), 1e-30)
    err = float(np.abs(got.astype(np.float64) - want.astype(np.float64)).max()) if want.size else 0.0
    assert err <= rel * scale + floor, f"max err {err:.3e} vs scale {scale:.3e} (rel {err / scale:.2e})"


# ------------------------------------------------------------------------------------------- splat / gather
@pytest.mark.parametrize("kernel", ["bilinear", "gauss"])
def test_splat_matches_oracle(kernel):
    pos, w, b, _ = rand_events(n=5000, seed=0)
    B, H, W = 2, 20, 24
    p = T(pos).requires_grad_(True)
    wt = T(w).requires_grad_(True)
    out = F.splat(p, wt, T(b), B, H, W, kernel=kernel, sigma=1.3)
    if kernel == "bilinear":
        ref = O.splat_bilinear_fwd(pos, w, b, B, H, W)
    else:
        ref = O.splat_gauss_fwd(pos, w, b, B, H, W, 1.3, int(math.ceil(3 * 1.3)))
    close_rel(N(out), ref, 1e-5)
    g = np.random.default_rng(1).standard_normal(ref.shape).astype(F32)
    (out * T(g)).sum().backward()
    if kernel == "bilinear":
        gp, gw = O.splat_bilinear_bwd(g, pos, w, b)
        assert np.array_equal(N(wt.grad), gw) and np.array_equal(N(p.grad), gp)   # same fp32 order, no atomics
    else:
        gp, gw = O.splat_gauss_bwd(g, pos, w, b, 1.3, 4)
        close_rel(N(wt.grad), gw, 1e-5)
        close_rel(N(p.grad), gp, 1e-4)


def test_gather_matches_oracle():
    pos, _, b, _ = rand_events(n=5000, seed=2)
    img = np.random.default_rng(3).standard_normal((2, 20, 24)).astype(F32)
    ti = T(img).requires_grad_(True)
    tp = T(pos).requires_grad_(True)
    out = F.gather(ti, tp, T(b))
    assert np.array_equal(N(out), O.gather_bilinear_fwd(img, pos, b))
    g = np.random.default_rng(4).standard_normal(5000).astype(F32)
    out.backward(T(g))
    gimg, gp = O.gather_bilinear_bwd(g, img, pos, b)
    assert np.array_equal(N(tp.grad), gp)
    close_rel(N(ti.grad), gimg, 1e-5)


@pytest.mark.parametrize("B,H,W", [(1, 480, 640), (20, 480, 640), (60, 480, 640), (2, 3, 2)])
def test_splat_gather_tile_paths(B, H, W):
    """The tile-binned splat forward and gather backward (16-px tiles; 32-px tiles when 16-px ones would
    exceed the binning histogram, B = 20; the per-corner atomic kernels beyond that, B = 60) against the
    oracle: a crowded pixel, events on the borders and just outside them, zero and negative weights."""
    print(f"tile paths B={B} {H}x{W}", flush=True)
    rng = np.random.default_rng(B)
    n = 60000
    pos = np.stack([rng.uniform(-1.5, W + 0.5, n), rng.uniform(-1.5, H + 0.5, n)], 1).astype(F32)
    pos[: n // 4] = np.array([min(W - 1, 7) + 0.25, min(H - 1, 5) + 0.5], F32)       # one crowded pixel
    pos[n // 4: n // 4 + 100, 0] = F32(-1.0)                                           # base corner -1
    pos[n // 4 + 100: n // 4 + 200, 1] = F32(H - 1)                                    # last row exactly
    w = rng.standard_normal(n).astype(F32)
    w[::17] = 0.0
    b = rng.integers(0, B, n).astype(np.int64)
    img = F.get_ext().splat_bilinear_fwd(T(pos), T(w), T(b), B, H, W)
    # signed weights cancel on the crowded pixel: the summation-order bar is relative to the sum of |terms|
    mag = float(O.splat_bilinear_fwd(pos, np.abs(w), b, B, H, W).max())
    close_rel(N(img), O.splat_bilinear_fwd(pos, w, b, B, H, W), 1e-5, floor=1e-6 * mag)
    src = rng.standard_normal((B, H, W)).astype(F32)
    g = rng.standard_normal(n).astype(F32)
    gimg, gp = F.get_ext().gather_bilinear_bwd(T(g), T(src), T(pos), T(b))
    want_img, want_p = O.gather_bilinear_bwd(g, src, pos, b)
    assert np.array_equal(N(gp), want_p)
    close_rel(N(gimg), want_img, 1e-5)


@pytest.mark.parametrize("B,H,W,sigma,R", [(1, 480, 640, 1.0, 3), (2, 60, 80, 2.5, 8), (20, 480, 640, 1.0, 3),
                                           (2, 40, 48, 3.0, 9), (1, 3, 2, 1.0, 3)])
def test_splat_gauss_tile_paths(B, H, W, sigma, R):
    """The tile-binned Gaussian splat (centres rounded into 16 or 32-px tiles, an LDS window of T + 2R) and its
    per-event fallback (R > 8) against the oracle: a crowded pixel, centres within R outside the image, zero
    weights."""
    print(f"gauss tile paths B={B} {H}x{W} sigma={sigma} R={R}", flush=True)
    rng = np.random.default_rng(B + R)
    n = 40000
    pos = np.stack([rng.uniform(-R - 1.5, W + R + 0.5, n), rng.uniform(-R - 1.5, H + R + 0.5, n)], 1).astype(F32)
    pos[: n // 4] = np.array([min(W - 1, 9) + 0.3, min(H - 1, 4) + 0.6], F32)          # one crowded pixel
    w = rng.standard_normal(n).astype(F32)
    w[::13] = 0.0
    b = rng.integers(0, B, n).astype(np.int64)
    img = F.get_ext().splat_gauss_fwd(T(pos), T(w), T(b), B, H, W, sigma, R)
    # signed weights cancel on the crowded pixel: the summation-order bar is relative to the sum of |terms|
    mag = float(O.splat_gauss_fwd(pos, np.abs(w), b, B, H, W, sigma, R).max())
    close_rel(N(img), O.splat_gauss_fwd(pos, w, b, B, H, W, sigma, R), 1e-5, floor=1e-6 * mag)


def test_voxel_matches_oracle():
    pos, _, b, t = rand_events(n=5000, seed=5)
    p = np.where(np.random.default_rng(6).random(5000) > 0.5, 1.0, -1.0).astype(F32)
    got = F.voxel_grid(T(pos), T(t), T(p), T(b), 2, 5, 20, 24, normalize=None)
    close_rel(N(got), O.voxel_grid(pos, t, p, b, 2, 5, 20, 24), 1e-5)


def _voxel_cases_close(got, want, mag):
    # same voxels touched (bit-exact corner indices); values within 1e-5 of the sum of |terms|
    assert np.array_equal(got != 0, want != 0) or np.abs(got - want).max() <= 1e-6 * mag
    assert np.abs(got - want).max() <= 1e-5 * mag


def test_voxel_tile_engine_at_full_sensor_and_edges():
    from x_amd.ops import _ext
    lib = _ext.load_library()
    win = synth.dense_flow_window(seed=3)                      # 1M line-segment events, time-sorted
    rng = np.random.default_rng(11)
    pos, t, b = win.xy, win.t, win.b
    p = np.where(rng.random(len(t)) > 0.5, 1.0, -1.0).astype(F32)
    print("voxel grid: 1M events 640x480, 15 bins, tile engine", flush=True)
    assert lib.atl_voxel_ws_bytes(len(t), 1, 15, 480, 640) > 0
    got = N(F.voxel_grid(T(pos), T(t), T(p), T(b), 1, 15, 480, 640, normalize=None))
    _voxel_cases_close(got, O.voxel_grid(pos, t, p, b, 1, 15, 480, 640),
                       float(O.voxel_grid(pos, t, np.abs(p), b, 1, 15, 480, 640).max()))
    # positions at and past the borders, times outside [0, 1], zero polarity, three batches
    n = 60_000
    pos = np.stack([rng.random(n) * 68 - 2, rng.random(n) * 52 - 2], 1).astype(F32)
    pos[:500] = np.floor(pos[:500])
    t = np.sort(rng.random(n) * 1.2 - 0.1).astype(F32)
    b = np.sort(rng.integers(0, 3, n)).astype(np.int64)
    p = rng.choice(np.array([-1.0, 0.0, 1.0], F32), n)
    for C in (1, 2, 5, 15):
        print(f"voxel grid edges C={C}", flush=True)
        got = N(F.voxel_grid(T(pos), T(t), T(p), T(b), 3, C, 48, 64, normalize=None))
        _voxel_cases_close(got, O.voxel_grid(pos, t, p, b, 3, C, 48, 64),
                           float(O.voxel_grid(pos, t, np.abs(p), b, 3, C, 48, 64).max()) + 1e-30)
    # more bins than an LDS window holds (64 x 17 x 17 floats): the per-event kernel takes over, same results
    print("voxel grid: 64 bins (per-event fallback)", flush=True)
    assert lib.atl_voxel_ws_bytes(n, 3, 64, 48, 64) < 0
    got = N(F.voxel_grid(T(pos), T(t), T(p), T(b), 3, 64, 48, 64, normalize=None))
    _voxel_cases_close(got, O.voxel_grid(pos, t, p, b, 3, 64, 48, 64),
                       float(O.voxel_grid(pos, t, np.abs(p), b, 3, 64, 48, 64).max()))


@pytest.mark.parametrize("form", ["gather", "scatter"])
def test_tile_accumulation_forms_match_oracle(form, monkeypatch):
    """Both accumulation forms of the tile engine (per-corner sums after an LDS sort by base corner, the default
    for the bilinear modes; LDS float atomics, ATL_TILE_SCATTER=1, and always for the voxel grid) against the
    oracle: the splat forward with a tile of more than 16384 events (2048-record chunks), the gather's image
    gradient, the voxel grid (5 bins, a crowded tile) and the flow-grid adjoint with 1, 2 and 4 channels."""
    monkeypatch.setenv("ATL_TILE_SCATTER", "1" if form == "scatter" else "0")
    print(f"tile accumulation form={form}", flush=True)
    rng = np.random.default_rng(11)
    H, W, n = 96, 128, 120000
    pos = np.stack([rng.uniform(-1.5, W + 0.5, n), rng.uniform(-1.5, H + 0.5, n)], 1).astype(F32)
    pos[: n // 3] = (np.array([40.0, 30.0]) + rng.uniform(0, 12, (n // 3, 2))).astype(F32)   # one crowded tile
    w = rng.standard_normal(n).astype(F32)
    b = rng.integers(0, 2, n).astype(np.int64)
    img = F.get_ext().splat_bilinear_fwd(T(pos), T(w), T(b), 2, H, W)
    mag = float(O.splat_bilinear_fwd(pos, np.abs(w), b, 2, H, W).max())
    close_rel(N(img), O.splat_bilinear_fwd(pos, w, b, 2, H, W), 1e-5, floor=1e-6 * mag)
    src = rng.standard_normal((2, H, W)).astype(F32)
    g = rng.standard_normal(n).astype(F32)
    gimg, _ = F.get_ext().gather_bilinear_bwd(T(g), T(src), T(pos), T(b))
    close_rel(N(gimg), O.gather_bilinear_bwd(g, src, pos, b)[0], 1e-5)
    print(f"tile accumulation form={form}: voxel grid", flush=True)
    tv = np.sort(rng.random(n) * 1.2 - 0.1).astype(F32)
    pv = np.where(rng.random(n) > 0.5, 1.0, -1.0).astype(F32)
    bs = np.sort(b)
    got = N(F.voxel_grid(T(pos), T(tv), T(pv), T(bs), 2, 5, H, W, normalize=None))
    _voxel_cases_close(got, O.voxel_grid(pos, tv, pv, bs, 2, 5, H, W),
                       float(O.voxel_grid(pos, tv, np.abs(pv), bs, 2, 5, H, W).max()))
    for C in (1, 2, 4):
        fld = rng.standard_normal((2, C, 24, 32)).astype(F32)
        tf = T(fld).requires_grad_(True)
        out = F.sample_grid_hip(tf, T(pos), T(b), img_hw=(H, W))
        want, idx, wts = O.sample_grid(fld, O.dense_grid_pos(pos, H, W, 24, 32), b)
        assert np.array_equal(N(out), want)
        go = rng.standard_normal(want.shape).astype(F32)
        out.backward(T(go))
        close_rel(N(tf.grad), O.sample_grid_bwd(go, idx, wts, fld.shape), 1e-5)


def test_splat_contention_4m_blob_events():
    """The contention shape: 4M events, 90% in 5 Gaussian blobs (sigma 8 px), transported to t = 0.5 by the Sim2
    flow, bilinear splat forward (tile engine) and backward against the oracle."""
    win = synth.blob_window(seed=0)
    th = win.motion["theta"].astype(F32)
    c = np.array([(win.width - 1) / 2.0, (win.height - 1) / 2.0], F32)
    d = (win.xy - c).astype(F32)
    v = np.stack([th[0] + (th[2] * d[:, 0] - th[3] * d[:, 1]), th[1] + (th[3] * d[:, 0] + th[2] * d[:, 1])], 1)
    y = (win.xy + v.astype(F32) * (F32(0.5) - win.t)[:, None]).astype(F32)
    w = np.ones(win.n, F32)
    H, W = win.height, win.width
    print("splat contention: 4M blob events, forward", flush=True)
    img = N(F.get_ext().splat_bilinear_fwd(T(y), T(w), T(win.b), 1, H, W))
    want = O.splat_bilinear_fwd(y, w, win.b, 1, H, W)
    assert np.array_equal(img != 0, want != 0)
    close_rel(img, want, 1e-5)
    assert float(want.max()) > 1000.0                          # the crowded pixels the config is about
    print("splat contention: backward", flush=True)
    gimg = (np.random.default_rng(4).standard_normal((1, H, W))).astype(F32)
    gpos, gw = F.get_ext().splat_bilinear_bwd(T(gimg), T(y), T(w), T(win.b))
    wp, ww = O.splat_bilinear_bwd(gimg, y, w, win.b)
    assert np.array_equal(N(gw), ww) and np.array_equal(N(gpos), wp)


def test_plumbing_translation_splat_gather_fwd_bwd():
    """100k events at 240x180, translation (2.0, -1.25) px/window: warp to t_ref = 0, splat, gather back."""
    win = synth.plumbing_translation(seed=0)
    th = win.motion["theta"]
    xy = win.xy + th[None, :] * (F32(0.0) - win.t)[:, None]
    xy = xy.astype(F32)
    w = np.ones(win.n, F32)
    b = win.b
    tp = T(xy).requires_grad_(True)
    img = F.splat(tp, T(w), T(b), 1, 180, 240)
    ref_img = O.splat_bilinear_fwd(xy, w, b, 1, 180, 240)
    close_rel(N(img), ref_img, 1e-5)
    val = F.gather(img, tp, T(b))
    close_rel(N(val), O.gather_bilinear_fwd(ref_img, xy, b), 1e-5)
    val.sum().backward()
    # d(sum gather(splat(pos), pos))/dpos = gather-pos-grad(1) + splat-pos-grad(gather-img-grad(1))
    gimg, gp1 = O.gather_bilinear_bwd(np.ones(win.n, F32), ref_img, xy, b)
    gp2, _ = O.splat_bilinear_bwd(gimg, xy, w, b)
    close_rel(N(tp.grad), gp1 + gp2, 1e-4)


# ------------------------------------------------------------------------------------------- flow grid
def test_sample_grid_matches_oracle():
    win = synth.small_window(seed=7, n=3000, B=2)
    grid = win.motion["grid"]
    H, W = win.height, win.width
    tg = T(grid).requires_grad_(True)
    v = F.sample_grid_hip(tg, T(win.xy), T(win.b), img_hw=(H, W))
    want, idx, wts = O.dense_velocity(grid, win.xy, win.b, H, W)
    assert np.array_equal(N(v), want)
    g = np.random.default_rng(8).standard_normal(want.shape).astype(F32)
    v.backward(T(g))
    close_rel(N(tg.grad), O.sample_grid_bwd(g, idx, wts, grid.shape), 1e-5)


@pytest.mark.parametrize("Hg,Wg,img", [(23, 31, True), (40, 48, True), (9, 2, False), (1, 5, True)])
def test_sample_flow_interleaved_same_bits(Hg, Wg, img):
    """Two-channel fields are sampled from the node-interleaved copy: bit-equal to the oracle (positions inside and
    outside the grid, absent batches zero), and an in-place update of the field makes a new copy."""
    print(f"sample_grid flow interleaved {Hg}x{Wg} img={img}", flush=True)
    rng = np.random.default_rng(Hg * 7 + Wg)
    n, B = 5000, 2
    H, W = (47, 61) if img else (0, 0)
    span_x, span_y = (W, H) if img else (Wg, Hg)
    pos = np.stack([rng.uniform(-3, span_x + 2, n), rng.uniform(-3, span_y + 2, n)], 1).astype(F32)
    b = rng.integers(0, B, n).astype(np.int64)
    b[::89] = B
    fld = rng.standard_normal((B, 2, Hg, Wg)).astype(F32)
    tf = T(fld)
    ok = b < B

    def check(f):
        out = N(F.sample_grid_hip(tf, T(pos), T(b), img_hw=(H, W)))
        want = (O.dense_velocity(f, pos[ok], b[ok], H, W) if img else O.sample_grid(f, pos[ok], b[ok]))[0]
        assert np.array_equal(out[ok], want) and not out[~ok].any()

    check(fld)
    with F.layout_scope():
        check(fld)
        check(fld)                                 # the scope's copy
        if Wg >= 2:                                # a view of the same field (detach) finds the same copy
            assert F._interleaved(tf.detach()) is F._interleaved(tf)
        with torch.no_grad():
            tf.mul_(-0.5)                          # a new version of the field: a new copy
        check(fld * np.float32(-0.5))
    tf.data.mul_(-2.0)                             # no version bump: seen outside a scope (each look-up copies)
    check(fld)


@pytest.mark.parametrize("C,img", [(4, False), (5, False), (20, False), (7, True), (20, True)])
def test_sample_grid_channels_last_same_bits(C, img):
    """Many-channel fields go through the channels-last copy: the forward equals the oracle bit for bit, the
    position gradient equals the plane kernel's bit for bit, and the field gradient matches the oracle adjoint;
    positions inside and outside the grid, and out-of-range batch indices (zero rows)."""
    print(f"sample_grid channels-last C={C} img={img}", flush=True)
    rng = np.random.default_rng(C * 10 + img)
    n, B, Hg, Wg = 4000, 3, 23, 31
    H, W = (47, 61) if img else (0, 0)
    span_x, span_y = (W, H) if img else (Wg, Hg)
    pos = np.stack([rng.uniform(-3, span_x + 2, n), rng.uniform(-3, span_y + 2, n)], 1).astype(F32)
    b = rng.integers(0, B, n).astype(np.int64)
    b[::97] = B                                    # rows of an absent batch: zero output, zero gradient
    fld = rng.standard_normal((B, C, Hg, Wg)).astype(F32)
    tf, tp = T(fld).requires_grad_(True), T(pos).requires_grad_(True)
    out = F.sample_grid_hip(tf, tp, T(b), img_hw=(H, W))
    ok = b < B
    if img:
        want, idx, wts = O.dense_velocity(fld, pos[ok], b[ok], H, W)
    else:
        want, idx, wts = O.sample_grid(fld, pos[ok], b[ok])
    got = N(out)
    assert np.array_equal(got[ok], want) and not got[~ok].any()
    g = rng.standard_normal((n, C)).astype(F32)
    out.backward(T(g))
    close_rel(N(tf.grad), O.sample_grid_bwd(g[ok], idx, wts, fld.shape), 1e-5)
    assert not N(tp.grad)[~ok].any()
    gp = torch.empty(n, 2, device=DEV)
    td, tb, tg = T(fld), T(b), T(g)
    F.call("atl_sample_grid_bwd_pos", F.ptr(tg), F.ptr(td), B, C, Hg, Wg, F.ptr(tp.detach()), F.ptr(tb), n, H, W,
           F.ptr(gp), F.stream_of(td))
    assert np.array_equal(N(tp.grad), N(gp))


@pytest.mark.parametrize("C", [1, 2, 3, 12])
@pytest.mark.parametrize("Hg,Wg", [(1, 1), (2, 3), (5, 1), (1, 7), (17, 13), (40, 37)])
def test_sample_grid_planned_backward_small_grids(Hg, Wg, C):
    """The tile adjoint on degenerate and odd grids, positions inside and far outside (clamped), some gradient
    rows zero: 1 or 2 channels bin their rows in the backward; 3 and 12 channels take the forward plan (3: the
    per-corner sums of the bilinear accumulation; 12: the many-channel gather form on grids of at least 2 x 2
    nodes, the scatter form otherwise)."""
    print(f"planned backward Hg={Hg} Wg={Wg} C={C}", flush=True)
    rng = np.random.default_rng(Hg * 100 + Wg + C)
    n = 3000
    pos = np.stack([rng.uniform(-5, Wg + 4, n), rng.uniform(-5, Hg + 4, n)], 1).astype(F32)
    b = rng.integers(0, 2, n).astype(np.int64)
    fld = rng.standard_normal((2, C, Hg, Wg)).astype(F32)
    tf = T(fld).requires_grad_(True)
    out = F.sample_grid_hip(tf, T(pos), T(b))
    want, idx, wts = O.sample_grid(fld, pos, b)
    assert np.array_equal(N(out), want)
    g = rng.standard_normal(want.shape).astype(F32)
    g[::7] = 0.0                                   # rows of zeros add nothing (and are skipped by the binning)
    out.backward(T(g))
    close_rel(N(tf.grad), O.sample_grid_bwd(g, idx, wts, fld.shape), 1e-5)


def test_sample_grid_planned_backward_full_size():
    """1M events on a 2x480x640 grid: the tile-plan adjoint equals the per-event atomic adjoint."""
    win = synth.dense_flow_window(seed=0)
    grid = T(win.motion["grid"]).requires_grad_(True)
    xy, b = T(win.xy), T(win.b)
    v = F.sample_grid_hip(grid, xy, b, img_hw=(480, 640))
    g = torch.randn_like(v)
    v.backward(g)
    ref = torch.zeros_like(grid)
    F.call("atl_sample_grid_bwd", F.ptr(g), 1, 2, 480, 640, F.ptr(xy), F.ptr(b), win.n, 480, 640, F.ptr(ref),
           F.stream_of(xy))
    close_rel(N(grid.grad), N(ref), 1e-5)


# ------------------------------------------------------------------------------------------- pair plan + sums
def _pair_case(seed=0, n=6000, B=2, H=40, W=48, h=1.0):
    win = synth.small_window(seed=seed, n=n // B, H=H, W=W, B=B)
    v, _, _ = O.dense_velocity(win.motion["grid"], win.xy, win.b, H, W)
    rng = np.random.default_rng(seed + 100)
    xs = (win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(F32)
    anchors = np.arange(win.n)
    xa = (xs + h * rng.standard_normal(xs.shape)).astype(F32)
    return win, xs, v, anchors, xa


def _cellwise_sorted(keys, ids):
    order = np.lexsort((ids, keys))
    return keys[order], ids[order], order


@pytest.mark.parametrize("tau,S,h", [(0.2, 16, 1.0), (1.0, 8, 1.5), (0.05, 4, 0.5)])
def test_plan_bit_exact(tau, S, h):
    win, xs, v, anchors, xa = _pair_case(seed=1, h=h)
    p = O.build_pair_plan(xs, win.t, v, win.b, 2, 40, 48, anchors, h, tau, 3.0, S, anchor_xy=xa)
    q = F.build_pair_plan(T(xs), T(win.t), T(v), T(win.b), 2, 40, 48, T(anchors), h, tau, 3.0, S, anchor_xy=T(xa))
    assert (q.GH, q.GW, q.S) == (p["GH"], p["GW"], p["S"])
    assert q.geometry["cell"] == p["geometry"]["cell"] and q.geometry["ox"] == p["geometry"]["ox"]
    assert np.array_equal(N(q.cell_start), p["cell_start"])
    # entries: same (key, source) multiset, same slice-centre positions
    cs = N(q.cell_start)
    qkey = np.repeat(np.arange(cs.shape[0] - 1), np.diff(cs))
    k1, i1, o1 = _cellwise_sorted(qkey, N(q.src_id))
    k2, i2, o2 = _cellwise_sorted(p["key"], p["src_id"])
    assert np.array_equal(k1, k2) and np.array_equal(i1, i2)
    assert np.array_equal(N(q.src_y)[o1], p["src_y"][o2])
    assert np.array_equal(N(q.src_v)[o1], p["src_v"][o2])
    assert np.array_equal(N(q.src_t)[o1], p["src_t"][o2])
    for f in ("anc_x", "anc_t", "anc_cell", "anc_id", "slice_c"):
        assert np.array_equal(N(getattr(q, f)), p[f]), f


@pytest.mark.parametrize("n,B,H,W,tau,S", [(20000, 2, 40, 48, 0.2, 16), (30000, 4, 480, 640, 0.05, 96),
                                            (7, 1, 40, 48, 0.3, 8)])
def test_sorted_plan_equals_the_atomic_plan(n, B, H, W, tau, S):
    """atl_plan_sort (bucketed counting sort, one call) against atl_plan_count + atl_scan_counts + atl_plan_fill
    (per-entry atomics) on the same geometry: cell_start bit for bit, the same (cell, source) entries with the same
    slice positions, velocities and times; events of an absent batch and positions leaving the grid are dropped by
    both.  The second case has about 9M cells (buckets of 1024 keys), the third seven events."""
    print(f"sorted plan n={n} B={B} {H}x{W} tau={tau} S={S}", flush=True)
    rng = np.random.default_rng(n + S)
    x = np.stack([rng.uniform(-30, W + 30, n), rng.uniform(-30, H + 30, n)], 1).astype(F32)
    t = np.sort(rng.uniform(0, 1, n)).astype(F32)
    v = rng.normal(0, 15, (n, 2)).astype(F32)
    b = rng.integers(0, B, n).astype(np.int64)
    b[::97] = B                                    # absent batch
    tx, tt, tv, tb = T(x), T(t), T(v), T(b)
    cell, ox, oy = 3.2, -5.0, -4.0
    GW, GH = int(np.ceil((W + 10) / cell)) + 1, int(np.ceil((H + 8) / cell)) + 1
    ncell = B * S * GH * GW
    lib = F.load_library()
    st = F.stream_of(tx)
    ecap = n * min(int(np.floor((2 * tau + 1 / S) * S)) + 2, S)
    nbytes = int(lib.atl_plan_sort_bytes(n, ecap, ncell))
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    cs1 = torch.empty(ncell + 1, dtype=torch.int64, device=DEV)
    out1 = [torch.empty(ecap, 2, device=DEV), torch.empty(ecap, 2, device=DEV), torch.empty(ecap, device=DEV),
            torch.empty(ecap, dtype=torch.int64, device=DEV)]
    F.call("atl_plan_sort", F.ptr(tx), F.ptr(tt), F.ptr(tv), F.ptr(tb), n, B, ox, oy, cell, tau, S, GH, GW, ecap,
           F.ptr(cs1), *[F.ptr(a) for a in out1], F.ptr(ws), nbytes, st)
    counts = torch.zeros(ncell, dtype=torch.int32, device=DEV)
    F.call("atl_plan_count", F.ptr(tx), F.ptr(tt), F.ptr(tv), F.ptr(tb), n, B, ox, oy, cell, tau, S, GH, GW,
           F.ptr(counts), st)
    cs2 = F._scan(counts)
    E = int(cs2[-1])
    assert torch.equal(cs1, cs2) and E > 0
    out2 = [torch.empty(E, 2, device=DEV), torch.empty(E, 2, device=DEV), torch.empty(E, device=DEV),
            torch.empty(E, dtype=torch.int64, device=DEV)]
    counts.zero_()
    F.call("atl_plan_fill", F.ptr(tx), F.ptr(tt), F.ptr(tv), F.ptr(tb), n, B, ox, oy, cell, tau, S, GH, GW,
           F.ptr(cs2), F.ptr(counts), *[F.ptr(a) for a in out2], st)
    key = np.repeat(np.arange(ncell), np.diff(N(cs2)))
    k1, i1, o1 = _cellwise_sorted(key, N(out1[3][:E]))
    k2, i2, o2 = _cellwise_sorted(key, N(out2[3]))
    assert np.array_equal(i1, i2)
    for a1, a2 in zip(out1[:3], out2[:3]):
        assert np.array_equal(N(a1[:E])[o1], N(a2)[o2])


@pytest.mark.parametrize("tau,S,h", [(0.2, 16, 1.0), (1.0, 8, 1.5), (0.05, 4, 0.5)])
def test_pair_sums_match_oracle(tau, S, h):
    win, xs, v, anchors, xa = _pair_case(seed=2, h=h)
    p = O.build_pair_plan(xs, win.t, v, win.b, 2, 40, 48, anchors, h, tau, 3.0, S, anchor_xy=xa)
    want, wcnt = O.ats_pair_fwd(p, h, tau, 3.0, with_counts=True)
    tv = T(v).requires_grad_(True)
    q = F.build_pair_plan(T(xs), T(win.t), tv, T(win.b), 2, 40, 48, T(anchors), h, tau, 3.0, S, anchor_xy=T(xa))
    Sg = F._ATSPair.apply(tv, q, h, tau, 3.0)
    assert np.array_equal(N(F.pair_counts(q, h, tau, 3.0)), wcnt)
    assert_sums_close(N(Sg), want)
    gS = np.random.default_rng(3).standard_normal(len(anchors)).astype(F32)
    Sg.backward(T(gS))
    close_rel(N(tv.grad), O.ats_pair_bwd(gS, p, h, tau, 3.0, win.n), 1e-4)


@pytest.mark.parametrize("scene,n,tau,S,h,zero_frac,B", [("segments", 6000, 0.2, 16, 1.0, 0.0, 1),
                                                         ("segments", 6000, 1.0, 8, 1.5, 0.7, 1),
                                                         ("segments", 6000, 0.05, 4, 0.5, 0.3, 1),
                                                         ("segments", 3000, 0.2, 8, 1.0, 0.2, 3),
                                                         ("blobs", 40000, 0.2, 16, 1.0, 0.5, 1)])
def test_pair_entries_match_oracle(scene, n, tau, S, h, zero_frac, B):
    """Both forward entry points over the reference-layout plan (binned anchors over a workspace; the plan's
    anchor order) and the backward ones (source-centric over a workspace, with per-entry atomics or
    per-(source, slice) slots; per-pair atomics) against the oracle:
    counts bit-exact, S within 1e-5, gv within 1e-4, with a share of the anchors' gS exactly zero (skipped by
    both backwards, or kept with their zero terms by the backward over the forward's binning).
    The anchors sit h * N(0, 1) off the events, so records two cells from an anchor pass the distance test and
    only the neighbourhood test keeps them out; the blob case fills cells with hundreds of records and
    anchors (several 64-wide chunks on both sides)."""
    win = synth.small_window(seed=4, n=n, H=40, W=48, B=B, scene=scene)
    v, _, _ = O.dense_velocity(win.motion["grid"], win.xy, win.b, 40, 48)
    rng = np.random.default_rng(104)
    xs = (win.xy + rng.uniform(-0.5, 0.5, win.xy.shape)).astype(F32)
    anchors = np.arange(win.n)
    xa = (xs + h * rng.standard_normal(xs.shape)).astype(F32)
    p = O.build_pair_plan(xs, win.t, v, win.b, B, 40, 48, anchors, h, tau, 3.0, S, anchor_xy=xa)
    q = F.build_pair_plan(T(xs), T(win.t), T(v), T(win.b), B, 40, 48, T(anchors), h, tau, 3.0, S, anchor_xy=T(xa))
    gS = rng.standard_normal(len(anchors)).astype(F32)
    gS[rng.random(len(anchors)) < zero_frac] = 0
    want = O.ats_pair_bwd(gS, p, h, tau, 3.0, win.n)
    e = F.get_ext()
    args = (q.src_y, q.src_v, q.src_t, q.src_id, q.cell_start, q.anc_x, q.anc_t, q.anc_cell, q.anc_id, q.slice_c,
            q.S, q.GH, q.GW, h, tau, 3.0, win.n)
    if scene == "blobs":
        assert np.diff(N(q.cell_start)).max() > 200
    want_s, want_n = O.ats_pair_fwd(p, h, tau, 3.0, with_counts=True)
    for plan_order in (False, True):
        cnt = torch.full((len(anchors),), -7, dtype=torch.int32, device=DEV)
        got = N(e.ats_pair_fwd(*args[:-1], count=cnt, plan_order=plan_order))
        assert np.array_equal(N(cnt), want_n)
        assert_sums_close(got, want_s)
    for atomics in (False, True):
        close_rel(N(e.ats_pair_bwd(T(gS), *args, per_pair_atomics=atomics)), want, 1e-4)
    # the backward over the forward's anchor binning (the workspace kept from the forward): two atomics per
    # entry, or (the workspace sized with the source count) one slot per source and slice, added per source
    for n_src in (None, win.n):
        _, ws = e.ats_pair_fwd(*args[:-1], keep_ws=True, n_src=n_src)
        close_rel(N(e.ats_pair_bwd(T(gS), *args, ws=ws)), want, 1e-4)


def test_ats_pair_sums_api_matches_bruteforce():
    """Reference test_ats_pair_matches_bruteforce (tests/test_ops.py:62-77) on the device: plan + kernel vs the
    O(MN) brute force, values and gradients."""
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


# ------------------------------------------------------------------------------------------- anchored pieces
def test_window_counts_bit_exact():
    _, _, b, t = rand_events(n=20000, B=3, seed=4)
    idx = np.arange(0, 20000, 3)
    for tau in (0.01, 0.2, 1.0):
        got = F.window_counts(T(t), T(b), T(idx), tau)
        assert np.array_equal(N(got), O.window_counts(t, b, idx, tau))
    got = F.window_counts(T(np.array([0.0, 0.1, 0.2, 0.9, 0.0, 0.5], F32)), T(np.array([0, 0, 0, 0, 1, 1])),
                          T(np.arange(6)), 0.15)
    assert N(got).tolist() == [1, 2, 1, 0, 0, 0]
    perm = np.random.default_rng(5).permutation(20000)          # unsorted input is sorted first
    got = F.window_counts(T(t[perm]), T(b[perm]), T(idx), 0.2)
    assert np.array_equal(N(got), O.window_counts(t[perm], b[perm], idx, 0.2))


@pytest.mark.parametrize("sorted_path", [False, True])
def test_visible_fraction_bit_exact(sorted_path):
    win, xs, v, anchors, xa = _pair_case(seed=6)
    grid = win.motion["grid"]
    va, _, _ = O.dense_velocity(grid, xa, win.b[anchors], 40, 48)
    got = F.visible_fraction_linear(T(xa), T(va), T(win.t[anchors]), T(win.b[anchors]), T(win.t), T(win.b), 2, 40,
                                    48, 0.2, assume_sorted=sorted_path)
    want = O.visible_fraction_dense(grid, xa, win.t[anchors], win.b[anchors], win.t, win.b, 2, 40, 48, 0.2)
    assert np.array_equal(N(got), want)


@pytest.mark.parametrize("n_check", [16, 10, 1])
def test_bin_counts_sorted_matches_index_put(n_check):
    """Counts per (batch, time bin) from the bin-edge searches over (b, t)-sorted events vs the reference's
    index_put accumulate (atl/objectives/ats.py:39-41): times on bin edges, below 0, at and above 1, an empty
    batch."""
    rng = np.random.default_rng(3)
    B = 4
    t = np.concatenate([rng.random(30000), np.arange(n_check + 1) / n_check, [-0.5, -1e-7, 1.0, 1.5, 7.0]])
    t = t.astype(F32)
    b = rng.choice([0, 1, 3], size=t.size).astype(np.int64)           # batch 2 empty
    order = np.lexsort((t, b))
    t, b = t[order], b[order]
    sl = np.clip(torch.as_tensor(t * F32(n_check)).long().numpy(), 0, n_check - 1)
    want = np.zeros((B, n_check), np.float32)
    np.add.at(want, (b, sl), 1.0)
    got_sorted = N(F.bin_counts(T(t), T(b), B, n_check, assume_sorted=True))
    got_atomic = N(F.bin_counts(T(t), T(b), B, n_check, assume_sorted=False))
    assert np.array_equal(got_sorted, want) and np.array_equal(got_atomic, want)


def test_anchored_exact_end_to_end():
    """AnchoredExact (dense linear flow) log scores and flow-grid gradient vs the oracle pipeline."""
    from x_amd.core import EventPacket
    from x_amd.motion import DenseLinearFlow
    from x_amd.objectives import AnchoredExact
    win = synth.small_window(seed=8, n=4000, B=2)
    H, W = win.height, win.width
    ev = EventPacket.from_window(win, DEV)
    grid = win.motion["grid"]
    m = DenseLinearFlow(2, H, W, grid=grid.shape[-2:], init=torch.as_tensor(grid)).to(DEV)
    obj = AnchoredExact(h=1.0, tau=0.2, n_anchors=None, seed=0, n_slices=16)
    ls, anchors = obj.log_scores(ev, m)
    (-ls.mean()).backward()
    # oracle: same draws (CPU generator, same order), then the plan, pair sums, counts, visibility, epilogue
    g = torch.Generator().manual_seed(0)
    xs = win.xy + (torch.rand(win.xy.shape, generator=g).numpy() - F32(0.5))
    xa = xs + F32(1.0) * torch.randn(xs.shape, generator=g).numpy()
    v, idx, wts = O.dense_velocity(grid, xs, win.b, H, W)
    p = O.build_pair_plan(xs, win.t, v, win.b, 2, H, W, np.arange(win.n), 1.0, 0.2, 3.0, 16, anchor_xy=xa)
    Sv = O.ats_pair_fwd(p, 1.0, 0.2, 3.0)
    wc = O.window_counts(win.t, win.b, np.arange(win.n), 0.2)
    vis = O.visible_fraction_dense(grid, xa, win.t, win.b, win.t, win.b, 2, H, W, 0.2)
    want, gS, _ = O.anchored_epilogue(Sv, wc, 1.0, H, W, vis=vis)
    assert_logs_close(N(ls), want)
    gv = O.ats_pair_bwd(gS, p, 1.0, 0.2, 3.0, win.n)
    ggrid = O.sample_grid_bwd(gv, idx, wts, grid.shape)
    close_rel(N(m.grid.grad), ggrid, 1e-4)


def test_anchored_exact_fused_loss():
    """The objective's loss (epilogue, mean and negation fused in one launch, double sum in a fixed order) and
    its flow-grid gradient vs the oracle pipeline; score = -loss."""
    from x_amd.core import EventPacket
    from x_amd.motion import DenseLinearFlow
    from x_amd.objectives import AnchoredExact
    win = synth.small_window(seed=8, n=4000, B=2)
    H, W = win.height, win.width
    ev = EventPacket.from_window(win, DEV)
    grid = win.motion["grid"]
    m = DenseLinearFlow(2, H, W, grid=grid.shape[-2:], init=torch.as_tensor(grid)).to(DEV)
    out = AnchoredExact(h=1.0, tau=0.2, n_anchors=None, seed=0, n_slices=16)(ev, m)
    out["loss"].backward()
    assert float(out["score"]) == -float(out["loss"].detach()) and not out["score"].requires_grad
    g = torch.Generator().manual_seed(0)
    xs = win.xy + (torch.rand(win.xy.shape, generator=g).numpy() - F32(0.5))
    xa = xs + F32(1.0) * torch.randn(xs.shape, generator=g).numpy()
    v, idx, wts = O.dense_velocity(grid, xs, win.b, H, W)
    p = O.build_pair_plan(xs, win.t, v, win.b, 2, H, W, np.arange(win.n), 1.0, 0.2, 3.0, 16, anchor_xy=xa)
    Sv = O.ats_pair_fwd(p, 1.0, 0.2, 3.0)
    wc = O.window_counts(win.t, win.b, np.arange(win.n), 0.2)
    vis = O.visible_fraction_dense(grid, xa, win.t, win.b, win.t, win.b, 2, H, W, 0.2)
    want, gS, _ = O.anchored_epilogue(Sv, wc, 1.0, H, W, vis=vis)
    loss = -float(np.mean(want.astype(np.float64)))
    assert abs(float(out["loss"].detach()) - loss) <= 1e-5 * abs(loss)
    gv = O.ats_pair_bwd(gS, p, 1.0, 0.2, 3.0, win.n)
    close_rel(N(m.grid.grad), O.sample_grid_bwd(gv, idx, wts, grid.shape), 1e-4)


def test_anchored_exact_device_rng_full_size():
    """The benchmarked step end to end: AnchoredExact(rng="device") on the 1M-event 640x480 dense-flow window
    (h = 1, tau = 0.2, cut = 3, 16 slices, every event an anchor), whose noise is the fused Philox draw.  The
    oracle gets the same draw (event_noise with the objective's seed and first offset) and runs the whole
    pipeline: log scores within 1e-5, the fused loss within 1e-5 and the flow-grid gradient within 1e-4."""
    from x_amd.core import EventPacket
    from x_amd.motion import DenseLinearFlow
    from x_amd.objectives import AnchoredExact
    print("anchored exact rng=device, 1M events", flush=True)
    win = synth.dense_flow_window(seed=0)
    H, W, n = win.height, win.width, win.n
    ev = EventPacket.from_window(win, DEV)
    grid = win.motion["grid"]
    xs_d, xa_d = F.event_noise(ev.xy, 0, 0, 1.0)                 # the draw of the objective's first call
    xs, xa = N(xs_d), N(xa_d)
    v, idx, wts = O.dense_velocity(grid, xs, win.b, H, W)
    p = O.build_pair_plan(xs, win.t, v, win.b, 1, H, W, np.arange(n), 1.0, 0.2, 3.0, 16, anchor_xy=xa)
    Sv = O.ats_pair_fwd(p, 1.0, 0.2, 3.0)
    wc = O.window_counts(win.t, win.b, np.arange(n), 0.2)
    vis = O.visible_fraction_dense(grid, xa, win.t, win.b, win.t, win.b, 1, H, W, 0.2)
    want, gS, _ = O.anchored_epilogue(Sv, wc, 1.0, H, W, vis=vis)
    ggrid = O.sample_grid_bwd(O.ats_pair_bwd(gS, p, 1.0, 0.2, 3.0, n), idx, wts, grid.shape)
    for form in ("log_scores", "loss"):
        m = DenseLinearFlow(1, H, W, grid=grid.shape[-2:], init=torch.as_tensor(grid)).to(DEV)
        obj = AnchoredExact(h=1.0, tau=0.2, cut=3.0, n_slices=16, n_anchors=None, seed=0, rng="device")
        if form == "log_scores":
            ls, _ = obj.log_scores(ev, m)
            assert_logs_close(N(ls), want)
            (-ls.mean()).backward()
        else:
            out = obj(ev, m)
            loss = -float(np.mean(want.astype(np.float64)))
            assert abs(float(out["loss"].detach()) - loss) <= 1e-5 * abs(loss)
            out["loss"].backward()
        close_rel(N(m.grid.grad), ggrid, 1e-4)


def test_window_counts_and_pair_sums_without_index():
    """anchors=None (every event, in order) gives the same window counts and pair sums as anchors=arange(N)
    (the sums to the last bits only: the order of the records within a cell, and so the summation order, is set
    by LDS atomics in the sort)."""
    pos, _, bb, tt = rand_events(seed=5, n=5000, B=2, H=30, W=40)
    t, b, x = T(tt), T(bb), T(pos)
    v = torch.randn(x.shape, device=DEV)
    ar = torch.arange(x.shape[0], device=DEV)
    assert torch.equal(F.window_counts(t, b, None, 0.2), F.window_counts(t, b, ar, 0.2))
    s0 = F.ats_pair_sums(x, t, v, b, 2, 30, 40, None, 1.0, 0.2)
    s1 = F.ats_pair_sums(x, t, v, b, 2, 30, 40, ar, 1.0, 0.2)
    close_rel(N(s0), N(s1), 1e-6)


@pytest.mark.parametrize("n,B,dup", [(1_000_000, 1, False), (300_000, 3, True), (700, 2, True)])
def test_window_counts_every_event_bit_exact(n, B, dup):
    """Window counts with every event as anchor (the block-cooperative bound search) vs the oracle, bit-exact:
    1M events in one window, several batches, and runs of equal timestamps."""
    print(f"window counts n={n} B={B} dup={dup}", flush=True)
    rng = np.random.default_rng(n)
    t = rng.random(n).astype(np.float32)
    if dup:
        t = np.round(t * 997).astype(np.float32) / np.float32(997)   # many equal keys
    b = rng.integers(0, B, n).astype(np.int64)
    order = np.lexsort((t, b))
    t, b = t[order], b[order]
    got = N(F.window_counts(T(t), T(b), None, 0.2, assume_sorted=True))
    assert np.array_equal(got, O.window_counts(t, b, np.arange(n), 0.2))


# ------------------------------------------------------------------------------------------- full size
def test_full_size_splat_gather_properties():
    """1M events at 640x480 (dense flow, warp to t_ref = 0.5): mass conservation of the splat and the adjoint
    identities <splat(w), G> = <w, gather(G)> and splat_bwd.gw = gather_fwd at the same positions."""
    win = synth.dense_flow_window(seed=0)
    grid = T(win.motion["grid"])
    xy, t, b = T(win.xy), T(win.t), T(win.b)
    v = F.sample_grid_hip(grid, xy, b, img_hw=(480, 640))
    pos = xy + v * (0.5 - t)[:, None]
    inside = ((pos[:, 0] >= 0) & (pos[:, 0] <= 639) & (pos[:, 1] >= 0) & (pos[:, 1] <= 479)).float()
    img = F.splat(pos, inside, b, 1, 480, 640)
    assert abs(float(img.double().sum()) - float(inside.double().sum())) < 1e-6 * win.n + 1.0
    G = torch.randn(1, 480, 640, device=DEV)
    val = F.gather(G, pos, b)
    lhs = float((img.double() * G.double()).sum())
    rhs = float((inside.double() * val.double()).sum())
    assert abs(lhs - rhs) < 1e-4 * (abs(lhs) + float(inside.sum()))
    _, gw = F.get_ext().splat_bilinear_bwd(G.contiguous(), pos.contiguous(), inside.contiguous(), b)
    assert torch.equal(gw, val)


@pytest.mark.parametrize("kernel,sigma,polarity,mask,dt", [("bilinear", 0.0, "pooled", True, False),
                                                          ("bilinear", 1.0, "split", True, True),
                                                          ("bilinear", 2.5, "pooled", False, True),
                                                          ("gauss", 1.0, "split", False, False),
                                                          ("gauss", 0.7, "pooled", True, True)])
def test_make_iwe_matches_oracle(kernel, sigma, polarity, mask, dt):
    """make_iwe on the device (weights, border mask, time weighting, polarity split, splat, blur) against the
    oracle's IWE (atl/objectives/base.py:40-60): within 1e-5 of the largest pixel."""
    from x_amd.core import EventPacket
    from x_amd.objectives import IWEConfig, make_iwe
    print(f"make_iwe {kernel} sigma={sigma} {polarity} mask={mask} dt={dt}", flush=True)
    win = synth.small_window(seed=17, n=5000, B=2)
    rng = np.random.default_rng(17)
    xy_ref = (win.xy + rng.normal(0, 2, win.xy.shape)).astype(F32)          # some outside the sensor
    ev = EventPacket.from_window(win, DEV)
    cfg = IWEConfig(kernel=kernel, sigma=sigma, polarity=polarity, mask_border=mask, scale_by_dt=dt)
    got = N(make_iwe(ev, T(xy_ref), 0.3, cfg))
    want = O.make_iwe(xy_ref, win.t, win.p, win.b, 2, win.height, win.width, 0.3, kernel, sigma, polarity, mask, dt)
    assert got.shape == want.shape
    close_rel(got, want, 1e-5)


def test_blur_matches_oracle_and_keeps_interior_mass():
    """blur (two 1-D passes) against the oracle's scipy correlate1d blur, (B, H, W) and (B, C, H, W); an image
    whose support stays 3 sigma from the border keeps its mass."""
    rng = np.random.default_rng(18)
    for shape, sigma in (((2, 40, 52), 1.0), ((2, 3, 30, 31), 1.7)):
        img = rng.standard_normal(shape).astype(F32)
        close_rel(N(F.blur(T(img), sigma)), O.blur(img, sigma), 1e-5)
    img = np.zeros((1, 40, 40), F32)
    img[0, 10:30, 12:28] = rng.random((20, 16))
    out = N(F.blur(T(img), 2.0))
    assert abs(float(out.sum()) - float(img.sum())) <= 1e-5 * float(img.sum())


@pytest.mark.parametrize("shape", [(4, 480, 640), (1, 37, 53), (2, 3, 5, 7), (3, 1, 1)])
def test_image_variance_matches_fp64(shape):
    """The IWE contrast's per-image variance (atl/objectives/cmax.py:23-25, iwe.var(dim=(-2, -1))) and its
    gradient against torch's float64 var on the same images: an IWE-like image (counts plus a constant offset,
    where the one-pass sum of squares cancels most), a small odd size, extra leading dimensions, and one-pixel
    images (NaN, as torch.var)."""
    print(f"image_variance shape={shape}", flush=True)
    rng = np.random.default_rng(len(shape) + shape[-1])
    img = (rng.poisson(2.0, shape) + 50.0 + rng.uniform(0, 1, shape)).astype(F32)
    g = rng.standard_normal(shape[:-2]).astype(F32)
    x = T(img).requires_grad_(True)
    v = F.image_variance(x)
    if shape[-1] * shape[-2] == 1:
        assert torch.isnan(v).all()
        return
    x64 = torch.as_tensor(img.astype(np.float64)).requires_grad_(True)
    v64 = x64.var(dim=(-2, -1))
    close_rel(N(v), v64.detach().numpy(), 1e-6)
    (v * T(g)).sum().backward()
    (v64 * torch.as_tensor(g.astype(np.float64))).sum().backward()
    close_rel(N(x.grad), x64.grad.numpy(), 1e-5)
