"""The fused warp -> splat -> gather launches (atl_warp_splat_gather_fwd/bwd) against the oracle's composition of
the same steps (dense-flow lookup, linear warp, inside mask, bilinear splat, gather, and their adjoints) and
against the package's composed device path, on identical seeded inputs.

Bars: image and gathered values within 1e-5 of the largest magnitude (float sums in another order), flow-grid
gradient within 1e-4 of its largest magnitude."""
import numpy as np
import pytest
import torch

import oracle as O
from x_amd import synth
from x_amd.core import EventPacket
from x_amd.motion import DenseLinearFlow
from x_amd.objectives import IWEConfig, iwe_at_events, make_iwe
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


def oracle_wsg(grid, xy, t, b, t_ref, B, H, W, mask, gvals, gimg):
    """The composed reference steps on the host: returns img, vals, the flow-grid gradient of
    <gvals, vals> + <gimg, img>."""
    v, idx, wts = O.dense_velocity(grid, xy, b, H, W)
    step = (F32(t_ref) - t).astype(F32)
    y = (xy + v * step[:, None]).astype(F32)
    if mask:
        w = ((y[:, 0] >= 0) & (y[:, 0] <= W - 1) & (y[:, 1] >= 0) & (y[:, 1] <= H - 1)).astype(F32)
    else:
        w = np.ones(len(t), F32)
    img = O.splat_bilinear_fwd(y, w, b, B, H, W)
    vals = O.gather_bilinear_fwd(img, y, b)
    gi, gp1 = O.gather_bilinear_bwd(gvals, img, y, b)
    G = (gi + gimg).astype(F32)
    gp2, _ = O.splat_bilinear_bwd(G, y, w, b)
    gv = ((gp1 + gp2) * step[:, None]).astype(F32)
    return img, vals, O.sample_grid_bwd(gv, idx, wts, grid.shape)


@pytest.mark.parametrize("mask", [True, False])
@pytest.mark.parametrize("B,H,W,vmax", [(1, 40, 48, 6.0), (2, 37, 53, 12.0), (3, 20, 24, 30.0)])
def test_warp_splat_gather_matches_oracle(B, H, W, vmax, mask):
    """Small windows: several batch entries, flows that carry events out of the sensor (masked, or splatted onto
    the border with base corner -1), a value gradient and an image gradient together."""
    print(f"warp_splat_gather oracle B={B} {H}x{W} vmax={vmax} mask={mask}", flush=True)
    win = synth.small_window(seed=B + H, n=4000, H=H, W=W, vmax=vmax, B=B)
    rng = np.random.default_rng(B)
    grid = win.motion["grid"].astype(F32)
    gvals = rng.standard_normal(win.n).astype(F32)
    gimg = rng.standard_normal((B, H, W)).astype(F32)
    t_ref = 0.37
    want_img, want_vals, want_g = oracle_wsg(grid, win.xy, win.t, win.b, t_ref, B, H, W, mask, gvals, gimg)
    tg = T(grid).requires_grad_(True)
    img, vals = F.warp_splat_gather(tg, T(win.xy), T(win.t), T(win.b), t_ref, H, W, mask)
    close_rel(N(img), want_img, 1e-5)
    close_rel(N(vals), want_vals, 1e-5)
    ((vals * T(gvals)).sum() + (img * T(gimg)).sum()).backward()
    close_rel(N(tg.grad), want_g, 1e-4)


@pytest.mark.parametrize("B,H,W,Hg,Wg", [(2, 40, 48, 9, 14), (8, 480, 640, 480, 640)])
def test_warp_splat_gather_grid_shapes(B, H, W, Hg, Wg):
    """A coarse flow grid, and eight full-sensor windows: their image and flow-grid tile histograms together
    exceed one workgroup's histogram, so the backward counts the flow-grid tiles itself.  Outputs are written,
    not accumulated: the buffers the wrapper allocates hold whatever was there before."""
    print(f"warp_splat_gather grid shape B={B} {H}x{W} grid {Hg}x{Wg}", flush=True)
    win = synth.small_window(seed=B, n=2500, H=H, W=W, vmax=10.0, B=B)
    rng = np.random.default_rng(Hg)
    grid = rng.uniform(-10.0, 10.0, (B, 2, Hg, Wg)).astype(F32)
    gvals = rng.standard_normal(win.n).astype(F32)
    gimg = rng.standard_normal((B, H, W)).astype(F32)
    want_img, want_vals, want_g = oracle_wsg(grid, win.xy, win.t, win.b, 0.5, B, H, W, True, gvals, gimg)
    stale = torch.full((B * H * W * 4,), float("nan"), device=DEV)
    del stale                                                    # NaNs left in the allocator's free blocks
    tg = T(grid).requires_grad_(True)
    img, vals = F.warp_splat_gather(tg, T(win.xy), T(win.t), T(win.b), 0.5, H, W, True)
    close_rel(N(img), want_img, 1e-5)
    close_rel(N(vals), want_vals, 1e-5)
    ((vals * T(gvals)).sum() + (img * T(gimg)).sum()).backward()
    close_rel(N(tg.grad), want_g, 1e-4)


def test_warp_splat_gather_values_only_and_image_only():
    """Gradients through one output at a time (the other's gradient absent)."""
    win = synth.small_window(seed=5, n=5000, H=30, W=44, vmax=8.0, B=2)
    grid = win.motion["grid"].astype(F32)
    rng = np.random.default_rng(9)
    gvals = rng.standard_normal(win.n).astype(F32)
    gimg = rng.standard_normal((2, 30, 44)).astype(F32)
    for use_vals in (True, False):
        print(f"warp_splat_gather one output: vals={use_vals}", flush=True)
        gv = gvals if use_vals else np.zeros_like(gvals)
        gi = np.zeros_like(gimg) if use_vals else gimg
        _, _, want_g = oracle_wsg(grid, win.xy, win.t, win.b, 0.5, 2, 30, 44, True, gv, gi)
        tg = T(grid).requires_grad_(True)
        img, vals = F.warp_splat_gather(tg, T(win.xy), T(win.t), T(win.b), 0.5, 30, 44)
        ((vals * T(gvals)).sum() if use_vals else (img * T(gimg)).sum()).backward()
        close_rel(N(tg.grad), want_g, 1e-4)


def test_warp_splat_gather_full_size_matches_oracle_and_composed():
    """The IWE workload itself: 1M events, 640x480, dense flow of up to 20 px per window, t_ref = 0.5, inside
    mask, loss = sum of the gathered values; against the oracle and against transport -> make_iwe -> gather on
    the device."""
    win = synth.dense_flow_window(seed=0)
    ev = EventPacket.from_window(win, DEV)
    grid = win.motion["grid"].astype(F32)
    H, W = win.height, win.width
    print("warp_splat_gather full size: oracle", flush=True)
    want_img, want_vals, want_g = oracle_wsg(grid, win.xy, win.t, win.b, 0.5, 1, H, W, True,
                                             np.ones(win.n, F32), np.zeros((1, H, W), F32))
    print("warp_splat_gather full size: fused", flush=True)
    motion = DenseLinearFlow(1, H, W, grid=grid.shape[-2:], init=torch.as_tensor(grid)).to(DEV)
    cfg = IWEConfig(kernel="bilinear", sigma=0.0, mask_border=True)
    img, vals = iwe_at_events(ev, motion, 0.5, cfg)
    vals.sum().backward()
    g_fused = N(motion.grid.grad)
    close_rel(N(img), want_img, 1e-5)
    close_rel(N(vals), want_vals, 1e-5)
    close_rel(g_fused, want_g, 1e-4)
    print("warp_splat_gather full size: composed device path", flush=True)
    motion.grid.grad = None
    y = motion.transport(ev.xy, ev.t, 0.5, ev.b)
    img2 = make_iwe(ev, y, 0.5, cfg)
    F.gather(img2, y, ev.b).sum().backward()
    close_rel(N(img), N(img2), 1e-5)
    close_rel(g_fused, N(motion.grid.grad), 1e-4)


@pytest.mark.parametrize("B", [1, 3])
def test_translation_iwe_takes_the_fused_launches(B):
    """A translation's IWE at the events runs the fused launches on a one-node grid (whose bilinear sample is theta
    exactly, so the warped positions are the composed transport's): image, values and theta's gradient within
    1e-5 of transport -> make_iwe -> gather (sums in another order); on the plumbing workload (100k events
    240x180) and on a batch of three windows."""
    from x_amd.motion import Translation
    win = synth.plumbing_translation(seed=B) if B == 1 else synth.small_window(seed=B, n=3000, B=B)
    ev = EventPacket.from_window(win, DEV)
    theta = (np.asarray(win.motion["theta"], F32)[None] if B == 1 else
             np.random.default_rng(B).uniform(-3, 3, (B, 2)).astype(F32))
    cfg = IWEConfig(kernel="bilinear", sigma=0.0, mask_border=True)
    w = T(np.random.default_rng(B + 7).standard_normal(win.n).astype(F32))
    res = []
    for fused in (True, False):
        m = Translation(B, win.height, win.width, init=torch.as_tensor(theta)).to(DEV)
        if fused:
            img, vals = iwe_at_events(ev, m, 0.0 if B == 1 else 0.5, cfg)
        else:
            y = m.transport(ev.xy, ev.t, 0.0 if B == 1 else 0.5, ev.b)
            img = make_iwe(ev, y, 0.0 if B == 1 else 0.5, cfg)
            vals = F.gather(img, y, ev.b)
        (vals * w).sum().backward()
        res.append((img.detach(), vals.detach(), m.theta.grad.clone()))
    close_rel(N(res[0][0]), N(res[1][0]), 1e-5)
    close_rel(N(res[0][1]), N(res[1][1]), 1e-5)
    close_rel(N(res[0][2]), N(res[1][2]), 1e-5)


@pytest.mark.parametrize("kind", ["translation", "dense"])
def test_iwe_step_graph_replays_match_eager(kind):
    """The IWE step (fused launches, then the sum's backward to the motion) captured as one HIP graph, as the
    bench times it: every replay, with eager work and a synchronisation between replays, gives the eager step's
    values and gradient (to the order of the atomic additions)."""
    from x_amd.motion import Translation
    print(f"graph replays: {kind}", flush=True)
    if kind == "translation":
        win = synth.plumbing_translation(seed=3)
        m = Translation(1, win.height, win.width, init=torch.as_tensor(np.asarray(win.motion["theta"], F32))[None])
    else:
        win = synth.small_window(seed=3, n=20000, H=40, W=48)
        m = DenseLinearFlow(1, 40, 48, grid=(40, 48), init=torch.as_tensor(win.motion["grid"].astype(F32)))
    m = m.to(DEV)
    ev = EventPacket.from_window(win, DEV)
    cfg = IWEConfig(kernel="bilinear", sigma=0.0, mask_border=True)
    prm = list(m.parameters())
    ones = torch.ones(ev.n, device=DEV)        # d sum(vals) / d vals: no reduction (and no memset) in the graph

    def body():
        _, vals = iwe_at_events(ev, m, 0.5, cfg)
        vals.backward(ones)
        return vals

    for q in prm:
        q.grad = None
    v_ref = body().detach().clone()
    g_ref = [N(q.grad) for q in prm]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            for q in prm:
                q.grad = None
            body()
    torch.cuda.current_stream().wait_stream(side)
    for q in prm:
        q.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        v_out = body()
    for r in range(4):
        for q in prm:
            q.grad.fill_(123.0)                    # eager work between replays; the replay overwrites it
        _ = torch.randn(1000, device=DEV).sum().item()
        graph.replay()
        torch.cuda.synchronize()
        close_rel(N(v_out), N(v_ref), 1e-5)
        for q, gr in zip(prm, g_ref):
            close_rel(N(q.grad), gr, 1e-4)


def _hip_runtime():
    """The HIP runtime this process already loaded (torch's), so the graph handles below belong to it."""
    import ctypes
    import os
    with open("/proc/self/maps") as f:
        for line in f:
            path = line.split()[-1]
            if os.path.basename(path).startswith("libamdhip64.so"):
                return ctypes.CDLL(path)
    return ctypes.CDLL("libamdhip64.so")


def _graph_node_types(graph):
    import ctypes
    lib = _hip_runtime()
    g = ctypes.c_void_p(int(graph.raw_cuda_graph()))
    n = ctypes.c_size_t(0)
    assert lib.hipGraphGetNodes(g, None, ctypes.byref(n)) == 0
    nodes = (ctypes.c_void_p * max(n.value, 1))()
    assert lib.hipGraphGetNodes(g, nodes, ctypes.byref(n)) == 0
    types = []
    for i in range(n.value):
        kind = ctypes.c_int(-1)
        assert lib.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(kind)) == 0
        types.append(kind.value)
    return types


def test_iwe_step_graph_has_no_memset_node():
    """The bench's captured IWE step (fused launches, then the backward seeded with ones) holds kernel nodes only:
    no memset node (hipGraphNodeTypeMemset = 2), which gave wrong results on replays on these GPUs; every fill is a
    kernel.  The graph is kept and inspected, not replayed."""
    print("graph node types: iwe step", flush=True)
    win = synth.small_window(seed=3, n=20000, H=40, W=48)
    m = DenseLinearFlow(1, 40, 48, grid=(40, 48), init=torch.as_tensor(win.motion["grid"].astype(F32))).to(DEV)
    ev = EventPacket.from_window(win, DEV)
    cfg = IWEConfig(kernel="bilinear", sigma=0.0, mask_border=True)
    prm = list(m.parameters())
    ones = torch.ones(ev.n, device=DEV)

    def body():
        _, vals = iwe_at_events(ev, m, 0.5, cfg)
        vals.backward(ones)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            for q in prm:
                q.grad = None
            body()
    torch.cuda.current_stream().wait_stream(side)
    for q in prm:
        q.grad = None
    graph = torch.cuda.CUDAGraph(keep_graph=True)
    with torch.cuda.graph(graph):
        body()
    torch.cuda.synchronize()
    types = _graph_node_types(graph)
    graph.reset()
    assert types, "no nodes captured"
    print(f"{len(types)} nodes, types {sorted(set(types))}", flush=True)
    assert 2 not in types, f"memset nodes in the captured step: {types.count(2)} of {len(types)}"
    assert types.count(0) >= 8                     # the step's kernels


def test_warp_splat_gather_no_events():
    """No events: the image and the flow-grid gradient are still written (zeros), though the wrapper allocates
    both uninitialised, with NaNs left in the allocator's free blocks."""
    stale = torch.full((4 * 2 * 30 * 44,), float("nan"), device=DEV)
    del stale
    tg = torch.ones(2, 2, 30, 44, device=DEV, requires_grad=True)
    xy = torch.zeros(0, 2, device=DEV)
    img, vals = F.warp_splat_gather(tg, xy, torch.zeros(0, device=DEV), torch.zeros(0, dtype=torch.long, device=DEV),
                                    0.5, 30, 44)
    assert img.shape == (2, 30, 44) and vals.shape == (0,)
    assert torch.count_nonzero(img).item() == 0 and not torch.isnan(img).any()
    (img * torch.randn_like(img)).sum().backward()
    assert torch.count_nonzero(tg.grad).item() == 0 and not torch.isnan(tg.grad).any()


def test_warp_splat_gather_rejects_bad_shapes():
    xy = torch.zeros(10, 2, device=DEV)
    t = torch.zeros(10, device=DEV)
    b = torch.zeros(10, dtype=torch.long, device=DEV)
    with pytest.raises(ValueError):
        F.warp_splat_gather(torch.zeros(1, 3, 8, 8, device=DEV), xy, t, b, 0.5, 8, 8)
    with pytest.raises(ValueError):
        F.warp_splat_gather(torch.zeros(1, 2, 8, 8, device=DEV), xy, t[:5], b, 0.5, 8, 8)


def test_warp_splat_gather_backward_in_the_other_accumulation_form(monkeypatch):
    """The backward reuses the forward's chunk list.  With a tile of more than 16384 events the gather form lists
    2048-record chunks; a backward run in the scatter form (ATL_TILE_SCATTER=1 set between the two) takes them in
    rounds, so the flow-grid gradient still matches the oracle."""
    print("warp_splat_gather: forward gather form, backward scatter form, crowded tile", flush=True)
    H, W, n = 40, 48, 60000
    rng = np.random.default_rng(21)
    xy = np.stack([rng.uniform(0, W - 1, n), rng.uniform(0, H - 1, n)], 1).astype(F32)
    xy[: n // 2] = (np.array([20.0, 16.0]) + rng.uniform(0, 8, (n // 2, 2))).astype(F32)    # one crowded tile
    t = np.sort(rng.random(n)).astype(F32)
    b = np.zeros(n, np.int64)
    grid = (rng.standard_normal((1, 2, H, W)) * 0.5).astype(F32)
    gvals = rng.standard_normal(n).astype(F32)
    want_img, want_vals, want_g = oracle_wsg(grid, xy, t, b, 0.5, 1, H, W, True, gvals, np.zeros((1, H, W), F32))
    monkeypatch.setenv("ATL_TILE_SCATTER", "0")
    tg = T(grid).requires_grad_(True)
    img, vals = F.warp_splat_gather(tg, T(xy), T(t), T(b), 0.5, H, W)
    close_rel(N(img), want_img, 1e-5)
    close_rel(N(vals), want_vals, 1e-5)
    monkeypatch.setenv("ATL_TILE_SCATTER", "1")
    (vals * T(gvals)).sum().backward()
    close_rel(N(tg.grad), want_g, 1e-4)
