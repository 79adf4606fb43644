"""atl_splat_bilinear_fwd_noalloc (the splat forward without device allocation) against the workspace form
atl_splat_bilinear_fwd_ws, both called through the C-ABI: two calls in a row, the second smaller and on another
image shape (the library's scratch keeps the first call's contents), a call too large for the scratch, which
must fail before any launch, and the call recorded in a HIP graph (its scratch address resolved by atl_init at
load), replayed with eager work between replays."""
import numpy as np
import pytest
import torch

from x_amd.ops import _ext
from x_amd.ops._ext import HipLibraryError, call, ptr

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _events(n, B, H, W, seed):
    rng = np.random.default_rng(seed)
    pos = np.stack([rng.random(n) * (W + 4) - 2, rng.random(n) * (H + 4) - 2], 1).astype(np.float32)
    pos[: n // 10] = np.floor(pos[: n // 10])              # integer positions: one pixel each
    w = (rng.random(n) + 0.1).astype(np.float32)
    w[n // 10: n // 10 + 100] = 0.0                        # zero weights add nothing
    b = np.sort(rng.integers(0, B, n)).astype(np.int64)
    return (torch.as_tensor(pos, device=DEV), torch.as_tensor(w, device=DEV), torch.as_tensor(b, device=DEV))


def _both(pos, w, b, B, H, W):
    N = pos.shape[0]
    s = torch.cuda.current_stream().cuda_stream
    nbytes = _ext.load_library().atl_tile_ws_bytes(N, B, H, W)
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    ref = torch.zeros(B, H, W, device=DEV)
    call("atl_splat_bilinear_fwd_ws", ptr(pos), ptr(w), ptr(b), N, B, H, W, ptr(ref), ptr(ws), nbytes, s)
    got = torch.zeros(B, H, W, device=DEV)
    call("atl_splat_bilinear_fwd_noalloc", ptr(pos), ptr(w), ptr(b), N, B, H, W, ptr(got), s)
    torch.cuda.synchronize()
    return ref.cpu().numpy(), got.cpu().numpy()


def _check(ref, got):
    # same pixels (bit-exact support), values within 1e-5 of the largest (float sums in another order)
    assert np.array_equal(ref != 0, got != 0)
    scale = max(float(np.abs(ref).max()), 1e-30)
    assert float(np.abs(got - ref).max()) <= 1e-5 * scale
    assert abs(float(got.sum()) - float(ref.sum())) <= 1e-5 * max(abs(float(ref.sum())), 1.0)


def test_noalloc_splat_matches_workspace_form_twice():
    print("noalloc: call 1, 1M events, 640x480, B=1", flush=True)
    pos, w, b = _events(1_000_000, 1, 480, 640, seed=0)
    _check(*_both(pos, w, b, 1, 480, 640))
    print("noalloc: call 2, 60k events, 100x120, B=3", flush=True)
    pos, w, b = _events(60_000, 3, 100, 120, seed=1)
    _check(*_both(pos, w, b, 3, 100, 120))


def test_noalloc_splat_rejects_sizes_beyond_its_scratch():
    N = 5_000_000                                          # 80 MB of records: more than the 64 MiB scratch
    pos = torch.zeros(N, 2, device=DEV)
    w = torch.ones(N, device=DEV)
    b = torch.zeros(N, dtype=torch.int64, device=DEV)
    img = torch.zeros(1, 480, 640, device=DEV)
    with pytest.raises(HipLibraryError, match="more than the library's"):
        call("atl_splat_bilinear_fwd_noalloc", ptr(pos), ptr(w), ptr(b), N, 1, 480, 640, ptr(img),
             torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert float(img.abs().sum()) == 0.0                   # nothing launched


def test_noalloc_splat_under_graph_capture():
    print("noalloc: captured call, 300k events, 480x640", flush=True)
    lib = _ext.load_library()
    assert lib.atl_init() == 0
    B, H, W = 1, 480, 640
    pos, w, b = _events(300_000, B, H, W, seed=2)
    N = pos.shape[0]
    nbytes = lib.atl_tile_ws_bytes(N, B, H, W)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    ref = torch.zeros(B, H, W, device=DEV)
    call("atl_splat_bilinear_fwd_ws", ptr(pos), ptr(w), ptr(b), N, B, H, W, ptr(ref), ptr(ws), nbytes,
         torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    img = torch.zeros(B, H, W, device=DEV)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call("atl_splat_bilinear_fwd_noalloc", ptr(pos), ptr(w), ptr(b), N, B, H, W, ptr(img),
             torch.cuda.current_stream().cuda_stream)
    for r in range(3):
        img.zero_()                                        # the image is accumulated: cleared outside the graph
        _ = torch.randn(1000, device=DEV).sum().item()     # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        _check(ref.cpu().numpy(), img.cpu().numpy())
