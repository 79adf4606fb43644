"""The ops API on CPU tensors (pure-torch semantics, as the reference without its extension) agrees with the
oracle; device tensors never take this path."""
import math

import numpy as np
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


def test_sliced_score_all_slices_matches_slice_loop():
    """The sliced score computed over every slice at once equals the reference's slice-by-slice loop (the loop
    path is taken with an anchor cap no slice reaches): same anchors in the same order, same scores, same
    coefficient gradient; with a random subset of slices and anchor and source masks."""
    from x_amd import synth
    from x_amd.core import EventPacket
    from x_amd.motion import PixelTrajectories
    from x_amd.objectives import AnchoredSliced
    win = synth.small_window(seed=5, n=1500, B=2)
    rng = np.random.default_rng(5)
    coeffs = synth.trajectory_coeffs(rng, 2, 3, win.height, win.width, sigma_px=8.0, dmax=3.0)
    ev = EventPacket.from_window(win, "cpu")
    g = torch.Generator().manual_seed(1)
    amask = torch.rand(ev.n, generator=g) < 0.7
    smask = torch.rand(ev.n, generator=g) < 0.8
    for smooth, sps, masks in ((True, None, False), (False, 3, True), (True, 4, True)):
        res = []
        for nap in (None, 10 ** 9):
            c = torch.tensor(coeffs, requires_grad=True)
            obj = AnchoredSliced(n_slices=6, slices_per_step=sps, sigma=1.0, tau=0.3, seed=0, smooth_anchors=smooth,
                                 n_anchors_per_slice=nap)
            ls, ai = obj.log_scores(ev, PixelTrajectories(c, 3, "bezier"), anchor_mask=amask if masks else None,
                                    source_mask=smask if masks else None)
            ls.sum().backward()
            res.append((ls.detach().numpy(), ai.numpy(), c.grad.numpy()))
        (l0, a0, g0), (l1, a1, g1) = res
        assert np.array_equal(a0, a1) and len(a0) > 0
        assert np.allclose(l0, l1, rtol=1e-6, atol=1e-6)
        assert np.allclose(g0, g1, rtol=1e-5, atol=1e-5 * np.abs(g1).max())
