"""The fused dequantisation / smoothing noise (atl_event_noise): Philox4x32-10 pinned by its published
known-answer vectors on the CPU, then the device words and transforms against that restatement."""
import numpy as np
import pytest
import torch

from tests import philox as P


# Random123's known-answer vectors for philox4x32-10 (counter, key -> output)
KAT = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    got = P.philox4x32_10(*[np.array([c], np.uint32) for c in ctr], *key)
    assert [int(w[0]) for w in got] == list(want)


def test_philox_counter_layout():
    """Event i uses counter (i lo, i hi, offset lo, offset hi): event 0 at offset 0 under key 0 is the first
    known-answer vector."""
    r = P.event_noise_words(3, 0, 0)
    assert [int(w[0]) for w in r] == list(KAT[0][2])
    r2 = P.event_noise_words(3, 0, 1)
    assert all(int(a[0]) != int(b[0]) for a, b in zip(r, r2))


@pytest.mark.gpu
def test_event_noise_matches_words():
    from x_amd.ops import functional as F
    n, seed, off, h = 200_003, 0x1234_5678_9ABC_DEF0, 7, 1.5
    xy = torch.zeros(n, 2, device="cuda")
    xs, xa = F.event_noise(xy, seed, off, h)
    ws, wa = P.event_noise(np.zeros((n, 2)), seed, off, h)
    # with xy = 0 the uniform part is the words' top 24 bits exactly
    np.testing.assert_array_equal(xs.cpu().numpy().astype(np.float64), ws)
    np.testing.assert_allclose(xa.cpu().numpy(), wa, rtol=0, atol=2e-5 * h * 6)


@pytest.mark.gpu
def test_event_noise_statistics_and_flags():
    from x_amd.ops import functional as F
    n, h = 1_000_000, 0.7
    g = torch.Generator().manual_seed(0)
    xy = (torch.rand(n, 2, generator=g) * 600).round().cuda()
    xs, xa = F.event_noise(xy, 42, 3, h)
    u = (xs - xy).cpu().double().numpy()
    z = ((xa - xs) / h).cpu().double().numpy()
    assert u.min() >= -0.5 and u.max() <= 0.5        # [-1/2, 1/2) before xy + u rounds to fp32
    assert abs(u.mean()) < 2e-3 and abs(u.var() - 1 / 12) < 1e-3
    assert abs(z.mean()) < 3e-3 and abs(z.var() - 1) < 6e-3
    assert abs(np.mean(np.abs(z) <= 1) - 0.682689) < 3e-3
    assert abs(np.corrcoef(z[:, 0], z[:, 1])[0, 1]) < 5e-3 and abs(np.corrcoef(u[:, 0], z[:, 0])[0, 1]) < 5e-3
    xs2, xa2 = F.event_noise(xy, 42, 3, h)
    assert torch.equal(xs, xs2) and torch.equal(xa, xa2)
    xs3, _ = F.event_noise(xy, 42, 4, h)
    assert not torch.equal(xs, xs3)
    xs4, xa4 = F.event_noise(xy, 42, 3, h, dequantize=False, smooth=False)
    assert torch.equal(xs4, xy) and xa4 is None
