"""NumPy Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC 2011) and the event-noise transform of atl_event_noise,
used to check the device noise word for word.  Test helper, not part of the product."""
import numpy as np

M0, M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
W0, W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
MASK = np.uint64(0xFFFFFFFF)


def philox4x32_10(c0, c1, c2, c3, k0, k1):
    """Arrays of counters (uint32) and a key -> the four output words (uint32 arrays)."""
    x = [np.asarray(c, dtype=np.uint32).copy() for c in (c0, c1, c2, c3)]
    k0, k1 = np.uint32(k0), np.uint32(k1)
    with np.errstate(over="ignore"):
        for _ in range(10):
            p0 = M0 * x[0].astype(np.uint64)
            p1 = M1 * x[2].astype(np.uint64)
            hi0, lo0 = (p0 >> np.uint64(32)).astype(np.uint32), (p0 & MASK).astype(np.uint32)
            hi1, lo1 = (p1 >> np.uint64(32)).astype(np.uint32), (p1 & MASK).astype(np.uint32)
            x = [hi1 ^ x[1] ^ k0, lo1, hi0 ^ x[3] ^ k1, lo0]
            k0 = np.uint32(k0 + W0)
            k1 = np.uint32(k1 + W1)
    return x


def event_noise_words(n, seed, offset):
    """The four words event i (0 <= i < n) draws under (seed, offset)."""
    i = np.arange(n, dtype=np.uint64)
    return philox4x32_10((i & MASK).astype(np.uint32), (i >> np.uint64(32)).astype(np.uint32),
                         np.full(n, offset & 0xFFFFFFFF, np.uint32), np.full(n, (offset >> 32) & 0xFFFFFFFF, np.uint32),
                         seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF)


def event_noise(xy, seed, offset, h, dequantize=True):
    """(xs, xa) as atl_event_noise forms them, in float64 (the device rounds to fp32)."""
    r = event_noise_words(xy.shape[0], seed, offset)
    f = lambda w: (w >> np.uint32(8)).astype(np.float64) / 16777216.0
    xs = xy.astype(np.float64).copy()
    if dequantize:
        xs[:, 0] += f(r[0]) - 0.5
        xs[:, 1] += f(r[1]) - 0.5
    u1 = ((r[2] >> np.uint32(8)).astype(np.float64) + 1.0) / 16777216.0
    u2 = f(r[3])
    rad = np.sqrt(-2.0 * np.log(u1))
    xa = np.stack([xs[:, 0] + h * rad * np.cos(2 * np.pi * u2), xs[:, 1] + h * rad * np.sin(2 * np.pi * u2)], 1)
    return xs, xa
