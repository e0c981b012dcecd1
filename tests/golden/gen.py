"""Deterministic test data from integer hashing only (splitmix64's output function), so any numpy on any machine
regenerates the same bytes. Used by the golden fixtures (make_golden.py) and the tests that check against them."""
import numpy as np

M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def mix64(z):
    z = np.asarray(z, np.uint64)
    with np.errstate(over="ignore"):
        z = z + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def words(seed, stream, count):
    key = mix64(np.uint64(seed) * np.uint64(1000003) + np.uint64(stream))
    with np.errstate(over="ignore"):
        return mix64(key + np.arange(count, dtype=np.uint64))


def uniform(seed, stream, shape, scale=1.0):
    """floats uniform in [-scale, scale): 24 random bits -> exact float, one rounding when scaled"""
    n = int(np.prod(shape))
    w = (words(seed, stream, n) >> np.uint64(40)).astype(np.int64).astype(np.float32)
    v = w * np.float32(2.0 ** -23) - np.float32(1.0)
    return (v * np.float32(scale)).astype(np.float32).reshape(shape)


def iq2_matrix(seed, stream, rows, cols):
    """ggml-layout IQ2_XXS matrix bytes: qs from hash words, fp16 d bits drawn from [0x0100, 0x1C00)
    (subnormals up to ~0.004)."""
    nb = rows * (cols // 256)
    w = words(seed, stream, nb * 9).reshape(nb, 9)
    blk = np.empty((nb, 66), np.uint8)
    blk[:, 2:] = w[:, :8].copy().view(np.uint8).reshape(nb, 64)
    d = (np.uint64(0x0100) + w[:, 8] % np.uint64(0x1B00)).astype(np.uint16)
    blk[:, :2] = d.view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1)


# K-quant block bytes and the offsets of their fp16 d / dmin fields (FL_* format codes)
KQ_LAYOUT = {5: (84, 80, 82), 6: (110, 108, None), 3: (176, 0, 2), 1: (210, 208, None)}


def kq_matrix(seed, stream, fmt, rows, cols):
    """ggml-layout K-quant matrix bytes (fmt = FL_Q2K 5, FL_Q3K 6, FL_Q5K 3, FL_Q6K 1): quant and scale bytes from
    hash words, fp16 d (and dmin) bits drawn from [0x0C00, 0x1C00) (about 6e-5 .. 4e-3)."""
    bs, od, om = KQ_LAYOUT[fmt]
    nb = rows * (cols // 256)
    nw = (bs + 7) // 8 + 1
    w = words(seed, stream, nb * nw).reshape(nb, nw)
    blk = w[:, :nw - 1].copy().view(np.uint8).reshape(nb, -1)[:, :bs].copy()
    dd = (np.uint64(0x0C00) + w[:, nw - 1] % np.uint64(0x1000)).astype(np.uint16)
    blk[:, od:od + 2] = dd.view(np.uint8).reshape(nb, 2)
    if om is not None:
        dm = (np.uint64(0x0C00) + (w[:, nw - 1] >> np.uint64(32)) % np.uint64(0x1000)).astype(np.uint16)
        blk[:, om:om + 2] = dm.view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1)


def layer(seed, n_exp, E, H, bias_scale=0.01):
    W = uniform(seed, 1, (n_exp, E), 0.035)
    b = uniform(seed, 2, (n_exp,), bias_scale)
    gate = [iq2_matrix(seed, 10 + 3 * e, H, E) for e in range(n_exp)]
    up = [iq2_matrix(seed, 11 + 3 * e, H, E) for e in range(n_exp)]
    down = [iq2_matrix(seed, 12 + 3 * e, E, H) for e in range(n_exp)]
    sh = (iq2_matrix(seed, 5, H, E), iq2_matrix(seed, 6, H, E), iq2_matrix(seed, 7, E, H))
    return W, b, gate, up, down, sh
