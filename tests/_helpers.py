"""Shared test helpers: synthetic layers on the device and host copies of what the CPU checker needs."""
import numpy as np

E, H, NEXP = 7168, 2048, 256


def iq2_bytes(rows, cols):
    return rows * (cols // 256) * 66


def make_layer(ctx, seed, bias_sigma=0.01, hot=None, hot_bias=0.5):
    from loki_amd import MoeLayerWeights
    return MoeLayerWeights.synthetic(ctx, seed, bias_sigma=bias_sigma, hot=hot, hot_bias=hot_bias)


def make_x(ctx, n, seed, stream=100):
    import torch
    x = torch.empty((n, E), dtype=torch.float32, device="cuda")
    ctx.synth_normal(x, seed, stream, 0.0, 1.0)
    ctx.sync()
    return x


def host_matrix(ctx, tiled, rows, cols):
    """One tiled matrix (device) -> ggml layout bytes (host numpy), through the library's unpack."""
    g = ctx.unpack(tiled, rows, cols, 1)
    ctx.sync()
    return g.cpu().numpy()


def host_layer(ctx, layer, experts):
    """Router weights and the given experts' matrices in ggml layout on the host (dicts expert -> bytes)."""
    gate, up, down = {}, {}, {}
    for e in sorted(set(int(v) for v in experts)):
        gate[e] = host_matrix(ctx, layer.expert_slice("gate", e), H, E)
        up[e] = host_matrix(ctx, layer.expert_slice("up", e), H, E)
        down[e] = host_matrix(ctx, layer.expert_slice("down", e), E, H)
    sh = (host_matrix(ctx, layer.sh_gate, H, E), host_matrix(ctx, layer.sh_up, H, E), host_matrix(ctx, layer.sh_down, E, H))
    return layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy(), gate, up, down, sh


def rel_errors(y, ref):
    y = np.asarray(y, np.float64); ref = np.asarray(ref, np.float64)
    mx = np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30)
    l2 = np.linalg.norm(y - ref) / max(np.linalg.norm(ref), 1e-30)
    return mx, l2


def numpy_pack_tiled(ggml_bytes, rows, cols):
    """Independent restatement of the tiled layout: 64-row groups, per block four 16-byte chunks of 64 rows each, then
    the fp16 d of (row group, block, row); sign words re-packed so byte l = 7 sign bits of group l | scale bit l << 7."""
    nb = cols // 256
    blk = np.asarray(ggml_bytes, np.uint8).reshape(rows, nb, 66)
    d = blk[:, :, :2].reshape(rows // 64, 64, nb, 2).transpose(0, 2, 1, 3)
    w = blk[:, :, 2:].copy().view("<u4").reshape(rows, nb, 16).astype(np.uint64)
    a1 = w[:, :, 1::2]
    t = np.zeros_like(a1)
    for l in range(4):
        t |= (((a1 >> np.uint64(7 * l)) & np.uint64(127)) | (((a1 >> np.uint64(28 + l)) & np.uint64(1)) << np.uint64(7))) << np.uint64(8 * l)
    w[:, :, 1::2] = t
    qs = w.astype("<u4").view(np.uint8).reshape(rows // 64, 64, nb, 4, 16).transpose(0, 2, 3, 1, 4)
    return np.concatenate([qs.reshape(-1), d.reshape(-1)])


def iq2_grid():
    """The IQ2_XXS codebook as 256 x 8 bytes (the library's table source)."""
    import os
    import re
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "loki_amd", "csrc", "iq2xxs_grid.inc")
    vals = [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]+", open(path).read())]
    return np.array([[(v >> (8 * k)) & 255 for k in range(8)] for v in vals], np.int64)


def adversarial_iq2(rows, cols, seed, sign_pattern):
    """IQ2_XXS rows (ggml layout) whose block sums against Q8_K(sign_pattern) reach the format's extreme: every scale
    nibble 15, every group an entry of the codebook's largest byte sums (>= 168, at most 203), and the stored signs equal
    to sign_pattern's (x = +-1 with an even count of minus signs per 8-group), so every product of a block has the same
    sign and |q| = 127. Each block's entry sum is made odd, so |bsum| = 3937 * sum is odd and above 2^24.
    Returns the bytes and the per-(row, block) sum of the chosen entries' bytes."""
    grid = iq2_grid()
    esum = grid.sum(axis=1)
    big = np.nonzero(esum >= 168)[0]
    big_odd, big_even = big[esum[big] % 2 == 1], big[esum[big] % 2 == 0]
    rng = np.random.default_rng(seed)
    nb = cols // 256
    # sign words: 7 stored bits per group from the pattern (bit k = element k negative), scale nibble 15
    neg = (np.asarray(sign_pattern, np.float32).reshape(nb, 8, 4, 8)[..., :7] < 0).astype(np.int64)
    bits = (neg << np.arange(7, dtype=np.int64)).sum(axis=-1)                      # [nb][8][4]
    a1 = ((bits << (7 * np.arange(4, dtype=np.int64))).sum(axis=-1) | (15 << 28)).astype(np.uint32)   # [nb][8]
    idx = rng.choice(big, size=(rows, nb, 32))
    tot = esum[idx].sum(axis=2)
    fix = tot % 2 == 0                                                             # one odd-sum entry flips the parity
    first = idx[..., 0]
    first_odd = esum[first] % 2 == 1
    repl = np.where(first_odd, rng.choice(big_even, size=first.shape), rng.choice(big_odd, size=first.shape))
    idx[..., 0] = np.where(fix, repl, first)
    sums = esum[idx].sum(axis=2)
    a0 = (idx.reshape(rows, nb, 8, 4).astype(np.uint32) << (8 * np.arange(4, dtype=np.uint32))).sum(axis=-1).astype(np.uint32)
    words = np.empty((rows, nb, 8, 2), np.uint32)
    words[..., 0] = a0
    words[..., 1] = a1[None, :, :]
    out = np.empty((rows, nb, 66), np.uint8)
    d = np.full((rows, nb), np.float16(0.00097)).view(np.uint8).reshape(rows, nb, 2)
    out[:, :, :2] = d
    out[:, :, 2:] = words.reshape(rows, nb, 16).view(np.uint8)
    return out.reshape(-1), sums


def sign_pattern_even(cols, seed):
    """+-1 values with an even number of minus signs in every group of 8 (representable by IQ2_XXS's 7 sign bits)."""
    rng = np.random.default_rng(seed)
    s = np.where(rng.integers(0, 2, cols) == 1, -1.0, 1.0).reshape(-1, 8)
    odd = (s < 0).sum(axis=1) % 2 == 1
    s[odd, 7] *= -1.0
    return s.reshape(-1).astype(np.float32)
