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
