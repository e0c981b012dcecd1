"""CPU: the K-quant checker (oracle/kquant_oracle.c) pinned by hand-made known answers, an independent numpy decoder
of each ggml block layout, and fp64 brute force for the dot products.

The reference runs the routed down projection in Q2_K / Q3_K and the shared expert in Q5_K / Q5_K / Q6_K
(src/fused_layer.cu:102-158, 203-254). ggml is not vendored, so the layouts are restated from their published
definitions; the checks below fail on a misplaced bit, a wrong offset or a dropped min term."""
import numpy as np
import pytest

from oracle import oracle as orc

FMTS = [orc.Q2K, orc.Q3K, orc.Q5K, orc.Q6K]
NAMES = {orc.Q2K: "q2_K", orc.Q3K: "q3_K", orc.Q5K: "q5_K", orc.Q6K: "q6_K"}


def half(v):
    return np.frombuffer(np.float16(v).tobytes(), np.uint8)


def random_blocks(fmt, nblk, rng):
    """random bytes with finite fp16 d / dmin fields"""
    bb = orc.kq_block_bytes(fmt)
    b = rng.integers(0, 256, (nblk, bb), dtype=np.uint8)
    for i in range(nblk):
        d = half(rng.uniform(0.001, 0.05)); m = half(rng.uniform(0.001, 0.05))
        if fmt == orc.Q2K: b[i, 80:82] = d; b[i, 82:84] = m
        elif fmt == orc.Q3K: b[i, 108:110] = d
        elif fmt == orc.Q5K: b[i, 0:2] = d; b[i, 2:4] = m
        else: b[i, 208:210] = d
    return b


# ---------------------------------------------------------------- an independent decoder (numpy, per bit plane)
def np_decode(fmt, blk):
    """one block -> (q int [256], scale per element, min per element, d, dmin) from the ggml struct definitions"""
    f16 = lambda lo: float(np.frombuffer(blk[lo:lo + 2].tobytes(), np.float16)[0])
    e = np.arange(256)
    if fmt == orc.Q2K:                      # scales[16] qs[64] d dmin; element 128 n + 32 s + l = bits 2s of qs[32 n + l]
        n, s, l = e // 128, (e % 128) // 32, e % 32
        q = (blk[16 + 32 * n + l].astype(int) >> (2 * s)) & 3
        sc = blk[:16][e // 16].astype(int)
        return q, sc & 15, sc >> 4, f16(80), f16(82)
    if fmt == orc.Q3K:                      # hmask[32] qs[64] scales[12] d; hmask bit 4 n + s clear -> -4
        n, s, l = e // 128, (e % 128) // 32, e % 32
        q = ((blk[32 + 32 * n + l].astype(int) >> (2 * s)) & 3) - np.where((blk[l].astype(int) >> (4 * n + s)) & 1, 0, 4)
        raw = blk[96:108].astype(int)
        j = e // 16
        low = np.where(j < 8, raw[j % 8] & 15, raw[j % 8] >> 4)
        high = (raw[8 + j % 4] >> (2 * (j // 4))) & 3
        return q, (low | (high << 4)) - 32, np.zeros(256, int), f16(108), 0.0
    if fmt == orc.Q5K:                      # d dmin scales[12] qh[32] qs[128]; element 64 c + 32 h + l
        c, hh, l = e // 64, (e % 64) // 32, e % 32
        q = ((blk[48 + 32 * c + l].astype(int) >> (4 * hh)) & 15) + 16 * ((blk[16 + l].astype(int) >> (2 * c + hh)) & 1)
        raw = blk[4:16].astype(int)
        j = e // 32
        sc = np.where(j < 4, raw[j % 4] & 63, (raw[8 + j % 4] & 15) | ((raw[j % 4] >> 6) << 4))
        mn = np.where(j < 4, raw[4 + j % 4] & 63, (raw[8 + j % 4] >> 4) | ((raw[4 + j % 4] >> 6) << 4))
        return q, sc, mn, f16(0), f16(2)
    # Q6_K: ql[128] qh[64] scales[16] d; element 128 n + 32 p + l: nibble p // 2 of ql[64 n + 32 (p % 2) + l],
    # 2 high bits p of qh[32 n + l]
    n, p, l = e // 128, (e % 128) // 32, e % 32
    lo = (blk[64 * n + 32 * (p % 2) + l].astype(int) >> (4 * (p // 2))) & 15
    hi = (blk[128 + 32 * n + l].astype(int) >> (2 * p)) & 3
    sc = blk[192:208].view(np.int8).astype(int)[e // 16]
    return (lo | (hi << 4)) - 32, sc, np.zeros(256, int), f16(208), 0.0


@pytest.mark.parametrize("fmt", FMTS, ids=lambda f: NAMES[f])
def test_dequant_matches_independent_decoder(fmt):
    rng = np.random.default_rng(11 + fmt)
    b = random_blocks(fmt, 6, rng)
    y = orc.dequant_kq(fmt, b.reshape(1, -1), 6 * 256)[0]
    for i in range(6):
        q, sc, mn, d, dmin = np_decode(fmt, b[i])
        want = (np.float32(d) * sc.astype(np.float32)) * q.astype(np.float32)
        if fmt in (orc.Q2K, orc.Q5K):
            want = want - np.float32(dmin) * mn.astype(np.float32)
        assert np.array_equal(y[256 * i:256 * (i + 1)].view(np.uint32), want.astype(np.float32).view(np.uint32)), i


def test_known_answers():
    # Q6_K: zero quants are -32; ql[0] = 0x21, qh[0] = 0b11100100 set elements 0, 32, 64, 96
    b = np.zeros(210, np.uint8); b[192:208] = 1; b[208:210] = half(1.0)
    b[0] = 0x21; b[128] = 0b11100100
    y = orc.dequant_kq(orc.Q6K, b, 256)[0]
    assert (y[0], y[32], y[64], y[96], y[1]) == (-31.0, -16.0, 2.0, 16.0, -32.0)
    # Q2_K: scale 3, min 5, d 2, dmin 1: zero quants give -5; qs[0] = 0b11100100 -> elements 0, 32, 64, 96 = 0..3
    b = np.zeros(84, np.uint8); b[:16] = 0x53; b[80:82] = half(2.0); b[82:84] = half(1.0); b[16] = 0b11100100
    y = orc.dequant_kq(orc.Q2K, b, 256)[0]
    assert (y[0], y[32], y[64], y[96], y[5]) == (-5.0, 1.0, 7.0, 13.0, -5.0)
    # Q3_K: every 6-bit scale 33 (low nibbles 1, high pairs 0b10) -> 1; hmask bit set: q = qs bits, clear: q - 4
    b = np.zeros(110, np.uint8); b[96:104] = 0x11; b[104:108] = 0xAA; b[108:110] = half(1.0)
    b[:32] = 0xFF; b[32] = 0b11100100
    y = orc.dequant_kq(orc.Q3K, b, 256)[0]
    assert (y[0], y[32], y[64], y[96], y[1]) == (0.0, 1.0, 2.0, 3.0, 0.0)
    b[0] = 0xFE   # element 0's high bit clear
    assert orc.dequant_kq(orc.Q3K, b, 256)[0][0] == -4.0
    # Q5_K: scales 2, mins 1, d = dmin = 1 -> 2 q - 1; qs[0] = 0x35, qh[0] bit 0 -> element 0 = 21, element 32 = 3
    b = np.zeros(176, np.uint8); b[0:2] = half(1.0); b[2:4] = half(1.0); b[4:8] = 2; b[8:12] = 1; b[12:16] = 0x12
    b[16] = 1; b[48] = 0x35
    y = orc.dequant_kq(orc.Q5K, b, 256)[0]
    assert (y[0], y[32], y[1], y[255]) == (41.0, 5.0, -1.0, -1.0)


@pytest.mark.parametrize("fmt", FMTS, ids=lambda f: NAMES[f])
def test_dot_matches_fp64_brute_force(fmt):
    rng = np.random.default_rng(23 + fmt)
    K = 2048
    w = random_blocks(fmt, K // 256, rng).reshape(-1)
    x = rng.normal(0, 1, K).astype(np.float32)
    q, d, bs = orc.quantize_q8k(x)
    got = orc.vec_dot_kq(fmt, w, q, d, bs)
    wd = orc.dequant_kq(fmt, w, K)[0].astype(np.float64)
    xd = q.astype(np.float64) * np.repeat(d.astype(np.float64), 256)
    ref = float(wd @ xd)
    scale = float(np.abs(wd * xd).sum())
    assert abs(got - ref) <= 1e-5 * scale, (got, ref)
    # the bsums the min terms use are the 16-value sums of q
    assert np.array_equal(bs, q.reshape(-1, 16).astype(np.int64).sum(1).astype(np.int16))
    # matvec = per-row dots
    w2 = random_blocks(fmt, 3 * K // 256, rng).reshape(3, -1)
    y = orc.matvec_kq(fmt, w2, 3, K, q.reshape(1, -1), d.reshape(1, -1), bs.reshape(1, -1))
    assert np.array_equal(y[0].view(np.uint32), np.array([orc.vec_dot_kq(fmt, w2[r], q, d, bs) for r in range(3)], np.float32).view(np.uint32))


def test_expert_composition_per_format():
    """or_moe_experts_fmt: IQ2_XXS everywhere equals the original composition bit for bit; with K-quant formats each
    matrix is read in its own format and row stride: the shared expert equals matvec_kq(gate / up) -> silu * u -> Q8_K
    -> matvec_kq(down), and the routed outputs use the down format (E, H scaled down to keep the check quick)."""
    from tests.golden import gen
    E, H, n, topk, n_exp = 512, 256, 2, 2, 4
    rng = np.random.default_rng(7)
    x = rng.normal(0, 1, (n, E)).astype(np.float32)
    sel = np.array([[0, 2], [3, 0]], np.int32); wts = np.array([[0.7, 0.3], [0.6, 0.4]], np.float32)
    gate = [gen.iq2_matrix(3, e, H, E) for e in range(n_exp)]
    up = [gen.iq2_matrix(4, e, H, E) for e in range(n_exp)]
    down_iq2 = [gen.iq2_matrix(5, e, E, H) for e in range(n_exp)]
    sh_iq2 = (gen.iq2_matrix(6, 0, H, E), gen.iq2_matrix(6, 1, H, E), gen.iq2_matrix(6, 2, E, H))
    a = orc.moe_experts(x, sel, wts, gate, up, down_iq2, *sh_iq2, H=H, n_exp=n_exp, want=("o", "sh"))
    b = orc.moe_experts(x, sel, wts, gate, up, down_iq2, *sh_iq2, H=H, n_exp=n_exp, want=("o", "sh"), fmts=(4, 4, 4, 4))
    assert all(np.array_equal(a[k].view(np.uint32), b[k].view(np.uint32)) for k in ("y", "o", "sh"))
    # K-quants: Q3_K routed down, Q5_K / Q5_K / Q6_K shared
    down = [gen.kq_matrix(7, e, orc.Q3K, E, H) for e in range(n_exp)]
    ksh = (gen.kq_matrix(8, 0, orc.Q5K, H, E), gen.kq_matrix(8, 1, orc.Q5K, H, E), gen.kq_matrix(8, 2, orc.Q6K, E, H))
    r = orc.moe_experts(x, sel, wts, gate, up, down, *ksh, H=H, n_exp=n_exp, want=("o", "sh"), fmts=(orc.Q3K, orc.Q5K, orc.Q5K, orc.Q6K))
    q, d, bs = orc.quantize_q8k(x)
    g = orc.matvec_kq(orc.Q5K, ksh[0], H, E, q, d, bs); u = orc.matvec_kq(orc.Q5K, ksh[1], H, E, q, d, bs)
    h = (orc.silu(g).reshape(g.shape) * u).astype(np.float32)
    hq, hd, hb = orc.quantize_q8k(h)
    sh = orc.matvec_kq(orc.Q6K, ksh[2], E, H, hq, hd, hb)
    assert np.array_equal(r["sh"].view(np.uint32), sh.view(np.uint32))
    # a routed output: token 1, k = 0 (expert 3) -> its h from the IQ2_XXS gate/up (the IQ2 run's o of the same pair
    # differs only by the down format), through the Q3_K down
    o_iq2 = b["o"].reshape(n, topk, E)[1, 0]
    o_q3 = r["o"].reshape(n, topk, E)[1, 0]
    assert not np.array_equal(o_iq2, o_q3)
    gi = orc.matvec(gate[3], H, E, q[1], d[1]); ui = orc.matvec(up[3], H, E, q[1], d[1])
    hi = (orc.silu(gi) * ui).astype(np.float32)
    hiq, hid, hib = orc.quantize_q8k(hi.reshape(1, -1))
    assert np.array_equal(o_q3.view(np.uint32), orc.matvec_kq(orc.Q3K, down[3], E, H, hiq, hid, hib)[0].view(np.uint32))
