"""CPU: the block-sum bound behind the prefill GEMM's exactness, on the adversarial blocks the GPU test uses.

The MFMA kernel forms each 256-value block sum as two chains of four matrix-core steps (sub-blocks 0, 2, 4, 6 and
1, 3, 5, 7) and adds the two chain totals once in fp32. These checks pin, with the checker, that (1) on the adversarial
rows every block sum is odd and above 2^24 -- so a rounding anywhere would show --, (2) each chain's absolute sum stays
below 2^24 (exact), (3) the two-chain value equals ggml's float(int32 bsum) on every block, and (4) one fp32 chain over
all eight steps (what the kernel did before) rounds differently on some of them.
"""
import numpy as np

from oracle import oracle as orc
from tests._helpers import adversarial_iq2, iq2_grid, sign_pattern_even

K = 2048


def _blocks(w, x):
    """per block: the exact integer chain sums (even / odd sub-blocks) and the eight per-step sums, from the bytes"""
    grid = iq2_grid()
    nb = K // 256
    rows = w.reshape(-1, nb, 66)
    q, d, _ = orc.quantize_q8k(x[None, :])
    q = q[0].astype(np.int64)
    out = []
    for r in range(rows.shape[0]):
        per_row = []
        for j in range(nb):
            words = rows[r, j, 2:].copy().view("<u4").astype(np.int64)
            sub = np.zeros(8, np.int64)
            steps = np.zeros(8, np.int64)
            for ib in range(8):
                a0, a1 = int(words[2 * ib]), int(words[2 * ib + 1])
                ls = 2 * (a1 >> 28) + 1
                for l in range(4):
                    g = grid[(a0 >> (8 * l)) & 255]
                    sb = (a1 >> (7 * l)) & 127
                    sgn = np.array([-1 if (sb >> k) & 1 else 1 for k in range(7)] + [1], np.int64)
                    if bin(sb).count("1") % 2:
                        sgn[7] = -1
                    v = int(np.dot(g * sgn, q[j * 256 + ib * 32 + l * 8: j * 256 + ib * 32 + l * 8 + 8])) * ls
                    sub[ib] += v
                    steps[4 * (ib % 2) + l] += v     # step t = 4 (ib % 2) + l covers group l of sub-blocks of ib's parity
            per_row.append((sub, steps))
        out.append(per_row)
    return out


def test_adversarial_blocks_and_two_chain_bound():
    xs = sign_pattern_even(K, 3)
    w, sums = adversarial_iq2(4, K, 11, xs)
    blocks = _blocks(w, xs)
    two_to_24 = 1 << 24
    diff_single = 0
    for per_row in blocks:
        for sub, steps in per_row:
            bsum = int(sub.sum())
            assert abs(bsum) > two_to_24 and bsum % 2 == 1
            even, odd = int(sub[0::2].sum()), int(sub[1::2].sum())
            assert max(abs(even), abs(odd)) < two_to_24 and np.abs(sub).sum() <= 25_574_752
            two_chain = np.float32(np.float32(even) + np.float32(odd))   # each chain exact, one rounding
            assert two_chain == np.float32(bsum)                          # = ggml's (float) of the int32 sum
            acc = np.float32(0)                                           # one chain: a rounding per step above 2^24
            for t in range(8):
                acc = np.float32(float(acc) + float(steps[t]))
            diff_single += int(acc != np.float32(bsum))
    assert diff_single > 0


def test_adversarial_dot_matches_exact_integer_path():
    """The checker's vec_dot on those rows equals the fp32 fold of float(exact bsum) block by block."""
    xs = sign_pattern_even(K, 3)
    w, _ = adversarial_iq2(3, K, 12, xs)
    q, d, _ = orc.quantize_q8k(xs[None, :])
    blocks = _blocks(w, xs)
    rows = w.reshape(3, -1)
    for r in range(3):
        acc = np.float32(0)
        for j, (sub, _) in enumerate(blocks[r]):
            dw = np.frombuffer(rows[r, j * 66:j * 66 + 2].tobytes(), np.float16)[0].astype(np.float32)
            acc = np.float32(acc + np.float32(dw * d[0, j]) * np.float32(int(sub.sum())))
        want = np.float32(acc * np.float32(0.125))
        got = orc.vec_dot(rows[r], q[0], d[0])
        assert np.float32(got).view(np.uint32) == want.view(np.uint32)
