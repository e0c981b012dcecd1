"""CPU: pin the checker (oracle/) against what the mathematics and the format definitions fix.

The reference holds no golden vectors or kernel tests for this path (its only tests are UI tests, loki/tests.py), so
each oracle function is pinned by closed forms, invariants, brute force on small inputs, constructed known answers,
the committed golden fixtures (tests/golden/) and -- for the codebook -- a digest of the reference's table.
Each test names the mistake it would catch.
"""
import hashlib
import math
import os

import numpy as np
import pytest

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GRID_SHA256 = "05826b5d3e472a3a78f196be62ac78acf81df0f909626e12ab9fa2a5d490dd54"   # src/iq2_tables.cuh:4-69, 2048 LE bytes


def grid_table():
    src = open(os.path.join(os.path.dirname(GOLDEN), "..", "loki_amd", "csrc", "iq2xxs_grid.inc")).read()
    vals = [int(t.rstrip("ul,"), 16) for t in src.replace(",", " ").split() if t.startswith("0x")]
    return np.array(vals, dtype=np.uint64)


# ---------------------------------------------------------------- codebook and signs
def test_grid_matches_reference_digest():
    g = grid_table()
    assert g.size == 256
    assert hashlib.sha256(g.astype("<u8").tobytes()).hexdigest() == GRID_SHA256   # a transcription slip changes it


def test_grid_invariants():
    g = grid_table()
    b = g.astype("<u8").view(np.uint8).reshape(256, 8)
    assert set(np.unique(b).tolist()) == {0x08, 0x19, 0x2B}      # magnitudes 8, 25, 43 only
    assert np.unique(g).size == 256                                # 256 distinct codewords
    assert int(g[0]) == 0x0808080808080808                         # index 0 = all-8 (the qs = 0 known answer below)


def block(d16, qs):
    return np.frombuffer(np.uint16(d16).tobytes() + np.asarray(qs, np.uint16).tobytes(), np.uint8)


# ---------------------------------------------------------------- IQ2_XXS dequantisation
def test_dequant_all_zero_qs_gives_d():
    # qs = 0: codeword 0 (all 8), no signs, scale nibble 0 -> w = d * 0.5 * 0.25 * 8 = d exactly
    for d in (1.0, 0.0019989013671875, 6.103515625e-05, 5.960464477539063e-08):
        h = orc.fp32_to_fp16(d)[0]
        w = orc.dequant_iq2xxs(block(h, np.zeros(32)), 256)[0]
        assert np.all(w == np.float32(orc.fp16_to_fp32([h])[0])), d


def test_dequant_scale_nibble_and_signs():
    qs = np.zeros(32, np.uint16)
    qs[3] = 0xF000                       # sub-block 0: a1 top nibble 15 -> scale (0.5 + 15) * 0.25 = 3.875
    qs[2] = 0x0001                       # sign index of group 0 = 1 -> weight 0 negated, parity flips weight 7
    w = orc.dequant_iq2xxs(block(0x3C00, qs), 256)[0]   # d = 1.0
    assert w[0] == -8 * 3.875 and w[7] == -8 * 3.875 and np.all(w[1:7] == 8 * 3.875)
    assert np.all(w[8:32] == 8 * 3.875)                  # groups 1..3 of sub-block 0: no signs
    assert np.all(w[32:] == 8 * 0.125)                   # sub-blocks 1..7: scale nibble 0


def test_dequant_matches_independent_numpy_decode():
    rng = np.random.default_rng(3)
    g = grid_table().astype("<u8").view(np.uint8).reshape(256, 8).astype(np.float64)
    raw = rng.integers(0, 256, size=(4, 66), dtype=np.uint8)
    raw[:, 1] &= 0x3F                    # keep d finite
    w = orc.dequant_iq2xxs(raw.reshape(-1), 1024).reshape(4, 256)
    for i in range(4):
        d = float(np.frombuffer(raw[i, :2].tobytes(), np.float16)[0])
        for ib in range(8):
            a0 = int.from_bytes(raw[i, 2 + 8 * ib:6 + 8 * ib].tobytes(), "little")
            a1 = int.from_bytes(raw[i, 6 + 8 * ib:10 + 8 * ib].tobytes(), "little")
            db = d * (0.5 + (a1 >> 28)) * 0.25
            for l in range(4):
                s7 = (a1 >> (7 * l)) & 127
                s8 = s7 | ((bin(s7).count("1") & 1) << 7)
                for j in range(8):
                    want = db * g[(a0 >> (8 * l)) & 255, j] * (-1 if (s8 >> j) & 1 else 1)
                    assert w[i, 32 * ib + 8 * l + j] == np.float32(want)


def test_fp16_conversion_exact_including_subnormals():
    h = np.arange(0, 65536, dtype=np.uint16)
    f = orc.fp16_to_fp32(h)
    ref = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(f[fin].view(np.uint32), ref[fin].view(np.uint32))
    back = orc.fp32_to_fp16(f[fin])
    assert np.array_equal(back, h[fin])


# ---------------------------------------------------------------- Q8_K
def test_q8k_known_answers():
    x = np.zeros((3, 256), np.float32)
    x[1, 0] = -127.0; x[1, 1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]
    x[2, 5] = 2.0; x[2, 9] = -2.0; x[2, 10] = 1.0
    q, d, bs = orc.quantize_q8k(x)
    assert d[0, 0] == 0 and not q[0].any() and not bs[0].any()                 # zero block
    assert d[1, 0] == np.float32(1.0)                                           # d = 1/iscale, iscale = -127/max = 1
    assert q[1, 0] == -127                                                      # the max-|x| element maps to -127
    assert list(q[1, 1:9]) == [0, 2, 2, 0, -2, -2, 126, -126]                   # ties to even
    assert q[2, 5] == -127 and q[2, 9] == 127 and q[2, 10] == -64              # first occurrence of |x| max wins
    assert np.array_equal(bs, q.reshape(3, 16, 16).sum(-1))


def test_q8k_invariants_random():
    rng = np.random.default_rng(5)
    x = (rng.normal(0, 1, (64, 1024)) * rng.uniform(1e-3, 1e3, (64, 1))).astype(np.float32)
    q, d, _ = orc.quantize_q8k(x)
    xb = x.reshape(64, 4, 256)
    qb = q.reshape(64, 4, 256).astype(np.float64)
    assert q.min() >= -127 and q.max() <= 127
    am = np.argmax(np.abs(xb), axis=-1)
    assert np.all(np.take_along_axis(qb, am[..., None], -1) == -127)
    err = np.abs(qb * d[..., None].astype(np.float64) - xb)
    assert np.all(err <= np.abs(d[..., None]) * (0.5 + 1e-5) + 1e-30)     # half a step


# ---------------------------------------------------------------- vec_dot
def test_vec_dot_equals_fp64_dot_of_dequantised_operands():
    rng = np.random.default_rng(7)
    for K in (256, 2048, 7168):
        raw = rng.integers(0, 256, size=(K // 256, 66), dtype=np.uint8)
        raw[:, 1] = rng.integers(0, 0x18, size=K // 256)          # fp16 d in a normal range, including subnormals
        x = rng.normal(0, 1, K).astype(np.float32)
        q, d, _ = orc.quantize_q8k(x)
        w = orc.dequant_iq2xxs(raw.reshape(-1), K)[0].astype(np.float64)
        xq = (q.astype(np.float64).reshape(-1, 256) * d.reshape(-1, 1)).reshape(-1)
        exact = float(np.dot(w, xq))
        got = orc.vec_dot(raw.reshape(-1), q, d)
        scale = float(np.dot(np.abs(w), np.abs(xq)))
        assert abs(got - exact) <= 4e-7 * K / 256 * scale + 1e-30, (K, got, exact)


def test_vec_dot_brute_force_integer_path():
    # one block, d_w = d_x = 1: the result is exactly 0.125 * sum_ib (2*nib+1) * sum g*sign*q
    rng = np.random.default_rng(11)
    g = grid_table().astype("<u8").view(np.uint8).reshape(256, 8).astype(np.int64)
    qs = rng.integers(0, 65536, size=32).astype(np.uint16)
    raw = block(0x3C00, qs)
    q = rng.integers(-127, 128, size=256).astype(np.int8)
    tot = 0
    for ib in range(8):
        a0 = int(qs[4 * ib]) | int(qs[4 * ib + 1]) << 16
        a1 = int(qs[4 * ib + 2]) | int(qs[4 * ib + 3]) << 16
        s = 0
        for l in range(4):
            s7 = (a1 >> (7 * l)) & 127
            s8 = s7 | ((bin(s7).count("1") & 1) << 7)
            for j in range(8):
                s += int(g[(a0 >> (8 * l)) & 255, j]) * int(q[32 * ib + 8 * l + j]) * (-1 if (s8 >> j) & 1 else 1)
        tot += s * (2 * (a1 >> 28) + 1)
    assert orc.vec_dot(raw, q, np.ones(1, np.float32)) == np.float32(np.float32(tot) * np.float32(0.125))


# ---------------------------------------------------------------- exp contract
def test_expf_close_to_correctly_rounded():
    rng = np.random.default_rng(13)
    x = np.concatenate([rng.uniform(-100, 88, 20000), rng.normal(0, 2, 20000)]).astype(np.float32)
    got = orc.expf(x)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= 0.5 * ulp * (1 + 1e-9))   # correctly rounded: within half an ulp
    assert orc.expf([0.0])[0] == 1.0 and orc.expf([-200.0])[0] == 0.0 and np.isinf(orc.expf([100.0])[0])


def test_sigmoid_silu_definitions():
    x = np.float32([-20, -3.5, -1, 0, 0.25, 1, 3.5, 20])
    e = orc.expf(-x)
    assert np.array_equal(orc.sigmoid(x), np.float32(1) / (np.float32(1) + e))
    assert np.array_equal(orc.silu(x), x / (np.float32(1) + e))
    s = orc.sigmoid(x).astype(np.float64)
    assert np.allclose(s, 1 / (1 + np.exp(-x.astype(np.float64))), rtol=2e-7)


# ---------------------------------------------------------------- router
def brute_router(W, b, x, n_group, topk_group, topk, scale):
    """Independent fp64 restatement (different summation order) with explicit tie rules."""
    l = (W.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    p = 1 / (1 + np.exp(-l.astype(np.float64)))
    p = p.astype(np.float32)
    c = (p + b).astype(np.float32)
    per = len(c) // n_group
    gs = []
    for g in range(n_group):
        v = sorted(c[g * per:(g + 1) * per].tolist(), reverse=True)
        gs.append(np.float32(v[0]) + np.float32(v[1]))
    order = sorted(range(n_group), key=lambda g: (-gs[g], g))[:topk_group]
    allowed = [e for e in range(len(c)) if e // per in order]
    sel = sorted(allowed, key=lambda e: (-c[e], e))[:topk]
    s = np.float32(0)
    for e in sel:
        s = np.float32(s + p[e])
    s = max(s, np.float32(6.103515625e-05))
    return np.array(sel), np.array([np.float32(np.float32(p[e] / s) * np.float32(scale)) for e in sel]), c, order


def test_router_logit_contract_close_to_exact():
    rng = np.random.default_rng(17)
    W = rng.normal(0, 0.02, (8, 7168)).astype(np.float32); x = rng.normal(0, 1, 7168).astype(np.float32)
    for e in range(8):
        exact = math.fsum(float(a) * float(b) for a, b in zip(W[e], x))
        assert abs(orc.router_logit(W[e], x) - exact) <= np.spacing(np.float32(abs(exact))) * 0.5 + 1e-12


def test_router_matches_brute_force():
    rng = np.random.default_rng(19)
    W = rng.normal(0, 0.02, (256, 7168)).astype(np.float32); b = rng.normal(0, 0.05, 256).astype(np.float32)
    x = rng.normal(0, 1, (6, 7168)).astype(np.float32)
    for rule in ((8, 4), (1, 1), (4, 2)):
        _, _, sel, wts = orc.router(W, b, x, rule[0], rule[1], 8, 2.5)
        for t in range(6):
            s_ref, w_ref, c, groups = brute_router(W, b, x[t], rule[0], rule[1], 8, 2.5)
            assert np.array_equal(sel[t], s_ref), (rule, t)
            assert np.allclose(wts[t], w_ref, rtol=1e-6)
            per = 256 // rule[0]
            assert all(e // per in groups for e in sel[t])            # inside the chosen groups
            assert np.all(np.diff(c[sel[t]]) <= 0)                     # descending biased score
            assert abs(float(wts[t].astype(np.float64).sum()) - 2.5) < 1e-5


def test_router_closed_form_one_hot():
    # x = e_0, W[e, 0] = v_e: logits are exactly v_e; ties resolve to the lower index
    W = np.zeros((256, 7168), np.float32)
    v = np.linspace(-2, 2, 256).astype(np.float32)
    v[200] = v[201] = v[255]                  # three-way tie at the top (indices 200, 201, 255)
    W[:, 0] = v
    x = np.zeros((1, 7168), np.float32); x[0, 0] = 1
    b = np.zeros(256, np.float32)
    logits, probs, sel, wts = orc.router(W, b, x, 1, 1, 8, 2.5)
    assert np.array_equal(logits[0], v)
    assert list(sel[0][:3]) == [200, 201, 255]
    assert list(sel[0][3:]) == [254, 253, 252, 251, 250]
    # grouped, 8 groups / top-1 group: group 6 (192..223) holds the two top values (200, 201) and beats group 7
    # (255 and 254), so every selection comes from group 6, best first
    _, _, sel2, _ = orc.router(W, b, x, 8, 1, 8, 2.5)
    assert list(sel2[0][:2]) == [200, 201] and all(192 <= e < 224 for e in sel2[0])


def test_router_weight_clamp():
    W = np.zeros((256, 7168), np.float32); W[:, 0] = -200.0       # every sigmoid underflows to 0
    x = np.zeros((1, 7168), np.float32); x[0, 0] = 1
    _, probs, sel, wts = orc.router(W, np.zeros(256, np.float32), x, 1, 1, 8, 2.5)
    assert np.all(probs == 0) and np.all(wts == 0) and list(sel[0]) == list(range(8))


# ---------------------------------------------------------------- dispatch
def test_dispatch_is_stable_counting_sort():
    rng = np.random.default_rng(23)
    for n in (1, 3, 64, 700):
        sel = np.stack([rng.choice(256, 8, replace=False) for _ in range(n)]).astype(np.int32)
        counts, offsets, perm = orc.dispatch(sel)
        pairs = sorted(range(n * 8), key=lambda i: (sel.ravel()[i], i))
        assert np.array_equal(perm, pairs)
        assert np.array_equal(counts, np.bincount(sel.ravel(), minlength=256))
        assert offsets[-1] == n * 8 and np.array_equal(np.diff(offsets), counts)
        assert np.array_equal(np.sort(perm), np.arange(n * 8))


def test_dispatch_rejects_out_of_range():
    with pytest.raises(ValueError):
        orc.dispatch(np.array([[0, 256]], np.int32))


# ---------------------------------------------------------------- keep-KE (engine narrow dispatch)
def _keep_brute(sel, w, ke, renorm, n_pad):
    """Pure-Python statement of eng:793-815: order the k of a row by weight descending with equal weights in k order
    (what a stable insertion sort with `w[a] > w[b]` leaves), keep the first ke, sum them in that order in fp32 and
    multiply each by f = renorm / sum when the sum exceeds 1e-6; pad rows copy row 0's kept experts at weight 0."""
    n, topk = sel.shape
    so = np.empty((n, ke), np.int32); wo = np.empty((n, ke), np.float32)
    for i in range(n):
        order = sorted(range(topk), key=lambda k: (-float(w[i, k]), k))[:ke]
        so[i] = sel[i, order]; wo[i] = w[i, order]
        if renorm > 0:
            sw = np.float32(0)
            for k in range(ke):
                sw = np.float32(sw + wo[i, k])
            if sw > np.float32(1e-6):
                f = np.float32(np.float32(renorm) / sw)
                wo[i] = (wo[i] * f).astype(np.float32)
    for i in range(max(n_pad, 1), n):
        so[i] = so[0]; wo[i] = 0
    return so, wo


@pytest.mark.parametrize("ke,renorm", [(2, 2.5), (1, 2.5), (4, 2.5), (2, 0.0), (8, 2.5)])
def test_keep_experts_matches_brute_force(ke, renorm):
    rng = np.random.default_rng(ke * 7 + int(renorm))
    n = 40
    sel = np.stack([rng.choice(256, 8, replace=False) for _ in range(n)]).astype(np.int32)
    w = rng.uniform(0.01, 0.8, (n, 8)).astype(np.float32)
    w[3, :] = 0.3125                          # all weights equal: k order
    w[4, [1, 6]] = w[4].max() + 0.25          # a tie at the top: the lower k first
    w[5, :] = 0.0                             # sum below the threshold: no rescale
    for n_pad in (n, 33):
        so, wo = orc.keep_experts(sel, w, ke, renorm, n_pad)
        bs, bw = _keep_brute(sel, w, ke, renorm, n_pad)
        assert np.array_equal(so, bs)
        assert np.array_equal(wo.view(np.uint32), bw.view(np.uint32))
    so, wo = orc.keep_experts(sel, w, ke, renorm)
    assert list(so[4][:2]) == [sel[4, 1], sel[4, 6]][:min(ke, 2)] or ke == 1 and so[4][0] == sel[4, 1]
    assert np.all(wo[5] == 0)
    if renorm > 0:   # the kept weights carry the routed scale (within the fp32 rounding of the rescale)
        rows = [i for i in range(n) if i != 5]
        assert np.allclose(wo[rows].sum(axis=1, dtype=np.float64), renorm, rtol=ke * 2e-7)


def test_keep_experts_is_top_ke_set():
    """Invariant independent of the ordering rule: the kept weights are the ke largest of the row."""
    rng = np.random.default_rng(5)
    sel = np.tile(np.arange(8, dtype=np.int32), (200, 1))
    w = rng.uniform(0, 1, (200, 8)).astype(np.float32)
    so, wo = orc.keep_experts(sel, w, 3, 0.0)
    assert np.array_equal(np.sort(wo, axis=1)[:, ::-1], -np.sort(-w, axis=1)[:, :3])
    assert np.all(np.diff(wo, axis=1) <= 0)


def _share_brute(sel, w, ke, renorm, n_pad):
    """--share-experts (src/server_core_fused.cpp:798-806) stated over Python sets: rank each row's picks by weight
    (descending, ties in k order); own = the top min(2, ke); U = the union of the own experts of the real rows; rows in
    order take their own, then (weight order) picks whose expert U holds, then the rest, which join U."""
    n, topk = sel.shape
    so = np.zeros((n, ke), np.int32); wo = np.zeros((n, ke), np.float32)
    rank = [sorted(range(topk), key=lambda k, i=i: (-float(w[i, k]), k)) for i in range(n)]
    own = min(2, ke)
    U = {int(sel[i, k]) for i in range(min(n, n_pad)) for k in rank[i][:own]}
    for i in range(n):
        rest = rank[i][own:]
        shared = [k for k in rest if int(sel[i, k]) in U]
        take = rank[i][:own] + shared[:ke - own]
        fill = [k for k in rest if k not in take][:ke - len(take)]
        U |= {int(sel[i, k]) for k in fill}
        take += fill
        so[i] = sel[i, take]; wo[i] = w[i, take]
        if renorm > 0:
            sw = np.float32(0)
            for k in range(ke):
                sw = np.float32(sw + wo[i, k])
            if sw > np.float32(1e-6):
                wo[i] = (wo[i] * np.float32(np.float32(renorm) / sw)).astype(np.float32)
    for i in range(max(n_pad, 1), n):
        so[i] = so[0]; wo[i] = 0
    return so, wo


@pytest.mark.parametrize("ke,renorm", [(3, 2.5), (2, 2.5), (4, 0.0), (1, 2.5), (8, 2.5)])
def test_keep_experts_share_matches_brute_force(ke, renorm):
    """The --share-experts rule against the set formulation, on rows drawing from a small expert pool (so rows share
    experts) with ties and a pad tail; share=False and n = 1 reduce to the plain keep."""
    rng = np.random.default_rng(100 + ke)
    n = 24
    sel = np.stack([rng.choice(20, 8, replace=False) for _ in range(n)]).astype(np.int32)
    w = rng.uniform(0.01, 0.8, (n, 8)).astype(np.float32)
    w[2, :] = 0.25                            # all equal: k order
    w[7, [0, 5]] = w[7].max() + 0.1           # a tie at the top
    for n_pad in (n, 17):
        so, wo = orc.keep_experts(sel, w, ke, renorm, n_pad, share=True)
        bs, bw = _share_brute(sel, w, ke, renorm, n_pad)
        assert np.array_equal(so, bs)
        assert np.array_equal(wo.view(np.uint32), bw.view(np.uint32))
    a = orc.keep_experts(sel, w, ke, renorm, share=False); b = orc.keep_experts(sel, w, ke, renorm)
    assert all(np.array_equal(x.view(np.uint32), y.view(np.uint32)) for x, y in zip(a, b))
    a = orc.keep_experts(sel[:1], w[:1], ke, renorm, share=True); b = orc.keep_experts(sel[:1], w[:1], ke, renorm)
    assert all(np.array_equal(x.view(np.uint32), y.view(np.uint32)) for x, y in zip(a, b))


def test_keep_experts_share_known_answer():
    """Three rows worked by hand (ke = 3, weights descending in k so rank = k): own tops {10, 11}, {20, 21}, {30, 31},
    U = {10, 11, 20, 21, 30, 31}. Row 0 = 10 11 | 12 20 ..: 12 is not in U, 20 is -> 10 11 20. Row 1 = 20 21 | 40 41
    ..: none in U -> the next by weight, 40, which joins U. Row 2 = 30 31 | 41 40 ..: 40 is in U now, 41 is not -> 30
    31 40 (the plain keep would take 41)."""
    sel = np.array([[10, 11, 12, 20, 13, 14, 15, 16], [20, 21, 40, 41, 42, 43, 44, 45], [30, 31, 41, 40, 46, 47, 48, 49]], np.int32)
    w = np.tile(np.linspace(0.8, 0.1, 8, dtype=np.float32), (3, 1))
    so, wo = orc.keep_experts(sel, w, 3, 0.0, share=True)
    assert so.tolist() == [[10, 11, 20], [20, 21, 40], [30, 31, 40]]
    want_w = np.array([[w[0, 0], w[0, 1], w[0, 3]], [w[1, 0], w[1, 1], w[1, 2]], [w[2, 0], w[2, 1], w[2, 3]]], np.float32)
    assert np.array_equal(wo, want_w)
    plain, _ = orc.keep_experts(sel, w, 3, 0.0)
    assert plain.tolist() == [[10, 11, 12], [20, 21, 40], [30, 31, 41]]


# ---------------------------------------------------------------- whole block
def _rand_experts(rng, n_exp, E, H):
    def mat(rows, cols):
        raw = rng.integers(0, 256, size=(rows, cols // 256, 66), dtype=np.uint8)
        d = np.abs(rng.normal(0, 0.002, (rows, cols // 256))).astype(np.float16)
        raw[:, :, :2] = d.view(np.uint8).reshape(rows, cols // 256, 2)
        return raw.reshape(-1)
    return [mat(H, E) for _ in range(n_exp)], [mat(H, E) for _ in range(n_exp)], [mat(E, H) for _ in range(n_exp)]


def test_block_against_fp64_composition():
    """mul_mat_id mapping, swiglu order (silu(gate) * up), down, k-ordered combine and the shared add, against an
    fp64 evaluation of the same quantised operands (catches swapped gate/up, a dropped term, wrong weights)."""
    rng = np.random.default_rng(29)
    E, H, n_exp, n = 1024, 512, 16, 3
    gate, up, down = _rand_experts(rng, n_exp, E, H)
    sg, su, sd = [m[0] for m in _rand_experts(rng, 1, E, H)]
    W = rng.normal(0, 0.02, (n_exp, E)).astype(np.float32); b = rng.normal(0, 0.01, n_exp).astype(np.float32)
    x = rng.normal(0, 1, (n, E)).astype(np.float32)
    out = orc.moe_forward(x, W, b, gate, up, down, sg, su, sd, n_group=4, topk_group=2, topk=4, H=H, want=("g", "u", "o", "sh"))
    deq = lambda m, r, c: orc.dequant_iq2xxs(m, c).reshape(r, c).astype(np.float64)
    for t in range(n):
        q, d, _ = orc.quantize_q8k(x[t]); xq = (q.reshape(-1, 256) * d.reshape(-1, 1).astype(np.float64)).reshape(-1)
        y = np.zeros(E)
        for k in range(4):
            e = out["sel"][t, k]
            g = deq(gate[e], H, E) @ xq; u = deq(up[e], H, E) @ xq
            assert np.allclose(out["g"][t * 4 + k], g, rtol=1e-4, atol=1e-4 * np.abs(g).max())
            assert np.allclose(out["u"][t * 4 + k], u, rtol=1e-4, atol=1e-4 * np.abs(u).max())
            h = orc.silu(out["g"][t * 4 + k]) * out["u"][t * 4 + k]          # swiglu: silu(gate) * up, fp32
            qh, dh, _ = orc.quantize_q8k(h); hq = (qh.reshape(-1, 256) * dh.reshape(-1, 1).astype(np.float64)).reshape(-1)
            o = deq(down[e], E, H) @ hq
            assert np.allclose(out["o"][t * 4 + k], o, rtol=1e-4, atol=1e-4 * np.abs(o).max())
            y += out["wts"][t, k] * out["o"][t * 4 + k]
        gs = deq(sg, H, E) @ xq; us = deq(su, H, E) @ xq
        hs = gs / (1 + np.exp(-gs)) * us
        qh, dh, _ = orc.quantize_q8k(hs.astype(np.float32)); hq = (qh.reshape(-1, 256) * dh.reshape(-1, 1).astype(np.float64)).reshape(-1)
        sh = deq(sd, E, H) @ hq
        mx = np.abs(out["sh"][t] - sh).max() / np.abs(sh).max()
        assert mx < 2e-2, mx           # h rounded in fp64 here: a Q8 step may flip, so this one is loose
        y = y + out["sh"][t]
        assert np.allclose(out["y"][t], y, rtol=1e-5, atol=1e-5 * np.abs(y).max())


def test_rmsnorm_matches_definition():
    rng = np.random.default_rng(31)
    x = rng.normal(0, 3, (4, 7168)).astype(np.float32)
    y = orc.rmsnorm(x)
    ref = x / np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=1, keepdims=True) + 1e-6)
    assert np.allclose(y, ref, rtol=1e-6)


# ---------------------------------------------------------------- committed golden fixtures
@pytest.mark.parametrize("name", ["block_small", "decode_full"])
def test_golden_fixtures(name):
    """The checker against the committed vectors of tests/golden (weights regenerated from their seed)."""
    from tests.golden import gen
    z = np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)
    c = {k: int(z[k]) for k in ("seed", "n_exp", "E", "H", "n", "n_group", "topk_group", "topk")}
    W, b, gate, up, down, sh = gen.layer(c["seed"], c["n_exp"], c["E"], c["H"])
    x = gen.uniform(c["seed"], 3, (c["n"], c["E"]), 2.0)
    assert np.array_equal(x, z["x"])
    out = orc.moe_forward(x, W, b, gate, up, down, *sh, n_group=c["n_group"], topk_group=c["topk_group"],
                          topk=c["topk"], H=c["H"])
    assert np.array_equal(out["sel"], z["sel"])
    assert np.array_equal(out["wts"].view(np.uint32), z["wts"].view(np.uint32))
    assert np.array_equal(out["y"].view(np.uint32), z["y"].view(np.uint32))
    q, d, _ = orc.quantize_q8k(x)
    assert np.array_equal(q, z["xq"]) and np.array_equal(d.view(np.uint32), z["xd"].view(np.uint32))
