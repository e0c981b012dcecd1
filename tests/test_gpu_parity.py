"""GPU parity: every stage of the HIP MoE block against the CPU checker (oracle/), through the C ABI.

The kernels reproduce the checker's arithmetic contract, so most comparisons are bit-exact: Q8_K, router logits,
probabilities, selections, weights, dispatch, gate/up/h, down outputs and the block output. The task's tolerance
(max relative 1e-2, L2 relative 2e-3) is asserted as well for the block output.
"""
import numpy as np
import pytest

from tests._helpers import (E, H, NEXP, adversarial_iq2, host_layer, iq2_bytes, make_layer, make_x, numpy_pack_tiled,
                            rel_errors, sign_pattern_even)
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

MAX_REL, L2_REL = 1e-2, 2e-3   # the block output tolerance: max relative error 1e-2, relative L2 error 2e-3


@pytest.fixture(scope="module")
def layer(ctx):
    return make_layer(ctx, seed=1234)


def test_exp_contract_bitwise(ctx):
    import torch
    rng = np.random.default_rng(0)
    xs = np.concatenate([rng.normal(0, 3, 20000), rng.uniform(-120, 100, 5000), [0.0, -0.0, 1e-30, -1e-30, 88.7, 89.0, -103.9, -104.0, -150.0, 200.0]]).astype(np.float32)
    x = torch.from_numpy(xs).cuda()
    for which, ref in ((0, orc.expf), (1, orc.sigmoid), (2, orc.silu)):
        y = ctx.probe_exp(x, which); ctx.sync()
        got = y.cpu().numpy()
        want = ref(xs)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), "exp contract mismatch (probe %d)" % which


def test_q8k_bitwise(ctx):
    import torch
    rng = np.random.default_rng(1)
    x = rng.normal(0, 1, (6, 2 * E)).astype(np.float32)
    x[0, :256] = 0.0                                    # zero block -> d = 0, q = 0
    x[1, :256] = 0.25; x[1, 7] = -3.0; x[1, 9] = 3.0    # first occurrence of max |x| is negative
    mid = np.zeros(256, np.float32); mid[0] = -127.0    # iscale = 1: exact half-way products round to even
    mid[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]
    x[2, 256:512] = mid
    x[3, :] *= 1e-30                                    # tiny magnitudes
    x[4, 512:768] = 7.0                                 # all equal
    q, d = ctx.quant_q8k(torch.from_numpy(x).cuda()); ctx.sync()
    qo, do, _ = orc.quantize_q8k(x)
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(d.cpu().numpy().view(np.uint32), do.view(np.uint32))


def test_pack_layout(ctx):
    import torch
    rows, cols = 64, 2048
    g = torch.empty(iq2_bytes(rows, cols), dtype=torch.uint8, device="cuda")
    ctx.synth_iq2(g, rows, cols, 1, 0, seed=7, mat0=3)
    t = ctx.pack(g, rows, cols, 1)
    back = ctx.unpack(t, rows, cols, 1); ctx.sync()
    gh = g.cpu().numpy()
    assert np.array_equal(t.cpu().numpy(), numpy_pack_tiled(gh, rows, cols))
    assert np.array_equal(back.cpu().numpy(), gh)
    # the generator writes the same block contents in either layout
    t2 = torch.empty_like(g)
    ctx.synth_iq2(t2, rows, cols, 1, 1, seed=7, mat0=3); ctx.sync()
    assert np.array_equal(t2.cpu().numpy(), t.cpu().numpy())


# n covers every logit kernel: the logits and the selection in one launch (n <= 8; 5 gives one wave two tokens), one
# workgroup per expert (k_router_wg, n < 40), LDS-staged 32 x 32 tiles with the chunks split over 16 workgroups and
# joined (40..2048) and whole (above 2048: the ragged-expert test), with ragged last tiles
@pytest.mark.parametrize("n,rule", [(1, (8, 4)), (5, (8, 4)), (8, (8, 4)), (21, (8, 4)), (39, (8, 4)), (40, (8, 4)), (77, (8, 4)),
                                    (200, (8, 4)), (300, (8, 4)), (1037, (8, 4)), (8, (1, 1))])
def test_router_bitwise(ctx, layer, n, rule):
    x = make_x(ctx, n, seed=10 + n)
    ctx.set_routing(rule[0], rule[1], 8, 2.5)
    try:
        logits, probs, sel, w = ctx.route(layer.gate_inp, layer.probs_b, x)
        ctx.sync()
    finally:
        ctx.set_routing()
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    lo, po, so, wo = orc.router(W, b, x.cpu().numpy(), rule[0], rule[1], 8, 2.5)
    assert np.array_equal(logits.cpu().numpy().view(np.uint32), lo.view(np.uint32))
    assert np.array_equal(probs.cpu().numpy().view(np.uint32), po.view(np.uint32))
    assert np.array_equal(sel.cpu().numpy(), so)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), wo.view(np.uint32))


# a layer whose expert count is not a multiple of the 32-expert tiles (48 = 8 groups of 6): the last expert tile is
# ragged in every logit kernel, the K-split tiles (96, 1030) and the whole tiles (2050) included
@pytest.mark.parametrize("n", [9, 96, 1030, 2050])
def test_router_bitwise_ragged_experts(ctx, n):
    import torch
    g = torch.Generator(device="cpu").manual_seed(500 + n)
    W = (torch.randn(48, E, generator=g) * 0.02).cuda()
    b = (torch.randn(48, generator=g) * 0.05).cuda()
    x = make_x(ctx, n, seed=600 + n)
    logits, probs, sel, w = ctx.route(W, b, x)
    ctx.sync()
    lo, po, so, wo = orc.router(W.cpu().numpy(), b.cpu().numpy(), x.cpu().numpy(), 8, 4, 8, 2.5)
    assert np.array_equal(logits.cpu().numpy().view(np.uint32), lo.view(np.uint32))
    assert np.array_equal(probs.cpu().numpy().view(np.uint32), po.view(np.uint32))
    assert np.array_equal(sel.cpu().numpy(), so)
    assert np.array_equal(w.cpu().numpy().view(np.uint32), wo.view(np.uint32))


# n * 8 pairs: one workgroup (rounds of 1024 in turn) up to 4096 pairs, the rounds as workgroups of their own above
# (129, 513: a ragged last round)
@pytest.mark.parametrize("n,skew", [(1, 0), (8, 0), (129, 0), (512, 0), (513, 1), (2048, 1), (2048, 2)])
def test_dispatch_bitwise(ctx, n, skew):
    import torch
    rng = np.random.default_rng(n + 17 * skew)
    if skew == 0:
        sel = np.stack([rng.choice(NEXP, 8, replace=False) for _ in range(n)]).astype(np.int32)
    elif skew == 1:   # a few hot experts in almost every row
        hot = rng.choice(NEXP, 16, replace=False)
        sel = np.stack([np.concatenate([rng.choice(hot, 4, replace=False), rng.choice(np.setdiff1d(np.arange(NEXP), hot), 4, replace=False)]) for _ in range(n)]).astype(np.int32)
    else:             # every row the same 8 experts
        sel = np.tile(np.arange(8, dtype=np.int32) * 31, (n, 1))
    counts, offsets, perm, inv, act, nact = ctx.dispatch(torch.from_numpy(sel).cuda())
    ctx.sync()
    co, oo, po = orc.dispatch(sel)
    assert np.array_equal(counts.cpu().numpy(), co)
    assert np.array_equal(offsets.cpu().numpy(), oo)
    assert np.array_equal(perm.cpu().numpy(), po)
    invo = np.empty_like(po); invo[po] = np.arange(po.size, dtype=np.int32)
    assert np.array_equal(inv.cpu().numpy(), invo)
    used = np.nonzero(co)[0]
    assert int(nact.cpu().numpy()[0]) == used.size
    assert np.array_equal(act.cpu().numpy()[:used.size], used)


def _block_vs_oracle(ctx, layer, x, tokens, capture=True):
    """Run the device block on all rows of x, compare the rows `tokens` (independent per token) with the checker."""
    ctx.set_debug(capture)
    y = ctx.moe_layer(layer, x)
    ctx.sync()
    dbg = ctx.debug()
    ctx.set_debug(False)
    xs = x.cpu().numpy()[tokens]
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    _, _, so, _ = orc.router(W, b, xs)
    _, _, gate, up, down, sh = host_layer(ctx, layer, so.ravel())
    ref = orc.moe_forward(xs, W, b, gate, up, down, *sh, want=("g", "u", "o", "sh"))
    return y.cpu().numpy()[tokens], ref, dbg


@pytest.mark.parametrize("n", [1, 8])
def test_block_decode_bitwise(ctx, layer, n):
    x = make_x(ctx, n, seed=200 + n)
    tokens = np.arange(n)
    with ctx.using_fused(0):   # the per-pass kernels keep their intermediates in plain buffers
        y, ref, dbg = _block_vs_oracle(ctx, layer, x, tokens)
        mx, l2 = rel_errors(y, ref["y"])
        assert mx <= MAX_REL and l2 <= L2_REL, (mx, l2)
        # intermediates per (token, k) pair: the device keeps them per dispatch slot, inv maps pair -> slot
        P = n * 8
        inv = ctx.d2h(dbg.inv, (P,), np.int32)
        g = ctx.d2h(dbg.g, (P + n, H), np.float32); u = ctx.d2h(dbg.u, (P + n, H), np.float32)
        o = ctx.d2h(dbg.o, (P + n, E), np.float32)
        assert np.array_equal(g[inv].view(np.uint32), ref["g"].view(np.uint32))
        assert np.array_equal(u[inv].view(np.uint32), ref["u"].view(np.uint32))
        assert np.array_equal(o[inv].view(np.uint32), ref["o"].view(np.uint32))
        assert np.array_equal(o[P:].view(np.uint32), ref["sh"].view(np.uint32))
        assert np.array_equal(y.view(np.uint32), ref["y"].view(np.uint32)), "block output not bit-identical (max rel %.3g)" % mx
    # the single-launch decode block on the same rows: regular launch (mode 2, the library default and what bench.py
    # times) and cooperative launch (mode 1); routing outputs too
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    _, _, so, wo = orc.router(W, b, x.cpu().numpy())
    for mode in (2, 1):
        with ctx.using_fused(mode):
            yf = ctx.moe_layer(layer, x)
            ctx.sync()
            assert ctx.debug().fused == 1
            st = _routing_state(ctx, n)
        assert np.array_equal(yf.cpu().numpy()[tokens].view(np.uint32), ref["y"].view(np.uint32)), mode
        assert np.array_equal(st["sel"], so.ravel()), mode
        assert np.array_equal(st["wts"].view(np.uint32), wo.ravel().view(np.uint32)), mode


def test_block_prefill512_rows(ctx):
    layer = make_layer(ctx, seed=4321, bias_sigma=0.05)
    x = make_x(ctx, 512, seed=512)
    tokens = np.array([0, 1, 77, 255, 256, 400, 510, 511])
    y, ref, _ = _block_vs_oracle(ctx, layer, x, tokens, capture=False)
    mx, l2 = rel_errors(y, ref["y"])
    assert mx <= MAX_REL and l2 <= L2_REL, (mx, l2)
    assert np.array_equal(y.view(np.uint32), ref["y"].view(np.uint32)), "prefill rows not bit-identical (max rel %.3g)" % mx


def _prefill_state(ctx, layer, x, mfma):
    """y and the per-slot intermediates of one batch through the MFMA grouped GEMMs or the per-pass kernels."""
    n = x.shape[0]
    ctx.set_prefill_mfma(mfma)
    ctx.set_debug(True)
    try:
        y = ctx.moe_layer(layer, x).clone()
        ctx.sync()
        d = ctx.debug()
        P = d.P
        out = {"y": y.cpu().numpy(), "h": ctx.d2h(d.h, (P + n, H), np.float32), "o": ctx.d2h(d.o, (P + n, E), np.float32),
               "g": ctx.d2h(d.g, (P + n, H), np.float32), "u": ctx.d2h(d.u, (P + n, H), np.float32),
               "hd": ctx.d2h(d.hd, (P + n, H // 256), np.float32), "hq": ctx.d2h(d.hq, (P + n, H), np.int8)}
    finally:
        ctx.set_debug(False)
        ctx.set_prefill_mfma(True)
    return out


def test_combine_unaligned_output(ctx):
    """The k-ordered combine's 4-wide kernel needs 16-byte aligned rows; an output 4 bytes off takes the one-column
    kernel, with the same arithmetic: y bit-identical to the aligned call (prefill-40, plain and normed with the
    residual; the inputs stay aligned, as the other kernels read them 16 bytes at a time)."""
    import torch
    n = 40
    layer = make_layer(ctx, seed=950, bias_sigma=0.05)
    x = make_x(ctx, n, seed=951)
    off = lambda: torch.empty(n * E + 1, dtype=torch.float32, device="cuda")[1:].view(n, E)
    ref = ctx.moe_layer(layer, x).cpu().numpy()
    y = off()
    got = ctx.moe_layer(layer, x, y).cpu().numpy()
    assert y.data_ptr() % 16 == 4
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    refn = ctx.moe_layer_normed(layer, x, residual=True).cpu().numpy()
    gotn = ctx.moe_layer_normed(layer, x, y=off(), residual=True).cpu().numpy()
    assert np.array_equal(gotn.view(np.uint32), refn.view(np.uint32))


def test_combine_row_loops(ctx):
    """The k-ordered combine kernels loop over token rows beyond their grid's y extent (65535 rows); with the extent
    capped at 7 (fl_set_debug bit 1) the loops run at prefill-40: y bit-identical to the uncapped call, for an aligned
    output (the 4-wide kernel) and one 4 bytes off (the one-column kernel)."""
    import torch
    n = 40
    layer = make_layer(ctx, seed=952, bias_sigma=0.05)
    x = make_x(ctx, n, seed=953)
    ref = ctx.moe_layer(layer, x).cpu().numpy()
    y1 = torch.empty(n * E + 1, dtype=torch.float32, device="cuda")[1:].view(n, E)
    ctx.set_debug(False, small_grids=True)
    try:
        got = ctx.moe_layer(layer, x).cpu().numpy()
        got1 = ctx.moe_layer(layer, x, y1).cpu().numpy()
        ctx.sync()
    finally:
        ctx.set_debug(False)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(got1.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("n,hot", [(9, False), (40, False), (512, False), (2048, True)])
def test_prefill_mfma_matches_per_pass(ctx, n, hot):
    """The grouped GEMMs on the matrix cores reproduce the per-pass mat-vec kernels bit for bit: gate/up outputs, h and
    its Q8_K, the down outputs and y (columns of 1..32 slots, the shared expert's full columns, hot experts with many
    columns)."""
    hot_ids = list(range(3, 256, 16)) if hot else None
    layer = make_layer(ctx, seed=900 + n, bias_sigma=0.05, hot=hot_ids)
    x = make_x(ctx, n, seed=40 + n)
    ref = _prefill_state(ctx, layer, x, False)
    got = _prefill_state(ctx, layer, x, True)
    for k in ref:
        assert np.array_equal(got[k].view(np.uint8), ref[k].view(np.uint8)), k


def test_block_deterministic(ctx, layer):
    x = make_x(ctx, 8, seed=99)
    y1 = ctx.moe_layer(layer, x).clone()
    y2 = ctx.moe_layer(layer, x)
    ctx.sync()
    assert np.array_equal(y1.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32))


def _routing_state(ctx, n):
    """Routing outputs of the last fl_moe_layer call, copied to the host."""
    dbg = ctx.debug()
    P = n * 8
    out = {
        "sel": ctx.d2h(dbg.sel, (P,), np.int32), "wts": ctx.d2h(dbg.wts, (P,), np.float32),
        "perm": ctx.d2h(dbg.perm, (P,), np.int32), "inv": ctx.d2h(dbg.inv, (P,), np.int32),
        "nact": ctx.d2h(dbg.nact, (1,), np.int32), "counts": ctx.d2h(dbg.counts, (NEXP,), np.int32),
        "offsets": ctx.d2h(dbg.offsets, (NEXP + 1,), np.int32),
        "xq": ctx.d2h(dbg.xq, (n, E), np.int8), "xd": ctx.d2h(dbg.xd, (n, E // 256), np.float32),
    }
    out["act"] = ctx.d2h(dbg.act, (int(out["nact"][0]),), np.int32)
    return out


@pytest.mark.parametrize("mode", [2, 1])
@pytest.mark.parametrize("n", [1, 2, 5, 8])
def test_fused_decode_matches_per_pass(ctx, layer, n, mode):
    """The single-launch decode block (regular or cooperative launch) and the per-pass kernels give bit-identical
    outputs and routing."""
    x = make_x(ctx, n, seed=300 + n)
    with ctx.using_fused(0):
        y_ref = ctx.moe_layer(layer, x).clone()
        ctx.sync()
        ref = _routing_state(ctx, n)
    with ctx.using_fused(mode):
        y = ctx.moe_layer(layer, x)
        ctx.sync()
        assert ctx.debug().fused == 1
        got = _routing_state(ctx, n)
    for k in ref:
        assert np.array_equal(np.asarray(got[k]).view(np.uint8), np.asarray(ref[k]).view(np.uint8)), k
    assert np.array_equal(y.cpu().numpy().view(np.uint32), y_ref.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("mode", [2, 1])
def test_fused_decode_repeated_launches(ctx, layer, mode):
    """Epoch flags and self-resetting counters: a sequence of launches with changing batch sizes stays exact, both
    back to back without a host wait in between and with one after every launch."""
    xs = {n: make_x(ctx, n, seed=400 + n) for n in (1, 3, 8)}
    want = {}
    with ctx.using_fused(0):
        for n, x in xs.items():
            want[n] = ctx.moe_layer(layer, x).cpu().numpy()
    order = (1, 8, 3, 1, 1, 8, 3, 8)
    with ctx.using_fused(mode):
        for n in order:
            y = ctx.moe_layer(layer, xs[n])
            ctx.sync()
            assert np.array_equal(y.cpu().numpy().view(np.uint32), want[n].view(np.uint32)), n
        ys = [ctx.moe_layer(layer, xs[n]) for n in order]
        ctx.sync()
    for n, y in zip(order, ys):
        assert np.array_equal(y.cpu().numpy().view(np.uint32), want[n].view(np.uint32)), n


def test_rmsnorm_matches_checker(ctx):
    """The device RMSNorm (fp64 sum of fp32 squares, fp32 mean, 1/sqrtf) against the checker's sequential sum: the
    sums differ only in fp64 rounding, which the fp32 mean almost never keeps."""
    import torch
    rng = np.random.default_rng(77)
    x = rng.normal(0, 2, (16, E)).astype(np.float32)
    x[3] *= 1e-3; x[5] *= 40.0; x[7, :] = 0.0
    y = ctx.rmsnorm(torch.from_numpy(x).cuda())
    ctx.sync()
    ref = orc.rmsnorm(x)
    yg = y.cpu().numpy()
    ulps = np.abs(yg.view(np.int32).astype(np.int64) - ref.view(np.int32).astype(np.int64))
    assert ulps.max() <= 1, ulps.max()
    assert (ulps != 0).mean() < 1e-3


def test_stack_chain(ctx):
    """configs[3] on three independently seeded layers: x_{L+1} = RMSNorm(y_L), the norm fused into the next layer's
    block (fl_moe_layer_normed). Each layer's device output is bit-identical to the checker on that layer's input
    (RMSNorm(y_{L-1}) from the separate device norm, which the fused one reproduces), and the device chain ends where
    the checker's own chain (run from x_0 on the CPU) ends, within the task's tolerance."""
    import torch
    nl = 3
    layers = [make_layer(ctx, seed=5000 + 1000 * L) for L in range(nl)]
    x0 = make_x(ctx, 1, seed=88)
    xin, outs = [], []
    prev = None
    for L in layers:
        if prev is None:
            xin.append(x0.cpu().numpy())
            y = ctx.moe_layer(L, x0)
        else:
            xin.append(ctx.rmsnorm(prev).cpu().numpy())
            y = ctx.moe_layer_normed(L, prev)
        outs.append(y.cpu().numpy())
        prev = y
    ctx.sync()
    xc = x0.cpu().numpy()
    for L, layer in enumerate(layers):
        W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
        _, _, so, _ = orc.router(W, b, xin[L])
        _, _, gate, up, down, sh = host_layer(ctx, layer, so.ravel())
        ref = orc.moe_forward(xin[L], W, b, gate, up, down, *sh)
        assert np.array_equal(outs[L].view(np.uint32), ref["y"].view(np.uint32)), "layer %d" % L
        # the checker's own chain
        _, _, sc, _ = orc.router(W, b, xc)
        _, _, gate, up, down, sh = host_layer(ctx, layer, sc.ravel())
        yc = orc.moe_forward(xc, W, b, gate, up, down, *sh)["y"]
        mx, l2 = rel_errors(outs[L], yc)
        assert mx <= MAX_REL and l2 <= L2_REL, (L, mx, l2)
        xc = orc.rmsnorm(yc)
    del layers
    torch.cuda.empty_cache()


@pytest.mark.parametrize("n", [1, 8, 40])
@pytest.mark.parametrize("weighted", [False, True])
def test_prenorm_matches_separate_norm(ctx, layer, n, weighted):
    """fl_moe_layer_normed (the norm inside the decode block for n <= 8, a k_rmsnorm pass before the per-pass path
    above) is bit-identical to fl_rmsnorm_dev followed by fl_moe_layer."""
    import torch
    h = make_x(ctx, n, seed=300 + n) * 3.0
    w = None
    if weighted:
        w = torch.empty(E, dtype=torch.float32, device="cuda")
        ctx.synth_normal(w, 41, 5, 1.0, 0.1)
    y1 = ctx.moe_layer_normed(layer, h, w, 1e-6)
    fused = ctx.debug().fused
    y2 = ctx.moe_layer(layer, ctx.rmsnorm(h, w, 1e-6))
    ctx.sync()
    assert fused == (1 if n <= 8 else 0)
    assert np.array_equal(y1.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32))
    # the residual variant adds h once more: (moe + shared) + h
    y4 = ctx.moe_layer_normed(layer, h, w, 1e-6, residual=True)
    ctx.sync()
    ref4 = (y1.cpu().numpy() + h.cpu().numpy()).astype(np.float32)
    assert np.array_equal(y4.cpu().numpy().view(np.uint32), ref4.view(np.uint32))
    if n <= 8:   # the per-pass kernels take the same normalised input, with and without the residual
        with ctx.using_fused(0):
            y3 = ctx.moe_layer_normed(layer, h, w, 1e-6)
            y5 = ctx.moe_layer_normed(layer, h, w, 1e-6, residual=True)
            ctx.sync()
            assert ctx.debug().fused == 0
        assert np.array_equal(y3.cpu().numpy().view(np.uint32), y2.cpu().numpy().view(np.uint32))
        assert np.array_equal(y5.cpu().numpy().view(np.uint32), ref4.view(np.uint32))


@pytest.mark.parametrize("n", [1, 8])
def test_residual_reference_rule(ctx, layer, n):
    """The reference's ungrouped routing rule (one group: the decode block's selection does not take it, so the
    per-pass kernels run): the residual variant is (moe + shared) + h bit for bit, and moe + shared equals the checker."""
    h = make_x(ctx, n, seed=620 + n) * 2.0
    ctx.set_routing(1, 1, 8, 2.5)
    try:
        y0 = ctx.moe_layer_normed(layer, h)
        y1 = ctx.moe_layer_normed(layer, h, residual=True)
        xn = ctx.rmsnorm(h)
        ctx.sync()
        assert ctx.debug().fused == 0
    finally:
        ctx.set_routing()
    hn = h.cpu().numpy()
    ref = (y0.cpu().numpy() + hn).astype(np.float32)
    assert np.array_equal(y1.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    xs = xn.cpu().numpy()
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    _, _, so, _ = orc.router(W, b, xs, 1, 1, 8, 2.5)
    _, _, gate, up, down, sh = host_layer(ctx, layer, so.ravel())
    want = orc.moe_forward(xs, W, b, gate, up, down, *sh, n_group=1, topk_group=1)["y"]
    assert np.array_equal(y0.cpu().numpy().view(np.uint32), want.view(np.uint32))


def _hot_ids(seed):
    """16 hot experts drawn the way bench.py draws them for prefill-2048."""
    import torch
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(NEXP, generator=g)[:16].tolist()


def _margins(probs, bias, n_group=8, topk_group=4, topk=8):
    """Smallest gap between the topk-th and the next eligible biased score, and between the kept and the next group."""
    c = (probs + bias[None, :]).astype(np.float32)
    n = c.shape[0]
    g = np.sort(c.reshape(n, n_group, -1), axis=2)[:, :, ::-1]
    gs = (g[:, :, 0] + g[:, :, 1]).astype(np.float32)
    gsort = -np.sort(-gs, axis=1)
    keep = gs >= gsort[:, topk_group - 1:topk_group]
    ce = np.where(np.repeat(keep, c.shape[1] // n_group, axis=1), c, -np.inf)
    cs = -np.sort(-ce, axis=1)
    return float(np.min(cs[:, topk - 1] - cs[:, topk])), float(np.min(gsort[:, topk_group - 1] - gsort[:, topk_group]))


@pytest.mark.parametrize("n,hot", [(512, False), (2048, True)])
def test_routing_all_rows_prefill(ctx, n, hot):
    """configs[2] (512 tokens, bias sigma 0.05) and configs[4] (2048 tokens, +0.5 on 16 hot experts): the routing of
    every row through fl_moe_layer -- selections, weights, the dispatch permutation and its inverse, counts, offsets and
    the active-expert list -- is bit-identical to the checker's router and dispatch. Output rows of the most and the least
    hot-routed tokens are bit-identical to the checker's block as well."""
    hot_ids = _hot_ids(20260101) if hot else None
    layer = make_layer(ctx, seed=20260101 + n, bias_sigma=0.05, hot=hot_ids)
    x = make_x(ctx, n, seed=7000 + n)
    y = ctx.moe_layer(layer, x)
    ctx.sync()
    st = _routing_state(ctx, n)
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    xs = x.cpu().numpy()
    _, po, so, wo = orc.router(W, b, xs)
    co, oo, pe = orc.dispatch(so)
    invo = np.empty_like(pe); invo[pe] = np.arange(pe.size, dtype=np.int32)
    used = np.nonzero(co)[0]
    assert np.array_equal(st["sel"], so.ravel())
    assert np.array_equal(st["wts"].view(np.uint32), wo.ravel().view(np.uint32))
    assert np.array_equal(st["perm"], pe)
    assert np.array_equal(st["inv"], invo)
    assert np.array_equal(st["counts"], co)
    assert np.array_equal(st["offsets"], oo)
    assert int(st["nact"][0]) == used.size and np.array_equal(st["act"], used)
    km, gm = _margins(po, b)
    print("routing margins n=%d hot=%s: top-8 gap %.3g, group gap %.3g" % (n, hot, km, gm))
    if hot:
        nhot = np.isin(so, hot_ids).sum(axis=1)
        order = np.argsort(nhot, kind="stable")
        rows = np.concatenate([order[:4], order[-4:]])
        assert nhot[order[-1]] > nhot[order[0]]
    else:
        rows = np.array([0, 3, 200, 511])
    _, _, gate, up, down, sh = host_layer(ctx, layer, so[rows].ravel())
    ref = orc.moe_forward(xs[rows], W, b, gate, up, down, *sh)
    assert np.array_equal(y.cpu().numpy()[rows].view(np.uint32), ref["y"].view(np.uint32))


def test_prefill512_every_row_vs_checker(ctx):
    """configs[2] at full size: all 512 output rows of fl_moe_layer (MFMA grouped GEMMs, columns of up to 64 slots)
    against the CPU checker's whole block (router, keep-all dispatch, Q8_K, IQ2_XXS x Q8_K products, SwiGLU, k-ordered
    combine, shared expert): bit for bit, and within the task's tolerance."""
    n = 512
    layer = make_layer(ctx, seed=20260512, bias_sigma=0.05)
    x = make_x(ctx, n, seed=9512)
    y = ctx.moe_layer(layer, x).cpu().numpy()
    ctx.sync()
    xs = x.cpu().numpy()
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    _, _, so, _ = orc.router(W, b, xs)
    _, _, gate, up, down, sh = host_layer(ctx, layer, so.ravel())
    ref = orc.moe_forward(xs, W, b, gate, up, down, *sh)
    mx, l2 = rel_errors(y, ref["y"])
    assert mx <= MAX_REL and l2 <= L2_REL, (mx, l2)
    bad = np.nonzero(~np.all(y.view(np.uint32) == ref["y"].view(np.uint32), axis=1))[0]
    assert bad.size == 0, "rows not bit-identical: %s (max rel %.3g)" % (bad[:16].tolist(), mx)


def test_prefill2048_hot_columns_vs_checker(ctx):
    """configs[4] (2048 tokens, +0.5 on 16 hot experts): the output rows whose dispatch slots fall in each hot expert's
    first, middle and last (partial) 64-slot column -- first and last slot of each -- and the tokens of the shared
    expert's first and last columns, against the CPU checker's whole block, bit for bit (at least 64 rows)."""
    n = 2048
    hot_ids = _hot_ids(20260101)
    layer = make_layer(ctx, seed=20262048, bias_sigma=0.05, hot=hot_ids)
    x = make_x(ctx, n, seed=92048)
    y = ctx.moe_layer(layer, x).cpu().numpy()
    ctx.sync()
    st = _routing_state(ctx, n)
    rows = set()
    for e in hot_ids:
        s0, s1 = int(st["offsets"][e]), int(st["offsets"][e + 1])
        ncol = (s1 - s0 + 63) // 64
        assert ncol >= 3, (e, s1 - s0)   # every hot expert spans several columns at this load
        for c in (0, ncol // 2, ncol - 1):
            first, last = s0 + 64 * c, min(s0 + 64 * c + 63, s1 - 1)
            rows.add(int(st["perm"][first]) // 8); rows.add(int(st["perm"][last]) // 8)
    rows |= {0, 1, 62, 63, n - 64, n - 63, n - 2, n - 1}   # the shared expert's first and last 64-token columns
    rows = np.array(sorted(rows))
    assert rows.size >= 64, rows.size
    xs = x.cpu().numpy()[rows]
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    _, _, so, _ = orc.router(W, b, xs)
    assert np.array_equal(so.ravel(), st["sel"].reshape(n, 8)[rows].ravel())
    _, _, gate, up, down, sh = host_layer(ctx, layer, so.ravel())
    ref = orc.moe_forward(xs, W, b, gate, up, down, *sh)
    mx, l2 = rel_errors(y[rows], ref["y"])
    assert mx <= MAX_REL and l2 <= L2_REL, (mx, l2)
    bad = rows[~np.all(y[rows].view(np.uint32) == ref["y"].view(np.uint32), axis=1)]
    assert bad.size == 0, "rows not bit-identical: %s (max rel %.3g)" % (bad[:16].tolist(), mx)


def test_stack58_routing(ctx):
    """all 58 independently seeded layers resident (~170 GB), one token chained through them with the norm
    inside each next layer's launch. Every layer's routing (selections and weights) is bit-identical to the checker's
    router on that layer's own input, RMSNorm(y_{L-1}) from the separate device norm (bit-identical to the fused one)."""
    import torch
    nl = 58
    layers = [make_layer(ctx, seed=20260301 + 1000 * L) for L in range(nl)]
    x = make_x(ctx, 1, seed=2001)
    prev = None
    kmin = np.inf
    try:
        for L, layer in enumerate(layers):
            if prev is None:
                xin = x
                y = ctx.moe_layer(layer, x)
            else:
                xin = ctx.rmsnorm(prev)
                y = ctx.moe_layer_normed(layer, prev)
            ctx.sync()
            assert ctx.debug().fused == 1
            st = _routing_state(ctx, 1)
            W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
            _, po, so, wo = orc.router(W, b, xin.cpu().numpy())
            assert np.array_equal(st["sel"], so.ravel()), L
            assert np.array_equal(st["wts"].view(np.uint32), wo.ravel().view(np.uint32)), L
            kmin = min(kmin, _margins(po, b)[0])
            prev = y
        print("stack routing: smallest top-8 gap over 58 layers %.3g" % kmin)
    finally:
        del layers
        torch.cuda.empty_cache()


@pytest.mark.parametrize("n,mode", [(1, 2), (8, 2), (8, 0), (40, 2)])
def test_keep2_layer_bitwise(ctx, layer, n, mode):
    """The reference engine's production setting: each row keeps its 2 heaviest experts, rescaled to 2.5
    (src/server_core_fused.cpp:793-813, KE = 2 at :340). fl_moe_layer with fl_set_keep(2, 2.5) -- inside the single
    decode launch (mode 2), on the per-pass kernels (mode 0) and on the MFMA grouped GEMMs (n = 40) -- gives the
    checker's router -> keep_experts -> expert block bit for bit, kept selections and weights included."""
    x = make_x(ctx, n, seed=900 + n)
    ctx.set_keep(2, 2.5)
    try:
        with ctx.using_fused(mode):
            y = ctx.moe_layer(layer, x)
            ctx.sync()
            dbg = ctx.debug()
            assert dbg.P == 2 * n and dbg.topk == 2
            assert dbg.fused == (1 if (mode and n <= 8) else 0)
            sel = ctx.d2h(dbg.sel, (n, 2), np.int32); wts = ctx.d2h(dbg.wts, (n, 2), np.float32)
    finally:
        ctx.set_keep(0)
    xs = x.cpu().numpy()
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    _, _, so, wo = orc.router(W, b, xs)
    sk, wk = orc.keep_experts(so, wo, 2, 2.5)
    assert np.array_equal(sel, sk)
    assert np.array_equal(wts.view(np.uint32), wk.view(np.uint32))
    rows = np.arange(n) if n <= 8 else np.array([0, 1, 17, 39])
    _, _, gate, up, down, sh = host_layer(ctx, layer, sk[rows].ravel())
    ref = orc.moe_experts(xs[rows], sk[rows], wk[rows], gate, up, down, *sh)
    assert np.array_equal(y.cpu().numpy()[rows].view(np.uint32), ref["y"].view(np.uint32))


@pytest.fixture(scope="module")
def hot_layer(ctx):
    """A layer whose router favours 12 experts (+0.3 bias), so the rows of a batch keep running into each other's
    experts: the case the engine's --share-experts rule is for."""
    return make_layer(ctx, seed=4242, bias_sigma=0.01, hot=[3, 40, 77, 90, 130, 131, 160, 199, 200, 222, 240, 251], hot_bias=0.3)


@pytest.mark.parametrize("n,mode", [(8, 2), (8, 1), (8, 0), (2, 2), (40, 2), (300, 2)])
def test_keep3_share_experts_bitwise(ctx, hot_layer, n, mode):
    """The production client's setting, --experts 3 --share-experts (loki/chat.py:35; src/server_core_fused.cpp:798-806):
    fl_set_keep(3, 2.5) with fl_set_share_experts -- across the rows inside the single decode launch (mode 2, and
    cooperative: mode 1), on the per-pass kernels (mode 0), and before the MFMA grouped GEMMs (n = 40, 300) -- gives the
    checker's router -> keep_experts(share) -> expert block bit for bit, kept selections and weights included. From 8
    rows the batch is one where the rule changes some row's kept experts (checked on the checker)."""
    layer = hot_layer
    x = make_x(ctx, n, seed=1900 + n)
    ctx.set_keep(3, 2.5)
    ctx.set_share_experts(True)
    try:
        with ctx.using_fused(mode):
            y = ctx.moe_layer(layer, x)
            ctx.sync()
            dbg = ctx.debug()
            assert dbg.P == 3 * n and dbg.topk == 3
            assert dbg.fused == (1 if (mode and n <= 8) else 0)
            sel = ctx.d2h(dbg.sel, (n, 3), np.int32); wts = ctx.d2h(dbg.wts, (n, 3), np.float32)
    finally:
        ctx.set_share_experts(False)
        ctx.set_keep(0)
    xs = x.cpu().numpy()
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    _, _, so, wo = orc.router(W, b, xs)
    sk, wk = orc.keep_experts(so, wo, 3, 2.5, share=True)
    plain, _ = orc.keep_experts(so, wo, 3, 2.5)
    if n >= 8:
        assert not np.array_equal(sk, plain), "the batch does not exercise the shared-expert preference"
    assert np.array_equal(sel, sk)
    assert np.array_equal(wts.view(np.uint32), wk.view(np.uint32))
    rows = np.arange(n) if n <= 8 else np.array([0, 1, 17, 39])
    _, _, gate, up, down, sh = host_layer(ctx, layer, sk[rows].ravel())
    ref = orc.moe_experts(xs[rows], sk[rows], wk[rows], gate, up, down, *sh)
    assert np.array_equal(y.cpu().numpy()[rows].view(np.uint32), ref["y"].view(np.uint32))


@pytest.mark.parametrize("n", [16, 40])
def test_prefill_mfma_exact_on_extreme_blocks(ctx, n):
    """Blocks at the format's extreme (scale nibble 15, the codebook's largest entries, signs aligned with the tokens,
    |q| = 127): every block sum of the routed gate rows is odd and above 2^24 in magnitude. The MFMA grouped GEMM
    (two exact four-step chains per block, one fp32 addition) gives the gate outputs of ggml's int32 block sums --
    bit-identical to the per-pass integer kernels and to the checker -- for a 16-slot and a 32 + 8-slot column."""
    import torch
    from loki_amd import MoeLayerWeights
    base = make_layer(ctx, seed=31337)
    chosen = [0, 1, 32, 33, 64, 65, 96, 97]          # two per group in groups 0..3: every token routes to them
    pattern = sign_pattern_even(E, 5)
    mb = iq2_bytes(H, E)
    gate = base.gate.clone()
    for i, e in enumerate(chosen):
        w, sums = adversarial_iq2(H, E, 100 + i, pattern)
        assert (sums * 3937).min() > (1 << 24)
        ctx.pack(torch.from_numpy(w).cuda(), H, E, 1, dst=gate[e * mb:(e + 1) * mb])
    W = torch.zeros_like(base.gate_inp)
    b = torch.zeros_like(base.probs_b); b[chosen] = 1.0
    layer = MoeLayerWeights(W, b, gate, base.up, base.down, base.sh_gate, base.sh_up, base.sh_down)
    scale = np.linspace(0.5, 2.0, n, dtype=np.float32)[:, None]
    x = torch.from_numpy(np.ascontiguousarray(pattern[None, :] * scale)).cuda()
    ref = _prefill_state(ctx, layer, x, False)
    got = _prefill_state(ctx, layer, x, True)
    for k in ("g", "u", "h", "hq", "hd", "o", "y"):
        assert np.array_equal(got[k].view(np.uint8), ref[k].view(np.uint8)), k
    # the checker on two tokens (their gate rows are the extreme ones)
    tokens = np.array([0, n - 1])
    xs = x.cpu().numpy()[tokens]
    Wn, bn = W.cpu().numpy(), b.cpu().numpy()
    _, _, so, _ = orc.router(Wn, bn, xs)
    assert set(so.ravel().tolist()) == set(chosen)
    _, _, gt, up, down, sh = host_layer(ctx, layer, so.ravel())
    want = orc.moe_forward(xs, Wn, bn, gt, up, down, *sh, want=("g",))
    with ctx.using_fused(0):
        ctx.set_prefill_mfma(True)
        ctx.set_debug(True)
        try:
            ctx.moe_layer(layer, x)
            ctx.sync()
            dbg = ctx.debug()
            inv = ctx.d2h(dbg.inv, (n * 8,), np.int32)
            g = ctx.d2h(dbg.g, (n * 9, H), np.float32)
        finally:
            ctx.set_debug(False)
    for i, t in enumerate(tokens):
        assert np.array_equal(g[inv[t * 8:(t + 1) * 8]].view(np.uint32), want["g"][i * 8:(i + 1) * 8].view(np.uint32)), t


@pytest.mark.parametrize("mode", [2, 1])
def test_decode1_matches_general_and_checker(ctx, layer, mode):
    """The one-token kernel organised by XCD (fl_set_decode1, default on) against the general single-launch decode
    block and the per-pass kernels: y, the Q8_K of x, logits, probabilities and every routing output bit for bit, for
    several tokens in a row; y also against the checker."""
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    for i in range(3):
        x = make_x(ctx, 1, seed=1100 + i)
        got = {}
        for name, m, d1 in (("decode1", mode, True), ("general", mode, False), ("per_pass", 0, True)):
            ctx.set_decode1(d1)
            try:
                with ctx.using_fused(m):
                    y = ctx.moe_layer(layer, x).clone()
                    ctx.sync()
                    st = _routing_state(ctx, 1)
                    dbg = ctx.debug()
                    assert dbg.kernel == {"decode1": 2, "general": 1, "per_pass": 0}[name], (name, dbg.kernel)
                    st["logits"] = ctx.d2h(dbg.logits, (NEXP,), np.float32)
                    st["probs"] = ctx.d2h(dbg.probs, (NEXP,), np.float32)
                    st["y"] = y.cpu().numpy()
                    got[name] = st
            finally:
                ctx.set_decode1(True)
        for k in got["per_pass"]:
            for other in ("decode1", "general"):
                assert np.array_equal(np.asarray(got[other][k]).view(np.uint8), np.asarray(got["per_pass"][k]).view(np.uint8)), (other, k, i)
        xs = x.cpu().numpy()
        _, _, so, _ = orc.router(W, b, xs)
        _, _, gate, up, down, sh = host_layer(ctx, layer, so.ravel())
        ref = orc.moe_forward(xs, W, b, gate, up, down, *sh)
        assert np.array_equal(got["decode1"]["y"].view(np.uint32), ref["y"].view(np.uint32)), i


@pytest.mark.parametrize("weighted", [False, True])
def test_decode1_prenorm_residual(ctx, layer, weighted):
    """fl_moe_layer_normed at n = 1 (the 58-layer stack's call) through the kernel organised by XCD: the norm inside
    the launch and the residual in its combine, bit-identical to the general decode block."""
    import torch
    h = make_x(ctx, 1, seed=1200) * 4.0
    w = None
    if weighted:
        w = torch.empty(E, dtype=torch.float32, device="cuda")
        ctx.synth_normal(w, 43, 6, 1.0, 0.1)
    out = {}
    for d1 in (True, False):
        ctx.set_decode1(d1)
        try:
            out[d1] = (ctx.moe_layer_normed(layer, h, w, 1e-6).cpu().numpy(),
                       ctx.moe_layer_normed(layer, h, w, 1e-6, residual=True).cpu().numpy())
            ctx.sync()
            assert ctx.debug().kernel == (2 if d1 else 1)
        finally:
            ctx.set_decode1(True)
    for i in range(2):
        assert np.array_equal(out[True][i].view(np.uint32), out[False][i].view(np.uint32)), i
    assert np.array_equal(out[True][1].view(np.uint32), (out[True][0] + h.cpu().numpy()).astype(np.float32).view(np.uint32))


def test_decode1_fewer_experts(ctx):
    """A 64-expert layer (8 groups of 8): workgroups 64..255 own no router expert but still run their gate/up, down and
    combine shares. The one-token kernel is bit-identical to the per-pass kernels and the checker."""
    import torch
    from loki_amd import MoeLayerWeights
    layer = MoeLayerWeights.synthetic(ctx, 6464, n_exp=64)
    x = make_x(ctx, 1, seed=6465)
    y1 = ctx.moe_layer(layer, x).clone()
    ctx.sync()
    assert ctx.debug().fused == 1 and ctx.debug().kernel == 2
    with ctx.using_fused(0):
        y0 = ctx.moe_layer(layer, x)
        ctx.sync()
    assert np.array_equal(y1.cpu().numpy().view(np.uint32), y0.cpu().numpy().view(np.uint32))
    xs = x.cpu().numpy()
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    _, _, so, _ = orc.router(W, b, xs)
    _, _, gate, up, down, sh = host_layer(ctx, layer, so.ravel())
    ref = orc.moe_forward(xs, W, b, gate, up, down, *sh)
    assert np.array_equal(y1.cpu().numpy().view(np.uint32), ref["y"].view(np.uint32))
    del layer
    torch.cuda.empty_cache()


@pytest.mark.parametrize("pattern", ["pairs", "groups", "quads"])
def test_decode1_selection_ties(ctx, pattern):
    """Exact ties in the selection, made by copying router rows and biases: "pairs" (expert e ^ 1 = e: tied keys
    inside every group), "groups" (group g ^ 1 = group g: tied group scores at every rank), "quads" (expert e % 64 for
    all e: four copies of every key and group scores tied in two classes of four). The one-token kernel (its selection on
    four waves, one expert per thread) gives the picks, weights and y of the general decode block, the per-pass kernels
    and the checker bit for bit: ties to the lower index, groups tied to the lower group."""
    import torch
    from loki_amd import MoeLayerWeights
    layer = MoeLayerWeights.synthetic(ctx, 7070)
    W, b = layer.gate_inp, layer.probs_b
    idx = torch.arange(NEXP, device=W.device)
    src = {"pairs": idx & ~1, "groups": idx & ~32, "quads": idx % 64}[pattern]
    W.copy_(W[src].clone())
    b.copy_(b[src].clone())
    torch.cuda.synchronize()
    Wh, bh = W.cpu().numpy(), b.cpu().numpy()
    for i in range(2):
        x = make_x(ctx, 1, seed=7100 + i)
        got = {}
        for name, m, d1 in (("decode1", 2, True), ("general", 2, False), ("per_pass", 0, True)):
            ctx.set_decode1(d1)
            try:
                with ctx.using_fused(m):
                    y = ctx.moe_layer(layer, x).clone()
                    ctx.sync()
                    assert ctx.debug().kernel == {"decode1": 2, "general": 1, "per_pass": 0}[name]
                    st = _routing_state(ctx, 1)
                    got[name] = (st["sel"], st["wts"], y.cpu().numpy())
            finally:
                ctx.set_decode1(True)
        for other in ("decode1", "general"):
            for k in range(3):
                assert np.array_equal(np.asarray(got[other][k]).view(np.uint8), np.asarray(got["per_pass"][k]).view(np.uint8)), (pattern, other, k, i)
        xs = x.cpu().numpy()
        _, _, so, wo = orc.router(Wh, bh, xs)
        assert np.array_equal(got["decode1"][0], so.ravel().astype(np.int32)) and np.array_equal(got["decode1"][1].view(np.uint32), wo.ravel().view(np.uint32))
        _, _, gate, up, down, sh = host_layer(ctx, layer, so.ravel())
        ref = orc.moe_forward(xs, Wh, bh, gate, up, down, *sh)
        assert np.array_equal(got["decode1"][2].view(np.uint32), ref["y"].view(np.uint32)), (pattern, i)
        assert len(set(so.ravel().tolist())) == 8
    del layer
    torch.cuda.empty_cache()


@pytest.mark.parametrize("kind", ["continuous", "levels16", "levels3", "hot", "flat"])
def test_decode1_selection_crafted_logits(ctx, kind):
    """The one-token kernel's selection (a threshold from the kept groups' second-best scores, then a rank of the
    candidates, with the round-by-round argmax as the fallback for more than 32 candidates) against the per-pass
    router (the round-by-round argmax) and the checker, on logits set directly: x = e_0 and router column 0 = the
    logits, so each logit is W[e, 0] exactly. "levels16" / "levels3" draw the logits and biases from 16 or 3 values
    (ties in scores, group scores and at the threshold; "levels3" mostly takes the fallback), "hot" adds +0.5 to 16
    experts, "flat" makes every logit equal (ties decided by index alone)."""
    import torch
    from loki_amd import MoeLayerWeights
    layer = MoeLayerWeights.synthetic(ctx, 7300)
    W, b = layer.gate_inp, layer.probs_b
    rng = np.random.default_rng({"continuous": 1, "levels16": 2, "levels3": 3, "hot": 4, "flat": 5}[kind])
    x = torch.zeros((1, E), dtype=torch.float32, device="cuda")
    x[0, 0] = 1.0
    for case in range(6):
        if kind == "continuous":
            lg, bias = rng.normal(0, 1.2, NEXP), rng.normal(0, 0.01, NEXP)
        elif kind == "levels16":
            lg, bias = rng.integers(-8, 8, NEXP) / 4.0, rng.integers(-2, 3, NEXP) / 64.0
        elif kind == "levels3":
            lg, bias = rng.integers(-1, 2, NEXP).astype(np.float64), rng.integers(0, 2, NEXP) / 8.0
        elif kind == "hot":
            lg, bias = rng.normal(0, 1.2, NEXP), rng.normal(0, 0.05, NEXP)
            bias[rng.choice(NEXP, 16, replace=False)] += 0.5
        else:
            lg, bias = np.full(NEXP, 0.25), np.zeros(NEXP)
        Wh = W.cpu().numpy()
        Wh[:, 0] = lg.astype(np.float32)
        W.copy_(torch.from_numpy(Wh))
        b.copy_(torch.from_numpy(bias.astype(np.float32)))
        torch.cuda.synchronize()
        got = {}
        for name, m in (("decode1", 2), ("per_pass", 0)):
            with ctx.using_fused(m):
                ctx.moe_layer(layer, x)
                ctx.sync()
                assert ctx.debug().kernel == {"decode1": 2, "per_pass": 0}[name]
                st = _routing_state(ctx, 1)
                got[name] = (st["sel"], st["wts"])
        assert np.array_equal(got["decode1"][0], got["per_pass"][0]), (kind, case)
        assert np.array_equal(got["decode1"][1].view(np.uint32), got["per_pass"][1].view(np.uint32)), (kind, case)
        _, _, so, wo = orc.router(W.cpu().numpy(), b.cpu().numpy(), x.cpu().numpy())
        assert np.array_equal(got["decode1"][0], so.ravel().astype(np.int32)), (kind, case)
        assert np.array_equal(got["decode1"][1].view(np.uint32), wo.ravel().view(np.uint32)), (kind, case)
    del layer
    torch.cuda.empty_cache()
