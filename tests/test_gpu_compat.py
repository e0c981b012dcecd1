"""GPU: the reference-named entry points (fl_ffn_begin / fl_fetch / fl_moe / fl_skip / fl_wide_*) driven the way the
reference's engine drives them (src/server_core_fused.cpp:793-818 narrow dispatch, :930-949 wide pass), and the
device-resident block against the committed full-shape golden vector."""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as orc
from tests.golden import gen

pytestmark = pytest.mark.gpu

E, H, KE = 7168, 2048, 8
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def cptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


@pytest.fixture(scope="module")
def small_layer(ctx):
    """16 routed experts (ggml layout, host) from the deterministic generator, and their device copies."""
    import torch
    W, b, gate, up, down, sh = gen.layer(202, 16, E, H)
    dev = dict(W=torch.from_numpy(W).cuda(), b=torch.from_numpy(b).cuda(),
               gate=torch.from_numpy(np.concatenate(gate)).cuda(), up=torch.from_numpy(np.concatenate(up)).cuda(),
               down=torch.from_numpy(np.concatenate(down)).cuda(),
               sh=[torch.from_numpy(m).cuda() for m in sh])
    ctx.set_experts(16)   # the reference-named entry points route over 16 experts in these tests
    yield (W, b, gate, up, down, sh), dev
    ctx.set_experts()


def test_golden_decode_full_on_device(ctx, small_layer):
    """fl_moe_layer (tiled copies of the generator's experts) reproduces the committed checker output bit for bit."""
    import torch
    from loki_amd import MoeLayerWeights
    z = np.load(os.path.join(GOLDEN, "decode_full.npz"), allow_pickle=False)
    (W, b, gate, up, down, sh), dev = small_layer
    mg = H * (E // 256) * 66
    L = MoeLayerWeights(dev["W"], dev["b"], ctx.pack(dev["gate"], H, E, 16), ctx.pack(dev["up"], H, E, 16),
                        ctx.pack(dev["down"], E, H, 16), ctx.pack(dev["sh"][0], H, E, 1), ctx.pack(dev["sh"][1], H, E, 1),
                        ctx.pack(dev["sh"][2], E, H, 1), n_exp=16)
    assert mg * 16 == dev["gate"].numel()
    y = ctx.moe_layer(L, torch.from_numpy(z["x"]).cuda())
    ctx.sync()
    dbg = ctx.debug()
    assert np.array_equal(ctx.d2h(dbg.sel, z["sel"].shape, np.int32), z["sel"])
    assert np.array_equal(y.cpu().numpy().view(np.uint32), z["y"].view(np.uint32))


def _flw(dev):
    from loki_amd import FLW
    w = FLW()
    w.gate_inp = dev["W"].data_ptr(); w.probs_b = dev["b"].data_ptr()
    w.sh_gate, w.sh_up, w.sh_down = (t.data_ptr() for t in dev["sh"])
    w.gate_f16 = 0
    return w


def _arena(dev, used):
    """The engine's expert arena for the experts `used`: gate/up/down of each, packed at ggml stride."""
    import torch
    mg = H * (E // 256) * 66
    idx = torch.as_tensor(used, dtype=torch.long)
    take = lambda t: t.view(16, mg)[idx.cuda()].contiguous().view(-1)
    return take(dev["gate"]), take(dev["up"]), take(dev["down"])


def test_fetch_mirrors_hold(ctx, small_layer):
    """fl_fetch's ncur / fi mirrors: the rows handed to fl_ffn_begin, still intact after the next fl_ffn_begin (the
    reference replaces its mirrors at the next call; here they hold until the second fl_ffn_begin after them), and the
    next fl_fetch hands out that call's rows."""
    from loki_amd import FLOut, lib
    (W, b, gate, up, down, sh), dev = small_layer
    ctx.set_routing(8, 4, 8, 2.5)
    flw = _flw(dev)
    rows = [(gen.uniform(7, 30 + i, (n, E), 2.0), gen.uniform(7, 40 + i, (n, E), 1.0)) for i, n in enumerate((5, 64, 2))]
    outs = []
    for x, fi in rows:
        ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(flw), x.shape[0], cptr(x), cptr(fi), -1))
        if outs:   # the previous fetch's mirrors survive this call
            px, pfi, po = outs[-1]
            n0 = px.shape[0]
            assert np.array_equal(np.ctypeslib.as_array(po.ncur, shape=(n0 * E,)).reshape(n0, E), px)
            assert np.array_equal(np.ctypeslib.as_array(po.fi, shape=(n0 * E,)).reshape(n0, E), pfi)
        out = FLOut()
        lib().fl_fetch(ctx.ctx, x.shape[0], 1, ctypes.byref(out))
        n = x.shape[0]
        assert np.array_equal(np.ctypeslib.as_array(out.ncur, shape=(n * E,)).reshape(n, E), x)
        assert np.array_equal(np.ctypeslib.as_array(out.fi, shape=(n * E,)).reshape(n, E), fi)
        outs.append((x, fi, out))
    ctx.sync()


def test_narrow_pass(ctx, small_layer):
    """fl_ffn_begin -> fl_fetch -> host dispatch (sorted unique experts, slot ids) -> fl_moe, as the engine does;
    h = routed + shared + ffn_inp with moe_combine's ascending-slot order (src/fused_layer.cu:366-372)."""
    from loki_amd import FLOut, lib
    (W, b, gate, up, down, sh), dev = small_layer
    ctx.set_routing(8, 4, 8, 2.5)
    n = 3
    x = gen.uniform(7, 3, (n, E), 2.0); fi = gen.uniform(7, 4, (n, E), 1.0)
    flw = _flw(dev)
    ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(flw), n, cptr(x), cptr(fi), -1))
    out = FLOut()
    lib().fl_fetch(ctx.ctx, n, 1, ctypes.byref(out))
    sel = np.ctypeslib.as_array(out.sel, shape=(n * KE,)).reshape(n, KE).copy()
    wts = np.ctypeslib.as_array(out.wts, shape=(n * KE,)).reshape(n, KE).copy()
    ncur = np.ctypeslib.as_array(out.ncur, shape=(n * E,)).reshape(n, E).copy()
    _, _, so, wo = orc.router(W, b, x, 8, 4, 8, 2.5)
    assert np.array_equal(sel, so) and np.array_equal(wts.view(np.uint32), wo.view(np.uint32))
    assert np.array_equal(ncur, x)
    used = sorted(set(sel.ravel().tolist()))
    remap = {e: i for i, e in enumerate(used)}
    ids = np.array([[remap[e] for e in row] for row in sel], np.int32)
    ga, ua, da = _arena(dev, used)
    lib().fl_moe(ctx.ctx, ga.data_ptr(), ua.data_ptr(), da.data_ptr(), len(used), 4, cptr(ids), cptr(f32(wts)), KE, n, ctypes.byref(out))
    h = np.ctypeslib.as_array(out.h, shape=(n * E,)).reshape(n, E).copy()
    moe = np.ctypeslib.as_array(out.moe, shape=(n * E,)).reshape(n, E).copy()
    ref = orc.moe_experts(x, so, wo, gate, up, down, *sh, want=("o", "sh"), n_exp=16)
    o = ref["o"].reshape(n, KE, E)
    for t in range(n):
        v = np.zeros(E, np.float32)
        for m in range(len(used)):
            ks = [k for k in range(KE) if ids[t, k] == m]
            if not ks:
                continue
            wt = np.float32(0)
            for k in ks:
                wt = np.float32(wt + wts[t, k])
            v = (v + wt * o[t, ks[0]]).astype(np.float32)
        assert np.array_equal(moe[t].view(np.uint32), v.view(np.uint32))
        want = ((v + ref["sh"][t]).astype(np.float32) + fi[t]).astype(np.float32)
        assert np.array_equal(h[t].view(np.uint32), want.view(np.uint32))
    # attribution of row 1: w_k * expert output, as the combine added them
    att = np.empty((KE, E), np.float32)
    lib().fl_moe_outs(ctx.ctx, 1, cptr(ids[1].copy()), cptr(f32(wts[1])), KE, cptr(att))
    assert np.array_equal(att.view(np.uint32), (wts[1][:, None] * o[1]).astype(np.float32).view(np.uint32))
    # fl_skip: h = mo + shared + ffn_inp
    mo = gen.uniform(7, 9, (n, E), 3.0)
    lib().fl_skip(ctx.ctx, cptr(mo), n, ctypes.byref(out))
    hs = np.ctypeslib.as_array(out.h, shape=(n * E,)).reshape(n, E).copy()
    want = (((np.float32(0) + mo) + ref["sh"]).astype(np.float32) + fi).astype(np.float32)
    assert np.array_equal(hs.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n", [3, 8])
def test_narrow_rows_single_launch(ctx, small_layer, n):
    """fl_moe on up to 8 rows of an all-IQ2_XXS layer runs as one launch of the n <= 8 block on the caller's picks
    (regular or cooperative launch; router and selection skipped, the shared expert recomputed in the launch, fl_moe's
    combine: the distinct ids ascending with their weights summed in k order, zero sums dropped). h, moe, the per-slot
    attribution (fl_moe_outs) and a following fl_skip are bit-identical to the per-pass kernels; one row gets a repeated
    id and one pick a zero weight."""
    from loki_amd import FLOut, lib
    (W, b, gate, up, down, sh), dev = small_layer
    ctx.set_routing(8, 4, 8, 2.5)
    x = gen.uniform(12, n, (n, E), 2.0); fi = gen.uniform(12, n + 10, (n, E), 1.0)
    mo = gen.uniform(12, n + 20, (n, E), 3.0)
    flw = _flw(dev)
    out = FLOut()
    _, _, so, wo = orc.router(W, b, x, 8, 4, 8, 2.5)
    ids = so.astype(np.int32).copy(); wts = f32(wo).copy()
    ids[1, 4] = ids[1, 2]; wts[n - 1, 6] = np.float32(0)
    got = {}
    for mode in (2, 1, 0):   # 2: the library default (regular launch); 1: cooperative; 0: the per-pass kernels
        with ctx.using_fused(mode):
            ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(flw), n, cptr(x), cptr(fi), -1))
            lib().fl_fetch(ctx.ctx, n, 1, ctypes.byref(out))
            lib().fl_moe(ctx.ctx, dev["gate"].data_ptr(), dev["up"].data_ptr(), dev["down"].data_ptr(), 16, 4, cptr(ids.ravel().copy()),
                         cptr(wts.ravel().copy()), KE, n, ctypes.byref(out))
            assert ctx.debug().kernel == (1 if mode else 0), mode
            hm = (np.ctypeslib.as_array(out.h, shape=(n * E,)).copy(), np.ctypeslib.as_array(out.moe, shape=(n * E,)).copy())
            atts = []
            for r in (0, 1, n - 1):
                att = np.zeros((KE, E), np.float32)
                lib().fl_moe_outs(ctx.ctx, r, cptr(ids[r].copy()), cptr(wts[r].copy()), KE, cptr(att))
                atts.append(att)
            lib().fl_skip(ctx.ctx, cptr(mo), n, ctypes.byref(out))
            got[mode] = hm + tuple(atts) + (np.ctypeslib.as_array(out.h, shape=(n * E,)).copy(),)
    for mode in (2, 1):
        for i, (a_, b_) in enumerate(zip(got[mode], got[0])):
            assert np.array_equal(a_.view(np.uint32), b_.view(np.uint32)), (mode, i)


def test_f16_router(ctx, small_layer):
    """fl_ffn_begin with an F16 router weight (FLW.gate_f16, fl.cu:317-319): widened exactly, it routes like the F32
    router holding the same values (selections, weights and the shared-expert path), and like the checker on them."""
    import torch
    from loki_amd import FLOut, lib
    (W, b, gate, up, down, sh), dev = small_layer
    ctx.set_routing(8, 4, 8, 2.5)
    n = 4
    x = gen.uniform(8, 3, (n, E), 2.0); fi = gen.uniform(8, 4, (n, E), 1.0)
    w16 = dev["W"].to(torch.float16)
    w32 = w16.to(torch.float32)
    res = []
    for wt, f16 in ((w16, 1), (w32, 0)):
        flw = _flw(dev)
        flw.gate_inp = wt.data_ptr(); flw.gate_f16 = f16
        ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(flw), n, cptr(x), cptr(fi), -1))
        out = FLOut()
        lib().fl_fetch(ctx.ctx, n, 1, ctypes.byref(out))
        res.append((np.ctypeslib.as_array(out.sel, shape=(n * KE,)).copy(), np.ctypeslib.as_array(out.wts, shape=(n * KE,)).copy()))
    assert np.array_equal(res[0][0], res[1][0]) and np.array_equal(res[0][1].view(np.uint32), res[1][1].view(np.uint32))
    _, _, so, wo = orc.router(w32.cpu().numpy(), b, x, 8, 4, 8, 2.5)
    assert np.array_equal(res[0][0].reshape(n, KE), so) and np.array_equal(res[0][1].reshape(n, KE).view(np.uint32), wo.view(np.uint32))


@pytest.mark.parametrize("mfma", [True, False], ids=["gemm", "per_pass"])
@pytest.mark.parametrize("waits", [True, False])
def test_wide_pass(ctx, small_layer, waits, mfma):
    """fl_wide_init -> fl_ffn_begin(wrow) per group -> per arena batch fl_wide_moe (slots of <= 8 (row, k) pairs in the
    engine's byexp order) -> fl_wide_finish; h = (ffn_inp + shared) + sum_k w_k o_k (src/fused_layer.cu:351-360).
    fl_wide_moe only enqueues: with waits=False the batches are issued back to back without fl_wide_wait, and the
    library's own per-parity guard keeps each parity's slot tables intact until their copies ran. The batches (about
    20 pairs per expert) run on the grouped MFMA GEMMs, or with fl_set_prefill_mfma(0) on the per-pass kernels."""
    ctx.set_prefill_mfma(mfma)
    try:
        _wide_pass(ctx, small_layer, waits)
    finally:
        ctx.set_prefill_mfma(True)


def test_wide_pass_row_loop(ctx, small_layer):
    """The wide pass's scatter kernel loops over (row, k) pairs beyond its grid's y extent (65535 pairs); with the extent
    capped at 7 (fl_set_debug bit 1) the loop runs over the 320 pairs here, and every output still equals the checker's."""
    ctx.set_debug(False, small_grids=True)
    try:
        _wide_pass(ctx, small_layer, True)
    finally:
        ctx.set_debug(False)


def _wide_pass(ctx, small_layer, waits):
    from loki_amd import FLOut, lib
    (W, b, gate, up, down, sh), dev = small_layer
    n, EB = 40, 5
    assert lib().fl_wide_init(ctx.ctx, 64, KE) == 1
    x = gen.uniform(8, 3, (n, E), 2.0); fi = gen.uniform(8, 4, (n, E), 1.0)
    flw = _flw(dev)
    sels, wtss = [], []
    out = FLOut()
    for r0 in range(0, n, 16):   # groups of rows, as the engine's fl_attn(wrow) loop
        g = min(16, n - r0)
        ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(flw), g, cptr(x[r0:r0 + g].copy()), cptr(fi[r0:r0 + g].copy()), r0))
        lib().fl_fetch(ctx.ctx, g, 1, ctypes.byref(out))
        sels.append(np.ctypeslib.as_array(out.sel, shape=(g * KE,)).reshape(g, KE).copy())
        wtss.append(np.ctypeslib.as_array(out.wts, shape=(g * KE,)).reshape(g, KE).copy())
    sel, wts = np.concatenate(sels), np.concatenate(wtss)
    used = sorted(set(sel.ravel().tolist()))
    byexp = {e: [] for e in used}
    for i in range(n):
        for k in range(KE):
            byexp[sel[i, k]].append((i, k))
    for bi, b0 in enumerate(range(0, len(used), EB)):
        batch = used[b0:b0 + EB]
        par = bi & 1
        if waits:
            lib().fl_wide_wait(ctx.ctx, par)
        midx, rows, kidx, wk = [], [], [], []
        for u, e in enumerate(batch):
            lst = byexp[e]
            for i0 in range(0, len(lst), 8):
                midx.append(u)
                for j in range(8):
                    if i0 + j < len(lst):
                        r, k = lst[i0 + j]; rows.append(r); kidx.append(k); wk.append(wts[r, k])
                    else:
                        rows.append(-1); kidx.append(0); wk.append(0.0)
        ga, ua, da = _arena(dev, batch)
        lib().fl_wide_moe(ctx.ctx, ga.data_ptr(), ua.data_ptr(), da.data_ptr(), 4, len(batch), cptr(np.int32(midx)),
                          cptr(np.int32(rows)), cptr(np.int32(kidx)), cptr(f32(wk)), len(midx), KE, par)
        lib().fl_wide_mark(ctx.ctx, par)
    lib().fl_wide_finish(ctx.ctx, n, KE, ctypes.byref(out))
    h = np.ctypeslib.as_array(out.h, shape=(n * E,)).reshape(n, E).copy()
    moe = np.ctypeslib.as_array(out.moe, shape=(n * E,)).reshape(n, E).copy()
    ref = orc.moe_experts(x, sel, wts, gate, up, down, *sh, want=("o", "sh"), n_exp=16)
    o = ref["o"].reshape(n, KE, E)
    m = np.zeros((n, E), np.float32)
    for k in range(KE):
        m = (m + wts[:, k:k + 1] * o[:, k]).astype(np.float32)
    base = (fi + ref["sh"]).astype(np.float32)
    assert np.array_equal(moe.view(np.uint32), m.view(np.uint32))
    assert np.array_equal(h.view(np.uint32), (base + m).astype(np.float32).view(np.uint32))
    outs = np.empty((KE, E), np.float32)
    lib().fl_wide_outs(ctx.ctx, 5, KE, cptr(outs))
    assert np.array_equal(outs.view(np.uint32), (wts[5][:, None] * o[5]).astype(np.float32).view(np.uint32))
    mo = gen.uniform(8, 9, (n, E), 3.0)
    lib().fl_wide_skip(ctx.ctx, cptr(mo), n, ctypes.byref(out))
    hs = np.ctypeslib.as_array(out.h, shape=(n * E,)).reshape(n, E).copy()
    assert np.array_equal(hs.view(np.uint32), (base + mo).astype(np.float32).view(np.uint32))


def test_narrow_pass_declared_tiled(ctx, small_layer):
    """A resident arena of every expert (ids = expert ids) in the tiled layout, declared with fl_register_tiled, and a
    declared-tiled shared expert: fl_ffn_begin / fl_moe read them in place (no repack) and give h and moe bit for bit
    as the same arena and shared expert in ggml's layout; after fl_unregister_tiled the ggml arena still runs."""
    import torch
    from loki_amd import FLOut, lib
    (W, b, gate, up, down, sh), dev = small_layer
    ctx.set_routing(8, 4, 8, 2.5)
    n = 2
    x = gen.uniform(9, 3, (n, E), 2.0); fi = gen.uniform(9, 4, (n, E), 1.0)
    tiled = dict(gate=ctx.pack(dev["gate"], H, E, 16), up=ctx.pack(dev["up"], H, E, 16), down=ctx.pack(dev["down"], E, H, 16),
                 sh=[ctx.pack(dev["sh"][0], H, E, 1), ctx.pack(dev["sh"][1], H, E, 1), ctx.pack(dev["sh"][2], E, H, 1)])
    torch.cuda.synchronize()

    def run(g, u, d, shm):
        flw = _flw(dict(dev, sh=shm))
        ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(flw), n, cptr(x), cptr(fi), -1))
        out = FLOut()
        lib().fl_fetch(ctx.ctx, n, 1, ctypes.byref(out))
        sel = np.ctypeslib.as_array(out.sel, shape=(n * KE,)).copy().astype(np.int32)
        wts = np.ctypeslib.as_array(out.wts, shape=(n * KE,)).copy()
        lib().fl_moe(ctx.ctx, g.data_ptr(), u.data_ptr(), d.data_ptr(), 16, 4, cptr(sel), cptr(f32(wts)), KE, n, ctypes.byref(out))
        return (np.ctypeslib.as_array(out.h, shape=(n * E,)).copy(), np.ctypeslib.as_array(out.moe, shape=(n * E,)).copy())

    want = run(dev["gate"], dev["up"], dev["down"], dev["sh"])
    for t in (tiled["gate"], tiled["up"], tiled["down"], *tiled["sh"]):
        ctx.register_tiled(t)
    try:
        got = run(tiled["gate"], tiled["up"], tiled["down"], tiled["sh"])
    finally:
        for t in (tiled["gate"], tiled["up"], tiled["down"], *tiled["sh"]):
            ctx.unregister_tiled(t)
    for a_, b_ in zip(got, want):
        assert np.array_equal(a_.view(np.uint32), b_.view(np.uint32))
    again = run(dev["gate"], dev["up"], dev["down"], dev["sh"])
    for a_, b_ in zip(again, want):
        assert np.array_equal(a_.view(np.uint32), b_.view(np.uint32))


def test_narrow_pass_keep2_with_pad_rows(ctx, small_layer):
    """The engine's production decode call (src/server_core_fused.cpp:793-818, KE = 2 at :340): a fixed-width pass of
    8 rows whose last 3 are padding. fl_fetch's routing goes through the host keep-2 with the 2.5 rescale, pad rows take
    row 0's kept experts at weight 0, the used experts become the arena, and fl_moe runs KE = 2. h and moe follow
    moe_combine's ascending-slot order with merged weights (src/fused_layer.cu:366-372)."""
    from loki_amd import FLOut, lib
    (W, b, gate, up, down, sh), dev = small_layer
    ctx.set_routing(8, 4, 8, 2.5)
    n, n_real, ke = 8, 5, 2
    x = gen.uniform(9, 3, (n, E), 2.0); fi = gen.uniform(9, 4, (n, E), 1.0)
    flw = _flw(dev)
    ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(flw), n, cptr(x), cptr(fi), -1))
    out = FLOut()
    lib().fl_fetch(ctx.ctx, n, 1, ctypes.byref(out))
    sel = np.ctypeslib.as_array(out.sel, shape=(n * KE,)).reshape(n, KE).copy()
    wts = np.ctypeslib.as_array(out.wts, shape=(n * KE,)).reshape(n, KE).copy()
    _, _, so, wo = orc.router(W, b, x, 8, 4, 8, 2.5)
    assert np.array_equal(sel, so) and np.array_equal(wts.view(np.uint32), wo.view(np.uint32))
    sk, wk = orc.keep_experts(sel, wts, ke, 2.5, n_real)
    assert np.all(wk[n_real:] == 0) and np.all(sk[n_real:] == sk[0])
    used = sorted(set(sk.ravel().tolist()))
    remap = {e: i for i, e in enumerate(used)}
    ids = np.array([[remap[e] for e in row] for row in sk], np.int32)
    ga, ua, da = _arena(dev, used)
    lib().fl_moe(ctx.ctx, ga.data_ptr(), ua.data_ptr(), da.data_ptr(), len(used), 4, cptr(ids), cptr(f32(wk)), ke, n, ctypes.byref(out))
    h = np.ctypeslib.as_array(out.h, shape=(n * E,)).reshape(n, E).copy()
    moe = np.ctypeslib.as_array(out.moe, shape=(n * E,)).reshape(n, E).copy()
    ref = orc.moe_experts(x, sk, wk, gate, up, down, *sh, want=("o", "sh"), n_exp=16)
    o = ref["o"].reshape(n, ke, E)
    for t in range(n):
        v = np.zeros(E, np.float32)
        for m in range(len(used)):
            ks = [k for k in range(ke) if ids[t, k] == m]
            if not ks:
                continue
            wt = np.float32(0)
            for k in ks:
                wt = np.float32(wt + wk[t, k])
            v = (v + wt * o[t, ks[0]]).astype(np.float32)
        assert np.array_equal(moe[t].view(np.uint32), v.view(np.uint32)), t
        want = ((v + ref["sh"][t]).astype(np.float32) + fi[t]).astype(np.float32)
        assert np.array_equal(h[t].view(np.uint32), want.view(np.uint32)), t


@pytest.mark.parametrize("case", ["picks", "repeats"])
def test_narrow_one_row_single_launch(ctx, small_layer, case):
    """fl_moe on one row with all 8 picks runs as one launch of the one-token kernel on the caller's picks (router and
    selection skipped, the shared expert recomputed in the launch, fl_moe's combine: the distinct ids ascending with
    their weights summed in k order, zero sums dropped). h and moe are bit-identical to the per-pass kernels and to the
    checker's experts combined by that rule; "repeats" gives the row a repeated id and a zero weight."""
    from loki_amd import FLOut, lib
    (W, b, gate, up, down, sh), dev = small_layer
    ctx.set_routing(8, 4, 8, 2.5)
    x = gen.uniform(11, 3, (1, E), 2.0); fi = gen.uniform(11, 4, (1, E), 1.0)
    flw = _flw(dev)
    out = FLOut()
    _, _, so, wo = orc.router(W, b, x, 8, 4, 8, 2.5)
    ids = so[0].astype(np.int32).copy(); wts = f32(wo[0]).copy()
    if case == "repeats":
        ids[3] = ids[1]; wts[5] = np.float32(0)
    mo = gen.uniform(11, 5, (1, E), 3.0)
    got = {}
    for mode in (2, 0):   # 2: the library default (the one-token kernel); 0: the per-pass kernels
        with ctx.using_fused(mode):
            ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(flw), 1, cptr(x), cptr(fi), -1))
            lib().fl_fetch(ctx.ctx, 1, 1, ctypes.byref(out))
            lib().fl_moe(ctx.ctx, dev["gate"].data_ptr(), dev["up"].data_ptr(), dev["down"].data_ptr(), 16, 4, cptr(ids), cptr(wts),
                         KE, 1, ctypes.byref(out))
            assert ctx.debug().kernel == (2 if mode else 0), mode
            hm = (np.ctypeslib.as_array(out.h, shape=(E,)).copy(), np.ctypeslib.as_array(out.moe, shape=(E,)).copy())
            att = np.zeros((KE, E), np.float32)   # the per-slot attribution of that call
            lib().fl_moe_outs(ctx.ctx, 0, cptr(ids), cptr(wts), KE, cptr(att))
            lib().fl_skip(ctx.ctx, cptr(mo), 1, ctypes.byref(out))   # needs the shared expert the launch did not keep
            got[mode] = hm + (att, np.ctypeslib.as_array(out.h, shape=(E,)).copy())
    for a_, b_ in zip(got[2], got[0]):
        assert np.array_equal(a_.view(np.uint32), b_.view(np.uint32)), case
    ref = orc.moe_experts(x, ids[None, :], wts[None, :], gate, up, down, *sh, want=("o", "sh"), n_exp=16)
    o = ref["o"].reshape(KE, E)
    v = np.zeros(E, np.float32)
    for m in sorted(set(ids.tolist())):
        ks = [k for k in range(KE) if ids[k] == m]
        wt = np.float32(0)
        for k in ks:
            wt = np.float32(wt + wts[k])
        if wt == 0:
            continue
        v = (v + wt * o[ks[0]]).astype(np.float32)
    assert np.array_equal(got[2][1].view(np.uint32), v.view(np.uint32))
    want = ((v + ref["sh"][0]).astype(np.float32) + fi[0]).astype(np.float32)
    assert np.array_equal(got[2][0].view(np.uint32), want.view(np.uint32))
    first = [list(ids).index(ids[k]) for k in range(KE)]
    att = (wts[:, None] * o[first]).astype(np.float32)
    assert np.array_equal(got[2][2].view(np.uint32), att.view(np.uint32))
    skip = (((np.float32(0) + mo[0]) + ref["sh"][0]).astype(np.float32) + fi[0]).astype(np.float32)
    assert np.array_equal(got[2][3].view(np.uint32), skip.view(np.uint32))


def _hip():
    """The HIP runtime, for the host allocations an engine makes itself (pinned staging, events)."""
    h = ctypes.CDLL("libamdhip64.so")
    h.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
    h.hipHostFree.argtypes = [ctypes.c_void_p]
    return h


def test_h2d_kernel_and_copy_engine(ctx):
    """fl_h2d (src/fused_layer.cu:414-420): pinned sources are copied by a kernel reading the mapped memory (aligned
    16-byte words and the unaligned byte path), pageable ones by the copy engine; the counts of fl_h2d_bytes say which
    path ran, and every destination byte equals its source."""
    import torch
    from loki_amd import lib
    hip = _hip()
    nbytes = (3 << 20) + 4096
    p = ctypes.c_void_p()
    assert hip.hipHostMalloc(ctypes.byref(p), nbytes, 0) == 0
    try:
        pinned = np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint8)), shape=(nbytes,))
        pinned[:] = np.random.default_rng(5).integers(0, 256, nbytes, dtype=np.uint8)
        dst = torch.zeros(nbytes + 64, dtype=torch.uint8, device="cuda")
        zc0, ce0 = ctypes.c_size_t(), ctypes.c_size_t()
        ctx.check(lib().fl_h2d_bytes(ctx.ctx, ctypes.byref(zc0), ctypes.byref(ce0)))
        cases = [(0, 0, 3 << 20), (16, 32, 4096 * 7), (3, 5, 100_003), (1, 0, 17)]   # (src off, dst off, bytes)
        for so, do, n in cases:
            lib().fl_h2d(ctx.ctx, dst.data_ptr() + do, p.value + so, n)
        ctx.sync()
        zc1, ce1 = ctypes.c_size_t(), ctypes.c_size_t()
        ctx.check(lib().fl_h2d_bytes(ctx.ctx, ctypes.byref(zc1), ctypes.byref(ce1)))
        assert zc1.value - zc0.value == sum(n for _, _, n in cases) and ce1.value == ce0.value
        got = dst.cpu().numpy()
        # later cases overwrite earlier ones' bytes: check each case on its own, in order, against a host replay
        want = np.zeros(nbytes + 64, np.uint8)
        for so, do, n in cases:
            want[do:do + n] = pinned[so:so + n]
        assert np.array_equal(got, want)
        # pageable host memory: the copy engine
        page = np.random.default_rng(6).integers(0, 256, 50_001, dtype=np.uint8)
        lib().fl_h2d(ctx.ctx, dst.data_ptr() + 7, page.ctypes.data, page.size)
        ctx.sync()
        zc2, ce2 = ctypes.c_size_t(), ctypes.c_size_t()
        ctx.check(lib().fl_h2d_bytes(ctx.ctx, ctypes.byref(zc2), ctypes.byref(ce2)))
        assert zc2.value == zc1.value and ce2.value - ce1.value == page.size
        assert np.array_equal(dst[7:7 + page.size].cpu().numpy(), page)
    finally:
        hip.hipHostFree(p)


def test_wait_event_orders_the_context_stream(ctx):
    """fl_wait_event (src/fused_layer.cu:421): work enqueued on the context's stream after the call starts only once
    the event of another stream (the engine's loader) has completed. Another stream is kept busy for milliseconds
    before it writes a marker and records the event; a copy of the marker on the context's stream reads the old value
    without the wait (the control) and the new one with it."""
    import torch
    from loki_amd import lib
    big = torch.ones(1 << 27, dtype=torch.float32, device="cuda")   # 512 MB: each pass ~0.15 ms
    side = torch.cuda.Stream()
    assert torch.cuda.current_stream().cuda_stream == (ctx.stream_handle or 0)   # the context runs on torch's current stream
    for waited in (False, True):
        marker = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        with torch.cuda.stream(side):
            for _ in range(200):
                big.mul_(1.0)
            marker.fill_(7.0)
            ev = torch.cuda.Event()
            ev.record(side)
        if waited:
            lib().fl_wait_event(ctx.ctx, ctypes.c_void_p(ev.cuda_event))
        seen = marker.clone()   # on the context's stream
        torch.cuda.synchronize()
        assert bool((seen == (7.0 if waited else 0.0)).all()), "waited=%s" % waited


def test_gpu_ms_accounts_the_calls(ctx, small_layer):
    """fl_gpu_ms (src/fused_layer.cu:620): 1 accumulates the experts' GPU time of fl_moe / fl_skip, 0 and 2 that of
    fl_ffn_begin (the router this library runs in the reference's attention phase), 3 (speculation) stays 0."""
    from loki_amd import FLOut, lib
    (W, b, gate, up, down, sh), dev = small_layer
    ctx.set_routing(8, 4, 8, 2.5)
    flw = _flw(dev)
    n = 2
    x = gen.uniform(7, 13, (n, E), 2.0); fi = gen.uniform(7, 14, (n, E), 1.0)
    m0, a0, s0 = (lib().fl_gpu_ms(ctx.ctx, w) for w in (1, 0, 3))
    ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(flw), n, cptr(x), cptr(fi), -1))
    out = FLOut()
    lib().fl_fetch(ctx.ctx, n, 1, ctypes.byref(out))
    a1 = lib().fl_gpu_ms(ctx.ctx, 0)
    assert a1 > a0 and lib().fl_gpu_ms(ctx.ctx, 2) == a1
    sel = np.ctypeslib.as_array(out.sel, shape=(n * KE,)).reshape(n, KE).copy()
    wts = np.ctypeslib.as_array(out.wts, shape=(n * KE,)).reshape(n, KE).copy()
    used = sorted(set(sel.ravel().tolist()))
    ids = np.array([[used.index(e) for e in row] for row in sel], np.int32)
    ga, ua, da = _arena(dev, used)
    lib().fl_moe(ctx.ctx, ga.data_ptr(), ua.data_ptr(), da.data_ptr(), len(used), 4, cptr(ids), cptr(f32(wts)), KE, n, ctypes.byref(out))
    m1 = lib().fl_gpu_ms(ctx.ctx, 1)
    assert m1 > m0
    mo = gen.uniform(7, 15, (n, E), 3.0)
    lib().fl_skip(ctx.ctx, cptr(mo), n, ctypes.byref(out))
    assert lib().fl_gpu_ms(ctx.ctx, 1) > m1
    assert lib().fl_gpu_ms(ctx.ctx, 3) == s0 == 0.0


def test_speculative_one_token_launch(ctx):
    """The engine's decode-1 loop on a resident arena of all 256 experts, declared tiled (ids = expert ids): after the
    first fl_moe on the routing's own picks, each fl_ffn_begin runs the whole block in its routing launch and fl_moe
    only waits for it (FLDebug.kernel 3). h and moe are bit-identical to the per-pass kernels on the same calls. A call
    whose weights differ from the routing's (one weight scaled) runs its own launch on them (kernel 2), and so does
    the call after it (the speculation restarts only after an fl_moe on the routing's own picks)."""
    import torch
    from loki_amd import FLOut, FLW, MoeLayerWeights, lib
    L = MoeLayerWeights.synthetic(ctx, 7400)
    mats = (L.gate, L.up, L.down, L.sh_gate, L.sh_up, L.sh_down)
    ctx.set_routing(8, 4, 8, 2.5)
    ctx.set_experts(256)   # this module's other tests route over 16 experts
    rng = np.random.default_rng(7400)
    T = 6
    xs = rng.standard_normal((T, E)).astype(np.float32)
    fis = rng.standard_normal((T, E)).astype(np.float32)
    w = FLW()
    w.gate_inp = L.gate_inp.data_ptr(); w.probs_b = L.probs_b.data_ptr(); w.gate_f16 = 0
    w.sh_gate, w.sh_up, w.sh_down = (m.data_ptr() for m in mats[3:])

    def run(changed):
        out = FLOut()
        res = []
        for i in range(T):
            ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(w), 1, cptr(xs[i]), cptr(fis[i]), -1))
            lib().fl_fetch(ctx.ctx, 1, 1, ctypes.byref(out))
            sel = np.ctypeslib.as_array(out.sel, shape=(KE,)).astype(np.int32).copy()
            wts = np.ctypeslib.as_array(out.wts, shape=(KE,)).copy()
            if i == changed:
                wts[3] = np.float32(wts[3] * np.float32(0.5))
            lib().fl_moe(ctx.ctx, L.gate.data_ptr(), L.up.data_ptr(), L.down.data_ptr(), 256, 4, cptr(sel), cptr(f32(wts)), KE, 1,
                         ctypes.byref(out))
            res.append((ctx.debug().kernel, np.ctypeslib.as_array(out.h, shape=(E,)).copy(),
                        np.ctypeslib.as_array(out.moe, shape=(E,)).copy(), sel))
        return res

    for t in mats:
        ctx.register_tiled(t)
    try:
        for changed in (-1, 2):
            spec = run(changed)
            with ctx.using_fused(0):
                plain = run(changed)
            kernels = [r[0] for r in spec]
            want = [2, 3, 3, 3, 3, 3] if changed < 0 else [2, 3, 2, 2, 3, 3]
            assert kernels == want, (changed, kernels)
            assert all(r[0] == 0 for r in plain)
            for i in range(T):
                assert np.array_equal(spec[i][3], plain[i][3]), (changed, i)
                assert np.array_equal(spec[i][1].view(np.uint32), plain[i][1].view(np.uint32)), (changed, i)
                assert np.array_equal(spec[i][2].view(np.uint32), plain[i][2].view(np.uint32)), (changed, i)
    finally:
        for t in mats:
            ctx.unregister_tiled(t)
        ctx.set_experts(16)
    del L
    torch.cuda.empty_cache()
