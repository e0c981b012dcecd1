"""GPU: the K-quant formats of the reference's real shards against the CPU checker (oracle/kquant_oracle.c):
fl_kq_matvec_dev per format and shape (the reference's tc_matvec<F_Q2K/Q3K/Q5K/Q6K>, src/fused_layer.cu:102-158,
203-254), the routed down in Q2_K / Q3_K through fl_moe and fl_wide_moe (:541-550, 599-608), and the shared expert in
Q5_K / Q5_K / Q6_K through fl_ffn_begin (:520-524).

Tolerances: the integer sub-block sums are exact, and Q2_K's fp32 order is ggml's (bit-identical). Q3_K / Q5_K / Q6_K
add the per-block terms in block order where ggml keeps 8 column-residue partial sums, so they differ by fp32 rounding
only: |y - ref| <= 1e-5 * sum |w x| per output. Block outputs behind a non-exact stage are held to 1e-4 (L2, relative)
and 1e-3 of the largest |output| (max), inside the 2e-3 / 1e-2 parity bar."""
import ctypes

import numpy as np
import pytest

from oracle import oracle as orc
from tests.golden import gen

pytestmark = pytest.mark.gpu

E, H, KE = 7168, 2048, 8
FMTS = [orc.Q2K, orc.Q3K, orc.Q5K, orc.Q6K]
NAMES = {orc.Q2K: "q2_K", orc.Q3K: "q3_K", orc.Q5K: "q5_K", orc.Q6K: "q6_K"}


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def cptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def within_rounding(got, ref, wd, xd, rel=1e-5):
    """|got - ref| <= rel * sum |w x| elementwise; wd [R, K] and xd [n, K] dequantized operands"""
    scale = np.abs(xd.astype(np.float64)) @ np.abs(wd.astype(np.float64)).T
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    return bool(np.all(err <= rel * scale)), float((err / np.maximum(scale, 1e-30)).max())


def bar_close(got, ref, l2=1e-4, mx=1e-3):
    d = got.astype(np.float64) - ref.astype(np.float64)
    r = ref.astype(np.float64)
    e_l2 = np.linalg.norm(d) / max(np.linalg.norm(r), 1e-30)
    e_mx = np.abs(d).max() / max(np.abs(r).max(), 1e-30)
    return e_l2 <= l2 and e_mx <= mx, (e_l2, e_mx)


@pytest.mark.parametrize("fmt", FMTS, ids=lambda f: NAMES[f])
@pytest.mark.parametrize("K,R,n", [(2048, 130, 3), (7168, 66, 2), (256, 98, 5), (4096, 64, 1), (2048, 200, 9)])
def test_kq_matvec(ctx, fmt, K, R, n):
    import torch
    w = gen.kq_matrix(31 + fmt, K + R, fmt, R, K)
    x = gen.uniform(32 + fmt, K + n, (n, K), 3.0)
    q, d, bs = orc.quantize_q8k(x)
    ref = orc.matvec_kq(fmt, w, R, K, q, d, bs)
    print("kq_matvec fmt %d K %d R %d n %d" % (fmt, K, R, n), flush=True)
    y = ctx.kq_matvec(fmt, torch.from_numpy(w).cuda(), R, K, torch.from_numpy(q).cuda(), torch.from_numpy(d).cuda())
    ctx.sync()
    y = y.cpu().numpy()
    if fmt == orc.Q2K:
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
    else:
        wd = orc.dequant_kq(fmt, w, K)
        xd = q.astype(np.float32) * np.repeat(d, 256, axis=1)
        ok, worst = within_rounding(y, ref, wd, xd)
        assert ok, worst


def test_kq_matvec_rejects(ctx):
    """argument errors come back as FL_EINVAL with a message, before any launch"""
    import torch
    from loki_amd import lib, FL_EINVAL, FL_Q3K
    w = torch.zeros(110, dtype=torch.uint8, device="cuda")
    q = torch.zeros((1, 256), dtype=torch.int8, device="cuda"); d = torch.zeros((1, 1), dtype=torch.float32, device="cuda")
    y = torch.zeros((1, 1), dtype=torch.float32, device="cuda")
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    assert lib().fl_kq_matvec_dev(ctx.ctx, 4, P(w), 1, 256, P(q), P(d), 1, P(y)) == FL_EINVAL          # IQ2 is not a K-quant
    assert lib().fl_kq_matvec_dev(ctx.ctx, FL_Q3K, P(w), 1, 256, P(q), P(d), 1, P(y)) == FL_EINVAL     # 110 B: not 4-byte sized
    assert lib().fl_kq_matvec_dev(ctx.ctx, FL_Q3K, P(w), 2, 256, P(q), P(d), -1, P(y)) == FL_EINVAL    # n < 0
    assert lib().fl_kq_matvec_dev(ctx.ctx, FL_Q3K, P(w), 1, 300, P(q), P(d), 1, P(y)) == FL_EINVAL     # K % 256
    assert b"K-quant" in lib().fl_last_error(ctx.ctx) or b"256" in lib().fl_last_error(ctx.ctx)


# ---------------------------------------------------------------- the reference-named entry points
@pytest.fixture(scope="module")
def real_layer(ctx):
    """16 routed experts: IQ2_XXS gate/up (ggml layout) with Q2_K and Q3_K downs, IQ2_XXS and K-quant shared experts"""
    import torch
    W, b, gate, up, down, sh = gen.layer(202, 16, E, H)
    kdown = {f: [gen.kq_matrix(203, 40 + e, f, E, H) for e in range(16)] for f in (orc.Q2K, orc.Q3K)}
    ksh = (gen.kq_matrix(204, 1, orc.Q5K, H, E), gen.kq_matrix(204, 2, orc.Q5K, H, E), gen.kq_matrix(204, 3, orc.Q6K, E, H))
    dev = dict(W=torch.from_numpy(W).cuda(), b=torch.from_numpy(b).cuda(),
               gate=torch.from_numpy(np.concatenate(gate)).cuda(), up=torch.from_numpy(np.concatenate(up)).cuda(),
               kdown={f: torch.from_numpy(np.concatenate(m)).cuda() for f, m in kdown.items()},
               sh=[torch.from_numpy(m).cuda() for m in sh], ksh=[torch.from_numpy(m).cuda() for m in ksh])
    ctx.set_experts(16)
    yield dict(W=W, b=b, gate=gate, up=up, kdown=kdown, sh=sh, ksh=ksh), dev
    ctx.set_experts()
    ctx.set_shared_formats()


def _flw(dev, kshared):
    from loki_amd import FLW
    w = FLW()
    w.gate_inp = dev["W"].data_ptr(); w.probs_b = dev["b"].data_ptr()
    w.sh_gate, w.sh_up, w.sh_down = (t.data_ptr() for t in (dev["ksh"] if kshared else dev["sh"]))
    w.gate_f16 = 0
    return w


def _arena(dev, used, fmt):
    import torch
    mg = H * (E // 256) * 66
    md = E * (H // 256) * orc.kq_block_bytes(fmt)
    idx = torch.as_tensor(used, dtype=torch.long).cuda()
    return (dev["gate"].view(16, mg)[idx].contiguous().view(-1), dev["up"].view(16, mg)[idx].contiguous().view(-1),
            dev["kdown"][fmt].view(16, md)[idx].contiguous().view(-1))


def _route(ctx, flw, x, fi, wrow=-1):
    from loki_amd import FLOut, lib
    n = x.shape[0]
    ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(flw), n, cptr(x), cptr(fi), wrow))
    out = FLOut()
    lib().fl_fetch(ctx.ctx, n, 1, ctypes.byref(out))
    sel = np.ctypeslib.as_array(out.sel, shape=(n * KE,)).reshape(n, KE).copy()
    wts = np.ctypeslib.as_array(out.wts, shape=(n * KE,)).reshape(n, KE).copy()
    return sel, wts


@pytest.mark.parametrize("down_fmt", [orc.Q2K, orc.Q3K], ids=["q2_K", "q3_K"])
@pytest.mark.parametrize("kshared", [False, True], ids=["iq2_shared", "q5q5q6_shared"])
def test_narrow_real_formats(ctx, real_layer, down_fmt, kshared):
    """fl_ffn_begin -> fl_fetch -> fl_moe with the routed down in Q2_K / Q3_K and the shared expert in IQ2_XXS or
    Q5_K / Q5_K / Q6_K; with Q2_K down and the IQ2_XXS shared expert every stage is exact, so h and moe are bit-identical
    to the checker composed with moe_combine's slot order (src/fused_layer.cu:366-372)."""
    from loki_amd import FLOut, lib
    host, dev = real_layer
    ctx.set_routing(8, 4, 8, 2.5)
    if kshared:
        ctx.set_shared_formats(orc.Q5K, orc.Q5K, orc.Q6K)
    else:
        ctx.set_shared_formats()
    n = 5
    x = gen.uniform(9, 3, (n, E), 2.0); fi = gen.uniform(9, 4, (n, E), 1.0)
    print("narrow down_fmt %d kshared %d n %d" % (down_fmt, kshared, n), flush=True)
    sel, wts = _route(ctx, _flw(dev, kshared), x, fi)
    used = sorted(set(sel.ravel().tolist()))
    remap = {e: i for i, e in enumerate(used)}
    ids = np.array([[remap[e] for e in row] for row in sel], np.int32)
    ga, ua, da = _arena(dev, used, down_fmt)
    out = FLOut()
    lib().fl_moe(ctx.ctx, ga.data_ptr(), ua.data_ptr(), da.data_ptr(), len(used), down_fmt, cptr(ids), cptr(f32(wts)), KE, n,
                 ctypes.byref(out))
    h = np.ctypeslib.as_array(out.h, shape=(n * E,)).reshape(n, E).copy()
    moe = np.ctypeslib.as_array(out.moe, shape=(n * E,)).reshape(n, E).copy()
    sh = host["ksh"] if kshared else host["sh"]
    fm = (down_fmt,) + ((orc.Q5K, orc.Q5K, orc.Q6K) if kshared else (4, 4, 4))
    ref = orc.moe_experts(x, sel, wts, host["gate"], host["up"], host["kdown"][down_fmt], *sh, want=("o", "sh"), n_exp=16, fmts=fm)
    o = ref["o"].reshape(n, KE, E)
    vm = np.zeros((n, E), np.float32)
    for t in range(n):
        for m in range(len(used)):
            ks = [k for k in range(KE) if ids[t, k] == m]
            if not ks:
                continue
            wt = np.float32(0)
            for k in ks:
                wt = np.float32(wt + wts[t, k])
            vm[t] = (vm[t] + wt * o[t, ks[0]]).astype(np.float32)
    want_h = ((vm + ref["sh"]).astype(np.float32) + fi).astype(np.float32)
    if down_fmt == orc.Q2K:
        assert np.array_equal(moe.view(np.uint32), vm.view(np.uint32))
    else:
        ok, err = bar_close(moe, vm)
        assert ok, err
    if down_fmt == orc.Q2K and not kshared:
        assert np.array_equal(h.view(np.uint32), want_h.view(np.uint32))
    else:
        ok, err = bar_close(h, want_h)
        assert ok, err


@pytest.mark.parametrize("down_fmt", [orc.Q2K, orc.Q3K], ids=["q2_K", "q3_K"])
def test_narrow_one_row_real_formats_single_launch(ctx, real_layer, down_fmt):
    """fl_moe on one row with all 8 picks, routed down Q2_K / Q3_K and the shared expert Q5_K / Q5_K / Q6_K (the real
    shards' formats): one launch of the one-token kernel's K-quant variant on the caller's picks, h and moe bit-identical
    to the per-pass kernels (fl_set_fused(0)), on a remapped arena of the picked experts"""
    from loki_amd import FLOut, lib
    host, dev = real_layer
    ctx.set_routing(8, 4, 8, 2.5)
    ctx.set_shared_formats(orc.Q5K, orc.Q5K, orc.Q6K)
    x = gen.uniform(13, 3, (1, E), 2.0); fi = gen.uniform(13, 4, (1, E), 1.0)
    got = {}
    for mode in (2, 0):
        with ctx.using_fused(mode):
            sel, wts = _route(ctx, _flw(dev, True), x, fi)
            used = sorted(set(sel.ravel().tolist()))
            remap = {e: i for i, e in enumerate(used)}
            ids = np.array([remap[e] for e in sel[0]], np.int32)
            ga, ua, da = _arena(dev, used, down_fmt)
            out = FLOut()
            lib().fl_moe(ctx.ctx, ga.data_ptr(), ua.data_ptr(), da.data_ptr(), len(used), down_fmt, cptr(ids), cptr(f32(wts[0])), KE, 1,
                         ctypes.byref(out))
            assert ctx.debug().kernel == (2 if mode else 0), mode
            got[mode] = (np.ctypeslib.as_array(out.h, shape=(E,)).copy(), np.ctypeslib.as_array(out.moe, shape=(E,)).copy())
    for a_, b_ in zip(got[2], got[0]):
        assert np.array_equal(a_.view(np.uint32), b_.view(np.uint32)), down_fmt


def test_wide_q3k_down(ctx, real_layer):
    """the wide pass (fl_wide_init / fl_ffn_begin(wrow) / fl_wide_moe / fl_wide_finish) with a Q3_K down and the
    K-quant shared expert: 16 experts and top-8 give each expert about 20 of the 320 pairs. The batches run on the
    grouped GEMMs (IQ2_XXS gate/up, Q3_K down) and again on the per-pass kernels (fl_set_prefill_mfma(0), the mat-vec
    in several token groups per expert): h and moe bit-identical, and within the K-quant bar of the checker"""
    from loki_amd import FLOut, lib
    host, dev = real_layer
    ctx.set_routing(1, 1, 8, 1.0)
    ctx.set_shared_formats(orc.Q5K, orc.Q5K, orc.Q6K)
    n, EB = 40, 6
    assert lib().fl_wide_init(ctx.ctx, 64, KE) == 1
    x = gen.uniform(10, 3, (n, E), 2.0); fi = gen.uniform(10, 4, (n, E), 1.0)
    flw = _flw(dev, True)
    sels, wtss = [], []
    for r0 in range(0, n, 16):
        g = min(16, n - r0)
        s, w = _route(ctx, flw, x[r0:r0 + g].copy(), fi[r0:r0 + g].copy(), r0)
        sels.append(s); wtss.append(w)
    sel, wts = np.concatenate(sels), np.concatenate(wtss)
    used = sorted(set(sel.ravel().tolist()))
    byexp = {e: [] for e in used}
    for i in range(n):
        for k in range(KE):
            byexp[sel[i, k]].append((i, k))
    print("wide q3_K: %d experts, max %d pairs" % (len(used), max(len(v) for v in byexp.values())), flush=True)

    def batches():
        for bi, b0 in enumerate(range(0, len(used), EB)):
            batch = used[b0:b0 + EB]
            par = bi & 1
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
            ga, ua, da = _arena(dev, batch, orc.Q3K)
            lib().fl_wide_moe(ctx.ctx, ga.data_ptr(), ua.data_ptr(), da.data_ptr(), orc.Q3K, len(batch), cptr(np.int32(midx)),
                              cptr(np.int32(rows)), cptr(np.int32(kidx)), cptr(f32(wk)), len(midx), KE, par)
            lib().fl_wide_mark(ctx.ctx, par)
        out = FLOut()
        lib().fl_wide_finish(ctx.ctx, n, KE, ctypes.byref(out))
        return (np.ctypeslib.as_array(out.h, shape=(n * E,)).reshape(n, E).copy(),
                np.ctypeslib.as_array(out.moe, shape=(n * E,)).reshape(n, E).copy())

    h, moe = batches()   # the grouped GEMMs (about 20 pairs per expert)
    ctx.set_prefill_mfma(False)
    try:
        h_pp, moe_pp = batches()   # the per-pass kernels
    finally:
        ctx.set_prefill_mfma(True)
    assert np.array_equal(h.view(np.uint32), h_pp.view(np.uint32)) and np.array_equal(moe.view(np.uint32), moe_pp.view(np.uint32))
    ref = orc.moe_experts(x, sel, wts, host["gate"], host["up"], host["kdown"][orc.Q3K], *host["ksh"], want=("o", "sh"),
                          n_exp=16, fmts=(orc.Q3K, orc.Q5K, orc.Q5K, orc.Q6K))
    o = ref["o"].reshape(n, KE, E)
    m = np.zeros((n, E), np.float32)
    for k in range(KE):
        m = (m + wts[:, k:k + 1] * o[:, k]).astype(np.float32)
    ok, err = bar_close(moe, m)
    assert ok, err
    ok, err = bar_close(h, ((fi + ref["sh"]).astype(np.float32) + m).astype(np.float32))
    assert ok, err
    ctx.set_routing(8, 4, 8, 2.5)


def test_shared_formats_rejects(ctx):
    from loki_amd import lib, FL_EINVAL
    assert lib().fl_set_shared_formats(ctx.ctx, 3, 4, 1) == FL_EINVAL   # gate K-quant, up IQ2_XXS
    assert lib().fl_set_shared_formats(ctx.ctx, 0, 0, 1) == FL_EINVAL   # Q4_K is not supported
    ctx.set_shared_formats()


# (block bytes, offset of d, offset of dmin) of the ggml K-quant blocks
KQ_BLOCK = {orc.Q2K: (84, 80, 82), orc.Q3K: (110, 108, None), orc.Q5K: (176, 0, 2), orc.Q6K: (210, 208, None)}


def _kq_device(torch, fmt, R, K, seed):
    """random K-quant matrix bytes on the device: uniform quant and scale bytes, fp16 d (and dmin) in [6e-5, 4e-3]"""
    bs, od, om = KQ_BLOCK[fmt]
    nb = R * (K // 256)
    g = torch.Generator(device="cuda").manual_seed(seed)
    blk = torch.randint(0, 256, (nb, bs), dtype=torch.uint8, device="cuda", generator=g)
    for off in (od, om):
        if off is not None:
            d = torch.randint(0x0C00, 0x1C00, (nb,), dtype=torch.int32, device="cuda", generator=g).to(torch.int16)
            blk[:, off:off + 2] = d.view(torch.uint8).view(nb, 2)
    return blk.view(-1)


@pytest.mark.parametrize("down_fmt", [orc.Q2K, orc.Q3K], ids=["q2_K", "q3_K"])
def test_decode1_real_formats(ctx, down_fmt):
    """One decode token on the real shards' formats (routed gate/up IQ2_XXS tiled; routed down Q2_K / Q3_K and the
    shared expert Q5_K / Q5_K / Q6_K read in place) through the one-token kernel: y, picks and weights bit-identical to
    the per-pass kernels for tokens in a row, also under fl_moe_layer_normed with the residual; y against the checker
    within the K-quant bar. A 64-expert layer (the kernel's workgroups past the experts still run their shares)."""
    import torch
    from loki_amd import MoeLayerWeights
    from tests._helpers import make_x, host_matrix
    ne = 64
    base = MoeLayerWeights.synthetic(ctx, 8080 + down_fmt, n_exp=ne)
    down = _kq_device(torch, down_fmt, ne * E, H, 8090 + down_fmt)
    sh = (_kq_device(torch, orc.Q5K, H, E, 8091), _kq_device(torch, orc.Q5K, H, E, 8092), _kq_device(torch, orc.Q6K, E, H, 8093))
    layer = MoeLayerWeights(base.gate_inp, base.probs_b, base.gate, base.up, down, *sh, n_exp=ne)
    fm = (down_fmt, orc.Q5K, orc.Q5K, orc.Q6K)
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    mb = E * (H // 256) * KQ_BLOCK[down_fmt][0]
    ctx.set_layer_formats(*fm)
    try:
        for i in range(3):
            x = make_x(ctx, 1, seed=8100 + i)
            print("decode-1 real formats: down %s token %d" % (NAMES[down_fmt], i), flush=True)
            got = {}
            for name, m in (("decode1", 2), ("per_pass", 0)):
                with ctx.using_fused(m):
                    y = ctx.moe_layer(layer, x).clone()
                    ctx.sync()
                    dbg = ctx.debug()
                    assert dbg.kernel == {"decode1": 2, "per_pass": 0}[name], (name, dbg.kernel)
                    got[name] = (ctx.d2h(dbg.sel, (KE,), np.int32), ctx.d2h(dbg.wts, (KE,), np.float32), y.cpu().numpy())
                    if i == 0:
                        got[name] += (ctx.moe_layer_normed(layer, x * 3.0, None, 1e-6, residual=True).cpu().numpy(),)
                        ctx.sync()
                        assert ctx.debug().kernel == {"decode1": 2, "per_pass": 0}[name]
            for k in range(len(got["per_pass"])):
                assert np.array_equal(got["decode1"][k].view(np.uint8), got["per_pass"][k].view(np.uint8)), (i, k)
            xs = x.cpu().numpy()
            _, _, so, wo = orc.router(W, b, xs)
            assert np.array_equal(got["decode1"][0], so.ravel().astype(np.int32))
            sel = sorted(set(int(e) for e in so.ravel()))
            gate = {e: host_matrix(ctx, layer.expert_slice("gate", e), H, E) for e in sel}
            up = {e: host_matrix(ctx, layer.expert_slice("up", e), H, E) for e in sel}
            dn = {e: down[e * mb:(e + 1) * mb].cpu().numpy() for e in sel}
            ref = orc.moe_experts(xs, so, wo, gate, up, dn, *(m.cpu().numpy() for m in sh), n_exp=ne, fmts=fm)["y"]
            ok, err = bar_close(got["decode1"][2], ref)
            assert ok, (i, err)
    finally:
        ctx.set_layer_formats()
    del layer, base, down, sh
    torch.cuda.empty_cache()


DEC_FMTS = [(orc.Q3K, orc.Q5K, orc.Q5K, orc.Q6K), (4, orc.Q5K, orc.Q5K, orc.Q6K)]


@pytest.mark.parametrize("fm", DEC_FMTS, ids=["q3k_q5q5q6", "iq2_q5q5q6"])
def test_decode_batch_real_formats(ctx, fm):
    """fl_moe_layer on 2..8 rows with a K-quant shared expert (the per-pass kernels; the shared expert's mat-vecs run
    on a second stream beside the routed launches and the combine waits for them): calls of 8, 3 and 8 rows in a row
    give the first result again, bit for bit (each call's second-stream work is ordered after the previous call's
    combine), and equal the same calls with the shared expert on the context's stream (fl_set_debug bit 2); y against
    the checker within the parity bar at n = 8 and 3 (the Q5_K / Q6_K shared outputs differ from ggml's by fp32
    rounding, which the Q8_K of h can carry to a quantisation step). A 64-expert layer."""
    import torch
    from loki_amd import MoeLayerWeights
    from tests._helpers import make_x, host_matrix
    ne = 64
    seed = 8300 + 10 * DEC_FMTS.index(fm)
    base = MoeLayerWeights.synthetic(ctx, seed, n_exp=ne, bias_sigma=0.01)
    down = _kq_device(torch, fm[0], ne * E, H, seed + 1) if fm[0] != 4 else base.down
    sh = (_kq_device(torch, fm[1], H, E, seed + 2), _kq_device(torch, fm[2], H, E, seed + 3), _kq_device(torch, fm[3], E, H, seed + 4))
    layer = MoeLayerWeights(base.gate_inp, base.probs_b, base.gate, base.up, down, *sh, n_exp=ne)
    x8, x3 = make_x(ctx, 8, seed=seed + 5), make_x(ctx, 3, seed=seed + 6)
    ctx.set_layer_formats(*fm)
    try:
        print("decode batch real formats %s: n 8, 3, 8" % (fm,), flush=True)
        y8 = ctx.moe_layer(layer, x8).clone()
        y3 = ctx.moe_layer(layer, x3).clone()
        y8b = ctx.moe_layer(layer, x8).clone()
        ctx.sync()
        assert ctx.debug().kernel == 0
        print("decode batch real formats %s: shared expert on the context's stream" % (fm,), flush=True)
        ctx.set_debug(False, shared_on_stream=True)
        y8s = ctx.moe_layer(layer, x8).clone()
        y3s = ctx.moe_layer(layer, x3).clone()
        ctx.sync()
    finally:
        ctx.set_debug(False); ctx.set_layer_formats()
    for a_, b_ in ((y8, y8b), (y8, y8s), (y3, y3s)):
        assert np.array_equal(a_.cpu().numpy().view(np.uint8), b_.cpu().numpy().view(np.uint8))
    W, b = layer.gate_inp.cpu().numpy(), layer.probs_b.cpu().numpy()
    for x, y in ((x8, y8), (x3, y3)):
        xs = x.cpu().numpy()
        _, _, so, wo = orc.router(W, b, xs)
        sel = sorted(set(int(e) for e in so.ravel()))
        gate = {e: host_matrix(ctx, layer.expert_slice("gate", e), H, E) for e in sel}
        up = {e: host_matrix(ctx, layer.expert_slice("up", e), H, E) for e in sel}
        if fm[0] == 4:
            dn = {e: host_matrix(ctx, layer.expert_slice("down", e), E, H) for e in sel}
        else:
            mb = E * (H // 256) * KQ_BLOCK[fm[0]][0]
            dn = {e: down[e * mb:(e + 1) * mb].cpu().numpy() for e in sel}
        ref = orc.moe_experts(xs, so, wo, gate, up, dn, *(m.cpu().numpy() for m in sh), n_exp=ne, fmts=fm)["y"]
        ok, err = bar_close(y.cpu().numpy(), ref, l2=2e-3, mx=1e-2)
        assert ok, (x.shape[0], err)
    del layer, base, down, sh
    torch.cuda.empty_cache()


# (routed down, shared gate, up, down): the real shards'; a K-quant routed down with the shared expert in IQ2_XXS (GEMM
# columns); a K-quant shared expert beside an IQ2_XXS routed down (the down GEMM); an IQ2_XXS shared gate/up with a
# Q6_K shared down (the shared gate/up on the per-pass kernel)
PF_FMTS = [(orc.Q3K, orc.Q5K, orc.Q5K, orc.Q6K), (orc.Q2K, 4, 4, 4), (4, orc.Q5K, orc.Q5K, orc.Q6K), (4, 4, 4, orc.Q6K)]


@pytest.mark.parametrize("n", [40, 512])
@pytest.mark.parametrize("fm", PF_FMTS, ids=["q3k_q5q5q6", "q2k_iq2", "iq2_q5q5q6", "iq2_iq2iq2q6"])
def test_prefill_mixed_formats_mfma(ctx, fm, n):
    """fl_moe_layer at prefill sizes with K-quant matrices: the routed gate/up on the MFMA GEMM (the shared expert's
    columns only when all of it is IQ2_XXS) and the K-quant matrices on their mat-vecs give g, u, h and its Q8_K, o and
    y bit-identical to the per-pass kernels (fl_set_prefill_mfma(0)). A 64-expert layer; the real shards' formats are
    also checked against the CPU checker on sampled rows."""
    import torch
    from loki_amd import MoeLayerWeights
    from tests._helpers import make_x, host_matrix
    ne = 64
    seed = 8200 + 10 * PF_FMTS.index(fm)
    base = MoeLayerWeights.synthetic(ctx, seed, n_exp=ne, bias_sigma=0.05)
    down = _kq_device(torch, fm[0], ne * E, H, seed + 1) if fm[0] != 4 else base.down
    shg = _kq_device(torch, fm[1], H, E, seed + 2) if fm[1] != 4 else base.sh_gate
    shu = _kq_device(torch, fm[2], H, E, seed + 3) if fm[2] != 4 else base.sh_up
    shd = _kq_device(torch, fm[3], E, H, seed + 4) if fm[3] != 4 else base.sh_down
    layer = MoeLayerWeights(base.gate_inp, base.probs_b, base.gate, base.up, down, shg, shu, shd, n_exp=ne)
    x = make_x(ctx, n, seed=seed + 5)
    ctx.set_layer_formats(*fm)
    got = {}
    try:
        for mfma in (True, False):
            print("prefill mixed formats %s n %d mfma %d" % (fm, n, mfma), flush=True)
            ctx.set_prefill_mfma(mfma)
            ctx.set_debug(True)
            y = ctx.moe_layer(layer, x).clone()
            ctx.sync()
            d = ctx.debug()
            P = d.P
            got[mfma] = {"y": y.cpu().numpy(), "h": ctx.d2h(d.h, (P + n, H), np.float32), "o": ctx.d2h(d.o, (P + n, E), np.float32),
                         "g": ctx.d2h(d.g, (P + n, H), np.float32), "u": ctx.d2h(d.u, (P + n, H), np.float32),
                         "hd": ctx.d2h(d.hd, (P + n, H // 256), np.float32), "hq": ctx.d2h(d.hq, (P + n, H), np.int8),
                         "sel": ctx.d2h(d.sel, (n, KE), np.int32), "wts": ctx.d2h(d.wts, (n, KE), np.float32)}
            ctx.set_debug(False)
    finally:
        ctx.set_debug(False); ctx.set_prefill_mfma(True); ctx.set_layer_formats()
    for k in got[False]:
        assert np.array_equal(got[True][k].view(np.uint8), got[False][k].view(np.uint8)), k
    if fm == PF_FMTS[0]:   # sampled rows against the checker
        rows = np.array([0, 1, n // 2, n - 1])
        xs = x.cpu().numpy()[rows]
        so, wo = got[True]["sel"][rows], got[True]["wts"][rows]
        sel = sorted(set(int(e) for e in so.ravel()))
        mb = E * (H // 256) * KQ_BLOCK[fm[0]][0]
        gate = {e: host_matrix(ctx, layer.expert_slice("gate", e), H, E) for e in sel}
        up = {e: host_matrix(ctx, layer.expert_slice("up", e), H, E) for e in sel}
        dn = {e: down[e * mb:(e + 1) * mb].cpu().numpy() for e in sel}
        ref = orc.moe_experts(xs, so, wo, gate, up, dn, shg.cpu().numpy(), shu.cpu().numpy(), shd.cpu().numpy(), n_exp=ne, fmts=fm)["y"]
        ok, err = bar_close(got[True]["y"][rows], ref)
        assert ok, err
    del layer, base, down, shg, shu, shd
    torch.cuda.empty_cache()
