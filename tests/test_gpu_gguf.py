"""GPU: MoE layers loaded from GGUF shards (fl_gguf_load_moe_layer) into HBM and run.
- tiled layout: the layer of the committed golden vector written as a GGUF file runs through fl_moe_layer bit-identical
  to the golden output;
- ggml layout with the real shards' formats (Q3_K routed down, Q5_K / Q5_K / Q6_K shared expert, F16 router as the
  reference's ffn_gate_inp_f16 sidecar): fl_ffn_begin / fl_fetch / fl_moe with the loaded layer as the arena, against
  the checker (tolerances as tests/test_gpu_kquant.py)."""
import ctypes
import os

import numpy as np
import pytest

from oracle import oracle as orc
from tests import _gguf
from tests.golden import gen

pytestmark = pytest.mark.gpu

E, H, NE, KE = 7168, 2048, 16, 8
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def layer_tensors(L, W, b, gate, up, down, sh, types, norm=None, router="F32"):
    p = "blk.%d." % L
    rt = W.astype(np.float16) if router == "F16" else W
    t = [(p + ("ffn_gate_inp_f16.weight" if router == "F16" else "ffn_gate_inp.weight"), router, [E, NE], rt.view(np.uint8).reshape(-1)),
         (p + "exp_probs_b.bias", "F32", [NE], b.view(np.uint8)),
         (p + "ffn_gate_exps.weight", types[0], [E, H, NE], np.concatenate(gate)),
         (p + "ffn_up_exps.weight", types[1], [E, H, NE], np.concatenate(up)),
         (p + "ffn_down_exps.weight", types[2], [H, E, NE], np.concatenate(down)),
         (p + "ffn_gate_shexp.weight", types[3], [E, H], sh[0]),
         (p + "ffn_up_shexp.weight", types[4], [E, H], sh[1]),
         (p + "ffn_down_shexp.weight", types[5], [H, E], sh[2])]
    if norm is not None:
        t.append((p + "ffn_norm.weight", "F32", [E], norm.view(np.uint8)))
    return t


def test_gguf_layer_tiled_golden(ctx, tmp_path):
    import torch
    from loki_amd import Gguf, lib, FL_LAYOUT_TILED
    z = np.load(os.path.join(GOLDEN, "decode_full.npz"), allow_pickle=False)
    W, b, gate, up, down, sh = gen.layer(202, NE, E, H)
    norm = gen.uniform(5, 1, (E,), 1.0)
    path = str(tmp_path / "layer3.gguf")
    _gguf.write(path, layer_tensors(3, W, b, gate, up, down, sh, ["IQ2_XXS"] * 6, norm=norm),
                [("general.architecture", "str", "deepseek2")])
    print("gguf tiled layer: %d bytes" % os.path.getsize(path), flush=True)
    g = Gguf(path)
    gl = ctx.load_gguf_layer(g, 3, FL_LAYOUT_TILED)
    try:
        assert gl.L.n_exp == NE and gl.L.E == E and gl.L.H == H and gl.L.layout == FL_LAYOUT_TILED
        assert gl.expert_stride[0] == H * (E // 256) * 66 and gl.expert_stride[2] == E * (H // 256) * 66
        assert gl.ffn_norm
        nrm = np.empty(E, np.float32); ctx.check(lib().fl_d2h(ctx.ctx, nrm.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(gl.ffn_norm), E * 4))
        assert np.array_equal(nrm, norm)
        x = torch.from_numpy(z["x"]).cuda()
        y = torch.empty_like(x)
        ctx.check(lib().fl_moe_layer(ctx.ctx, ctypes.byref(gl.L), ctypes.c_void_p(x.data_ptr()), x.shape[0], ctypes.c_void_p(y.data_ptr())))
        ctx.sync()
        assert np.array_equal(y.cpu().numpy().view(np.uint32), z["y"].view(np.uint32))
    finally:
        ctx.free_gguf_layer(gl)
        g.close()


def test_gguf_layer_ggml_real_formats(ctx, tmp_path):
    """a real-shard layer: the loaded layer is the fl_moe arena (ids = expert ids, nexp = all experts)"""
    from loki_amd import FLOut, FLW, Gguf, lib, FL_LAYOUT_GGML
    W, b, gate, up, _, _ = gen.layer(202, NE, E, H)
    down = [gen.kq_matrix(203, 40 + e, orc.Q3K, E, H) for e in range(NE)]
    ksh = (gen.kq_matrix(204, 1, orc.Q5K, H, E), gen.kq_matrix(204, 2, orc.Q5K, H, E), gen.kq_matrix(204, 3, orc.Q6K, E, H))
    path = str(tmp_path / "layer7.gguf")
    _gguf.write(path, layer_tensors(7, W, b, gate, up, down, ksh, ["IQ2_XXS", "IQ2_XXS", "Q3_K", "Q5_K", "Q5_K", "Q6_K"], router="F16"))
    print("gguf ggml layer: %d bytes" % os.path.getsize(path), flush=True)
    g = Gguf(path)
    gl = ctx.load_gguf_layer(g, 7, FL_LAYOUT_GGML)
    try:
        assert (gl.fmt_down, gl.fmt_sh_gate, gl.fmt_sh_up, gl.fmt_sh_down) == (orc.Q3K, orc.Q5K, orc.Q5K, orc.Q6K)
        assert not gl.ffn_norm
        ctx.set_experts(NE); ctx.set_routing(8, 4, 8, 2.5)
        ctx.set_shared_formats(gl.fmt_sh_gate, gl.fmt_sh_up, gl.fmt_sh_down)
        flw = FLW()
        flw.gate_inp = gl.L.gate_inp; flw.probs_b = gl.L.probs_b   # F32 after loading (the F16 file widened exactly)
        flw.sh_gate, flw.sh_up, flw.sh_down = gl.L.sh_gate, gl.L.sh_up, gl.L.sh_down
        flw.gate_f16 = 0
        n = 4
        x = gen.uniform(11, 3, (n, E), 2.0); fi = gen.uniform(11, 4, (n, E), 1.0)
        ctx.check(lib().fl_ffn_begin(ctx.ctx, ctypes.byref(flw), n, x.ctypes.data_as(ctypes.c_void_p), fi.ctypes.data_as(ctypes.c_void_p), -1))
        out = FLOut()
        lib().fl_fetch(ctx.ctx, n, 1, ctypes.byref(out))
        sel = np.ctypeslib.as_array(out.sel, shape=(n * KE,)).reshape(n, KE).copy()
        wts = np.ctypeslib.as_array(out.wts, shape=(n * KE,)).reshape(n, KE).copy()
        W16 = W.astype(np.float16).astype(np.float32)
        _, _, so, wo = orc.router(W16, b, x, 8, 4, 8, 2.5)
        assert np.array_equal(sel, so) and np.array_equal(wts.view(np.uint32), wo.view(np.uint32))
        lib().fl_moe(ctx.ctx, ctypes.c_void_p(gl.L.gate_exps), ctypes.c_void_p(gl.L.up_exps), ctypes.c_void_p(gl.L.down_exps), NE,
                     gl.fmt_down, sel.ctypes.data_as(ctypes.c_void_p), wts.ctypes.data_as(ctypes.c_void_p), KE, n, ctypes.byref(out))
        h = np.ctypeslib.as_array(out.h, shape=(n * E,)).reshape(n, E).copy()
        ref = orc.moe_experts(x, so, wo, gate, up, down, *ksh, want=("o", "sh"), n_exp=NE, fmts=(orc.Q3K, orc.Q5K, orc.Q5K, orc.Q6K))
        want = (ref["y"] + fi).astype(np.float32)
        d = h.astype(np.float64) - want
        e_l2 = np.linalg.norm(d) / np.linalg.norm(want.astype(np.float64))
        e_mx = np.abs(d).max() / np.abs(want).max()
        assert e_l2 <= 1e-4 and e_mx <= 1e-3, (e_l2, e_mx)
    finally:
        ctx.set_shared_formats(); ctx.set_experts()
        ctx.free_gguf_layer(gl)
        g.close()


def test_gguf_layer_real_formats_device_resident(ctx, tmp_path):
    """a real-shard layer loaded tiled (IQ2_XXS gate/up packed, Q2_K down and Q5_K / Q5_K / Q6_K shared as stored) runs
    on the device with no host round trip: fl_moe_layer at a decode size and fl_moe_layer_normed (ffn_norm from the
    file, residual added) at a prefill size, against the checker; routing bit-identical"""
    import torch
    from loki_amd import Gguf, lib, FL_LAYOUT_TILED
    W, b, gate, up, _, _ = gen.layer(206, NE, E, H)
    down = [gen.kq_matrix(207, e, orc.Q2K, E, H) for e in range(NE)]
    ksh = (gen.kq_matrix(208, 1, orc.Q5K, H, E), gen.kq_matrix(208, 2, orc.Q5K, H, E), gen.kq_matrix(208, 3, orc.Q6K, E, H))
    norm = gen.uniform(208, 4, (E,), 1.0) + np.float32(1.0)
    path = str(tmp_path / "layer9.gguf")
    _gguf.write(path, layer_tensors(9, W, b, gate, up, down, ksh, ["IQ2_XXS", "IQ2_XXS", "Q2_K", "Q5_K", "Q5_K", "Q6_K"], norm=norm))
    g = Gguf(path)
    gl = ctx.load_gguf_layer(g, 9, FL_LAYOUT_TILED)
    fm = (orc.Q2K, orc.Q5K, orc.Q5K, orc.Q6K)
    try:
        assert (gl.fmt_down, gl.fmt_sh_gate, gl.fmt_sh_up, gl.fmt_sh_down) == fm
        ctx.set_experts(NE); ctx.set_routing(8, 4, 8, 2.5)
        ctx.set_layer_formats(*fm)
        for n, normed in ((5, False), (40, True)):
            print("device-resident real formats: n %d normed %d" % (n, normed), flush=True)
            x = gen.uniform(12, n, (n, E), 2.0)
            xt = torch.from_numpy(x).cuda(); y = torch.empty_like(xt)
            if normed:
                ctx.check(lib().fl_moe_layer_normed(ctx.ctx, ctypes.byref(gl.L), ctypes.c_void_p(gl.ffn_norm), ctypes.c_float(1e-6),
                                                    ctypes.c_void_p(xt.data_ptr()), n, 1, ctypes.c_void_p(y.data_ptr())))
                xin = orc.rmsnorm(x, norm, 1e-6)
            else:
                ctx.check(lib().fl_moe_layer(ctx.ctx, ctypes.byref(gl.L), ctypes.c_void_p(xt.data_ptr()), n, ctypes.c_void_p(y.data_ptr())))
                xin = x
            ctx.sync()
            dbg = ctx.debug()
            _, _, so, wo = orc.router(W, b, xin, 8, 4, 8, 2.5)
            assert np.array_equal(ctx.d2h(dbg.sel, (n, KE), np.int32), so)
            ref = orc.moe_experts(xin, so, wo, gate, up, down, *ksh, n_exp=NE, fmts=fm)["y"]
            if normed:
                ref = (ref + x).astype(np.float32)
            got = y.cpu().numpy().astype(np.float64)
            e_l2 = np.linalg.norm(got - ref) / np.linalg.norm(ref.astype(np.float64))
            e_mx = np.abs(got - ref).max() / np.abs(ref).max()
            assert e_l2 <= 1e-4 and e_mx <= 1e-3, (n, e_l2, e_mx)
    finally:
        ctx.set_layer_formats(); ctx.set_experts()
        ctx.free_gguf_layer(gl)
        g.close()


def test_gguf_layer_rejects(ctx, tmp_path):
    """an absent layer and a routed gate in a K-quant come back as error codes"""
    from loki_amd import Gguf, LokiError, FL_LAYOUT_TILED
    W, b, gate, up, down, sh = gen.layer(203, NE, E, H)
    gate_q2 = [gen.kq_matrix(205, e, orc.Q2K, H, E) for e in range(NE)]
    path = str(tmp_path / "l.gguf")
    _gguf.write(path, layer_tensors(5, W, b, gate_q2, up, down, sh, ["Q2_K", "IQ2_XXS", "IQ2_XXS", "IQ2_XXS", "IQ2_XXS", "IQ2_XXS"]))
    g = Gguf(path)
    with pytest.raises(LokiError):
        ctx.load_gguf_layer(g, 5, FL_LAYOUT_TILED)
    with pytest.raises(LokiError):
        ctx.load_gguf_layer(g, 6, FL_LAYOUT_TILED)
    g.close()
