"""TEST INFRASTRUCTURE ONLY -- numpy/ctypes front of the C oracle (oracle/moe_oracle.c).

The oracle restates ggml's CPU semantics for the DeepSeek-R1 MoE block (see moe_oracle.c's header for the
reference file:line each function follows). Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg may import this module; the product (loki_amd) never does.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

QK_K = 256
IQ2_BYTES = 66


def build(force=False):
    """Compile liboracle.so with the committed Makefile (gcc, -ffp-contract=off)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "-q", "-C", _HERE], check=False)
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P, I64, I, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float
        L.or_fp16_to_fp32.restype = F; L.or_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.or_fp32_to_fp16.restype = ctypes.c_uint16; L.or_fp32_to_fp16.argtypes = [F]
        L.or_expf.restype = F; L.or_expf.argtypes = [F]
        L.or_silu.restype = F; L.or_silu.argtypes = [F]
        L.or_sigmoid.restype = F; L.or_sigmoid.argtypes = [F]
        L.or_quantize_row_q8_K.restype = None; L.or_quantize_row_q8_K.argtypes = [P, P, P, P, I64]
        L.or_dequantize_row_iq2_xxs.restype = None; L.or_dequantize_row_iq2_xxs.argtypes = [P, P, I64]
        L.or_vec_dot_iq2_xxs_q8_K.restype = F; L.or_vec_dot_iq2_xxs_q8_K.argtypes = [I64, P, P, P]
        L.or_matvec_iq2_xxs.restype = None; L.or_matvec_iq2_xxs.argtypes = [P, I64, I64, P, P, P]
        L.or_kq_block_bytes.restype = ctypes.c_int; L.or_kq_block_bytes.argtypes = [ctypes.c_int]
        L.or_dequantize_row_kq.restype = None; L.or_dequantize_row_kq.argtypes = [ctypes.c_int, P, P, I64]
        L.or_vec_dot_kq_q8_K.restype = ctypes.c_float; L.or_vec_dot_kq_q8_K.argtypes = [ctypes.c_int, I64, P, P, P, P]
        L.or_matvec_kq.restype = None; L.or_matvec_kq.argtypes = [ctypes.c_int, P, I64, I64, P, P, P, I64, P]
        L.or_router_logit.restype = F; L.or_router_logit.argtypes = [P, P, I64]
        L.or_router.restype = I; L.or_router.argtypes = [P, P, P, I64, I, I64, I, I, I, F, P, P, P, P]
        L.or_dispatch.restype = I; L.or_dispatch.argtypes = [P, I64, I, I, P, P, P]
        L.or_keep_experts.restype = I; L.or_keep_experts.argtypes = [P, P, I64, I, I, F, I64, P, P]
        L.or_keep_experts_share.restype = I; L.or_keep_experts_share.argtypes = [P, P, I64, I, I, F, I64, I, P, P]
        L.or_moe_forward.restype = I
        L.or_moe_forward.argtypes = [P, I64, I64, I64, P, P, I, I, I, I, F, P, P, P, P, P, P, P, P, P, P, P, P, P, I]
        L.or_moe_experts.restype = I
        L.or_moe_experts.argtypes = [P, I64, I64, I64, I, P, P, P, P, P, P, P, P, P, P, P, P, P, I]
        L.or_moe_experts_fmt.restype = I
        L.or_moe_experts_fmt.argtypes = [P, I64, I64, I64, I, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I]
        L.or_rmsnorm.restype = None; L.or_rmsnorm.argtypes = [P, P, P, I64, I64, F]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---------------------------------------------------------------- scalars
def fp16_to_fp32(h):
    h = np.asarray(h, dtype=np.uint16).ravel()
    return np.array([lib().or_fp16_to_fp32(int(v)) for v in h], dtype=np.float32)


def fp32_to_fp16(f):
    f = np.asarray(f, dtype=np.float32).ravel()
    return np.array([lib().or_fp32_to_fp16(float(v)) for v in f], dtype=np.uint16)


def expf(x):
    x = np.asarray(x, dtype=np.float32).ravel()
    return np.array([lib().or_expf(float(v)) for v in x], dtype=np.float32)


def silu(x):
    x = np.asarray(x, dtype=np.float32).ravel()
    return np.array([lib().or_silu(float(v)) for v in x], dtype=np.float32)


def sigmoid(x):
    x = np.asarray(x, dtype=np.float32).ravel()
    return np.array([lib().or_sigmoid(float(v)) for v in x], dtype=np.float32)


# ---------------------------------------------------------------- formats
def quantize_q8k(x):
    """x [..., K] fp32 -> (q int8 [..., K], d fp32 [..., K/256], bsums int16 [..., K/16])."""
    x = _c(x, np.float32)
    K = x.shape[-1]
    rows = x.reshape(-1, K)
    q = np.empty(rows.shape, np.int8); d = np.empty((rows.shape[0], K // QK_K), np.float32)
    bs = np.empty((rows.shape[0], K // 16), np.int16)
    for i in range(rows.shape[0]):
        lib().or_quantize_row_q8_K(_p(rows[i]), _p(q[i]), _p(d[i]), _p(bs[i]), K)
    return q.reshape(x.shape), d.reshape(x.shape[:-1] + (K // QK_K,)), bs.reshape(x.shape[:-1] + (K // 16,))


# K-quant formats (kquant_oracle.c): the FL_* codes of include/loki_moe.h
Q2K, Q3K, Q5K, Q6K = 5, 6, 3, 1


def kq_block_bytes(fmt):
    return lib().or_kq_block_bytes(fmt)


def dequant_kq(fmt, blocks, K):
    """blocks uint8 [rows, K/256*bytes] -> fp32 [rows, K] (dequantize_row_q*_K)."""
    b = _c(blocks, np.uint8).reshape(-1, K // QK_K * kq_block_bytes(fmt))
    y = np.empty((b.shape[0], K), np.float32)
    for i in range(b.shape[0]):
        lib().or_dequantize_row_kq(fmt, _p(b[i]), _p(y[i]), K)
    return y


def vec_dot_kq(fmt, row_blocks, q, d, bsums):
    """ggml_vec_dot_q*_K_q8_K of one row (blocks) with one Q8_K row (q, d, bsums)."""
    K = q.shape[-1]
    return float(lib().or_vec_dot_kq_q8_K(fmt, K, _p(_c(row_blocks, np.uint8)), _p(_c(q, np.int8)), _p(_c(d, np.float32)),
                                           _p(_c(bsums, np.int16))))


def matvec_kq(fmt, w, rows, K, q, d, bsums):
    """y [nt, rows] = w (rows x K, ggml layout) . Q8_K rows (q [nt, K], d [nt, K/256], bsums [nt, K/16])."""
    q = _c(q, np.int8).reshape(-1, K); nt = q.shape[0]
    y = np.empty((nt, rows), np.float32)
    lib().or_matvec_kq(fmt, _p(_c(w, np.uint8)), rows, K, _p(q), _p(_c(d, np.float32)), _p(_c(bsums, np.int16)), nt, _p(y))
    return y


def dequant_iq2xxs(blocks, K):
    """blocks uint8 [rows, K/256*66] -> fp32 [rows, K]."""
    b = _c(blocks, np.uint8).reshape(-1, K // QK_K * IQ2_BYTES)
    y = np.empty((b.shape[0], K), np.float32)
    for i in range(b.shape[0]):
        lib().or_dequantize_row_iq2_xxs(_p(b[i]), _p(y[i]), K)
    return y


def vec_dot(wrow, q, d):
    wrow = _c(wrow, np.uint8); q = _c(q, np.int8); d = _c(d, np.float32)
    return lib().or_vec_dot_iq2_xxs_q8_K(q.shape[-1], _p(wrow), _p(q), _p(d))


def matvec(w, rows, K, q, d):
    w = _c(w, np.uint8); q = _c(q, np.int8); d = _c(d, np.float32)
    y = np.empty(rows, np.float32)
    lib().or_matvec_iq2_xxs(_p(w), rows, K, _p(q), _p(d), _p(y))
    return y


# ---------------------------------------------------------------- router / dispatch
def router_logit(w, x):
    w = _c(w, np.float32); x = _c(x, np.float32)
    return lib().or_router_logit(_p(w), _p(x), x.shape[-1])


def router(W, bias, x, n_group=8, topk_group=4, topk=8, scale=2.5):
    W = _c(W, np.float32); bias = _c(bias, np.float32); x = _c(x, np.float32).reshape(-1, W.shape[1])
    n, n_exp, K = x.shape[0], W.shape[0], W.shape[1]
    logits = np.empty((n, n_exp), np.float32); probs = np.empty((n, n_exp), np.float32)
    sel = np.empty((n, topk), np.int32); wts = np.empty((n, topk), np.float32)
    rc = lib().or_router(_p(W), _p(bias), _p(x), n, n_exp, K, n_group, topk_group, topk, scale,
                         _p(logits), _p(probs), _p(sel), _p(wts))
    if rc != 0:
        raise ValueError("oracle router rejected its arguments (%d)" % rc)
    return logits, probs, sel, wts


def keep_experts(sel, w, ke, renorm=2.5, n_pad=None, share=False):
    """The engine's keep-KE (src/server_core_fused.cpp:793-815): per row the ke heaviest experts (stable, weight
    descending), rescaled to sum to renorm (<= 0: off); rows >= n_pad take row 0's kept experts at weight 0. share:
    the --share-experts rule (:798-806) for n > 1."""
    sel = _c(sel, np.int32); w = _c(w, np.float32)
    n, topk = sel.shape
    so = np.empty((n, ke), np.int32); wo = np.empty((n, ke), np.float32)
    rc = lib().or_keep_experts_share(_p(sel), _p(w), n, topk, ke, renorm, n if n_pad is None else n_pad, 1 if share else 0,
                                     _p(so), _p(wo))
    if rc != 0:
        raise ValueError("oracle keep_experts failed (%d)" % rc)
    return so, wo


def dispatch(sel, n_exp=256):
    sel = _c(sel, np.int32)
    n, topk = sel.shape
    counts = np.empty(n_exp, np.int32); offsets = np.empty(n_exp + 1, np.int32); perm = np.empty(n * topk, np.int32)
    rc = lib().or_dispatch(_p(sel), n, topk, n_exp, _p(counts), _p(offsets), _p(perm))
    if rc != 0:
        raise ValueError("oracle dispatch failed (%d)" % rc)
    return counts, offsets, perm


# ---------------------------------------------------------------- block
def _ptr_array(mats, n_exp):
    arr = (ctypes.c_void_p * n_exp)()
    keep = []
    for e in range(n_exp):
        m = mats.get(e) if isinstance(mats, dict) else mats[e]
        if m is None:
            arr[e] = None
        else:
            m = _c(m, np.uint8); keep.append(m); arr[e] = m.ctypes.data
    return arr, keep


def moe_forward(x, W, bias, gate, up, down, sh_gate, sh_up, sh_down, n_group=8, topk_group=4, topk=8,
                scale=2.5, H=2048, want=(), nthreads=0):
    """Whole block. gate/up/down: list or dict expert -> uint8 matrix in ggml layout (None where unused).
    Returns dict with y, sel, wts and any of g/u/o/sh named in `want`."""
    x = _c(x, np.float32); n, E = x.shape
    W = _c(W, np.float32); bias = _c(bias, np.float32); n_exp = W.shape[0]
    y = np.empty((n, E), np.float32); sel = np.empty((n, topk), np.int32); wts = np.empty((n, topk), np.float32)
    P = n * topk
    out = {k: np.empty(s, np.float32) for k, s in
           (("g", (P, H)), ("u", (P, H)), ("o", (P, E)), ("sh", (n, E))) if k in want}
    ga, k1 = _ptr_array(gate, n_exp); ua, k2 = _ptr_array(up, n_exp); da, k3 = _ptr_array(down, n_exp)
    sg, su, sd = _c(sh_gate, np.uint8), _c(sh_up, np.uint8), _c(sh_down, np.uint8)
    rc = lib().or_moe_forward(_p(x), n, E, H, _p(W), _p(bias), n_exp, n_group, topk_group, topk, scale,
                              ga, ua, da, _p(sg), _p(su), _p(sd), _p(y), _p(sel), _p(wts),
                              _p(out.get("g")), _p(out.get("u")), _p(out.get("o")), _p(out.get("sh")), nthreads)
    if rc != 0:
        raise ValueError("oracle moe_forward failed (%d)" % rc)
    out.update(y=y, sel=sel, wts=wts)
    return out


def moe_experts(x, sel, wts, gate, up, down, sh_gate, sh_up, sh_down, H=2048, want=(), nthreads=0, n_exp=256, fmts=None):
    """Experts on given routing. fmts = (routed down, shared gate, shared up, shared down) format codes (IQ2 = 4 or a
    K-quant); None = IQ2_XXS everywhere."""
    x = _c(x, np.float32); n, E = x.shape
    sel = _c(sel, np.int32); wts = _c(wts, np.float32); topk = sel.shape[1]
    y = np.empty((n, E), np.float32); P = n * topk
    out = {k: np.empty(s, np.float32) for k, s in
           (("g", (P, H)), ("u", (P, H)), ("o", (P, E)), ("sh", (n, E))) if k in want}
    ga, k1 = _ptr_array(gate, n_exp); ua, k2 = _ptr_array(up, n_exp); da, k3 = _ptr_array(down, n_exp)
    sg, su, sd = _c(sh_gate, np.uint8), _c(sh_up, np.uint8), _c(sh_down, np.uint8)
    fm = None if fmts is None else np.ascontiguousarray(fmts, np.int32)
    rc = lib().or_moe_experts_fmt(_p(x), n, E, H, topk, _p(sel), _p(wts), ga, ua, da, _p(sg), _p(su), _p(sd), _p(fm), _p(y),
                                  _p(out.get("g")), _p(out.get("u")), _p(out.get("o")), _p(out.get("sh")), nthreads)
    if rc != 0:
        raise ValueError("oracle moe_experts failed (%d)" % rc)
    out["y"] = y
    return out


def rmsnorm(x, w=None, eps=1e-6):
    x = _c(x, np.float32); n, d = x.reshape(-1, x.shape[-1]).shape
    y = np.empty_like(x)
    lib().or_rmsnorm(_p(x), _p(None if w is None else _c(w, np.float32)), _p(y), n, d, eps)
    return y
