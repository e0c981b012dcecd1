"""loki_amd -- MI355X (gfx950) DeepSeek-R1 MoE feed-forward block behind loki's fused_layer C ABI.

The product is libloki_moe.so (HIP kernels + the C ABI declared in include/loki_moe.h). This module is the host-side
mirror used by tests and bench: ctypes bindings of that ABI, plus helpers that allocate device memory through torch
(plumbing only; every computation runs in the library's HIP kernels). There is no CPU fallback: without the built
library every entry point raises.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_lib", "libloki_moe.so")

E_HIDDEN = 7168       # DeepSeek-R1 hidden size
H_EXPERT = 2048       # expert intermediate size
N_EXPERT = 256        # routed experts per layer
QK_K = 256
IQ2_BYTES = 66

FL_IQ2 = 4
FL_Q6K, FL_Q5K, FL_Q2K, FL_Q3K = 1, 3, 5, 6
KQ_BYTES = {FL_Q2K: 84, FL_Q3K: 110, FL_Q5K: 176, FL_Q6K: 210}
FL_LAYOUT_GGML, FL_LAYOUT_TILED = 0, 1
FL_OK, FL_EINVAL, FL_ENOMEM, FL_EHIP, FL_ERANGE, FL_ESCOPE = 0, -1, -2, -3, -4, -5

P_ = ctypes.c_void_p


class FLMoeLayer(ctypes.Structure):
    _fields_ = [("gate_inp", P_), ("probs_b", P_), ("gate_exps", P_), ("up_exps", P_), ("down_exps", P_),
                ("sh_gate", P_), ("sh_up", P_), ("sh_down", P_), ("layout", ctypes.c_int), ("n_exp", ctypes.c_int),
                ("E", ctypes.c_int), ("H", ctypes.c_int)]


class FLGgufTensor(ctypes.Structure):
    _fields_ = [("file", ctypes.c_int), ("type", ctypes.c_int), ("fl_format", ctypes.c_int), ("n_dims", ctypes.c_int),
                ("ne", ctypes.c_int64 * 4), ("offset", ctypes.c_uint64), ("nbytes", ctypes.c_uint64), ("row_bytes", ctypes.c_uint64)]


class FLGgufLayer(ctypes.Structure):
    _fields_ = [("L", FLMoeLayer), ("ffn_norm", P_), ("fmt_down", ctypes.c_int), ("fmt_sh_gate", ctypes.c_int),
                ("fmt_sh_up", ctypes.c_int), ("fmt_sh_down", ctypes.c_int), ("expert_stride", ctypes.c_uint64 * 3),
                ("mem", P_), ("bytes", ctypes.c_size_t)]


class Gguf:
    """Tensor index over GGUF shard files (libloki_moe's native reader; host only)."""

    def __init__(self, paths):
        if isinstance(paths, (str, bytes, os.PathLike)):
            paths = [paths]
        arr = (ctypes.c_char_p * len(paths))(*[os.fsencode(p) for p in paths])
        err = ctypes.create_string_buffer(512)
        self.h = lib().fl_gguf_open(arr, len(paths), err, 512)
        if not self.h:
            raise LokiError("fl_gguf_open: " + err.value.decode(errors="replace"))

    def close(self):
        if self.h:
            lib().fl_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def names(self):
        return [lib().fl_gguf_tensor_name(self.h, i).decode() for i in range(lib().fl_gguf_n_tensors(self.h))]

    def tensor(self, name):
        t = FLGgufTensor()
        rc = lib().fl_gguf_tensor(self.h, name.encode(), ctypes.byref(t))
        if rc != FL_OK:
            raise KeyError(name)
        return t

    def get_int(self, key):
        v = ctypes.c_int64()
        rc = lib().fl_gguf_get_int(self.h, key.encode(), ctypes.byref(v))
        return v.value if rc == FL_OK else None

    def get_float(self, key):
        v = ctypes.c_double()
        rc = lib().fl_gguf_get_float(self.h, key.encode(), ctypes.byref(v))
        return v.value if rc == FL_OK else None

    def get_str(self, key):
        v = lib().fl_gguf_get_str(self.h, key.encode())
        return None if v is None else v.decode()

    def read(self, name, off=0, nbytes=None):
        import numpy as np
        t = self.tensor(name)
        n = t.nbytes - off if nbytes is None else nbytes
        out = np.empty(n, np.uint8)
        rc = lib().fl_gguf_read(self.h, ctypes.byref(t), off, n, out.ctypes.data_as(ctypes.c_void_p))
        if rc != FL_OK:
            raise LokiError("fl_gguf_read(%s) = %d" % (name, rc))
        return out


class FLDebug(ctypes.Structure):
    _fields_ = [(n, P_) for n in ("xq", "xd", "logits", "probs", "sel", "wts", "counts", "offsets", "perm", "inv",
                                  "act", "nact", "h", "hq", "hd", "o", "g", "u")] + \
               [("n", ctypes.c_int), ("P", ctypes.c_int), ("topk", ctypes.c_int), ("fused", ctypes.c_int),
                                                                           ("kernel", ctypes.c_int)]


class FLW(ctypes.Structure):
    _fields_ = [(n, P_) for n in ("attn_norm", "q_a", "q_a_norm", "q_b", "kv_a", "kv_a_norm", "kv_b", "k_bT", "attn_out",
                                  "ffn_norm", "gate_inp", "probs_b", "sh_gate", "sh_up", "sh_down", "d_gate", "d_up",
                                  "d_down")] + [("kv_b_v", ctypes.c_int), ("gate_f16", ctypes.c_int)]


class FLOut(ctypes.Structure):
    _fields_ = [("sel", ctypes.POINTER(ctypes.c_int)), ("wts", ctypes.POINTER(ctypes.c_float)),
                ("ncur", ctypes.POINTER(ctypes.c_float)), ("fi", ctypes.POINTER(ctypes.c_float)),
                ("skt", P_), ("sel_s", P_), ("wts_s", P_), ("sc", P_), ("ccat", P_),
                ("h", ctypes.POINTER(ctypes.c_float)), ("moe", ctypes.POINTER(ctypes.c_float))]


# every symbol include/loki_moe.h declares (the ABI test checks the library exports all of them)
ABI_SYMBOLS = [
    "fl_init", "fl_attn", "fl_wide_init", "fl_wide_moe", "fl_wide_mark", "fl_wide_wait", "fl_wide_finish", "fl_moe_outs",
    "fl_wide_outs", "fl_wide_skip", "fl_spec", "fl_sketch", "fl_fetch", "fl_moe", "fl_skip", "fl_h2d", "fl_h2d_bytes", "fl_wait_event",
    "fl_gpu_ms", "fl_ffn_begin", "fl_set_experts", "fl_set_routing", "fl_set_keep", "fl_set_share_experts", "fl_set_shared_formats", "fl_set_layer_formats", "fl_kq_matvec_dev",
    "fl_gguf_open", "fl_gguf_close", "fl_gguf_n_tensors", "fl_gguf_tensor_name", "fl_gguf_tensor", "fl_gguf_tensor_at",
    "fl_gguf_get_int", "fl_gguf_get_float", "fl_gguf_get_str", "fl_gguf_read", "fl_gguf_load_moe_layer", "fl_gguf_free_layer", "fl_moe_layer", "fl_moe_layer_normed", "fl_moe_layer_noalloc", "fl_route_dev", "fl_dispatch_dev", "fl_quant_q8k_dev",
    "fl_pack_iq2xxs", "fl_unpack_iq2xxs", "fl_register_tiled", "fl_unregister_tiled", "fl_rmsnorm_dev", "fl_synth_iq2xxs", "fl_synth_normal", "fl_probe_exp",
    "fl_debug", "fl_set_debug", "fl_set_fused", "fl_set_decode1", "fl_set_prefill_mfma", "fl_stream", "fl_set_stream", "fl_d2h", "fl_set_profile", "fl_stage_ms", "fl_sync", "fl_last_error", "fl_free",
]

_lib = None


class LokiError(RuntimeError):
    pass


def lib():
    """Load libloki_moe.so (raises if it was not built: there is no fallback path)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise LokiError("libloki_moe.so is not built (%s); run python -m loki_amd.build" % LIB_PATH)
        L = ctypes.CDLL(LIB_PATH)
        I, I64, U64, F, D, S = ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_double, ctypes.c_size_t
        sig = {
            "fl_init": (P_, [I, I]),
            "fl_free": (None, [P_]),
            "fl_stream": (P_, [P_]),
            "fl_set_stream": (I, [P_, P_]),
            "fl_d2h": (I, [P_, P_, P_, S]),
            "fl_sync": (I, [P_]),
            "fl_last_error": (ctypes.c_char_p, [P_]),
            "fl_set_routing": (I, [P_, I, I, I, F]),
            "fl_set_experts": (I, [P_, I]),
            "fl_set_keep": (I, [P_, I, F]),
            "fl_set_share_experts": (I, [P_, I]),
            "fl_set_shared_formats": (I, [P_, I, I, I]),
            "fl_set_layer_formats": (I, [P_, I, I, I, I]),
            "fl_kq_matvec_dev": (I, [P_, I, P_, I, I, P_, P_, I, P_]),
            "fl_gguf_open": (P_, [ctypes.POINTER(ctypes.c_char_p), I, ctypes.c_char_p, S]),
            "fl_gguf_close": (None, [P_]),
            "fl_gguf_n_tensors": (I, [P_]),
            "fl_gguf_tensor_name": (ctypes.c_char_p, [P_, I]),
            "fl_gguf_tensor": (I, [P_, ctypes.c_char_p, ctypes.POINTER(FLGgufTensor)]),
            "fl_gguf_tensor_at": (I, [P_, I, ctypes.POINTER(FLGgufTensor)]),
            "fl_gguf_get_int": (I, [P_, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
            "fl_gguf_get_float": (I, [P_, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
            "fl_gguf_get_str": (ctypes.c_char_p, [P_, ctypes.c_char_p]),
            "fl_gguf_read": (I, [P_, ctypes.POINTER(FLGgufTensor), U64, U64, P_]),
            "fl_gguf_load_moe_layer": (I, [P_, P_, I, I, ctypes.POINTER(FLGgufLayer)]),
            "fl_gguf_free_layer": (None, [ctypes.POINTER(FLGgufLayer)]),
            "fl_set_debug": (I, [P_, I]),
            "fl_set_fused": (I, [P_, I]),
            "fl_set_decode1": (I, [P_, I]),
            "fl_set_prefill_mfma": (I, [P_, I]),
            "fl_moe_layer": (I, [P_, ctypes.POINTER(FLMoeLayer), P_, I, P_]),
            "fl_moe_layer_normed": (I, [P_, ctypes.POINTER(FLMoeLayer), P_, F, P_, I, I, P_]),
            "fl_moe_layer_noalloc": (I, [P_, ctypes.POINTER(FLMoeLayer), P_, I, P_]),
            "fl_route_dev": (I, [P_, P_, P_, P_, I, I, I, P_, P_, P_, P_]),
            "fl_dispatch_dev": (I, [P_, P_, I, I, I, P_, P_, P_, P_, P_, P_]),
            "fl_quant_q8k_dev": (I, [P_, P_, I, I, P_, P_]),
            "fl_pack_iq2xxs": (I, [P_, P_, S, P_, S, I, I, I]),
            "fl_register_tiled": (I, [P_, P_, S]),
            "fl_unregister_tiled": (I, [P_, P_, S]),
            "fl_unpack_iq2xxs": (I, [P_, P_, S, P_, S, I, I, I]),
            "fl_rmsnorm_dev": (I, [P_, P_, P_, P_, I, I, F]),
            "fl_synth_iq2xxs": (I, [P_, P_, S, I, I, I, I, U64, U64, F]),
            "fl_synth_normal": (I, [P_, P_, I64, U64, U64, F, F]),
            "fl_probe_exp": (I, [P_, P_, P_, I64, I]),
            "fl_debug": (I, [P_, ctypes.POINTER(FLDebug)]),
            "fl_gpu_ms": (D, [P_, I]),
            "fl_ffn_begin": (I, [P_, ctypes.POINTER(FLW), I, P_, P_, I]),
            "fl_fetch": (None, [P_, I, I, ctypes.POINTER(FLOut)]),
            "fl_moe": (None, [P_, P_, P_, P_, I, I, P_, P_, I, I, ctypes.POINTER(FLOut)]),
            "fl_skip": (None, [P_, P_, I, ctypes.POINTER(FLOut)]),
            "fl_moe_outs": (None, [P_, I, P_, P_, I, P_]),
            "fl_wide_init": (I, [P_, I, I]),
            "fl_wide_moe": (None, [P_, P_, P_, P_, I, I, P_, P_, P_, P_, I, I, I]),
            "fl_wide_mark": (None, [P_, I]),
            "fl_wide_wait": (None, [P_, I]),
            "fl_wide_finish": (None, [P_, I, I, ctypes.POINTER(FLOut)]),
            "fl_wide_outs": (None, [P_, I, I, P_]),
            "fl_wide_skip": (None, [P_, P_, I, ctypes.POINTER(FLOut)]),
            "fl_h2d": (None, [P_, P_, P_, S]),
            "fl_h2d_bytes": (I, [P_, ctypes.POINTER(S), ctypes.POINTER(S)]),
            "fl_wait_event": (None, [P_, P_]),
            "fl_set_profile": (I, [P_, I]),
            "fl_stage_ms": (I, [P_, ctypes.POINTER(ctypes.c_double), I, I]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    """Names of ABI_SYMBOLS that the built library exports (no GPU needed)."""
    L = ctypes.CDLL(LIB_PATH)
    out = []
    for s in ABI_SYMBOLS:
        try:
            getattr(L, s)
            out.append(s)
        except AttributeError:
            pass
    return out


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def iq2_matrix_bytes(rows, cols):
    return rows * (cols // QK_K) * IQ2_BYTES


class Context:
    """An FLCtx (one HIP stream). Calls are asynchronous on that stream unless stated otherwise."""

    def __init__(self):
        import torch  # device memory and the current device come from torch
        if not torch.cuda.is_available():
            raise LokiError("no GPU visible: libloki_moe runs only on the device")
        self.torch = torch
        self.ctx = lib().fl_init(0, 0)
        if not self.ctx:
            raise LokiError("fl_init failed")
        # share torch's current stream so library kernels and torch ops on the same buffers stay ordered
        self.check(lib().fl_set_stream(self.ctx, torch.cuda.current_stream().cuda_stream))

    def close(self):
        if self.ctx:
            lib().fl_free(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, rc):
        if rc != FL_OK:
            raise LokiError("libloki_moe: %s (code %d)" % (lib().fl_last_error(self.ctx).decode(), rc))

    @property
    def stream_handle(self):
        return lib().fl_stream(self.ctx)

    def d2h(self, ptr, shape, dtype):
        """Copy a device buffer (raw pointer, e.g. from debug()) into a new numpy array (waited)."""
        import numpy as np
        out = np.empty(shape, dtype=dtype)
        if out.nbytes:
            self.check(lib().fl_d2h(self.ctx, out.ctypes.data_as(ctypes.c_void_p), ptr, out.nbytes))
        return out

    def sync(self):
        self.check(lib().fl_sync(self.ctx))

    def set_routing(self, n_group=8, topk_group=4, topk=8, scale=2.5):
        self.check(lib().fl_set_routing(self.ctx, n_group, topk_group, topk, scale))

    def set_keep(self, keep=0, renorm=2.5):
        """fl_moe_layer keeps each row's `keep` heaviest experts, rescaled to sum to renorm (0 = all topk, default)."""
        self.check(lib().fl_set_keep(self.ctx, keep, renorm))

    def set_share_experts(self, on=True):
        """The engine's --share-experts rule for set_keep's keep (rows prefer experts other rows already use)."""
        self.check(lib().fl_set_share_experts(self.ctx, 1 if on else 0))

    def set_experts(self, n_exp=N_EXPERT):
        self.check(lib().fl_set_experts(self.ctx, n_exp))

    def set_shared_formats(self, gate=FL_IQ2, up=FL_IQ2, down=FL_IQ2):
        """Formats of FLW's shared expert for fl_ffn_begin; the reference's shards: (FL_Q5K, FL_Q5K, FL_Q6K)."""
        self.check(lib().fl_set_shared_formats(self.ctx, gate, up, down))

    def set_layer_formats(self, down=FL_IQ2, sh_gate=FL_IQ2, sh_up=FL_IQ2, sh_down=FL_IQ2):
        """Formats of fl_moe_layer's routed down and shared matrices (K-quants read in place, IQ2_XXS tiled)."""
        self.check(lib().fl_set_layer_formats(self.ctx, down, sh_gate, sh_up, sh_down))

    def set_debug(self, capture_gate_up, small_grids=False, shared_on_stream=False):
        """capture_gate_up: keep the per-pass gate / up outputs (debug()); small_grids: the row-looping combine / scatter
        kernels run with a y extent of 7 (process-wide), so their loops over rows are exercised at small sizes;
        shared_on_stream: the per-pass decode's K-quant shared expert runs on the context's stream instead of beside the
        routed launches on a second stream."""
        self.check(lib().fl_set_debug(self.ctx, (1 if capture_gate_up else 0) | (2 if small_grids else 0) | (4 if shared_on_stream else 0)))

    def set_prefill_mfma(self, on):
        """Batches above 8 tokens: True (default) = grouped GEMMs on the matrix cores, False = the per-pass kernels."""
        self.check(lib().fl_set_prefill_mfma(self.ctx, 1 if on else 0))

    def set_fused(self, mode):
        """Decode batches (n <= 8): 2 = one regular launch (default), 1 = the same kernel as a cooperative launch,
        0 = one launch per pass."""
        self.check(lib().fl_set_fused(self.ctx, int(mode)))
        self._fused = int(mode)

    def set_decode1(self, on):
        """One-token decode: True (default) = the kernel organised by XCD, False = the general decode block."""
        self.check(lib().fl_set_decode1(self.ctx, 1 if on else 0))

    @property
    def fused_mode(self):
        """The decode mode last set on this context (the library's default 2 until set_fused is called)."""
        return getattr(self, "_fused", 2)

    def using_fused(self, mode):
        """Context manager: run the body with decode mode `mode`, then restore the previous mode."""
        import contextlib

        @contextlib.contextmanager
        def cm():
            prev = self.fused_mode
            self.set_fused(mode)
            try:
                yield self
            finally:
                self.set_fused(prev)
        return cm()

    # ---- building blocks
    def quant_q8k(self, x):
        t = self.torch
        n, K = x.shape
        q = t.empty((n, K), dtype=t.int8, device=x.device)
        d = t.empty((n, K // QK_K), dtype=t.float32, device=x.device)
        self.check(lib().fl_quant_q8k_dev(self.ctx, _ptr(x), n, K, _ptr(q), _ptr(d)))
        return q, d

    def load_gguf_layer(self, gguf, layer, layout=None):
        """One MoE layer of a Gguf index, resident in HBM (FLGgufLayer; free with free_gguf_layer)."""
        out = FLGgufLayer()
        self.check(lib().fl_gguf_load_moe_layer(self.ctx, gguf.h, layer, FL_LAYOUT_TILED if layout is None else layout,
                                                ctypes.byref(out)))
        return out

    def free_gguf_layer(self, gl):
        lib().fl_gguf_free_layer(ctypes.byref(gl))

    def kq_matvec(self, fmt, w, R, K, q, d, y=None):
        """y [n][R] = K-quant matrix w (uint8 device tensor, R x K/256 ggml blocks) . Q8_K rows (q [n][K], d [n][K/256])."""
        t = self.torch
        n = q.shape[0]
        if y is None:
            y = t.empty((n, R), dtype=t.float32, device=q.device)
        self.check(lib().fl_kq_matvec_dev(self.ctx, fmt, _ptr(w), R, K, _ptr(q), _ptr(d), n, _ptr(y)))
        return y

    def route(self, W, bias, x, topk=8):
        t = self.torch
        n, E = x.shape
        ne = W.shape[0]
        logits = t.empty((n, ne), dtype=t.float32, device=x.device)
        probs = t.empty((n, ne), dtype=t.float32, device=x.device)
        sel = t.empty((n, topk), dtype=t.int32, device=x.device)
        w = t.empty((n, topk), dtype=t.float32, device=x.device)
        self.check(lib().fl_route_dev(self.ctx, _ptr(W), _ptr(bias), _ptr(x), n, ne, E, _ptr(logits), _ptr(probs), _ptr(sel), _ptr(w)))
        return logits, probs, sel, w

    def dispatch(self, sel, n_exp=N_EXPERT):
        t = self.torch
        n, topk = sel.shape
        P = n * topk
        dev = sel.device
        counts = t.empty(n_exp, dtype=t.int32, device=dev); offsets = t.empty(n_exp + 1, dtype=t.int32, device=dev)
        perm = t.empty(max(P, 1), dtype=t.int32, device=dev); inv = t.empty(max(P, 1), dtype=t.int32, device=dev)
        act = t.empty(n_exp, dtype=t.int32, device=dev); nact = t.empty(1, dtype=t.int32, device=dev)
        self.check(lib().fl_dispatch_dev(self.ctx, _ptr(sel), n, topk, n_exp, _ptr(counts), _ptr(offsets), _ptr(perm),
                                         _ptr(inv), _ptr(act), _ptr(nact)))
        return counts, offsets, perm[:P], inv[:P], act, nact

    def pack(self, src, rows, cols, nmat, src_stride=None, dst=None):
        t = self.torch
        mb = iq2_matrix_bytes(rows, cols)
        if dst is None:
            dst = t.empty(nmat * mb, dtype=t.uint8, device=src.device)
        self.check(lib().fl_pack_iq2xxs(self.ctx, _ptr(src), src_stride or mb, _ptr(dst), mb, rows, cols, nmat))
        return dst

    def register_tiled(self, t):
        """Declare a device tensor as tiled IQ2_XXS matrices: fl_moe / fl_wide_moe / fl_ffn_begin read it in place."""
        self.check(lib().fl_register_tiled(self.ctx, _ptr(t), t.numel() * t.element_size()))

    def unregister_tiled(self, t):
        self.check(lib().fl_unregister_tiled(self.ctx, _ptr(t), t.numel() * t.element_size()))

    def unpack(self, src, rows, cols, nmat, dst=None):
        t = self.torch
        mb = iq2_matrix_bytes(rows, cols)
        if dst is None:
            dst = t.empty(nmat * mb, dtype=t.uint8, device=src.device)
        self.check(lib().fl_unpack_iq2xxs(self.ctx, _ptr(src), mb, _ptr(dst), mb, rows, cols, nmat))
        return dst

    def rmsnorm(self, x, w=None, eps=1e-6, out=None):
        n, D = x.shape
        y = out if out is not None else self.torch.empty_like(x)
        self.check(lib().fl_rmsnorm_dev(self.ctx, _ptr(x), _ptr(w), _ptr(y), n, D, eps))
        return y

    def synth_iq2(self, dst, rows, cols, nmat, layout, seed, mat0, sigma=0.002):
        mb = iq2_matrix_bytes(rows, cols)
        self.check(lib().fl_synth_iq2xxs(self.ctx, _ptr(dst), mb, rows, cols, nmat, layout, seed, mat0, sigma))
        return dst

    def synth_normal(self, dst, seed, stream, mean=0.0, sigma=1.0):
        self.check(lib().fl_synth_normal(self.ctx, _ptr(dst), dst.numel(), seed, stream, mean, sigma))
        return dst

    def probe_exp(self, x, which=0):
        y = self.torch.empty_like(x)
        self.check(lib().fl_probe_exp(self.ctx, _ptr(x), _ptr(y), x.numel(), which))
        return y

    # ---- the block
    def moe_layer(self, layer, x, y=None):
        n, E = x.shape
        if y is None:
            y = self.torch.empty_like(x)
        self.check(lib().fl_moe_layer(self.ctx, ctypes.byref(layer.abi()), _ptr(x), n, _ptr(y)))
        return y

    def moe_layer_normed(self, layer, h, norm_w=None, eps=1e-6, y=None, residual=False):
        """y = MoE(RMSNorm(h) * norm_w) (norm_w None: ones) -- the layer's ffn_norm inside the block; residual adds h."""
        n, E = h.shape
        if y is None:
            y = self.torch.empty_like(h)
        self.check(lib().fl_moe_layer_normed(self.ctx, ctypes.byref(layer.abi()), _ptr(norm_w), eps, _ptr(h), n,
                                             1 if residual else 0, _ptr(y)))
        return y

    def debug(self):
        d = FLDebug()
        self.check(lib().fl_debug(self.ctx, ctypes.byref(d)))
        return d

    def gpu_ms(self, which=1):
        return lib().fl_gpu_ms(self.ctx, which)

    STAGES = ("quant_x", "router_logits", "router_select", "dispatch", "gate_up", "down")

    def set_profile(self, on):
        self.check(lib().fl_set_profile(self.ctx, 1 if on else 0))

    def stage_ms(self, reset=True):
        """(calls, {stage: summed ms}) of the profiled fl_moe_layer calls since the last reset (waits for them)."""
        arr = (ctypes.c_double * len(self.STAGES))()
        n = lib().fl_stage_ms(self.ctx, arr, len(self.STAGES), 1 if reset else 0)
        if n < 0:
            self.check(n)
        return n, dict(zip(self.STAGES, list(arr)))


class MoeLayerWeights:
    """Device-resident weights of one MoE layer in the tiled IQ2_XXS layout (torch uint8 / float32 tensors)."""

    def __init__(self, gate_inp, probs_b, gate, up, down, sh_gate, sh_up, sh_down, n_exp=N_EXPERT, E=E_HIDDEN, H=H_EXPERT):
        self.gate_inp, self.probs_b = gate_inp, probs_b
        self.gate, self.up, self.down = gate, up, down
        self.sh_gate, self.sh_up, self.sh_down = sh_gate, sh_up, sh_down
        self.n_exp, self.E, self.H = n_exp, E, H
        self._abi = FLMoeLayer(gate_inp.data_ptr(), probs_b.data_ptr(), gate.data_ptr(), up.data_ptr(), down.data_ptr(),
                               sh_gate.data_ptr(), sh_up.data_ptr(), sh_down.data_ptr(), FL_LAYOUT_TILED, n_exp, E, H)

    def abi(self):
        return self._abi

    def nbytes_expert(self):
        return 3 * iq2_matrix_bytes(self.H, self.E)

    def expert_slice(self, which, e):
        """Bytes of routed expert e's matrix ('gate' / 'up' / 'down') in the tiled layout (device tensor view)."""
        mb = iq2_matrix_bytes(self.H, self.E)
        return getattr(self, which)[e * mb:(e + 1) * mb]

    @staticmethod
    def synthetic(ctx, seed, n_exp=N_EXPERT, E=E_HIDDEN, H=H_EXPERT, bias_sigma=0.01, hot=None, hot_bias=0.5,
                  w_sigma=0.02, d_sigma=0.002, device="cuda"):
        """A layer of the task's synthetic distribution, generated on the device: router W ~ N(0, w_sigma^2) [n_exp, E],
        bias ~ N(0, bias_sigma^2) (+hot_bias on the experts in `hot`), every expert's qs uniform bytes and
        d = fp16(|N(0, d_sigma^2)|). Matrix ids: expert e gate/up/down = 3e, 3e+1, 3e+2; shared = 3*n_exp + 0..2."""
        t = ctx.torch
        mb = iq2_matrix_bytes(H, E)
        W = t.empty((n_exp, E), dtype=t.float32, device=device)
        b = t.empty(n_exp, dtype=t.float32, device=device)
        ctx.synth_normal(W, seed, 1, 0.0, w_sigma)
        ctx.synth_normal(b, seed, 2, 0.0, bias_sigma)
        mats = []
        for k, (rows, cols) in enumerate(((H, E), (H, E), (E, H))):
            m = t.empty(n_exp * mb, dtype=t.uint8, device=device)
            ctx.check(_synth_strided(ctx, m, rows, cols, n_exp, seed, 0, k, d_sigma))
            mats.append(m)
        sh = []
        for k, (rows, cols) in enumerate(((H, E), (H, E), (E, H))):
            m = t.empty(mb, dtype=t.uint8, device=device)
            ctx.check(lib().fl_synth_iq2xxs(ctx.ctx, _ptr(m), mb, rows, cols, 1, FL_LAYOUT_TILED, seed, 3 * n_exp + k, d_sigma))
            sh.append(m)
        ctx.sync()
        if hot is not None:
            hb = t.zeros(n_exp, dtype=t.float32, device=device)
            hb[t.as_tensor(list(hot), device=device, dtype=t.long)] = hot_bias
            b = b + hb
        return MoeLayerWeights(W, b, mats[0], mats[1], mats[2], sh[0], sh[1], sh[2], n_exp, E, H)


def _synth_strided(ctx, sub, rows, cols, ne, seed, e0, k, d_sigma):
    """Expert e's matrix k gets matrix id 3e + k (one launch per expert)."""
    mb = iq2_matrix_bytes(rows, cols)
    for j in range(ne):
        rc = lib().fl_synth_iq2xxs(ctx.ctx, _ptr(sub[j * mb:(j + 1) * mb]), mb, rows, cols, 1, FL_LAYOUT_TILED, seed,
                                   3 * (e0 + j) + k, d_sigma)
        if rc != FL_OK:
            return rc
    return FL_OK
