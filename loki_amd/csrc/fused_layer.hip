// fused_layer.hip -- FLCtx and the C ABI of include/loki_moe.h (host side of the MoE block on MI355X).
//
// Reference host side: src/fused_layer.cu:391-620 (FLCtx, fl_init, fl_moe, fl_wide_*, fl_fetch, fl_gpu_ms). The
// device-resident path fl_moe_layer runs the whole block on the context's stream with no host round-trip:
//   Q8_K(x) -> router logits (fp64 contract) -> sigmoid / grouped top-k / weights -> dispatch (histogram, scan,
//   stable permutation) -> gate+up mat-vecs with the SwiGLU epilogue -> Q8_K(h) -> down mat-vecs -> k-ordered combine.
#include "moe_common.h"
#include "moe_kernels.h"
#include "../../include/loki_moe.h"
#include "fl_ctx.h"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

using namespace lk;

[[noreturn]] static void out_of_scope(const char * fn) {
    std::fprintf(stderr, "[fused] %s: attention, speculation and sketches are not part of the MoE-block library\n", fn);
    std::exit(7);
}

// ================================================================ allocation-free decode (fl_moe_layer_noalloc)
// Every device buffer the single-launch decode block needs beyond the caller's inputs and outputs, in one file-scope
// array that each GPU holds from module load until the process ends. Byte offsets (256-aligned):
namespace {
constexpr size_t NA_ALIGN = 256;
constexpr size_t na_up(size_t v) { return (v + NA_ALIGN - 1) / NA_ALIGN * NA_ALIGN; }
constexpr int NA_MAXN = 8;                          // tokens per call (the decode block's batch)
constexpr int NA_MAXP = NA_MAXN * MAXK;             // routed pairs per call
constexpr size_t NA_TAB = 0;                                                   // LDS table image
constexpr size_t NA_TLOG = na_up(NA_TAB + TAB_BYTES);                          // tagged probabilities
constexpr size_t NA_TH = na_up(NA_TLOG + DEC_TLOGITS * 8);                     // tagged h
constexpr size_t NA_TO = na_up(NA_TH + DEC_TH * 8);                            // tagged o
constexpr size_t NA_ERR = na_up(NA_TO + DEC_TO * 8);                           // error word
constexpr size_t NA_XQ = na_up(NA_ERR + 4);                                    // Q8_K of x
constexpr size_t NA_XD = na_up(NA_XQ + (size_t) NA_MAXN * 7168);
constexpr size_t NA_LOG = na_up(NA_XD + (size_t) NA_MAXN * 28 * 4);            // logits, probabilities
constexpr size_t NA_PRB = na_up(NA_LOG + (size_t) NA_MAXN * NEXP_MAX * 4);
constexpr size_t NA_SEL = na_up(NA_PRB + (size_t) NA_MAXN * NEXP_MAX * 4);     // routing and dispatch outputs
constexpr size_t NA_WTS = na_up(NA_SEL + NA_MAXP * 4);
constexpr size_t NA_PERM = na_up(NA_WTS + NA_MAXP * 4);
constexpr size_t NA_INV = na_up(NA_PERM + NA_MAXP * 4);
constexpr size_t NA_CNT = na_up(NA_INV + NA_MAXP * 4);
constexpr size_t NA_OFF = na_up(NA_CNT + NEXP_MAX * 4);
constexpr size_t NA_ACT = na_up(NA_OFF + (NEXP_MAX + 1) * 4);
constexpr size_t NA_NACT = na_up(NA_ACT + NEXP_MAX * 4);
constexpr size_t NA_BYTES = na_up(NA_NACT + 4);
static_assert(NA_BYTES == 5502720, "the allocation-free entry point's documented scratch size (5.25 MiB per GPU)");
constexpr size_t NA_CLEAR0 = NA_TLOG, NA_CLEAR1 = NA_XQ;   // the tagged words and the error word start at zero
static_assert((NA_ERR - NA_CLEAR0) % 16 == 0 && (NA_CLEAR1 - NA_CLEAR0) % 16 == 0, "cleared as 16-byte words");
constexpr unsigned NA_EPOCH = 1;   // every call tags its hand-off words with this one epoch, after clearing them (below)
constexpr int NA_MAXDEV = 64;
}  // namespace
static __device__ __align__(256) uint8_t scratch[NA_BYTES];

struct NaDev { uint8_t * ptr = nullptr; int resolved = 0; int ready = 0; };   // ready: table image built, words cleared
static NaDev g_na[NA_MAXDEV];
static std::mutex g_na_mu;

// the device address of `scratch` on device dev (current), once per device; null if HIP cannot resolve it
static uint8_t * na_resolve(int dev) {
    if (dev < 0 || dev >= NA_MAXDEV) { return nullptr; }
    std::lock_guard<std::mutex> lk(g_na_mu);
    NaDev & d = g_na[dev];
    if (!d.resolved) {
        void * p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) { (void) hipGetLastError(); p = nullptr; }
        d.ptr = (uint8_t *) p; d.resolved = 1;
    }
    return d.ptr;
}

// zero fill of 16-byte words (no memset node: the call may be captured into a graph)
__global__ void __launch_bounds__(256) k_zero16(uint4 * p, size_t n) {
    for (size_t i = (size_t) blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t) gridDim.x * 256) { p[i] = make_uint4(0, 0, 0, 0); }
}

static bool decode_ready(FLCtx * c);
static bool decode1_ready(FLCtx * c);

// ================================================================ lifecycle
extern "C" FLCtx * fl_init(int kvp, int sc_cap) {
    (void) kvp; (void) sc_cap;
    FLCtx * c = new FLCtx();
    CK(hipGetDevice(&c->dev));
    CK(hipDeviceGetAttribute(&c->ncu, hipDeviceAttributeMultiprocessorCount, c->dev));
    CK(hipStreamCreateWithFlags(&c->own, hipStreamNonBlocking)); c->st = c->own;
    CK(hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking));
    CK(hipEventCreateWithFlags(&c->efork, hipEventDisableTiming)); CK(hipEventCreateWithFlags(&c->ejoin, hipEventDisableTiming));
    CK(hipEventCreate(&c->em0)); CK(hipEventCreate(&c->em1));
    if (hipHostMalloc((void **) &c->herr, sizeof(int), hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) {
        (void) hipGetLastError(); c->herr = nullptr;
    } else if (hipHostGetDevicePointer((void **) &c->herr_dev, c->herr, 0) != hipSuccess) {
        (void) hipGetLastError(); (void) hipHostFree(c->herr); c->herr = nullptr;
    } else {
        __atomic_store_n(c->herr, 0, __ATOMIC_RELEASE);
    }
    // the allocation-free entry point's scratch on this device: resolved, its table image built and its tagged words
    // and error word cleared here, once per device, so that entry point only launches kernels
    if (uint8_t * S = na_resolve(c->dev)) {
        std::lock_guard<std::mutex> lk(g_na_mu);
        NaDev & nd = g_na[c->dev];
        if (!nd.ready) {
            CK(build_table_image(reinterpret_cast<uint4 *>(S + NA_TAB), c->st));
            k_zero16<<<512, 256, 0, c->st>>>(reinterpret_cast<uint4 *>(S + NA_CLEAR0), (NA_CLEAR1 - NA_CLEAR0) / 16);
            CK(hipGetLastError());
            CK(hipStreamSynchronize(c->st));
            nd.ready = 1;
        }
    }
    (void) decode_ready(c);      // its set-up (attributes, XCD probe) here, not in a call that must not allocate
    (void) decode1_ready(c);
    return c;
}

extern "C" void fl_free(FLCtx * c) {
    if (!c) { return; }
    (void) hipStreamSynchronize(c->st);
    c->xq.release(); c->hq.release(); c->xd.release(); c->logits.release(); c->probs.release(); c->wts.release();
    c->h.release(); c->hd.release(); c->o.release(); c->g.release(); c->u.release(); c->xn.release();
    c->sel8.release(); c->w8.release();
    c->sel.release(); c->counts.release(); c->offsets.release(); c->perm.release(); c->inv.release(); c->act.release(); c->nact.release();
    compat_free(c); c->zero_i.release(); c->terms.release(); c->cnt.release();
    c->tab.release(); c->derr.release(); c->dlogit.release(); c->dth.release(); c->dto.release(); c->dxq.release();
    c->ptab.release(); c->pcols.release(); c->pncols.release(); c->xh.release(); c->hh.release();
    c->ksg.release(); c->ksu.release(); c->rcnt.release(); c->rpart.release(); c->dscr.release();
    for (auto & v : c->ev_free) { for (auto e : v) { (void) hipEventDestroy(e); } }
    for (auto & v : c->ev_pending) { for (auto e : v) { (void) hipEventDestroy(e); } }
    for (auto * l : { &c->ffn_ev_pending, &c->ffn_ev_free, &c->moe_ev_pending, &c->moe_ev_free }) { for (auto & e : *l) { (void) hipEventDestroy(e.first); (void) hipEventDestroy(e.second); } }
    (void) hipEventDestroy(c->em0); (void) hipEventDestroy(c->em1); (void) hipStreamDestroy(c->own);
    (void) hipEventDestroy(c->efork); (void) hipEventDestroy(c->ejoin); (void) hipStreamDestroy(c->side);
    if (c->herr) { (void) hipHostFree(c->herr); }
    delete c;
}

extern "C" hipStream_t fl_stream(FLCtx * c) { return c ? c->st : nullptr; }
extern "C" int fl_set_stream(FLCtx * c, hipStream_t s) {
    if (!c) { return FL_EINVAL; }
    TRY(c, hipStreamSynchronize(c->st));   // work already queued on the old stream finishes first
    c->st = s; return FL_OK;
}
extern "C" int fl_d2h(FLCtx * c, void * host, const void * dev, size_t bytes) {
    if (!c) { return FL_EINVAL; }
    if (bytes == 0) { return FL_OK; }
    if (!host || !dev) { return fail(c, FL_EINVAL, "null pointer"); }
    TRY(c, hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, c->st));
    TRY(c, hipStreamSynchronize(c->st));
    return FL_OK;
}
// waits for the context's stream, then reports a wait timeout of the single-launch decode block (and clears it)
extern "C" int fl_sync(FLCtx * c) {
    if (!c) { return FL_EINVAL; }
    TRY(c, hipStreamSynchronize(c->st));
    int e = 0;
    if (c->derr.p) {
        TRY(c, hipMemcpy(&e, c->derr.p, sizeof e, hipMemcpyDeviceToHost));
        if (e) { TRY(c, hipMemset(c->derr.p, 0, sizeof e)); }
    }
    if (c->na_used) {   // fl_moe_layer_noalloc reports into the scratch's error word of the device
        if (uint8_t * S = na_resolve(c->dev)) {
            int w = 0;
            TRY(c, hipMemcpy(&w, S + NA_ERR, sizeof w, hipMemcpyDeviceToHost));
            if (w) { const int z = 0; TRY(c, hipMemcpy(S + NA_ERR, &z, sizeof z, hipMemcpyHostToDevice)); }
            e |= w;
        }
    }
    if (c->herr) { e |= __atomic_exchange_n(c->herr, 0, __ATOMIC_ACQ_REL); }
    if (e) {
        return fail(c, FL_EHIP, "a device kernel reported error code %d (decode block: a wait timed out or a workgroup ran on an unexpected XCD; prefill: bad LDS base); its outputs are invalid", e);
    }
    return FL_OK;
}
extern "C" const char * fl_last_error(FLCtx * c) { return c ? c->err.c_str() : "null context"; }

extern "C" int fl_set_routing(FLCtx * c, int n_group, int topk_group, int topk, float scale) {
    if (!c) { return FL_EINVAL; }
    if (n_group <= 0 || topk_group <= 0 || topk_group > n_group || topk <= 0 || topk > MAXK || !(scale > 0.f)) {
        return fail(c, FL_EINVAL, "bad routing rule (n_group %d, topk_group %d, topk %d, scale %g)", n_group, topk_group, topk, (double) scale);
    }
    c->n_group = n_group; c->topk_group = topk_group; c->topk = topk; c->scale = scale; return FL_OK;
}
extern "C" int fl_set_keep(FLCtx * c, int keep, float renorm) {
    if (!c) { return FL_EINVAL; }
    if (keep < 0 || keep > MAXK || !(renorm >= 0.f)) { return fail(c, FL_EINVAL, "keep %d outside 0..%d or renorm %g negative", keep, MAXK, (double) renorm); }
    c->keep = keep; c->renorm = renorm; return FL_OK;
}
extern "C" int fl_set_share_experts(FLCtx * c, int on) {
    if (!c) { return FL_EINVAL; }
    c->share = on ? 1 : 0; return FL_OK;
}
extern "C" int fl_set_experts(FLCtx * c, int n_exp) {
    if (!c) { return FL_EINVAL; }
    if (n_exp <= 0 || n_exp > NEXP_MAX) { return fail(c, FL_EINVAL, "n_exp %d outside 1..%d", n_exp, NEXP_MAX); }
    c->n_exp = n_exp; return FL_OK;
}
extern "C" int fl_set_debug(FLCtx * c, int flags) {
    if (!c) { return FL_EINVAL; }
    c->dbg_gu = (flags & 1) ? 1 : 0;
    c->no_side = (flags & 4) ? 1 : 0;
    set_grid_ycap((flags & 2) ? 7 : 65535);   // process-wide: the row loops of the combine / scatter kernels at small sizes
    return FL_OK;
}
extern "C" int fl_set_prefill_mfma(FLCtx * c, int on) { if (!c) { return FL_EINVAL; } c->pf_mfma = on ? 1 : 0; return FL_OK; }
extern "C" int fl_set_decode1(FLCtx * c, int on) { if (!c) { return FL_EINVAL; } c->d1 = on ? 1 : 0; return FL_OK; }
extern "C" int fl_set_fused(FLCtx * c, int mode) {
    if (!c) { return FL_EINVAL; }
    if (mode < 0 || mode > 2) { return fail(c, FL_EINVAL, "fused mode %d outside 0..2", mode); }
    c->fused = mode; return FL_OK;
}

// ================================================================ building blocks
static int check_rule(FLCtx * c, int n_exp) {
    if (n_exp <= 0 || n_exp > NEXP_MAX) { return fail(c, FL_EINVAL, "n_exp %d outside 1..%d", n_exp, NEXP_MAX); }
    if (n_exp % c->n_group) { return fail(c, FL_EINVAL, "n_exp %d not divisible by n_group %d", n_exp, c->n_group); }
    if (c->n_group > 64) { return fail(c, FL_EINVAL, "n_group %d above 64", c->n_group); }
    const int per = n_exp / c->n_group;
    if (per < 2 || c->topk > c->topk_group * per) { return fail(c, FL_EINVAL, "top-%d cannot be drawn from %d groups of %d", c->topk, c->topk_group, per); }
    return FL_OK;
}

static int decode_tagged(FLCtx * c, hipStream_t st);
int route_dev(FLCtx * c, const float * W, const float * bias, const float * x, int n, int n_exp, int E, float * logits, float * probs,
              int * sel, float * w, unsigned * done) {
    if (!c) { return FL_EINVAL; }
    if (n < 0 || n > 65536) { return fail(c, FL_ERANGE, "n = %d outside 0..65536", n); }
    if (n == 0) { return FL_OK; }
    if (!W || !bias || !x || !sel || !w) { return fail(c, FL_EINVAL, "null pointer"); }
    if (E <= 0 || E % 1024) { return fail(c, FL_EINVAL, "E = %d must be a positive multiple of 1024", E); }
    if (int rc = check_rule(c, n_exp)) { return rc; }
    if (!covers(W, (size_t) n_exp * E * 4) || !covers(bias, (size_t) n_exp * 4) || !covers(x, (size_t) n * E * 4)) {
        return fail(c, FL_EINVAL, "router weight, bias or x allocation smaller than its shape (%d experts, %d rows of %d)", n_exp, n, E);
    }
    if (!logits) { ALLOC(c, c->logits, (size_t) n * n_exp); logits = c->logits.p; }
    if (router_fused_ok(n, E)) {   // a few rows: logits and selection in one launch, the logits handed over tagged
        if (!c->rcnt.p) { ALLOC(c, c->rcnt, 1); TRY(c, hipMemsetAsync(c->rcnt.p, 0, sizeof(unsigned), c->st)); }
        if (int rc = decode_tagged(c, c->st)) { return rc; }   // a fresh epoch for the tagged logit buffer
        TRY(c, launch_router_fused(W, x, n, n_exp, E, logits, bias, c->n_group, c->topk_group, c->topk, c->scale, probs, sel, w, c->dlogit.p,
                                   c->epoch, c->rcnt.p, done, c->derr.p, c->herr ? c->herr_dev : nullptr, c->st));
        return FL_OK;
    }
    double * rp = nullptr;   // the K-split tiles' parts (n from RL_SPLIT_MIN to RL_SPLIT_MAX)
    if (const size_t nd = router_split_doubles(n, n_exp, E)) { ALLOC(c, c->rpart, nd); rp = c->rpart.p; }
    TRY(c, launch_router_logits(W, x, n, n_exp, E, logits, rp, c->st));
    TRY(c, launch_router_select(logits, bias, n, n_exp, c->n_group, c->topk_group, c->topk, c->scale, probs, sel, w, c->st));
    return FL_OK;
}
extern "C" int fl_route_dev(FLCtx * c, const float * W, const float * bias, const float * x, int n, int n_exp, int E,
                            float * logits, float * probs, int * sel, float * w) {
    return route_dev(c, W, bias, x, n, n_exp, E, logits, probs, sel, w, nullptr);
}

extern "C" int fl_dispatch_dev(FLCtx * c, const int * sel, int n, int topk, int n_exp, int * counts, int * offsets, int * perm, int * inv, int * act, int * nact) {
    if (!c) { return FL_EINVAL; }
    if (n < 0 || topk <= 0 || topk > MAXK || (int64_t) n * topk > (1 << 24)) { return fail(c, FL_ERANGE, "n*topk out of range"); }
    if (n_exp <= 0 || n_exp > NEXP_MAX) { return fail(c, FL_EINVAL, "n_exp %d outside 1..%d", n_exp, NEXP_MAX); }
    if (!sel || !counts || !offsets || !perm || !inv || !act || !nact) { return fail(c, FL_EINVAL, "null pointer"); }
    int * dsc = nullptr;
    if (const size_t nd = dispatch_scratch_ints(n * topk)) { ALLOC(c, c->dscr, nd); dsc = c->dscr.p; }
    TRY(c, launch_dispatch(sel, n * topk, n_exp, counts, offsets, perm, inv, act, nact, c->st, dsc));
    return FL_OK;
}

extern "C" int fl_quant_q8k_dev(FLCtx * c, const float * x, int nrows, int K, int8_t * q, float * d) {
    if (!c) { return FL_EINVAL; }
    if (nrows < 0 || K <= 0 || K % 256) { return fail(c, FL_EINVAL, "K = %d must be a positive multiple of 256", K); }
    if (nrows == 0) { return FL_OK; }
    if (!x || !q || !d) { return fail(c, FL_EINVAL, "null pointer"); }
    TRY(c, launch_quant_q8k(x, nrows, K, q, d, c->st));
    return FL_OK;
}

extern "C" int fl_kq_matvec_dev(FLCtx * c, int fmt, const void * w, int R, int K, const int8_t * q, const float * d, int n, float * y) {
    if (!c) { return FL_EINVAL; }
    const int bs = kq_block_bytes(fmt);
    if (bs == 0) { return fail(c, FL_EINVAL, "format %d is not a K-quant (FL_Q2K, FL_Q3K, FL_Q5K, FL_Q6K)", fmt); }
    if (R <= 0 || K <= 0 || K % 256 || K > 8192 || n < 0) { return fail(c, FL_EINVAL, "R %d, K %d (a multiple of 256, at most 8192), n %d", R, K, n); }
    if (n == 0) { return FL_OK; }
    if (!w || !q || !d || !y) { return fail(c, FL_EINVAL, "null pointer"); }
    const size_t mb = (size_t) R * (size_t) (K / 256) * (size_t) bs;
    if (mb % 4 || (reinterpret_cast<uintptr_t>(w) & 3u)) { return fail(c, FL_EINVAL, "the matrix must start and end on 4-byte boundaries (%zu bytes)", mb); }
    if (!covers(w, mb) || !covers(q, (size_t) n * K) || !covers(d, (size_t) n * (K / 256) * 4) || !covers(y, (size_t) n * R * 4)) {
        return fail(c, FL_EINVAL, "an allocation is smaller than its shape");
    }
    KqArgs a{};
    a.w = (const uint8_t *) w; a.estride = mb; a.aq = q; a.ad = d; a.K = K; a.R = R;
    a.act = nullptr; a.nact = nullptr; a.offsets = nullptr; a.n = n; a.out = y; a.ldo = R;
    TRY(c, launch_kq_matvec(a, fmt, n, 1, c->st));
    return FL_OK;
}

static int pack_args(FLCtx * c, const void * s, const void * d, int R, int K, int nmat) {
    if (!s || !d) { return fail(c, FL_EINVAL, "null pointer"); }
    if (R <= 0 || R % 4 || K <= 0 || K % 1024 || nmat <= 0) { return fail(c, FL_EINVAL, "tiled layout needs R %% 4 == 0 and K %% 1024 == 0 (R %d, K %d)", R, K); }
    return FL_OK;
}
extern "C" int fl_pack_iq2xxs(FLCtx * c, const void * src, size_t ss, void * dst, size_t ds, int R, int K, int nmat) {
    if (!c) { return FL_EINVAL; }
    if (int rc = pack_args(c, src, dst, R, K, nmat)) { return rc; }
    TRY(c, launch_pack_tiled((const uint8_t *) src, ss, (uint8_t *) dst, ds, R, K, nmat, c->st));
    return FL_OK;
}
extern "C" int fl_unpack_iq2xxs(FLCtx * c, const void * src, size_t ss, void * dst, size_t ds, int R, int K, int nmat) {
    if (!c) { return FL_EINVAL; }
    if (int rc = pack_args(c, src, dst, R, K, nmat)) { return rc; }
    TRY(c, launch_unpack_tiled((const uint8_t *) src, ss, (uint8_t *) dst, ds, R, K, nmat, c->st));
    return FL_OK;
}
extern "C" int fl_rmsnorm_dev(FLCtx * c, const float * x, const float * w, float * y, int n, int D, float eps) {
    if (!c) { return FL_EINVAL; }
    if (n < 0 || D <= 0) { return fail(c, FL_EINVAL, "bad shape"); }
    if (n > 0 && (!x || !y)) { return fail(c, FL_EINVAL, "null pointer"); }
    TRY(c, launch_rmsnorm(x, w, y, n, D, eps, c->st));
    return FL_OK;
}
extern "C" int fl_synth_iq2xxs(FLCtx * c, void * dst, size_t ds, int R, int K, int nmat, int layout, uint64_t seed, uint64_t mat0, float sigma) {
    if (!c) { return FL_EINVAL; }
    if (int rc = pack_args(c, dst, dst, R, K, nmat)) { return rc; }
    if (layout != FL_LAYOUT_GGML && layout != FL_LAYOUT_TILED) { return fail(c, FL_EINVAL, "unknown layout %d", layout); }
    TRY(c, launch_synth_iq2((uint8_t *) dst, ds, R, K, nmat, layout, seed, mat0, sigma, c->st));
    return FL_OK;
}
extern "C" int fl_synth_normal(FLCtx * c, float * dst, int64_t count, uint64_t seed, uint64_t stream, float mean, float sigma) {
    if (!c) { return FL_EINVAL; }
    if (count < 0 || (count > 0 && !dst)) { return fail(c, FL_EINVAL, "bad destination"); }
    TRY(c, launch_synth_normal(dst, count, seed, stream, mean, sigma, c->st));
    return FL_OK;
}
extern "C" int fl_probe_exp(FLCtx * c, const float * x, float * y, int64_t n, int which) {
    if (!c) { return FL_EINVAL; }
    if (n < 0 || which < 0 || which > 2 || (n > 0 && (!x || !y))) { return fail(c, FL_EINVAL, "bad probe arguments"); }
    TRY(c, launch_expf_probe(x, y, n, which, c->st));
    return FL_OK;
}

// ================================================================ persistent expert kernels: scratch and counters
// block-term scratch sized for `rows` slots of both passes; the self-resetting counters are zeroed once, here
int ensure_expert_scratch(FLCtx * c, size_t rows, int E, int H) {
    const size_t need = std::max(experts_terms_floats(2, (int) rows, H, E), experts_terms_floats(1, (int) rows, E, H));
    ALLOC(c, c->terms, need);
    if (!c->cnt.p) {
        ALLOC(c, c->cnt, CNT_ALL);
        TRY(c, hipMemset(c->cnt.p, 0, CNT_ALL * sizeof(unsigned)));
        TRY(c, experts_init());
    }
    if (!c->tab.p) {
        ALLOC(c, c->tab, TAB_BYTES / 16);
        TRY(c, build_table_image(c->tab.p, c->st));
    }
    return FL_OK;
}
ExpertArgs expert_args(FLCtx * c, int n, int P, int shared) {
    ExpertArgs a{};
    a.n = n; a.P = P; a.shared = shared; a.terms = c->terms.p; a.tab = c->tab.p;
    return a;
}

// the single-launch decode block is available (cooperative launch, one resident workgroup per CU)
static bool decode_ready(FLCtx * c) {
    if (c->dec_grid < 0) {
        int coop = 0;
        if (hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, c->dev) != hipSuccess || !coop) { (void) hipGetLastError(); c->dec_grid = 0; return false; }
        int g = 0;
        if (decode_init(c->ncu, &g) != hipSuccess) { (void) hipGetLastError(); g = 0; }
        c->dec_grid = g;
    }
    return c->dec_grid > 0;
}

// the decode-1 kernel organised by XCD is available (a 256-CU device) and selected
static bool decode1_ready(FLCtx * c) {
    if (c->d1_ok < 0) {
        int ok = 0;
        if (decode1_init(c->ncu, &ok) != hipSuccess) { (void) hipGetLastError(); ok = 0; }
        c->d1_ok = ok;
    }
    return c->d1 && c->d1_ok > 0;
}
// the single-launch blocks' shared state: error word, tagged buffers and a new epoch per launch (the buffers cleared on
// first use and whenever the epoch wraps, so no stale word can carry the new epoch)
static int decode_tagged(FLCtx * c, hipStream_t st) {
    if (!c->derr.p) { ALLOC(c, c->derr, 1); TRY(c, hipMemsetAsync(c->derr.p, 0, sizeof(int), st)); }
    if (!c->dlogit.p) {
        ALLOC(c, c->dlogit, DEC_TLOGITS); ALLOC(c, c->dth, DEC_TH); ALLOC(c, c->dto, DEC_TO); ALLOC(c, c->dxq, decode_xq_bytes() / 8);
        c->epoch = 0;
    }
    if (++c->epoch == 0) { c->epoch = 1; }   // epoch 0 is the cleared state of the tagged words
    if (c->epoch == 1) {
        TRY(c, hipMemsetAsync(c->dlogit.p, 0, DEC_TLOGITS * sizeof(uint64_t), st));
        TRY(c, hipMemsetAsync(c->dth.p, 0, DEC_TH * sizeof(uint64_t), st));
        TRY(c, hipMemsetAsync(c->dto.p, 0, DEC_TO * sizeof(uint64_t), st));
        TRY(c, hipMemsetAsync(c->dxq.p, 0, decode_xq_bytes(), st));   // its tagged words
    }
    return FL_OK;
}
// the n <= 8 block may share each XCD's Q8_K of the tokens: a grid of 256 workgroups that the dispatch places
// round-robin over the 8 XCDs (decode1_init's probe)
static uint8_t * decode_xq(FLCtx * c) {
    if (c->d1_ok < 0) { (void) decode1_ready(c); }
    return c->dec_grid == 256 && c->d1_ok > 0 ? reinterpret_cast<uint8_t *>(c->dxq.p) : nullptr;
}
bool decode1_available(FLCtx * c) { return c->fused != 0 && decode_ready(c) && decode1_ready(c); }
bool decode_block_available(FLCtx * c) { return c->fused != 0 && decode_ready(c); }
int decode_picks(FLCtx * c, DecodeArgs & d) {
    if (int rc = decode_tagged(c, c->st)) { return rc; }
    d.tab = c->tab.p; d.tlogits = c->dlogit.p; d.th = c->dth.p; d.to = c->dto.p; d.xqx = decode_xq(c);
    d.epoch = c->epoch; d.err = c->derr.p; d.herr = c->herr ? c->herr_dev : nullptr;
    if (d.n == 1 && d.topk == MAXK && d.keep == MAXK && decode1_ready(c)) {
        TRY(c, launch_moe_decode1(d, c->fused == 1, c->st));
        c->last_kernel = 2;
    } else {
        TRY(c, launch_moe_decode(d, c->dec_grid, c->fused == 1, c->st));
        c->last_kernel = 1;
    }
    c->last_fused = 1;
    return FL_OK;
}
static hipError_t launch_decode(FLCtx * c, const DecodeArgs & d, hipStream_t st) {
    if (d.n == 1 && d.topk == MAXK && d.keep == MAXK && decode1_ready(c)) { c->last_kernel = 2; return launch_moe_decode1(d, c->fused == 1, st); }
    c->last_kernel = 1;
    return launch_moe_decode(d, c->dec_grid, c->fused == 1, st);
}

// ================================================================ the device-resident block
// the block on x, or on RMSNorm(x) * nw when prenorm (nw may be null: ones); resid (may be null) is added to the output
// bytes of one R x K matrix in format f (IQ2_XXS or a K-quant)
static size_t fmt_mat_bytes(int f, int R, int K) { return (size_t) R * (K / 256) * (size_t) (f == FL_IQ2 ? IQ2B : kq_block_bytes(f)); }
// K-quant mat-vec of one matrix (ggml layout, in place) on n Q8_K rows -> out [n][R]
static hipError_t kq_one(FLCtx * c, int fmt, const void * w, const int8_t * q, const float * d, int n, int K, int R, float * out, hipStream_t st) {
    KqArgs k{};
    k.w = (const uint8_t *) w; k.estride = fmt_mat_bytes(fmt, R, K); k.aq = q; k.ad = d; k.K = K; k.R = R;
    k.n = n; k.out = out; k.ldo = R;
    return launch_kq_matvec(k, fmt, n, 1, st);
}

// The shared expert outside the GEMM columns / the routed tasks (fl_moe_layer, formats c->lf), on the context's buffers.
// Gate/up: h rows P .. P + n - 1 and their Q8_K from the rows' Q8_K (xq / xd): K-quants (src/fused_layer.cu:520-523)
// by one mat-vec launch for both matrices (or one each) and swiglu_q8k; IQ2_XXS by the per-pass kernel on an empty
// routed list.
// h = silu(g) * u of the shared expert's K-quant gate / up outputs (ksg, ksu) into rows P .. P + n - 1 of h and Q8_K(h)
static int shared_swiglu(FLCtx * c, int n, int P, int H, hipStream_t st) {
    TRY(c, launch_swiglu_q8k(c->ksg.p, c->ksu.p, n, H, c->h.p + (size_t) P * H, c->hq.p + (size_t) P * H, c->hd.p + (size_t) P * (H / 256), st));
    if (c->dbg_gu) {
        TRY(c, hipMemcpyAsync(c->g.p + (size_t) P * H, c->ksg.p, (size_t) n * H * 4, hipMemcpyDeviceToDevice, st));
        TRY(c, hipMemcpyAsync(c->u.p + (size_t) P * H, c->ksu.p, (size_t) n * H * 4, hipMemcpyDeviceToDevice, st));
    }
    return FL_OK;
}
static int shared_gateup_sep(FLCtx * c, const FLMoeLayer * L, int n, int P, int E, int H, int tk, hipStream_t st) {
    const int * lf = c->lf;
    if (lf[1] == FL_IQ2) {
        ExpertArgs s = expert_args(c, n, P, 1);
        s.sh[0] = (const uint8_t *) L->sh_gate; s.sh[1] = (const uint8_t *) L->sh_up; s.aq = c->xq.p; s.ad = c->xd.p; s.K = E; s.R = H; s.nmat = 2;
        s.act = zero_int(c); s.nact = zero_int(c); s.offsets = zero_int(c); s.perm = zero_int(c); s.topk = tk;
        s.h = c->h.p; s.hq = c->hq.p; s.hd = c->hd.p;
        s.gdbg = c->dbg_gu ? c->g.p : nullptr; s.udbg = c->dbg_gu ? c->u.p : nullptr;
        expert_counters(c, s, 0);
        TRY(c, launch_experts_gateup(s, c->ncu, st));
        return FL_OK;
    }
    ALLOC(c, c->ksg, (size_t) n * H); ALLOC(c, c->ksu, (size_t) n * H);
    if (lf[1] == lf[2]) {   // gate and up in one launch
        KqArgs k{};
        k.w = (const uint8_t *) L->sh_gate; k.w2 = (const uint8_t *) L->sh_up; k.estride = fmt_mat_bytes(lf[1], H, E);
        k.aq = c->xq.p; k.ad = c->xd.p; k.K = E; k.R = H; k.n = n; k.out = c->ksg.p; k.out2 = c->ksu.p; k.ldo = H;
        TRY(c, launch_kq_matvec(k, lf[1], n, 1, st));
    } else {
        TRY(c, kq_one(c, lf[1], L->sh_gate, c->xq.p, c->xd.p, n, E, H, c->ksg.p, st));
        TRY(c, kq_one(c, lf[2], L->sh_up, c->xq.p, c->xd.p, n, E, H, c->ksu.p, st));
    }
    return shared_swiglu(c, n, P, H, st);
}
// Down: o rows P .. P + n - 1 from h's Q8_K (hq / hd rows P ..): a K-quant mat-vec, or the per-pass kernel alone.
static int shared_down_sep(FLCtx * c, const FLMoeLayer * L, int n, int P, int E, int H, int tk, hipStream_t st) {
    if (c->lf[3] != FL_IQ2) {
        TRY(c, kq_one(c, c->lf[3], L->sh_down, c->hq.p + (size_t) P * H, c->hd.p + (size_t) P * (H / 256), n, H, E, c->o.p + (size_t) P * E, st));
        return FL_OK;
    }
    ExpertArgs s = expert_args(c, n, P, 1);
    s.sh[0] = (const uint8_t *) L->sh_down; s.sh[1] = nullptr; s.aq = c->hq.p; s.ad = c->hd.p; s.K = H; s.R = E; s.nmat = 1;
    s.act = zero_int(c); s.nact = zero_int(c); s.offsets = zero_int(c); s.perm = zero_int(c); s.topk = tk;
    s.h = nullptr; s.hq = nullptr; s.hd = nullptr; s.o = c->o.p; s.y = nullptr;
    expert_counters(c, s, 1);
    TRY(c, launch_experts_down(s, c->ncu, st));
    return FL_OK;
}
// The routed down in a K-quant (src/fused_layer.cu:607-608): o of every routed slot, each active expert's slots in
// token groups sized for the expected slots per expert (an expert with more runs extra groups).
static hipError_t routed_down_kq(FLCtx * c, const FLMoeLayer * L, int P, int E, int H, int ne) {
    KqArgs k{};
    k.w = (const uint8_t *) L->down_exps; k.estride = fmt_mat_bytes(c->lf[0], E, H); k.aq = c->hq.p; k.ad = c->hd.p; k.K = H; k.R = E;
    k.act = c->act.p; k.nact = c->nact.p; k.offsets = c->offsets.p; k.out = c->o.p; k.ldo = E;
    return launch_kq_matvec(k, c->lf[0], (P + ne - 1) / ne, ne < P ? ne : P, c->st);
}

// the grouped GEMMs' one-time set-up on this context: fp16 table image, launch attributes, error word
int prefill_ready(FLCtx * c) {
    if (c->pf_ready) { return FL_OK; }
    ALLOC(c, c->ptab, prefill_table_bytes() / 16);
    TRY(c, build_prefill_tables(c->ptab.p, c->st));
    TRY(c, prefill_init());
    TRY(c, kq_gemm_init());
    if (!c->derr.p) { ALLOC(c, c->derr, 1); TRY(c, hipMemsetAsync(c->derr.p, 0, sizeof(int), c->st)); }
    c->pf_ready = 1;
    return FL_OK;
}

static int moe_layer(FLCtx * c, const FLMoeLayer * L, const float * x, int n, float * y, bool prenorm, const float * nw, float eps,
                     const float * resid) {
    if (!c) { return FL_EINVAL; }
    if (!L) { return fail(c, FL_EINVAL, "null layer"); }
    if (n < 0 || n > 65536) { return fail(c, FL_ERANGE, "n = %d outside 0..65536", n); }
    if (L->layout != FL_LAYOUT_TILED) { return fail(c, FL_EINVAL, "fl_moe_layer reads the tiled layout; convert with fl_pack_iq2xxs"); }
    if (L->E <= 0 || L->E % 1024 || L->H <= 0 || L->H % 1024) { return fail(c, FL_EINVAL, "E %d and H %d must be positive multiples of 1024", L->E, L->H); }
    if (int rc = check_rule(c, L->n_exp)) { return rc; }
    if (c->herr) {   // an earlier launch on this context failed (seen without waiting); fl_sync reports and clears it
        const int e = __atomic_load_n(c->herr, __ATOMIC_ACQUIRE);
        if (e) { return fail(c, FL_EHIP, "an earlier launch on this context reported device error code %d; call fl_sync", e); }
    }
    if (n == 0) { return FL_OK; }
    if (!x || !y || !L->gate_inp || !L->probs_b || !L->gate_exps || !L->up_exps || !L->down_exps || !L->sh_gate || !L->sh_up || !L->sh_down) {
        return fail(c, FL_EINVAL, "null pointer in the layer or x / y");
    }
    if (c->keep > c->topk) { return fail(c, FL_EINVAL, "keep %d above topk %d", c->keep, c->topk); }
    // the selection draws topk experts per row; the block runs the kept ones (fl_set_keep), tk per row
    const int E = L->E, H = L->H, ne = L->n_exp, tsel = c->topk, tk = c->keep > 0 ? c->keep : tsel, P = n * tk;
    const float renorm = c->keep > 0 ? c->renorm : 0.f;
    const bool share = c->share && c->keep > 0 && tk < tsel && n > 1;   // the --share-experts keep across the rows
    const int * lf = c->lf;
    const bool kq = lf[0] != FL_IQ2 || lf[1] != FL_IQ2 || lf[2] != FL_IQ2 || lf[3] != FL_IQ2;
    {
        const size_t mg = (size_t) H * (E / 256) * IQ2B;   // one gate/up matrix
        if (!covers(L->gate_inp, (size_t) ne * E * 4) || !covers(L->probs_b, (size_t) ne * 4) || !covers(x, (size_t) n * E * 4) ||
            !covers(y, (size_t) n * E * 4) || !covers(L->gate_exps, ne * mg) || !covers(L->up_exps, ne * mg) ||
            !covers(L->down_exps, ne * fmt_mat_bytes(lf[0], E, H)) || !covers(L->sh_gate, fmt_mat_bytes(lf[1], H, E)) ||
            !covers(L->sh_up, fmt_mat_bytes(lf[2], H, E)) || !covers(L->sh_down, fmt_mat_bytes(lf[3], E, H))) {
            return fail(c, FL_EINVAL, "an allocation of the layer, x or y is smaller than its shape (%d experts, E %d, H %d, n %d)", ne, E, H, n);
        }
        if (prenorm && nw && !covers(nw, (size_t) E * 4)) { return fail(c, FL_EINVAL, "the norm weight is smaller than E = %d floats", E); }
        const void * km[4] = { L->down_exps, L->sh_gate, L->sh_up, L->sh_down };
        for (int i = 0; i < 4; ++i) {
            if (lf[i] != FL_IQ2 && (reinterpret_cast<uintptr_t>(km[i]) & 3u)) { return fail(c, FL_EINVAL, "K-quant matrices must be 4-byte aligned"); }
        }
        if (prenorm && !(eps >= 0.f)) { return fail(c, FL_EINVAL, "bad norm eps %g", (double) eps); }
    }
    const size_t rows = (size_t) P + n;
    // K-quant matrices: at decode sizes the per-pass path (the n <= 8 decode block reads IQ2_XXS tiles), except for
    // one token on the real shards' formats (routed down Q2_K / Q3_K, shared expert Q5_K / Q5_K / Q6_K), which the
    // one-token kernel reads in place; at prefill sizes the routed gate/up (always IQ2_XXS) on the MFMA GEMM and the
    // K-quant matrices on the K-quant mat-vecs
    static_assert(FL_Q6K == 1 && FL_Q5K == 3 && FL_Q2K == 5 && FL_Q3K == 6, "the FL_ codes are the K-quant kernels' format codes");
    const int kd1 = (lf[0] == FL_Q2K || lf[0] == FL_Q3K) && lf[1] == FL_Q5K && lf[2] == FL_Q5K && lf[3] == FL_Q6K ? lf[0] : 0;
    const bool kq1 = kq && kd1 != 0 && n == 1 && tsel == MAXK && tk == MAXK && decode1_ready(c);
    const bool fused = (!kq || kq1) && c->fused && n <= 8 && E == 7168 && H == 2048 && decode_rule_ok(ne, c->n_group) && decode_ready(c);
    const bool mfma = !fused && c->pf_mfma && n > 8 && E == 7168 && H == 2048;
    ALLOC(c, c->xq, (size_t) n * E); ALLOC(c, c->xd, (size_t) n * (E / 256));
    ALLOC(c, c->logits, (size_t) n * ne); ALLOC(c, c->probs, (size_t) n * ne);
    ALLOC(c, c->sel, P); ALLOC(c, c->wts, P); ALLOC(c, c->perm, P); ALLOC(c, c->inv, P);
    ALLOC(c, c->counts, ne); ALLOC(c, c->offsets, ne + 1); ALLOC(c, c->act, ne); ALLOC(c, c->nact, 1);
    if (!fused) { ALLOC(c, c->h, rows * H); ALLOC(c, c->hq, rows * H); ALLOC(c, c->hd, rows * (H / 256)); ALLOC(c, c->o, rows * E); }
    if (c->dbg_gu) { ALLOC(c, c->g, rows * H); ALLOC(c, c->u, rows * H); }
    if (int rc = ensure_expert_scratch(c, rows, E, H)) { return rc; }
    c->last_n = n; c->last_P = P; c->last_fused = fused ? 1 : 0; c->last_kernel = 0;
    hipStream_t st = c->st;
    std::vector<hipEvent_t> * ev = prof_begin(c);
    if (fused) {
        if (int rc = decode_tagged(c, st)) { return rc; }
        DecodeArgs d{};
        d.tab = c->tab.p; d.x = x; d.n = n; d.prenorm = prenorm ? 1 : 0; d.nw = nw; d.eps = eps; d.resid = resid;
        d.Wr = L->gate_inp; d.bias = L->probs_b; d.n_exp = ne; d.n_group = c->n_group; d.topk_group = c->topk_group; d.topk = tsel; d.scale = c->scale;
        d.keep = tk; d.renorm = renorm; d.share = share ? 1 : 0;
        d.gate = (const uint8_t *) L->gate_exps; d.up = (const uint8_t *) L->up_exps; d.down = (const uint8_t *) L->down_exps;
        d.estride = (size_t) H * (E / 256) * IQ2B;
        d.sh_gate = (const uint8_t *) L->sh_gate; d.sh_up = (const uint8_t *) L->sh_up; d.sh_down = (const uint8_t *) L->sh_down;
        d.kdown = kq ? kd1 : 0; d.dstride = fmt_mat_bytes(lf[0], E, H);
        d.E = E; d.H = H;
        d.xq = c->xq.p; d.xd = c->xd.p; d.logits = c->logits.p; d.probs = c->probs.p; d.sel = c->sel.p; d.wts = c->wts.p;
        d.counts = c->counts.p; d.offsets = c->offsets.p; d.perm = c->perm.p; d.inv = c->inv.p; d.act = c->act.p; d.nact = c->nact.p;
        d.tlogits = c->dlogit.p; d.th = c->dth.p; d.to = c->dto.p; d.xqx = decode_xq(c); d.y = y;
        d.epoch = c->epoch; d.err = c->derr.p; d.herr = c->herr ? c->herr_dev : nullptr;
        // stages: the whole block is one launch, reported as stage 4; the others are empty
        for (int i = 0; i <= 4; ++i) { prof_mark(c, ev, i); }
        TRY(c, launch_decode(c, d, st));
        prof_mark(c, ev, 5); prof_mark(c, ev, 6);
        return FL_OK;
    }
    if (mfma) {
        if (int rc = prefill_ready(c)) { return rc; }
        ALLOC(c, c->xh, (size_t) n * E); ALLOC(c, c->hh, rows * H);
        ALLOC(c, c->pcols, rows / 32 + NEXP_MAX + 2); ALLOC(c, c->pncols, PF_NCOLS);
    }
    prof_mark(c, ev, 0);
    if (prenorm) {   // the per-pass path normalises into a context buffer first (k_rmsnorm: the same arithmetic)
        ALLOC(c, c->xn, (size_t) n * E);
        TRY(c, launch_rmsnorm(x, nw, c->xn.p, n, E, eps, st));
        x = c->xn.p;
    }
    TRY(c, launch_quant_q8k(x, n, E, c->xq.p, c->xd.p, st));
    if (mfma) { TRY(c, launch_q8_to_h(c->xq.p, c->xh.p, (int64_t) n * E, st)); }
    prof_mark(c, ev, 1);
    double * rp = nullptr;   // the K-split tiles' parts (n from RL_SPLIT_MIN to RL_SPLIT_MAX)
    if (const size_t nd = router_split_doubles(n, ne, E)) { ALLOC(c, c->rpart, nd); rp = c->rpart.p; }
    TRY(c, launch_router_logits(L->gate_inp, x, n, ne, E, c->logits.p, rp, st));
    prof_mark(c, ev, 2);
    if (share) {   // every row's topk picks, then the keep across the rows
        ALLOC(c, c->sel8, (size_t) n * tsel); ALLOC(c, c->w8, (size_t) n * tsel);
        TRY(c, launch_router_select(c->logits.p, L->probs_b, n, ne, c->n_group, c->topk_group, tsel, c->scale, c->probs.p, c->sel8.p, c->w8.p, st, tsel, 0.f));
        TRY(c, launch_keep_share(c->sel8.p, c->w8.p, n, tsel, tk, renorm, c->sel.p, c->wts.p, st));
    } else {
        TRY(c, launch_router_select(c->logits.p, L->probs_b, n, ne, c->n_group, c->topk_group, tsel, c->scale, c->probs.p, c->sel.p, c->wts.p, st, tk, renorm));
    }
    prof_mark(c, ev, 3);
    int * dsc = nullptr;
    if (const size_t nd = dispatch_scratch_ints(P)) { ALLOC(c, c->dscr, nd); dsc = c->dscr.p; }
    TRY(c, launch_dispatch(c->sel.p, P, ne, c->counts.p, c->offsets.p, c->perm.p, c->inv.p, c->act.p, c->nact.p, st, dsc));
    if (mfma) {
        TRY(c, launch_prefill_cols(c->act.p, c->nact.p, c->offsets.p, n, P, c->pcols.p, c->pncols.p, st));
        prof_mark(c, ev, 4);
        // Columns: the shared expert's first (nsh of them), then the routed experts'. Each matrix runs where its format
        // does: IQ2_XXS on the IQ2_XXS GEMM, Q2_K / Q3_K / Q6_K downs and a Q5_K shared gate / up on the K-quant GEMM,
        // any other K-quant on the mat-vecs.
        const int nsh = prefill_shared_cols(n);
        PrefillArgs g{};
        g.ptab = c->ptab.p; g.w[0] = (const uint8_t *) L->gate_exps; g.w[1] = (const uint8_t *) L->up_exps;
        g.estride = (size_t) H * (E / 256) * IQ2B; g.sh[0] = (const uint8_t *) L->sh_gate; g.sh[1] = (const uint8_t *) L->sh_up;
        g.perm = c->perm.p; g.topk = tk; g.P = P; g.R = H; g.K = E; g.nmat = 2; g.cols = c->pcols.p; g.ncols = c->pncols.p;
        g.bh = c->xh.p; g.bd = c->xd.p; g.out = c->h.p; g.gdbg = c->dbg_gu ? c->g.p : nullptr; g.udbg = c->dbg_gu ? c->u.p : nullptr;
        g.err = c->derr.p; g.herr = c->herr ? c->herr_dev : nullptr;
        g.col0 = lf[1] == FL_IQ2 ? 0 : nsh;
        TRY(c, launch_prefill_gemm(g, c->ncu, st));
        if (lf[1] == FL_Q5K && lf[2] == FL_Q5K) {   // the real shards' shared gate / up: ksg / ksu rows 0 .. n - 1
            ALLOC(c, c->ksg, (size_t) n * H); ALLOC(c, c->ksu, (size_t) n * H);
            for (int m = 0; m < 2; ++m) {
                PrefillArgs k{};
                k.sh[0] = (const uint8_t *) (m ? L->sh_up : L->sh_gate); k.w[0] = k.sh[0];
                k.R = H; k.K = E; k.cols = c->pcols.p; k.ncols = c->pncols.p; k.col0 = 0; k.col1 = nsh;
                k.bh = c->xh.p; k.bd = c->xd.p; k.arow0 = P; k.orow0 = P; k.out = m ? c->ksu.p : c->ksg.p;
                TRY(c, launch_kq_gemm(k, FL_Q5K, c->ncu, st));
            }
            if (int rc = shared_swiglu(c, n, P, H, st)) { return rc; }
        } else if (lf[1] != FL_IQ2) {
            if (int rc = shared_gateup_sep(c, L, n, P, E, H, tk, st)) { return rc; }
        }
        TRY(c, launch_quant_q8k(c->h.p, (int64_t) rows, H, c->hq.p, c->hd.p, st));
        TRY(c, launch_q8_to_h(c->hq.p, c->hh.p, (int64_t) rows * H, st));
        prof_mark(c, ev, 5);
        PrefillArgs d = g;   // the down pass: activations Q8_K(h) of every slot, o rows by slot
        d.w[0] = (const uint8_t *) L->down_exps; d.w[1] = nullptr; d.sh[0] = (const uint8_t *) L->sh_down; d.sh[1] = nullptr;
        d.R = E; d.K = H; d.nmat = 1; d.bh = c->hh.p; d.bd = c->hd.p; d.out = c->o.p; d.gdbg = nullptr; d.udbg = nullptr;
        const bool sh_iq = lf[3] == FL_IQ2, sh_kg = lf[3] == FL_Q2K || lf[3] == FL_Q3K || lf[3] == FL_Q6K;
        if (lf[0] == FL_IQ2) {   // routed (+ the shared expert when it is IQ2_XXS)
            d.col0 = sh_iq ? 0 : nsh;
            TRY(c, launch_prefill_gemm(d, c->ncu, st));
        } else {
            PrefillArgs k = d;
            k.estride = fmt_mat_bytes(lf[0], E, H); k.col0 = nsh;
            TRY(c, launch_kq_gemm(k, lf[0], c->ncu, st));
            if (sh_iq) { d.col0 = 0; d.col1 = nsh; TRY(c, launch_prefill_gemm(d, c->ncu, st)); }
        }
        if (sh_kg) {
            PrefillArgs k = d;
            k.col0 = 0; k.col1 = nsh;
            TRY(c, launch_kq_gemm(k, lf[3], c->ncu, st));
        } else if (!sh_iq) {
            if (int rc = shared_down_sep(c, L, n, P, E, H, tk, st)) { return rc; }
        }
        TRY(c, launch_combine(c->o.p, c->inv.p, c->wts.p, n, tk, E, P, resid, y, nullptr, st));
        prof_mark(c, ev, 6);
        return FL_OK;
    }
    prof_mark(c, ev, 4);
    const bool ksh = lf[1] != FL_IQ2;   // the shared gate / up in K-quants: run beside the routed IQ2_XXS tasks
    ExpertArgs a = expert_args(c, n, P, ksh ? 0 : 1);
    a.w[0] = (const uint8_t *) L->gate_exps; a.w[1] = (const uint8_t *) L->up_exps; a.estride = (size_t) H * (E / 256) * IQ2B;
    a.sh[0] = (const uint8_t *) L->sh_gate; a.sh[1] = (const uint8_t *) L->sh_up;
    a.aq = c->xq.p; a.ad = c->xd.p; a.K = E; a.R = H; a.nmat = 2;
    a.act = c->act.p; a.nact = c->nact.p; a.offsets = c->offsets.p; a.perm = c->perm.p; a.topk = tk;
    a.h = c->h.p; a.hq = c->hq.p; a.hd = c->hd.p;
    a.gdbg = c->dbg_gu ? c->g.p : nullptr; a.udbg = c->dbg_gu ? c->u.p : nullptr;
    expert_counters(c, a, 0);
    // A K-quant shared expert (one latency-bound mat-vec of 10-12 MB per matrix) runs on the side stream beside the
    // routed launches: it reads x's Q8_K and writes only its own rows (h / Q8_K(h) rows P .. P + n - 1, o rows P ..,
    // ksg / ksu), which no routed kernel touches; the combine waits for it.
    const bool side = ksh && kq && lf[3] != FL_IQ2 && !c->no_side;
    if (side) {
        ALLOC(c, c->ksg, (size_t) n * H); ALLOC(c, c->ksu, (size_t) n * H);
        TRY(c, hipEventRecord(c->efork, st)); TRY(c, hipStreamWaitEvent(c->side, c->efork, 0));
        if (int rc = shared_gateup_sep(c, L, n, P, E, H, tk, c->side)) { return rc; }
        if (int rc = shared_down_sep(c, L, n, P, E, H, tk, c->side)) { return rc; }
        TRY(c, hipEventRecord(c->ejoin, c->side));
    }
    TRY(c, launch_experts_gateup(a, c->ncu, st));
    if (ksh && !side) { if (int rc = shared_gateup_sep(c, L, n, P, E, H, tk, st)) { return rc; } }   // h rows P .. P + n - 1
    prof_mark(c, ev, 5);
    if (kq) {   // o of every slot by its matrix's format, then the k-ordered combine (+ shared, + residual)
        if (lf[0] == FL_IQ2) {
            ExpertArgs d = a;
            d.shared = 0; d.aq = c->hq.p; d.ad = c->hd.p; d.K = H; d.R = E; d.nmat = 1;
            d.h = nullptr; d.hq = nullptr; d.hd = nullptr; d.gdbg = nullptr; d.udbg = nullptr; d.o = c->o.p; d.y = nullptr;
            d.w[0] = (const uint8_t *) L->down_exps; d.w[1] = nullptr; d.sh[0] = nullptr; d.sh[1] = nullptr;
            expert_counters(c, d, 1);
            TRY(c, launch_experts_down(d, c->ncu, st));
        } else {
            TRY(c, routed_down_kq(c, L, P, E, H, ne));
        }
        if (side) { TRY(c, hipStreamWaitEvent(st, c->ejoin, 0)); }
        else if (int rc = shared_down_sep(c, L, n, P, E, H, tk, st)) { return rc; }
        TRY(c, launch_combine(c->o.p, c->inv.p, c->wts.p, n, tk, E, P, resid, y, nullptr, st));
        prof_mark(c, ev, 6);
        return FL_OK;
    }
    ExpertArgs d = a;
    d.w[0] = (const uint8_t *) L->down_exps; d.w[1] = nullptr; d.sh[0] = (const uint8_t *) L->sh_down; d.sh[1] = nullptr;
    d.aq = c->hq.p; d.ad = c->hd.p; d.K = H; d.R = E; d.nmat = 1;
    d.h = nullptr; d.hq = nullptr; d.hd = nullptr; d.gdbg = nullptr; d.udbg = nullptr;
    // the down kernel's fused combine has no residual term: with one, the k-ordered combine runs after it
    d.o = c->o.p; d.inv = c->inv.p; d.wts = c->wts.p; d.y = resid ? nullptr : y;
    expert_counters(c, d, 1);
    TRY(c, launch_experts_down(d, c->ncu, st));
    if (resid) { TRY(c, launch_combine(c->o.p, c->inv.p, c->wts.p, n, tk, E, P, resid, y, nullptr, st)); }
    prof_mark(c, ev, 6);
    return FL_OK;
}
extern "C" int fl_set_layer_formats(FLCtx * c, int down_fmt, int sh_gate_fmt, int sh_up_fmt, int sh_down_fmt) {
    if (!c) { return FL_EINVAL; }
    const int f[4] = { down_fmt, sh_gate_fmt, sh_up_fmt, sh_down_fmt };
    for (int i = 0; i < 4; ++i) {
        if (f[i] != FL_IQ2 && kq_block_bytes(f[i]) == 0) { return fail(c, FL_EINVAL, "format %d is not IQ2_XXS or a K-quant (Q2_K, Q3_K, Q5_K, Q6_K)", f[i]); }
    }
    if ((sh_gate_fmt == FL_IQ2) != (sh_up_fmt == FL_IQ2)) { return fail(c, FL_EINVAL, "shared gate and up must both be IQ2_XXS or both K-quants"); }
    for (int i = 0; i < 4; ++i) { c->lf[i] = f[i]; }
    return FL_OK;
}

extern "C" int fl_moe_layer(FLCtx * c, const FLMoeLayer * L, const float * x, int n, float * y) {
    return moe_layer(c, L, x, n, y, false, nullptr, 0.f, nullptr);
}
extern "C" int fl_moe_layer_normed(FLCtx * c, const FLMoeLayer * L, const float * ffn_norm, float eps, const float * h, int n,
                                   int residual, float * y) {
    if (c && residual && h == y) { return fail(c, FL_EINVAL, "h and y must not alias when the residual is added"); }
    return moe_layer(c, L, h, n, y, true, ffn_norm, eps, residual ? h : nullptr);
}

// fl_moe_layer for decode batches with no device allocation: the single-launch decode block on the file-scope scratch of
// the context's device (routing outputs, tagged hand-off words, table image, error word) instead of the context's
// buffers. Every call enqueues the same two kernels with arguments that depend only on its own inputs -- a fill kernel
// that clears the tagged words, then the decode block tagging them with the fixed epoch NA_EPOCH -- and changes no
// host-side state, so a call captured into a HIP graph stays correct on every replay (a consumer's wait is satisfied
// only by a word this call's launch wrote). Calls that overlap on one device race on the scratch.
extern "C" int fl_moe_layer_noalloc(FLCtx * c, const FLMoeLayer * L, const float * x, int n, float * y) {
    if (!c) { return FL_EINVAL; }
    if (!L || !x || !y) { return fail(c, FL_EINVAL, "null layer, x or y"); }
    if (n < 1 || n > NA_MAXN) { return fail(c, FL_ERANGE, "fl_moe_layer_noalloc: n = %d outside 1..%d (its scratch holds one decode batch)", n, NA_MAXN); }
    if (L->layout != FL_LAYOUT_TILED || L->E != 7168 || L->H != 2048) {
        return fail(c, FL_ESCOPE, "fl_moe_layer_noalloc runs the decode block only: tiled IQ2_XXS, E 7168, H 2048");
    }
    for (int i = 0; i < 4; ++i) { if (c->lf[i] != FL_IQ2) { return fail(c, FL_ESCOPE, "fl_moe_layer_noalloc reads IQ2_XXS matrices only"); } }
    if (int rc = check_rule(c, L->n_exp)) { return rc; }
    if (!decode_rule_ok(L->n_exp, c->n_group)) { return fail(c, FL_ESCOPE, "routing rule outside the decode block's selection"); }
    if (c->keep > c->topk) { return fail(c, FL_EINVAL, "keep %d above topk %d", c->keep, c->topk); }
    if (!L->gate_inp || !L->probs_b || !L->gate_exps || !L->up_exps || !L->down_exps || !L->sh_gate || !L->sh_up || !L->sh_down) {
        return fail(c, FL_EINVAL, "null pointer in the layer");
    }
    {
        const size_t mg = (size_t) 2048 * 28 * IQ2B;
        const int ne = L->n_exp;
        if (!covers(L->gate_inp, (size_t) ne * 7168 * 4) || !covers(L->probs_b, (size_t) ne * 4) || !covers(x, (size_t) n * 7168 * 4) ||
            !covers(y, (size_t) n * 7168 * 4) || !covers(L->gate_exps, ne * mg) || !covers(L->up_exps, ne * mg) ||
            !covers(L->down_exps, ne * mg) || !covers(L->sh_gate, mg) || !covers(L->sh_up, mg) || !covers(L->sh_down, mg)) {
            return fail(c, FL_EINVAL, "an allocation of the layer, x or y is smaller than its shape");
        }
    }
    if (c->herr) {
        const int e = __atomic_load_n(c->herr, __ATOMIC_ACQUIRE);
        if (e) { return fail(c, FL_EHIP, "an earlier launch on this context reported device error code %d; call fl_sync", e); }
    }
    if (!decode_ready(c)) { return fail(c, FL_ESCOPE, "the single-launch decode block is not available on this device"); }
    uint8_t * S = na_resolve(c->dev);
    if (!S) { return fail(c, FL_EHIP, "hipGetSymbolAddress of the decode scratch failed on device %d", c->dev); }
    if (!g_na[c->dev].ready) { return fail(c, FL_EHIP, "the decode scratch of device %d was not set up by fl_init", c->dev); }
    c->na_used = 1;
    hipStream_t st = c->st;
    // the tagged words (not the error word, which fl_sync reads) back to zero: no word holds NA_EPOCH when the block starts
    k_zero16<<<1024, 256, 0, st>>>(reinterpret_cast<uint4 *>(S + NA_CLEAR0), (NA_ERR - NA_CLEAR0) / 16);
    TRY(c, hipGetLastError());
    const int tk = c->keep > 0 ? c->keep : c->topk;
    DecodeArgs d{};
    d.tab = reinterpret_cast<const uint4 *>(S + NA_TAB); d.x = x; d.n = n; d.prenorm = 0; d.nw = nullptr; d.eps = 0.f; d.resid = nullptr;
    d.Wr = L->gate_inp; d.bias = L->probs_b; d.n_exp = L->n_exp; d.n_group = c->n_group; d.topk_group = c->topk_group;
    d.topk = c->topk; d.scale = c->scale; d.keep = tk; d.renorm = c->keep > 0 ? c->renorm : 0.f;
    d.share = c->share && c->keep > 0 && tk < c->topk && n > 1 ? 1 : 0;
    d.gate = (const uint8_t *) L->gate_exps; d.up = (const uint8_t *) L->up_exps; d.down = (const uint8_t *) L->down_exps;
    d.estride = (size_t) 2048 * 28 * IQ2B;
    d.sh_gate = (const uint8_t *) L->sh_gate; d.sh_up = (const uint8_t *) L->sh_up; d.sh_down = (const uint8_t *) L->sh_down;
    d.E = 7168; d.H = 2048;
    d.xq = reinterpret_cast<int8_t *>(S + NA_XQ); d.xd = reinterpret_cast<float *>(S + NA_XD);
    d.logits = reinterpret_cast<float *>(S + NA_LOG); d.probs = reinterpret_cast<float *>(S + NA_PRB);
    d.sel = reinterpret_cast<int *>(S + NA_SEL); d.wts = reinterpret_cast<float *>(S + NA_WTS);
    d.counts = reinterpret_cast<int *>(S + NA_CNT); d.offsets = reinterpret_cast<int *>(S + NA_OFF);
    d.perm = reinterpret_cast<int *>(S + NA_PERM); d.inv = reinterpret_cast<int *>(S + NA_INV);
    d.act = reinterpret_cast<int *>(S + NA_ACT); d.nact = reinterpret_cast<int *>(S + NA_NACT);
    d.tlogits = reinterpret_cast<uint64_t *>(S + NA_TLOG); d.th = reinterpret_cast<uint64_t *>(S + NA_TH);
    d.to = reinterpret_cast<uint64_t *>(S + NA_TO); d.y = y;
    d.epoch = NA_EPOCH; d.err = reinterpret_cast<int *>(S + NA_ERR); d.herr = c->herr ? c->herr_dev : nullptr;
    TRY(c, launch_decode(c, d, st));
    return FL_OK;
}

extern "C" int fl_set_profile(FLCtx * c, int on) { if (!c) { return FL_EINVAL; } c->prof = on ? 1 : 0; return FL_OK; }

// summed stage durations (ms) of every profiled call since the last reset; ms[NSTAGE], returns the call count
extern "C" int fl_stage_ms(FLCtx * c, double * ms, int nstage, int reset) {
    if (!c) { return FL_EINVAL; }
    for (auto & ev : c->ev_pending) {
        TRY(c, hipEventSynchronize(ev[NSTAGE]));
        for (int i = 0; i < NSTAGE; ++i) { float t = 0.f; TRY(c, hipEventElapsedTime(&t, ev[i], ev[i + 1])); c->stage_ms[i] += t; }
        c->stage_n++; c->ev_free.push_back(ev);
    }
    c->ev_pending.clear();
    for (int i = 0; i < nstage && i < NSTAGE; ++i) { ms[i] = c->stage_ms[i]; }
    const int n = (int) c->stage_n;
    if (reset) { for (double & v : c->stage_ms) { v = 0.0; } c->stage_n = 0; }
    return n;
}

extern "C" int fl_debug(FLCtx * c, FLDebug * out) {
    if (!c || !out) { return FL_EINVAL; }
    std::memset(out, 0, sizeof(FLDebug));
    out->xq = c->xq.p; out->xd = c->xd.p; out->logits = c->logits.p; out->probs = c->probs.p; out->sel = c->sel.p; out->wts = c->wts.p;
    out->counts = c->counts.p; out->offsets = c->offsets.p; out->perm = c->perm.p; out->inv = c->inv.p; out->act = c->act.p; out->nact = c->nact.p;
    if (!c->last_fused) {   // the single-launch block keeps h and o in its epoch-tagged buffers only
        out->h = c->h.p; out->hq = c->hq.p; out->hd = c->hd.p; out->o = c->o.p; out->g = c->dbg_gu ? c->g.p : nullptr; out->u = c->dbg_gu ? c->u.p : nullptr;
    }
    out->n = c->last_n; out->P = c->last_P; out->topk = c->last_n > 0 ? c->last_P / c->last_n : c->topk; out->fused = c->last_fused; out->kernel = c->last_kernel;
    return FL_OK;
}

// ================================================================ reference entry points
extern "C" void fl_attn(FLCtx *, const FLW *, int, int, const int *, void *, void *, const float *, int, int, int) { out_of_scope("fl_attn"); }
extern "C" void fl_spec(FLCtx *, const FLW *, void *, void *) { out_of_scope("fl_spec"); }
extern "C" void fl_sketch(FLCtx *, const float *, const void *, int) { out_of_scope("fl_sketch"); }

extern "C" void fl_wait_event(FLCtx * c, hipEvent_t ev) { CK(hipStreamWaitEvent(c->st, ev, 0)); }
// accumulated GPU time in ms (src/fused_layer.cu:620): 1 = the experts (fl_moe, fl_skip: their launches to their
// stream wait, as the reference times them); 0 and 2 = fl_ffn_begin's work, the MoE tail of the reference's attention
// phase that this library owns (the router, and the copy in of its rows); 3..7 (speculation, attention parts) = 0
extern "C" double fl_gpu_ms(FLCtx * c, int which) {
    if (!c) { return 0.0; }
    fold_ffn_events(c, true);
    return which == 1 ? c->ms_moe : which == 0 || which == 2 ? c->ms_ffn : 0.0;
}
