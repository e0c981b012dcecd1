// fl_ctx.h -- FLCtx (the context behind the C ABI) and host helpers shared by fused_layer.hip and compat.hip.
#pragma once
#include "moe_common.h"
#include "moe_kernels.h"
#include "../../include/loki_moe.h"

#include <algorithm>
#include <cstdarg>
#include <cstring>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <utility>
#include <vector>

template <class T> struct DBuf {
    T * p = nullptr; size_t cap = 0;
    hipError_t ensure(size_t want) {
        if (want <= cap && p) { return hipSuccess; }
        if (p) { (void) hipFree(p); p = nullptr; cap = 0; }
        const size_t n = want > 0 ? want : 1;
        hipError_t e = hipMalloc(reinterpret_cast<void **>(&p), n * sizeof(T));
        if (e == hipSuccess) { cap = n; } else { p = nullptr; }
        return e;
    }
    void release() { if (p) { (void) hipFree(p); } p = nullptr; cap = 0; }
};

[[noreturn]] inline void fatal(const char * what, hipError_t e, const char * file, int line) {
    std::fprintf(stderr, "[fused] HIP error %s (%s) at %s:%d\n", hipGetErrorString(e), what, file, line);
    std::exit(7);
}
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { fatal(#x, e_, __FILE__, __LINE__); } } while (0)

struct FLCtx {
    hipStream_t st = nullptr, own = nullptr; int dev = 0, ncu = 0;
    hipStream_t side = nullptr; hipEvent_t efork = nullptr, ejoin = nullptr;   // the per-pass decode's shared K-quant expert
    int no_side = 0;                     // fl_set_debug bit 2: that expert on the context's stream instead
    hipEvent_t em0 = nullptr, em1 = nullptr;
    int n_group = 8, topk_group = 4, topk = 8; float scale = 2.5f;
    int keep = 0; float renorm = 0.f;   // fl_moe_layer keeps each row's `keep` heaviest experts (0: all topk)
    int share = 0;                       // ... by the engine's --share-experts rule (fl_set_share_experts)
    int na_used = 0;                     // fl_moe_layer_noalloc ran on this context: fl_sync reads the scratch's error word
    DBuf<int> sel8; DBuf<float> w8;      // every row's topk picks before that keep (per-pass path)
    int n_exp = 256;   // routed experts behind the reference-named entry points (FLW carries no count)
    double ms_moe = 0.0;
    std::string err;
    int dbg_gu = 0;
    DBuf<int8_t> xq, hq; DBuf<float> xd, logits, probs, wts, h, hd, o, g, u, xn;
    DBuf<int> sel, counts, offsets, perm, inv, act, nact;
    int last_n = 0, last_P = 0, last_fused = 0, last_kernel = 0;
    // stage timing (fl_set_profile): one set of NSTAGE+1 events per profiled call, summed by fl_stage_ms
    int prof = 0;
    std::vector<std::vector<hipEvent_t>> ev_free, ev_pending;
    double stage_ms[16] = {0}; long stage_n = 0;
    int zero_dev_init = 0; DBuf<int> zero_i;
    DBuf<float> terms; DBuf<unsigned> cnt;   // per-pass expert kernels: (unused) term scratch, self-resetting counters
    DBuf<uint4> tab;                         // LDS table image (build_table_image)
    // single-launch decode block: epoch-tagged logits / h / o, wait-timeout word; fused = 0 forces the per-pass kernels
    DBuf<int> derr; DBuf<uint64_t> dlogit, dth, dto, dxq; unsigned epoch = 0; int fused = 2; int dec_grid = -1;
    int d1 = 1, d1_ok = -1;   // decode-1 kernel organised by XCD (fl_set_decode1); availability on this device
    // pinned, device-mapped copy of the last code a kernel reported (null if the host allocation failed): every
    // fl_moe_layer call checks it without waiting for the stream, fl_sync reports and clears it
    int * herr = nullptr, * herr_dev = nullptr;   // host pointer, and the address kernels store to
    // prefill grouped GEMM on MFMA (batches above the decode sizes): fp16 table image, columns, fp16 activation copies
    int pf_mfma = 1, pf_ready = 0; DBuf<uint4> ptab; DBuf<int4> pcols; DBuf<int> pncols; DBuf<_Float16> xh, hh;
    struct Compat * compat = nullptr;          // reference-API state (compat.hip), created on first use
    // formats of fl_moe_layer's matrices (fl_set_layer_formats): routed down, shared gate, up, down; K-quant matrices
    // are read in place (ggml layout), IQ2_XXS ones tiled
    int lf[4] = { FL_IQ2, FL_IQ2, FL_IQ2, FL_IQ2 };
    DBuf<float> ksg, ksu;                      // K-quant shared gate / up outputs
    DBuf<unsigned> rcnt;                       // the one-launch routing's self-resetting counter (launch_router_fused)
    DBuf<double> rpart;                        // the K-split router tiles' parts [KS][n][n_exp]
    DBuf<int> dscr;                            // the multi-workgroup dispatch's per-round counts and bases
    size_t h2d_zc = 0, h2d_ce = 0; int h2d_said = 0;   // fl_h2d bytes by kernel (mapped pinned) / by copy engine
    // fl_ffn_begin's event pairs (recorded, not yet folded into ms_ffn by fl_gpu_ms) and the reusable ones
    std::vector<std::pair<hipEvent_t, hipEvent_t>> ffn_ev_pending, ffn_ev_free; double ms_ffn = 0.0;
    // fl_moe's pairs when the call returned on the launch's completion word rather than the stream (folded likewise)
    std::vector<std::pair<hipEvent_t, hipEvent_t>> moe_ev_pending, moe_ev_free;
};
// fl_route_dev with, for the one-launch routing of a few rows (router_fused_ok), a host word set to the context's epoch
// (as it is after the call) once the picks are written; done may be null, other sizes leave it alone
int route_dev(FLCtx * c, const float * W, const float * bias, const float * x, int n, int n_exp, int E, float * logits, float * probs,
              int * sel, float * w, unsigned * done);
// a device int 0 (empty expert lists of the per-pass kernels)
const int * zero_int(FLCtx * c);
static const int NSTAGE = 6;   // quant_x, router_logits, router_select, dispatch, gate_up (+SwiGLU, Q8_K(h)), down (+combine)
// counters of the persistent expert kernels: per (expert slot, row group) and per h block / combine row group
static const size_t CNT_RG = (size_t) (lk::NEXP_MAX + 1) * 112;           // 112 = 7168 / 64 row groups (the largest R)
static const size_t CNT_ALL = 2 * (2 * CNT_RG + 2);                        // gate/up and down sets: cnt_rg, cnt_2, queue[2]

inline int fail(FLCtx * c, int code, const char * fmt, ...) {
    char buf[512]; va_list ap; va_start(ap, fmt); std::vsnprintf(buf, sizeof buf, fmt, ap); va_end(ap);
    if (c) { c->err = buf; }
    return code;
}
#define TRY(c, x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { return fail((c), FL_EHIP, "%s: %s", #x, hipGetErrorString(e_)); } } while (0)
#define ALLOC(c, buf, n) do { if ((buf).ensure(n) != hipSuccess) { (void) hipGetLastError(); return fail((c), FL_ENOMEM, "device allocation of %zu elements failed", (size_t) (n)); } } while (0)

// true unless the HIP allocation holding p is known to end before p + bytes (pointers HIP cannot resolve pass)
inline bool covers(const void * p, size_t bytes) {
    hipDeviceptr_t base = nullptr; size_t size = 0;
    if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t) p) != hipSuccess) { (void) hipGetLastError(); return true; }
    return (const char *) p + bytes <= (const char *) base + size;
}

static std::vector<hipEvent_t> * prof_begin(FLCtx * c) {
    if (!c->prof) { return nullptr; }
    if (c->ev_free.empty()) {
        std::vector<hipEvent_t> ev(NSTAGE + 1);
        for (auto & e : ev) { if (hipEventCreate(&e) != hipSuccess) { return nullptr; } }
        c->ev_free.push_back(ev);
    }
    c->ev_pending.push_back(c->ev_free.back()); c->ev_free.pop_back();
    return &c->ev_pending.back();
}
static void prof_mark(FLCtx * c, std::vector<hipEvent_t> * ev, int i) { if (ev) { (void) hipEventRecord((*ev)[i], c->st); } }

// fold recorded event pairs into a millisecond total: every pair when wait, else only those already complete
typedef std::vector<std::pair<hipEvent_t, hipEvent_t>> EvPairs;
inline void fold_events(EvPairs & pending, EvPairs & freel, double & acc, bool wait) {
    size_t keep = 0;
    for (size_t i = 0; i < pending.size(); ++i) {
        auto ev = pending[i];
        hipError_t q = wait ? hipEventSynchronize(ev.second) : hipEventQuery(ev.second);
        float ms = 0.f;
        if (q == hipSuccess && hipEventElapsedTime(&ms, ev.first, ev.second) == hipSuccess) { acc += ms; freel.push_back(ev); continue; }
        (void) hipGetLastError();
        if (q == hipSuccess) { freel.push_back(ev); continue; }   // an unmeasurable pair is dropped, not kept
        pending[keep++] = ev;
    }
    pending.resize(keep);
}
// a pair to record around a call's enqueued work (reused or created); false if HIP cannot create events
inline bool take_events(EvPairs & freel, std::pair<hipEvent_t, hipEvent_t> & ev) {
    if (!freel.empty()) { ev = freel.back(); freel.pop_back(); return true; }
    ev = { nullptr, nullptr };
    if (hipEventCreate(&ev.first) != hipSuccess || hipEventCreate(&ev.second) != hipSuccess) { (void) hipGetLastError(); return false; }
    return true;
}
// fl_ffn_begin's pairs into ms_ffn, fl_moe's (those not waited for at once) into ms_moe
inline void fold_ffn_events(FLCtx * c, bool wait) {
    fold_events(c->ffn_ev_pending, c->ffn_ev_free, c->ms_ffn, wait);
    fold_events(c->moe_ev_pending, c->moe_ev_free, c->ms_moe, wait);
}

void compat_free(FLCtx * c);   // compat.hip
// device ranges declared to hold IQ2_XXS matrices in the tiled layout (compat.hip; process-wide): fl_register_tiled,
// and the tiled layers of fl_gguf_load_moe_layer
void tiled_add(const void * p, size_t bytes);
void tiled_remove_within(const void * p, size_t bytes);
bool tiled_holds(const void * p, size_t bytes);
int ensure_expert_scratch(FLCtx * c, size_t rows, int E, int H);   // fused_layer.hip
int prefill_ready(FLCtx * c);   // fused_layer.hip: the grouped GEMMs' set-up (tables, attributes), once per context
// the one-token kernel is available (a 256-CU device, the fused decode not switched off); the n <= 8 single-launch
// block is; and their launch on caller-given picks (d.ext_sel / ext_w set; this fills the tables, tagged buffers,
// epoch and error words of d): the one-token kernel for one row with all 8 picks when it is available, else the block
bool decode1_available(FLCtx * c);
bool decode_block_available(FLCtx * c);
int decode_picks(FLCtx * c, lk::DecodeArgs & d);
lk::ExpertArgs expert_args(FLCtx * c, int n, int P, int shared);
// counter sets of the two persistent kernels inside FLCtx::cnt
inline void expert_counters(FLCtx * c, lk::ExpertArgs & a, int down) {
    unsigned * base = c->cnt.p + (down ? 2 * CNT_RG + 2 : 0);
    a.cnt_rg = base; a.cnt_2 = base + CNT_RG; a.queue = base + 2 * CNT_RG;
}

