// compat.hip -- the reference's host-driven MoE entry points (src/fused_layer.h:29-52) on top of the device kernels.
//
// The reference's engine drives one layer as: fl_attn (attention + router + shared expert) -> fl_fetch (routing to the
// host) -> host dispatch -> fl_moe (narrow, n <= 8) or fl_wide_moe per arena batch + fl_wide_finish (prefill).
// Attention stays outside this library, so fl_ffn_begin takes the MoE tail of fl_attn (router input ncur and the
// residual ffn_inp; src/fused_layer.cu:498-525) from the host. Everything else keeps the reference's names, parameters,
// ownership (context-owned pinned mirrors, overwritten by the next call) and synchronisation (fl_fetch, fl_moe, fl_skip,
// fl_wide_finish and fl_wide_skip wait; fl_ffn_begin and fl_wide_moe only enqueue). Expert arenas arrive in ggml's
// layout and are repacked into the tiled layout on the device before the mat-vecs -- on every call, since the reference's
// engine refills its arenas in place (src/server_core_fused.cpp:295-305) -- unless they lie in a range declared tiled
// (fl_register_tiled, or a layer loaded with FL_LAYOUT_TILED), which is read as it is.
// Summation orders follow each reference kernel: moe_combine (src/fused_layer.cu:366-372) adds slots in ascending slot
// order with the weights of equal slots merged; base_rows/wide_finish (:351-360) add fi + shared, then the k outputs.
#include "fl_ctx.h"

#include <chrono>
#include <mutex>

using namespace lk;

// ---------------------------------------------------------------- declared tiled ranges
// The registry is created on first use and never destroyed: the library registers no exit-time destructor of its own,
// so process exit runs nothing of it but the HIP runtime's module unregistration (a destructor here would run from
// __cxa_finalize, interleaved with whatever teardown the runtime or a profiler's preloaded tool does at exit).
namespace {
std::mutex g_tiled_mu;   // trivially destructible
std::vector<std::pair<uintptr_t, uintptr_t>> & g_tiled() {   // [begin, end)
    static auto * v = new std::vector<std::pair<uintptr_t, uintptr_t>>();
    return *v;
}
}
void tiled_add(const void * p, size_t bytes) {
    std::lock_guard<std::mutex> lk(g_tiled_mu);
    g_tiled().emplace_back((uintptr_t) p, (uintptr_t) p + bytes);
}
void tiled_remove_within(const void * p, size_t bytes) {
    const uintptr_t b = (uintptr_t) p, e = b + bytes;
    std::lock_guard<std::mutex> lk(g_tiled_mu);
    std::vector<std::pair<uintptr_t, uintptr_t>> keep;
    for (const auto & r : g_tiled()) { if (r.first < b || r.second > e) { keep.push_back(r); } }
    g_tiled().swap(keep);
}
bool tiled_holds(const void * p, size_t bytes) {
    const uintptr_t b = (uintptr_t) p, e = b + bytes;
    std::lock_guard<std::mutex> lk(g_tiled_mu);
    for (const auto & r : g_tiled()) { if (r.first <= b && e <= r.second) { return true; } }
    return false;
}
extern "C" int fl_register_tiled(FLCtx * c, const void * base, size_t bytes) {
    if (!c) { return FL_EINVAL; }
    if (!base || bytes == 0) { return fail(c, FL_EINVAL, "fl_register_tiled: empty range"); }
    if (!covers(base, bytes)) { return fail(c, FL_EINVAL, "fl_register_tiled: the range runs past its allocation"); }
    tiled_add(base, bytes);
    return FL_OK;
}
extern "C" int fl_unregister_tiled(FLCtx * c, const void * base, size_t bytes) {
    if (!c) { return FL_EINVAL; }
    tiled_remove_within(base, bytes);
    return FL_OK;
}

namespace {

constexpr int RMAX = 64;           // rows per fl_ffn_begin call (the reference's RMAX, src/fused_layer.cu:402)
constexpr int NB = 8;              // rows of a narrow pass (src/fused_layer.cu:18)
constexpr int E_ = 7168, H_ = 2048, NEXP_ = 256;
constexpr int ZS_DONE = 2 * RMAX * MAXK + 16;   // the routing's done word in z_sel (its own cache line)
constexpr int ZS_FDONE = ZS_DONE + 1;           // fl_moe's one-token launch's completion word
constexpr int ZS_TSTAMP = ZS_DONE + 4;          // its start and end clocks (two 64-bit words, 16-byte aligned)
static_assert(ZS_TSTAMP % 4 == 0 && ZS_TSTAMP + 4 <= ZS_DONE + 16, "z_sel layout");

template <class T> T * pinned(size_t n) {
    void * p = nullptr;
    if (hipHostMalloc(&p, n * sizeof(T) > 0 ? n * sizeof(T) : 1, hipHostMallocDefault) != hipSuccess) { (void) hipGetLastError(); return nullptr; }
    std::memset(p, 0, n * sizeof(T));
    return static_cast<T *>(p);
}
// pinned host memory that kernels read and write in place (coherent: not cached on the device, a kernel's stores are
// seen by the host once the stream has been waited); *dev = the address kernels use
// spins until every word of w[0 .. n) reads tag (stores of a kernel to host memory), at most max_us; false: not seen
static bool spin_words(const unsigned * w, int n, unsigned tag, double max_us) {
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < n; ++i) {
        for (unsigned it = 0; __atomic_load_n(w + i, __ATOMIC_ACQUIRE) != tag; ++it) {
            if ((it & 255u) == 255u && std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count() > max_us) {
                return false;
            }
        }
    }
    return true;
}
template <class T> T * mapped(size_t n, T ** dev) {
    void * p = nullptr;
    if (hipHostMalloc(&p, n * sizeof(T), hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess) { (void) hipGetLastError(); return nullptr; }
    std::memset(p, 0, n * sizeof(T));
    if (hipHostGetDevicePointer(reinterpret_cast<void **>(dev), p, 0) != hipSuccess) { (void) hipGetLastError(); (void) hipHostFree(p); return nullptr; }
    return static_cast<T *>(p);
}

// ---------------------------------------------------------------- small kernels with the reference's orders
// block (x, b): elements 256 x .. of row b. The row's distinct slot ids in ascending order, each with its weights
// summed in k order and its first k, are formed once in LDS; every element then adds them in that order.
__global__ void __launch_bounds__(256) k_combine_slots(const float * __restrict__ o, const int * __restrict__ inv, const int * __restrict__ ids,
                                                      const float * __restrict__ w, int n, int KE, const float * __restrict__ sh, const float * __restrict__ fi,
                                                      float * __restrict__ h, float * __restrict__ moe) {
#pragma clang fp contract(off)
    __shared__ float s_wt[MAXK]; __shared__ int s_row[MAXK]; __shared__ int s_cnt;
    const int b = blockIdx.y;
    if (threadIdx.x == 0) {
        const int * idr = ids + b * KE; const float * wr = w + b * KE;
        int prev = -1, cnt = 0;
        for (;;) {   // distinct slot ids of the row, ascending
            int m = 0x7fffffff;
            for (int k = 0; k < KE; ++k) { if (idr[k] > prev && idr[k] < m) { m = idr[k]; } }
            if (m == 0x7fffffff) { break; }
            float wt = 0.f; int kf = -1;
            for (int k = 0; k < KE; ++k) { if (idr[k] == m) { wt += wr[k]; if (kf < 0) { kf = k; } } }
            prev = m;
            if (wt == 0.f) { continue; }
            s_wt[cnt] = wt; s_row[cnt] = inv[b * KE + kf]; ++cnt;
        }
        s_cnt = cnt;
    }
    __syncthreads();
    const int e = blockIdx.x * 256 + threadIdx.x;
    if (e >= E_) { return; }
    float v = 0.f;
    for (int q = 0; q < s_cnt; ++q) { v += s_wt[q] * o[(size_t) s_row[q] * E_ + e]; }
    const size_t i = (size_t) b * E_ + e;
    if (moe) { moe[i] = v; }
    h[i] = (v + sh[i]) + fi[i];
}

__global__ void k_skip_rows(const float * __restrict__ mo, const float * __restrict__ sh, const float * __restrict__ fi, int64_t tot, float * __restrict__ h) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= tot) { return; }
    const float v = 0.f + mo[i];
    h[i] = (v + sh[i]) + fi[i];
}

__global__ void k_base_rows(const float * __restrict__ fi, const float * __restrict__ sh, int64_t tot, float * __restrict__ base) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i < tot) { base[i] = fi[i] + sh[i]; }
}

// block (x, p): pair p's columns 1024 x .. + 1023, four per thread (rows of E_ floats in hipMalloc'd buffers: 16-byte
// aligned); the pair's row, slot and weight are uniform per block
__global__ void __launch_bounds__(256) k_wide_scatter(const float * __restrict__ o, const int * __restrict__ prow, const int * __restrict__ pk,
                                                      const float * __restrict__ pw, int npairs, int KE, float * __restrict__ out_all) {
    static_assert(E_ % 4 == 0, "4-wide rows");
    const int e = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (e >= E_) { return; }
    for (int p = blockIdx.y; p < npairs; p += gridDim.y) {   // the grid's y extent is capped at 65535
        const float w = pw[p];
        const float4 v = *reinterpret_cast<const float4 *>(o + (size_t) p * E_ + e);
        *reinterpret_cast<float4 *>(out_all + ((size_t) prow[p] * KE + pk[p]) * E_ + e) = make_float4(w * v.x, w * v.y, w * v.z, w * v.w);
    }
}

__global__ void k_wide_finish(const float * __restrict__ base, const float * __restrict__ out_all, int KE, int64_t tot,
                              float * __restrict__ h, float * __restrict__ moe) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= tot) { return; }
    const int64_t r = i / E_, e = i % E_;
    float m = 0.f;
    for (int k = 0; k < KE; ++k) { m += out_all[((size_t) r * KE + k) * E_ + e]; }
    moe[i] = m; h[i] = base[i] + m;
}

__global__ void k_wide_skip(const float * __restrict__ base, const float * __restrict__ mo, int64_t tot, float * __restrict__ h) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i < tot) { h[i] = base[i] + mo[i]; }
}

inline unsigned nblk(int64_t tot) { return (unsigned) ((tot + 255) / 256); }

// fl_h2d's copy by kernel: 16-byte words, four loads in flight per thread (each a PCIe read of the mapped host
// memory), grid-stride; and the byte copy for unaligned ranges
__global__ void __launch_bounds__(256) k_copy16(const uint4 * __restrict__ src, uint4 * __restrict__ dst, size_t n) {
    const size_t stride = (size_t) gridDim.x * 256;
    size_t i = (size_t) blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * stride < n; i += 4 * stride) {
        const uint4 a = src[i], b = src[i + stride], c2 = src[i + 2 * stride], d = src[i + 3 * stride];
        dst[i] = a; dst[i + stride] = b; dst[i + 2 * stride] = c2; dst[i + 3 * stride] = d;
    }
    for (; i < n; i += stride) { dst[i] = src[i]; }
}
__global__ void __launch_bounds__(256) k_copy1(const uint8_t * __restrict__ src, uint8_t * __restrict__ dst, size_t n) {
    for (size_t i = (size_t) blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t) gridDim.x * 256) { dst[i] = src[i]; }
}

}  // namespace

struct Compat {
    // rows of the last fl_ffn_begin (narrow pass); sh_pending / xq_pending: its shared expert / the Q8_K of its rows not
    // computed yet (fl_moe's one-token launch computes both itself; the per-pass fl_moe and fl_skip compute them first)
    int N = 0; bool sh_pending = false, xq_pending = false;
    // ncur: the N rows of ncur then the N rows of ffn_inp (one copy in); fi points at the second part
    DBuf<float> ncur, logits, probs, wts, h, o, sh_o, wr32; float * fi = nullptr; DBuf<int8_t> xq, hq; DBuf<float> xd, hd;
    DBuf<uint8_t> sh_t; const void * sh_key[3] = { nullptr, nullptr, nullptr }; int sh_fkey[3] = { -1, -1, -1 };
    bool sh_tkey[3] = { false, false, false };   // whether each was a declared-tiled matrix when sh_t was filled
    int shf[3] = { FL_IQ2, FL_IQ2, FL_IQ2 };   // shared gate / up / down formats (fl_set_shared_formats)
    DBuf<float> sg, su;                         // K-quant shared gate / up outputs
    // fl_moe
    DBuf<uint8_t> ag, au, ad; DBuf<int> ids, counts, offsets, perm, inv, act, nact; DBuf<float> w, hout, moe;
    // the grouped GEMMs of routed_experts: the rows' Q8_K as fp16, Q8_K(h) as fp16, the columns
    DBuf<_Float16> xh, hh; DBuf<int4> pcols; DBuf<int> pncols;
    std::vector<int> last_ids; int last_KE = 0, last_n = 0; bool last_fast = false;   // last_fast: o holds slot k at row k
    // wide pass
    int wmax = 0, wke = 0;
    // wide pass: ffn_inp and the Q8_K of every row (fl_ffn_begin(wrow)); the shared expert of all rows (sh_all) and
    // base = ffn_inp + shared, formed once by the first fl_wide_finish / fl_wide_skip after the rows came in
    // (wide_pending), so the shared expert runs on all the rows in one pass
    DBuf<float> fi_all, sh_all, base_all, out_all, xd_all; DBuf<int8_t> xq_all; bool wide_pending = false;
    DBuf<int> w_act, w_off, w_perm, w_nact, w_row, w_k; DBuf<float> w_wk;
    hipEvent_t wev[2] = { nullptr, nullptr };
    // fl_wide_moe's slot tables for each parity in pinned host memory (act | off | perm | row | k | nact, then wk): the
    // call only enqueues, so a parity's tables stay untouched until fl_wide_wait(par) (the engine's own discipline)
    int * wt_i[2] = { nullptr, nullptr }; float * wt_w[2] = { nullptr, nullptr }; size_t wt_cap[2] = { 0, 0 };
    hipEvent_t wt_ev[2] = { nullptr, nullptr }; bool wt_rec[2] = { false, false };   // after each parity's table copies
    // pinned host mirrors
    int * h_sel = nullptr; float * h_wts = nullptr, * h_h = nullptr, * h_moe = nullptr;
    // kernel-written host memory (no copies): the router's picks of the RMAX rows then their weights (z_sel), then
    // the one-launch routing's done word (at ZS_DONE); fl_moe's single launch's ids then (at NB * MAXK) weights (z_in)
    // and its h rows then (at NB * E) moe rows (z_out); *_d = the device addresses. r_tagged: the last fl_ffn_begin's routing sets the done word, to rtag
    int * z_sel = nullptr, * z_sel_d = nullptr, * z_in = nullptr, * z_in_d = nullptr; float * z_out = nullptr, * z_out_d = nullptr;
    unsigned rtag = 0; bool r_tagged = false;
    // fl_moe's one-token launch signals its end in z_sel[ZS_FDONE] (fcnt: its workgroup counter, zero between launches)
    DBuf<unsigned> fcnt; bool fcnt_zero = false;
    // The speculative one-token launch. After an fl_moe on one row whose ids and weights were the routing's own picks
    // and whose arena is declared resident and tiled (fl_register_tiled), spec_ok holds that arena; the next
    // fl_ffn_begin on one row then routes and runs the whole block in one launch on its picks (fl_moe's combine, h and
    // moe into z_out), and fl_moe, if called on exactly those picks, weights and arena, only waits for it (spec_live)
    bool spec_ok = false, spec_live = false; const void * spec_g = nullptr, * spec_u = nullptr, * spec_d = nullptr;
    int spec_nexp = 0; unsigned spec_epoch = 0;
    // the wide pass's h / moe rows in mapped host memory, written there by k_wide_finish / k_wide_skip (no copy back)
    float * h_wh = nullptr, * h_wmoe = nullptr, * h_wh_d = nullptr, * h_wmoe_d = nullptr;
    // pinned staging of the host inputs (pageable copies would wait for the stream). fl_ffn_begin's ncur / ffn_inp go
    // to in_st[p] (ncur's rows, then ffn_inp's), p alternating per call; in_ncur / in_fi point at the last call's, and
    // fl_fetch hands them out as its ncur / fi mirrors, which therefore hold until the second fl_ffn_begin after it
    // (the reference's mirrors are replaced by the next call). st_ev[p] is recorded after in_st[p]'s copy and waited
    // before it is refilled. fl_moe's ids / w go to in_ids, in_ev likewise.
    float * in_st[2] = { nullptr, nullptr }, * in_ncur = nullptr, * in_fi = nullptr, * in_w = nullptr; int * in_ids = nullptr;
    hipEvent_t st_ev[2] = { nullptr, nullptr }; bool st_rec[2] = { false, false }; int st_par = 0, st_spec = 0;
    float * in_st_d[2] = { nullptr, nullptr };   // the stagings' device addresses (the one-row copy kernel reads them)
    hipEvent_t in_ev = nullptr; bool in_rec = false;
};

static Compat * cs(FLCtx * c) {
    if (!c->compat) {
        Compat * s = new Compat();
        s->z_sel = mapped<int>(ZS_DONE + 16, &s->z_sel_d); s->z_in = mapped<int>(2 * NB * MAXK, &s->z_in_d);
        s->z_out = mapped<float>((size_t) 2 * NB * E_, &s->z_out_d);
        s->h_sel = pinned<int>(RMAX * MAXK); s->h_wts = pinned<float>(RMAX * MAXK);
        s->h_h = pinned<float>((size_t) RMAX * E_); s->h_moe = pinned<float>((size_t) RMAX * E_);
        s->in_st[0] = mapped<float>((size_t) 2 * RMAX * E_, &s->in_st_d[0]); s->in_st[1] = mapped<float>((size_t) 2 * RMAX * E_, &s->in_st_d[1]);
        s->in_ids = pinned<int>(2 * NB * MAXK); s->in_w = pinned<float>(NB * MAXK);   // in_ids: ids, then the weights
        if (!s->z_sel || !s->z_in || !s->z_out || !s->h_sel || !s->h_wts || !s->h_h || !s->h_moe || !s->in_st[0] || !s->in_st[1] || !s->in_ids || !s->in_w) {
            fatal("hipHostMalloc (fused-layer mirrors)", hipErrorOutOfMemory, __FILE__, __LINE__);
        }
        CK(hipEventCreateWithFlags(&s->in_ev, hipEventDisableTiming));
        for (hipEvent_t & e : s->st_ev) { CK(hipEventCreateWithFlags(&e, hipEventDisableTiming)); }
        c->compat = s;
    }
    return c->compat;
}

void compat_free(FLCtx * c) {
    Compat * s = c->compat;
    if (!s) { return; }
    if (s->in_ev) { (void) hipEventSynchronize(s->in_ev); (void) hipEventDestroy(s->in_ev); }
    for (hipEvent_t e : s->st_ev) { if (e) { (void) hipEventSynchronize(e); (void) hipEventDestroy(e); } }
    for (void * p : { (void *) s->z_sel, (void *) s->z_in, (void *) s->z_out, (void *) s->h_sel, (void *) s->h_wts, (void *) s->h_h, (void *) s->h_moe, (void *) s->h_wh, (void *) s->h_wmoe,
                      (void *) s->in_st[0], (void *) s->in_st[1], (void *) s->in_ids, (void *) s->in_w }) {
        if (p) { (void) hipHostFree(p); }
    }
    for (hipEvent_t e : s->wev) { if (e) { (void) hipEventDestroy(e); } }
    for (int p = 0; p < 2; ++p) {
        if (s->wt_i[p]) { (void) hipHostFree(s->wt_i[p]); } if (s->wt_w[p]) { (void) hipHostFree(s->wt_w[p]); }
        if (s->wt_ev[p]) { (void) hipEventDestroy(s->wt_ev[p]); }
    }
    s->ncur.release(); s->logits.release(); s->probs.release(); s->wts.release(); s->h.release(); s->o.release(); s->sh_o.release(); s->wr32.release();
    s->xq.release(); s->hq.release(); s->xd.release(); s->hd.release(); s->sh_t.release(); s->sg.release(); s->su.release();
    s->ag.release(); s->au.release(); s->ad.release(); s->ids.release(); s->counts.release(); s->offsets.release(); s->perm.release(); s->inv.release();
    s->act.release(); s->nact.release(); s->w.release(); s->hout.release(); s->moe.release();
    s->xh.release(); s->hh.release(); s->pcols.release(); s->pncols.release();
    s->fcnt.release();
    s->fi_all.release(); s->sh_all.release(); s->base_all.release(); s->out_all.release(); s->xd_all.release(); s->xq_all.release();
    s->w_act.release(); s->w_off.release(); s->w_perm.release(); s->w_nact.release(); s->w_row.release(); s->w_k.release(); s->w_wk.release();
    delete s; c->compat = nullptr;
}

const int * zero_int(FLCtx * c) {
    if (!c->zero_dev_init) {
        CK(c->zero_i.ensure(1) == hipSuccess ? hipSuccess : hipErrorOutOfMemory);
        const int z = 0; CK(hipMemcpy(c->zero_i.p, &z, sizeof z, hipMemcpyHostToDevice));
        c->zero_dev_init = 1;
    }
    return c->zero_i.p;
}

#define FCK(x) CK(x)
#define FALLOC(buf, n) CK((buf).ensure(n))

static size_t mat_bytes(int R, int K) { return (size_t) R * (K / QK) * IQ2B; }
// bytes of one R x K matrix in format fmt (IQ2_XXS or a K-quant)
static size_t fmt_bytes(int fmt, int R, int K) { return (size_t) R * (K / QK) * (size_t) (fmt == FL_IQ2 ? IQ2B : kq_block_bytes(fmt)); }

// K-quant mat-vec of one matrix (ggml layout) on n Q8_K rows -> out [n][R]
static void kq_single(FLCtx * c, int fmt, const void * w, const int8_t * q, const float * d, int n, int K, int R, float * out) {
    KqArgs k{};
    k.w = (const uint8_t *) w; k.estride = fmt_bytes(fmt, R, K); k.aq = q; k.ad = d; k.K = K; k.R = R;
    k.act = nullptr; k.nact = nullptr; k.offsets = nullptr; k.n = n; k.out = out; k.ldo = R;
    FCK(launch_kq_matvec(k, fmt, n, 1, c->st));
}

// shared expert of N rows whose Q8_K activations are xq/xd -> out [N][E]: IQ2_XXS matrices from the tiled copy sh_t,
// K-quant matrices (the reference's Q5_K / Q5_K / Q6_K) read in place
static void shared_expert(FLCtx * c, Compat * s, const int8_t * xq, const float * xd, int N, float * out) {
    const size_t mg = mat_bytes(H_, E_);
    // IQ2_XXS shared matrices: a declared-tiled one as it is, else its tiled copy in sh_t
    const uint8_t * tm[3];
    for (int i = 0; i < 3; ++i) {
        const size_t b = i < 2 ? mg : mat_bytes(E_, H_);
        tm[i] = tiled_holds(s->sh_key[i], b) ? (const uint8_t *) s->sh_key[i] : s->sh_t.p + i * mg;
    }
    FALLOC(s->h, (size_t) N * H_); FALLOC(s->hq, (size_t) N * H_); FALLOC(s->hd, (size_t) N * (H_ / QK));
    CK(ensure_expert_scratch(c, (size_t) N, E_, H_) == FL_OK ? hipSuccess : hipErrorOutOfMemory);
    // Above 8 rows the matrices whose format has one run on the grouped GEMMs, as the shared expert's columns (slots
    // 0 .. N - 1 = the rows): IQ2_XXS on the IQ2_XXS GEMM, a Q5_K gate / up and a Q2_K / Q3_K / Q6_K down on the
    // K-quant GEMM. Same bits as the per-pass kernels below.
    const bool kq_gu = s->shf[0] == FL_Q5K && s->shf[1] == FL_Q5K;
    const bool kq_dn = s->shf[2] == FL_Q2K || s->shf[2] == FL_Q3K || s->shf[2] == FL_Q6K;
    const bool gemm = N > 8 && c->pf_mfma;
    const bool gu_gemm = gemm && (s->shf[0] == FL_IQ2 || kq_gu), dn_gemm = gemm && (s->shf[2] == FL_IQ2 || kq_dn);
    PrefillArgs g{};
    if (gu_gemm || dn_gemm) {
        CK(prefill_ready(c) == FL_OK ? hipSuccess : hipErrorOutOfMemory);
        // ceil(N / 64) shared columns (wide_base runs every row of a wide pass here, so N is not bounded by 64)
        FALLOC(s->pcols, (size_t) prefill_shared_cols(N) + NEXP_MAX + 2); FALLOC(s->pncols, PF_NCOLS);
        FCK(launch_prefill_cols(zero_int(c), zero_int(c), zero_int(c), N, 0, s->pcols.p, s->pncols.p, c->st));   // no routed columns
        g.ptab = c->ptab.p; g.perm = zero_int(c); g.topk = 1; g.P = 0; g.cols = s->pcols.p; g.ncols = s->pncols.p;
        g.err = c->derr.p; g.herr = c->herr ? c->herr_dev : nullptr;
    }
    ExpertArgs a = expert_args(c, N, 0, 1);
    if (gu_gemm) {
        FALLOC(s->xh, (size_t) N * E_);
        FCK(launch_q8_to_h(xq, s->xh.p, (int64_t) N * E_, c->st));
        PrefillArgs k = g;
        k.R = H_; k.K = E_; k.bh = s->xh.p; k.bd = xd;
        if (s->shf[0] == FL_IQ2) {
            k.w[0] = tm[0]; k.w[1] = tm[1]; k.sh[0] = tm[0]; k.sh[1] = tm[1]; k.nmat = 2; k.out = s->h.p;
            FCK(launch_prefill_gemm(k, c->ncu, c->st));
        } else {
            FALLOC(s->sg, (size_t) N * H_); FALLOC(s->su, (size_t) N * H_);
            for (int m = 0; m < 2; ++m) {
                k.sh[0] = k.w[0] = (const uint8_t *) s->sh_key[m]; k.nmat = 1; k.out = m ? s->su.p : s->sg.p;
                FCK(launch_kq_gemm(k, FL_Q5K, c->ncu, c->st));
            }
            FCK(launch_swiglu(s->sg.p, s->su.p, (int64_t) N * H_, s->h.p, c->st));
        }
        FCK(launch_quant_q8k(s->h.p, N, H_, s->hq.p, s->hd.p, c->st));
    } else if (s->shf[0] == FL_IQ2) {
        a.sh[0] = tm[0]; a.sh[1] = tm[1]; a.aq = xq; a.ad = xd; a.K = E_; a.R = H_; a.nmat = 2;
        a.act = zero_int(c); a.nact = zero_int(c); a.offsets = zero_int(c); a.perm = zero_int(c); a.topk = 1;
        a.h = s->h.p; a.hq = s->hq.p; a.hd = s->hd.p;
        expert_counters(c, a, 0);
        FCK(launch_experts_gateup(a, c->ncu, c->st));
    } else {   // g, u, then h = silu(g) * u and its Q8_K (src/fused_layer.cu:522-523)
        FALLOC(s->sg, (size_t) N * H_); FALLOC(s->su, (size_t) N * H_);
        if (s->shf[0] == s->shf[1]) {   // gate and up in one launch
            KqArgs k{};
            k.w = (const uint8_t *) s->sh_key[0]; k.w2 = (const uint8_t *) s->sh_key[1]; k.estride = fmt_bytes(s->shf[0], H_, E_);
            k.aq = xq; k.ad = xd; k.K = E_; k.R = H_; k.n = N; k.out = s->sg.p; k.out2 = s->su.p; k.ldo = H_;
            FCK(launch_kq_matvec(k, s->shf[0], N, 1, c->st));
        } else {
            kq_single(c, s->shf[0], s->sh_key[0], xq, xd, N, E_, H_, s->sg.p);
            kq_single(c, s->shf[1], s->sh_key[1], xq, xd, N, E_, H_, s->su.p);
        }
        FCK(launch_swiglu_q8k(s->sg.p, s->su.p, N, H_, s->h.p, s->hq.p, s->hd.p, c->st));
    }
    if (dn_gemm) {
        FALLOC(s->hh, (size_t) N * H_);
        FCK(launch_q8_to_h(s->hq.p, s->hh.p, (int64_t) N * H_, c->st));
        PrefillArgs k = g;
        k.R = E_; k.K = H_; k.nmat = 1; k.bh = s->hh.p; k.bd = s->hd.p; k.out = out;
        if (s->shf[2] == FL_IQ2) {
            k.w[0] = k.sh[0] = tm[2];
            FCK(launch_prefill_gemm(k, c->ncu, c->st));
        } else {
            k.w[0] = k.sh[0] = (const uint8_t *) s->sh_key[2];
            FCK(launch_kq_gemm(k, s->shf[2], c->ncu, c->st));
        }
    } else if (s->shf[2] == FL_IQ2) {
        ExpertArgs d = a;
        d.sh[0] = tm[2]; d.sh[1] = nullptr; d.aq = s->hq.p; d.ad = s->hd.p; d.K = H_; d.R = E_; d.nmat = 1;
        d.act = zero_int(c); d.nact = zero_int(c); d.offsets = zero_int(c); d.perm = zero_int(c); d.topk = 1;
        d.h = nullptr; d.hq = nullptr; d.hd = nullptr; d.o = out; d.y = nullptr;
        expert_counters(c, d, 1);
        FCK(launch_experts_down(d, c->ncu, c->st));
    } else {
        kq_single(c, s->shf[2], s->sh_key[2], s->hq.p, s->hd.p, N, H_, E_, out);   // src/fused_layer.cu:524
    }
}

// the shared expert of the last fl_ffn_begin into sh_o, if not computed yet
static void quant_now(FLCtx * c, Compat * s) {
    if (!s->xq_pending) { return; }
    CK(launch_quant_q8k(s->ncur.p, s->N, E_, s->xq.p, s->xd.p, c->st));
    s->xq_pending = false;
}
static void shared_now(FLCtx * c, Compat * s) {
    if (!s->sh_pending) { return; }
    quant_now(c, s);
    shared_expert(c, s, s->xq.p, s->xd.p, s->N, s->sh_o.p);
    s->sh_pending = false;
}

// an arena's matrices in the tiled layout: declared-tiled matrices as they are, the others repacked into ag/au/ad
struct Arena { const uint8_t * g, * u, * d; };

// routed experts of an arena (tiled gate/up/down in ar) for the pairs described by offsets/perm/act/nact -> o [P][E]
// down_fmt: FL_IQ2 (tiled ar.d) or FL_Q2K / FL_Q3K read in place from down (expert stride E x H/256 blocks);
// max_slots bounds the pairs of one expert
// With two or more pairs per arena expert on average (a wide batch), the pairs run on the grouped MFMA GEMMs (gate/up,
// then Q8_K(h), then the down on the IQ2_XXS or the K-quant GEMM), else on the per-pass kernels; both give the same
// bits. fl_set_prefill_mfma(0) keeps the per-pass kernels.
static void routed_experts(FLCtx * c, Compat * s, const Arena & ar, const int8_t * xq, const float * xd, int n, int P, int KE, int nexp,
                           const int * act, const int * nact, const int * offsets, const int * perm, float * o,
                           int down_fmt, const void * down, int max_slots) {
    FALLOC(s->h, (size_t) P * H_); FALLOC(s->hq, (size_t) P * H_); FALLOC(s->hd, (size_t) P * (H_ / QK));
    if (c->pf_mfma && P >= 32 && P >= 2 * nexp) {
        CK(prefill_ready(c) == FL_OK ? hipSuccess : hipErrorOutOfMemory);
        hipStream_t st = c->st;
        FALLOC(s->xh, (size_t) n * E_); FALLOC(s->hh, (size_t) P * H_);
        FALLOC(s->pcols, (size_t) P / 32 + NEXP_MAX + 2); FALLOC(s->pncols, PF_NCOLS);
        FCK(launch_q8_to_h(xq, s->xh.p, (int64_t) n * E_, st));
        FCK(launch_prefill_cols(act, nact, offsets, 0, P, s->pcols.p, s->pncols.p, st));
        PrefillArgs g{};
        g.ptab = c->ptab.p; g.w[0] = ar.g; g.w[1] = ar.u; g.estride = mat_bytes(H_, E_); g.sh[0] = ar.g; g.sh[1] = ar.u;   // no shared columns
        g.perm = perm; g.topk = KE; g.P = P; g.R = H_; g.K = E_; g.nmat = 2; g.cols = s->pcols.p; g.ncols = s->pncols.p;
        g.bh = s->xh.p; g.bd = xd; g.out = s->h.p; g.err = c->derr.p; g.herr = c->herr ? c->herr_dev : nullptr;
        FCK(launch_prefill_gemm(g, c->ncu, st));
        FCK(launch_quant_q8k(s->h.p, P, H_, s->hq.p, s->hd.p, st));
        FCK(launch_q8_to_h(s->hq.p, s->hh.p, (int64_t) P * H_, st));
        PrefillArgs d = g;
        d.R = E_; d.K = H_; d.nmat = 1; d.bh = s->hh.p; d.bd = s->hd.p; d.out = o; d.w[1] = nullptr; d.sh[1] = nullptr;
        if (down_fmt == FL_IQ2) {
            d.w[0] = ar.d; d.sh[0] = ar.d; d.estride = mat_bytes(E_, H_);
            FCK(launch_prefill_gemm(d, c->ncu, st));
        } else {   // src/fused_layer.cu:607-608 (tc_matvec<F_Q2K / F_Q3K>)
            d.w[0] = (const uint8_t *) down; d.sh[0] = (const uint8_t *) down; d.estride = fmt_bytes(down_fmt, E_, H_);
            FCK(launch_kq_gemm(d, down_fmt, c->ncu, st));
        }
        return;
    }
    CK(ensure_expert_scratch(c, (size_t) P + n, E_, H_) == FL_OK ? hipSuccess : hipErrorOutOfMemory);
    ExpertArgs a = expert_args(c, n, P, 0);
    a.w[0] = ar.g; a.w[1] = ar.u; a.estride = mat_bytes(H_, E_); a.aq = xq; a.ad = xd; a.K = E_; a.R = H_; a.nmat = 2;
    a.act = act; a.nact = nact; a.offsets = offsets; a.perm = perm; a.topk = KE;
    a.h = s->h.p; a.hq = s->hq.p; a.hd = s->hd.p;
    expert_counters(c, a, 0);
    FCK(launch_experts_gateup(a, c->ncu, c->st));
    if (down_fmt != FL_IQ2) {   // src/fused_layer.cu:607-608 (tc_matvec<F_Q2K / F_Q3K>)
        KqArgs k{};
        k.w = (const uint8_t *) down; k.estride = fmt_bytes(down_fmt, E_, H_); k.aq = s->hq.p; k.ad = s->hd.p; k.K = H_; k.R = E_;
        k.act = act; k.nact = nact; k.offsets = offsets; k.n = 0; k.out = o; k.ldo = E_;
        FCK(launch_kq_matvec(k, down_fmt, max_slots, std::min(nexp, P), c->st));
        return;
    }
    ExpertArgs d = a;
    d.w[0] = ar.d; d.w[1] = nullptr; d.estride = mat_bytes(E_, H_); d.aq = s->hq.p; d.ad = s->hd.p; d.K = H_; d.R = E_; d.nmat = 1;
    d.h = nullptr; d.hq = nullptr; d.hd = nullptr; d.o = o; d.y = nullptr;
    expert_counters(c, d, 1);
    FCK(launch_experts_down(d, c->ncu, c->st));
}

// IQ2_XXS arena matrices in the tiled layout: declared-tiled ones as they are, the others repacked into the context's
// copies (a K-quant down stays where it is)
static Arena pack_arena(FLCtx * c, Compat * s, const void * gate, const void * up, const void * down, int nexp, int down_fmt) {
    const size_t mg = mat_bytes(H_, E_), md = mat_bytes(E_, H_);
    Arena ar{ (const uint8_t *) gate, (const uint8_t *) up, (const uint8_t *) down };
    if (!tiled_holds(gate, (size_t) nexp * mg)) {
        FALLOC(s->ag, (size_t) nexp * mg);
        FCK(launch_pack_tiled((const uint8_t *) gate, mg, s->ag.p, mg, H_, E_, nexp, c->st));
        ar.g = s->ag.p;
    }
    if (!tiled_holds(up, (size_t) nexp * mg)) {
        FALLOC(s->au, (size_t) nexp * mg);
        FCK(launch_pack_tiled((const uint8_t *) up, mg, s->au.p, mg, H_, E_, nexp, c->st));
        ar.u = s->au.p;
    }
    if (down_fmt == FL_IQ2 && !tiled_holds(down, (size_t) nexp * md)) {
        FALLOC(s->ad, (size_t) nexp * md);
        FCK(launch_pack_tiled((const uint8_t *) down, md, s->ad.p, md, E_, H_, nexp, c->st));
        ar.d = s->ad.p;
    }
    return ar;
}

// routed down formats: the reference's Q2_K / Q3_K (src/fused_layer.cu:608) and IQ2_XXS (the all-IQ2_XXS configs).
// The reference maps every code but FL_Q3K to Q2_K; codes outside these three are rejected here instead.
static void need_down_fmt(const char * fn, int fmt, const void * down) {
    if (fmt != FL_IQ2 && fmt != FL_Q2K && fmt != FL_Q3K) {
        std::fprintf(stderr, "[fused] %s: down format %d is not supported (FL_IQ2, FL_Q2K or FL_Q3K)\n", fn, fmt);
        std::exit(7);
    }
    if (fmt != FL_IQ2 && (reinterpret_cast<uintptr_t>(down) & 3u)) {
        std::fprintf(stderr, "[fused] %s: the down arena must be 4-byte aligned\n", fn);
        std::exit(7);
    }
}

// ================================================================ entry points
static int ffn_begin_body(FLCtx * c, const FLW * W, int N, const float * ncur, const float * ffn_inp, int wrow, DecodeArgs * spec);
// whether fl_ffn_begin on these rows runs the speculative one-token launch (the last fl_moe's arena still declared)
static bool spec_candidate(FLCtx * c, int N, int wrow) {
    Compat * s = c->compat;
    if (!s || N != 1 || wrow >= 0 || !s->spec_ok) { return false; }
    const size_t mg = (size_t) H_ * (E_ / QK) * IQ2B, md = (size_t) E_ * (H_ / QK) * IQ2B;
    const int ne = c->n_exp;
    return s->shf[0] == FL_IQ2 && s->shf[1] == FL_IQ2 && s->shf[2] == FL_IQ2 && s->spec_nexp == ne && c->topk == MAXK &&
           decode1_available(c) && decode_rule_ok(ne, c->n_group) && tiled_holds(s->spec_g, (size_t) ne * mg) &&
           tiled_holds(s->spec_u, (size_t) ne * mg) && tiled_holds(s->spec_d, (size_t) ne * md);
}
// fl_ffn_begin's enqueued work is bracketed by a pair of events, folded into fl_gpu_ms(0 / 2) when that is read
extern "C" int fl_ffn_begin(FLCtx * c, const FLW * W, int N, const float * ncur, const float * ffn_inp, int wrow) {
    if (!c) { return FL_EINVAL; }
    if (!c->ffn_ev_pending.empty()) { fold_ffn_events(c, c->ffn_ev_pending.size() >= 64); }   // bounded: never more than 64 pairs
    std::pair<hipEvent_t, hipEvent_t> ev{ nullptr, nullptr };
    if (!c->ffn_ev_free.empty()) { ev = c->ffn_ev_free.back(); c->ffn_ev_free.pop_back(); }
    else if (hipEventCreate(&ev.first) != hipSuccess || hipEventCreate(&ev.second) != hipSuccess) {
        (void) hipGetLastError(); return fail(c, FL_EHIP, "hipEventCreate");
    }
    // the pair brackets the call's enqueued work, except on the speculative path (the launch keeps its own clock; the
    // call enqueues only the row's copy kernel besides it once the shared expert is packed)
    const bool timed = !spec_candidate(c, N, wrow);
    if (timed) { TRY(c, hipEventRecord(ev.first, c->st)); }
    DecodeArgs spec{};
    const int rc = ffn_begin_body(c, W, N, ncur, ffn_inp, wrow, &spec);
    if (timed) { TRY(c, hipEventRecord(ev.second, c->st)); c->ffn_ev_pending.push_back(ev); }
    else { c->ffn_ev_free.push_back(ev); }
    if (rc == FL_OK && cs(c)->spec_live) {
        // the speculative one-token launch: no events around it (each costs several us here); its GPU time comes from
        // its own clock words and counts as the experts' (fl_gpu_ms(1)) once fl_moe has waited for it
        Compat * s = cs(c);
        if (int r2 = decode_picks(c, spec)) { s->spec_live = false; return r2; }
        TRY(c, hipEventRecord(s->st_ev[s->st_spec], c->st)); s->st_rec[s->st_spec] = true;   // the copy kernel read the staging
        s->spec_epoch = c->epoch; s->r_tagged = true; s->rtag = c->epoch;
    }
    return rc;
}
// the device counter behind fl_moe's completion word (zero before the first launch; each launch's last workgroup
// resets it)
static unsigned * fcnt_of(FLCtx * c, Compat * s) {
    if (!s->fcnt_zero) {
        FALLOC(s->fcnt, 1);
        CK(hipMemsetAsync(s->fcnt.p, 0, sizeof(unsigned), c->st));
        s->fcnt_zero = true;
    }
    return s->fcnt.p;
}
// a one-token launch's shared expert: IQ2_XXS matrices declared tiled as they are, else fl_ffn_begin's tiled copy;
// K-quants in place
static void one_token_shared(Compat * s, bool iq_sh, DecodeArgs & d) {
    const size_t mg = mat_bytes(H_, E_);
    for (int i = 0; i < 3; ++i) {
        const uint8_t * m = (const uint8_t *) s->sh_key[i];
        if (iq_sh && !tiled_holds(m, i < 2 ? mg : mat_bytes(E_, H_))) { m = s->sh_t.p + i * mg; }
        (i == 0 ? d.sh_gate : i == 1 ? d.sh_up : d.sh_down) = m;
    }
}
static int ffn_begin_body(FLCtx * c, const FLW * W, int N, const float * ncur, const float * ffn_inp, int wrow, DecodeArgs * spec) {
    if (!W || !ncur || !ffn_inp) { return fail(c, FL_EINVAL, "null pointer"); }
    if (N <= 0 || N > RMAX) { return fail(c, FL_ERANGE, "N = %d outside 1..%d", N, RMAX); }
    if (!W->gate_inp || !W->probs_b || !W->sh_gate || !W->sh_up || !W->sh_down) { return fail(c, FL_EINVAL, "router or shared-expert weight missing"); }
    Compat * s = cs(c);
    if (wrow >= 0 && (s->wmax == 0 || wrow + N > s->wmax)) { return fail(c, FL_ERANGE, "wide rows %d..%d exceed fl_wide_init's %d", wrow, wrow + N, s->wmax); }
    const size_t R = (size_t) RMAX * E_;
    const int ne = c->n_exp;
    if (!covers(W->gate_inp, (size_t) ne * E_ * (W->gate_f16 ? 2 : 4)) || !covers(W->probs_b, (size_t) ne * 4)) {
        return fail(c, FL_EINVAL, "router weight or bias allocation is smaller than %d experts x %d", ne, E_);
    }
    if (!covers(W->sh_gate, fmt_bytes(s->shf[0], H_, E_)) || !covers(W->sh_up, fmt_bytes(s->shf[1], H_, E_)) || !covers(W->sh_down, fmt_bytes(s->shf[2], E_, H_))) {
        return fail(c, FL_EINVAL, "shared-expert allocation smaller than one matrix of its format (%d, %d, %d)", s->shf[0], s->shf[1], s->shf[2]);
    }
    for (int i = 0; i < 3; ++i) {
        const void * m = i == 0 ? W->sh_gate : i == 1 ? W->sh_up : W->sh_down;
        if (s->shf[i] != FL_IQ2 && (reinterpret_cast<uintptr_t>(m) & 3u)) { return fail(c, FL_EINVAL, "K-quant shared matrices must be 4-byte aligned"); }
    }
    ALLOC(c, s->ncur, 2 * R); ALLOC(c, s->logits, RMAX * ne); ALLOC(c, s->probs, RMAX * ne);
    ALLOC(c, s->xq, R); ALLOC(c, s->xd, RMAX * (E_ / QK)); ALLOC(c, s->sh_o, R);
    hipStream_t st = c->st;
    const size_t mg1 = mat_bytes(H_, E_), md1 = mat_bytes(E_, H_);
    s->spec_live = spec_candidate(c, N, wrow);
    const int sp = s->st_par ^= 1;
    if (s->st_rec[sp]) { TRY(c, hipEventSynchronize(s->st_ev[sp])); }   // this staging's previous reader has run
    s->in_ncur = s->in_st[sp]; s->in_fi = s->in_ncur + (size_t) N * E_; s->fi = s->ncur.p + (size_t) N * E_;
    s->st_spec = sp;
    if (s->spec_live) {   // one row: the row and its residual in by a small copy kernel reading the mapped staging (no copy engine)
        std::memcpy(s->in_ncur, ncur, (size_t) E_ * 4); std::memcpy(s->in_fi, ffn_inp, (size_t) E_ * 4);
        k_copy16<<<(2 * E_ / 4 + 255) / 256, 256, 0, st>>>((const uint4 *) s->in_st_d[sp], (uint4 *) s->ncur.p, (size_t) 2 * E_ / 4);
        TRY(c, hipGetLastError());
    } else if ((size_t) N * E_ * 4 <= ((size_t) 1 << 20)) {   // a few rows: one copy in (each copy costs a DMA start, ~2-5 us)
        std::memcpy(s->in_ncur, ncur, (size_t) N * E_ * 4); std::memcpy(s->in_fi, ffn_inp, (size_t) N * E_ * 4);
        TRY(c, hipMemcpyAsync(s->ncur.p, s->in_ncur, (size_t) 2 * N * E_ * 4, hipMemcpyHostToDevice, st));
    } else {   // staged and sent in pieces: each piece's DMA runs while the next piece is copied into the staging
        constexpr size_t PIECE = (size_t) 1 << 20;
        const size_t nb = (size_t) N * E_ * 4;
        const uint8_t * src[2] = { reinterpret_cast<const uint8_t *>(ncur), reinterpret_cast<const uint8_t *>(ffn_inp) };
        uint8_t * stg[2] = { reinterpret_cast<uint8_t *>(s->in_ncur), reinterpret_cast<uint8_t *>(s->in_fi) };
        uint8_t * dst[2] = { reinterpret_cast<uint8_t *>(s->ncur.p), reinterpret_cast<uint8_t *>(s->fi) };
        for (int a = 0; a < 2; ++a) {
            for (size_t o = 0; o < nb; o += PIECE) {
                const size_t len = std::min(PIECE, nb - o);
                std::memcpy(stg[a] + o, src[a] + o, len);
                TRY(c, hipMemcpyAsync(dst[a] + o, stg[a] + o, len, hipMemcpyHostToDevice, st));
            }
        }
    }
    if (!s->spec_live) { TRY(c, hipEventRecord(s->st_ev[sp], st)); s->st_rec[sp] = true; }   // the launch records it (fl_ffn_begin)
    const size_t mg = mat_bytes(H_, E_);
    const void * shm[3] = { W->sh_gate, W->sh_up, W->sh_down };
    bool sht[3];
    for (int i = 0; i < 3; ++i) { sht[i] = s->shf[i] == FL_IQ2 && tiled_holds(shm[i], i < 2 ? mg : mat_bytes(E_, H_)); }
    if (s->sh_key[0] != shm[0] || s->sh_key[1] != shm[1] || s->sh_key[2] != shm[2] ||
        s->sh_fkey[0] != s->shf[0] || s->sh_fkey[1] != s->shf[1] || s->sh_fkey[2] != s->shf[2] ||
        s->sh_tkey[0] != sht[0] || s->sh_tkey[1] != sht[1] || s->sh_tkey[2] != sht[2]) {
        ALLOC(c, s->sh_t, 3 * mg);
        for (int i = 0; i < 3; ++i) {   // IQ2_XXS matrices get a tiled copy unless declared tiled; K-quant ones are read in place
            if (s->shf[i] == FL_IQ2 && !sht[i]) {
                TRY(c, launch_pack_tiled((const uint8_t *) shm[i], mg, s->sh_t.p + i * mg, mg, i < 2 ? H_ : E_, i < 2 ? E_ : H_, 1, st));
            }
            s->sh_key[i] = shm[i]; s->sh_fkey[i] = s->shf[i]; s->sh_tkey[i] = sht[i];
        }
    }
    // the F16 router (W->gate_f16, fl.cu:317-319) is widened exactly to fp32 first; the logits then follow the same
    // contract as an F32 router holding the same values
    const float * wr = (const float *) W->gate_inp;
    if (W->gate_f16) {
        ALLOC(c, s->wr32, (size_t) ne * E_);
        TRY(c, launch_f16_to_f32((const uint16_t *) W->gate_inp, s->wr32.p, (int64_t) ne * E_, st));
        wr = s->wr32.p;
    }
    // the picks of row t at z_sel[t * topk ..], their weights right after the N rows' picks, written by the selection
    // straight into host memory (fl_fetch only waits)
    float * wts = reinterpret_cast<float *>(s->z_sel_d + (size_t) N * c->topk);
    unsigned * done = reinterpret_cast<unsigned *>(s->z_sel_d + ZS_DONE);
    if (s->spec_live) {
        // route and run the block in one launch on the last fl_moe's arena (the launch itself is fl_ffn_begin's last)
        FALLOC(s->ids, 2 * MAXK); FALLOC(s->w, MAXK); FALLOC(s->counts, ne); FALLOC(s->offsets, ne + 1); FALLOC(s->perm, MAXK);
        FALLOC(s->inv, MAXK); FALLOC(s->act, ne); FALLOC(s->nact, 1); FALLOC(s->o, (size_t) MAXK * E_);
        if (int rc = ensure_expert_scratch(c, 1, E_, H_)) { s->spec_live = false; return rc; }
        DecodeArgs & d = *spec;
        d.x = s->ncur.p; d.n = 1; d.resid = s->fi;
        d.Wr = wr; d.bias = (const float *) W->probs_b;
        d.n_exp = ne; d.n_group = c->n_group; d.topk_group = c->topk_group; d.topk = MAXK; d.keep = MAXK; d.scale = c->scale;
        d.gate = (const uint8_t *) s->spec_g; d.up = (const uint8_t *) s->spec_u; d.down = (const uint8_t *) s->spec_d; d.estride = mg1;
        d.dstride = md1; d.kdown = 0;
        one_token_shared(s, true, d);
        d.E = E_; d.H = H_; d.xq = s->xq.p; d.xd = s->xd.p;
        d.logits = s->logits.p; d.probs = s->probs.p; d.sel = s->ids.p; d.wts = s->w.p; d.counts = s->counts.p; d.offsets = s->offsets.p;
        d.perm = s->perm.p; d.inv = s->inv.p; d.act = s->act.p; d.nact = s->nact.p;
        d.moe_out = s->z_out_d + (size_t) NB * E_; d.o_out = s->o.p; d.y = s->z_out_d;
        d.spec_combine = 1; d.hsel = s->z_sel_d; d.hdone = done;
        d.tstamp = reinterpret_cast<uint64_t *>(s->z_sel_d + ZS_TSTAMP);
        d.fcnt = fcnt_of(c, s); d.fdone = reinterpret_cast<unsigned *>(s->z_sel_d + ZS_FDONE);
    } else {
        if (int rc = route_dev(c, wr, (const float *) W->probs_b, s->ncur.p, N, ne, E_, s->logits.p, s->probs.p, s->z_sel_d, wts, done)) {
            return rc;
        }
        s->r_tagged = router_fused_ok(N, E_); s->rtag = c->epoch;
    }
    s->N = N;
    s->sh_pending = true; s->xq_pending = true;
    if (wrow >= 0) {   // the wide pass: the rows' Q8_K (fl_wide_moe) and ffn_inp (base = ffn_inp + shared, formed later)
        quant_now(c, s);
        TRY(c, hipMemcpyAsync(s->xq_all.p + (size_t) wrow * E_, s->xq.p, (size_t) N * E_, hipMemcpyDeviceToDevice, st));
        TRY(c, hipMemcpyAsync(s->xd_all.p + (size_t) wrow * (E_ / QK), s->xd.p, (size_t) N * (E_ / QK) * 4, hipMemcpyDeviceToDevice, st));
        TRY(c, hipMemcpyAsync(s->fi_all.p + (size_t) wrow * E_, s->fi, (size_t) N * E_ * 4, hipMemcpyDeviceToDevice, st));
        s->wide_pending = true;
    }
    return FL_OK;
}

// Pinned host -> device on the context's stream (src/fused_layer.cu:414-420): a kernel reads the mapped host memory, so
// the copy is ordered with the context's launches and uses no copy engine; memory HIP cannot map (pageable) goes
// through the copy engine instead. Either way the call only enqueues: src must stay valid until the stream reaches it.
extern "C" void fl_h2d(FLCtx * c, void * dst, const void * src, size_t bytes) {
    if (bytes == 0) { return; }
    if (!dst || !src) { std::fprintf(stderr, "[fused] fl_h2d: null pointer\n"); std::exit(7); }
    void * dp = nullptr;
    if (hipHostGetDevicePointer(&dp, const_cast<void *>(src), 0) != hipSuccess) { (void) hipGetLastError(); dp = nullptr; }
    if (dp) {
        if ((((uintptr_t) dst | (uintptr_t) dp | bytes) & 15) == 0) {
            const size_t n = bytes / 16;
            k_copy16<<<(unsigned) std::min<size_t>((n + 1023) / 1024, 2048), 256, 0, c->st>>>((const uint4 *) dp, (uint4 *) dst, n);
        } else {
            k_copy1<<<(unsigned) std::min<size_t>((bytes + 255) / 256, 8192), 256, 0, c->st>>>((const uint8_t *) dp, (uint8_t *) dst, bytes);
        }
        CK(hipGetLastError());
        c->h2d_zc += bytes;
    } else {
        CK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->st));
        c->h2d_ce += bytes;
    }
    if (!c->h2d_said && c->h2d_zc + c->h2d_ce > ((size_t) 64 << 20)) {
        c->h2d_said = 1;
        std::fprintf(stderr, "[fused] host->device by kernel (mapped pinned) %.0f MB, by copy engine %.0f MB so far\n",
                     c->h2d_zc / 1048576.0, c->h2d_ce / 1048576.0);
    }
}
extern "C" int fl_h2d_bytes(FLCtx * c, size_t * by_kernel, size_t * by_copy_engine) {
    if (!c) { return FL_EINVAL; }
    if (by_kernel) { *by_kernel = c->h2d_zc; }
    if (by_copy_engine) { *by_copy_engine = c->h2d_ce; }
    return FL_OK;
}

extern "C" void fl_fetch(FLCtx * c, int n, int what, FLOut * out) {
    std::memset(out, 0, sizeof(FLOut));
    Compat * s = cs(c);
    if (n < 0 || n > s->N) { std::fprintf(stderr, "[fused] fl_fetch: %d rows requested, %d routed\n", n, s->N); std::exit(7); }
    // the picks and weights are in z_sel once the routing has run: its done word says so for a routing in one launch
    // (nothing else that the call returns is pending then); otherwise, or if the word is late, the stream is waited
    const bool seen = (what & ~1) == 0 && s->r_tagged && spin_words(reinterpret_cast<const unsigned *>(s->z_sel + ZS_DONE), 1, s->rtag, 20000.0);
    if (!seen) { CK(hipStreamSynchronize(c->st)); }
    if (c->herr && __atomic_load_n(c->herr, __ATOMIC_ACQUIRE)) {   // the routing's poll timed out: its picks are -1
        std::fprintf(stderr, "[fused] fl_fetch: the routing launch reported device code %d\n", *c->herr); std::exit(7);
    }
    if (what & 1) {
        // the mirrors keep this call's values until the next fl_fetch whatever is enqueued meanwhile (the reference's
        // lifetime). ncur and ffn_inp are on the device exactly as the caller handed them to fl_ffn_begin (nothing
        // writes them), and that call's pinned staging holds them until the second fl_ffn_begin after it: the ncur and
        // fi mirrors are that staging itself
        const size_t pk = (size_t) n * c->topk;
        std::memcpy(s->h_sel, s->z_sel, pk * 4); std::memcpy(s->h_wts, s->z_sel + (size_t) s->N * c->topk, pk * 4);
        out->sel = s->h_sel; out->wts = s->h_wts; out->ncur = s->in_ncur; out->fi = s->in_fi;
    }
}

extern "C" void fl_moe(FLCtx * c, const void * gate, const void * up, const void * down, int nexp, int down_fmt, const int * ids,
                       const float * w, int KE, int n, FLOut * out) {
    std::memset(out, 0, sizeof(FLOut));
    need_down_fmt("fl_moe", down_fmt, down);
    Compat * s = cs(c);
    if (n <= 0 || n > NB || n > s->N || KE <= 0 || KE > MAXK || nexp <= 0 || nexp > NEXP_) {
        std::fprintf(stderr, "[fused] fl_moe: n %d (routed rows %d), KE %d, nexp %d out of range\n", n, s->N, KE, nexp); std::exit(7);
    }
    for (int i = 0; i < n * KE; ++i) {
        if (ids[i] < 0 || ids[i] >= nexp) { std::fprintf(stderr, "[fused] fl_moe: slot id %d outside the arena of %d\n", ids[i], nexp); std::exit(7); }
    }
    if (!covers(gate, nexp * mat_bytes(H_, E_)) || !covers(up, nexp * mat_bytes(H_, E_)) || !covers(down, nexp * fmt_bytes(down_fmt, E_, H_))) {
        std::fprintf(stderr, "[fused] fl_moe: an arena allocation is smaller than %d experts\n", nexp); std::exit(7);
    }
    hipStream_t st = c->st; const int P = n * KE;
    if (!c->moe_ev_pending.empty()) { fold_events(c->moe_ev_pending, c->moe_ev_free, c->ms_moe, c->moe_ev_pending.size() >= 64); }
    const bool kq_sh = s->shf[0] == FL_Q5K && s->shf[1] == FL_Q5K && s->shf[2] == FL_Q6K;
    const bool iq_sh = s->shf[0] == FL_IQ2 && s->shf[1] == FL_IQ2 && s->shf[2] == FL_IQ2;
    // the routing's own picks and weights of the last fl_ffn_begin on one row (z_sel: 8 ids, then 8 weights)
    const bool own_picks = n == 1 && KE == MAXK && s->N == 1 && s->r_tagged &&
                           std::memcmp(ids, s->z_sel, MAXK * 4) == 0 && std::memcmp(w, s->z_sel + MAXK, MAXK * 4) == 0;
    if (s->spec_live) {
        s->spec_live = false;
        if (own_picks && gate == s->spec_g && up == s->spec_u && down == s->spec_d && nexp == s->spec_nexp && down_fmt == FL_IQ2 && iq_sh) {
            // fl_ffn_begin's launch computed exactly this call: wait for its completion word (or the stream)
            if (!spin_words(reinterpret_cast<const unsigned *>(s->z_sel + ZS_FDONE), 1, s->spec_epoch, 20000.0)) { CK(hipStreamSynchronize(st)); }
            const uint64_t * ts = reinterpret_cast<const uint64_t *>(s->z_sel + ZS_TSTAMP);
            const uint64_t t0 = __atomic_load_n(ts, __ATOMIC_ACQUIRE), t1 = __atomic_load_n(ts + 1, __ATOMIC_ACQUIRE);
            if (t1 > t0) { c->ms_moe += (double) (t1 - t0) * 1e-5; }   // 100 MHz ticks
            if (c->herr && __atomic_load_n(c->herr, __ATOMIC_ACQUIRE)) {
                std::fprintf(stderr, "[fused] fl_moe: the one-token launch reported device code %d\n", *c->herr); std::exit(7);
            }
            c->last_kernel = 3; c->last_fused = 1;
            s->last_ids.assign(ids, ids + P); s->last_KE = KE; s->last_n = n; s->last_fast = true;
            out->h = s->z_out; out->moe = s->z_out + (size_t) NB * E_;
            return;
        }
    }
    c->last_kernel = 0;   // fl_debug: 2 / 1 when the one-token kernel / the n <= 8 block below runs the call
    int max_slots = 1;
    { std::vector<int> per(nexp, 0); for (int i = 0; i < P; ++i) { max_slots = std::max(max_slots, ++per[ids[i]]); } }
    std::pair<hipEvent_t, hipEvent_t> mv;
    if (!take_events(c->moe_ev_free, mv)) { fatal("hipEventCreate", hipErrorOutOfMemory, __FILE__, __LINE__); }
    CK(hipEventRecord(mv.first, st));
    FALLOC(s->ids, 2 * P); FALLOC(s->counts, nexp); FALLOC(s->offsets, nexp + 1); FALLOC(s->perm, P); FALLOC(s->inv, P);
    FALLOC(s->act, nexp); FALLOC(s->nact, 1); FALLOC(s->o, (size_t) P * E_); FALLOC(s->hout, (size_t) NB * E_); FALLOC(s->moe, (size_t) NB * E_);
    // One launch on the caller's picks (router and selection skipped; the shared expert and the Q8_K of fl_ffn_begin's
    // rows computed in the same launch; the combine in this function's order): one row with all 8 picks on the
    // one-token kernel, when the formats are one of its variants (every matrix IQ2_XXS, or the routed down Q2_K / Q3_K
    // with a Q5_K / Q5_K / Q6_K shared expert); up to 8 rows of an all-IQ2_XXS layer on the n <= 8 block. Results
    // bit-identical to the per-pass kernels below. The launch reads the picks from host memory and writes h and moe
    // there (z_in, z_out): no copies either way.
    const bool fast1 = n == 1 && KE == MAXK && decode1_available(c) &&
                       ((down_fmt == FL_IQ2 && iq_sh) || ((down_fmt == FL_Q2K || down_fmt == FL_Q3K) && kq_sh && !(reinterpret_cast<uintptr_t>(down) & 3u)));
    const bool fast = fast1 || (down_fmt == FL_IQ2 && iq_sh && decode_block_available(c));
    const float * dw = nullptr;   // the device weights of the per-pass path
    if (!fast) {
        if (s->in_rec) { CK(hipEventSynchronize(s->in_ev)); }
        std::memcpy(s->in_ids, ids, (size_t) P * 4); std::memcpy(s->in_ids + P, w, (size_t) P * 4);   // ids, then weights
        CK(hipMemcpyAsync(s->ids.p, s->in_ids, (size_t) 2 * P * 4, hipMemcpyHostToDevice, st));
        dw = reinterpret_cast<const float *>(s->ids.p + P);
        CK(hipEventRecord(s->in_ev, st)); s->in_rec = true;
    } else {   // the previous fl_moe has ended (each call waits for its stream): the launch that read z_in is done
        std::memcpy(s->z_in, ids, (size_t) P * 4); std::memcpy(s->z_in + NB * MAXK, w, (size_t) P * 4);
    }
    const Arena ar = pack_arena(c, s, gate, up, down, nexp, down_fmt);
    if (fast) {
        CK(ensure_expert_scratch(c, (size_t) n, E_, H_) == FL_OK ? hipSuccess : hipErrorOutOfMemory);
        const size_t mg = mat_bytes(H_, E_);
        DecodeArgs d{};
        d.x = s->ncur.p; d.n = n; d.resid = s->fi;
        d.n_exp = nexp; d.n_group = c->n_group; d.topk_group = c->topk_group; d.topk = KE; d.keep = KE; d.scale = c->scale;
        d.gate = ar.g; d.up = ar.u; d.estride = mg;
        d.down = down_fmt == FL_IQ2 ? ar.d : (const uint8_t *) down; d.dstride = fmt_bytes(down_fmt, E_, H_);
        one_token_shared(s, iq_sh, d);
        d.kdown = down_fmt == FL_IQ2 ? 0 : down_fmt;
        d.E = E_; d.H = H_; d.xq = s->xq.p; d.xd = s->xd.p;
        d.ext_sel = s->z_in_d; d.ext_w = reinterpret_cast<const float *>(s->z_in_d + NB * MAXK);
        d.moe_out = s->z_out_d + (size_t) NB * E_; d.o_out = s->o.p; d.y = s->z_out_d;
        if (fast1) { d.fcnt = fcnt_of(c, s); d.fdone = reinterpret_cast<unsigned *>(s->z_sel_d + ZS_FDONE); }
        if (decode_picks(c, d) != FL_OK) { std::fprintf(stderr, "[fused] fl_moe: %s\n", c->err.c_str()); std::exit(7); }
    } else {
        quant_now(c, s); shared_now(c, s);
        CK(launch_dispatch(s->ids.p, P, nexp, s->counts.p, s->offsets.p, s->perm.p, s->inv.p, s->act.p, s->nact.p, st));
        routed_experts(c, s, ar, s->xq.p, s->xd.p, n, P, KE, nexp, s->act.p, s->nact.p, s->offsets.p, s->perm.p, s->o.p, down_fmt, down, max_slots);
        k_combine_slots<<<dim3(E_ / 256, n), 256, 0, st>>>(s->o.p, s->inv.p, s->ids.p, dw, n, KE, s->sh_o.p, s->fi, s->hout.p, s->moe.p);
        CK(hipGetLastError());
        CK(hipMemcpyAsync(s->h_h, s->hout.p, (size_t) n * E_ * 4, hipMemcpyDeviceToHost, st));
        CK(hipMemcpyAsync(s->h_moe, s->moe.p, (size_t) n * E_ * 4, hipMemcpyDeviceToHost, st));
    }
    CK(hipEventRecord(mv.second, st));
    // the one-token launch is waited for on its completion word (its outputs are in host memory by then); otherwise,
    // or if the word is late, on the stream
    const bool seen = fast1 && c->last_kernel == 2 && spin_words(reinterpret_cast<const unsigned *>(s->z_sel + ZS_FDONE), 1, c->epoch, 20000.0);
    if (seen) {
        c->moe_ev_pending.push_back(mv);
    } else {
        CK(hipStreamSynchronize(st));
        float ms = 0.f; CK(hipEventElapsedTime(&ms, mv.first, mv.second)); c->ms_moe += ms;
        c->moe_ev_free.push_back(mv);
    }
    if (fast && c->herr && __atomic_load_n(c->herr, __ATOMIC_ACQUIRE)) {   // a wait of the launch timed out
        std::fprintf(stderr, "[fused] fl_moe: the one-token launch reported device code %d\n", *c->herr); std::exit(7);
    }
    // a resident arena used on the routing's own picks: the next fl_ffn_begin on one row may run this block itself
    s->spec_ok = fast1 && own_picks && down_fmt == FL_IQ2 && iq_sh && tiled_holds(gate, (size_t) nexp * mat_bytes(H_, E_)) &&
                 tiled_holds(up, (size_t) nexp * mat_bytes(H_, E_)) && tiled_holds(down, (size_t) nexp * mat_bytes(E_, H_));
    if (s->spec_ok) { s->spec_g = gate; s->spec_u = up; s->spec_d = down; s->spec_nexp = nexp; }
    s->last_ids.assign(ids, ids + P); s->last_KE = KE; s->last_n = n; s->last_fast = fast;
    out->h = fast ? s->z_out : s->h_h; out->moe = fast ? s->z_out + (size_t) NB * E_ : s->h_moe;
}

extern "C" void fl_skip(FLCtx * c, const float * mo, int n, FLOut * out) {
    std::memset(out, 0, sizeof(FLOut));
    Compat * s = cs(c);
    if (n <= 0 || n > s->N) { std::fprintf(stderr, "[fused] fl_skip: n %d outside the %d routed rows\n", n, s->N); std::exit(7); }
    hipStream_t st = c->st;
    CK(hipEventRecord(c->em0, st));
    FALLOC(s->moe, (size_t) RMAX * E_); FALLOC(s->hout, (size_t) RMAX * E_);
    shared_now(c, s);
    CK(hipMemcpyAsync(s->moe.p, mo, (size_t) n * E_ * 4, hipMemcpyHostToDevice, st));
    k_skip_rows<<<nblk((int64_t) n * E_), 256, 0, st>>>(s->moe.p, s->sh_o.p, s->fi, (int64_t) n * E_, s->hout.p);
    CK(hipGetLastError());
    CK(hipMemcpyAsync(s->h_h, s->hout.p, (size_t) n * E_ * 4, hipMemcpyDeviceToHost, st));
    CK(hipEventRecord(c->em1, st));
    CK(hipStreamSynchronize(st));
    float ms = 0.f; CK(hipEventElapsedTime(&ms, c->em0, c->em1)); c->ms_moe += ms;
    out->h = s->h_h;
}

extern "C" void fl_moe_outs(FLCtx * c, int b, const int * ids, const float * w, int KE, float * out) {
    Compat * s = cs(c);
    CK(hipStreamSynchronize(c->st));
    if (b < 0 || b >= s->last_n || KE != s->last_KE) { std::fprintf(stderr, "[fused] fl_moe_outs: row %d / KE %d do not match the last fl_moe\n", b, KE); std::exit(7); }
    std::vector<int> inv((size_t) s->last_n * KE);
    if (s->last_fast) { for (size_t i = 0; i < inv.size(); ++i) { inv[i] = (int) i; } }   // the one-token launch: slot k at row k
    else { CK(hipMemcpy(inv.data(), s->inv.p, inv.size() * 4, hipMemcpyDeviceToHost)); }
    std::vector<float> row(E_);
    for (int k = 0; k < KE; ++k) {
        int kf = -1;
        for (int j = 0; j < KE; ++j) { if (s->last_ids[(size_t) b * KE + j] == ids[k]) { kf = j; break; } }
        if (kf < 0) { std::memset(out + (size_t) k * E_, 0, E_ * 4); continue; }   // this row never ran that slot
        CK(hipMemcpy(row.data(), s->o.p + (size_t) inv[(size_t) b * KE + kf] * E_, E_ * 4, hipMemcpyDeviceToHost));
        for (int e = 0; e < E_; ++e) { out[(size_t) k * E_ + e] = w[k] * row[e]; }
    }
}

extern "C" int fl_wide_init(FLCtx * c, int wmax, int KE) {
    Compat * s = cs(c);
    if (wmax <= 0 || KE <= 0 || KE > MAXK) { std::fprintf(stderr, "[fused] fl_wide_init: wmax %d, KE %d\n", wmax, KE); std::exit(7); }
    s->wmax = wmax; s->wke = KE;
    const size_t R = (size_t) wmax * E_;
    FALLOC(s->fi_all, R); FALLOC(s->sh_all, R); FALLOC(s->base_all, R); s->wide_pending = false; FALLOC(s->out_all, R * KE); FALLOC(s->xq_all, R); FALLOC(s->xd_all, (size_t) wmax * (E_ / QK));
    CK(hipMemset(s->out_all.p, 0, R * KE * 4));
    if (s->h_wh) { (void) hipHostFree(s->h_wh); } if (s->h_wmoe) { (void) hipHostFree(s->h_wmoe); }
    s->h_wh = mapped<float>(R, &s->h_wh_d); s->h_wmoe = mapped<float>(R, &s->h_wmoe_d);
    if (!s->h_wh || !s->h_wmoe) { fatal("hipHostMalloc (wide-pass mirrors)", hipErrorOutOfMemory, __FILE__, __LINE__); }
    for (hipEvent_t & e : s->wev) { if (!e) { CK(hipEventCreateWithFlags(&e, hipEventDisableTiming)); } }
    return 1;
}

extern "C" void fl_wide_moe(FLCtx * c, const void * gate, const void * up, const void * down, int down_fmt, int nexp, const int * midx,
                            const int * rows, const int * kidx, const float * wk, int nslots, int KE, int par) {
    need_down_fmt("fl_wide_moe", down_fmt, down);
    Compat * s = cs(c);
    if (KE != s->wke || nexp <= 0 || nexp > NEXP_ || nslots < 0) { std::fprintf(stderr, "[fused] fl_wide_moe: KE %d (init %d), nexp %d, nslots %d\n", KE, s->wke, nexp, nslots); std::exit(7); }
    // the slot tables as (expert, row, k, w) pairs, grouped by expert in slot order (a stable counting sort)
    std::vector<int> cnt(nexp + 1, 0);
    for (int sl = 0; sl < nslots; ++sl) {
        if (midx[sl] < 0 || midx[sl] >= nexp) { std::fprintf(stderr, "[fused] fl_wide_moe: slot expert %d outside the batch of %d\n", midx[sl], nexp); std::exit(7); }
        for (int j = 0; j < NB; ++j) {
            const int r = rows[sl * NB + j];
            if (r < 0) { continue; }
            if (r >= s->wmax || kidx[sl * NB + j] < 0 || kidx[sl * NB + j] >= KE) { std::fprintf(stderr, "[fused] fl_wide_moe: pair (row %d, k %d) out of range\n", r, kidx[sl * NB + j]); std::exit(7); }
            cnt[midx[sl] + 1]++;
        }
    }
    for (int e = 0; e < nexp; ++e) { cnt[e + 1] += cnt[e]; }
    const int P = cnt[nexp];
    if (P == 0) { return; }
    if (!covers(gate, nexp * mat_bytes(H_, E_)) || !covers(up, nexp * mat_bytes(H_, E_)) || !covers(down, nexp * fmt_bytes(down_fmt, E_, H_))) {
        std::fprintf(stderr, "[fused] fl_wide_moe: an arena allocation is smaller than %d experts\n", nexp); std::exit(7);
    }
    int max_slots = 1;
    for (int e = 0; e < nexp; ++e) { max_slots = std::max(max_slots, cnt[e + 1] - cnt[e]); }
    // the tables go to this parity's pinned buffers: [act nexp | off nexp + 1 | perm P | row P | k P | nact 1], wk P.
    // Their previous copies were queued two batches ago (the engine alternates parities and waits for each before
    // reusing it); the event recorded after those copies makes sure of it whatever the caller does.
    const int pb = par & 1;
    if (!s->wt_ev[pb]) { CK(hipEventCreateWithFlags(&s->wt_ev[pb], hipEventDisableTiming)); }
    if (s->wt_rec[pb]) { CK(hipEventSynchronize(s->wt_ev[pb])); }
    const size_t ni = (size_t) nexp + (nexp + 1) + 3 * (size_t) P + 1;
    if (ni > s->wt_cap[pb] || (size_t) P > s->wt_cap[pb]) {
        if (s->wt_i[pb]) { (void) hipHostFree(s->wt_i[pb]); } if (s->wt_w[pb]) { (void) hipHostFree(s->wt_w[pb]); }
        const size_t cap = std::max(ni, (size_t) 4096);
        s->wt_i[pb] = pinned<int>(cap); s->wt_w[pb] = pinned<float>(cap);
        if (!s->wt_i[pb] || !s->wt_w[pb]) { fatal("hipHostMalloc (wide-pass slot tables)", hipErrorOutOfMemory, __FILE__, __LINE__); }
        s->wt_cap[pb] = cap;
    }
    int * h_act = s->wt_i[pb], * h_off = h_act + nexp, * h_perm = h_off + nexp + 1, * h_row = h_perm + P, * h_k = h_row + P, * h_nact = h_k + P;
    float * h_wk = s->wt_w[pb];
    std::vector<int> fillp(cnt.begin(), cnt.end() - 1);
    for (int e = 0; e <= nexp; ++e) { h_off[e] = cnt[e]; }
    for (int sl = 0; sl < nslots; ++sl) {
        for (int j = 0; j < NB; ++j) {
            const int r = rows[sl * NB + j];
            if (r < 0) { continue; }
            const int pos = fillp[midx[sl]]++;
            h_perm[pos] = r * KE + kidx[sl * NB + j]; h_row[pos] = r; h_k[pos] = kidx[sl * NB + j]; h_wk[pos] = wk[sl * NB + j];
        }
    }
    int na = 0;
    for (int e = 0; e < nexp; ++e) { if (cnt[e + 1] > cnt[e]) { h_act[na++] = e; } }
    *h_nact = na;
    hipStream_t st = c->st;
    FALLOC(s->w_act, nexp); FALLOC(s->w_off, nexp + 1); FALLOC(s->w_perm, P); FALLOC(s->w_nact, 1); FALLOC(s->w_row, P); FALLOC(s->w_k, P); FALLOC(s->w_wk, P);
    FALLOC(s->o, (size_t) P * E_);
    CK(hipMemcpyAsync(s->w_act.p, h_act, (size_t) na * 4, hipMemcpyHostToDevice, st));
    CK(hipMemcpyAsync(s->w_off.p, h_off, (size_t) (nexp + 1) * 4, hipMemcpyHostToDevice, st));
    CK(hipMemcpyAsync(s->w_perm.p, h_perm, (size_t) P * 4, hipMemcpyHostToDevice, st));
    CK(hipMemcpyAsync(s->w_nact.p, h_nact, 4, hipMemcpyHostToDevice, st));
    CK(hipMemcpyAsync(s->w_row.p, h_row, (size_t) P * 4, hipMemcpyHostToDevice, st));
    CK(hipMemcpyAsync(s->w_k.p, h_k, (size_t) P * 4, hipMemcpyHostToDevice, st));
    CK(hipMemcpyAsync(s->w_wk.p, h_wk, (size_t) P * 4, hipMemcpyHostToDevice, st));
    CK(hipEventRecord(s->wt_ev[pb], st)); s->wt_rec[pb] = true;
    const Arena ar = pack_arena(c, s, gate, up, down, nexp, down_fmt);
    routed_experts(c, s, ar, s->xq_all.p, s->xd_all.p, s->wmax, P, KE, nexp, s->w_act.p, s->w_nact.p, s->w_off.p, s->w_perm.p, s->o.p,
                   down_fmt, down, max_slots);
    k_wide_scatter<<<dim3((E_ / 4 + 255) / 256, grid_y(P)), 256, 0, st>>>(s->o.p, s->w_row.p, s->w_k.p, s->w_wk.p, P, KE, s->out_all.p);
    CK(hipGetLastError());
    // no wait: the reference's call only enqueues too (src/fused_layer.cu:528-555); fl_wide_mark / fl_wide_wait order
    // the engine's reuse of its staging and of these tables
}

extern "C" void fl_wide_mark(FLCtx * c, int par) { Compat * s = cs(c); if (s->wev[par & 1]) { CK(hipEventRecord(s->wev[par & 1], c->st)); } }
extern "C" void fl_wide_wait(FLCtx * c, int par) { Compat * s = cs(c); if (s->wev[par & 1]) { CK(hipEventSynchronize(s->wev[par & 1])); } }

// base = ffn_inp + shared for the wide pass's rows 0 .. n - 1: the shared expert on all of them at once (the rows'
// Q8_K as fl_ffn_begin(wrow) left them), once per set of rows
static void wide_base(FLCtx * c, Compat * s, int n) {
    if (!s->wide_pending) { return; }
    shared_expert(c, s, s->xq_all.p, s->xd_all.p, n, s->sh_all.p);
    k_base_rows<<<nblk((int64_t) n * E_), 256, 0, c->st>>>(s->fi_all.p, s->sh_all.p, (int64_t) n * E_, s->base_all.p);
    CK(hipGetLastError());
    s->wide_pending = false;
}

extern "C" void fl_wide_finish(FLCtx * c, int n, int KE, FLOut * out) {
    std::memset(out, 0, sizeof(FLOut));
    Compat * s = cs(c);
    if (n <= 0 || n > s->wmax || KE != s->wke) { std::fprintf(stderr, "[fused] fl_wide_finish: n %d (wmax %d), KE %d (init %d)\n", n, s->wmax, KE, s->wke); std::exit(7); }
    hipStream_t st = c->st; const int64_t tot = (int64_t) n * E_;
    wide_base(c, s, n);
    k_wide_finish<<<nblk(tot), 256, 0, st>>>(s->base_all.p, s->out_all.p, KE, tot, s->h_wh_d, s->h_wmoe_d);
    CK(hipGetLastError());
    CK(hipStreamSynchronize(st));
    out->h = s->h_wh; out->moe = s->h_wmoe;
}

extern "C" void fl_wide_skip(FLCtx * c, const float * mo, int n, FLOut * out) {
    std::memset(out, 0, sizeof(FLOut));
    Compat * s = cs(c);
    if (n <= 0 || n > s->wmax) { std::fprintf(stderr, "[fused] fl_wide_skip: n %d (wmax %d)\n", n, s->wmax); std::exit(7); }
    hipStream_t st = c->st; const int64_t tot = (int64_t) n * E_;
    FALLOC(s->moe, (size_t) tot);
    wide_base(c, s, n);
    CK(hipMemcpyAsync(s->moe.p, mo, (size_t) tot * 4, hipMemcpyHostToDevice, st));
    k_wide_skip<<<nblk(tot), 256, 0, st>>>(s->base_all.p, s->moe.p, tot, s->h_wh_d);
    CK(hipGetLastError());
    CK(hipStreamSynchronize(st));
    out->h = s->h_wh;
}

extern "C" void fl_wide_outs(FLCtx * c, int row, int KE, float * out) {
    Compat * s = cs(c);
    if (row < 0 || row >= s->wmax || KE != s->wke) { std::fprintf(stderr, "[fused] fl_wide_outs: row %d, KE %d\n", row, KE); std::exit(7); }
    CK(hipStreamSynchronize(c->st));
    CK(hipMemcpy(out, s->out_all.p + (size_t) row * KE * E_, (size_t) KE * E_ * 4, hipMemcpyDeviceToHost));
}

// formats of FLW's shared expert for fl_ffn_begin: IQ2_XXS (default) or the reference's shards' Q5_K / Q5_K / Q6_K
// (src/fused_layer.h:14, src/fused_layer.cu:520-524); gate and up are both IQ2_XXS or both K-quants
extern "C" int fl_set_shared_formats(FLCtx * c, int gate_fmt, int up_fmt, int down_fmt) {
    if (!c) { return FL_EINVAL; }
    const int f[3] = { gate_fmt, up_fmt, down_fmt };
    for (int i = 0; i < 3; ++i) {
        if (f[i] != FL_IQ2 && kq_block_bytes(f[i]) == 0) { return fail(c, FL_EINVAL, "format %d is not IQ2_XXS or a K-quant (Q2_K, Q3_K, Q5_K, Q6_K)", f[i]); }
    }
    if ((gate_fmt == FL_IQ2) != (up_fmt == FL_IQ2)) { return fail(c, FL_EINVAL, "gate and up must both be IQ2_XXS or both K-quants"); }
    Compat * s = cs(c);
    s->shf[0] = gate_fmt; s->shf[1] = up_fmt; s->shf[2] = down_fmt;
    return FL_OK;
}
