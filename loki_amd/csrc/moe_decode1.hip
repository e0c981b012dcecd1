// moe_decode1.hip -- the MoE block for one decode token (top-8 kept) in one launch, organised by XCD.
//
// Reference path (src/fused_layer.cu): router_probs + router_topk (:313-332), the host round-trip (fl_fetch :587-598,
// eng:793-818), fl_moe (:599-612): quant_x, tc_matvec gate/up, swiglu_q8, tc_matvec down, moe_combine. Here the
// 256 workgroups (one per CU, 16 waves, 32 per XCD) run the block end to end. A workgroup's role is (x, i): x the XCD
// it runs on (hardware register XCC_ID), i = b / 8; the dispatch places workgroup b on XCD (r + b) % 8, so every role
// is taken once.
//   1. every workgroup b computes the router logit of expert b (the fp64 chunk-and-tree contract, waves 0-3) and
//      publishes the logit as an epoch-tagged word, while waves 4-15 stage the codebook/sign tables and Q8_K(x)
//      in LDS and the last 7 waves then run one gate/up task of the shared expert (routing-independent: shared h rows
//      8 t .. 8 t + 7 with t = 32 x + i, so XCD x produces the shared expert's h block x);
//   2. one workgroup per XCD selects the token's experts and broadcasts the picks to its XCD; pick k (0..7, selection
//      order) is slot k, and slot k runs on XCD k. With every matrix IQ2_XXS, role (x, i) computes the h rows of
//      expert sel[x] in two phases of 32 rows, 256 kb_p + 32 (i % 8) .. + 31 with kb_0 = i / 8 and kb_1 = 4 + i / 8,
//      each 28 items (one matrix, two 256-weight blocks, 32 rows) that the waves claim from an LDS counter, so the
//      eight workgroups of (slot, i / 8) complete h block kb_0 half-way through the gate/up and h block kb_1 at its end
//      (the K-quant variants: h rows kb * 256 + q * 64 .. + 63 with kb = i / 4, q = i % 4, as 56 items of 64 rows);
//   3. each workgroup quantises the h blocks it needs to Q8_K and runs the slot's down on them (split-K: one
//      256-weight block per row, one row per lane): K-block kb_0 for an eighth of its 7168 rows, 3 or 4 row groups of
//      the shared expert's down for K-block x, then K-block kb_1 for the same eighth -- the first two while block kb_1's
//      hand-off completes (K-quant variants: K-block kb for a quarter of the rows). Each row's block term
//      (d_w * d_x) * bsum is published as a tagged word;
//   4. workgroup b combines rows 28 b .. 28 b + 27: per slot the 8 block terms folded in block order (ggml's sumf),
//      * 0.125, then y = sum_k w_k o_k in k order + the shared o (+ the residual).
// The arithmetic is that of the other decode kernels and the CPU checker step for step (the same device functions and
// fold orders), so y is bit-identical to them. The down waits on the workgroups of its own XCD that complete its h
// block rather than on every gate/up task of the expert, and no dispatch table is built (one token: the picks are distinct experts). Hand-offs
// inside an XCD (the picks, h) stay in its L2; those across XCDs (logits, down partials) go through the device's
// coherence point. Every wait is bounded: a timeout sets the error word and the wave skips the work, so the grid
// always drains.
#include "kquant_device.h"
#include "moe_kernels.h"

namespace lk {

#ifdef LK_D1_WAVES
constexpr int W1 = LK_D1_WAVES;
#else
constexpr int W1 = 16;                 // waves per workgroup: 4 per SIMD (the block product's issue rate rises with them)
#endif
constexpr int NT1 = W1 * 64;
constexpr int NQW1 = W1 - 4;           // waves staging the tables and the token (the router runs on waves 0-3)
static_assert(NQW1 >= 4 && W1 >= 8, "four router waves and at least four staging waves");
constexpr int G1 = 256, NX1 = 8;       // workgroups, XCDs
constexpr int E1 = 7168, H1 = 2048;
using GX1 = Geo<7, 0>;                 // the token's staged Q8_K row: 28 blocks, no padding
constexpr int NBX1 = E1 / QK, NBH1 = H1 / QK;    // 28, 8 blocks
constexpr int SLOTS1 = 9;              // 8 picks + the shared expert (slot 8)
constexpr int BCAST1 = 1024;           // tagged words 1024 + 16 x .. + 15: XCD x's picks and weights (one-token calls use 0..255)
constexpr int QROWS1 = E1 / 4;         // routed down rows per workgroup (a quarter): 1792 = 28 row groups
constexpr int RGQ1 = QROWS1 / 64;      // 28
constexpr int RGE1 = E1 / 64;          // 112 row groups of the shared expert's down block
constexpr int CROWS1 = E1 / G1;        // combine rows per workgroup: 28
constexpr int GU_STEPS1 = NBX1 / 4;    // 7
constexpr int NITEM1 = 2 * NBX1;       // routed gate/up items of a workgroup: (matrix, block) of its 64 h rows
static_assert(G1 == 32 * NX1 && H1 == NX1 * QK && CROWS1 * G1 == E1, "decode-1 geometry");
static_assert((size_t) SLOTS1 * H1 <= DEC_TH && (size_t) SLOTS1 * NBH1 * E1 <= DEC_TO && BCAST1 >= 256 &&
              (size_t) BCAST1 + 16 * 8 <= DEC_TLOGITS, "tagged buffers");

// LDS layout (bytes)
constexpr int M_X = TAB_BYTES;                     // staged Q8_K of the token
constexpr int M_HR = M_X + GX1::XROW;              // staged Q8_K of the routed h block (256 B + scale)
constexpr int M_HS = M_HR + 272;                   // staged Q8_K of the shared h block
constexpr int M_HB = M_HS + 272;                   // staged Q8_K of the second routed h block (two-phase gate/up)
constexpr int SHKP1 = 2 * NBX1;                    // K-quant shared task: (matrix, block) passes of 8 rows
// shared task block terms: IQ2_XXS [7 steps][64 lanes]; K-quant [matrix][8 rows][28 blocks], then the min terms
constexpr int PRE1 = GU_STEPS1 * 64 * 4 > 2 * SHKP1 * 8 * 4 ? GU_STEPS1 * 64 * 4 : 2 * SHKP1 * 8 * 4;
constexpr int M_PRE = M_HB + 272;
constexpr int M_TERMS = M_PRE + PRE1;                  // routed block terms [matrix][block][64 rows]
constexpr int M_SCR = M_TERMS + NITEM1 * 64 * 4;   // router / norm partial sums [4] (fp64)
constexpr int M_CMB = M_SCR + 64;                  // combine: o [28 rows][9 slots]
constexpr int M_SEL = M_CMB + CROWS1 * SLOTS1 * 4; // picks [8] and weights [8]
constexpr int NCTL1 = 32;
constexpr int M_CTL = M_SEL + 2 * MAXK * 4;        // control words
constexpr int M_NRM = M_CTL + NCTL1 * 4;           // RMSNorm scale
constexpr int M_EXT = M_NRM + 16;                  // caller's picks: the distinct ids' slots [8], summed weights [8], count
constexpr int DEC1_LDS = M_EXT + 2 * MAXK * 4 + 16;
static_assert(DEC1_LDS <= 160 * 1024 && (M_X % 16) == 0 && (M_HR % 16) == 0 && (M_HS % 16) == 0, "LDS layout");
enum { C_RT = 0, C_STAGED = 1, C_SH = 2, C_READY = 3, C_HR = 4, C_HS = 5, C_CMBFAIL = 6, C_NRM = 7, C_RISSUED = 8,
       C_GUCLAIM = 9, C_DNCLAIM = 10, C_GUDONE = 11, C_SHCLAIM = 14, C_GUDONE2 = 15,
       C_HB = 16, C_LR = 17, C_LS = 18, C_LB = 19 };

typedef LK_LOCAL uint8_t * lds1_t;
typedef LK_CONST DecodeArgs D1Args;

__device__ __forceinline__ void report1(const D1Args & a, int code) {
    if (lane_id() == 0) {
        __hip_atomic_fetch_or(gptr(a.err), code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a.herr) { __hip_atomic_store(gptr(a.herr), code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); }
    }
}
__device__ __forceinline__ void st_tag1(uint64_t * p, uint32_t epoch, float v) {
    __hip_atomic_store(gptr(p), ((uint64_t) epoch << 32) | __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A tagged word for readers on the writer's own XCD: a plain 64-bit store (workgroup scope emits no write-through), which
// stays in the XCD's shared L2 where the readers' device-scope loads (ld_tag1) find it, instead of travelling to the
// device's coherence point and back. Writer and readers share an XCD by construction (roles come from XCC_ID; set-up
// checks that the dispatch is a rotation over the XCDs); were a role missing, the readers' bounded waits would time out
// and report the error -- never a stale value, since every word carries the call's epoch.
__device__ __forceinline__ void st_xcd1(uint64_t * p, uint32_t epoch, uint32_t bits) {
    __hip_atomic_store(gptr(p), ((uint64_t) epoch << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint64_t ld_tag1(const uint64_t * p) { return __hip_atomic_load(gptr(const_cast<uint64_t *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ bool tag1_ok(uint64_t w, uint32_t epoch) { return (uint32_t) (w >> 32) == epoch; }
__device__ __forceinline__ float tag1_val(uint64_t w) { return __builtin_bit_cast(float, (uint32_t) w); }
constexpr int POLL1 = 1 << 20;   // polls before a wait gives up (each poll is a memory round trip)

// LDS hand-offs between the waves of one workgroup (always co-resident)
__device__ __forceinline__ bool arrive1(LK_LOCAL unsigned * c, unsigned expected) {
    lds_visible();
    unsigned old = 0;
    if (lane_id() == 0) { old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
    old = __builtin_amdgcn_readfirstlane(old);
    return old + 1 == expected;
}
__device__ __forceinline__ unsigned wait1(LK_LOCAL unsigned * w, unsigned want_at_least) {
    for (int i = 0; i < (1 << 24); ++i) {
        const unsigned v = __builtin_amdgcn_readfirstlane(__hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (v >= want_at_least) { return v; }
        __builtin_amdgcn_s_sleep(1);
    }
    return 0;
}
__device__ __forceinline__ void flag1(LK_LOCAL unsigned * w, unsigned v) {
    lds_visible();
    if (lane_id() == 0) { __hip_atomic_store(w, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
}
// the XCD this workgroup runs on (hardware register XCC_ID)
__device__ __forceinline__ int xcc_id1() {
    unsigned x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return (int) (x & 0xFu);
}
__device__ __forceinline__ const uint8_t * uniform1(const uint8_t * p) {
    const uint64_t v = (uint64_t) p;
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) (v >> 32));
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) v);
    return (const uint8_t *) (((uint64_t) hi << 32) | (uint64_t) lo);
}

#ifdef LOKI_TRACE
constexpr int TRACE1_SLOTS = 64;
__device__ uint64_t g_trace1[1024 * W1 * TRACE1_SLOTS];
#define TRACE1(slot) do { if (lane_id() == 0) { g_trace1[(blockIdx.x * W1 + (threadIdx.x >> 6)) * TRACE1_SLOTS + (slot)] = __builtin_amdgcn_s_memrealtime(); } } while (0)
#define TRACE1V(slot, v) do { if (lane_id() == 0) { g_trace1[(blockIdx.x * W1 + (threadIdx.x >> 6)) * TRACE1_SLOTS + (slot)] = (v); } } while (0)
extern "C" hipError_t fl_trace1_copy(void * host, size_t bytes) { return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace1), bytes); }
extern "C" hipError_t fl_trace1_clear() {
    void * p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_trace1));
    return e == hipSuccess ? hipMemset(p, 0, sizeof(g_trace1)) : e;
}
#else
#define TRACE1(slot) do { } while (0)
#define TRACE1V(slot, v) do { } while (0)
#endif

// the block's input at column col: x, or (x * scale) * w under prenorm (k_rmsnorm's arithmetic)
__device__ __forceinline__ float4 in1(const D1Args & a, lds1_t lds, int col, float4 v) {
#pragma clang fp contract(off)
    if (!a.prenorm) { return v; }
    const float sc = *reinterpret_cast<const LK_LOCAL float *>(lds + M_NRM);
    v.x = v.x * sc; v.y = v.y * sc; v.z = v.z * sc; v.w = v.w * sc;
    if (a.nw) { const float4 w = gloadf4(a.nw + col); v.x = v.x * w.x; v.y = v.y * w.y; v.z = v.z * w.z; v.w = v.w * w.w; }
    return v;
}

// ---------------------------------------------------------------- 1. router (waves 0-3) and staging (waves 4-7)
// Thread (quarter w = wave, lane) owns chunk 64 w + lane (28 values) of expert b's logit: in-order fp64 chunk sum,
// tree levels 1-6 by DPP (tree64), levels 7-8 over the four waves' totals in LDS; the last wave to arrive publishes
// p = sigmoid(logit) (the selecting wave reads probabilities; the logit goes to the layer's logits output). Under prenorm the same threads first form the token's RMSNorm scale (the chunked sum-of-squares
// contract of k_rmsnorm, over the same chunks). Workgroups past the layer's experts only form the scale.
__device__ __noinline__ void router1(const D1Args & a, lds1_t lds, int wave, LK_LOCAL unsigned * ctl) {
#pragma clang fp contract(off)
    constexpr int L4 = E1 / 1024;
    const int lane = lane_id(), c = wave * 64 + lane, e = blockIdx.x;
    LK_LOCAL double * part = reinterpret_cast<LK_LOCAL double *>(lds + M_SCR);
    const bool has_e = e < a.n_exp;
    float4 wv[L4], xv[L4];
    const float * wc = a.Wr + (size_t) (has_e ? e : 0) * E1 + (size_t) c * 4 * L4;
    const float * xc = a.x + (size_t) c * 4 * L4;
    if (has_e) {
#pragma unroll
        for (int i = 0; i < L4; ++i) { wv[i] = gloadf4(wc + 4 * i); }
    }
#pragma unroll
    for (int i = 0; i < L4; ++i) { xv[i] = gloadf4(xc + 4 * i); }
    // the router's loads are in the CU's memory queue: the table copy (waves 4-7) may follow
    __builtin_amdgcn_sched_barrier(0);
    if (lane == 0) { __hip_atomic_fetch_add(reinterpret_cast<LK_LOCAL unsigned *>(lds + M_CTL) + C_RISSUED, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
    if (a.prenorm) {
        double s = 0.0;
#pragma unroll
        for (int i = 0; i < L4; ++i) {
            const float q0 = xv[i].x * xv[i].x, q1 = xv[i].y * xv[i].y, q2 = xv[i].z * xv[i].z, q3 = xv[i].w * xv[i].w;
            s += (double) q0; s += (double) q1; s += (double) q2; s += (double) q3;
        }
        const double q = tree64(s);
        if (lane == 0) { part[wave] = q; }
        if (arrive1(ctl + C_RT, 4)) {
            if (lane == 0) {
                *reinterpret_cast<LK_LOCAL float *>(lds + M_NRM) = rms_scale(part[0], part[1], part[2], part[3], E1, a.eps);
            }
            flag1(ctl + C_NRM, 1);   // the scale is ready
        }
        if (!has_e) { return; }
        if (!wait1(ctl + C_NRM, 1)) { report1(a, 64); return; }
        lds_visible();
#pragma unroll
        for (int i = 0; i < L4; ++i) { xv[i] = in1(a, lds, c * 4 * L4 + 4 * i, xv[i]); }
    }
    if (!has_e) { return; }
    double s = 0.0;
    TRACE1(11);
#pragma unroll
    for (int i = 0; i < L4; ++i) {
        s += (double) xv[i].x * (double) wv[i].x; s += (double) xv[i].y * (double) wv[i].y;
        s += (double) xv[i].z * (double) wv[i].z; s += (double) xv[i].w * (double) wv[i].w;
    }
    const double q = tree64(s);
    lds_visible();   // (prenorm) every wave has read part[] as norm sums before it is reused
    if (a.prenorm) {
        if (lane == 0) { reinterpret_cast<LK_LOCAL double *>(lds + M_SCR + 32)[wave] = q; }
    } else if (lane == 0) {
        part[wave] = q;
    }
    const unsigned want = a.prenorm ? 8u : 4u;
    if (arrive1(ctl + C_RT, want) && lane == 0) {
        const LK_LOCAL double * pp = a.prenorm ? reinterpret_cast<const LK_LOCAL double *>(lds + M_SCR + 32) : part;
        const float l = (float) ((pp[0] + pp[1]) + (pp[2] + pp[3]));
        const float pe = det_sigmoid(l);
        st_tag1(a.tlogits + e, a.epoch, pe);   // the selecting wave reads probabilities
        gptr(a.logits)[e] = l;
        if (a.probs) { gptr(a.probs)[e] = pe; }
    }
}

// ---------------------------------------------------------------- selection (one workgroup per XCD)
// Wave 0 of the selecting workgroup polls the 256 tagged probabilities, four per lane (experts 4 lane .. + 3, the
// order the selection reads them), and selects; every other wave of that workgroup stays idle until the picks are out
// (the selection is a serial chain on one wave, and work beside it slows it).
constexpr int S_P = M_TERMS;   // select_ds8's scratch (the gate/up terms' space, unused until the picks are known)
static_assert(S_P + 112 * 4 <= M_TERMS + NITEM1 * 64 * 4, "select_ds8's scratch inside the gate/up terms");

// returns whether the picks and weights in M_SEL are valid
__device__ __forceinline__ bool select1(const D1Args & a, lds1_t lds) {
#pragma clang fp contract(off)
    const int lane = lane_id();
    float bv[4];
    load_bias(a.bias, a.n_exp, bv);   // issued before the polls: its latency hides behind them
    uint64_t w[4];
    auto issue = [&]() {
#pragma unroll
        for (int j = 0; j < 4; ++j) { w[j] = 4 * lane + j < a.n_exp ? ld_tag1(a.tlogits + 4 * lane + j) : 0; }
    };
    issue();
    bool ok = false;
    for (int it = 0; it < POLL1; ++it) {
        bool v = true;
#pragma unroll
        for (int j = 0; j < 4; ++j) { v = v && (4 * lane + j >= a.n_exp || tag1_ok(w[j], a.epoch)); }
        if (__ballot(!v) == 0) { ok = true; break; }
        __builtin_amdgcn_s_sleep(1);
        issue();
    }
    TRACE1(3);
    if (!ok) { report1(a, 2); return false; }
    float pv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) { pv[j] = 4 * lane + j < a.n_exp ? tag1_val(w[j]) : 0.f; }
    int * so = (int *) (lds + M_SEL); float * wo = (float *) (lds + M_SEL + MAXK * 4);
    if (a.n_exp == 256 && a.n_group == 8 && a.topk_group == 4) {
        // DeepSeek's rule: the threshold selection, or the same rule as constants (its divisions, bounds and loop
        // counts folded) for what it leaves
        TRACE1(22);
        const bool fast = select_ds8(pv, bv, a.scale, reinterpret_cast<LK_LOCAL uint32_t *>(lds + S_P), so, wo);
        TRACE1(23);
        if (!fast) { select_token_p<false>(pv, bv, 256, 8, 4, MAXK, a.scale, nullptr, so, wo, MAXK, 0.f); }
        TRACE1V(24, fast ? 1 : 2);
    } else {
        select_token_p<false>(pv, bv, a.n_exp, a.n_group, a.topk_group, MAXK, a.scale, nullptr, so, wo, MAXK, 0.f);
    }
    return true;
}

// Q8_K of the token's 28 blocks into LDS (staged layout) by the staging waves: a pass quantises 4 consecutive blocks,
// one per 16-lane row (q8k_row16); workgroup 0 also writes the layer's xq / xd.
__device__ __forceinline__ void quant1(const D1Args & a, lds1_t lds, int w4) {
    const int lane = lane_id(), i = lane & 15;
    for (int p = w4; p < NBX1 / 4; p += NQW1) {
        const int j = 4 * p + (lane >> 4), col = j * QK + 16 * i;
        // the four loads are issued before any is used (with the input transform applied per load the compiler
        // waited for each load before issuing the next)
        float4 xv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) { xv[q] = gloadf4(a.x + col + 4 * q); }
        if (a.prenorm) {
#pragma unroll
            for (int q = 0; q < 4; ++q) { xv[q] = in1(a, lds, col + 4 * q, xv[q]); }
        }
        float xs[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) { xs[4 * q] = xv[q].x; xs[4 * q + 1] = xv[q].y; xs[4 * q + 2] = xv[q].z; xs[4 * q + 3] = xv[q].w; }
        uint32_t packed[4]; float d;
        q8k_row16(xs, packed, d);
#pragma unroll
        for (int w = 0; w < 4; ++w) { *reinterpret_cast<LK_LOCAL uint32_t *>(lds + M_X + j * GX1::XBLK + staged_word(4 * i + w)) = packed[w]; }
        if (i == 0) { reinterpret_cast<LK_LOCAL float *>(lds + M_X + NBX1 * GX1::XBLK)[j] = d; }
        if (blockIdx.x == 0) {
            *(LK_GLOBAL u32x4 *) (a.xq + (size_t) j * QK + 16 * i) = u32x4{ packed[0], packed[1], packed[2], packed[3] };
            if (i == 0) { gptr(a.xd)[j] = d; }
        }
    }
}

// ---------------------------------------------------------------- the shared expert's gate/up task: 8 h rows
// Lane 16 q + r reads row r of the task's 16 weight rows (r < 8: gate rows, r >= 8: the same h rows of up) and blocks
// 4 jj + q at step jj. Per step: the block's exact integer sum against the staged token (block_bsum_dpp), the term
// (d_w * d_x) * bsum, and the row total advanced in block order (fold_rows). h = silu(0.125 g) * (0.125 u).
struct Gu1 { const uint8_t * ql; const uint8_t * dl; };
__device__ __forceinline__ Gu1 gu1_task(const uint8_t * gm, const uint8_t * um, int hrow0, int q, int r) {
    const uint8_t * mat = r >= 8 ? um : gm;
    const int row = hrow0 + (r & 7);
    Gu1 t;
    t.ql = mat + (size_t) (row >> 6) * NBX1 * 4096 + q * 4096 + (row & 63) * 16;
    t.dl = mat + (size_t) (H1 / 64) * NBX1 * 4096 + (size_t) (row >> 6) * NBX1 * 128 + q * 128 + (row & 63) * 2;
    return t;
}
constexpr size_t GU1_QSTEP = 4 * 4096, GU1_DSTEP = 4 * 128;
__device__ __forceinline__ void gu1_issue(const Gu1 & t, int s, uint4 (&pf)[4], uint16_t & pd) {
#pragma unroll
    for (int c = 0; c < 4; ++c) { pf[c] = load_nt(t.ql + s * GU1_QSTEP + c * 1024); }
    pd = *gptr(reinterpret_cast<const uint16_t *>(t.dl + s * GU1_DSTEP));
}
// h of the task's 8 rows: lanes 0..7 hold the gate totals, lanes 8..15 the up totals (row_ror:8 brings them over)
__device__ __forceinline__ void gu1_publish(const D1Args & a, int slot, int hrow0, int q, int r, float acc) {
#pragma clang fp contract(off)
    const float other = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, acc), 0x128, 0xF, 0xF, false));
    if (q == 0 && r < 8) {
        st_xcd1(a.th + (size_t) slot * H1 + hrow0 + r, a.epoch, __builtin_bit_cast(uint32_t, det_silu(0.125f * acc) * (0.125f * other)));
    }
}

// The shared expert's task (8 h rows) split over the last 7 waves (one step each): block terms to LDS, the last wave
// folds them in block order and publishes h -- a pass's arithmetic, finished while the routing runs.
__device__ __forceinline__ void shared_gu1(const D1Args & a, lds1_t lds, int wave, int xcd, int li, uint32_t tr, int q, int r,
                                           LK_LOCAL unsigned * ctl) {
#pragma clang fp contract(off)
    const int lane = lane_id(), hrow0 = (xcd * 32 + li) * 8;
    const Gu1 t = gu1_task(uniform1(a.sh_gate), uniform1(a.sh_up), hrow0, q, r);
    LK_LOCAL float * terms = reinterpret_cast<LK_LOCAL float *>(lds + M_PRE);
    const uint8_t * xr = (const uint8_t *) (lds + M_X);
    const int s = wave - (W1 - GU_STEPS1);
    uint4 pf[4]; uint16_t pd;
    gu1_issue(t, s, pf, pd);
    const int j = s * 4 + q;
    const int bsum = block_bsum_dpp(pf, tr, xr + j * GX1::XBLK, r);
    const float dx = reinterpret_cast<const float *>(xr + NBX1 * GX1::XBLK)[j];
    terms[s * 64 + lane] = (h2f(pd) * dx) * (float) bsum;
    if (!arrive1(ctl + C_SH, GU_STEPS1)) { return; }
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < GU_STEPS1; ++k) { acc = fold_rows(acc, terms[k * 64 + lane]); }
    gu1_publish(a, 8, hrow0, q, r, acc);
}

// ---------------------------------------------------------------- K-quant matrices (ggml's block layout, in place)
// The token and the h blocks are staged for the IQ2_XXS lookups (staged_word): values 8 w .. 8 w + 7 of a block sit
// contiguously at (w % 4) * 64 + (w / 4) * 8, so a K-quant slice's 8-byte runs are read from there.
__device__ __forceinline__ int staged8(int v) { return ((v >> 3) & 3) * 64 + (v >> 5) * 8; }
// load_x (kquant_device.h) on a staged block: the same words and per-piece sums
template <int F> __device__ __forceinline__ void load_x_st(const LK_LOCAL int8_t * xb, int q, XChunk & x) {
    const int ones = 0x01010101;
    if constexpr (F == KF_Q5K) {
        const int jj = q >> 1, hf = q & 1;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int v0 = 64 * jj + 32 * h + 16 * hf;
            const uint2 a0 = kx8(xb + staged8(v0)), a1 = kx8(xb + staged8(v0 + 8));
            x.x[4 * h] = a0.x; x.x[4 * h + 1] = a0.y; x.x[4 * h + 2] = a1.x; x.x[4 * h + 3] = a1.y;
            int sm = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) { sm = __builtin_amdgcn_sdot4((int) x.x[4 * h + i], ones, sm, false); }
            x.bx[h] = sm;
        }
        x.bx[2] = x.bx[3] = 0;
    } else {
        const int n = q >> 2, jq = q & 3;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint2 v = kx8(xb + staged8(128 * n + 32 * s + 8 * jq));
            x.x[2 * s] = v.x; x.x[2 * s + 1] = v.y;
            x.bx[s] = __builtin_amdgcn_sdot4((int) v.y, ones, __builtin_amdgcn_sdot4((int) v.x, ones, 0, false), false);
        }
    }
    x_starts<F>(x);
}
// a buffer resource over a matrix of `bytes` (wave-uniform base); lane offsets in vb, the row offset in so
__device__ __forceinline__ Src src1(const uint8_t * mat, uint64_t bytes, uint32_t vb) {
    Src s;
    s.rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(uniform1(mat)), (short) 0,
                                             (int) (bytes < 0x7fffffffull ? bytes : 0x7fffffffull), 0x00020000);
    s.vb = vb; s.so = 0;
    return s;
}
// a slice's exact integer block sums (red8 over the 8 lanes of its row) and the fp32 block term of the K-quant
// mat-vec (kquant.hip), valid in the row's first lane: Q2_K (d8 d) isum - (d8 dmin) summ, Q3_K / Q6_K (d d8) isum,
// Q5_K (d d8) isum with the min term (dmin d8) summ beside it
template <int F> __device__ __forceinline__ float kq_term1(const Raw<F> & raw, const XChunk & xc, int c, float & tmin) {
#pragma clang fp contract(off)
    Chunk ck; decode<F>(raw, c, ck);
    int is, sm;
    chunk_dot<F>(ck, xc, is, sm);
    is = red8(is);
    const float d8 = xc.d8;
    tmin = 0.f;
    if constexpr (F == KF_Q2K) { sm = red8(sm); return (d8 * ck.d) * (float) is - (d8 * ck.dmin) * (float) sm; }
    else if constexpr (F == KF_Q5K) { sm = red8(sm); tmin = (ck.dmin * d8) * (float) sm; return (ck.d * d8) * (float) is; }
    else { return (ck.d * d8) * (float) is; }
}

// The shared expert's gate/up task in Q5_K (h rows 8 t .. 8 t + 7, t = 32 x + i): 56 passes (matrix, block), each 8
// rows (lane = row r8, slice c), claimed from an LDS counter by the waves free before the picks arrive, each keeping
// DS1 passes' bytes in flight. Block terms to LDS; the wave that completes the 56th pass folds each row's terms in block
// order (the K-quant mat-vec's order: acc += t, accm -= t_min, acc_m + acc) and publishes h = silu(g) * u.
constexpr int QR5 = NBX1 * kbytes<KF_Q5K>();   // Q5_K row bytes at K = 7168
constexpr int DS1 = 3;
__device__ __forceinline__ bool shared_gu1_kq(const D1Args & a, lds1_t lds, int xcd, int li, LK_LOCAL unsigned * ctl) {
#pragma clang fp contract(off)
    const int lane = lane_id(), r8 = lane >> 3, c = lane & 7, hrow0 = (xcd * 32 + li) * 8;
    LK_LOCAL float * ts = reinterpret_cast<LK_LOCAL float *>(lds + M_PRE);   // [matrix][row][block]
    LK_LOCAL float * tm = ts + 2 * 8 * NBX1;
    const LK_LOCAL int8_t * xs = reinterpret_cast<const LK_LOCAL int8_t *>(lds + M_X);
    const LK_LOCAL float * dx = reinterpret_cast<const LK_LOCAL float *>(lds + M_X + NBX1 * GX1::XBLK);
    Raw<KF_Q5K> rg[DS1];
    int sp[DS1];   // the pass each slot holds (>= 56: empty); claims rise, so the slots hold passes in order
    // the resource is formed per pass from the wave-uniform matrix pointer (scalar registers; a resource picked from
    // an array would be taken as per-lane and every load would loop over its lanes' resources)
    auto refill = [&](int k) {
        unsigned cl = 0;
        if (lane == 0) { cl = __hip_atomic_fetch_add(ctl + C_SHCLAIM, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
        const int p = (int) __builtin_amdgcn_readfirstlane(cl);
        sp[k] = p;
        if (p < SHKP1) {
            Src s = src1((p & 1) ? a.sh_up : a.sh_gate, (uint64_t) H1 * QR5, (uint32_t) r8 * QR5 + (uint32_t) (p >> 1) * kbytes<KF_Q5K>());
            s.so = (uint32_t) hrow0 * QR5;
            load_raw<KF_Q5K>(s, c, rg[k]);
        }
    };
    auto run = [&](const Raw<KF_Q5K> & r, int p) {
        const int m = p & 1, j = p >> 1;
        XChunk xc;
        load_x_st<KF_Q5K>(xs + j * GX1::XBLK, c, xc);
        xc.d8 = dx[j];
        float tmin;
        const float t = kq_term1<KF_Q5K>(r, xc, c, tmin);
        if (c == 0) { ts[(m * 8 + r8) * NBX1 + j] = t; tm[(m * 8 + r8) * NBX1 + j] = tmin; }
        if (arrive1(ctl + C_SH, SHKP1)) {
            float v = 0.f;
            if (lane < 16) {
                const LK_LOCAL float * tp = ts + lane * NBX1, * mp = tm + lane * NBX1;   // lanes 0-7: gate rows, 8-15: up
                float acc = 0.f, accm = 0.f;
                for (int k = 0; k < NBX1; ++k) { acc = acc + tp[k]; accm = accm - mp[k]; }
                v = accm + acc;
            }
            const float u = __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x128, 0xF, 0xF, false));
            if (lane < 8) { st_xcd1(a.th + (size_t) 8 * H1 + hrow0 + lane, a.epoch, __builtin_bit_cast(uint32_t, det_silu(v) * u)); }
        }
    };
#pragma unroll
    for (int k = 0; k < DS1; ++k) { refill(k); }
    if (!wait1(ctl + C_STAGED, NQW1)) { report1(a, 8); return false; }   // the token's Q8_K
    lds_visible();
    bool more = sp[0] < SHKP1;
    while (more) {
#pragma unroll
        for (int k = 0; k < DS1; ++k) {
            if (more && sp[k] >= SHKP1) { more = false; }
            if (more) { run(rg[k], sp[k]); refill(k); }
        }
    }
    return true;
}

// The workgroup's routed gate/up: h rows hrow0 .. hrow0 + 63 (one 64-row group of both matrices) as 56 items, item c =
// matrix c % 2 (gate, up) at block c / 2, claimed in order by all waves from an LDS counter; a wave claims its next
// item when it has used the last. Lane l owns row hrow0 + l of the item's matrix, so each of its 16-byte loads is one contiguous 1 KB
// per wave (the tiled layout's chunk of 64 rows) and the scales one 128-byte line; every lane uses the same staged
// token block, whose words come by DPP (block_bsum_dpp). The block terms (d_w * d_x) * bsum go to LDS; the wave that
// completes the 56th item folds each row's 28 terms in block order (ggml's sumf, the order of every other path) and
// publishes h = silu(0.125 g) * (0.125 u) for the 64 rows.
struct GuItem { uint4 w[4]; uint16_t d; int c; };
__device__ __forceinline__ void gate_up1(const D1Args & a, lds1_t lds, LK_LOCAL unsigned * ctl, const uint8_t * gm,
                                         const uint8_t * um, int slot, int hrow0, uint32_t tr, int r) {
#pragma clang fp contract(off)
    const int lane = lane_id(), g64 = hrow0 >> 6;
    LK_LOCAL float * terms = reinterpret_cast<LK_LOCAL float *>(lds + M_TERMS);   // [matrix][block][64 rows]
    const uint8_t * xr = (const uint8_t *) (lds + M_X);
    auto claim = [&](GuItem & it) {
        unsigned c = 0;
        if (lane == 0) { c = __hip_atomic_fetch_add(ctl + C_GUCLAIM, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
        it.c = (int) __builtin_amdgcn_readfirstlane(c);
        if (it.c >= NITEM1) { return; }
        const int j = it.c >> 1;
        const uint8_t * mat = uniform1((it.c & 1) ? um : gm);
        // the scale first: memory waits count loads in issue order
        it.d = *gptr(reinterpret_cast<const uint16_t *>(mat + (size_t) (H1 / 64) * NBX1 * 4096 + ((size_t) g64 * NBX1 + j) * 128 + lane * 2));
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t * qb = mat + ((size_t) g64 * NBX1 + j) * 4096 + lane * 16;
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) { it.w[c4] = load_nt(qb + c4 * 1024); }
        __builtin_amdgcn_sched_barrier(0);
    };
    // false past the end (claims rise across the workgroup, so every later item of this wave is past the end too)
    auto run = [&](const GuItem & it) -> bool {
        if (it.c >= NITEM1) { return false; }
        const int j = it.c >> 1;
        const int bsum = block_bsum_dpp(it.w, tr, xr + j * GX1::XBLK, r);
        const float dx = reinterpret_cast<const float *>(xr + NBX1 * GX1::XBLK)[j];
        terms[it.c * 64 + lane] = (h2f(it.d) * dx) * (float) bsum;   // [matrix][block] = item c
        if (arrive1(ctl + C_GUDONE, NITEM1)) {
            TRACE1(12);
            float g = 0.f, u = 0.f;
#pragma unroll 4
            for (int k = 0; k < NBX1; ++k) { g = g + terms[(2 * k) * 64 + lane]; u = u + terms[(2 * k + 1) * 64 + lane]; }
            st_xcd1(a.th + (size_t) slot * H1 + hrow0 + lane, a.epoch, __builtin_bit_cast(uint32_t, det_silu(0.125f * g) * (0.125f * u)));
            TRACE1(13);
        }
        return true;
    };
    // one item in flight per wave: with 16 waves per CU, deeper look-ahead measured slower (more bytes in flight per
    // CU than the memory path serves without queueing). The four waves of a SIMD run at distinct priorities, so when
    // their items land together they compute one after another and request their next items at staggered times
    // instead of all at once after the last of them (measured -0.2 to -0.4 us per launch)
    switch ((threadIdx.x >> 8) & 3) {
        case 0: __builtin_amdgcn_s_setprio(0); break;
        case 1: __builtin_amdgcn_s_setprio(1); break;
        case 2: __builtin_amdgcn_s_setprio(2); break;
        default: __builtin_amdgcn_s_setprio(3); break;
    }
    GuItem it;
    claim(it);
    while (run(it)) { claim(it); }
    __builtin_amdgcn_s_setprio(0);
}

// The routed gate/up of an all-IQ2_XXS layer in two phases. Phase p of role (x, i) computes the 32 h rows
// 256 kb_p + 32 (i % 8) .. + 31 of expert sel[x], kb_0 = i / 8, kb_1 = 4 + i / 8: the eight workgroups i / 8 = const
// of an XCD complete h block kb_0 in phase 0 and kb_1 in phase 1. A phase is 28 items (matrix c % 2, blocks 2 (c / 2)
// and 2 (c / 2) + 1: lanes 0-31 the first, lanes 32-63 the second, lane l row l % 32), each one 512-byte run of 32 rows
// per chunk and block, claimed in order by all waves (phase 0's first). The wave completing a phase's 28th item folds
// each row's 28 terms per matrix in block order (the gate rows in lanes 0-31, the up rows in lanes 32-63) and publishes
// that phase's 32 h values. Block kb_0 is complete while phase 1 streams, so the down of K-block kb_0 runs while block
// kb_1's hand-off completes (the single-phase order leaves every CU idle for that hand-off).
constexpr int NIT2 = NBX1;               // items per phase: 2 matrices x 14 block pairs
constexpr int TERMS2 = 2 * NBX1 * 32;    // a phase's terms: [matrix][block][32 rows]
static_assert(2 * TERMS2 * 4 <= NITEM1 * 64 * 4, "both phases' terms in the gate/up terms' space");
__device__ __forceinline__ int hrow2(int li, int ph) { return ((ph ? 4 : 0) + (li >> 3)) * QK + 32 * (li & 7); }
__device__ __forceinline__ void gate_up2(const D1Args & a, lds1_t lds, LK_LOCAL unsigned * ctl, const uint8_t * gm,
                                         const uint8_t * um, int slot, int li, uint32_t tr, int r) {
#pragma clang fp contract(off)
    const int lane = lane_id(), hl = lane >> 5, rr = lane & 31;
    LK_LOCAL float * terms = reinterpret_cast<LK_LOCAL float *>(lds + M_TERMS);   // [phase][matrix][block][32 rows]
    const uint8_t * xr = (const uint8_t *) (lds + M_X);
    constexpr size_t DREG = (size_t) (H1 / 64) * NBX1 * 4096;
    auto claim = [&](GuItem & it) {
        unsigned c = 0;
        if (lane == 0) { c = __hip_atomic_fetch_add(ctl + C_GUCLAIM, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
        it.c = (int) __builtin_amdgcn_readfirstlane(c);
        if (it.c >= 2 * NIT2) { return; }
        const int ph = it.c >= NIT2 ? 1 : 0, ci = it.c - ph * NIT2, j = 2 * (ci >> 1) + hl;
        const int h0 = hrow2(li, ph), g64 = h0 >> 6, row = (h0 & 63) + rr;   // a 32-row half of one 64-row group
        const uint8_t * mat = uniform1((ci & 1) ? um : gm);
        // the scale first: memory waits count loads in issue order
        it.d = *gptr(reinterpret_cast<const uint16_t *>(mat + DREG + ((size_t) g64 * NBX1 + j) * 128 + row * 2));
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t * qb = mat + ((size_t) g64 * NBX1 + j) * 4096 + row * 16;
#pragma unroll
        for (int c4 = 0; c4 < 4; ++c4) { it.w[c4] = load_nt(qb + c4 * 1024); }
        __builtin_amdgcn_sched_barrier(0);
    };
    auto run = [&](const GuItem & it) -> bool {
        if (it.c >= 2 * NIT2) { return false; }
        const int ph = it.c >= NIT2 ? 1 : 0, ci = it.c - ph * NIT2, j = 2 * (ci >> 1) + hl, m = ci & 1;
        const int bsum = block_bsum_dpp(it.w, tr, xr + j * GX1::XBLK, r);   // each 16-lane row reads its own block
        const float dx = reinterpret_cast<const float *>(xr + NBX1 * GX1::XBLK)[j];
        terms[ph * TERMS2 + (m * NBX1 + j) * 32 + rr] = (h2f(it.d) * dx) * (float) bsum;
        if (arrive1(ctl + (ph ? C_GUDONE2 : C_GUDONE), NIT2)) {
            TRACE1(ph ? 13 : 12);
            const LK_LOCAL float * tp = terms + ph * TERMS2 + hl * NBX1 * 32 + rr;
            float v = 0.f;
#pragma unroll 4
            for (int k = 0; k < NBX1; ++k) { v = v + tp[k * 32]; }
            const float u = __builtin_bit_cast(float, lanes_32_63(__builtin_bit_cast(uint32_t, v)));   // lanes 0-31: the up sums
            if (hl == 0) {
                st_xcd1(a.th + (size_t) slot * H1 + hrow2(li, ph) + rr, a.epoch, __builtin_bit_cast(uint32_t, det_silu(0.125f * v) * (0.125f * u)));
            }
        }
        return true;
    };
    switch ((threadIdx.x >> 8) & 3) {   // staggered priorities, as in gate_up1
        case 0: __builtin_amdgcn_s_setprio(0); break;
        case 1: __builtin_amdgcn_s_setprio(1); break;
        case 2: __builtin_amdgcn_s_setprio(2); break;
        default: __builtin_amdgcn_s_setprio(3); break;
    }
    GuItem it;
    claim(it);
    while (run(it)) { claim(it); }
    __builtin_amdgcn_s_setprio(0);
}

// ---------------------------------------------------------------- down: one 256-weight block per row
// A unit is one 64-row group of one down matrix at one K-block: lane l owns row l (4 chunks + d); every lane's block
// product uses the same staged h block, so the activations come by DPP from the 16 lanes that hold them.
struct Dn1 { uint4 w[4]; uint16_t d; };
__device__ __forceinline__ void dn1_issue(const uint8_t * mat, int g64, int kb, Dn1 & u) {
    const int lane = lane_id();
    const uint8_t * q = mat + ((size_t) g64 * NBH1 + kb) * 4096 + lane * 16;
#pragma unroll
    for (int c = 0; c < 4; ++c) { u.w[c] = load_nt(q + c * 1024); }
    u.d = *gptr(reinterpret_cast<const uint16_t *>(mat + (size_t) (E1 / 64) * NBH1 * 4096 + ((size_t) g64 * NBH1 + kb) * 128 + lane * 2));
}
// polls the 256 tagged h values of one block and stages their Q8_K (one wave); false on timeout
__device__ __forceinline__ bool stage_h1(const D1Args & a, const uint64_t * src, LK_LOCAL uint8_t * dst) {
    const int lane = lane_id();
    uint64_t w[4];
    auto issue = [&]() {
#pragma unroll
        for (int k = 0; k < 4; ++k) { w[k] = ld_tag1(src + 4 * lane + k); }
    };
    issue();
    int it = 0;
    for (; it < POLL1; ++it) {
        bool v = true;
#pragma unroll
        for (int k = 0; k < 4; ++k) { v = v && tag1_ok(w[k], a.epoch); }
        if (__ballot(!v) == 0) { break; }
        __builtin_amdgcn_s_sleep(1);
        issue();
    }
    if (it == POLL1) { return false; }
    const float xs[4] = { tag1_val(w[0]), tag1_val(w[1]), tag1_val(w[2]), tag1_val(w[3]) };
    float dq; const uint32_t packed = q8k_lane(xs, dq);
    *reinterpret_cast<LK_LOCAL uint32_t *>(dst + staged_word(lane)) = packed;
    if (lane == 0) { *reinterpret_cast<LK_LOCAL float *>(dst + QK) = dq; }
    return true;
}

// the same for two blocks polled together (one memory round trip per poll for both); false on timeout
__device__ __forceinline__ bool stage_h2(const D1Args & a, const uint64_t * s0, LK_LOCAL uint8_t * d0, const uint64_t * s1,
                                         LK_LOCAL uint8_t * d1) {
    const int lane = lane_id();
    uint64_t w[8];
    auto issue = [&]() {
#pragma unroll
        for (int k = 0; k < 4; ++k) { w[k] = ld_tag1(s0 + 4 * lane + k); w[4 + k] = ld_tag1(s1 + 4 * lane + k); }
    };
    issue();
    int it = 0;
    for (; it < POLL1; ++it) {
        bool v = true;
#pragma unroll
        for (int k = 0; k < 8; ++k) { v = v && tag1_ok(w[k], a.epoch); }
        if (__ballot(!v) == 0) { break; }
        __builtin_amdgcn_s_sleep(1);
        issue();
    }
    if (it == POLL1) { return false; }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const float xs[4] = { tag1_val(w[4 * b]), tag1_val(w[4 * b + 1]), tag1_val(w[4 * b + 2]), tag1_val(w[4 * b + 3]) };
        float dq; const uint32_t packed = q8k_lane(xs, dq);
        LK_LOCAL uint8_t * dst = b ? d1 : d0;
        *reinterpret_cast<LK_LOCAL uint32_t *>(dst + staged_word(lane)) = packed;
        if (lane == 0) { *reinterpret_cast<LK_LOCAL float *>(dst + QK) = dq; }
    }
    return true;
}

// K-quant down units (one 64-row group at one K-block): 8 passes of 8 rows (lane = row r8, slice c), each row's block
// term published as a tagged word as the IQ2_XXS units publish theirs. A pass's arithmetic is short against the load
// latency, so a wave keeps DR1 passes' bytes in flight, in a ring of raw slices refilled as each pass is used. The
// wave's claimed units below the stream's end run in order; the next unit is claimed when the look-ahead reaches it.
constexpr int DR1 = 4;
template <int F> struct DnRing1 {
    Raw<F> r[DR1];
    int su[DR1], sp[DR1];   // the (unit, pass) each slot holds; su at or past the end: empty
    int ul, pl;             // the next pass to issue
};
template <int F, class G64, class Claim>
__device__ __forceinline__ void dn_issue1(DnRing1<F> & g, int k, int uend, const Src & base, G64 g64_of, Claim claim) {
    constexpr uint32_t RB = NBH1 * kbytes<F>();   // row bytes at K = 2048
    g.su[k] = g.ul; g.sp[k] = g.pl;
    if (g.ul < uend) {
        Src s = base;
        s.so = (uint32_t) (g64_of(g.ul) * 64 + 8 * g.pl) * RB;
        load_raw<F>(s, lane_id() & 7, g.r[k]);
        if (++g.pl == 8) { g.ul = claim(); g.pl = 0; }
    }
}
// fills the ring from unit u (claimed) on
template <int F, class G64, class Claim>
__device__ __forceinline__ void dn_prime1(DnRing1<F> & g, int u, int uend, const Src & base, G64 g64_of, Claim claim) {
    g.ul = u; g.pl = 0;
#pragma unroll
    for (int k = 0; k < DR1; ++k) { dn_issue1<F>(g, k, uend, base, g64_of, claim); }
}
// runs the ring's passes against the staged h block hb; returns the first claim at or past uend
template <int F, class G64, class Claim>
__device__ __forceinline__ int dn_run1(const D1Args & a, DnRing1<F> & g, int uend, const Src & base, const LK_LOCAL int8_t * hb,
                                       float d8, int slot, int blk, G64 g64_of, Claim claim) {
#pragma clang fp contract(off)
    const int lane = lane_id(), r8 = lane >> 3, c = lane & 7;
    XChunk xc;
    load_x_st<F>(hb, c, xc);
    xc.d8 = d8;
    bool more = g.su[0] < uend;
    while (more) {
#pragma unroll
        for (int k = 0; k < DR1; ++k) {
            if (more && g.su[k] >= uend) { more = false; }   // the ring holds consecutive passes: the rest are empty too
            if (more) {
                float tmin;
                const float t = kq_term1<F>(g.r[k], xc, c, tmin);
                if (c == 0) { st_tag1(a.to + ((size_t) slot * NBH1 + blk) * E1 + (size_t) g64_of(g.su[k]) * 64 + 8 * g.sp[k] + r8, a.epoch, t); }
                dn_issue1<F>(g, k, uend, base, g64_of, claim);
            }
        }
    }
    return g.ul;
}

// ---------------------------------------------------------------- 4. combine
// thread (row i, slot s) of the first 252: the 8 tagged block terms of its row and slot, folded in block order,
// * 0.125 for an IQ2_XXS matrix (its grid scale; the K-quant terms carry their scales); then thread i < 28 forms
// y = sum_k w_k o_k (k order) + o_shared (+ the residual)
template <bool KQ> __device__ __forceinline__ bool combine1(const D1Args & a, lds1_t lds) {
#pragma clang fp contract(off)
    LK_LOCAL float * cmb = reinterpret_cast<LK_LOCAL float *>(lds + M_CMB);
    const LK_LOCAL float * wts = reinterpret_cast<const LK_LOCAL float *>(lds + M_SEL + MAXK * 4);
    const int t = threadIdx.x, row0 = blockIdx.x * CROWS1;
    bool ok = true;
    if (t < CROWS1 * SLOTS1) {
        const int i = t / SLOTS1, s = t % SLOTS1, row = row0 + i;
        uint64_t w[NBH1];
        auto issue = [&]() {
#pragma unroll
            for (int kb = 0; kb < NBH1; ++kb) { w[kb] = ld_tag1(a.to + ((size_t) s * NBH1 + kb) * E1 + row); }
        };
        issue();
        int it = 0;
        for (; it < POLL1; ++it) {
            bool v = true;
#pragma unroll
            for (int kb = 0; kb < NBH1; ++kb) { v = v && tag1_ok(w[kb], a.epoch); }
            if (v) { break; }
            __builtin_amdgcn_s_sleep(1);
            issue();
        }
        ok = it < POLL1;
        TRACE1(14);
        if (!ok) { __hip_atomic_store(reinterpret_cast<LK_LOCAL unsigned *>(lds + M_CTL) + C_CMBFAIL, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
        float o = 0.f;
#pragma unroll
        for (int kb = 0; kb < NBH1; ++kb) { o = o + tag1_val(w[kb]); }
        const float ov = KQ ? o : 0.125f * o;
        cmb[i * SLOTS1 + s] = ov;
        if (a.o_out && s < MAXK) { gptr(a.o_out)[(size_t) s * E1 + row] = ov; }
    }
    __syncthreads();
    if (t < CROWS1) {
        const int row = row0 + t;
        if (a.ext_sel || a.spec_combine) {   // fl_moe's combine: the distinct ids ascending, moe = their weighted sum, y = (moe + shared) + resid
            const LK_LOCAL int * xs = reinterpret_cast<const LK_LOCAL int *>(lds + M_EXT);
            const LK_LOCAL float * xw = reinterpret_cast<const LK_LOCAL float *>(lds + M_EXT + MAXK * 4);
            const int cnt = reinterpret_cast<const LK_LOCAL int *>(lds + M_EXT + 2 * MAXK * 4)[0];
            float v = 0.f;
            for (int q = 0; q < cnt; ++q) { v = v + xw[q] * cmb[t * SLOTS1 + xs[q]]; }
            gptr(a.moe_out)[row] = v;
            gptr(a.y)[row] = (v + cmb[t * SLOTS1 + MAXK]) + gptr(a.resid)[row];
        } else {
            float mv = cmb[t * SLOTS1] * wts[0];
#pragma unroll
            for (int k = 1; k < MAXK; ++k) { mv = mv + cmb[t * SLOTS1 + k] * wts[k]; }
            float yv = mv + cmb[t * SLOTS1 + MAXK];
            if (a.resid) { yv = yv + gptr(a.resid)[row]; }
            gptr(a.y)[row] = yv;
        }
    }
    (void) ok;
    return true;
}

// the layer's routing outputs from the picks (workgroup 0): for one token the eight picks are distinct experts, so the
// dispatch is their sort by expert id (ties impossible): perm / inv / act from the ranks, counts / offsets by expert
__device__ __noinline__ void routing1(const D1Args & a, lds1_t lds) {
    const LK_LOCAL int * sel = reinterpret_cast<const LK_LOCAL int *>(lds + M_SEL);
    const LK_LOCAL float * wts = reinterpret_cast<const LK_LOCAL float *>(lds + M_SEL + MAXK * 4);
    const int lane = lane_id();
    if (lane < MAXK) {
        const int e = sel[lane];
        int rank = 0;
#pragma unroll
        for (int j = 0; j < MAXK; ++j) { rank += sel[j] < e ? 1 : 0; }
        gptr(a.sel)[lane] = e; gptr(a.wts)[lane] = wts[lane];
        gptr(a.perm)[rank] = lane; gptr(a.inv)[lane] = rank; gptr(a.act)[rank] = e;
    }
    if (lane == 0) { *gptr(a.nact) = MAXK; }
    for (int x = lane; x <= a.n_exp; x += 64) {
        int lt = 0, eq = 0;
#pragma unroll
        for (int j = 0; j < MAXK; ++j) { const int ej = sel[j]; lt += ej < x ? 1 : 0; eq += ej == x ? 1 : 0; }
        gptr(a.offsets)[x] = lt;
        if (x < a.n_exp) { gptr(a.counts)[x] = eq; }
    }
}

// fl_moe's combine list from the picks and weights in M_SEL (lane 0): the distinct ids in ascending order, each with
// its weights summed in k order and its first slot; zero sums are dropped, as fl_moe does
__device__ __forceinline__ void ext_list1(lds1_t lds) {
    if (lane_id() != 0) { return; }
    const LK_LOCAL int * so = reinterpret_cast<const LK_LOCAL int *>(lds + M_SEL);
    const LK_LOCAL float * wo = reinterpret_cast<const LK_LOCAL float *>(lds + M_SEL + MAXK * 4);
    LK_LOCAL int * xs = reinterpret_cast<LK_LOCAL int *>(lds + M_EXT);
    LK_LOCAL float * xw = reinterpret_cast<LK_LOCAL float *>(lds + M_EXT + MAXK * 4);
    int prev = -1, cnt = 0;
    for (int it = 0; it < MAXK; ++it) {
        int m = 0x7fffffff;
        for (int k = 0; k < MAXK; ++k) { if (so[k] > prev && so[k] < m) { m = so[k]; } }
        if (m == 0x7fffffff) { break; }
        float wt = 0.f; int kf = -1;
        for (int k = 0; k < MAXK; ++k) { if (so[k] == m) { wt += wo[k]; if (kf < 0) { kf = k; } } }
        prev = m;
        if (wt == 0.f) { continue; }
        xs[cnt] = kf; xw[cnt] = wt; ++cnt;
    }
    reinterpret_cast<LK_LOCAL int *>(lds + M_EXT + 2 * MAXK * 4)[0] = cnt;
}

// ---------------------------------------------------------------- the kernel
// FD: 0 (every matrix IQ2_XXS), or the routed down's K-quant (the shared expert then Q5_K / Q5_K / Q6_K)
template <int FD>
__global__ void __launch_bounds__(NT1, 1) k_moe_decode1(const DecodeArgs args) {
#pragma clang fp contract(off)
    (void) sizeof(args);   // read in place in the kernarg segment (scalar loads), as the general decode kernel does
    const D1Args & a = *(const D1Args *) __builtin_amdgcn_kernarg_segment_ptr();
    extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds1[];
    const lds1_t lds = (lds1_t) dyn_lds1;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
    // roles by the XCD the workgroup runs on: the hardware dispatches workgroups round-robin over the XCDs from
    // wherever the previous dispatch stopped, so XCD (r + b) % 8 runs workgroup b; under any such rotation
    // (XCC_ID, b / 8) takes each of the 8 x 32 roles once
    const int xcd = xcc_id1(), li = blockIdx.x / NX1;
    LK_LOCAL unsigned * ctl = reinterpret_cast<LK_LOCAL unsigned *>(lds + M_CTL);
    const int q = lane >> 4, r = lane & 15;
    const uint32_t tr = tab_word_grid(lds_addr(dyn_lds1), lane);
    TRACE1(0);
    TRACE1V(63, 100 + xcd);
    if (a.tstamp && blockIdx.x == 0 && threadIdx.x == 0) {
        __hip_atomic_store(gptr(a.tstamp), (uint64_t) __builtin_amdgcn_s_memrealtime(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    if (lds_addr(dyn_lds1) & 0xFFFFu) { report1(a, 4); return; }   // table addressing needs a 64 KB aligned base
    if (threadIdx.x < NCTL1) { ctl[threadIdx.x] = 0; }
    __syncthreads();

    // 1. router on waves 0-3; table copy and token quantisation on the others; the shared gate/up task on the last 7
    if (wave < 4) {
        if (!a.ext_sel) { router1(a, lds, wave, ctl); }   // with the caller's picks there is no routing
        TRACE1(1);
    } else {
        if (!a.ext_sel) { (void) wait1(ctl + C_RISSUED, 4); }   // the router's weight and token loads go first (the critical path)
        tables_fill(reinterpret_cast<const uint8_t *>(a.tab), lds, threadIdx.x - 256, NQW1 * 64);
        if (a.prenorm && !wait1(ctl + C_NRM, 1)) { report1(a, 64); return; }
        quant1(a, lds, wave - 4);
        arrive1(ctl + C_STAGED, NQW1);   // (its LDS writes are done: arrive1 waits for them)
        TRACE1(1);
    }
    if (li == 0 && wave >= 4) {
        // the selecting workgroups keep their CU quiet until the picks are out: the selection is a serial chain of
        // cross-lane steps on one wave, and work of the other waves beside it (the shared expert's task) slows it by
        // about half; their shared task runs after the picks, beside the routed gate/up
        const unsigned rd = wait1(ctl + C_READY, 1);
        if (rd != 1) { if (rd == 0) { report1(a, 8); } return; }
    }
    if constexpr (FD == 0) {
        if (wave >= W1 - GU_STEPS1) {   // the shared expert's gate/up task, one step per wave
            if (!wait1(ctl + C_STAGED, NQW1)) { report1(a, 8); return; }
            lds_visible();
            shared_gu1(a, lds, wave, xcd, li, tr, q, r, ctl);
            TRACE1(2);
        }
    } else if (wave >= (li == 0 ? 4 : 1)) {
        // in Q5_K: every wave but the one polling the picks (wave 0), after its router part; in the selecting
        // workgroups not the router waves, which form the probabilities and select
        if (!shared_gu1_kq(a, lds, xcd, li, ctl)) { return; }
        TRACE1(2);
    }

    // 2. selection, two levels: on each XCD one workgroup (li = 0) selects (select1: its wave 0 polls the probabilities
    //    and selects) and broadcasts the picks and weights through its XCD's L2 (st_xcd1); the XCD's other workgroups
    //    poll that one line. Only 8 workgroups poll the device-wide probabilities, which every router workgroup is
    //    writing at the same time.
    if (a.ext_sel) {
        // the caller's picks: pick k is slot k (on XCD k); lane 0 also lists the distinct ids in ascending order, each
        // with its weights summed in k order and its first slot, for the combine (zero sums are dropped, as fl_moe does)
        if (wave == 0) {
            LK_LOCAL int * so = reinterpret_cast<LK_LOCAL int *>(lds + M_SEL);
            LK_LOCAL float * wo = reinterpret_cast<LK_LOCAL float *>(lds + M_SEL + MAXK * 4);
            if (lane < MAXK) { so[lane] = gptr(a.ext_sel)[lane]; wo[lane] = gptr(a.ext_w)[lane]; }
            lds_visible();
            ext_list1(lds);
            flag1(ctl + C_READY, 1u);
        }
    } else if (li == 0 && wave == 0) {
        __builtin_amdgcn_s_setprio(3);
        const bool ok = select1(a, lds);
        __builtin_amdgcn_s_setprio(0);
        {
            lds_visible();
            TRACE1(21);
            if (ok && lane < 16) {
                st_xcd1(a.tlogits + BCAST1 + xcd * 16 + lane, a.epoch, reinterpret_cast<const LK_LOCAL uint32_t *>(lds + M_SEL)[lane]);
            }
            flag1(ctl + C_READY, ok ? 1u : 2u);
            TRACE1(4);
            if (a.spec_combine && xcd == 0 && a.hsel) {   // the picks and weights for fl_fetch, then its done word
                if (lane < 16) { gptr(a.hsel)[lane] = ok ? reinterpret_cast<const LK_LOCAL int *>(lds + M_SEL)[lane] : (lane < MAXK ? -1 : 0); }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");   // system scope: the picks before the word
                if (lane == 0) { __hip_atomic_store(gptr(a.hdone), a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); }
            }
        }
    } else if (li != 0 && wave == 0) {
        const uint64_t * bc = a.tlogits + BCAST1 + xcd * 16;   // [8 picks, 8 weights] of this XCD
        uint64_t w = lane < 16 ? ld_tag1(bc + lane) : 0;
        bool ok = false;
        for (int it = 0; it < POLL1; ++it) {
            if (__ballot(lane < 16 && !tag1_ok(w, a.epoch)) == 0) { ok = true; break; }
            __builtin_amdgcn_s_sleep(1);
            if (lane < 16) { w = ld_tag1(bc + lane); }
        }
        TRACE1(3);
        if (ok && lane < 16) { reinterpret_cast<LK_LOCAL uint32_t *>(lds + M_SEL)[lane] = (uint32_t) w; }
        if (!ok) { report1(a, 2); }
        flag1(ctl + C_READY, ok ? 1u : 2u);
        TRACE1(4);
    }
    const unsigned ready = wait1(ctl + C_READY, 1);
    if (ready != 1) { if (ready == 0) { report1(a, 8); } return; }
    lds_visible();
    if (a.spec_combine && wave == 0) { ext_list1(lds); }   // fl_moe's combine on the kernel's own picks

    // 3. routed gate/up: expert sel[xcd], h rows kb * 256 + qq * 64 .. + 63 (one row group of gate and up), as items
    //    the waves claim from an LDS counter
    const int kb = li / 4, qq = li % 4;
    {
        const int e = reinterpret_cast<const LK_LOCAL int *>(lds + M_SEL)[xcd];
        if ((unsigned) e >= (unsigned) a.n_exp) { report1(a, 32); return; }
        const uint8_t * gm = uniform1(a.gate + (size_t) e * a.estride), * um = uniform1(a.up + (size_t) e * a.estride);
        TRACE1(5);
        if constexpr (FD == 0) { gate_up2(a, lds, ctl, gm, um, xcd, li, tr, r); }
        else { gate_up1(a, lds, ctl, gm, um, xcd, kb * QK + qq * 64, tr, r); }
        TRACE1(6);
    }

    // 4. down: the workgroup's units (28 routed row groups at K-block kb, 3 or 4 shared row groups at K-block xcd),
    //    claimed by the waves in order; each wave's first unit streams in while the h blocks are polled and staged
    const int nsh = li < RGE1 - 3 * 32 ? 4 : 3;   // shared row groups li, li + 32, .. (< 112)
    const int nunits = RGQ1 + nsh;
    const int e_dn = reinterpret_cast<const LK_LOCAL int *>(lds + M_SEL)[xcd];
    LK_LOCAL unsigned * dclaim = ctl + C_DNCLAIM;
    if constexpr (FD == 0) {
        // units in claim order: the 14 row groups (i % 8) * 14 .. + 13 at K-block kb_0 (h block kb_0, complete since
        // phase 1), the shared expert's row groups at K-block x, then the same 14 row groups at K-block kb_1. The first
        // wave to need an h block polls and stages it (the others wait on its LDS flag), so the hand-off of block kb_1
        // overlaps the units before it.
        constexpr int RG2 = E1 / 64 / 8;   // 14
        const int hs = li & 7, kb0 = li >> 3, kb1 = 4 + (li >> 3);
        const int nu2 = 2 * RG2 + nsh;
        const uint8_t * dmat = uniform1(a.down + (size_t) e_dn * a.estride);
        // unit u -> (matrix, row group, K-block, slot, staged block: 0 kb_0, 1 shared, 2 kb_1)
        auto unit = [&](int u, const uint8_t * & mat, int & g64, int & blk, int & slot, int & hb) {
            if (u < RG2) { mat = dmat; g64 = hs * RG2 + u; blk = kb0; slot = xcd; hb = 0; }
            else if (u < RG2 + nsh) { mat = uniform1(a.sh_down); g64 = li + 32 * (u - RG2); blk = xcd; slot = 8; hb = 1; }
            else { mat = dmat; g64 = hs * RG2 + (u - RG2 - nsh); blk = kb1; slot = xcd; hb = 2; }
        };
        auto claim_unit = [&](Dn1 & d, int & u) {
            unsigned c = 0;
            if (lane == 0) { c = __hip_atomic_fetch_add(dclaim, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
            u = (int) __builtin_amdgcn_readfirstlane(c);
            if (u < nu2) { const uint8_t * m; int g, b, sl, hb; unit(u, m, g, b, sl, hb); dn1_issue(m, g, b, d); }
        };
        // The first wave out of gate/up items stages the h blocks in the order they complete: kb_0 and the shared
        // block together (both long complete by now, polled in one round trip), then kb_1; the other waves claim their
        // units (loads in flight) and wait on the block's LDS flag.
        {
            unsigned got = 0;
            if (lane == 0) { got = __hip_atomic_fetch_add(ctl + C_LR, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
            if (__builtin_amdgcn_readfirstlane(got) == 0) {
                bool ok = stage_h2(a, a.th + (size_t) xcd * H1 + (size_t) kb0 * QK, lds + M_HR, a.th + (size_t) 8 * H1 + (size_t) xcd * QK, lds + M_HS);
                if (!ok) { report1(a, 1); }
                flag1(ctl + C_HR, ok ? 1u : 2u); flag1(ctl + C_HS, ok ? 1u : 2u);
                TRACE1(60);
                ok = stage_h1(a, a.th + (size_t) xcd * H1 + (size_t) kb1 * QK, lds + M_HB);
                if (!ok) { report1(a, 1); }
                flag1(ctl + C_HB, ok ? 1u : 2u);
                TRACE1(7);
            }
        }
        auto ensure = [&](int hb) -> bool {
            const unsigned v = wait1(ctl + (hb == 0 ? C_HR : hb == 1 ? C_HS : C_HB), 1);
            lds_visible();
            if (v == 0) { report1(a, 8); }
            return v == 1;
        };
        Dn1 dn; int un;
        claim_unit(dn, un);
        while (un < nu2) {
            const uint8_t * m; int g, b, sl, hb; unit(un, m, g, b, sl, hb);
#ifdef LOKI_TRACE
            if (un == 0) { TRACE1(58); }
            if (un == RG2 + nsh) { TRACE1(59); }
#endif
            if (!ensure(hb)) { return; }
            const uint8_t * hbp = (const uint8_t *) (lds + (hb == 0 ? M_HR : hb == 1 ? M_HS : M_HB));
            const int bsum = block_bsum_dpp(dn.w, tr, hbp, r);
            const float dx = *reinterpret_cast<const float *>(hbp + QK);
            st_tag1(a.to + ((size_t) sl * NBH1 + b) * E1 + (size_t) g * 64 + lane, a.epoch, (h2f(dn.d) * dx) * (float) bsum);
            claim_unit(dn, un);   // claims rise: the first past the end ends the list
        }
        TRACE1(8);
    } else {
        // K-quant: the shared expert's units (Q6_K) first -- its h block is complete long before the routed one, so
        // waves that finish their gate/up items early run them while the routed h block is still being formed -- then
        // the routed units (format FD); each stream waits only for its own h block
        constexpr uint32_t RBD = NBH1 * kbytes<FD>(), RB6 = NBH1 * kbytes<KF_Q6K>();
        auto claim = [&]() -> int {
            unsigned c = 0;
            if (lane == 0) { c = __hip_atomic_fetch_add(dclaim, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
            return (int) __builtin_amdgcn_readfirstlane(c);
        };
        const uint32_t r8 = (uint32_t) lane >> 3;
        const Src ssrc = src1(a.sh_down, (uint64_t) E1 * RB6, r8 * RB6 + (uint32_t) xcd * kbytes<KF_Q6K>());
        const Src rsrc = src1(a.down + (size_t) e_dn * a.dstride, (uint64_t) E1 * RBD, r8 * RBD + (uint32_t) kb * kbytes<FD>());
        auto g_s = [&](int u) { return li + 32 * u; };              // units 0 .. nsh - 1
        auto g_r = [&](int u) { return qq * RGQ1 + (u - nsh); };    // units nsh .. nunits - 1
        // wave 0 stages the routed h block first (it polls until the block is complete), the others claim and
        // prime their rings while the h blocks form
        if (wave == 0) {
            const bool ok = stage_h1(a, a.th + (size_t) xcd * H1 + (size_t) kb * QK, lds + M_HR);
            if (!ok) { report1(a, 1); }
            flag1(ctl + C_HR, ok ? 1u : 2u);
        }
        DnRing1<KF_Q6K> rs;
        dn_prime1<KF_Q6K>(rs, claim(), nsh, ssrc, g_s, claim);
        if (wave == 1) {
            const bool ok = stage_h1(a, a.th + (size_t) 8 * H1 + (size_t) xcd * QK, lds + M_HS);
            if (!ok) { report1(a, 1); }
            flag1(ctl + C_HS, ok ? 1u : 2u);
        }
        TRACE1(7);
        if (wait1(ctl + C_HS, 1) != 1) { return; }
        lds_visible();
        const int un = dn_run1<KF_Q6K>(a, rs, nsh, ssrc, reinterpret_cast<const LK_LOCAL int8_t *>(lds + M_HS),
                                       *reinterpret_cast<const LK_LOCAL float *>(lds + M_HS + QK), 8, xcd, g_s, claim);
        DnRing1<FD> rr;
        dn_prime1<FD>(rr, un, nunits, rsrc, g_r, claim);
        if (wait1(ctl + C_HR, 1) != 1) { return; }
        lds_visible();
        TRACE1(8);
        (void) dn_run1<FD>(a, rr, nunits, rsrc, reinterpret_cast<const LK_LOCAL int8_t *>(lds + M_HR),
                           *reinterpret_cast<const LK_LOCAL float *>(lds + M_HR + QK), xcd, kb, g_r, claim);
    }
    TRACE1(9);

    // 5. combine rows 28 b .. 28 b + 27 (a timed-out poll is flagged in LDS; no __syncthreads_and: it would take static
    //    LDS and move the table base off its 64 KB alignment)
    combine1<FD != 0>(a, lds);
    if (wave == 0 && __hip_atomic_load(ctl + C_CMBFAIL, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) { report1(a, 16); }
    TRACE1(10);
    if (blockIdx.x == 0 && wave == W1 - 1 && !a.ext_sel) { routing1(a, lds); }
    if (a.fdone && wave == 0) {
        // this workgroup's combine rows are written (wave 0 wrote them): count it; the last one tells the host. No fence
        // per workgroup (an L2 write-back each): the rows go to the caller's memory before the count, and the last
        // workgroup's system-scope release orders them before the word
        stores_done();
        unsigned old = 0;
        if (lane == 0) { old = __hip_atomic_fetch_add(gptr(a.fcnt), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
        old = __builtin_amdgcn_readfirstlane(old);
        if (old + 1 == (unsigned) G1) {
            if (lane == 0) { __hip_atomic_store(gptr(a.fcnt), 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
            if (a.tstamp && lane == 0) {
                __hip_atomic_store(gptr(a.tstamp) + 1, (uint64_t) __builtin_amdgcn_s_memrealtime(), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
            if (lane == 0) { __hip_atomic_store(gptr(a.fdone), a.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); }
        }
    }
}

size_t decode1_lds_bytes() { return DEC1_LDS; }

// set-up probe: the XCD of every workgroup of a 256-workgroup launch
__device__ int g_xcc1[G1];
__global__ void k_xcc_probe1() { if (threadIdx.x == 0) { g_xcc1[blockIdx.x] = xcc_id1(); } }

// the kernel's variants: every matrix IQ2_XXS; routed down Q2_K or Q3_K with the shared expert in Q5_K / Q5_K / Q6_K
static const void * const kernels1[3] = { (const void *) k_moe_decode1<0>, (const void *) k_moe_decode1<KF_Q2K>,
                                          (const void *) k_moe_decode1<KF_Q3K> };

hipError_t decode1_init(int ncu, int * ok) {
    *ok = 0;
    if (ncu != G1) { return hipSuccess; }   // the XCD mapping needs one workgroup on each of 256 CUs
    hipError_t e = hipSuccess;
    for (const void * k : kernels1) {   // every format variant fits one workgroup per CU
        if ((e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, DEC1_LDS)) != hipSuccess) { return e; }
        int per = 0;
        if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, k, NT1, DEC1_LDS)) != hipSuccess) { return e; }
        if (per < 1) { return hipSuccess; }
    }
    // roles come from the XCD a workgroup runs on, and hand-offs inside an XCD go through its L2: the dispatch must
    // place workgroup b on XCD (r + b) % 8 for one r
    hipLaunchKernelGGL(k_xcc_probe1, dim3(G1), dim3(64), 0, 0);
    if ((e = hipGetLastError()) != hipSuccess) { return e; }
    int x[G1];
    if ((e = hipMemcpyFromSymbol(x, HIP_SYMBOL(g_xcc1), sizeof x)) != hipSuccess) { return e; }
    for (int b = 0; b < G1; ++b) { if (x[b] != (x[0] + b) % NX1) { return hipSuccess; } }
    *ok = 1;
    return hipSuccess;
}

hipError_t launch_moe_decode1(const DecodeArgs & a, bool cooperative, hipStream_t st) {
    if ((a.ext_sel || a.spec_combine) && ((a.ext_sel && !a.ext_w) || !a.moe_out || !a.resid || a.prenorm)) { return hipErrorInvalidValue; }   // fl_moe's combine
    if ((a.spec_combine && (a.ext_sel || !a.hsel || !a.hdone)) || (a.fdone && !a.fcnt)) { return hipErrorInvalidValue; }
    if (a.n != 1 || a.topk != MAXK || a.keep != MAXK || (!a.ext_sel && !decode_rule_ok(a.n_exp, a.n_group)) || a.E != E1 || a.H != H1 ||
        !a.th || !a.to || !a.tlogits || a.n_exp > NEXP_MAX || (a.kdown != 0 && a.kdown != KF_Q2K && a.kdown != KF_Q3K) ||
        (a.kdown != 0 && ((reinterpret_cast<uintptr_t>(a.down) | reinterpret_cast<uintptr_t>(a.sh_gate) |
                           reinterpret_cast<uintptr_t>(a.sh_up) | reinterpret_cast<uintptr_t>(a.sh_down) | a.dstride) & 3u))) {
        return hipErrorInvalidValue;   // K-quant matrices: 4-byte aligned (the slices' word loads)
    }
    const void * k = kernels1[a.kdown == 0 ? 0 : a.kdown == KF_Q2K ? 1 : 2];
    DecodeArgs arg = a;
    void * params[] = { &arg };
    if (!cooperative) { return hipLaunchKernel(k, dim3(G1), dim3(NT1), params, DEC1_LDS, st); }
    return hipLaunchCooperativeKernel(k, dim3(G1), dim3(NT1), params, DEC1_LDS, st);
}

}  // namespace lk
