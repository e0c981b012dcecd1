// moe_decode.hip -- the whole MoE block for a decode batch (n <= 8 tokens) in one launch.
//
// Reference path (src/fused_layer.cu): router_probs + router_topk (:313-332, launched :506), a host round-trip for the
// routing (fl_fetch :587-598, eng:793-818), then per fl_moe (:599-612) quant_x, tc_matvec gate/up, swiglu_q8,
// tc_matvec down and moe_combine as separate launches. At batch 1-8 every one of those launches is latency-bound, so
// here one workgroup per CU (all resident) runs the block end to end:
//   1. on entry every workgroup starts the direct global->LDS copy of the codebook/sign table image; workgroup b then
//      computes the router logits of expert b for every token (the fp64 chunk-and-tree contract) and publishes each
//      probability sigmoid(logit) as an epoch-tagged 64-bit word;
//   2. wave t of every workgroup issues its poll of token t's tagged probabilities, all waves quantise the token blocks
//      to Q8_K into LDS (every workgroup from x, which its router pass left in L2), then wave t selects token t's
//      experts and the last selecting wave builds the dispatch (stable
//      counting sort of the n * topk pairs) in its own LDS -- redundant, but cheaper than another device-wide hand-off.
//      Waves without a token meanwhile run the shared expert's gate/up tasks (no routing needed);
//   3. gate/up tasks: a task computes 8 gate rows and the same 8 up rows of one expert for one token and publishes
//      h = silu(g) * u as epoch-tagged words; a workgroup's 8 waves take 8 consecutive tasks (one 64-row group);
//   4. down units round-robin over the workgroups: a unit is 256 output rows of one expert for one token (32 per wave).
//      The waves issue their first weight loads, then wave w polls the tagged h of Q8_K block w and quantises it into
//      LDS; after a barrier each wave computes its rows and publishes o as epoch-tagged words;
//   5. combine units (256 rows each) on the last workgroups: y = sum_k w_k o_k (k order) + shared, from the tagged o words.
// No counter, flag or store-completion wait sits between producer and consumer: a consumer polls the data words
// themselves, and a word is valid once it carries this launch's epoch (stale words hold older epochs; the host clears
// the tagged buffers whenever the epoch restarts at 1). Arithmetic is that of the per-pass kernels (same device
// functions), so y is bit-identical to theirs and to the CPU checker. Every wait is bounded: a timeout sets *err and the
// wave skips the work, so the grid always drains.
#include "moe_device.h"
#include "moe_kernels.h"

namespace lk {

constexpr int DW = 8, DNT = DW * 64;   // waves / threads per workgroup
constexpr int DMAX_N = 8, DMAX_P = DMAX_N * MAXK;
constexpr int DMAX_PS = DMAX_P + DMAX_N;   // task slots: the shared expert's n + one per routed pair
constexpr int SH = NEXP_MAX;           // expert-slot marker of the shared expert
using GG = Geo<7, 0>;                  // gate/up rows: K = 7168 (staged without padding)
using GD = Geo<2, 0>;                  // down rows: K = 2048
constexpr int DE = GG::K, DH = GD::K;
constexpr int GU_ROWS = 8;             // h rows per gate/up task (8 gate + the same 8 up rows)
constexpr int NGU = DH / GU_ROWS;      // gate/up tasks per expert
constexpr int DN_ROWS = DW * 32;       // output rows per down unit (32 per wave: two row sets of 16)
constexpr int NDN = DE / DN_ROWS;      // down units per expert (= combine units)
constexpr int GU_PD = 3, DN_PD = 3;   // blocks in flight per lane
constexpr int DN_PRE = 2;              // down steps issued before the h staging (register budget)
static_assert(DH == DW * QK, "a down unit's wave w quantises h block w");
static_assert(DMAX_N * (MAXK + 1) * DH <= (int) DEC_TH && DMAX_N * (MAXK + 1) * DE <= (int) DEC_TO, "tagged buffer sizes");

// LDS layout
constexpr int L_XS = TAB_BYTES;                                   // staged Q8_K tokens (gate/up), then the h of the down units
constexpr int L_PRE = L_XS + DMAX_N * GG::XROW;                   // early shared task's block terms [2][7][64] floats
constexpr int PRE_BYTES = 2 * 7 * 64 * 4;
constexpr int L_SCR = L_PRE;                                      // router sums [token][quarter] (phase 1) overlay them
constexpr int L_RT = L_PRE + PRE_BYTES;                           // routing tables
constexpr int RT_INTS = 4 * DMAX_P + 3 * (DMAX_P + 1) + 1 + 2 * DMAX_PS + 1;
constexpr int L_CTL = L_RT + RT_INTS * 4;                         // hand-off words [8], staging flags [DW]
constexpr int L_NRM = L_CTL + (8 + DW) * 4;                       // pre-norm scale per token [DMAX_N]
// the caller's picks (ext_sel): per token its distinct ids ascending as [first k][summed weight], then their count
constexpr int L_EXT = L_NRM + DMAX_N * 4, EXT_TOK = 2 * MAXK + 1;
constexpr int DEC_LDS = L_EXT + DMAX_N * EXT_TOK * 4;
static_assert(DEC_LDS <= 160 * 1024, "LDS budget");
static_assert(DMAX_N * 4 * 8 <= PRE_BYTES && DW * 112 * 4 <= PRE_BYTES, "router sums and selection scratch overlay the early task terms");

typedef LK_LOCAL uint8_t * lds_t;
typedef LK_CONST DecodeArgs DArgs;   // the launch arguments, read in place with scalar loads

// Routing of the launch, in LDS. The task list ps holds one entry per dispatch slot (one token of one expert), so every
// gate/up task and down unit costs one pass over its weights and the round-robin assignment is balanced; the two tokens
// of an expert are adjacent entries, whose tasks run side by side (same workgroup for gate/up) and share the weights
// through L2. ps_mi = act index or SH, ps_s = slot | token count (1) << 16; the shared expert's slots come first.
struct RT {
    LK_LOCAL int * sel; LK_LOCAL float * wts; LK_LOCAL int * perm, * inv, * act_e, * act_s0, * act_cnt, * nact;
    LK_LOCAL int * ps_mi, * ps_s, * nps;
    __device__ RT(lds_t lds) {
        LK_LOCAL int * b = reinterpret_cast<LK_LOCAL int *>(lds + L_RT);
        sel = b; wts = reinterpret_cast<LK_LOCAL float *>(b + DMAX_P); perm = b + 2 * DMAX_P; inv = b + 3 * DMAX_P;
        act_e = b + 4 * DMAX_P; act_s0 = act_e + DMAX_P + 1; act_cnt = act_s0 + DMAX_P + 1; nact = act_cnt + DMAX_P + 1;
        ps_mi = nact + 1; ps_s = ps_mi + DMAX_PS; nps = ps_s + DMAX_PS;
    }
};

// an error code into the device word (OR of every code) and, when the context has one, the host-mapped word (a plain
// system-scope store: the host checks it at its next call without waiting for the stream)
__device__ __forceinline__ void report(const DArgs & a, int code) {
    if (lane_id() == 0) {
        __hip_atomic_fetch_or(gptr(a.err), code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (a.herr) { __hip_atomic_store(gptr(a.herr), code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); }
    }
}

// epoch-tagged words: {epoch (bits 32..63), fp32 bits}, one 64-bit store / load each (single-copy atomic)
__device__ __forceinline__ void st_tag(uint64_t * p, uint32_t epoch, float v) {
    __hip_atomic_store(gptr(p), ((uint64_t) epoch << 32) | __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ld_tag(const uint64_t * p) { return __hip_atomic_load(gptr(const_cast<uint64_t *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ bool tag_ok(uint64_t w, uint32_t epoch) { return (uint32_t) (w >> 32) == epoch; }
__device__ __forceinline__ float tag_val(uint64_t w) { return __builtin_bit_cast(float, (uint32_t) w); }
constexpr int POLL_MAX = 1 << 20;   // polls before a wait gives up (each poll is a memory round trip)

// workgroup hand-off in LDS: counted arrivals and a ready word (waves of one workgroup are always co-resident)
__device__ __forceinline__ bool lds_arrive(LK_LOCAL unsigned * c, unsigned expected) {
    lds_visible();
    unsigned old = 0;
    if (lane_id() == 0) { old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
    old = __builtin_amdgcn_readfirstlane(old);
    return old + 1 == expected;
}
__device__ __forceinline__ unsigned lds_wait(LK_LOCAL unsigned * w) {
    for (int i = 0; i < (1 << 24); ++i) {
        const unsigned v = __builtin_amdgcn_readfirstlane(__hip_atomic_load(w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
        if (v) { return v; }
        __builtin_amdgcn_s_sleep(1);
    }
    return 0;
}
__device__ __forceinline__ bool lds_wait_count(LK_LOCAL unsigned * c, unsigned want) {
    for (int i = 0; i < (1 << 24); ++i) {
        if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) == want) { return true; }
        __builtin_amdgcn_s_sleep(1);
    }
    return false;
}
// a wave-uniform pointer kept in scalar registers (a per-lane select between two of them must not become a vector load
// of the argument block)
__device__ __forceinline__ const uint8_t * uniform_ptr(const uint8_t * p) {
    const uint64_t v = (uint64_t) p;
    // the builtin returns int: both halves go through uint32_t, so the low half is not sign-extended into the high one
    const uint32_t hi = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) (v >> 32));
    const uint32_t lo = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) v);
    return (const uint8_t *) (((uint64_t) hi << 32) | (uint64_t) lo);
}

// Timeline probe for tuning builds (-DLOKI_TRACE): per wave, 64-bit s_memrealtime stamps (100 MHz) at the phase
// boundaries (slots 0-8), the down phase (24: start, 25: h staged, 26: rows computed) and the combine (56, 58);
// slot 63 = counts.
#ifdef LOKI_TRACE
constexpr int TRACE_SLOTS = 64;
__device__ uint64_t g_trace[1024 * DW * TRACE_SLOTS];
#define TRACE(wave, slot) do { if (lane_id() == 0) { g_trace[(blockIdx.x * DW + (wave)) * TRACE_SLOTS + (slot)] = __builtin_amdgcn_s_memrealtime(); } } while (0)
#define TRACE_T(tb, k) do { if ((tb) >= 0) { TRACE(threadIdx.x >> 6, (tb) + (k)); } } while (0)
extern "C" hipError_t fl_trace_copy(void * host, size_t bytes) { return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace), bytes); }
extern "C" hipError_t fl_trace_clear() {
    void * p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_trace));
    return e == hipSuccess ? hipMemset(p, 0, sizeof(g_trace)) : e;
}
#else
#define TRACE(wave, slot) do { } while (0)
#define TRACE_T(tb, k) do { } while (0)
#endif

// ---------------------------------------------------------------- phase 1
// RMSNorm scales of the tokens (prenorm): waves 4 h .. 4 h + 3 take tokens h, h + 2, ..; thread (q = wave & 3, lane)
// sums chunk 64 q + lane (sumsq_chunk, the contract of k_rmsnorm), so the scale is bit-identical to a separate
// k_rmsnorm pass. Every workgroup computes them for itself from x (L2).
__device__ __noinline__ void norm_phase(const DArgs & a, lds_t lds, int wave) {
    LK_LOCAL double * part = reinterpret_cast<LK_LOCAL double *>(lds + L_SCR);   // [token][quarter]
    const int lane = lane_id(), qt = wave & 3;
    for (int t = wave >> 2; t < a.n; t += DW / 4) {
        const double s = tree64(sumsq_chunk<DE / 1024>(a.x + (size_t) t * DE, qt * 64 + lane));
        if (lane == 0) { part[t * 4 + qt] = s; }
    }
    __syncthreads();
    if (threadIdx.x < (unsigned) a.n) {
        const int t = threadIdx.x;
        reinterpret_cast<LK_LOCAL float *>(lds + L_NRM)[t] = rms_scale(part[t * 4], part[t * 4 + 1], part[t * 4 + 2], part[t * 4 + 3], DE, a.eps);
    }
    __syncthreads();
}
// the block's input: x, or (x * scale) * w under prenorm (k_rmsnorm's arithmetic), for 4 values at column col of token t
__device__ __forceinline__ float4 block_in(const DArgs & a, lds_t lds, int t, int col, float4 v) {
#pragma clang fp contract(off)
    if (!a.prenorm) { return v; }
    const float sc = reinterpret_cast<const LK_LOCAL float *>(lds + L_NRM)[t];
    v.x = v.x * sc; v.y = v.y * sc; v.z = v.z * sc; v.w = v.w * sc;
    if (a.nw) { const float4 w = gloadf4(a.nw + col); v.x = v.x * w.x; v.y = v.y * w.y; v.z = v.z * w.z; v.w = v.w * w.w; }
    return v;
}

// The table image into LDS with direct global->LDS loads (16 B per lane, 1 KB per wave instruction), issued first so
// they complete under the router's loads; visible to the workgroup after s_waitcnt vmcnt(0) and a barrier.
__device__ __forceinline__ void tables_dma(lds_t lds, const uint4 * img, int wave) {
    constexpr int PER = TAB_BYTES / 1024 / DW;
    const int lane = lane_id();
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int c = wave * PER + k;
        __builtin_amdgcn_global_load_lds((const LK_GLOBAL void *) (img + c * 64 + lane), (LK_LOCAL void *) (lds + c * 1024), 16, 0, 0);
    }
}

// Q8_K of every token block into this workgroup's LDS (staged layout): a pass of wave w quantises 4 consecutive
// blocks, one per 16-lane row (q8k_row16); the wave's passes (up to 7) load first, then compute. x is in L2 after the
// router's reads. Workgroup 0 also writes the layer's xq / xd.
__device__ __forceinline__ void local_quant(const DArgs & a, lds_t lds, int wave) {
    constexpr int MAXP = DMAX_N * GG::NB / (4 * DW);
    static_assert(GG::NB % 4 == 0 && MAXP * 4 * DW == DMAX_N * GG::NB, "four blocks per pass");
    const int nblk = a.n * GG::NB, lane = lane_id(), i = lane & 15;
    // every pass's loads are issued before any value is used (with the prenorm input transform applied per load the
    // compiler waited for each load before issuing the next)
    float4 xv[MAXP][4];
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
        const int k = 4 * (wave + DW * p) + (lane >> 4);
        if (4 * (wave + DW * p) < nblk) {
            const float * src = a.x + (size_t) (k / GG::NB) * DE + (k % GG::NB) * QK + 16 * i;
#pragma unroll
            for (int q = 0; q < 4; ++q) { xv[p][q] = gloadf4(src + 4 * q); }
        }
    }
    if (a.prenorm) {
#pragma unroll
        for (int p = 0; p < MAXP; ++p) {
            const int k = 4 * (wave + DW * p) + (lane >> 4);
            if (4 * (wave + DW * p) < nblk) {
#pragma unroll
                for (int q = 0; q < 4; ++q) { xv[p][q] = block_in(a, lds, k / GG::NB, (k % GG::NB) * QK + 16 * i + 4 * q, xv[p][q]); }
            }
        }
    }
    float xs[MAXP][16];
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            xs[p][4 * q] = xv[p][q].x; xs[p][4 * q + 1] = xv[p][q].y; xs[p][4 * q + 2] = xv[p][q].z; xs[p][4 * q + 3] = xv[p][q].w;
        }
    }
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
        if (4 * (wave + DW * p) < nblk) {
            const int k = 4 * (wave + DW * p) + (lane >> 4), t = k / GG::NB, j = k % GG::NB;
            uint32_t packed[4]; float d;
            q8k_row16(xs[p], packed, d);
            lds_t row = lds + L_XS + t * GG::XROW;
#pragma unroll
            for (int w = 0; w < 4; ++w) { *reinterpret_cast<LK_LOCAL uint32_t *>(row + j * GG::XBLK + staged_word(4 * i + w)) = packed[w]; }
            if (i == 0) { reinterpret_cast<LK_LOCAL float *>(row + GG::NB * GG::XBLK)[j] = d; }
            if (blockIdx.x == 0) {
                *(LK_GLOBAL u32x4 *) (a.xq + (size_t) t * DE + (size_t) j * QK + 16 * i) = u32x4{ packed[0], packed[1], packed[2], packed[3] };
                if (i == 0) { gptr(a.xd)[k] = d; }
            }
        }
    }
}

// XCD-shared Q8_K of the tokens (a.xqx): workgroup (x, li) -- x its XCD (hardware register XCC_ID), li = b / 8 --
// quantises blocks li, li + 32, .. of the n tokens (block k: token k / 28, block k % 28), one per 16-lane row
// (q8k_row16, as local_quant), into XCD x's copy of the staged token rows, waits for those stores (vmcnt(0): acknowledged
// by the XCD's L2) and tags each block's word with the launch's epoch (a plain store, read in the same L2). Every
// workgroup of the XCD then polls the tagged words of all n * 28 blocks and copies the rows into its LDS with direct
// loads (the launch started with an invalidated L1, and nothing of the copy was read before the tags: the loads come
// from the L2). One quantisation per block per XCD instead of per workgroup: local_quant costs every workgroup ~8 us
// at n = 8. Returns false on a timed-out wait.
constexpr size_t XQX_ROWS = (size_t) DMAX_N * GG::XROW;                          // staged rows of the n tokens
constexpr size_t XQX_BYTES = (XQX_ROWS + (size_t) DMAX_N * GG::NB * 8 + 255) / 256 * 256;   // + one tagged word per block
static_assert(XQX_ROWS % 16 == 0 && GG::XROW % 16 == 0, "16-byte copies of the staged rows");
__device__ __forceinline__ int xcc_id_d() {
    unsigned x;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
    return (int) (x & 0xFu);
}
__device__ __forceinline__ bool xcd_quant(const DArgs & a, lds_t lds, int wave) {
    const int lane = lane_id(), i = lane & 15, nblk = a.n * GG::NB, xcd = xcc_id_d(), li = (int) blockIdx.x / 8;
    uint8_t * mir = a.xqx + (size_t) xcd * XQX_BYTES;
    uint64_t * tags = reinterpret_cast<uint64_t *>(mir + XQX_ROWS);
    // produce: block k = li + 32 (4 wave + row)
    const int k = li + 32 * (4 * wave + (lane >> 4));
    if (4 * wave * 32 + li < nblk) {   // this wave has at least one block (rows past nblk idle)
        float4 xv[4];
        const int t = k < nblk ? k / GG::NB : 0, j = k < nblk ? k % GG::NB : 0;
        const float * src = a.x + (size_t) t * DE + j * QK + 16 * i;
#pragma unroll
        for (int q = 0; q < 4; ++q) { xv[q] = k < nblk ? gloadf4(src + 4 * q) : make_float4(0.f, 0.f, 0.f, 0.f); }
        if (a.prenorm && k < nblk) {
#pragma unroll
            for (int q = 0; q < 4; ++q) { xv[q] = block_in(a, lds, t, j * QK + 16 * i + 4 * q, xv[q]); }
        }
        float xs[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) { xs[4 * q] = xv[q].x; xs[4 * q + 1] = xv[q].y; xs[4 * q + 2] = xv[q].z; xs[4 * q + 3] = xv[q].w; }
        uint32_t packed[4]; float d;
        q8k_row16(xs, packed, d);   // (every lane of the wave joins the row reductions)
        if (k < nblk) {
            uint8_t * row = mir + (size_t) t * GG::XROW;
#pragma unroll
            for (int w = 0; w < 4; ++w) { *gptr(reinterpret_cast<uint32_t *>(row + j * GG::XBLK + staged_word(4 * i + w))) = packed[w]; }
            if (i == 0) { *gptr(reinterpret_cast<float *>(row + GG::NB * GG::XBLK + 4 * j)) = d; }
            if (xcd == 0) {   // the layer's xq / xd (XCD 0's producers)
                *(LK_GLOBAL u32x4 *) (a.xq + (size_t) t * DE + (size_t) j * QK + 16 * i) = u32x4{ packed[0], packed[1], packed[2], packed[3] };
                if (i == 0) { gptr(a.xd)[k] = d; }
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): the block's stores are in the L2
        if (k < nblk && i == 0) {
            __hip_atomic_store(gptr(tags + k), (uint64_t) a.epoch << 32, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    // consume: every block tagged, then the rows into LDS (16 bytes per lane per copy, wave-interleaved)
    constexpr int TPL = (DMAX_N * GG::NB + 63) / 64;   // tags per lane
    bool ok = false;
    for (int it = 0; it < POLL_MAX; ++it) {
        bool v = true;
#pragma unroll
        for (int q = 0; q < TPL; ++q) {
            const int kk = lane + 64 * q;
            if (kk < nblk) { v = v && tag_ok(ld_tag(tags + kk), a.epoch); }
        }
        if (__ballot(!v) == 0) { ok = true; break; }
        __builtin_amdgcn_s_sleep(1);
    }
    if (!ok) { return false; }
    const int nchunk = (int) (a.n * GG::XROW / 1024), tail = (int) (a.n * GG::XROW % 1024);
    for (int c = wave; c < nchunk; c += DW) {
        __builtin_amdgcn_global_load_lds((const LK_GLOBAL void *) (mir + (size_t) c * 1024 + 16 * lane), (LK_LOCAL void *) (lds + L_XS + c * 1024), 16, 0, 0);
    }
    if (tail && wave == (nchunk % DW) && 16 * lane < tail) {
        *reinterpret_cast<LK_LOCAL u32x4 *>(lds + L_XS + nchunk * 1024 + 16 * lane) = *(const LK_GLOBAL u32x4 *) (mir + (size_t) nchunk * 1024 + 16 * lane);
    }
    return true;
}
size_t decode_xq_bytes() { return 8 * XQX_BYTES; }

// Router logits of expert e for all n tokens by the whole workgroup (the contract of moe_device.h: 256 in-order chunk
// sums, pairwise tree, one rounding). Thread (quarter w = wave & 3, lane) owns chunk 64 w + lane (K/256 = 28 values)
// of every token t with t % 2 == wave / 4, so each thread issues its 7 + 7 * (tokens) 16-byte loads at once. Tree levels
// 1-6 run inside the wave (one chunk per lane), 7-8 combine the four quarters' totals through LDS. Thread t then
// publishes p = sigmoid(logit) as one 64-bit word {epoch, fp32 bits}, so the selection starts from probabilities.
__device__ __noinline__ void router_phase(const DArgs & a, lds_t lds, int wave, int e) {
#pragma clang fp contract(off)
    constexpr int L4 = DE / 1024;   // float4 per chunk (7)
    const int lane = lane_id(), qt = wave & 3, half = wave >> 2, c = qt * 64 + lane;
    LK_LOCAL double * part = reinterpret_cast<LK_LOCAL double *>(lds + L_SCR);   // [token][quarter]
    constexpr int TB = 2;   // tokens per load batch (register budget)
    float4 wv[L4];
    const float * wc = a.Wr + (size_t) e * DE + (size_t) c * 4 * L4;
#pragma unroll
    for (int i = 0; i < L4; ++i) { wv[i] = gloadf4(wc + 4 * i); }
    for (int k0 = 0; k0 < DMAX_N / 2; k0 += TB) {
        if (2 * k0 + half >= a.n) { break; }
        float4 xv[TB][L4];
#pragma unroll
        for (int k = 0; k < TB; ++k) {
            const int t = 2 * (k0 + k) + half;
            if (t < a.n) {
#pragma unroll
                for (int i = 0; i < L4; ++i) { xv[k][i] = gloadf4(a.x + (size_t) t * DE + (size_t) c * 4 * L4 + 4 * i); }
#pragma unroll
                for (int i = 0; i < L4; ++i) { xv[k][i] = block_in(a, lds, t, c * 4 * L4 + 4 * i, xv[k][i]); }
            }
        }
#pragma unroll
        for (int k = 0; k < TB; ++k) {
            const int t = 2 * (k0 + k) + half;
            if (t < a.n) {
                double s = 0.0;
#pragma unroll
                for (int i = 0; i < L4; ++i) {
                    s += (double) xv[k][i].x * (double) wv[i].x; s += (double) xv[k][i].y * (double) wv[i].y;
                    s += (double) xv[k][i].z * (double) wv[i].z; s += (double) xv[k][i].w * (double) wv[i].w;
                }
                const double q = tree64(s);
                if (lane == 0) { part[t * 4 + qt] = q; }
            }
        }
    }
    __syncthreads();
    if (threadIdx.x < (unsigned) a.n) {
        const int t = threadIdx.x;
        const float l = (float) ((part[t * 4 + 0] + part[t * 4 + 1]) + (part[t * 4 + 2] + part[t * 4 + 3]));
        const size_t o = (size_t) t * a.n_exp + e;
        const float p = det_sigmoid(l);
        st_tag(a.tlogits + o, a.epoch, p);
        gptr(a.logits)[o] = l;   // the layer's logits and probabilities (read after the launch)
        if (a.probs) { gptr(a.probs)[o] = p; }
    }
    __syncthreads();   // part[] is reused by the next expert
}

// ---------------------------------------------------------------- phase 2
// token t's tagged probabilities of the lane's experts 4 lane + j (issue, then complete: the caller works in between)
__device__ __forceinline__ void probs_issue(const DArgs & a, int t, uint64_t (&w)[4]) {
    const int lane = lane_id();
#pragma unroll
    for (int j = 0; j < 4; ++j) { const int e = 4 * lane + j; w[j] = e < a.n_exp ? ld_tag(a.tlogits + (size_t) t * a.n_exp + e) : 0; }
}
// completes the poll: every word carries this launch's epoch (re-polled until then); false on timeout
__device__ __forceinline__ bool probs_wait(const DArgs & a, int t, uint64_t (&w)[4], float (&p)[4]) {
    const int lane = lane_id();
    for (int it = 0; it < POLL_MAX; ++it) {
        bool ok = true;
#pragma unroll
        for (int j = 0; j < 4; ++j) { ok = ok && (4 * lane + j >= a.n_exp || tag_ok(w[j], a.epoch)); }
        if (__ballot(!ok) == 0) {
#pragma unroll
            for (int j = 0; j < 4; ++j) { p[j] = 4 * lane + j < a.n_exp ? tag_val(w[j]) : 0.f; }
            return true;
        }
        __builtin_amdgcn_s_sleep(2);
        probs_issue(a, t, w);
    }
    return false;
}

// dispatch of the n * topk pairs (one wave): stable counting sort by expert,
// pos(i) = #{pairs with a lower expert} + #{earlier pairs with the same expert}. Lane i holds pair i; comparing the
// expert ids bit by bit from the top with ballots gives every lane the mask of lanes with a smaller id and the mask of
// lanes with the same id (8 bits: ids < NEXP_MAX = 256).
__device__ __noinline__ void dispatch_wave(const DArgs & a, lds_t lds, int P) {
    const RT rt(lds);
    const int lane = lane_id();
    const bool valid = lane < P;
    const int e = valid ? rt.sel[lane] : 0;
    uint64_t eq = __ballot(valid), lt = 0;
#pragma unroll
    for (int b = 7; b >= 0; --b) {
        const bool bit = (e >> b) & 1;
        const uint64_t ones = __ballot(valid && bit);
        if (bit) { lt |= eq & ~ones; }
        eq &= bit ? ones : ~ones;
    }
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int rank = __popcll(eq & below);
    const uint64_t first = __ballot(valid && rank == 0);
    const int less = __popcll(lt), dless = __popcll(lt & first);
    const int pos = less + rank;
    if (valid) {
        rt.perm[pos] = lane; rt.inv[lane] = pos;
        if (rank == 0) { rt.act_e[dless] = e; rt.act_s0[dless] = less; rt.act_cnt[dless] = __popcll(eq); }
    }
    if (lane == 0) { *rt.nact = __popcll(first); }
    // task slots: the shared expert's (token t at slot P + t), then every active expert's in act order
    lds_visible();
    const int nact = __popcll(first), nsh = a.n;
    const int cnt_l = lane < nact ? rt.act_cnt[lane] : 0, s_l = lane < nact ? rt.act_s0[lane] : 0;
    const int np = cnt_l;
    const int incl = (int) wave_scan_u32((uint32_t) np), pos0 = nsh + incl - np;
    for (int k = 0; k < np; ++k) {
        if (pos0 + k < DMAX_PS) { rt.ps_mi[pos0 + k] = lane; rt.ps_s[pos0 + k] = (s_l + k) | (1 << 16); }
    }
    if (lane < nsh) { rt.ps_mi[lane] = SH; rt.ps_s[lane] = (P + lane) | (1 << 16); }
    if (lane == 63) { *rt.nps = nsh + incl < DMAX_PS ? nsh + incl : DMAX_PS; }
}
// the layer's routing outputs from workgroup 0's tables (one wave, after its work: they are read after the launch)
__device__ __noinline__ void routing_outputs(const DArgs & a, lds_t lds, int P) {
    const RT rt(lds);
    const int lane = lane_id(), nact = *rt.nact;
    if (lane < P) { gptr(a.perm)[rt.inv[lane]] = lane; gptr(a.inv)[lane] = rt.inv[lane]; gptr(a.sel)[lane] = rt.sel[lane]; gptr(a.wts)[lane] = rt.wts[lane]; }
    if (lane < nact) { gptr(a.act)[lane] = rt.act_e[lane]; }
    if (lane == 0) { *gptr(a.nact) = nact; }
    for (int x = lane; x <= a.n_exp; x += 64) {
        int lt = 0, eq = 0;
        for (int j = 0; j < P; ++j) { const int ej = rt.sel[j]; lt += ej < x ? 1 : 0; eq += ej == x ? 1 : 0; }
        gptr(a.offsets)[x] = lt;
        if (x < a.n_exp) { gptr(a.counts)[x] = eq; }
    }
}

// ---------------------------------------------------------------- phase 3: gate/up tasks
// A task is 8 h rows of one pair-slot: lane 4 r + q reads row r of a 16-row set and blocks 4 jj + q (jj = the step,
// 0..6); rows r < 8 are gate rows and r >= 8 the same h rows of the up matrix, so every lane streams from its own base
// address. A task makes one pass over its weights per token (the second pass of a pair reads them from L2 again: two
// tokens in one pass need more registers than the stream leaves). A wave runs its passes as one continuous stream: step
// s of every pass uses register slot s, and the loads of the next pass's first steps are issued while the current pass
// computes its last ones.
struct Lane { int q, r; uint32_t tr; };

struct GuTask {
    const uint8_t * ql; const uint8_t * dl;   // this lane's qs / d address at step 0
    int mi, s, c, row, u;                     // expert slot (act index or SH), first dispatch slot, tokens (1, 2), h row, pass
};
constexpr int GU_STEPS = GG::BPQ;             // 7
constexpr size_t GU_QSTEP = 4 * 4096, GU_DSTEP = 4 * 128;   // 4 blocks per step (one per quad lane)

// task tk of a wave's list: pre = the shared expert's pair-slots k = tk / NGU (tokens 2k, 2k + 1), else pair-slot
// ps0 + tk / NGU of the routing table; false past the end (or for an invalid table entry, reported)
__device__ __forceinline__ bool gu_task(const DArgs & a, lds_t lds, const Lane ln, int tk, int t_end, bool pre, int ps0, int P, int nact, GuTask & t) {
    if (tk >= t_end) { return false; }
    const RT rt(lds);
    const int k = tk / NGU, hb = tk % NGU;
    if (pre) {
        t.mi = SH; t.s = P + 2 * k; t.c = a.n - 2 * k >= 2 ? 2 : 1;
    } else {
        const int sc = rt.ps_s[ps0 + k];
        t.mi = rt.ps_mi[ps0 + k]; t.s = sc & 0xFFFF; t.c = sc >> 16;
        if (!((t.mi == SH || (unsigned) t.mi < (unsigned) nact) && (t.c == 1 || t.c == 2) && t.s + t.c <= P + a.n)) { report(a, 32); return false; }
    }
    const bool routed = t.mi != SH;
    const int e = routed ? rt.act_e[t.mi] : 0;
    const uint8_t * gm = uniform_ptr(routed ? a.gate + (size_t) e * a.estride : a.sh_gate);
    const uint8_t * um = uniform_ptr(routed ? a.up + (size_t) e * a.estride : a.sh_up);
    const uint8_t * mat = ln.r >= 8 ? um : gm;
    t.row = hb * GU_ROWS + (ln.r & 7); t.u = 0;
    t.ql = mat + (size_t) (t.row >> 6) * GG::NB * 4096 + ln.q * 4096 + (t.row & 63) * 16;
    t.dl = mat + (size_t) (DH / 64) * GG::NB * 4096 + (size_t) (t.row >> 6) * GG::NB * 128 + ln.q * 128 + (t.row & 63) * 2;
    return true;
}

template <int PD>
struct GuStream {
    uint4 pf[GU_STEPS][4]; uint16_t pd[GU_STEPS];
    __device__ __forceinline__ void issue(const GuTask & t, int s) {
#pragma unroll
        for (int c = 0; c < 4; ++c) { pf[s][c] = load_nt(t.ql + s * GU_QSTEP + c * 1024); }
        pd[s] = *gptr(reinterpret_cast<const uint16_t *>(t.dl + s * GU_DSTEP));
    }
    // one pass (7 steps, one token xr): the row total before * 0.125, folded over the quad in block order; while step s
    // computes, step s + PD of this pass or step s + PD - 7 of the next one (if any) is issued
    // hp: the wave's half of the workgroup. The two waves sharing a SIMD (w, w + 4) swap priority every step, so neither
    // finishes its stream long before the other (with the default oldest-first arbitration, the younger wave would run
    // its last steps alone, latency-bound)
    __device__ __forceinline__ float pass(const GuTask & cur, const GuTask & nxt, bool has_next, uint32_t tr, const uint8_t * xr, int q, int r, int hp) {
#pragma clang fp contract(off)
        float acc = 0.f;
#pragma unroll
        for (int s = 0; s < GU_STEPS; ++s) {
            if ((s & 1) ^ hp) { __builtin_amdgcn_s_setprio(1); } else { __builtin_amdgcn_s_setprio(0); }
            if (s + PD < GU_STEPS) { issue(cur, s + PD); } else if (has_next) { issue(nxt, s + PD - GU_STEPS); }
            const int j = s * 4 + q;
            const int bsum = block_bsum_dpp(pf[s], tr, xr + j * GG::XBLK, r);
            const float dx = reinterpret_cast<const float *>(xr + GG::NB * GG::XBLK)[j];
            acc = fold_rows(acc, (h2f(pd[s]) * dx) * (float) bsum);
        }
        return acc;
    }
};

// h = silu(g) * u of the task's rows for the pass's token: lanes 0..7 hold the gate totals of the 8 rows, lanes 8..15
// the up totals (row_ror:8 brings them over)
__device__ __forceinline__ void gu_publish(const DArgs & a, const Lane ln, const GuTask & t, float acc) {
#pragma clang fp contract(off)
    const float other = __builtin_bit_cast(float, dppi<0x128>(__builtin_bit_cast(int, acc)));
    if (ln.q == 0 && ln.r < 8) { st_tag(a.th + (size_t) (t.s + t.u) * DH + t.row, a.epoch, det_silu(0.125f * acc) * (0.125f * other)); }
}
__device__ __forceinline__ const uint8_t * gu_xrow(const DArgs & a, lds_t lds, const GuTask & t, int P) {
    const RT rt(lds);
    const int slot = t.s + t.u;
    return (const uint8_t *) (lds + L_XS + (t.mi != SH ? rt.perm[slot] / a.keep : slot - P) * GG::XROW);
}

// the wave's tasks tk, tk + tstep, .. < t_end (every token pass of each) as one stream; returns the number of passes
template <int PD>
__device__ __forceinline__ int gate_up_stream(const DArgs & a, lds_t lds, const Lane ln, int tk, int tstep, int t_end, bool pre, int ps0, int P, int nact) {
    GuTask cur, nxt;
    if (!gu_task(a, lds, ln, tk, t_end, pre, ps0, P, nact, cur)) { return 0; }
    auto next_pass = [&](const GuTask & c0, GuTask & t) -> bool {   // the pair's second token, else the next task
        if (c0.u + 1 < c0.c) { t = c0; t.u = c0.u + 1; return true; }
        return gu_task(a, lds, ln, tk + tstep, t_end, pre, ps0, P, nact, t);
    };
    bool has_next = next_pass(cur, nxt);
    GuStream<PD> st;
#pragma unroll
    for (int s = 0; s < PD; ++s) { st.issue(cur, s); }
    int npass = 0;
    for (;;) {
        const float acc = st.pass(cur, nxt, has_next, ln.tr, gu_xrow(a, lds, cur, P), ln.q, ln.r, (int) ((threadIdx.x >> 8) & 1));
        gu_publish(a, ln, cur, acc);
        ++npass;
        if (!has_next) { __builtin_amdgcn_s_setprio(0); break; }
        if (nxt.u == 0) { tk += tstep; }
        cur = nxt;
        has_next = next_pass(cur, nxt);
    }
    return npass;
}

// The shared expert's single pair-slot as early work (n <= 2, one task per workgroup): the waves without a token split
// the task's 7 steps (step s on wave n + s % (DW - n)), each lane's block terms go to LDS, and the last of those waves
// folds them in block order and publishes h -- the arithmetic of a pass, finished while the routing is still running.
__device__ __forceinline__ void pre_shared_split(const DArgs & a, lds_t lds, const Lane ln, int wave, int P, LK_LOCAL unsigned * cnt) {
#pragma clang fp contract(off)
    const int nw = DW - a.n, lane = lane_id();
    GuTask t;
    if (!gu_task(a, lds, ln, blockIdx.x, NGU, true, 0, P, 0, t)) { return; }
    LK_LOCAL float * terms = reinterpret_cast<LK_LOCAL float *>(lds + L_PRE);   // [u][step][lane]
    const uint8_t * xr0 = gu_xrow(a, lds, t, P);
    GuTask t1 = t; t1.u = 1;
    const uint8_t * xr1 = t.c == 2 ? gu_xrow(a, lds, t1, P) : xr0;
    for (int s = wave - a.n; s < GU_STEPS; s += nw) {
        uint4 pf[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) { pf[c] = load_nt(t.ql + s * GU_QSTEP + c * 1024); }
        const float dw = h2f(*gptr(reinterpret_cast<const uint16_t *>(t.dl + s * GU_DSTEP)));
        const int j = s * 4 + ln.q;
        for (int u = 0; u < t.c; ++u) {   // both tokens from one load
            const uint8_t * xr = u ? xr1 : xr0;
            const int bsum = block_bsum_dpp(pf, ln.tr, xr + j * GG::XBLK, ln.r);
            const float dx = reinterpret_cast<const float *>(xr + GG::NB * GG::XBLK)[j];
            terms[(u * GU_STEPS + s) * 64 + lane] = (dw * dx) * (float) bsum;
        }
    }
    if (!lds_arrive(cnt, (unsigned) nw)) { return; }
    for (int u = 0; u < t.c; ++u) {
        float acc = 0.f;
#pragma unroll
        for (int s = 0; s < GU_STEPS; ++s) { acc = fold_rows(acc, terms[(u * GU_STEPS + s) * 64 + lane]); }
        gu_publish(a, ln, u ? t1 : t, acc);
    }
}

// ---------------------------------------------------------------- phase 4: down units
// A unit is row group rg (256 output rows) of one pair-slot: wave w owns rows rg * 256 + 32 w .. + 31 (two 16-row sets of
// one 64-row group). Once its waves have finished their gate/up passes, a workgroup stages the h of all its units at
// once into the LDS of the token rows (no longer needed): row 2 k + i = token i of its unit k, wave w quantising Q8_K
// block w of every row. After one barrier each wave computes its rows of every unit without further synchronisation.
struct DnUnit { int mi, s, c, rg; };

__device__ __forceinline__ bool dn_unit(const RT & rt, int u, int nps, int nact, int P, int n, DnUnit & d) {
    const int ps = u % nps, mi = rt.ps_mi[ps], sc = rt.ps_s[ps];
    d.mi = mi; d.s = sc & 0xFFFF; d.c = sc >> 16; d.rg = u / nps;
    return (mi == SH || (unsigned) mi < (unsigned) nact) && (d.c == 1 || d.c == 2) && d.s + d.c <= P + n;
}
constexpr int HROWS = DMAX_N * GG::XROW / GD::XROW;   // staged h rows that fit the token rows' LDS (28)
constexpr int DN_KC = HROWS / 2;                      // units staged per chunk

// the workgroup's units blockIdx.x, + G, .. < nps * NDN; returns their number
__device__ __forceinline__ int down_phase(const DArgs & a, lds_t lds, const Lane ln, int wave, int nps, int nact, int P) {
#pragma clang fp contract(off)
    const RT rt(lds);
    const int G = gridDim.x, total = nps * NDN, lane = lane_id();
    const int K = (int) blockIdx.x < total ? (total - 1 - (int) blockIdx.x) / G + 1 : 0;
    LK_LOCAL unsigned * wok = reinterpret_cast<LK_LOCAL unsigned *>(lds + L_CTL) + 8;   // [DW] per-wave staging results
    const uint32_t lq = (uint32_t) ln.q * 4096 + 16 * ln.r, ld = (uint32_t) ln.q * 128 + 2 * ln.r;
    // this wave's weight bases (qs, d) of unit k (round-robin index); false for an invalid table entry
    auto unit_bases = [&](int k, DnUnit & d, const uint8_t * & qb, const uint8_t * & db) -> bool {
        if (!dn_unit(rt, (int) blockIdx.x + k * G, nps, nact, P, a.n, d)) { return false; }
        const int e = d.mi != SH ? rt.act_e[d.mi] : 0;
        const uint8_t * base = uniform_ptr(d.mi != SH ? a.down + (size_t) e * a.estride : a.sh_down);
        const int g64 = d.rg * (DN_ROWS / 64) + (wave >> 1), sub = (wave & 1) * 2;
        qb = base + (size_t) g64 * GD::NB * 4096 + sub * 256;
        db = base + (size_t) (DE / 64) * GD::NB * 4096 + (size_t) g64 * GD::NB * 128 + sub * 32;
        return true;
    };
    RowStream<GD::BPQ, 2, DN_PD> rs;
    for (int k0 = 0; k0 < K; k0 += DN_KC) {
        const int kn = K - k0 < DN_KC ? K - k0 : DN_KC;
        __syncthreads();   // the token rows (or the previous chunk's h) are no longer read
        // the chunk's first unit: its first DN_PRE steps stream in while the h words are polled and staged
        DnUnit d0; const uint8_t * qb0 = nullptr, * db0 = nullptr;
        if (unit_bases(k0, d0, qb0, db0)) { rs.template prologue<0, DN_PRE>(qb0, db0, lq, ld); }
        TRACE(wave, 24);
        // stage: rows r0 .. r0 + 3 at a time, all their words in flight together
        bool ok = true;
        for (int r0 = 0; r0 < 2 * kn && ok; r0 += 4) {
            uint64_t w[4][4];
            int src[4];
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int row = r0 + rr, k = k0 + row / 2, i = row & 1;
                DnUnit d;
                src[rr] = row < 2 * kn && dn_unit(rt, (int) blockIdx.x + k * G, nps, nact, P, a.n, d) && i < d.c ? d.s + i : -1;
            }
            auto issue = [&]() {
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    if (src[rr] >= 0) {
                        const uint64_t * p = a.th + (size_t) src[rr] * DH + wave * QK + 4 * lane;
#pragma unroll
                        for (int q4 = 0; q4 < 4; ++q4) { w[rr][q4] = ld_tag(p + q4); }
                    }
                }
            };
            issue();
            int it = 0;
            for (; it < POLL_MAX; ++it) {
                bool v = true;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) { v = v && (src[rr] < 0 || tag_ok(w[rr][q4], a.epoch)); }
                }
                if (__ballot(!v) == 0) { break; }
                __builtin_amdgcn_s_sleep(1);
                issue();
            }
            if (it == POLL_MAX) { ok = false; break; }
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                if (src[rr] >= 0) {
                    const float xs[4] = { tag_val(w[rr][0]), tag_val(w[rr][1]), tag_val(w[rr][2]), tag_val(w[rr][3]) };
                    float dq; const uint32_t packed = q8k_lane(xs, dq);
                    lds_t hrow = lds + L_XS + (r0 + rr) * GD::XROW;
                    *reinterpret_cast<LK_LOCAL uint32_t *>(hrow + wave * GD::XBLK + staged_word(lane)) = packed;
                    if (lane == 0) { reinterpret_cast<LK_LOCAL float *>(hrow + GD::NB * GD::XBLK)[wave] = dq; }
                }
            }
        }
        if (lane == 0) { wok[wave] = ok ? 1u : 0u; }
        __syncthreads();   // every wave's blocks of every row are staged
        bool all_ok = true;
#pragma unroll
        for (int w2 = 0; w2 < DW; ++w2) { all_ok = all_ok && wok[w2] != 0u; }
        TRACE(wave, 25);
        if (!all_ok) { report(a, 1); continue; }
        for (int k = 0; k < kn; ++k) {
            DnUnit d; const uint8_t * qb, * db;
            if (!unit_bases(k0 + k, d, qb, db)) { report(a, 1); continue; }
            // one token per pass: the second pass re-reads the unit's weights from L2
            for (int i = 0; i < d.c; ++i) {
                if (k > 0 || i > 0) { rs.prologue(qb, db, lq, ld); } else { rs.template prologue<DN_PRE, DN_PD>(qb, db, lq, ld); }
                float acc[2];
                rs.run_dpp<GD>(qb, db, lq, ld, ln.tr, (const uint8_t *) (lds + L_XS + (2 * k + i) * GD::XROW), ln.q, ln.r, acc);
                if (ln.q == 0) {
#pragma unroll
                    for (int r2 = 0; r2 < 2; ++r2) { st_tag(a.to + (size_t) (d.s + i) * DE + d.rg * DN_ROWS + wave * 32 + r2 * 16 + ln.r, a.epoch, 0.125f * acc[r2]); }
                }
            }
        }
        TRACE(wave, 26);
    }
    return K;
}

// ---------------------------------------------------------------- phase 5: combine
// rows cu * 256 .. + 255 of every token: y = sum_k w_k o_k in k order + the shared expert's o (+ the residual when
// given, the reference combine's moe + shared + ffn_inp order, fl.cu:366-372). Thread (row, t0) polls
// the tagged o words of its tokens t0, t0 + 2, .. all at once (one memory round trip per poll); false on timeout
__device__ __forceinline__ bool combine_unit(const DArgs & a, lds_t lds, int cu, int P) {
#pragma clang fp contract(off)
    constexpr int TS = DNT / DN_ROWS, CT = DMAX_N / TS;   // token stride, tokens per thread
    const RT rt(lds);
    const int rr = cu * DN_ROWS + (threadIdx.x & (DN_ROWS - 1)), t0 = threadIdx.x / DN_ROWS;
    uint64_t wv[CT][MAXK + 1];
    auto used = [&](int c, int k) { return t0 + c * TS < a.n && (k < a.keep || k == MAXK); };
    auto issue = [&]() {
#pragma unroll
        for (int c = 0; c < CT; ++c) {
            const int tok = t0 + c * TS;
#pragma unroll
            for (int k = 0; k <= MAXK; ++k) {
                if (used(c, k)) { wv[c][k] = ld_tag(a.to + (size_t) (k < MAXK ? rt.inv[tok * a.keep + k] : P + tok) * DE + rr); }
            }
        }
    };
    issue();
    int it = 0;
    for (; it < POLL_MAX; ++it) {
        bool v = true;
#pragma unroll
        for (int c = 0; c < CT; ++c) {
#pragma unroll
            for (int k = 0; k <= MAXK; ++k) { v = v && (!used(c, k) || tag_ok(wv[c][k], a.epoch)); }
        }
        if (__ballot(!v) == 0) { break; }
        __builtin_amdgcn_s_sleep(1);
        issue();
    }
    if (it == POLL_MAX) { return false; }
    if (a.ext_sel) {   // fl_moe's combine: the distinct ids ascending, moe = their weighted sum, y = (moe + shared) + resid
#pragma unroll
        for (int c = 0; c < CT; ++c) {
            const int tok = t0 + c * TS;
            if (tok >= a.n) { continue; }
            const LK_LOCAL int * xe = reinterpret_cast<const LK_LOCAL int *>(lds + L_EXT) + tok * EXT_TOK;
            const LK_LOCAL float * xw = reinterpret_cast<const LK_LOCAL float *>(xe + MAXK);
            const int cnt = xe[2 * MAXK];
            float v = 0.f;
            for (int q = 0; q < cnt; ++q) {
                const int kf = xe[q];
                float ov = 0.f;
#pragma unroll
                for (int k = 0; k < MAXK; ++k) { ov = k == kf ? tag_val(wv[c][k]) : ov; }
                v = v + xw[q] * ov;
            }
            gptr(a.moe_out)[(size_t) tok * DE + rr] = v;
            gptr(a.y)[(size_t) tok * DE + rr] = (v + tag_val(wv[c][MAXK])) + gptr(a.resid)[(size_t) tok * DE + rr];
            if (a.o_out) {   // the slots' outputs by pair index (token * keep + k)
#pragma unroll
                for (int k = 0; k < MAXK; ++k) { if (k < a.keep) { gptr(a.o_out)[(size_t) (tok * a.keep + k) * DE + rr] = tag_val(wv[c][k]); } }
            }
        }
        return true;
    }
#pragma unroll
    for (int c = 0; c < CT; ++c) {
        const int tok = t0 + c * TS;
        if (tok < a.n) {
            float mv = tag_val(wv[c][0]) * rt.wts[tok * a.keep];
#pragma unroll
            for (int k = 1; k < MAXK; ++k) { if (k < a.keep) { mv = mv + tag_val(wv[c][k]) * rt.wts[tok * a.keep + k]; } }
            float yv = mv + tag_val(wv[c][MAXK]);
            if (a.resid) { yv = yv + gptr(a.resid)[(size_t) tok * DE + rr]; }
            gptr(a.y)[(size_t) tok * DE + rr] = yv;
        }
    }
    return true;
}

// ---------------------------------------------------------------- the kernel
__global__ void __launch_bounds__(DNT, 1) k_moe_decode(const DecodeArgs args) {
    // The arguments are read in place in the kernarg segment (the only explicit argument, at offset 0) through a
    // constant-space pointer, so every field is a scalar load. Naming `args` itself would make a private copy.
    (void) sizeof(args);
    const DArgs & a = *(const DArgs *) __builtin_amdgcn_kernarg_segment_ptr();
    extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];
    const lds_t lds = (lds_t) dyn_lds;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
    const int G = gridDim.x, n = a.n, P = n * a.keep;
    // [0] waves with tokens and tables staged, [1] selections done, [2] routing ready (1 ok, 2 failed), [3] a wait failed,
    // [4] early shared task: waves done
    LK_LOCAL unsigned * ctl = reinterpret_cast<LK_LOCAL unsigned *>(lds + L_CTL);
    Lane ln;
    ln.r = lane & 15; ln.q = lane >> 4;   // lane 16 q + r: row r, block quarter q
    ln.tr = tab_word_grid(lds_addr(dyn_lds), lane);   // table base (64 KB aligned: the tables open the LDS) | copy

    // 1. table copy in flight; router (the whole workgroup)
    TRACE(wave, 0);
    if (lds_addr(dyn_lds) & 0xFFFFu) { report(a, 4); return; }   // table addressing needs a 64 KB aligned base
    if (threadIdx.x < 8) { ctl[threadIdx.x] = 0; }
    tables_dma(lds, a.tab, wave);
    __syncthreads();   // the hand-off words are clear
    if (a.prenorm) { norm_phase(a, lds, wave); }
    if (!a.ext_sel) {   // with the caller's picks there is no routing
        for (int e = blockIdx.x; e < a.n_exp; e += G) { router_phase(a, lds, wave, e); }
    }
    TRACE(wave, 2);

    // 2. wave t polls token t's probabilities while all waves quantise the tokens; wave t then selects token t's experts
    //    (every workgroup redundantly) and the last selecting wave builds the dispatch and opens the task phase. Waves
    //    without a token run the shared expert's gate/up meanwhile.
    const bool pre = n < DW;
    float bv[4]; uint64_t pw[4];
    if (wave < n && !a.ext_sel) { load_bias(a.bias, a.n_exp, bv); probs_issue(a, wave, pw); }
    TRACE(wave, 9);
    if (a.xqx) {
        if (!xcd_quant(a, lds, wave)) { report(a, 64); }
    } else {
        local_quant(a, lds, wave);
    }
    TRACE(wave, 10);
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): this wave's table loads have landed in LDS
    lds_arrive(ctl + 0, DW);              // [0] counts the waves whose tokens and table share are in LDS
    TRACE(wave, 1);
    if (wave < n) {
        // the selecting waves run ahead of the streaming ones on their SIMDs until the dispatch is built
        __builtin_amdgcn_s_setprio(3);
        const RT rt(lds);
        if (a.ext_sel) {
            // the caller's picks of token `wave`; lane 0 also lists its distinct ids ascending, each with its weights
            // summed in k order and its first k, for the combine (zero sums are dropped, as fl_moe does)
            const int kk = a.keep, b0 = wave * kk;
            if (lane < kk) { rt.sel[b0 + lane] = gptr(a.ext_sel)[b0 + lane]; rt.wts[b0 + lane] = gptr(a.ext_w)[b0 + lane]; }
            lds_visible();
            if (lane == 0) {
                LK_LOCAL int * xe = reinterpret_cast<LK_LOCAL int *>(lds + L_EXT) + wave * EXT_TOK;
                LK_LOCAL float * xw = reinterpret_cast<LK_LOCAL float *>(xe + MAXK);
                int prev = -1, cnt = 0;
                for (int it = 0; it < MAXK; ++it) {
                    int m = 0x7fffffff;
                    for (int k = 0; k < kk; ++k) { const int v = rt.sel[b0 + k]; if (v > prev && v < m) { m = v; } }
                    if (m == 0x7fffffff) { break; }
                    float wt = 0.f; int kf = -1;
                    for (int k = 0; k < kk; ++k) { if (rt.sel[b0 + k] == m) { wt += rt.wts[b0 + k]; if (kf < 0) { kf = k; } } }
                    prev = m;
                    if (wt == 0.f) { continue; }
                    xe[cnt] = kf; xw[cnt] = wt; ++cnt;
                }
                xe[2 * MAXK] = cnt;
            }
            TRACE(wave, 3);
        } else {
            float pv[4];
            const bool ok = probs_wait(a, wave, pw, pv);
            TRACE(wave, 3);
            if (!ok) { report(a, 2); }
            if (ok) {
                // with --share-experts every pick first (stride topk), the keep across the rows then runs in the
                // dispatch wave
                const int ks = a.share ? a.topk : a.keep;
                int * so = (int *) (rt.sel + wave * ks); float * wo = (float *) (rt.wts + wave * ks);
                // DeepSeek's rule with every pick kept: the threshold selection (select_ds8, the same picks and
                // weights in fewer dependent steps), its scratch in the early shared task's area (unused: no wave is
                // without a token)
                bool done = false;
                if (!pre && a.n_exp == 256 && a.n_group == 8 && a.topk_group == 4 && a.topk == MAXK && ks == MAXK) {
                    done = select_ds8(pv, bv, a.scale, reinterpret_cast<LK_LOCAL uint32_t *>(lds + L_PRE) + wave * 112, so, wo);
                }
                if (!done) {
                    select_token_p<false>(pv, bv, a.n_exp, a.n_group, a.topk_group, a.topk, a.scale, nullptr, so, wo, ks,
                                          a.share ? 0.f : a.renorm);
                }
            } else if (lane == 0) {
                __hip_atomic_fetch_or(ctl + 3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
        TRACE(wave, 4);
        if (lds_arrive(ctl + 1, (unsigned) n)) {
            const bool all_ok = __builtin_amdgcn_readfirstlane(__hip_atomic_load(ctl + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) == 0;
            if (a.share && all_ok) {   // the rows' kept picks, in place ([n][topk] -> [n][keep]); the set U in the EXT area
                keep_share_rows(rt.sel, rt.wts, n, a.topk, a.keep, a.renorm, rt.sel, rt.wts, reinterpret_cast<LK_LOCAL unsigned *>(lds + L_EXT), true);
                lds_visible();
            }
            dispatch_wave(a, lds, all_ok ? P : 0);
            const bool staged = lds_wait_count(ctl + 0, DW);   // the tasks read the tables and the tokens
            lds_visible();
            if (lane == 0) { __hip_atomic_store(ctl + 2, all_ok && staged ? 1u : 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
            TRACE(wave, 6);
        }
        __builtin_amdgcn_s_setprio(0);
    } else if (pre && lds_wait_count(ctl + 0, DW)) {   // the shared expert's pair-slots k: tokens 2k, 2k + 1
        if (n <= 2 && G >= NGU) {
            if (blockIdx.x < NGU) { pre_shared_split(a, lds, ln, wave, P, ctl + 4); }
        } else {
            gate_up_stream<GU_PD>(a, lds, ln, blockIdx.x * (DW - n) + (wave - n), (DW - n) * G, ((n + 1) >> 1) * NGU, true, 0, P, 0);
        }
    }
    const unsigned ready = lds_wait(ctl + 2);
    TRACE(wave, 5);
    // a failed routing wait leaves every later phase without its inputs: all waves leave (the error is reported)
    if (ready != 1) { if (ready == 0) { report(a, 8); } return; }

    // 3. gate/up tasks (pair-slot, 8 h rows): task tk on workgroup tk / DW % G, wave tk % DW, so a workgroup streams
    //    whole 64-row groups; the shared expert's pair-slots come first unless the early tasks covered them
    const RT rt(lds);
    const int nact = *rt.nact, nps = *rt.nps, ps0 = pre ? n : 0;
    const int t_gu = (nps - ps0) * NGU;
    TRACE(wave, 8);
    const int ntask = gate_up_stream<GU_PD>(a, lds, ln, blockIdx.x * DW + wave, G * DW, t_gu, false, ps0, P, nact);
    TRACE(wave, 7);

    // 4. down units (pair-slot, 256 rows), round-robin over the workgroups: unit u = row group u / nps of pair-slot u % nps
    const int nunit = down_phase(a, lds, ln, wave, nps, nact, P);

    // 5. combine units on the last workgroups
    for (int cu = G - 1 - blockIdx.x; cu < NDN; cu += G) {
        TRACE(wave, 56);
        if (!combine_unit(a, lds, cu, P)) { report(a, 16); }
        TRACE(wave, 58);
    }
    if (blockIdx.x == 0 && wave == DW - 1 && !a.ext_sel) { routing_outputs(a, lds, P); }
#ifdef LOKI_TRACE
    if (lane == 0) { g_trace[(blockIdx.x * DW + wave) * TRACE_SLOTS + 63] = (uint64_t) ntask | ((uint64_t) nunit << 16) | ((uint64_t) t_gu << 32); }
#endif
}

size_t decode_lds_bytes() { return DEC_LDS; }

// workgroups of k_moe_decode that can be resident at once on `ncu` CUs (0: the single launch is unavailable)
hipError_t decode_init(int ncu, int * grid) {
    *grid = 0;
    hipError_t e = hipFuncSetAttribute((const void *) k_moe_decode, hipFuncAttributeMaxDynamicSharedMemorySize, DEC_LDS);
    if (e != hipSuccess) { return e; }
    int per = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void *) k_moe_decode, DNT, DEC_LDS);
    if (e != hipSuccess) { return e; }
    *grid = per >= 1 ? ncu : 0;   // one workgroup per CU: the tables and token rows fill most of the LDS
    return hipSuccess;
}

bool decode_rule_ok(int n_exp, int n_group) {   // the selection's DPP group path: 4 experts per lane, 1..16 lanes per group
    if (n_exp < 1 || n_exp > NEXP_MAX || n_group < 1 || n_exp % n_group) { return false; }
    const int per = n_exp / n_group, lpg = per / 4;
    return per % 4 == 0 && lpg >= 1 && lpg <= 16 && (lpg & (lpg - 1)) == 0;
}

hipError_t launch_moe_decode(const DecodeArgs & a, int grid, bool cooperative, hipStream_t st) {
    if (a.ext_sel && (!a.ext_w || !a.moe_out || !a.resid || a.prenorm)) { return hipErrorInvalidValue; }   // the caller's picks
    if (a.n < 1 || a.n > DMAX_N || a.topk < 1 || a.topk > MAXK || a.keep < 1 || a.keep > a.topk ||
        (!a.ext_sel && !decode_rule_ok(a.n_exp, a.n_group)) || a.E != DE || a.H != DH || grid < 1 || !a.th || !a.to || !a.tlogits ||
        a.kdown != 0) {   // IQ2_XXS matrices only
        return hipErrorInvalidValue;
    }
    if (!cooperative) {   // one workgroup per CU fits the occupancy; co-residency is assumed, waits stay bounded
        k_moe_decode<<<grid, DNT, DEC_LDS, st>>>(a);
        return hipGetLastError();
    }
    DecodeArgs arg = a;
    void * params[] = { &arg };
    return hipLaunchCooperativeKernel((const void *) k_moe_decode, dim3(grid), dim3(DNT), params, DEC_LDS, st);
}

}  // namespace lk
