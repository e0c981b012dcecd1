// moe_decode.hip -- the whole MoE block for a decode batch (n <= 8 tokens) in one cooperative launch.
//
// Reference path (src/fused_layer.cu): router_probs + router_topk (:313-332, launched :506), a host round-trip for the
// routing (fl_fetch :587-598, eng:793-818), then per fl_moe (:599-612) quant_x, tc_matvec gate/up, swiglu_q8,
// tc_matvec down and moe_combine as separate launches. At batch 1-8 every one of those launches is latency-bound, so
// here one workgroup per CU (all resident: cooperative launch) runs the block end to end:
//   1. workgroup b computes the router logits of expert b for every token (the fp64 chunk-and-tree contract) and
//      publishes each as an epoch-tagged 64-bit word; then it copies the codebook/sign table image into LDS and
//      quantises the n token rows to Q8_K (staged layout of moe_device.h);
//   2. every workgroup polls the tagged logits, selects each token's experts (select_token, one wave per token) and
//      builds the dispatch (stable counting sort of the n * topk pairs) in its own LDS -- redundant, but cheaper than
//      another device-wide hand-off. Waves without a token meanwhile run the shared expert's gate/up tasks, which need
//      no routing;
//   3. tasks round-robin over all waves of the grid: gate/up tasks (expert slot, 16 rows, matrix) -- the second task of
//      a (gate, up) pair forms h = silu(g) * u, the last of a 256-row block quantises it to Q8_K, the last block of an
//      expert raises the expert's h flag -- then down tasks (expert slot, 32 rows) that prefetch their weights, wait for
//      the expert's h flag, and write o; the last expert of a row group computes y = sum_k w_k o_k (k order) + shared.
// Arithmetic is that of the per-pass kernels (same device functions), so y is bit-identical to theirs and to the CPU
// checker. Flags hold the launch's epoch (no clearing between launches); counters reset themselves. Every wait is
// bounded: a timeout sets *err and the wave skips the task, so the grid always drains.
#include "moe_device.h"
#include "moe_kernels.h"

namespace lk {

constexpr int DW = 8, DNT = DW * 64;   // waves / threads per workgroup
constexpr int DMAX_N = 8, DMAX_P = DMAX_N * MAXK;
constexpr int SH = NEXP_MAX;           // counter / flag index of the shared expert
using GG = Geo<7>;                     // gate/up rows: K = 7168
using GD = Geo<2>;                     // down rows: K = 2048
constexpr int DE = GG::K, DH = GD::K;
constexpr int NGU = DH / 16;           // gate/up tasks per matrix (16 rows)
constexpr int DRPL = 2;                // down: row sets of 16 per task
constexpr int NDN = DE / (16 * DRPL);  // down tasks per expert
constexpr int GU_PD = 3, GU1_PD = 6, DN_PD = 3;   // blocks in flight per lane (single-token gate/up: deeper)

// LDS layout
constexpr int L_XS = TAB_BYTES;                                   // staged Q8_K tokens
constexpr int L_DST = L_XS + DMAX_N * GG::XROW;                   // per-wave down staging / router sums / selection scratch
constexpr int DST_BYTES = DW * GD::XROW;
constexpr int L_RT = L_DST + DST_BYTES;                           // routing tables
constexpr int RT_INTS = 4 * DMAX_P + 3 * (DMAX_P + 1) + 1;
constexpr int L_CTL = L_RT + RT_INTS * 4;                         // workgroup hand-off words
constexpr int DEC_LDS = L_CTL + 16;
static_assert(DEC_LDS <= 160 * 1024, "LDS budget");
static_assert(DMAX_N * 64 * 8 <= DST_BYTES && DW * (NEXP_MAX + 2 * 64) * 4 <= DST_BYTES, "scratch overlays");

typedef LK_LOCAL uint8_t * lds_t;

struct RT {   // routing of the launch, in LDS
    LK_LOCAL int * sel; LK_LOCAL float * wts; LK_LOCAL int * perm, * inv, * act_e, * act_s0, * act_cnt, * nact;
    __device__ RT(lds_t lds) {
        LK_LOCAL int * b = reinterpret_cast<LK_LOCAL int *>(lds + L_RT);
        sel = b; wts = reinterpret_cast<LK_LOCAL float *>(b + DMAX_P); perm = b + 2 * DMAX_P; inv = b + 3 * DMAX_P;
        act_e = b + 4 * DMAX_P; act_s0 = act_e + DMAX_P + 1; act_cnt = act_s0 + DMAX_P + 1; nact = act_cnt + DMAX_P + 1;
    }
};

__device__ __forceinline__ void report(int * err, int code) { if (lane_id() == 0) { __hip_atomic_fetch_or(gptr(err), code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); } }

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

// Timeline probe for tuning builds (-DLOKI_TRACE): per wave, 64-bit s_memrealtime stamps (100 MHz) at the phase
// boundaries (slots 0-5, 30) and at the start and end of each of the first 12 tasks (slots 6-29); slot 31 = task count.
#ifdef LOKI_TRACE
constexpr int TRACE_SLOTS = 32;
__device__ uint64_t g_trace[1024 * DW * TRACE_SLOTS];
#define TRACE(wave, slot) do { if (lane_id() == 0) { g_trace[(blockIdx.x * DW + (wave)) * TRACE_SLOTS + (slot)] = __builtin_amdgcn_s_memrealtime(); } } while (0)
extern "C" hipError_t fl_trace_copy(void * host, size_t bytes) { return hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace), bytes); }
extern "C" hipError_t fl_trace_clear() {
    void * p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(g_trace));
    return e == hipSuccess ? hipMemset(p, 0, sizeof(g_trace)) : e;
}
#else
#define TRACE(wave, slot) do { } while (0)
#endif

// ---------------------------------------------------------------- phase 1: Q8_K of the token rows into LDS
__device__ __noinline__ void quant_tokens(const DecodeArgs & a, lds_t lds, int wave) {
    const int lane = lane_id(), nblk = a.n * GG::NB;
    constexpr int B = 8;   // blocks per batch: their loads are all issued before the first is used
    for (int b0 = wave; b0 < nblk; b0 += DW * B) {
        float4 v[B];
#pragma unroll
        for (int k = 0; k < B; ++k) {
            const int b = b0 + k * DW;
            if (b < nblk) { v[k] = gloadf4(a.x + (size_t) (b / GG::NB) * DE + (size_t) (b % GG::NB) * QK + 4 * lane); }
        }
#pragma unroll
        for (int k = 0; k < B; ++k) {
            const int b = b0 + k * DW;
            if (b < nblk) {
                const int t = b / GG::NB, j = b % GG::NB;
                const float xs[4] = { v[k].x, v[k].y, v[k].z, v[k].w };
                float d; const uint32_t packed = q8k_lane(xs, d);
                lds_t row = lds + L_XS + t * GG::XROW;
                *reinterpret_cast<LK_LOCAL uint32_t *>(row + j * GG::XBLK + staged_word(lane)) = packed;
                if (lane == 0) { reinterpret_cast<LK_LOCAL float *>(row + GG::NB * GG::XBLK)[j] = d; }
                if (blockIdx.x == 0) {   // the layer's xq / xd
                    gptr(reinterpret_cast<uint32_t *>(a.xq + (size_t) t * DE + (size_t) j * QK))[lane] = packed;
                    if (lane == 0) { gptr(a.xd)[(size_t) t * GG::NB + j] = d; }
                }
            }
        }
    }
}

// ---------------------------------------------------------------- phase 2: router logits of expert e for token t
// the contract of moe_device.h (256 in-order chunk sums, pairwise tree, one rounding); one wave per (expert, token)
// Router logits of expert e for all n tokens by the whole workgroup. Thread (quarter w = wave & 3, lane) owns chunk
// 64 w + lane (K/256 = 28 values) of every token t with t % 2 == wave / 4, so each thread issues its 7 + 7 * (tokens)
// 16-byte loads at once. Tree levels 1-6 run inside the wave (one chunk per lane), 7-8 combine the four quarters'
// totals through LDS. Each logit is published as one 64-bit word {epoch, fp32 bits}: consumers poll the words
// themselves, so no counter, flag or store-completion wait sits between the router and the selection.
__device__ __noinline__ void router_phase(const DecodeArgs & a, lds_t lds, int wave, int e) {
#pragma clang fp contract(off)
    constexpr int L4 = DE / 1024;   // float4 per chunk (7)
    const int lane = lane_id(), qt = wave & 3, half = wave >> 2, c = qt * 64 + lane;
    LK_LOCAL double * part = reinterpret_cast<LK_LOCAL double *>(lds + L_DST);   // [token][quarter]
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
        __hip_atomic_store(gptr(a.tlogits + o), ((uint64_t) a.epoch << 32) | __builtin_bit_cast(uint32_t, l), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        gptr(a.logits)[o] = l;   // the layer's logits (read after the launch)
    }
    __syncthreads();   // part[] is reused by the next expert
}

// token t's logits of the lane's experts 4 lane + j, once every word carries this launch's epoch; false on timeout
__device__ __forceinline__ bool wait_logits(const DecodeArgs & a, int t, float (&lg)[4]) {
    const int lane = lane_id();
    for (int it = 0; it < (1 << 20); ++it) {
        bool ok = true;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = 4 * lane + j;
            if (e < a.n_exp) {
                const uint64_t w = __hip_atomic_load(gptr(a.tlogits + (size_t) t * a.n_exp + e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = ok && (uint32_t) (w >> 32) == a.epoch;
                lg[j] = __builtin_bit_cast(float, (uint32_t) w);
            } else {
                lg[j] = 0.f;
            }
        }
        if (__ballot(!ok) == 0) { return true; }
        __builtin_amdgcn_s_sleep(2);
    }
    return false;
}

// ---------------------------------------------------------------- phase 3: dispatch of the n * topk pairs (one wave)
// stable counting sort by expert: pos(i) = #{pairs with a lower expert} + #{earlier pairs with the same expert}
__device__ __noinline__ void dispatch_wave(const DecodeArgs & a, lds_t lds, int P) {
    const RT rt(lds);
    const int lane = lane_id();
    const bool valid = lane < P;
    const int e = valid ? rt.sel[lane] : -1;
    uint64_t match = __ballot(valid);
#pragma unroll
    for (int b = 0; b < 9; ++b) {
        const bool bit = valid && ((e >> b) & 1);
        const uint64_t ones = __ballot(bit);
        match &= bit ? ones : ~ones;
    }
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int rank = __popcll(match & below);
    const uint64_t first = __ballot(valid && rank == 0);
    int less = 0, dless = 0;
    for (int j = 0; j < P; ++j) {
        const int ej = rt.sel[j];
        less += ej < e ? 1 : 0;
        dless += (ej < e && ((first >> j) & 1ull)) ? 1 : 0;
    }
    const int pos = less + rank;
    if (valid) {
        rt.perm[pos] = lane; rt.inv[lane] = pos;
        if (rank == 0) { rt.act_e[dless] = e; rt.act_s0[dless] = less; rt.act_cnt[dless] = __popcll(match); }
    }
    if (lane == 0) { *rt.nact = __popcll(first); }
    if (blockIdx.x == 0) {   // the layer's routing outputs
        if (valid) { gptr(a.perm)[pos] = lane; gptr(a.inv)[lane] = pos; gptr(a.sel)[lane] = e; gptr(a.wts)[lane] = rt.wts[lane]; }
        if (valid && rank == 0) { gptr(a.act)[dless] = e; }
        if (lane == 0) { *gptr(a.nact) = __popcll(first); }
        for (int x = lane; x <= a.n_exp; x += 64) {
            int lt = 0, eq = 0;
            for (int j = 0; j < P; ++j) { const int ej = rt.sel[j]; lt += ej < x ? 1 : 0; eq += ej == x ? 1 : 0; }
            gptr(a.offsets)[x] = lt;
            if (x < a.n_exp) { gptr(a.counts)[x] = eq; }
        }
    }
}

// ---------------------------------------------------------------- phase 4 tasks
struct Lane { int q, r; uint32_t tr, lq, ld; };

__device__ __noinline__ void gate_up_task(const DecodeArgs & a, lds_t lds, const Lane & ln, int mi, int g, int mat, int P) {
#pragma clang fp contract(off)
    const RT rt(lds);
    const bool routed = mi != SH;
    const int e = routed ? rt.act_e[mi] : 0;
    const int s0 = routed ? rt.act_s0[mi] : P, cnt = routed ? rt.act_cnt[mi] : a.n;
    const uint8_t * base = routed ? (mat ? a.up : a.gate) + (size_t) e * a.estride : (mat ? a.sh_up : a.sh_gate);
    const uint8_t * qb = base + (size_t) (g >> 2) * GG::NB * 4096 + (g & 3) * 256;
    const uint8_t * db = base + (size_t) (DH / 64) * GG::NB * 4096 + (size_t) (g >> 2) * GG::NB * 128 + (g & 3) * 32;
    float * outv = mat ? a.u : a.g;
    const int row = g * 16 + ln.r;
    for (int tok = 0; tok < cnt;) {
        if (cnt - tok >= 2) {
            RowStream<GG::BPQ, 1, GU_PD> rs;
            rs.prologue(qb, db, ln.lq, ln.ld);
            const uint8_t * xr[2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int s = s0 + tok + u;
                xr[u] = (const uint8_t *) (lds + L_XS + (routed ? rt.perm[s] / a.topk : s - P) * GG::XROW);
            }
            float acc[1][2];
            rs.run<2, GG>(qb, db, ln.lq, ln.ld, ln.tr, xr, ln.q, acc);
            if (ln.q == 0) {
#pragma unroll
                for (int u = 0; u < 2; ++u) { st_agent(outv + (size_t) (s0 + tok + u) * DH + row, 0.125f * acc[0][u]); }
            }
            tok += 2;
        } else {
            RowStream<GG::BPQ, 1, GU1_PD> rs;
            rs.prologue(qb, db, ln.lq, ln.ld);
            const int s = s0 + tok;
            const uint8_t * xr[1] = { (const uint8_t *) (lds + L_XS + (routed ? rt.perm[s] / a.topk : s - P) * GG::XROW) };
            float acc[1][1];
            rs.run<1, GG>(qb, db, ln.lq, ln.ld, ln.tr, xr, ln.q, acc);
            if (ln.q == 0) { st_agent(outv + (size_t) s * DH + row, 0.125f * acc[0][0]); }
            tok += 1;
        }
    }
    // the second task of the (gate, up) pair forms h for the pair's 16 rows
    if (!arrive_last(a.cnt + CNT_PAIR + mi * NGU + g, 2u)) { return; }
    const int lane = lane_id();
    for (int i = lane; i < cnt * 16; i += 64) {
        const size_t o = (size_t) (s0 + i / 16) * DH + g * 16 + i % 16;
        st_agent(a.h + o, det_silu(ld_agent(a.g + o)) * ld_agent(a.u + o));
    }
    // the last of the 16 pairs of a 256-row block quantises that block of h for every slot of the expert
    const int hb = g / 16;
    if (!arrive_last(a.cnt + CNT_HB + mi * (DH / QK) + hb, 16u)) { return; }
    for (int s = s0; s < s0 + cnt; ++s) {
        const float * hbp = a.h + (size_t) s * DH + hb * QK;
        const float xs[4] = { ld_agent(hbp + 4 * lane), ld_agent(hbp + 4 * lane + 1), ld_agent(hbp + 4 * lane + 2), ld_agent(hbp + 4 * lane + 3) };
        float d; const uint32_t packed = q8k_lane(xs, d);
        st_agent_u32(reinterpret_cast<uint32_t *>(a.hq + (size_t) s * DH + hb * QK) + lane, packed);
        if (lane == 0) { st_agent(a.hd + (size_t) s * (DH / QK) + hb, d); }
    }
    // the last block of the expert raises its flag
    if (!arrive_last(a.cnt + CNT_HQ + mi, (unsigned) (DH / QK))) { return; }
    if (lane == 0) { st_agent_u32(a.flags + FLAG_H + mi, a.epoch); }
}

__device__ __noinline__ void down_task(const DecodeArgs & a, lds_t lds, const Lane & ln, int wave, int mi, int g, int P, int nm) {
#pragma clang fp contract(off)
    const RT rt(lds);
    const bool routed = mi != SH;
    const int e = routed ? rt.act_e[mi] : 0;
    const int s0 = routed ? rt.act_s0[mi] : P, cnt = routed ? rt.act_cnt[mi] : a.n;
    const uint8_t * base = routed ? a.down + (size_t) e * a.estride : a.sh_down;
    const int rg = (g * 32) >> 6, sub = ((g * 32) & 63) >> 4;
    const uint8_t * qb = base + (size_t) rg * GD::NB * 4096 + sub * 256;
    const uint8_t * db = base + (size_t) (DE / 64) * GD::NB * 4096 + (size_t) rg * GD::NB * 128 + sub * 32;
    uint8_t * xw = (uint8_t *) (lds + L_DST + wave * GD::XROW);
    RowStream<GD::BPQ, DRPL, DN_PD> rs;
    rs.prologue(qb, db, ln.lq, ln.ld);   // the weights do not depend on h: in flight while the wave waits
    if (!wait_flag(a.flags + FLAG_H + mi, a.epoch)) { report(a.err, 1); return; }
    for (int s = s0; s < s0 + cnt; ++s) {
        if (s > s0) { rs.prologue(qb, db, ln.lq, ln.ld); }
        __builtin_amdgcn_wave_barrier();
        stage_row_agent<GD>(xw, a.hq + (size_t) s * DH, a.hd + (size_t) s * (DH / QK));
        lds_visible();
        const uint8_t * xr[1] = { xw };
        float acc[DRPL][1];
        rs.run<1, GD>(qb, db, ln.lq, ln.ld, ln.tr, xr, ln.q, acc);
        if (ln.q == 0) {
#pragma unroll
            for (int r2 = 0; r2 < DRPL; ++r2) { st_agent(a.o + (size_t) s * DE + g * 32 + r2 * 16 + ln.r, 0.125f * acc[r2][0]); }
        }
    }
    // the last expert of the row group combines: y = sum_k w_k o_k in k order + shared, for every token
    if (!arrive_last(a.cnt + CNT_COMB + g, (unsigned) nm)) { return; }
    const int lane = lane_id();
    for (int i = lane; i < a.n * 32; i += 64) {
        const int tok = i / 32, rr = g * 32 + i % 32;
        float ov[MAXK + 1];
#pragma unroll
        for (int k = 0; k < MAXK; ++k) { ov[k] = k < a.topk ? ld_agent(a.o + (size_t) rt.inv[tok * a.topk + k] * DE + rr) : 0.f; }
        ov[MAXK] = ld_agent(a.o + (size_t) (P + tok) * DE + rr);
        float mv = ov[0] * rt.wts[tok * a.topk];
        for (int k = 1; k < a.topk; ++k) { mv = mv + ov[k] * rt.wts[tok * a.topk + k]; }
        gptr(a.y)[(size_t) tok * DE + rr] = mv + ov[MAXK];
    }
}

// ---------------------------------------------------------------- the kernel
__global__ void __launch_bounds__(DNT, 1) k_moe_decode(const DecodeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t dyn_lds[];
    const lds_t lds = (lds_t) dyn_lds;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
    const int G = gridDim.x, n = a.n, P = n * a.topk;
    LK_LOCAL unsigned * ctl = reinterpret_cast<LK_LOCAL unsigned *>(lds + L_CTL);   // [1] selections done, [2] routing ready (1 ok, 2 failed), [3] a wait failed
    Lane ln;
    ln.r = lane >> 2; ln.q = lane & 3;
    ln.tr = lds_addr(dyn_lds) | ((uint32_t) (lane & 15) << 3);   // table base (64 KB aligned: the tables open the LDS) | replica
    ln.lq = (uint32_t) ln.q * 4096 + 16 * ln.r; ln.ld = (uint32_t) ln.q * 128 + 2 * ln.r;

    // 1. router logits (the whole workgroup), then tables and tokens
    TRACE(wave, 0);
    if (threadIdx.x < 4) { ctl[threadIdx.x] = 0; }
    for (int e = blockIdx.x; e < a.n_exp; e += G) { router_phase(a, lds, wave, e); }
    TRACE(wave, 2);
    tables_copy<DNT>(dyn_lds, a.tab);
    quant_tokens(a, lds, wave);
    __syncthreads();
    TRACE(wave, 1);
    if (lds_addr(dyn_lds) & 0xFFFFu) { report(a.err, 4); return; }   // table addressing needs a 64 KB aligned base

    // 2. selection (wave t = token t, every workgroup redundantly); the last selecting wave builds the dispatch and opens
    //    the task phase. Waves without a token run the shared expert's gate/up meanwhile.
    const bool pre = n < DW;
    if (wave < n) {
        float bv[4], lg[4];
        load_bias(a.bias, a.n_exp, bv);
        const bool ok = wait_logits(a, wave, lg);
        TRACE(wave, 3);
        if (!ok) { report(a.err, 2); }
        const RT rt(lds);
        float * scr = (float *) (lds + L_DST) + wave * (NEXP_MAX + 2 * 64);
        if (ok) {
            select_token(lg, bv, a.n_exp, a.n_group, a.topk_group, a.topk, a.scale, scr, (int *) (rt.sel + wave * a.topk),
                         (float *) (rt.wts + wave * a.topk), blockIdx.x == 0 && a.probs ? a.probs + (size_t) wave * a.n_exp : nullptr);
        } else if (lane == 0) {
            __hip_atomic_fetch_or(ctl + 3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        TRACE(wave, 4);
        if (lds_arrive(ctl + 1, (unsigned) n)) {
            const bool all_ok = __builtin_amdgcn_readfirstlane(__hip_atomic_load(ctl + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) == 0;
            dispatch_wave(a, lds, all_ok ? P : 0);
            lds_visible();
            if (lane == 0) { __hip_atomic_store(ctl + 2, all_ok ? 1u : 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP); }
            TRACE(wave, 30);
        }
    } else if (pre) {
        for (int tk = (wave - n) * G + blockIdx.x; tk < 2 * NGU; tk += (DW - n) * G) { gate_up_task(a, lds, ln, SH, tk >> 1, tk & 1, P); }
    }
    const unsigned ready = lds_wait(ctl + 2);
    TRACE(wave, 5);
    if (ready != 1) { if (ready == 0) { report(a.err, 8); } return; }

    // 4. expert tasks, round-robin over every wave of the grid (task tk on workgroup tk % G, wave tk / G % DW)
    const int nact = *RT(lds).nact, nm = nact + 1;
    const int t_gu = (nact + (pre ? 0 : 1)) * 2 * NGU, t_all = t_gu + nm * NDN;
    int ntask = 0;
    for (int tk = wave * G + blockIdx.x; tk < t_all; tk += G * DW) {
        if (ntask < 12) { TRACE(wave, 6 + 2 * ntask); }
        if (tk < t_gu) {
            const int m = tk / (2 * NGU), r = tk % (2 * NGU);
            gate_up_task(a, lds, ln, m < nact ? m : SH, r >> 1, r & 1, P);
        } else {
            const int d = tk - t_gu, m = d / NDN;
            down_task(a, lds, ln, wave, m < nact ? m : SH, d % NDN, P, nm);
        }
        if (ntask < 12) { TRACE(wave, 7 + 2 * ntask); }
        ++ntask;
    }
#ifdef LOKI_TRACE
    if (lane == 0) { g_trace[(blockIdx.x * DW + wave) * TRACE_SLOTS + 31] = (uint64_t) ntask | ((uint64_t) t_gu << 32); }
#endif
}

size_t decode_lds_bytes() { return DEC_LDS; }

// workgroups of k_moe_decode that can be resident at once on `ncu` CUs (0: the cooperative launch is unavailable)
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

hipError_t launch_moe_decode(const DecodeArgs & a, int grid, bool cooperative, hipStream_t st) {
    if (a.n < 1 || a.n > DMAX_N || a.topk < 1 || a.topk > MAXK || a.n_exp < 1 || a.n_exp > NEXP_MAX || a.n_group < 1 || a.n_group > 64 ||
        a.n_exp % a.n_group || a.E != DE || a.H != DH || grid < 1) {
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
