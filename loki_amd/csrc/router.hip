// router.hip -- the DeepSeek-V3/R1 grouped sigmoid router on the device (no host round-trip).
//
// Reference: router_probs / router_topk (src/fused_layer.cu:313-332, launched at :506) and the ggml graph
// (src/server_core_fused.cpp:646-650) compute p = sigmoid(W x), take the top-8 of p + bias with ties to the lower index,
// and weight w_k = p[sel_k] / max(sum p[sel], 2^-14) * 2.5. This build adds the grouped rule the task names (8 groups of
// 32 experts; a group's score is the sum of its two best biased scores; the top-4 groups stay eligible), which reduces
// to the reference's rule with n_group = topk_group = 1.
//
// Logit contract (shared bit for bit with the CPU checker, moe_device.h): 256 chunks of K/256 products, each summed in
// order in fp64 from exact fp32 x fp32 products, a fixed pairwise tree over the chunk sums, one rounding to fp32. The
// sigmoid uses the fp64 exp contract of moe_common.h. Selection and weights are plain fp32 compares, adds and one
// correctly rounded division, so sel and wts are bit-identical to the checker's.
#include "moe_device.h"
#include "moe_kernels.h"

namespace lk {

constexpr int RT = 8;   // tokens per router wave

// one wave per (expert, 8-token tile); every token's logit is a full wave reduction (logit_tree)
__global__ void __launch_bounds__(64) k_router_logits(const float * __restrict__ W, const float * __restrict__ x, int n, int n_exp, int K,
                                                      float * __restrict__ logits) {
    const int e = blockIdx.x, t0 = blockIdx.y * RT;
    const int nt = min(RT, n - t0);
    for (int t = 0; t < nt; ++t) {
        double s[4];
        if (K == 7168) { logit_chunks<7>(W + (size_t) e * K, x + (size_t) (t0 + t) * K, s); }
        else { logit_chunks_any(W + (size_t) e * K, x + (size_t) (t0 + t) * K, K, s); }
        const double tot = logit_tree(s);
        if (threadIdx.x == 0) { logits[(size_t) (t0 + t) * n_exp + e] = (float) tot; }
    }
}

// Batches below 256 tokens (K = 7168): one workgroup (4 waves) per expert; thread c owns chunk c (28 values) of every
// token and keeps its 28 weights in registers. Per token the chunk sum runs in element order with v_fma_f64 (exact
// products, one rounding each), tree levels 1-6 are lane butterflies inside the wave (chunks 64 q .. 64 q + 63 of wave
// q), and levels 7-8 add the four waves' totals as (q0 + q1) + (q2 + q3) through LDS. Four tokens per pass.
constexpr int RW_MAXN = 256;
__device__ __forceinline__ void router_wg_logits(const float * __restrict__ W, const float * __restrict__ x, int n, int n_exp,
                                                 float * __restrict__ logits, double (*part)[4]) {
#pragma clang fp contract(off)
    constexpr int CL = 28;
    const int e = blockIdx.x, c = threadIdx.x, q = c >> 6, lane = c & 63;
    float wv[CL];
#pragma unroll
    for (int i = 0; i < CL / 4; ++i) {
        const float4 v = gloadf4(W + (size_t) e * 7168 + CL * c + 4 * i);
        wv[4 * i] = v.x; wv[4 * i + 1] = v.y; wv[4 * i + 2] = v.z; wv[4 * i + 3] = v.w;
    }
    for (int t0 = 0; t0 < n; t0 += 4) {
        double sv[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            sv[k] = 0.0;
            if (t0 + k < n) {
                const float * xr = x + (size_t) (t0 + k) * 7168 + CL * c;
#pragma unroll
                for (int i = 0; i < CL / 4; ++i) {
                    const float4 v = gloadf4(xr + 4 * i);
                    const float xv[4] = { v.x, v.y, v.z, v.w };
#pragma unroll
                    for (int j = 0; j < 4; ++j) { sv[k] = __builtin_fma((double) xv[j], (double) wv[4 * i + j], sv[k]); }
                }
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) { sv[k] = sv[k] + __shfl_xor(sv[k], o); }
        }
        if (lane == 0) {
#pragma unroll
            for (int k = 0; k < 4; ++k) { if (t0 + k < n) { part[t0 + k][q] = sv[k]; } }
        }
    }
    __syncthreads();
    if (c < n) { logits[(size_t) c * n_exp + e] = (float) ((part[c][0] + part[c][1]) + (part[c][2] + part[c][3])); }
}
__global__ void __launch_bounds__(256) k_router_wg(const float * __restrict__ W, const float * __restrict__ x, int n, int n_exp,
                                                   float * __restrict__ logits) {
    __shared__ double part[RW_MAXN][4];
    router_wg_logits(W, x, n, n_exp, logits, part);
}

// A few tokens (n <= RF_MAXN): k_router_wg's logits, then k_router_select's rule for every token in the workgroup that
// finishes last (wave q selects tokens q, q + 4, ..), so the routing is one launch. The logits reach that workgroup as
// epoch-tagged words tl [n][n_exp] (agent-scope stores and loads, polled until they carry this launch's epoch) and the
// workgroups count themselves on cnt (zero before the launch, reset by the last one): no memory fences, which cost an
// L2 write-back per workgroup. Wave 0 writes every token's picks, then (done != null) one system-scope release and
// done = epoch, so the host can read them from host memory without waiting for the stream. A poll that times out
// (stores that never land) leaves the picks -1.
constexpr int RF_MAXN = 8, RF_POLL = 1 << 20;
__global__ void __launch_bounds__(256) k_router_wg_sel(const float * __restrict__ W, const float * __restrict__ x, int n, int n_exp,
                                                       float * __restrict__ logits, const float * __restrict__ bias, int n_group,
                                                       int topk_group, int topk, float scale, int keep, float renorm,
                                                       float * __restrict__ probs, int * __restrict__ sel, float * __restrict__ wts,
                                                       uint64_t * tl, unsigned epoch, unsigned * cnt, unsigned * done, int * err,
                                                       int * herr) {
    __shared__ double part[RF_MAXN][4];
    __shared__ float scr[4][NEXP_MAX + 2 * 64];
    __shared__ int so[RF_MAXN][MAXK]; __shared__ float wo[RF_MAXN][MAXK];
    __shared__ unsigned last;
    router_wg_logits(W, x, n, n_exp, logits, part);
    const int e0 = blockIdx.x, c = threadIdx.x;
    if (c < n) {   // the same logit again as a tagged word (part[] is final after router_wg_logits' barrier)
        const float v = (float) ((part[c][0] + part[c][1]) + (part[c][2] + part[c][3]));
        __hip_atomic_store(gptr(tl) + (size_t) c * n_exp + e0, ((uint64_t) epoch << 32) | __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (c == 0) { last = atomicAdd(cnt, 1u) == gridDim.x - 1; }
    __syncthreads();
    if (!last) { return; }
    const int q = c >> 6, lane = c & 63;
    if (c == 0) { *cnt = 0u; }
    float bv[4];
    load_bias(bias, n_exp, bv);
    for (int t = q; t < n; t += 4) {
        uint64_t w[4];
        bool ok = false;
        for (int it = 0; it < RF_POLL && !ok; ++it) {
            ok = true;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = 4 * lane + j;
                w[j] = e < n_exp ? __hip_atomic_load(gptr(tl) + (size_t) t * n_exp + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0;
                ok = ok && (e >= n_exp || (unsigned) (w[j] >> 32) == epoch);
            }
            ok = __ballot(!ok) == 0;
            if (!ok) { __builtin_amdgcn_s_sleep(1); }
        }
        if (!ok) {   // unreachable unless stores are lost: no picks rather than wrong ones, and the error reported
            if (lane < keep) { so[t][lane] = -1; wo[t][lane] = 0.f; }
            if (lane == 0) {
                if (err) { __hip_atomic_fetch_or(gptr(err), 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
                if (herr) { __hip_atomic_store(gptr(herr), 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); }
            }
            continue;
        }
        float lg[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) { lg[j] = __builtin_bit_cast(float, (uint32_t) w[j]); }
        select_token(lg, bv, n_exp, n_group, topk_group, topk, scale, scr[q], so[t], wo[t], probs ? probs + (size_t) t * n_exp : nullptr,
                     keep, renorm);
    }
    __syncthreads();
    if (q == 0) {
        for (int i = lane; i < n * keep; i += 64) { sel[i] = so[i / keep][i % keep]; wts[i] = wo[i / keep][i % keep]; }
        if (done) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");   // system scope: the picks before the word
            if (lane == 0) { __hip_atomic_store(gptr(done), epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM); }
        }
    }
}

// Large batches (K = 7168): register tiles. Lane (tg, eg) = (lane / 8, lane % 8) owns the logits of TT tokens x EE
// experts of the workgroup's (8 TT) x (8 EE) tile; wave q computes slice q of the contract (chunks q * 256 / NQ ..) with the
// same in-order fp64 chunk sums and pairwise tree as k_router_wg, and the slices are combined by the tree's top levels
// through LDS. Each 16-byte load of x or W feeds EE or TT fused multiply-adds, so x and W are read once per tile.
template <int TT, int EE> struct RgAcc { double v[TT][EE]; };
// one chunk's in-order sums (28 products each) for the lane's TT x EE logits; the loads of step i + 1 are in flight
// while step i computes, and nothing is hoisted further (register budget)
template <int TT, int EE>
__device__ __forceinline__ void rg_chunk(const float * const (&xr)[TT], const float * const (&wr)[EE], int c, RgAcc<TT, EE> & s) {
#pragma clang fp contract(off)
    constexpr int CL = 28, NS = CL / 4;
    float4 xv[2][TT], wv[2][EE];
#pragma unroll
    for (int t = 0; t < TT; ++t) {
#pragma unroll
        for (int e = 0; e < EE; ++e) { s.v[t][e] = 0.0; }
    }
    auto load = [&](int i, int b) {
#pragma unroll
        for (int t = 0; t < TT; ++t) { xv[b][t] = gloadf4(xr[t] + CL * c + 4 * i); }
#pragma unroll
        for (int e = 0; e < EE; ++e) { wv[b][e] = gloadf4(wr[e] + CL * c + 4 * i); }
    };
    load(0, 0);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
        const int b = i & 1;
        if (i + 1 < NS) { load(i + 1, b ^ 1); }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            double xd[TT], wd[EE];
#pragma unroll
            for (int t = 0; t < TT; ++t) { xd[t] = (double) (q == 0 ? xv[b][t].x : q == 1 ? xv[b][t].y : q == 2 ? xv[b][t].z : xv[b][t].w); }
#pragma unroll
            for (int e = 0; e < EE; ++e) { wd[e] = (double) (q == 0 ? wv[b][e].x : q == 1 ? wv[b][e].y : q == 2 ? wv[b][e].z : wv[b][e].w); }
#pragma unroll
            for (int t = 0; t < TT; ++t) {
#pragma unroll
                for (int e = 0; e < EE; ++e) { s.v[t][e] = __builtin_fma(xd[t], wd[e], s.v[t][e]); }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}
template <int TT, int EE>
__device__ __forceinline__ void rg_add(RgAcc<TT, EE> & d, const RgAcc<TT, EE> & l, const RgAcc<TT, EE> & r) {
#pragma clang fp contract(off)
#pragma unroll
    for (int t = 0; t < TT; ++t) {
#pragma unroll
        for (int e = 0; e < EE; ++e) { d.v[t][e] = l.v[t][e] + r.v[t][e]; }
    }
}
// the level-4 node over chunks c0 .. c0 + 15: the pairwise tree built as the chunks arrive (binary counter; pend[l]
// holds the pending left node of level l)
template <int TT, int EE>
__device__ __forceinline__ RgAcc<TT, EE> rg_tile16(const float * const (&xr)[TT], const float * const (&wr)[EE], int c0) {
    RgAcc<TT, EE> pend[4], v;
#pragma unroll 1
    for (int c = 0; c < 16; ++c) {
        rg_chunk<TT, EE>(xr, wr, c0 + c, v);
        if (!(c & 1)) { pend[0] = v; continue; }
        rg_add(v, pend[0], v);
        if (!(c & 2)) { pend[1] = v; continue; }
        rg_add(v, pend[1], v);
        if (!(c & 4)) { pend[2] = v; continue; }
        rg_add(v, pend[2], v);
        if (!(c & 8)) { pend[3] = v; continue; }
        rg_add(v, pend[3], v);
    }
    return v;
}
template <int TT, int EE, int NQ>
__global__ void __launch_bounds__(64 * NQ) k_router_tile(const float * __restrict__ W, const float * __restrict__ x, int n, int n_exp,
                                                       float * __restrict__ logits) {
#pragma clang fp contract(off)
    constexpr int K = 7168, CPW = 256 / NQ, LW = CPW == 64 ? 6 : CPW == 32 ? 5 : 4;   // chunks per wave, tree levels
    static_assert(CPW == (1 << LW) && LW >= 4, "slices of 16, 32 or 64 chunks");
    __shared__ double part[NQ][TT * EE][64];
    const int q = threadIdx.x >> 6, lane = lane_id(), tg = lane >> 3, eg = lane & 7;
    const int tb = blockIdx.y * 8 * TT + tg * TT, eb = blockIdx.x * 8 * EE + eg * EE;
    const float * xr[TT]; const float * wr[EE];
#pragma unroll
    for (int t = 0; t < TT; ++t) { xr[t] = x + (size_t) (tb + t < n ? tb + t : 0) * K; }
#pragma unroll
    for (int e = 0; e < EE; ++e) { wr[e] = W + (size_t) (eb + e < n_exp ? eb + e : 0) * K; }
    // the wave's slice as 16-chunk groups (level-4 nodes), combined pairwise in order (levels 5, 6)
    RgAcc<TT, EE> tot, l4, l5;
#pragma unroll 1
    for (int g = 0; g < CPW / 16; ++g) {
        RgAcc<TT, EE> v = rg_tile16<TT, EE>(xr, wr, q * CPW + 16 * g);
        if (LW == 4) { tot = v; break; }
        if (!(g & 1)) { l4 = v; continue; }
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
            for (int e = 0; e < EE; ++e) { v.v[t][e] = l4.v[t][e] + v.v[t][e]; }
        }
        if (LW == 5) { tot = v; break; }
        if (!(g & 2)) { l5 = v; continue; }
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
            for (int e = 0; e < EE; ++e) { tot.v[t][e] = l5.v[t][e] + v.v[t][e]; }
        }
    }
#pragma unroll
    for (int t = 0; t < TT; ++t) {
#pragma unroll
        for (int e = 0; e < EE; ++e) { part[q][t * EE + e][lane] = tot.v[t][e]; }
    }
    __syncthreads();
    // the tree's top levels over the NQ slices, pairwise in slice order; output o of the lane by wave o % NQ
    for (int o = q; o < TT * EE; o += NQ) {
        const int t = tb + o / EE, e = eb + o % EE;
        double v[NQ];
#pragma unroll
        for (int j = 0; j < NQ; ++j) { v[j] = part[j][o][lane]; }
#pragma unroll
        for (int w = 1; w < NQ; w *= 2) {
#pragma unroll
            for (int j = 0; j + w < NQ; j += 2 * w) { v[j] = v[j] + v[j + w]; }
        }
        if (t < n && e < n_exp) { logits[(size_t) t * n_exp + e] = (float) v[0]; }
    }
}

// Large batches (K = 7168), LDS-staged: the tiles, lanes and contract of k_router_tile<4, 4, NQ> (32 tokens x 32 experts
// per workgroup, lane (tg, eg) owns tokens 4 tg .. + 3 x experts 4 eg .. + 3, wave q the chunks q * 256 / NQ ..), but a
// chunk's 32 x rows and 32 W rows (28 values each) are loaded once per wave with coalesced 16-byte loads, converted to
// fp64 once and staged in the wave's own LDS buffer, where the lanes read them back (8 lanes share each row: a broadcast).
// Without the staging every lane loads and converts its 8 rows itself: 8x the load instructions and the conversions, and
// the texture unit's load rate bounds the kernel. The next chunk's raw values are in registers while a chunk computes.
// With KS > 1 the chunks are split over KS workgroups (blockIdx.z takes chunks z * 256 / KS ..), each forming its
// part's subtree into part2[z]; k_router_join adds the parts pairwise in order, the tree's top log2(KS) levels. The
// split that is launched, <2, 16>, gives each wave 8 chunks and needs 250 VGPRs, so two waves share a SIMD: the chunks'
// load latencies, which bound the whole tiles (64 chunks per wave, one wave per SIMD), overlap.
// Buffer layout, per operand: [block i (4 values)][row r % 4][half h][row r / 4] of 16 bytes (2 doubles), so a read of
// one (i, r % 4, h) by the wave touches 8 consecutive 16-byte slots: every bank once.
constexpr int RL_SLOTS = 7 * 4 * 2 * 8;   // 16-byte slots per operand and chunk
template <int NQ, int KS>
__global__ void __launch_bounds__(64 * NQ) k_router_lds(const float * __restrict__ W, const float * __restrict__ x, int n, int n_exp,
                                                         float * __restrict__ logits, double * __restrict__ part2) {
#pragma clang fp contract(off)
    constexpr int K = 7168, CL = 28, CPW = 256 / (NQ * KS), LW = CPW == 64 ? 6 : CPW == 32 ? 5 : CPW == 16 ? 4 : 3;
    constexpr int GN = CPW < 16 ? CPW : 16;   // chunks per tree group (the group's levels run as the chunks arrive)
    static_assert(CPW == (1 << LW) && LW >= 3, "slices of 8, 16, 32 or 64 chunks");
    static_assert(NQ * 16 * 64 * 8 <= NQ * 2 * RL_SLOTS * 16, "the slices' totals fit the staging buffers");
    __shared__ __attribute__((aligned(16))) double2 buf[NQ][2][RL_SLOTS];   // [wave][x, W][slot]; then the slices' totals
    const int q = threadIdx.x >> 6, lane = lane_id(), tg = lane >> 3, eg = lane & 7;
    const int tb = blockIdx.y * 32, eb = blockIdx.x * 32;
    // the lane's staging share: 16-byte pieces f = lane + 64 k (k < 7) of the chunk's 448 (x rows first, then W rows)
    const float * src[7]; int dst[7];
#pragma unroll
    for (int k = 0; k < 7; ++k) {
        const int f = lane + 64 * k, op = f >= 224, g = f - 224 * op, r = g / 7, i = g % 7;
        const int row = op ? (eb + r < n_exp ? eb + r : 0) : (tb + r < n ? tb + r : 0);
        src[k] = (op ? W : x) + (size_t) row * K + 4 * i;
        dst[k] = op * RL_SLOTS + ((i * 4 + (r & 3)) * 2) * 8 + (r >> 2);   // half 0; half 1 is 8 slots on
    }
    double2 * wb = &buf[q][0][0];
    float4 nv[7];
    auto fetch = [&](int c) {
#pragma unroll
        for (int k = 0; k < 7; ++k) { nv[k] = gloadf4(src[k] + CL * c); }
    };
    auto stage = [&]() {
#pragma unroll
        for (int k = 0; k < 7; ++k) {
            wb[dst[k]] = make_double2((double) nv[k].x, (double) nv[k].y);
            wb[dst[k] + 8] = make_double2((double) nv[k].z, (double) nv[k].w);
        }
    };
    // chunk c's in-order sums for the lane's 4 x 4 logits, from the staged buffer
    auto chunk = [&](RgAcc<4, 4> & s) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int e = 0; e < 4; ++e) { s.v[t][e] = 0.0; }
        }
#pragma unroll
        for (int i = 0; i < 7; ++i) {
            double xa[4][4], wa[4][4];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const double2 v = wb[((i * 4 + t) * 2 + h) * 8 + tg];
                    xa[t][2 * h] = v.x; xa[t][2 * h + 1] = v.y;
                    const double2 u = wb[RL_SLOTS + ((i * 4 + t) * 2 + h) * 8 + eg];
                    wa[t][2 * h] = u.x; wa[t][2 * h + 1] = u.y;
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) { s.v[t][e] = __builtin_fma(xa[t][j], wa[e][j], s.v[t][e]); }
                }
            }
        }
    };
    const int c0 = (KS == 1 ? 0 : (int) blockIdx.z * (256 / KS)) + q * CPW;
    fetch(c0);
    int cn = 0;   // chunks of the slice consumed
    // one chunk: stage the fetched values, fetch the next chunk's, compute (a wave's LDS operations run in order, so the
    // staging writes follow the previous chunk's reads)
    auto next_chunk = [&](RgAcc<4, 4> & v) {
        stage();
        if (cn + 1 < CPW) { fetch(c0 + cn + 1); }
        chunk(v);
        ++cn;
    };
    // the slice's pairwise tree: 16-chunk groups built as the chunks arrive (binary counter), then levels 5 and 6
    auto tile16 = [&]() {   // GN chunks (16; for 8-chunk slices the loop ends at c = 7 with v the group's total)
        RgAcc<4, 4> pend[4], v;
#pragma unroll 1
        for (int c = 0; c < GN; ++c) {
            next_chunk(v);
            if (!(c & 1)) { pend[0] = v; continue; }
            rg_add(v, pend[0], v);
            if (!(c & 2)) { pend[1] = v; continue; }
            rg_add(v, pend[1], v);
            if (!(c & 4)) { pend[2] = v; continue; }
            rg_add(v, pend[2], v);
            if (!(c & 8)) { pend[3] = v; continue; }
            rg_add(v, pend[3], v);
        }
        return v;
    };
    RgAcc<4, 4> tot, l4, l5;
#pragma unroll 1
    for (int g = 0; g < CPW / GN; ++g) {
        RgAcc<4, 4> v = tile16();
        if (LW <= 4) { tot = v; break; }
        if (!(g & 1)) { l4 = v; continue; }
        rg_add(v, l4, v);
        if (LW == 5) { tot = v; break; }
        if (!(g & 2)) { l5 = v; continue; }
        rg_add(tot, l5, v);
    }
    __syncthreads();   // every wave is done with its staging buffer: it now holds the slices' totals
    double * part = reinterpret_cast<double *>(&buf[0][0][0]);   // [NQ][16][64]
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
        for (int e = 0; e < 4; ++e) { part[(q * 16 + t * 4 + e) * 64 + lane] = tot.v[t][e]; }
    }
    __syncthreads();
    // the tree's top levels over the NQ slices, pairwise in slice order; output o of the lane by wave o % NQ
    for (int o = q; o < 16; o += NQ) {
        const int t = tb + tg * 4 + o / 4, e = eb + eg * 4 + o % 4;
        double v[NQ];
#pragma unroll
        for (int j = 0; j < NQ; ++j) { v[j] = part[(j * 16 + o) * 64 + lane]; }
#pragma unroll
        for (int w = 1; w < NQ; w *= 2) {
#pragma unroll
            for (int j = 0; j + w < NQ; j += 2 * w) { v[j] = v[j] + v[j + w]; }
        }
        if (t < n && e < n_exp) {
            if constexpr (KS == 1) { logits[(size_t) t * n_exp + e] = (float) v[0]; }
            else { part2[((size_t) blockIdx.z * n + t) * n_exp + e] = v[0]; }
        }
    }
}
// the top levels of the K-split tree: the KS parts added pairwise in order, then rounded to fp32
template <int KS>
__global__ void __launch_bounds__(256) k_router_join(const double * __restrict__ part2, int total, float * __restrict__ logits) {
#pragma clang fp contract(off)
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= total) { return; }
    double v[KS];
#pragma unroll
    for (int j = 0; j < KS; ++j) { v[j] = part2[(size_t) j * total + i]; }
#pragma unroll
    for (int w = 1; w < KS; w *= 2) {
#pragma unroll
        for (int j = 0; j + w < KS; j += 2 * w) { v[j] = v[j] + v[j + w]; }
    }
    logits[i] = (float) v[0];
}

// the K split for n tokens: 16 parts from RL_SPLIT_MIN to RL_SPLIT_MAX tokens, else none
static int router_split(int n, int n_exp, int K) {
    (void) n_exp;
    return K == 7168 && n >= RL_SPLIT_MIN && n <= RL_SPLIT_MAX ? 16 : 1;
}
size_t router_split_doubles(int n, int n_exp, int K) {
    const int ks = router_split(n, n_exp, K);
    return ks > 1 ? (size_t) ks * n * n_exp : 0;
}

hipError_t launch_router_logits(const float * W, const float * x, int n, int n_exp, int K, float * logits, double * part2, hipStream_t st) {
    if (n <= 0) { return hipSuccess; }
    if (K % 1024 != 0) { return hipErrorInvalidValue; }
    // measured on MI355X (route call wall time): k_router_wg costs ~0.6 us per token (every workgroup reads all of x),
    // 25 us at 32 tokens, 33 at 48; the split tiles 28 us to 64 tokens, 35 at 96, 53 at 255, 72 at 300, 103 at 512,
    // 180 at 1024, 343 at 2048 (the whole tiles 375)
    if (router_split(n, n_exp, K) > 1 && part2) {   // 32 x 32 tiles, the chunks split over 16 workgroups, then the join
        const int total = n * n_exp;
        k_router_lds<2, 16><<<dim3((n_exp + 31) / 32, (n + 31) / 32, 16), 128, 0, st>>>(W, x, n, n_exp, nullptr, part2);
        k_router_join<16><<<dim3((total + 255) / 256), 256, 0, st>>>(part2, total, logits);
        return hipGetLastError();
    }
    if (K == 7168 && n >= 1024) {   // 32 x 32 tiles (4 x 4 per lane), staged in LDS
        k_router_lds<4, 1><<<dim3((n_exp + 31) / 32, (n + 31) / 32), 256, 0, st>>>(W, x, n, n_exp, logits, nullptr);
        return hipGetLastError();
    }
    if (K == 7168 && n >= RW_MAXN) {   // 32 x 16 tiles (4 x 2 per lane)
        k_router_tile<4, 2, 4><<<dim3((n_exp + 15) / 16, (n + 31) / 32), 256, 0, st>>>(W, x, n, n_exp, logits);
        return hipGetLastError();
    }
    if (K == 7168) {
        k_router_wg<<<dim3(n_exp), 256, 0, st>>>(W, x, n, n_exp, logits);
        return hipGetLastError();
    }
    k_router_logits<<<dim3(n_exp, (n + RT - 1) / RT), 64, 0, st>>>(W, x, n, n_exp, K, logits);
    return hipGetLastError();
}

// one wave per token; lane l holds experts 4l..4l+3 (n_exp <= 256); the rule is select_token's (moe_device.h), with
// keep entries per token written (keep = topk: all of them)
__global__ void __launch_bounds__(64) k_router_select(const float * __restrict__ logits, const float * __restrict__ bias, int n, int n_exp,
                                                      int n_group, int topk_group, int topk, float scale, int keep, float renorm,
                                                      float * __restrict__ probs, int * __restrict__ sel, float * __restrict__ wts) {
    __shared__ float scr[NEXP_MAX + 2 * 64];
    __shared__ int so[MAXK]; __shared__ float wo[MAXK];
    const int t = blockIdx.x, lane = threadIdx.x;
    float lg[4], bv[4];
    load_bias(bias, n_exp, bv);
#pragma unroll
    for (int j = 0; j < 4; ++j) { const int e = 4 * lane + j; lg[j] = e < n_exp ? logits[(size_t) t * n_exp + e] : 0.f; }
    select_token(lg, bv, n_exp, n_group, topk_group, topk, scale, scr, so, wo, probs ? probs + (size_t) t * n_exp : nullptr, keep, renorm);
    lds_visible();
    if (lane < keep) { sel[(size_t) t * keep + lane] = so[lane]; wts[(size_t) t * keep + lane] = wo[lane]; }
}

static bool select_rule_ok(int n_exp, int n_group, int topk_group, int topk, int keep) {
    return !(n_exp > NEXP_MAX || n_exp % n_group || topk > MAXK || topk_group > n_group || topk > topk_group * (n_exp / n_group) ||
             n_exp / n_group < 2 || n_group > 64 || keep > topk);
}

bool router_fused_ok(int n, int K) { return n >= 1 && n <= RF_MAXN && K == 7168; }

hipError_t launch_router_fused(const float * W, const float * x, int n, int n_exp, int K, float * logits, const float * bias, int n_group,
                               int topk_group, int topk, float scale, float * probs, int * sel, float * wts, uint64_t * tl,
                               unsigned epoch, unsigned * cnt, unsigned * done, int * err, int * herr, hipStream_t st, int keep,
                               float renorm) {
    if (keep <= 0) { keep = topk; }
    if (!router_fused_ok(n, K) || !cnt || !tl || epoch == 0 || !select_rule_ok(n_exp, n_group, topk_group, topk, keep)) {
        return hipErrorInvalidValue;
    }
    k_router_wg_sel<<<dim3(n_exp), 256, 0, st>>>(W, x, n, n_exp, logits, bias, n_group, topk_group, topk, scale, keep, renorm, probs, sel,
                                                 wts, tl, epoch, cnt, done, err, herr);
    return hipGetLastError();
}

// --share-experts keep of n rows (keep_share_rows): every thread adds its rows' own picks to the LDS set, then wave 0
// runs the rows in order
__global__ void __launch_bounds__(256) k_keep_share(const int * __restrict__ sel8, const float * __restrict__ w8, int n, int topk, int ke,
                                                    float renorm, int * __restrict__ sel, float * __restrict__ wts) {
    __shared__ unsigned U[8];
    if (threadIdx.x < 8) { U[threadIdx.x] = 0u; }
    __syncthreads();
    const int own = ke < 2 ? ke : 2;
    for (int i = threadIdx.x; i < n; i += 256) {
        for (int k = 0; k < topk; ++k) {
            const float wk = gptr(w8)[(size_t) i * topk + k];
            int r = 0;
            for (int j = 0; j < topk; ++j) { const float o = gptr(w8)[(size_t) i * topk + j]; r += (o > wk || (o == wk && j < k)) ? 1 : 0; }
            if (r < own) { const int e = gptr(sel8)[(size_t) i * topk + k]; atomicOr(&U[(e >> 5) & 7], 1u << (e & 31)); }
        }
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        keep_share_rows(gptr(sel8), gptr(w8), n, topk, ke, renorm, gptr(sel), gptr(wts), (LK_LOCAL unsigned *) U, false);
    }
}
hipError_t launch_keep_share(const int * sel8, const float * w8, int n, int topk, int ke, float renorm, int * sel, float * wts, hipStream_t st) {
    if (n <= 0) { return hipSuccess; }
    if (topk < 1 || topk > MAXK || ke < 1 || ke > topk) { return hipErrorInvalidValue; }
    k_keep_share<<<1, 256, 0, st>>>(sel8, w8, n, topk, ke, renorm, sel, wts);
    return hipGetLastError();
}

hipError_t launch_router_select(const float * logits, const float * bias, int n, int n_exp, int n_group, int topk_group,
                                int topk, float scale, float * probs, int * sel, float * wts, hipStream_t st, int keep, float renorm) {
    if (n <= 0) { return hipSuccess; }
    if (keep <= 0) { keep = topk; }
    if (!select_rule_ok(n_exp, n_group, topk_group, topk, keep)) { return hipErrorInvalidValue; }
    k_router_select<<<n, 64, 0, st>>>(logits, bias, n, n_exp, n_group, topk_group, topk, scale, keep, renorm, probs, sel, wts);
    return hipGetLastError();
}

}  // namespace lk
