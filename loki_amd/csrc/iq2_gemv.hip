// iq2_gemv.hip -- IQ2_XXS x Q8_K expert mat-vecs (routed + shared experts) as persistent kernels, with the SwiGLU +
// Q8_K(h) epilogue (gate/up) and the weighted combine (down) fused in.
//
// Reference: tc_matvec<F_IQ2> (src/fused_layer.cu:178-202; launches :604-608) stages 16 rows x 4 blocks through shared
// memory into mma.m16n8k32 int8 tiles with split-K partials, then swiglu_q8 (:334-341) and moe_combine (:366-372) run as
// separate kernels. Here, for the few tokens per expert of decode:
//   * One workgroup per CU fills the bank-replicated codebook/sign tables (64 KB of LDS) once; its waves then take tasks
//     round-robin across all workgroups (task tk on workgroup tk % grid). A task is (expert slot, 16 rows): lane
//     4 r + q owns row r and the blocks j = 4 jj + q, streamed with non-temporal 16-byte loads PD blocks ahead (tiled
//     layout, moe_common.h). Gate and up of the same rows are streamed interleaved in the same task.
//   * Per block a lane dequantises its row's 8 sub-blocks into signed int8 (two replicated-table lookups and two
//     v_xad_u32 per 8 weights), runs v_dot4_i32_i8 against each token's Q8_K values (staged in LDS) into 8 independent
//     accumulators, and forms the exact integer block sum sum_ib (2 nibble + 1) * sumi and the block term
//     (d_w * d_x) * bsum -- the arithmetic of ggml_vec_dot_iq2_xxs_q8_K.
//   * At every step the 4 lanes of a quad hold 4 consecutive blocks of one row, so the row total advances in block order
//     through 4 quad broadcasts (DPP) and finally * 0.125: every output is bit-identical to the CPU checker and no
//     partial sum leaves the wave.
//   * Gate/up writes h = silu(g) * u; the last task of a 256-row block (device-scope counter) quantises that block of h
//     to Q8_K for every slot of the expert. Down writes o; the last expert of a row group computes
//     y = sum_k w_k o_k (k order) + shared (src/server_core_fused.cpp:970-975) for every token.
// h and o cross workgroups inside a launch, so they move with agent-scope relaxed atomic stores/loads: the XCDs' L2s are
// not coherent with each other, and an agent-scope fence would write back / invalidate a whole L2. Counters reset
// themselves (the last arriver writes 0), so a launch needs no clearing pass and can be replayed.
#include "moe_device.h"
#include "moe_kernels.h"

namespace lk {

struct TaskPtr {
    const uint8_t * q[2]; const uint8_t * d[2];   // the task's qs / d bases (uniform) of matrix 0 / 1 at step jj = 0
};

template <int NR, int PD, class G, int NMAT>
__device__ __forceinline__ void issue(const TaskPtr & tp, uint32_t lq, uint32_t ld, int s, uint4 (&pf)[NR][4], uint16_t (&pd)[NR], int slot) {
    const int mat = NMAT == 2 ? (s & 1) : 0, jj = NMAT == 2 ? (s >> 1) : s;
    const uint8_t * qb = tp.q[mat] + (size_t) jj * (G::QS * 4096);
#pragma unroll
    for (int c = 0; c < 4; ++c) { pf[slot][c] = load_nt(qb + lq + c * 1024); }
    pd[slot] = *gptr(reinterpret_cast<const uint16_t *>(tp.d[mat] + (size_t) jj * (G::QS * 128) + ld));
}

// one tile of T tokens (slots slot0 .. slot0 + T - 1) of a task: stream the lane's blocks (gate and up interleaved),
// fold each step's 4 blocks into the row totals, write h or o
template <bool GATEUP, class G, int T, int PD, bool XWG>
__device__ __forceinline__ void run_tile(const ExpertArgs & a, const uint8_t * lds, uint8_t * xs, const TaskPtr & tp,
                                         uint32_t lq, uint32_t ld, bool routed, int slot0, int row, int q, uint32_t rep) {
#pragma clang fp contract(off)
    constexpr int NMAT = GATEUP ? 2 : 1, STEPS = NMAT * G::BPQ, NR = PD + 1;
    static_assert(NMAT == 1 || NR % 2 == 0, "gate/up steps alternate matrices: the ring length must be even");
    const uint8_t * xr[T];
#pragma unroll
    for (int u = 0; u < T; ++u) {
        const int slot = slot0 + u;
        const int ar = GATEUP ? (routed ? a.perm[slot] / a.topk : slot - a.P) : slot;   // gate/up: token rows, down: slot rows
        if (XWG) {
            xr[u] = xs + ar * G::XROW;
        } else {
            if (u == 0) { __builtin_amdgcn_wave_barrier(); }   // the previous tile's reads are issued before the rows are overwritten
            stage_row<G>(xs + u * G::XROW, a.aq + (size_t) ar * G::K, a.ad + (size_t) ar * G::NB);
            xr[u] = xs + u * G::XROW;
        }
    }
    if (!XWG) {
        __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): the wave's LDS writes are done before any lane reads them
        __builtin_amdgcn_wave_barrier();
    }
    uint4 pf[NR][4]; uint16_t pd[NR];
#pragma unroll
    for (int k = 0; k < PD; ++k) {
        if (k < STEPS) { issue<NR, PD, G, NMAT>(tp, lq, ld, k, pf, pd, k); }
    }
    float acc[NMAT][T];
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
#pragma unroll
        for (int u = 0; u < T; ++u) { acc[m][u] = 0.f; }
    }
#pragma unroll 1
    for (int s0 = 0; s0 < STEPS; s0 += NR) {
#pragma unroll
        for (int k = 0; k < NR; ++k) {
            const int s = s0 + k;
            if (s < STEPS) {
                if (s + PD < STEPS) { issue<NR, PD, G, NMAT>(tp, lq, ld, s + PD, pf, pd, (k + PD) % NR); }
                const int mat = NMAT == 2 ? (k & 1) : 0;
                const int j = (NMAT == 2 ? (s >> 1) : s) * G::QS + q;
                const uint8_t * xb[T];
#pragma unroll
                for (int u = 0; u < T; ++u) { xb[u] = xr[u] + j * G::XBLK; }
                int bsum[T];
                block_bsum<T>(pf[k], rep, xb, bsum);
                const float dw = h2f(pd[k]);
#pragma unroll
                for (int u = 0; u < T; ++u) {
                    const float dx = reinterpret_cast<const float *>(xr[u] + G::NB * G::XBLK)[j];
                    acc[mat][u] = fold_quad(acc[mat][u], (dw * dx) * (float) bsum[u]);
                }
            }
        }
    }
#pragma unroll
    for (int u = 0; u < T; ++u) {
        const size_t o = (size_t) (slot0 + u) * a.R + row;
        if (q == 0) {
            if (GATEUP) {
                const float g = 0.125f * acc[0][u], up = 0.125f * acc[NMAT - 1][u];
                st_agent(a.h + o, det_silu(g) * up);
                if (a.gdbg) { a.gdbg[o] = g; a.udbg[o] = up; }
            } else {
                st_agent(a.o + o, 0.125f * acc[0][u]);
            }
        }
    }
}

template <bool GATEUP, int BPQ, int TT, int WAVES, int PD, bool XWG>
__global__ void __launch_bounds__(WAVES * 64) k_experts(const ExpertArgs a) {
#pragma clang fp contract(off)
    using G = Geo<BPQ>;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    tables_copy<WAVES * 64>(lds, a.tab);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = lane_id();
    uint8_t * xs = lds + TAB_BYTES;
    if (XWG) {   // every token's activations, once per workgroup
        for (int u = wave; u < a.n; u += WAVES) { stage_row<G>(xs + u * G::XROW, a.aq + (size_t) u * G::K, a.ad + (size_t) u * G::NB); }
    } else {
        xs += wave * TT * G::XROW;
    }
    __syncthreads();
    const int NG = a.R / G::RPW;
    const int nact = *a.nact;
    const int nm = nact + (a.shared ? 1 : 0);
    const int ntasks = nm * NG;
    const int r = lane >> 2, q = lane & 3;
    const uint32_t rep = tab_word_grid(lds_addr(lds), lane);   // table base (64 KB aligned: the tables open the LDS) | copy
    const uint32_t lq = (uint32_t) q * 4096 + 16 * r, ld = (uint32_t) q * 128 + 2 * r;   // the lane's part of its block addresses
    const size_t dreg = (size_t) (a.R / 64) * G::NB * 4096;                              // d region of a matrix
    // task tk runs on workgroup tk % grid: consecutive tasks spread over all CUs (and XCDs)
    for (int tk = wave * gridDim.x + blockIdx.x; tk < ntasks; tk += gridDim.x * WAVES) {
        const int m = tk / NG, g = tk - m * NG;
        const bool routed = m < nact;
        int e = 0, s0, cnt;
        if (routed) { e = a.act[m]; s0 = a.offsets[e]; cnt = a.offsets[e + 1] - s0; }
        else { s0 = a.P; cnt = a.n; }
        const int rg = g >> 2, sub = g & 3;   // 64-row group and the task's 16-row quarter of it
        TaskPtr tp;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const uint8_t * W = (GATEUP || mt == 0) ? (routed ? a.w[mt] + (size_t) e * a.estride : a.sh[mt]) : nullptr;
            tp.q[mt] = W + (size_t) rg * G::NB * 4096 + sub * 256;
            tp.d[mt] = W + dreg + (size_t) rg * G::NB * 128 + sub * 32;
        }
        const int row = g * G::RPW + r;
        for (int tok = 0; tok < cnt;) {
            if (TT > 1 && cnt - tok >= TT) { run_tile<GATEUP, G, TT, PD, XWG>(a, lds, xs, tp, lq, ld, routed, s0 + tok, row, q, rep); tok += TT; }
            else { run_tile<GATEUP, G, 1, PD, XWG>(a, lds, xs, tp, lq, ld, routed, s0 + tok, row, q, rep); tok += 1; }
        }
        if (GATEUP) {
            // the last task of a 256-row block quantises that block of h for every slot of the expert
            const int hb = (g * G::RPW) / QK;
            if (!arrive_last(a.cnt_2 + (size_t) m * (a.R / QK) + hb, (unsigned) (QK / G::RPW))) { continue; }
            for (int s = s0; s < s0 + cnt; ++s) {
                const float * hbp = a.h + (size_t) s * a.R + hb * QK;
                const float xv[4] = { ld_agent(hbp + 4 * lane), ld_agent(hbp + 4 * lane + 1), ld_agent(hbp + 4 * lane + 2), ld_agent(hbp + 4 * lane + 3) };
                float d; const uint32_t packed = q8k_lane(xv, d);
                reinterpret_cast<uint32_t *>(a.hq + (size_t) s * a.R + hb * QK)[lane] = packed;
                if (lane == 0) { a.hd[(size_t) s * (a.R / QK) + hb] = d; }
            }
        } else if (a.y) {
            // the last expert of a row group combines: y = sum_k w_k o_k in k order + shared, for every token
            if (!arrive_last(a.cnt_2 + g, (unsigned) nm)) { continue; }
            for (int i = lane; i < a.n * G::RPW; i += 64) {
                const int tok = i / G::RPW, rr = g * G::RPW + i % G::RPW;
                const int * iv = a.inv + (size_t) tok * a.topk; const float * w = a.wts + (size_t) tok * a.topk;
                float ov[MAXK + 1];
#pragma unroll
                for (int k = 0; k < MAXK; ++k) { ov[k] = k < a.topk ? ld_agent(a.o + (size_t) iv[k] * a.R + rr) : 0.f; }
                ov[MAXK] = ld_agent(a.o + (size_t) (a.P + tok) * a.R + rr);
                float mv = ov[0] * w[0];
                for (int k = 1; k < a.topk; ++k) { mv = mv + ov[k] * w[k]; }
                a.y[(size_t) tok * a.R + rr] = mv + ov[MAXK];
            }
        }
    }
}

// ---------------------------------------------------------------- configurations and launches
// gate/up (K = 7168, nb = 28): 7 steps of 4 blocks per matrix; down (K = 2048, nb = 8): 2 steps. 16 rows per task.
// Decode stages every token once per workgroup; larger batches stage each wave's tile per task.
//            GATEUP BPQ TT WAVES PD XWG
#define GU1   true,  7,  1, 8,   5, true    // n == 1
#define GU8   true,  7,  2, 8,   5, true    // n <= 8
#define GUP   true,  7,  1, 8,   3, false   // larger batches
#define DN1   false, 2,  1, 16,  2, false
#define DN8   false, 2,  2, 8,   2, false
constexpr int XWG_MAX = 8;

template <bool GATEUP, int BPQ, int TT, int WAVES, int PD, bool XWG>
constexpr size_t lds_of() { return TAB_BYTES + (size_t) (XWG ? XWG_MAX : WAVES * TT) * Geo<BPQ>::XROW; }

template <bool GATEUP, int BPQ, int TT, int WAVES, int PD, bool XWG>
static hipError_t set_lds() {
    static_assert(lds_of<GATEUP, BPQ, TT, WAVES, PD, XWG>() <= 160 * 1024, "LDS budget");
    return hipFuncSetAttribute((const void *) k_experts<GATEUP, BPQ, TT, WAVES, PD, XWG>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int) lds_of<GATEUP, BPQ, TT, WAVES, PD, XWG>());
}
template <bool GATEUP, int BPQ, int TT, int WAVES, int PD, bool XWG>
static hipError_t launch(const ExpertArgs & a, int grid, hipStream_t st) {
    k_experts<GATEUP, BPQ, TT, WAVES, PD, XWG><<<grid, WAVES * 64, lds_of<GATEUP, BPQ, TT, WAVES, PD, XWG>(), st>>>(a);
    return hipGetLastError();
}

hipError_t experts_init() {
    hipError_t e = set_lds<GU1>();
    if (e == hipSuccess) { e = set_lds<GU8>(); }
    if (e == hipSuccess) { e = set_lds<GUP>(); }
    if (e == hipSuccess) { e = set_lds<DN1>(); }
    if (e == hipSuccess) { e = set_lds<DN8>(); }
    return e;
}
size_t experts_terms_floats(int, int, int, int) { return 0; }

// the LDS table image (layout at TAB_BYTES in moe_common.h), once, in device memory
__global__ void k_table_image(uint64_t * img) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;   // 8-byte word: line i / 32, 8-byte slot i % 32
    if (i >= TAB_BYTES / 8) { return; }
    const int line = i >> 5, r = i & 31;
    if (line < 256) { img[i] = g_iq2xxs_grid[line]; return; }   // codebook: 32 copies
    const uint64_t m = sign_mask64(ksigns8((uint32_t) (line - 256)));
    img[i] = (r & 1) ? (m & 0x0101010101010101ull) : m;          // signs: 16 copies of {m, m & 0x01..}
}
hipError_t build_table_image(uint4 * img, hipStream_t st) {
    k_table_image<<<TAB_BYTES / 8 / 256, 256, 0, st>>>(reinterpret_cast<uint64_t *>(img));
    return hipGetLastError();
}

hipError_t launch_experts_gateup(const ExpertArgs & a, int grid, hipStream_t st) {
    if (a.K != Geo<7>::K || a.R % QK || a.nmat != 2 || a.n < 0) { return hipErrorInvalidValue; }
    if (a.n == 0 || grid <= 0) { return hipSuccess; }
    if (a.n == 1) { return launch<GU1>(a, grid, st); }
    if (a.n <= XWG_MAX) { return launch<GU8>(a, grid, st); }
    return launch<GUP>(a, grid, st);
}
hipError_t launch_experts_down(const ExpertArgs & a, int grid, hipStream_t st) {
    if (a.K != Geo<2>::K || a.R % 64 || a.nmat != 1 || a.n < 0) { return hipErrorInvalidValue; }
    if (a.n == 0 || grid <= 0) { return hipSuccess; }
    if (a.n == 1) { return launch<DN1>(a, grid, st); }
    return launch<DN8>(a, grid, st);
}

// k-ordered combine for callers that run the down pass without the fused epilogue: block (x, t) takes row t's columns
// 1024 x .. + 1023, four per thread (16-byte loads and stores); the row's slots and weights are uniform per block
__global__ void __launch_bounds__(256) k_combine(const float * __restrict__ o, const int * __restrict__ inv, const float * __restrict__ wts,
                                                 int n, int topk, int E, int P, const float * __restrict__ resid,
                                                 float * __restrict__ y, float * __restrict__ moe) {
#pragma clang fp contract(off)
    const int r = (blockIdx.x * 256 + threadIdx.x) * 4;
    if (r >= E) { return; }
    for (int t = blockIdx.y; t < n; t += gridDim.y) {   // the grid's y extent is capped at 65535
        const int * iv = inv + (size_t) t * topk; const float * w = wts + (size_t) t * topk;
        auto ld4 = [&](int slot) { return *reinterpret_cast<const float4 *>(o + (size_t) slot * E + r); };
        float4 m;
        {
            const float4 a = ld4(iv[0]); const float w0 = w[0];
            m = make_float4(a.x * w0, a.y * w0, a.z * w0, a.w * w0);
        }
        for (int k = 1; k < topk; ++k) {
            const float4 a = ld4(iv[k]); const float wk = w[k];
            m = make_float4(m.x + a.x * wk, m.y + a.y * wk, m.z + a.z * wk, m.w + a.w * wk);
        }
        const size_t i = (size_t) t * E + r;
        if (moe) { *reinterpret_cast<float4 *>(moe + i) = m; }
        const float4 sh = ld4(P + t);
        float4 v = make_float4(m.x + sh.x, m.y + sh.y, m.z + sh.z, m.w + sh.w);
        if (resid) {
            const float4 h = *reinterpret_cast<const float4 *>(resid + i);
            v = make_float4(v.x + h.x, v.y + h.y, v.z + h.z, v.w + h.w);
        }
        *reinterpret_cast<float4 *>(y + i) = v;
    }
}

// the same, one output per thread: for rows or pointers that are not 16-byte aligned
__global__ void __launch_bounds__(256) k_combine1(const float * __restrict__ o, const int * __restrict__ inv, const float * __restrict__ wts,
                                                  int n, int topk, int E, int P, const float * __restrict__ resid,
                                                  float * __restrict__ y, float * __restrict__ moe) {
#pragma clang fp contract(off)
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= E) { return; }
    for (int t = blockIdx.y; t < n; t += gridDim.y) {   // the grid's y extent is capped at 65535
        const int * iv = inv + (size_t) t * topk; const float * w = wts + (size_t) t * topk;
        float m = o[(size_t) iv[0] * E + r] * w[0];
        for (int k = 1; k < topk; ++k) { m = m + o[(size_t) iv[k] * E + r] * w[k]; }
        const size_t i = (size_t) t * E + r;
        if (moe) { moe[i] = m; }
        float v = m + o[(size_t) (P + t) * E + r];
        if (resid) { v = v + resid[i]; }
        y[i] = v;
    }
}

// the y extent of the row-looping grids (k_combine, k_combine1, k_wide_scatter): the hardware's 65535, or a small cap
// that a test sets (fl_set_debug) so that the loops over rows run at small sizes too
static int g_grid_ycap = 65535;
void set_grid_ycap(int cap) { g_grid_ycap = cap >= 1 && cap <= 65535 ? cap : 65535; }
unsigned grid_y(int rows) { return (unsigned) std::min(rows, g_grid_ycap); }

hipError_t launch_combine(const float * o, const int * inv, const float * wts, int n, int topk, int E, int P,
                          const float * resid, float * y, float * moe, hipStream_t st) {
    if ((int64_t) n * E <= 0) { return hipSuccess; }
    if (E % 4 == 0 && ((reinterpret_cast<uintptr_t>(o) | reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(moe) |
                        reinterpret_cast<uintptr_t>(resid)) & 15u) == 0) {
        k_combine<<<dim3((unsigned) ((E / 4 + 255) / 256), grid_y(n)), 256, 0, st>>>(o, inv, wts, n, topk, E, P, resid, y, moe);
    } else {
        k_combine1<<<dim3((unsigned) ((E + 255) / 256), grid_y(n)), 256, 0, st>>>(o, inv, wts, n, topk, E, P, resid, y, moe);
    }
    return hipGetLastError();
}

}  // namespace lk
