// iq2_gemv.hip -- IQ2_XXS x Q8_K expert mat-vecs for the routed + shared experts, and the weighted combine.
//
// Reference: tc_matvec<F_IQ2> (src/fused_layer.cu:178-202; launches :604-608) dequantises 16 rows x 8 activation rows
// through shared memory into mma.m16n8k32 int8 tiles, split-K, then swiglu_q8 (:334-341) and moe_combine (:366-372).
// Here, for the few tokens per expert of decode:
//   * one wave owns 4 rows of one expert's matrix and streams its tiled units (1056 B: 4 rows x 4 blocks) with one
//     16-byte load per lane; lane l holds qs bytes [16c, 16c+16) of block b of row r (r = l/16, b = l/4 % 4, c = l % 4),
//     i.e. sub-blocks 2c and 2c+1, and dequantises them once into 64 signed int8 weights in registers;
//   * every token routed to the expert then costs 16 v_dot4_i32_i8 per lane; the 4 lanes of a block add their
//     (2*(a1>>28)+1)-scaled integer sums (exact), the block term (d_w*d_x)*bsum is formed, and each row accumulates its
//     block terms in ascending block order in fp32 -- the order of ggml_vec_dot_iq2_xxs_q8_K -- then * 0.125. The
//     outputs are therefore bit-identical to the CPU checker's;
//   * gate and up run in the same wave and the epilogue writes h = silu(g) * u (the exp contract), so the gate/up
//     outputs never travel to HBM; the down pass writes o per (token, k) slot and the combine adds w_k * o_k in k order
//     plus the shared expert (src/server_core_fused.cpp:970-975).
// Token lists come from the device dispatch (offsets/perm); the shared expert is the extra expert slot m == nact.
#include "moe_common.h"
#include "moe_kernels.h"

namespace lk {

constexpr int GEMV_TT = 8;   // tokens per register tile

// 64 signed weights of sub-blocks (a0, a1) and (b0, b1) into w[16] (4 weights per int), scales 2*(a1>>28)+1
__device__ __forceinline__ void dequant_chunk(const Iq2Lds & tab, const uint4 & q, int * w, int & ls0, int & ls1) {
#pragma unroll
    for (int l = 0; l < 4; ++l) { iq2_group(tab, q.x, q.y, l, w[2 * l], w[2 * l + 1]); }
#pragma unroll
    for (int l = 0; l < 4; ++l) { iq2_group(tab, q.z, q.w, l, w[8 + 2 * l], w[8 + 2 * l + 1]); }
    ls0 = 2 * (int) (q.y >> 28) + 1; ls1 = 2 * (int) (q.w >> 28) + 1;
}

__device__ __forceinline__ int chunk_dot(const int * w, const int * xv, int ls0, int ls1) {
    int s0 = 0, s1 = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) { s0 = __builtin_amdgcn_sdot4(w[j], xv[j], s0, false); }
#pragma unroll
    for (int j = 0; j < 8; ++j) { s1 = __builtin_amdgcn_sdot4(w[8 + j], xv[8 + j], s1, false); }
    return ls0 * s0 + ls1 * s1;
}

template <bool GATEUP>
__global__ void __launch_bounds__(256) k_iq2_gemv(const GemvArgs a) {
#pragma clang fp contract(off)
    __shared__ Iq2Lds tab;
    iq2_lds_fill(tab);
    __syncthreads();
    const int bpe = a.R / 16;
    const int m = blockIdx.x / bpe;
    const int nact = *a.nact;
    if (m > nact || (m == nact && !a.shared)) { return; }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rq = (blockIdx.x % bpe) * 4 + wave;
    const bool routed = m < nact;
    const uint8_t * W0; const uint8_t * W1 = nullptr; int s0, cnt;
    if (routed) {
        const int e = a.act[m];
        W0 = a.w0 + (size_t) e * a.estride; if (GATEUP) { W1 = a.w1 + (size_t) e * a.estride; }
        s0 = a.offsets[e]; cnt = a.offsets[e + 1] - s0;
    } else {
        W0 = a.sh0; if (GATEUP) { W1 = a.sh1; }
        s0 = a.P; cnt = a.n;
    }
    const int nbq = a.K / (QK * UBLK), nbk = a.K / QK;
    const int r = lane >> 4, b = (lane >> 2) & 3, c = lane & 3;
    const size_t rq_off = (size_t) rq * nbq * UNIT;
    for (int tok0 = 0; tok0 < cnt; tok0 += GEMV_TT) {
        const int ntt = min(GEMV_TT, cnt - tok0);
        int arow[GEMV_TT];
        float acc0[GEMV_TT], acc1[GEMV_TT];
#pragma unroll
        for (int t = 0; t < GEMV_TT; ++t) {
            const int slot = s0 + tok0 + (t < ntt ? t : 0);
            arow[t] = GATEUP ? (routed ? a.perm[slot] / a.topk : slot - a.P) : slot;
            acc0[t] = 0.f; acc1[t] = 0.f;
        }
        for (int bq = 0; bq < nbq; ++bq) {
            const uint8_t * u0 = W0 + rq_off + (size_t) bq * UNIT;
            const uint4 q0 = *reinterpret_cast<const uint4 *>(u0 + 16 * lane);
            const float d0 = h2f(*reinterpret_cast<const uint16_t *>(u0 + 1024 + 2 * (lane >> 2)));
            int w0[16], l00, l01; dequant_chunk(tab, q0, w0, l00, l01);
            int w1[16], l10 = 0, l11 = 0; float d1 = 0.f;
            if (GATEUP) {
                const uint8_t * u1 = W1 + rq_off + (size_t) bq * UNIT;
                const uint4 q1 = *reinterpret_cast<const uint4 *>(u1 + 16 * lane);
                d1 = h2f(*reinterpret_cast<const uint16_t *>(u1 + 1024 + 2 * (lane >> 2)));
                dequant_chunk(tab, q1, w1, l10, l11);
            }
            const int blk = UBLK * bq + b;
#pragma unroll
            for (int t = 0; t < GEMV_TT; ++t) {
                if (t < ntt) {
                    const int4 * xp = reinterpret_cast<const int4 *>(a.aq + (size_t) arow[t] * a.K + (size_t) blk * QK + 64 * c);
                    const int4 x0 = xp[0], x1 = xp[1], x2 = xp[2], x3 = xp[3];
                    const int xv[16] = { x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w, x2.x, x2.y, x2.z, x2.w, x3.x, x3.y, x3.z, x3.w };
                    const float dx = a.ad[(size_t) arow[t] * nbk + blk];
                    int p0 = chunk_dot(w0, xv, l00, l01);
                    p0 += __shfl_xor(p0, 1); p0 += __shfl_xor(p0, 2);
                    const float t0 = (d0 * dx) * (float) p0;
#pragma unroll
                    for (int bb = 0; bb < UBLK; ++bb) { acc0[t] = acc0[t] + __shfl(t0, 16 * r + 4 * bb); }
                    if (GATEUP) {
                        int p1 = chunk_dot(w1, xv, l10, l11);
                        p1 += __shfl_xor(p1, 1); p1 += __shfl_xor(p1, 2);
                        const float t1 = (d1 * dx) * (float) p1;
#pragma unroll
                        for (int bb = 0; bb < UBLK; ++bb) { acc1[t] = acc1[t] + __shfl(t1, 16 * r + 4 * bb); }
                    }
                }
            }
        }
        if ((lane & 15) == 0) {
            const int row = UROWS * rq + r;
#pragma unroll
            for (int t = 0; t < GEMV_TT; ++t) {
                if (t < ntt) {
                    const size_t o = (size_t) (s0 + tok0 + t) * a.R + row;
                    const float v0 = 0.125f * acc0[t];
                    if (GATEUP) {
                        const float v1 = 0.125f * acc1[t];
                        a.out[o] = det_silu(v0) * v1;
                        if (a.dbg0) { a.dbg0[o] = v0; }
                        if (a.dbg1) { a.dbg1[o] = v1; }
                    } else {
                        a.out[o] = v0;
                    }
                }
            }
        }
    }
}

static hipError_t launch_gemv(const GemvArgs & a, bool gateup, hipStream_t st) {
    if (a.R % 16 != 0 || a.K % (QK * UBLK) != 0 || a.n < 0) { return hipErrorInvalidValue; }
    if (a.n == 0) { return hipSuccess; }
    const unsigned grid = (unsigned) ((a.max_act + (a.shared ? 1 : 0)) * (a.R / 16));
    if (grid == 0) { return hipSuccess; }
    if (gateup) { k_iq2_gemv<true><<<grid, 256, 0, st>>>(a); }
    else { k_iq2_gemv<false><<<grid, 256, 0, st>>>(a); }
    return hipGetLastError();
}
hipError_t launch_gemv_gateup(const GemvArgs & a, hipStream_t st) { return launch_gemv(a, true, st); }
hipError_t launch_gemv_down(const GemvArgs & a, hipStream_t st) { return launch_gemv(a, false, st); }

__global__ void __launch_bounds__(256) k_combine(const float * __restrict__ o, const int * __restrict__ inv, const float * __restrict__ wts,
                                                 int n, int topk, int E, int P, const float * __restrict__ resid,
                                                 float * __restrict__ y, float * __restrict__ moe) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t) n * E) { return; }
    const int t = (int) (i / E), r = (int) (i % E);
    const int * iv = inv + (size_t) t * topk; const float * w = wts + (size_t) t * topk;
    float m = o[(size_t) iv[0] * E + r] * w[0];
    for (int k = 1; k < topk; ++k) { m = m + o[(size_t) iv[k] * E + r] * w[k]; }
    if (moe) { moe[i] = m; }
    float v = m + o[(size_t) (P + t) * E + r];
    if (resid) { v = v + resid[i]; }
    y[i] = v;
}

hipError_t launch_combine(const float * o, const int * inv, const float * wts, int n, int topk, int E, int P,
                          const float * resid, float * y, float * moe, hipStream_t st) {
    const int64_t tot = (int64_t) n * E;
    if (tot <= 0) { return hipSuccess; }
    k_combine<<<(unsigned) ((tot + 255) / 256), 256, 0, st>>>(o, inv, wts, n, topk, E, P, resid, y, moe);
    return hipGetLastError();
}

}  // namespace lk
