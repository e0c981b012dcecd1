// kquant.hip -- mat-vecs of K-quant matrices (Q2_K, Q3_K, Q5_K, Q6_K, ggml block layout, read in place) on Q8_K
// activations: the formats of the reference's real shards, routed down Q2_K / Q3_K (src/fused_layer.cu:203-254, 608) and
// shared expert Q5_K / Q5_K / Q6_K (src/fused_layer.cu:102-158, 520-524).
//
// Arithmetic. Every product of a sub-block (16 or 32 weights sharing one 6/4-bit scale) is an exact int8 x int8 dot
// (v_dot4_i32_i8); the integer block sums are those of ggml's scalar routines (ggml_vec_dot_q{2,3,5,6}_K_q8_K): isum =
// sum_j scale_j * sum(q * x), and for Q2_K / Q5_K the min term sum_j min_j * bsum_j (bsums = 16-value sums of the
// Q8_K integers, formed here from the integers themselves). Quants with an offset (Q3_K: -4 where the high bit is
// clear; Q6_K: -32) are dotted unsigned and corrected by offset * bsum. The fp32 part runs over the blocks in order:
//   Q2_K:        acc += (d8 * d) * isum - (d8 * dmin) * summ          (ggml's order: bit-identical to the scalar code)
//   Q3_K, Q6_K:  acc += (d * d8) * isum                               (ggml keeps 8 partial sums split by column % 8;
//   Q5_K:        acc_s += (d * d8) * isum, acc_m -= (dmin * d8) * summ, result acc_m + acc_s    these differ from
//                ggml's by fp32 rounding of the partial sums only)
//
// Work: a workgroup (4 waves) takes one expert, a tile of rows and that expert's slots in token groups of up to 8 (their
// Q8_K columns held in registers). Lane = (block, column slice of 32 weights); a row's blocks are split over 1-4 waves (8 blocks per
// wave), the remaining waves take other rows of the tile. The next row's bytes are loaded while the current one is
// computed. Each block's fp32 term goes to LDS; one lane per (row, token) then adds them in block order.
#include "kquant_device.h"
#include "moe_kernels.h"

#include <algorithm>

namespace lk {

namespace {

constexpr int RT_MAX = 32;      // rows per workgroup tile
constexpr int NB_MAX = 32;      // blocks per row (K <= 8192)

// Workgroup: one expert, a tile of rt rows, token groups of TT. The row's blocks are split over wk waves (8 blocks
// per wave, lane = (block, column slice)); the 4 / wk wave groups take the tile's rows in turn. Each block's fp32 term goes
// to LDS; then one lane per (row, token) adds the terms in block order.
template <int F, int TT>
__global__ void __launch_bounds__(64 * KQ_WAVES) k_kq_matvec(KqArgs a) {
#pragma clang fp contract(off)
    constexpr int BS = kbytes<F>();
    constexpr bool MINS = F == KF_Q5K;
    extern __shared__ float s_lds[];   // [rw][TT][nb] terms, then the min terms (Q5_K)
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
    int e, s_beg, s_end;
    if (a.act) {
        if ((int) blockIdx.y >= *a.nact) { return; }
        e = a.act[blockIdx.y]; s_beg = a.offsets[e]; s_end = a.offsets[e + 1];
    } else { e = 0; s_beg = 0; s_end = a.n; }
    const bool second = !a.act && blockIdx.y == 1;   // the second matrix (w2 -> out2)
    const uint8_t * Wm = second ? a.w2 : a.w;
    float * Out = second ? a.out2 : a.out;
    const int tr0 = (int) blockIdx.x * a.rw;
    if (tr0 >= a.R || s_beg >= s_end) { return; }
    const int nrow = min(a.rw, a.R - tr0);
    const int nb = a.K / QK;
    float * s_t = s_lds; float * s_m = s_lds + a.rw * TT * nb;
    const int wk = (nb + 7) / 8, wr = KQ_WAVES / wk;          // waves along K, wave groups along rows
    const int kw = wv % wk, rg = wv / wk;
    const int b = 8 * kw + (lane >> 3), c = lane & 7;          // this lane's block and column slice
    const bool active = rg < wr && b < nb;
    const uint32_t rowb = (uint32_t) (nb * BS);
    Src src;
    {
        const uint8_t * W = Wm + (size_t) e * a.estride;
        const uint64_t wv = (uint64_t) W;   // wave-uniform: kept in scalar registers
        const uint32_t hi = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) (wv >> 32));
        const uint32_t lo = (uint32_t) __builtin_amdgcn_readfirstlane((int) (uint32_t) wv);
        const uint64_t mb = (uint64_t) a.R * rowb;
        src.rs = __builtin_amdgcn_make_buffer_rsrc((void *) (((uint64_t) hi << 32) | lo), (short) 0,
                                                   (int) (mb < 0x7fffffffull ? mb : 0x7fffffffull), 0x00020000);
        src.vb = (uint32_t) (b * BS); src.so = 0;
    }

    for (int sg = s_beg; sg < s_end; sg += TT) {
        const int nt = min(TT, s_end - sg);
        XChunk xc[TT];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
            XChunk & x = xc[t];
            if (active && t < nt) {
                load_x<F>(a.aq + (size_t) (sg + t) * a.K + 256 * b, c, x);
                x.d8 = a.ad[(size_t) (sg + t) * nb + b];
            } else {
#pragma unroll
                for (int i = 0; i < 8; ++i) { x.x[i] = 0u; }
#pragma unroll
                for (int i = 0; i < 4; ++i) { x.c0[i] = 0; x.bx[i] = 0; }
                x.d8 = 0.f;
            }
        }
        if (active) {
            auto row = [&](const Raw<F> & raw, int ri) {
                Chunk ck; decode<F>(raw, c, ck);
#pragma unroll
                for (int t = 0; t < TT; ++t) {
                    if (t < nt) {
                        int is, sm;
                        chunk_dot<F>(ck, xc[t], is, sm);
                        is = red8(is);
                        if constexpr (F == KF_Q2K || F == KF_Q5K) { sm = red8(sm); }
                        if (c == 0) {
                            const float d8 = xc[t].d8;
                            float term;
                            if constexpr (F == KF_Q2K) { term = (d8 * ck.d) * (float) is - (d8 * ck.dmin) * (float) sm; }
                            else { term = (ck.d * d8) * (float) is; }
                            s_t[(ri * TT + t) * nb + b] = term;
                            if constexpr (MINS) { s_m[(ri * TT + t) * nb + b] = (ck.dmin * d8) * (float) sm; }
                        }
                    }
                }
            };
            // two row buffers: the next row's bytes are in flight while the current row is computed
            const uint32_t step = (uint32_t) wr * rowb;
            Src sp = src; sp.so = (uint32_t) (tr0 + rg) * rowb;
            Raw<F> ra, rb;
            int ri = rg;
            if (ri < nrow) { load_raw<F>(sp, c, ra); }
            while (ri < nrow) {
                if (ri + wr < nrow) { Src sn = sp; sn.so += step; load_raw<F>(sn, c, rb); }
                row(ra, ri);
                ri += wr; sp.so += step;
                if (ri >= nrow) { break; }
                if (ri + wr < nrow) { Src sn = sp; sn.so += step; load_raw<F>(sn, c, ra); }
                row(rb, ri);
                ri += wr; sp.so += step;
            }
        }
        __syncthreads();
        // blocks in order, one lane per (row, token)
        for (int p = threadIdx.x; p < nrow * nt; p += 64 * KQ_WAVES) {
            const int ri = p / nt, t = p % nt;
            const float * tp = s_t + (ri * TT + t) * nb;
            float acc = 0.f;
            if constexpr (MINS) {
                const float * mp = s_m + (ri * TT + t) * nb;
                float accm = 0.f;
                for (int j = 0; j < nb; ++j) { acc = acc + tp[j]; accm = accm - mp[j]; }
                acc = accm + acc;
            } else {
                for (int j = 0; j < nb; ++j) { acc = acc + tp[j]; }
            }
            Out[(size_t) (sg + t) * a.ldo + tr0 + ri] = acc;
        }
        __syncthreads();
    }
}

template <int F, int TT> hipError_t go(const KqArgs & a, unsigned gy, hipStream_t st) {
    const dim3 grid((unsigned) ((a.R + a.rw - 1) / a.rw), gy);
    const size_t lds = (size_t) a.rw * TT * (a.K / QK) * sizeof(float) * (F == KF_Q5K ? 2 : 1);
    k_kq_matvec<F, TT><<<grid, 64 * KQ_WAVES, lds, st>>>(a);
    return hipGetLastError();
}

template <int F> hipError_t go_f(const KqArgs & a, int tt, unsigned gy, hipStream_t st) {
    return tt == 1 ? go<F, 1>(a, gy, st) : tt == 2 ? go<F, 2>(a, gy, st) : tt == 4 ? go<F, 4>(a, gy, st) : go<F, 8>(a, gy, st);
}

}  // namespace

int kq_block_bytes(int fmt) {
    switch (fmt) { case KF_Q2K: return 84; case KF_Q3K: return 110; case KF_Q5K: return 176; case KF_Q6K: return 210; default: return 0; }
}

hipError_t launch_kq_matvec(const KqArgs & args, int fmt, int max_slots, int grid_experts, hipStream_t st) {
    KqArgs a = args;
    if (a.K <= 0 || a.K % QK || a.K > QK * NB_MAX || a.R <= 0 || max_slots <= 0 || grid_experts <= 0 || kq_block_bytes(fmt) == 0) { return hipErrorInvalidValue; }
    const int tt = max_slots <= 1 ? 1 : max_slots <= 2 ? 2 : max_slots <= 4 ? 4 : 8;
    // rows per workgroup tile: RT_MAX when the launch has rows enough, else fewer so that it still spreads over ~1024
    // workgroups (~512 for token groups of 8: every workgroup loads the group's activations for its whole K range, so
    // two rows per workgroup re-read them 5.8x the Q5_K weights' bytes; the 10 MB shared gate at 8 tokens takes 17.4 us
    // over 1024 workgroups, 13.0 over 512, while a 1-token launch is fastest over 1024)
    const int64_t rows_total = (int64_t) a.R * (a.act ? grid_experts : (a.w2 ? 2 : 1));
    a.rw = (int) std::max<int64_t>(1, std::min<int64_t>(RT_MAX, rows_total / (tt >= 8 ? 512 : 1024)));
    const unsigned gy = a.act ? (unsigned) grid_experts : (a.w2 ? 2u : 1u);
    switch (fmt) {
        case KF_Q2K: return go_f<KF_Q2K>(a, tt, gy, st);
        case KF_Q3K: return go_f<KF_Q3K>(a, tt, gy, st);
        case KF_Q5K: return go_f<KF_Q5K>(a, tt, gy, st);
        default: return go_f<KF_Q6K>(a, tt, gy, st);
    }
}

// h = silu(g) * u under the library's exp contract (the reference's SwiGLU of the K-quant shared expert)
__global__ void k_swiglu(const float * __restrict__ g, const float * __restrict__ u, int64_t n, float * __restrict__ h) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i < n) { h[i] = det_silu(g[i]) * u[i]; }
}
hipError_t launch_swiglu(const float * g, const float * u, int64_t n, float * h, hipStream_t st) {
    if (n <= 0) { return hipSuccess; }
    k_swiglu<<<(unsigned) ((n + 255) / 256), 256, 0, st>>>(g, u, n, h);
    return hipGetLastError();
}

// the same h, and its Q8_K (ggml's quantize_row_q8_K: q8k_lane over one 256-value block per wave, 4 values per lane in
// element order), in one pass
__global__ void __launch_bounds__(256) k_swiglu_q8k(const float * __restrict__ g, const float * __restrict__ u, int64_t nblk,
                                                    float * __restrict__ h, int8_t * __restrict__ q, float * __restrict__ d) {
#pragma clang fp contract(off)
    const int64_t b = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblk) { return; }
    const int lane = threadIdx.x & 63;
    const int64_t i0 = b * QK + 4 * lane;
    const float4 gv = *reinterpret_cast<const float4 *>(g + i0), uv = *reinterpret_cast<const float4 *>(u + i0);
    const float xs[4] = { det_silu(gv.x) * uv.x, det_silu(gv.y) * uv.y, det_silu(gv.z) * uv.z, det_silu(gv.w) * uv.w };
    *reinterpret_cast<float4 *>(h + i0) = make_float4(xs[0], xs[1], xs[2], xs[3]);
    float dq;
    const uint32_t packed = q8k_lane(xs, dq);
    *reinterpret_cast<uint32_t *>(q + i0) = packed;
    if (lane == 0) { d[b] = dq; }
}
hipError_t launch_swiglu_q8k(const float * g, const float * u, int64_t nrows, int K, float * h, int8_t * q, float * d, hipStream_t st) {
    if (nrows <= 0) { return hipSuccess; }
    if (K <= 0 || K % QK) { return hipErrorInvalidValue; }
    const int64_t nblk = nrows * (K / QK);
    k_swiglu_q8k<<<(unsigned) ((nblk + 3) / 4), 256, 0, st>>>(g, u, nblk, h, q, d);
    return hipGetLastError();
}

}  // namespace lk
