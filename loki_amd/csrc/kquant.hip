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
// Work: a wave streams rows of one matrix; lane l owns the 32-weight chunks l, l + 64, .. of the row (chunk i = block
// i / 8, weights 32 (i % 8) .. +31), so the activation chunks stay in registers for every row of the wave's tile. A
// workgroup (4 waves) covers 4 * RW rows of one expert for all of that expert's slots (token groups of TT).
#include "moe_common.h"
#include "moe_kernels.h"

namespace lk {

namespace {

enum { KF_Q6K = 1, KF_Q5K = 3, KF_Q2K = 5, KF_Q3K = 6 };
template <int F> constexpr int kbytes() { return F == KF_Q2K ? 84 : F == KF_Q3K ? 110 : F == KF_Q5K ? 176 : 210; }

constexpr int RW = 16;          // rows per wave
constexpr int KQ_WAVES = 4;     // waves per workgroup

__device__ __forceinline__ uint32_t ld_u16(const uint8_t * p) { return *reinterpret_cast<const uint16_t *>(p); }

// N words from a 2-byte aligned address: aligned word loads, realigned with v_alignbyte. Only words that hold a needed
// byte are read, so a buffer whose start and size are multiples of 4 bytes is never overrun.
template <int N> __device__ __forceinline__ void ld_words_a2(const uint8_t * p, uint32_t (&w)[N]) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t * q = reinterpret_cast<const uint32_t *>(a & ~uintptr_t(3));
    const uint32_t sh = (uint32_t) (a & 3u);
    uint32_t t[N + 1];
#pragma unroll
    for (int i = 0; i < N; ++i) { t[i] = q[i]; }
    t[N] = sh ? q[N] : 0u;
#pragma unroll
    for (int i = 0; i < N; ++i) { w[i] = __builtin_amdgcn_alignbyte(t[i + 1], t[i], sh); }
}
template <int N> __device__ __forceinline__ void ld_words_a4(const uint8_t * p, uint32_t (&w)[N]) {
    const uint32_t * q = reinterpret_cast<const uint32_t *>(p);
#pragma unroll
    for (int i = 0; i < N; ++i) { w[i] = q[i]; }
}
__device__ __forceinline__ uint32_t byte_of3(uint32_t w0, uint32_t w1, uint32_t w2, int k) {
    const uint32_t w = k < 4 ? w0 : k < 8 ? w1 : w2;
    return (w >> (8 * (k & 3))) & 0xFFu;
}

// one 32-weight chunk of a block, decoded: u = unsigned quants (4 per word, weight order), per 16-weight half the scale
// sA/sB, the offset to remove (off * bsum), and min mA/mB (Q2_K: per half; Q5_K: one per chunk in mA, mB = mA)
struct Chunk {
    uint32_t u[8];
    int sA, sB, mA, mB;
    float d, dmin;
};

template <int F> __device__ __forceinline__ void load_chunk(const uint8_t * blk, int c, Chunk & k) {
    if constexpr (F == KF_Q2K) {   // scales[16] qs[64] d dmin: weight 128n + 32s + l = bits 2s of qs[32n + l]
        const int n = c >> 2, s = c & 3;
        uint32_t w[8]; ld_words_a4<8>(blk + 16 + 32 * n, w);
#pragma unroll
        for (int i = 0; i < 8; ++i) { k.u[i] = (w[i] >> (2 * s)) & 0x03030303u; }
        const uint32_t sc = ld_u16(blk + 2 * c);
        k.sA = (int) (sc & 15u); k.mA = (int) ((sc >> 4) & 15u); k.sB = (int) ((sc >> 8) & 15u); k.mB = (int) ((sc >> 12) & 15u);
        const uint32_t dd = *reinterpret_cast<const uint32_t *>(blk + 80);
        k.d = h2f((uint16_t) (dd & 0xFFFFu)); k.dmin = h2f((uint16_t) (dd >> 16));
    } else if constexpr (F == KF_Q3K) {   // hmask[32] qs[64] scales[12] d: high bit clear -> quant - 4
        const int n = c >> 2, s = c & 3;
        uint32_t q[8], h[8]; ld_words_a2<8>(blk + 32 + 32 * n, q); ld_words_a2<8>(blk, h);
        const int hb = 4 * n + s;
#pragma unroll
        for (int i = 0; i < 8; ++i) { k.u[i] = ((q[i] >> (2 * s)) & 0x03030303u) | (((h[i] >> hb) & 0x01010101u) << 2); }
        uint32_t a[3]; ld_words_a2<3>(blk + 96, a);
        // 6-bit scales j = 2c, 2c + 1: low nibbles from bytes (j % 8) (j < 8: low, else high nibble), 2 high bits from
        // byte 8 + j % 4 at bits 2 (j / 4)
        const int kk = c >> 1;
        const uint32_t lo = ((kk & 1 ? a[1] : a[0]) >> (kk & 2 ? 4 : 0)) & 0x0F0F0F0Fu;
        const uint32_t hi = ((a[2] >> (2 * kk)) & 0x03030303u) << 4;
        const uint32_t sw = (lo | hi) >> (16 * (c & 1));
        k.sA = (int) (sw & 0xFFu) - 32; k.sB = (int) ((sw >> 8) & 0xFFu) - 32; k.mA = 0; k.mB = 0;
        k.d = h2f((uint16_t) ld_u16(blk + 108)); k.dmin = 0.f;
    } else if constexpr (F == KF_Q5K) {   // d dmin scales[12] qh[32] qs[128]: weight 64 (c/2) + 32 (c%2) + l
        uint32_t l4[8], qh[8]; ld_words_a4<8>(blk + 48 + 32 * (c >> 1), l4); ld_words_a4<8>(blk + 16, qh);
        const int sh = 4 * (c & 1);
#pragma unroll
        for (int i = 0; i < 8; ++i) { k.u[i] = ((l4[i] >> sh) & 0x0F0F0F0Fu) | (((qh[i] >> c) & 0x01010101u) << 4); }
        uint32_t a[3]; ld_words_a4<3>(blk + 4, a);
        int s, m;
        if (c < 4) { s = (int) (byte_of3(a[0], a[1], a[2], c) & 63u); m = (int) (byte_of3(a[0], a[1], a[2], c + 4) & 63u); }
        else {
            const uint32_t b8 = byte_of3(a[0], a[1], a[2], c + 4);
            s = (int) ((b8 & 0xFu) | ((byte_of3(a[0], a[1], a[2], c - 4) >> 6) << 4));
            m = (int) ((b8 >> 4) | ((byte_of3(a[0], a[1], a[2], c) >> 6) << 4));
        }
        k.sA = s; k.sB = s; k.mA = m; k.mB = m;
        const uint32_t dd = *reinterpret_cast<const uint32_t *>(blk);
        k.d = h2f((uint16_t) (dd & 0xFFFFu)); k.dmin = h2f((uint16_t) (dd >> 16));
    } else {   // Q6_K: ql[128] qh[64] scales[16] d; weight 128n + 32p + l: nibble p/2 of ql[64n + 32 (p%2) + l], bits 2p of qh[32n + l], - 32
        const int n = c >> 2, p = c & 3;
        uint32_t l4[8], qh[8]; ld_words_a2<8>(blk + 64 * n + 32 * (p & 1), l4); ld_words_a2<8>(blk + 128 + 32 * n, qh);
#pragma unroll
        for (int i = 0; i < 8; ++i) { k.u[i] = ((l4[i] >> (4 * (p >> 1))) & 0x0F0F0F0Fu) | (((qh[i] >> (2 * p)) & 0x03030303u) << 4); }
        const uint32_t sc = ld_u16(blk + 192 + 2 * c);
        k.sA = (int) (int8_t) (sc & 0xFFu); k.sB = (int) (int8_t) (sc >> 8); k.mA = 0; k.mB = 0;
        k.d = h2f((uint16_t) ld_u16(blk + 208)); k.dmin = 0.f;
    }
}

struct XChunk { uint32_t x[8]; int bA, bB; float d8; };

__device__ __forceinline__ int dot8(const uint32_t * u, const uint32_t * x) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) { s = __builtin_amdgcn_sdot4((int) u[i], (int) x[i], s, false); }
    return s;
}

// integer partials of one chunk against one token: isum (scaled, offsets removed), summ (min term)
template <int F> __device__ __forceinline__ void chunk_dot(const Chunk & k, const XChunk & x, int & isum, int & summ) {
    const int dA = dot8(k.u, x.x), dB = dot8(k.u + 4, x.x + 4);
    if constexpr (F == KF_Q2K) { isum = k.sA * dA + k.sB * dB; summ = k.mA * x.bA + k.mB * x.bB; }
    else if constexpr (F == KF_Q3K) { isum = k.sA * (dA - 4 * x.bA) + k.sB * (dB - 4 * x.bB); summ = 0; }
    else if constexpr (F == KF_Q5K) { isum = k.sA * (dA + dB); summ = k.mA * (x.bA + x.bB); }
    else { isum = k.sA * (dA - 32 * x.bA) + k.sB * (dB - 32 * x.bB); summ = 0; }
}

__device__ __forceinline__ int red8(int v) {   // sum over the 8 lanes of an aligned group
    v += __shfl_xor(v, 1); v += __shfl_xor(v, 2); v += __shfl_xor(v, 4);
    return v;
}

template <int F, int NJ, int TT>
__global__ void __launch_bounds__(64 * KQ_WAVES) k_kq_matvec(KqArgs a) {
#pragma clang fp contract(off)
    constexpr int BS = kbytes<F>();
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int e, s_beg, s_end;
    if (a.act) {
        if ((int) blockIdx.y >= *a.nact) { return; }
        e = a.act[blockIdx.y]; s_beg = a.offsets[e]; s_end = a.offsets[e + 1];
    } else { e = 0; s_beg = 0; s_end = a.n; }
    const int r0 = ((int) blockIdx.x * KQ_WAVES + wv) * RW;
    if (r0 >= a.R || s_beg >= s_end) { return; }
    const int r1 = min(r0 + RW, a.R);
    const int nb = a.K / QK, nchunk = nb * 8;
    const size_t rowb = (size_t) nb * BS;
    const uint8_t * W = a.w + (size_t) e * a.estride;

    for (int sg = s_beg; sg < s_end; sg += TT) {
        const int nt = min(TT, s_end - sg);
        XChunk xc[TT][NJ];
#pragma unroll
        for (int t = 0; t < TT; ++t) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int ci = lane + 64 * j;
                XChunk & x = xc[t][j];
                if (t < nt && ci < nchunk) {
                    const int8_t * xr = a.aq + (size_t) (sg + t) * a.K + 32 * ci;
                    const uint4 v0 = *reinterpret_cast<const uint4 *>(xr), v1 = *reinterpret_cast<const uint4 *>(xr + 16);
                    x.x[0] = v0.x; x.x[1] = v0.y; x.x[2] = v0.z; x.x[3] = v0.w; x.x[4] = v1.x; x.x[5] = v1.y; x.x[6] = v1.z; x.x[7] = v1.w;
                    const uint32_t ones[4] = { 0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u };
                    x.bA = dot8(x.x, ones); x.bB = dot8(x.x + 4, ones);
                    x.d8 = a.ad[(size_t) (sg + t) * nb + (ci >> 3)];
                } else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) { x.x[i] = 0u; }
                    x.bA = 0; x.bB = 0; x.d8 = 0.f;
                }
            }
        }
        for (int r = r0; r < r1; ++r) {
            Chunk ck[NJ];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int ci = lane + 64 * j;
                if (ci < nchunk) { load_chunk<F>(W + (size_t) r * rowb + (size_t) (ci >> 3) * BS, ci & 7, ck[j]); }
                else {
#pragma unroll
                    for (int i = 0; i < 8; ++i) { ck[j].u[i] = 0u; }
                    ck[j].sA = ck[j].sB = ck[j].mA = ck[j].mB = 0; ck[j].d = 0.f; ck[j].dmin = 0.f;
                }
            }
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                if (t >= nt) { continue; }
                float term[NJ], termm[NJ];
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
                    int is, sm;
                    chunk_dot<F>(ck[j], xc[t][j], is, sm);
                    is = red8(is);
                    if constexpr (F == KF_Q2K || F == KF_Q5K) { sm = red8(sm); }
                    const float d8 = xc[t][j].d8;
                    if constexpr (F == KF_Q2K) { term[j] = (d8 * ck[j].d) * (float) is - (d8 * ck[j].dmin) * (float) sm; termm[j] = 0.f; }
                    else if constexpr (F == KF_Q5K) { term[j] = (ck[j].d * d8) * (float) is; termm[j] = (ck[j].dmin * d8) * (float) sm; }
                    else { term[j] = (ck[j].d * d8) * (float) is; termm[j] = 0.f; }
                }
                // blocks in order: block b sits in lanes 8 (b % 8) .. of chunk slot b / 8
                float acc = 0.f, accm = 0.f;
#pragma unroll
                for (int j = 0; j < NJ; ++j) {
#pragma unroll
                    for (int g = 0; g < 8; ++g) {
                        if (8 * j + g < nb) {
                            acc = acc + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, term[j]), 8 * g));
                            if constexpr (F == KF_Q5K) {
                                accm = accm - __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, termm[j]), 8 * g));
                            }
                        }
                    }
                }
                if constexpr (F == KF_Q5K) { acc = accm + acc; }
                if (lane == 0) { a.out[(size_t) (sg + t) * a.ldo + r] = acc; }
            }
        }
    }
}

template <int F, int NJ, int TT> hipError_t go(const KqArgs & a, unsigned gy, hipStream_t st) {
    const dim3 grid((unsigned) ((a.R + KQ_WAVES * RW - 1) / (KQ_WAVES * RW)), gy);
    k_kq_matvec<F, NJ, TT><<<grid, 64 * KQ_WAVES, 0, st>>>(a);
    return hipGetLastError();
}

template <int F> hipError_t go_f(const KqArgs & a, int nj, int tt, unsigned gy, hipStream_t st) {
    if (nj == 1) { return tt == 1 ? go<F, 1, 1>(a, gy, st) : tt == 2 ? go<F, 1, 2>(a, gy, st) : go<F, 1, 4>(a, gy, st); }
    if (nj == 2) { return tt == 1 ? go<F, 2, 1>(a, gy, st) : go<F, 2, 2>(a, gy, st); }
    return tt == 1 ? go<F, 4, 1>(a, gy, st) : go<F, 4, 2>(a, gy, st);
}

}  // namespace

int kq_block_bytes(int fmt) {
    switch (fmt) { case KF_Q2K: return 84; case KF_Q3K: return 110; case KF_Q5K: return 176; case KF_Q6K: return 210; default: return 0; }
}

hipError_t launch_kq_matvec(const KqArgs & a, int fmt, int max_slots, int grid_experts, hipStream_t st) {
    if (a.K <= 0 || a.K % QK || a.K > 8192 || a.R <= 0 || max_slots <= 0 || grid_experts <= 0 || kq_block_bytes(fmt) == 0) { return hipErrorInvalidValue; }
    const int nj = (a.K / QK * 8 + 63) / 64 <= 1 ? 1 : (a.K / QK * 8 + 63) / 64 <= 2 ? 2 : 4;
    const int tt = nj == 1 ? (max_slots <= 1 ? 1 : max_slots <= 2 ? 2 : 4) : (max_slots <= 1 ? 1 : 2);
    const unsigned gy = a.act ? (unsigned) grid_experts : 1u;
    switch (fmt) {
        case KF_Q2K: return go_f<KF_Q2K>(a, nj, tt, gy, st);
        case KF_Q3K: return go_f<KF_Q3K>(a, nj, tt, gy, st);
        case KF_Q5K: return go_f<KF_Q5K>(a, nj, tt, gy, st);
        default: return go_f<KF_Q6K>(a, nj, tt, gy, st);
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

}  // namespace lk
