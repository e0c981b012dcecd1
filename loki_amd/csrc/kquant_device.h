// kquant_device.h -- per-lane pieces of the K-quant x Q8_K block dot (Q2_K, Q3_K, Q5_K, Q6_K in ggml's block layout,
// read in place), shared by the K-quant mat-vec (kquant.hip) and the one-token decode block (moe_decode1.hip).
//
// A block's 256 weights are split over 8 lane slices q = 0..7; each slice's integer partials (isum, and summ for the
// formats with mins) are exact, and the 8 slices' sums (red8, or a lane's own loop) give ggml's integer block sums
// (ggml_vec_dot_q{2,3,5,6}_K_q8_K). The fp32 terms are formed by the callers in ggml's expressions.
#pragma once
#include "moe_device.h"

namespace lk {

enum { KF_Q6K = 1, KF_Q5K = 3, KF_Q2K = 5, KF_Q3K = 6 };
template <int F> constexpr int kbytes() { return F == KF_Q2K ? 84 : F == KF_Q3K ? 110 : F == KF_Q5K ? 176 : 210; }

constexpr int KQ_WAVES = 4;     // waves per workgroup

// Weight loads are buffer loads: a scalar resource over the expert's matrix, the lane's block offset (fixed for the
// whole launch) plus a field offset in one vector register, the row offset in a scalar register. Offsets past the
// resource's size read 0 instead of memory.
struct Src {
    __amdgpu_buffer_rsrc_t rs;
    uint32_t vb;      // this lane's block: b * block bytes
    uint32_t so;      // the current row: row * row bytes (wave-uniform)
};
__device__ __forceinline__ uint32_t ld32(const Src & s, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b32(s.rs, s.vb + off, s.so, 0); }
__device__ __forceinline__ uint32_t ld_u16(const Src & s, uint32_t off) { return (uint32_t) __builtin_amdgcn_raw_buffer_load_b16(s.rs, s.vb + off, s.so, 0); }
// several consecutive 4-byte aligned words in one load (load instructions, not bytes, limit these kernels)
typedef uint32_t u32v2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ u32v2 ld64(const Src & s, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b64(s.rs, s.vb + off, s.so, 0); }
__device__ __forceinline__ u32x4 ld128(const Src & s, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(s.rs, s.vb + off, s.so, 0); }

__device__ __forceinline__ uint32_t byte_of3(uint32_t w0, uint32_t w1, uint32_t w2, int k) {
    const uint32_t w = k < 4 ? w0 : k < 8 ? w1 : w2;
    return (w >> (8 * (k & 3))) & 0xFFu;
}

// Lane slice q (0..7) of a block. 16-weight sub-block formats (Q2_K, Q3_K, Q6_K): n = q / 4 picks the block half,
// jq = q % 4 the 8 columns l = 8 jq .. 8 jq + 7, taken in all four 32-weight rows s of the half: piece s = weights
// 128 n + 32 s + l (one sub-block, 2 words). Q5_K (32-weight sub-blocks, 64-weight quant groups jj): jj = q / 2,
// columns l = 16 (q % 2) .. + 15 of both halves h of the group: piece h = weights 64 jj + 32 h + l (sub-block 2 jj + h,
// 4 words). So each lane reads only the bytes of its own columns, 16 contiguous bytes per field.
template <int F> struct Raw;
template <> struct Raw<KF_Q2K> { uint32_t q[2], sc[2], dd; };
template <> struct Raw<KF_Q3K> { uint32_t q[3], h[3], s[4], dd; uint32_t shq, shh, shs; };
template <> struct Raw<KF_Q5K> { uint32_t q[4], h[4], s[3], dd; };
template <> struct Raw<KF_Q6K> { uint32_t qa[3], qb[3], h[3], sc[3], dd; uint32_t sha, shb, shh, shs; };

// N + 1 aligned words covering N words at a 2-byte aligned offset (rows and the matrix start on 4-byte boundaries, so
// the alignment is the lane's: block offset + field), in one vector load. Word N is needed only when the offset is
// not 4-aligned; past the matrix's last word the buffer load returns 0 instead of reading memory.
typedef uint32_t u32v3 __attribute__((ext_vector_type(3)));
template <int N> __device__ __forceinline__ uint32_t ld_aligned(const Src & s, uint32_t off, uint32_t (&t)[N + 1]) {
    static_assert(N == 2 || N == 3, "3- or 4-word windows");
    const uint32_t sh = (s.vb + off) & 3u, o = s.vb + off - sh;
    if constexpr (N == 2) {
        const u32v3 v = __builtin_amdgcn_raw_buffer_load_b96(s.rs, o, s.so, 0);
        t[0] = v.x; t[1] = v.y; t[2] = v.z;
    } else {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(s.rs, o, s.so, 0);
        t[0] = v.x; t[1] = v.y; t[2] = v.z; t[3] = v.w;
    }
    return sh;
}
template <int N> __device__ __forceinline__ uint32_t realign(const uint32_t (&t)[N + 1], uint32_t sh, int i) {
    return __builtin_amdgcn_alignbyte(t[i + 1], t[i], sh);
}

template <int F> __device__ __forceinline__ void load_raw(const Src & b, int q, Raw<F> & r) {
    const uint32_t n = (uint32_t) q >> 2, jq = (uint32_t) q & 3u;
    if constexpr (F == KF_Q2K) {   // scales[16] qs[64] d dmin
        const u32v2 q2 = ld64(b, 16 + 32 * n + 8 * jq), s2 = ld64(b, 8 * n);
        r.q[0] = q2.x; r.q[1] = q2.y; r.sc[0] = s2.x; r.sc[1] = s2.y;
        r.dd = ld32(b, 80);
    } else if constexpr (F == KF_Q3K) {   // hmask[32] qs[64] scales[12] d
        r.shq = ld_aligned<2>(b, 32 + 32 * n + 8 * jq, r.q); r.shh = ld_aligned<2>(b, 8 * jq, r.h);
        r.shs = ld_aligned<3>(b, 96, r.s); r.dd = ld_u16(b, 108);
    } else if constexpr (F == KF_Q5K) {   // d dmin scales[12] qh[32] qs[128]
        const uint32_t jj = (uint32_t) q >> 1, hf = (uint32_t) q & 1u;
        const u32x4 q4 = ld128(b, 48 + 32 * jj + 16 * hf), h4 = ld128(b, 16 + 16 * hf), hd = ld128(b, 0);   // qs, qh, d dmin scales
        r.q[0] = q4.x; r.q[1] = q4.y; r.q[2] = q4.z; r.q[3] = q4.w;
        r.h[0] = h4.x; r.h[1] = h4.y; r.h[2] = h4.z; r.h[3] = h4.w;
        r.dd = hd.x; r.s[0] = hd.y; r.s[1] = hd.z; r.s[2] = hd.w;
    } else {   // Q6_K: ql[128] qh[64] scales[16] d
        r.sha = ld_aligned<2>(b, 64 * n + 8 * jq, r.qa); r.shb = ld_aligned<2>(b, 64 * n + 32 + 8 * jq, r.qb);
        r.shh = ld_aligned<2>(b, 128 + 32 * n + 8 * jq, r.h); r.shs = ld_aligned<2>(b, 192 + 8 * n, r.sc);
        r.dd = ld_u16(b, 208);
    }
}

// decoded slice: u = unsigned quants (4 per word, an offset quant with its offset still added); piece p's scale sc[p]
// and min mn[p] (pieces: 4 of 2 words for the 16-weight formats, 2 of 4 words for Q5_K)
struct Chunk {
    uint32_t u[8];
    int sc[4], mn[4];
    float d, dmin;
};

// rotate right: bit b of the result is bit (b + n) % 32 of w. Moves a bit plane of every byte to another position in
// one instruction (no bit of another byte lands on the kept position: each caller masks one plane per byte).
__device__ __forceinline__ uint32_t rotr(uint32_t w, uint32_t n) { return __builtin_amdgcn_alignbit(w, w, n & 31u); }

template <int F> __device__ __forceinline__ void decode(const Raw<F> & r, int q, Chunk & k) {
    const int n = q >> 2, jq = q & 3, hi16 = jq >> 1;   // hi16: the columns sit in the second 16 of each 32-weight row
    if constexpr (F == KF_Q2K) {   // weight 128 n + 32 s + l = bits 2s of qs[32 n + l]; sub-block 8 n + 2 s + hi16
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            k.u[2 * s] = (r.q[0] >> (2 * s)) & 0x03030303u; k.u[2 * s + 1] = (r.q[1] >> (2 * s)) & 0x03030303u;
            const uint32_t o = 8u * (2 * (s & 1) + hi16);   // the sub-block's byte: scale nibble, min nibble
            k.sc[s] = (int) __builtin_amdgcn_ubfe(r.sc[s >> 1], o, 4u); k.mn[s] = (int) __builtin_amdgcn_ubfe(r.sc[s >> 1], o + 4u, 4u);
        }
        k.d = h2f((uint16_t) (r.dd & 0xFFFFu)); k.dmin = h2f((uint16_t) (r.dd >> 16));
    } else if constexpr (F == KF_Q3K) {   // high bit (hmask[l] bit 4 n + s) clear -> quant - 4 (the -4 is in the dot's start)
        const uint32_t q0 = realign<2>(r.q, r.shq, 0), q1 = realign<2>(r.q, r.shq, 1);
        const uint32_t h0 = realign<2>(r.h, r.shh, 0), h1 = realign<2>(r.h, r.shh, 1);
        const uint32_t a0 = realign<3>(r.s, r.shs, 0), a1 = realign<3>(r.s, r.shs, 1), a2 = realign<3>(r.s, r.shs, 2);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint32_t hr = (uint32_t) (4 * n + s) - 2u;   // hmask bit 4 n + s of each byte -> bit 2
            k.u[2 * s] = ((q0 >> (2 * s)) & 0x03030303u) | (rotr(h0, hr) & 0x04040404u);
            k.u[2 * s + 1] = ((q1 >> (2 * s)) & 0x03030303u) | (rotr(h1, hr) & 0x04040404u);
        }
        // 6-bit scale j = 8 n + 2 s + hi16: low nibble of byte j % 8 (nibble n), 2 high bits of byte 8 + j % 4 at
        // bits 2 (j / 4). The lane's four scales sit in bytes hi16 and hi16 + 2: s = 0, 1 in a0 / a2, s = 2, 3 in a1 /
        // a2 >> 2, so one shift per word puts each pair at bits 0 and 16 (the high bits by a rotate to bits 4, 5);
        // scale - 32 is the 6-bit field with its top bit flipped, read signed
        const uint32_t sh = 8 * hi16 + 4 * n;
        const uint32_t p01 = (((a0 >> sh) & 0x000F000Fu) | (rotr(a2, sh - 4u) & 0x00300030u)) ^ 0x00200020u;
        const uint32_t p23 = (((a1 >> sh) & 0x000F000Fu) | (rotr(a2, sh - 2u) & 0x00300030u)) ^ 0x00200020u;
        k.sc[0] = __builtin_amdgcn_sbfe((int) p01, 0u, 6u); k.sc[1] = __builtin_amdgcn_sbfe((int) p01, 16u, 6u);
        k.sc[2] = __builtin_amdgcn_sbfe((int) p23, 0u, 6u); k.sc[3] = __builtin_amdgcn_sbfe((int) p23, 16u, 6u);
        k.mn[0] = k.mn[1] = k.mn[2] = k.mn[3] = 0;
        k.d = h2f((uint16_t) r.dd); k.dmin = 0.f;
    } else if constexpr (F == KF_Q5K) {   // weight 64 jj + 32 h + l: nibble h of qs[32 jj + l], bit 2 jj + h of qh[l]
        const int jj = q >> 1;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int j = 2 * jj + h;
#pragma unroll
            for (int i = 0; i < 4; ++i) { k.u[4 * h + i] = ((r.q[i] >> (4 * h)) & 0x0F0F0F0Fu) | (rotr(r.h[i], (uint32_t) j - 4u) & 0x10101010u); }
            int sv, mv;
            if (j < 4) { sv = (int) (byte_of3(r.s[0], r.s[1], r.s[2], j) & 63u); mv = (int) (byte_of3(r.s[0], r.s[1], r.s[2], j + 4) & 63u); }
            else {
                const uint32_t b8 = byte_of3(r.s[0], r.s[1], r.s[2], j + 4);
                sv = (int) ((b8 & 0xFu) | ((byte_of3(r.s[0], r.s[1], r.s[2], j - 4) >> 6) << 4));
                mv = (int) ((b8 >> 4) | ((byte_of3(r.s[0], r.s[1], r.s[2], j) >> 6) << 4));
            }
            k.sc[h] = sv; k.mn[h] = mv;
        }
        k.sc[2] = k.sc[3] = k.mn[2] = k.mn[3] = 0;
        k.d = h2f((uint16_t) (r.dd & 0xFFFFu)); k.dmin = h2f((uint16_t) (r.dd >> 16));
    } else {   // Q6_K: weight 128 n + 32 p + l: nibble p / 2 of ql[64 n + 32 (p % 2) + l], bits 2 p of qh[32 n + l], - 32
        const uint32_t a0 = realign<2>(r.qa, r.sha, 0), a1 = realign<2>(r.qa, r.sha, 1);
        const uint32_t b0 = realign<2>(r.qb, r.shb, 0), b1 = realign<2>(r.qb, r.shb, 1);
        const uint32_t h0 = realign<2>(r.h, r.shh, 0), h1 = realign<2>(r.h, r.shh, 1);
        const uint32_t s0 = realign<2>(r.sc, r.shs, 0), s1 = realign<2>(r.sc, r.shs, 1);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t l0 = (p & 1) ? b0 : a0, l1 = (p & 1) ? b1 : a1;
            const uint32_t hr = (uint32_t) (2 * p) - 4u;   // qh bits 2 p, 2 p + 1 of each byte -> bits 4, 5
            k.u[2 * p] = ((l0 >> (4 * (p >> 1))) & 0x0F0F0F0Fu) | (rotr(h0, hr) & 0x30303030u);
            k.u[2 * p + 1] = ((l1 >> (4 * (p >> 1))) & 0x0F0F0F0Fu) | (rotr(h1, hr) & 0x30303030u);
            // scales[8 n + j], j = 2 p + hi16: byte j % 4 of s0 (j < 4) or s1, signed
            k.sc[p] = __builtin_amdgcn_sbfe((int) (p < 2 ? s0 : s1), 16u * (p & 1) + 8u * hi16, 8u); k.mn[p] = 0;
        }
        k.d = h2f((uint16_t) r.dd); k.dmin = 0.f;
    }
}

// the lane's activation words (same weight order as u), per piece the start value of its dot accumulator (the
// quants' offset folded in: Q3_K -4 * bsum, Q6_K -32 * bsum, else 0) and the sum of its Q8_K integers (bsum: the
// min term of Q2_K / Q5_K)
struct XChunk { uint32_t x[8]; int c0[4], bx[4]; float d8; };

// 8- and 16-byte activation reads from global memory or LDS
__device__ __forceinline__ uint4 kx16(const int8_t * p) { return *reinterpret_cast<const uint4 *>(p); }
__device__ __forceinline__ uint2 kx8(const int8_t * p) { return *reinterpret_cast<const uint2 *>(p); }
__device__ __forceinline__ uint4 kx16(const LK_LOCAL int8_t * p) {
    const u32x4 v = *reinterpret_cast<const LK_LOCAL u32x4 *>(p); return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 kx8(const LK_LOCAL int8_t * p) {
    const u32x2 v = *reinterpret_cast<const LK_LOCAL u32x2 *>(p); return make_uint2(v.x, v.y);
}
template <int F> __device__ __forceinline__ void x_starts(XChunk & x) {
#pragma unroll
    for (int s = 0; s < 4; ++s) { x.c0[s] = F == KF_Q3K ? -4 * x.bx[s] : F == KF_Q6K ? -32 * x.bx[s] : 0; }
}

// xb: the block's 256 Q8_K integers in element order (global memory or LDS)
template <int F, class P> __device__ __forceinline__ void load_x(P xb, int q, XChunk & x) {
    const uint32_t ones = 0x01010101u;
    if constexpr (F == KF_Q5K) {
        const int jj = q >> 1, hf = q & 1;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint4 v = kx16(xb + 64 * jj + 32 * h + 16 * hf);
            x.x[4 * h] = v.x; x.x[4 * h + 1] = v.y; x.x[4 * h + 2] = v.z; x.x[4 * h + 3] = v.w;
            int sm = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) { sm = __builtin_amdgcn_sdot4((int) x.x[4 * h + i], (int) ones, sm, false); }
            x.bx[h] = sm;
        }
        x.bx[2] = x.bx[3] = 0;
    } else {
        const int n = q >> 2, jq = q & 3;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint2 v = kx8(xb + 128 * n + 32 * s + 8 * jq);
            x.x[2 * s] = v.x; x.x[2 * s + 1] = v.y;
            x.bx[s] = __builtin_amdgcn_sdot4((int) v.y, (int) ones, __builtin_amdgcn_sdot4((int) v.x, (int) ones, 0, false), false);
        }
    }
    x_starts<F>(x);
}

// integer partials of the slice against one token: isum (scaled, offsets removed), summ (min term). Every factor fits
// 24 signed bits (scales and mins <= 8 bits, piece dots |.| < 2^17), so the products use the full-rate 24-bit multiply.
template <int F> __device__ __forceinline__ void chunk_dot(const Chunk & k, const XChunk & x, int & isum, int & summ) {
    isum = 0; summ = 0;
    if constexpr (F == KF_Q5K) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            int dp = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) { dp = __builtin_amdgcn_sdot4((int) k.u[4 * h + i], (int) x.x[4 * h + i], dp, false); }
            isum += __mul24(k.sc[h], dp);
            summ += __mul24(k.mn[h], x.bx[h]);
        }
    } else {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int dp = __builtin_amdgcn_sdot4((int) k.u[2 * s + 1], (int) x.x[2 * s + 1],
                                                  __builtin_amdgcn_sdot4((int) k.u[2 * s], (int) x.x[2 * s], x.c0[s], false), false);
            isum += __mul24(k.sc[s], dp);
            if constexpr (F == KF_Q2K) { summ += __mul24(k.mn[s], x.bx[s]); }
        }
    }
}

// sum over the 8 lanes of an aligned group, valid in the group's first lane: quad sums (DPP quad_perm), then lane i
// adds lane i + 4 (DPP row_shl:4)
__device__ __forceinline__ int red8(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);    // quad_perm [1,0,3,2]
    v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);    // quad_perm [2,3,0,1]
    v += __builtin_amdgcn_update_dpp(0, v, 0x104, 0xF, 0xF, false);   // row_shl:4
    return v;
}

}  // namespace lk
