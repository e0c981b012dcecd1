// moe_common.h -- device-side constants, tables and arithmetic contracts shared by the MoE-block kernels (gfx950).
//
// Formats (ggml's, as the reference's block uses them):
//   block_iq2_xxs = { fp16 d; u16 qs[32] } = 66 B per 256 weights (src/fused_layer.cu:19 BLK_IQ2 = 66). Sub-block ib
//   (32 weights) is the 8 bytes qs[4ib..4ib+3]: a0 = 4 codebook indices (byte l = group l), a1 = 4 x 7 sign bits
//   (bits 7l..7l+6 = group l) + the 4-bit scale nibble (a1 >> 28).
//   Q8_K activations: per 256 values an fp32 d and 256 int8 (quantize_row_q8_K_ref).
//
// Tiled layout (the resident layout, produced once by fl_pack_iq2xxs; same 66 B per block). A matrix of R rows x K
// columns (R % 64 == 0, K % 1024 == 0, nb = K / 256 blocks per row) is stored as
//   qs region: [R/64 row groups][nb blocks][4 chunks][64 rows][16 B]   -- chunk c = qs bytes 16c..16c+15 of the block
//   d region : [R/64 row groups][nb blocks][64 rows] fp16              -- after the qs region
// so a 64-lane wave that owns 64 rows reads each 16-byte chunk of a block with one fully coalesced 1 KB load.
// Inside every sub-block the sign word is re-packed (lossless): byte l holds group l's 7 sign bits in bits 0..6 and bit l
// of the scale nibble in bit 7, so a byte select addresses the sign table and one udot4 rebuilds 2 * nibble + 1.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace lk {

constexpr int QK = 256;             // weights per block
constexpr int IQ2B = 66;            // bytes per IQ2_XXS block
constexpr int RG = 64;              // rows per row group (one wave, one row per lane)
constexpr int MAXK = 8;             // top-k per token supported by the fused kernels
constexpr int NEXP_MAX = 256;       // experts per layer supported by the device router/dispatch

enum { LAYOUT_GGML = 0, LAYOUT_TILED = 1 };

// IQ2_XXS codebook (format constant, identical to ggml's iq2xxs_grid)
static __device__ const uint64_t g_iq2xxs_grid[256] = {
#include "iq2xxs_grid.inc"
};

__host__ __device__ inline uint32_t ksigns8(uint32_t i7) {   // 7 stored sign bits + parity bit 7
    return i7 | ((__builtin_popcount(i7) & 1u) << 7);
}

// byte masks 0x00/0xFF for the 8 signs of one 8-weight group: lo = weights 0..3, hi = 4..7
__host__ __device__ inline uint64_t sign_mask64(uint32_t s8) {
    uint64_t m = 0;
    for (int j = 0; j < 8; ++j) { m |= (uint64_t) (((s8 >> j) & 1u) * 0xFFu) << (8 * j); }
    return m;
}

// sign word <-> tiled sign word (lossless permutation of the 32 bits)
__host__ __device__ inline uint32_t a1_to_tiled(uint32_t a1) {
    uint32_t o = 0;
    for (int l = 0; l < 4; ++l) { o |= (((a1 >> (7 * l)) & 127u) | (((a1 >> (28 + l)) & 1u) << 7)) << (8 * l); }
    return o;
}
__host__ __device__ inline uint32_t a1_from_tiled(uint32_t t) {
    uint32_t a = 0;
    for (int l = 0; l < 4; ++l) { a |= ((t >> (8 * l)) & 127u) << (7 * l); a |= ((t >> (8 * l + 7)) & 1u) << (28 + l); }
    return a;
}

// byte offsets inside one tiled matrix
__host__ __device__ inline size_t tiled_qs_off(int rg, int j, int c, int nb) { return ((size_t) (rg * nb + j) * 4 + c) * 1024; }
__host__ __device__ inline size_t tiled_d_off(int rg, int j, int row, int R, int nb) {
    return (size_t) (R / RG) * nb * 4096 + ((size_t) (rg * nb + j) * RG + row) * 2;
}

// ---------------------------------------------------------------- LDS tables
// Codebook: entry e (0..255) owns the 256-byte line [256 e, 256 e + 256) = 32 copies of grid[e]; lane l reads copy
// l % 32, so the 32 lanes an LDS pass serves for an 8-byte read always hit 32 different bank pairs. Signs: the 7 stored
// sign bits b (0..127) own the line at 65536 + 256 b = 16 copies of the 16-byte entry {m, m & 0x01010101 per 4
// weights} (m = byte masks 0x00 / 0xFF of the 8 signs, parity included), so applying the signs is one v_xad_u32 per 4
// weights; lane l reads copy l % 16 (16 lanes per pass for 16-byte reads). The byte address is (index << 8) | copy
// offset, which one v_perm_b32 builds from the packed index word (sign words masked to their 7 stored bits first: bit
// 7 of each byte is a scale bit). The image is built once per context (build_table_image) and copied into LDS by every
// workgroup (tables_copy).
constexpr int TAB_GRID = 256 * 256, TAB_BYTES = TAB_GRID + 128 * 256;

__device__ __forceinline__ uint32_t xad(uint32_t a, uint32_t b, uint32_t c) { return (a ^ b) + c; }   // one v_xad_u32

// explicit address spaces: loads through generic pointers would compile to FLAT instructions, which also count against
// lgkmcnt and so make every LDS wait a wait for the outstanding global loads as well
#define LK_GLOBAL __attribute__((address_space(1)))
#define LK_LOCAL __attribute__((address_space(3)))
#define LK_CONST __attribute__((address_space(4)))   // kernel arguments: scalar loads, counted apart from vector memory
template <class T> __device__ __forceinline__ const LK_GLOBAL T * gptr(const T * p) { return (const LK_GLOBAL T *) p; }
template <class T> __device__ __forceinline__ LK_GLOBAL T * gptr(T * p) { return (LK_GLOBAL T *) p; }
__device__ __forceinline__ uint32_t lds_addr(const void * p) { return (uint32_t) (size_t) (const LK_LOCAL uint8_t *) p; }
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 gload16(const void * p) { const u32x4 v = *(const LK_GLOBAL u32x4 *) p; return make_uint4(v.x, v.y, v.z, v.w); }
__device__ __forceinline__ uint2 gload8(const void * p) { const u32x2 v = *(const LK_GLOBAL u32x2 *) p; return make_uint2(v.x, v.y); }
__device__ __forceinline__ float4 gloadf4(const void * p) { const f32x4 v = *(const LK_GLOBAL f32x4 *) p; return make_float4(v.x, v.y, v.z, v.w); }
__device__ __forceinline__ uint2 lload8(uint32_t addr) { const u32x2 v = *(const LK_LOCAL u32x2 *) (size_t) addr; return make_uint2(v.x, v.y); }
__device__ __forceinline__ uint4 lload16(uint32_t addr) { const u32x4 v = *(const LK_LOCAL u32x4 *) (size_t) addr; return make_uint4(v.x, v.y, v.z, v.w); }
// a lane's table words over the table base (64 KB aligned): grid copy (lane % 32) * 8; sign copy (lane % 16) * 16 in
// the sign half (derived from the grid word)
__device__ __forceinline__ uint32_t tab_word_grid(uint32_t base, int lane) { return base | ((uint32_t) (lane & 31) << 3); }
__device__ __forceinline__ uint32_t tab_sign_word(uint32_t tr) { return ((tr & ~255u) + (uint32_t) TAB_GRID) | ((tr & 0x78u) << 1); }
constexpr uint32_t SIGN_BITS = 0x7f7f7f7fu;   // the stored sign bits of a tiled sign word

// LDS byte address of the table entry for byte L of an index word: byte 1 = that byte; bytes 0, 2, 3 from `tr` = the
// table base (64 KB aligned) | the lane's replica offset
template <int L> __device__ __forceinline__ uint32_t tab_addr(uint32_t word, uint32_t tr) {
    return __builtin_amdgcn_perm(word, tr, 0x03020000u | ((4u + L) << 8));
}

// signed int8 weights of a group from its codebook word g and sign masks m: magnitudes with the signs applied. Grid bytes
// are never 0, so the per-byte two's-complement negation (g ^ 0xFF) + 1 never carries into the next byte.
__device__ __forceinline__ void iq2_apply(uint2 g, uint4 m, uint32_t & lo, uint32_t & hi) {
    lo = xad(g.x, m.x, m.z);
    hi = xad(g.y, m.y, m.w);
}
// tr / trs: this lane's grid / sign table words; a1m = a tiled sign word masked with SIGN_BITS
template <int L> __device__ __forceinline__ uint2 tab_grid(uint32_t a0, uint32_t tr) { return lload8(tab_addr<L>(a0, tr)); }
template <int L> __device__ __forceinline__ uint4 tab_sign(uint32_t a1m, uint32_t trs) { return lload16(tab_addr<L>(a1m, trs)); }

// 2 * scale nibble + 1 of a tiled sign word (nibble bit l = bit 7 of byte l)
__device__ __forceinline__ int iq2_scale(uint32_t a1t) {
    return (int) __builtin_amdgcn_udot4((a1t >> 7) & 0x01010101u, 0x10080402u, 1u, false);
}

// Activation rows of the MFMA GEMMs in LDS: a row (one token's 256-value block: 32 chunks of 16 B in a 512-byte row)
// keeps chunk c at slot pf_swz(c) ^ r, r = row % 16 (flips only the low four bits). gfx950 serves a ds_read_b128 in
// four passes of 16 lanes, each pass the lanes with equal bit 5 and equal (bit 4 ^ bit 3) of the lane id; a lane's bank
// quad is its slot mod 16. In the GEMMs lane (r, g) = 16 g + r reads row r: a pass holds every r once, g's bit 1 fixed
// and g's bit 0 = bit 3 of r ^ const. Chunk c's bits 3 and 4 being g's bits 0 and 1, pf_swz (which swaps them) moves
// g's bit 0 out of the slot's low four bits: the 16 lanes of a pass read 16 different bank quads. With the plain slot
// c ^ r two lanes of every pass would share one.
__device__ __forceinline__ uint32_t pf_swz(uint32_t c) { return (c & 7u) | ((c & 8u) << 1) | ((c & 16u) >> 1); }

__device__ __forceinline__ uint4 load_nt(const uint8_t * p) {   // streaming (non-temporal) 16-byte global load
    const u32x4 v = __builtin_nontemporal_load((const LK_GLOBAL u32x4 *) p);
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }

// ---------------------------------------------------------------- exp contract (bit-identical to the CPU checker)
// fp64 Cody-Waite reduction with a 29-bit head of ln2, degree-13 Taylor polynomial in Horner form, 2^k through the
// exponent field, one rounding to fp32. Contraction is off, so every step is one IEEE-rounded fp64 operation.
__device__ __forceinline__ double det_exp(double t) {
#pragma clang fp contract(off)
    t = t < -110.0 ? -110.0 : t; t = t > 90.0 ? 90.0 : t;
    const double inv_ln2 = 0x1.71547652b82fep+0, ln2_hi = 0x1.62e42ffp-1, ln2_lo = -0x1.718432a1b0e26p-35;
    const double kd = floor(t * inv_ln2 + 0.5);
    const double r = (t - kd * ln2_hi) - kd * ln2_lo;
    double p = 0x1.6124613a86d09p-33;
    p = p * r + 0x1.1eed8eff8d898p-29;
    p = p * r + 0x1.ae64567f544e4p-26;
    p = p * r + 0x1.27e4fb7789f5cp-22;
    p = p * r + 0x1.71de3a556c734p-19;
    p = p * r + 0x1.a01a01a01a01ap-16;
    p = p * r + 0x1.a01a01a01a01ap-13;
    p = p * r + 0x1.6c16c16c16c17p-10;
    p = p * r + 0x1.1111111111111p-7;
    p = p * r + 0x1.5555555555555p-5;
    p = p * r + 0x1.5555555555555p-3;
    p = p * r + 0x1.0p-1;
    p = p * r + 1.0;
    p = p * r + 1.0;
    const int k = (int) kd;
    return p * __longlong_as_double((long long) (k + 1023) << 52);
}
__device__ __forceinline__ float det_expf(float x) { return x != x ? x : (float) det_exp((double) x); }
__device__ __forceinline__ float det_silu(float x) {
#pragma clang fp contract(off)
    return x / (1.0f + det_expf(-x));
}
__device__ __forceinline__ float det_sigmoid(float x) {
#pragma clang fp contract(off)
    return 1.0f / (1.0f + det_expf(-x));
}

// ---------------------------------------------------------------- wave helpers (wave64)
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Q8_K of one 256-value block by one wave (quantize_row_q8_K_ref): lane l handles values 4l..4l+3
__device__ __forceinline__ void q8k_block_wave(const float * __restrict__ xb, int8_t * __restrict__ qb, float * __restrict__ db) {
    const int lane = lane_id();
    const float4 v = reinterpret_cast<const float4 *>(xb)[lane];
    const float xs[4] = { v.x, v.y, v.z, v.w };
    float ba = -1.f, bv = 0.f; int bi = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) { const float ax = fabsf(xs[i]); if (ax > ba) { ba = ax; bv = xs[i]; bi = 4 * lane + i; } }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {   // first occurrence of the largest |x|: larger |x| wins, ties to the lower index
        const float oa = __shfl_xor(ba, off), ov = __shfl_xor(bv, off); const int oi = __shfl_xor(bi, off);
        if (oa > ba || (oa == ba && oi < bi)) { ba = oa; bv = ov; bi = oi; }
    }
    uint32_t packed = 0; float d = 0.f;
    if (ba > 0.f) {
        const float iscale = -127.f / bv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = iscale * xs[i];
            int iv = (int) rintf(p); iv = iv < 127 ? iv : 127;
            packed |= ((uint32_t) (iv & 0xff)) << (8 * i);
        }
        d = 1.f / iscale;
    }
    reinterpret_cast<uint32_t *>(qb)[lane] = packed;
    if (lane == 0) { *db = d; }
}

}  // namespace lk
