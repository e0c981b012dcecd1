// moe_common.h -- device-side constants, tables and arithmetic contracts shared by the MoE-block kernels (gfx950).
//
// Formats (ggml's, as the reference's block uses them):
//   block_iq2_xxs = { fp16 d; u16 qs[32] } = 66 B per 256 weights (src/fused_layer.cu:19 BLK_IQ2 = 66). Sub-block ib
//   (32 weights) is the 8 bytes qs[4ib..4ib+3]: a0 = 4 codebook indices, a1 = 4x7 sign bits + 4-bit scale (a1 >> 28).
//   Q8_K activations: per 256 values an fp32 d and 256 int8 (quantize_row_q8_K_ref).
// Tiled layout (this build's resident layout, produced once by fl_pack_iq2xxs): a matrix of R rows x K columns is cut
// into units of 4 rows x 4 blocks (R % 4 == 0, K % 1024 == 0); a unit is 1056 B = 16 blocks' qs (row-major over
// (row, block), 64 B each) followed by their 16 fp16 d. Units are ordered row-quad major, then block-quad. The total
// size equals ggml's (66 B per block); a 64-lane wave reads one unit with one 16-byte load per lane.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace lk {

constexpr int QK = 256;             // weights per block
constexpr int IQ2B = 66;            // bytes per IQ2_XXS block
constexpr int UROWS = 4, UBLK = 4;  // tiled unit: 4 rows x 4 blocks
constexpr int UNIT = 1056;          // bytes per unit
constexpr int MAXK = 8;             // top-k per token supported by the fused kernels
constexpr int NEXP_MAX = 256;       // experts per layer supported by the device router/dispatch

enum { LAYOUT_GGML = 0, LAYOUT_TILED = 1 };

// IQ2_XXS codebook (format constant, identical to ggml's iq2xxs_grid)
static __device__ const uint64_t g_iq2xxs_grid[256] = {
#include "iq2xxs_grid.inc"
};

__device__ __forceinline__ uint32_t ksigns8(uint32_t i7) {   // 7 stored sign bits + parity bit 7
    return i7 | ((__builtin_popcount(i7) & 1u) << 7);
}

// byte masks 0x00/0xFF for the 8 signs of one 8-weight group: lo = weights 0..3, hi = 4..7
__device__ __forceinline__ uint64_t sign_mask64(uint32_t s8) {
    uint64_t m = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) { m |= (uint64_t) (((s8 >> j) & 1u) * 0xFFu) << (8 * j); }
    return m;
}

// LDS tables used by the IQ2 kernels: the codebook (2 KB) and the 128 sign masks (1 KB).
struct Iq2Lds {
    uint64_t grid[256];
    uint64_t smask[128];
};

__device__ __forceinline__ void iq2_lds_fill(Iq2Lds & t) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) { t.grid[i] = g_iq2xxs_grid[i]; }
    for (int i = threadIdx.x; i < 128; i += blockDim.x) { t.smask[i] = sign_mask64(ksigns8((uint32_t) i)); }
}

// signed int8 weights of one 8-group: grid magnitudes with the group's signs applied. Grid bytes are never 0, so the
// per-byte two's-complement negation (g ^ 0xFF) + 1 never carries into the next byte and plain 32-bit ops suffice.
__device__ __forceinline__ void iq2_group(const Iq2Lds & t, uint32_t a0, uint32_t a1, int l, int & lo, int & hi) {
    const uint64_t g = t.grid[(a0 >> (8 * l)) & 255u];
    const uint64_t m = t.smask[(a1 >> (7 * l)) & 127u];
    const uint32_t glo = (uint32_t) g, ghi = (uint32_t) (g >> 32), mlo = (uint32_t) m, mhi = (uint32_t) (m >> 32);
    lo = (int) ((glo ^ mlo) + (mlo & 0x01010101u));
    hi = (int) ((ghi ^ mhi) + (mhi & 0x01010101u));
}

// exact int32 dot of one sub-block (32 weights) with 32 int8 activations (8 dwords)
__device__ __forceinline__ int iq2_sub_dot(const Iq2Lds & t, uint32_t a0, uint32_t a1, const int * xv) {
    int s = 0;
#pragma unroll
    for (int l = 0; l < 4; ++l) {
        int lo, hi; iq2_group(t, a0, a1, l, lo, hi);
        s = __builtin_amdgcn_sdot4(lo, xv[2 * l], s, false);
        s = __builtin_amdgcn_sdot4(hi, xv[2 * l + 1], s, false);
    }
    return s;
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

}  // namespace lk
