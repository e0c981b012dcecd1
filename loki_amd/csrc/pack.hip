// pack.hip -- IQ2_XXS layout conversion (ggml <-> tiled) and the synthetic-data generators used by tests and bench.
//
// The reference reads experts in ggml's layout straight from its NVMe-fed arena (expert e of a [K, N, 256] tensor at
// e * N * (K/256) * 66 B, src/fused_layer.cu:604). With every expert resident in HBM the block is repacked once at load
// into the tiled layout of moe_common.h (same bytes per block: 64-row groups, 16-byte chunks, re-packed sign words).
#include "moe_common.h"
#include "moe_kernels.h"

namespace lk {

// one thread per 16-byte chunk (4 per block): qs chunk c of block (m, r, j); chunk 0 also moves d
__global__ void k_pack(const uint8_t * __restrict__ src, size_t sstride, uint8_t * __restrict__ dst, size_t dstride,
                       int R, int nb, int nmat, int to_tiled) {
    const uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t per = (uint64_t) R * nb * 4;
    if (i >= (uint64_t) nmat * per) { return; }
    const int m = (int) (i / per); const uint64_t rem = i % per;
    const int c = (int) (rem % 4), j = (int) ((rem / 4) % nb), r = (int) (rem / 4 / nb);
    const size_t go = ((size_t) r * nb + j) * IQ2B;
    const size_t tq = tiled_qs_off(r / RG, j, c, nb) + 16 * (r % RG), td = tiled_d_off(r / RG, j, r % RG, R, nb);
    if (to_tiled) {
        const uint16_t * s = reinterpret_cast<const uint16_t *>(src + (size_t) m * sstride + go);
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) { w[k] = (uint32_t) s[1 + 8 * c + 2 * k] | ((uint32_t) s[2 + 8 * c + 2 * k] << 16); }
        w[1] = a1_to_tiled(w[1]); w[3] = a1_to_tiled(w[3]);
        uint8_t * d = dst + (size_t) m * dstride;
        *reinterpret_cast<uint4 *>(d + tq) = make_uint4(w[0], w[1], w[2], w[3]);
        if (c == 0) { *reinterpret_cast<uint16_t *>(d + td) = s[0]; }
    } else {
        const uint8_t * s = src + (size_t) m * sstride;
        const uint4 v = *reinterpret_cast<const uint4 *>(s + tq);
        const uint32_t w[4] = { v.x, a1_from_tiled(v.y), v.z, a1_from_tiled(v.w) };
        uint16_t * d = reinterpret_cast<uint16_t *>(dst + (size_t) m * dstride + go);
#pragma unroll
        for (int k = 0; k < 4; ++k) { d[1 + 8 * c + 2 * k] = (uint16_t) w[k]; d[2 + 8 * c + 2 * k] = (uint16_t) (w[k] >> 16); }
        if (c == 0) { d[0] = *reinterpret_cast<const uint16_t *>(s + td); }
    }
}

static hipError_t pack_common(const uint8_t * src, size_t sstride, uint8_t * dst, size_t dstride, int R, int K, int nmat, int to_tiled, hipStream_t st) {
    if (R % RG || K % 1024 || nmat <= 0) { return hipErrorInvalidValue; }
    const uint64_t tot = (uint64_t) nmat * R * (K / QK) * 4;
    k_pack<<<(unsigned) ((tot + 255) / 256), 256, 0, st>>>(src, sstride, dst, dstride, R, K / QK, nmat, to_tiled);
    return hipGetLastError();
}
hipError_t launch_pack_tiled(const uint8_t * src, size_t s, uint8_t * dst, size_t d, int R, int K, int nmat, hipStream_t st) { return pack_common(src, s, dst, d, R, K, nmat, 1, st); }
hipError_t launch_unpack_tiled(const uint8_t * src, size_t s, uint8_t * dst, size_t d, int R, int K, int nmat, hipStream_t st) { return pack_common(src, s, dst, d, R, K, nmat, 0, st); }

// ---------------------------------------------------------------- synthetic data (counter-based, any layout)
// splitmix64's output function (Steele, Lea & Flood 2014) as a counter hash: word w of block (row r, block j) of matrix
// id is mix(key(seed, id) + 16 * (r * nb + j) + w); words 0..7 are the 64 qs bytes (ggml order), words 8 and 9 feed
// Box-Muller for d. The block contents do not depend on the layout they are written in.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t stream_key(uint64_t seed, uint64_t id) { return mix64(mix64(seed) ^ (id * 0xd1b54a32d192ed03ull + 0x632be59bd9b4e019ull)); }
__device__ __forceinline__ double gauss(uint64_t h1, uint64_t h2) {
    const double u1 = (double) ((h1 >> 11) + 1) * 0x1p-53;   // (0, 1]
    const double u2 = (double) (h2 >> 11) * 0x1p-53;         // [0, 1)
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

__global__ void k_synth_iq2(uint8_t * __restrict__ dst, size_t dstride, int R, int nb, int nmat, int layout, uint64_t seed, uint64_t mat0, float sigma) {
    const uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t per = (uint64_t) R * nb;
    if (i >= (uint64_t) nmat * per) { return; }
    const int m = (int) (i / per); const uint64_t rem = i % per;
    const int r = (int) (rem / nb), j = (int) (rem % nb);
    const uint64_t key = stream_key(seed, mat0 + (uint64_t) m) + 16ull * rem;
    uint64_t wds[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) { wds[w] = mix64(key + (uint64_t) w); }
    const float dv = (float) (fabs(gauss(mix64(key + 8), mix64(key + 9))) * (double) sigma);
    const uint16_t dh = __half_as_ushort(__float2half_rn(dv));
    uint8_t * base = dst + (size_t) m * dstride;
    if (layout == LAYOUT_TILED) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {   // chunk c = sub-blocks 2c, 2c+1 = words 2c, 2c+1 (a0 low, a1 high)
            const uint64_t s0 = wds[2 * c], s1 = wds[2 * c + 1];
            const uint4 v = make_uint4((uint32_t) s0, a1_to_tiled((uint32_t) (s0 >> 32)), (uint32_t) s1, a1_to_tiled((uint32_t) (s1 >> 32)));
            *reinterpret_cast<uint4 *>(base + tiled_qs_off(r / RG, j, c, nb) + 16 * (r % RG)) = v;
        }
        *reinterpret_cast<uint16_t *>(base + tiled_d_off(r / RG, j, r % RG, R, nb)) = dh;
    } else {
        uint16_t * b16 = reinterpret_cast<uint16_t *>(base + rem * IQ2B);
        b16[0] = dh;
#pragma unroll
        for (int w = 0; w < 8; ++w) { for (int k = 0; k < 4; ++k) { b16[1 + 4 * w + k] = (uint16_t) (wds[w] >> (16 * k)); } }
    }
}

hipError_t launch_synth_iq2(uint8_t * dst, size_t dstride, int R, int K, int nmat, int layout, uint64_t seed, uint64_t mat0, float sigma, hipStream_t st) {
    if (R % RG || K % 1024 || nmat <= 0) { return hipErrorInvalidValue; }
    const uint64_t tot = (uint64_t) nmat * R * (K / QK);
    k_synth_iq2<<<(unsigned) ((tot + 255) / 256), 256, 0, st>>>(dst, dstride, R, K / QK, nmat, layout, seed, mat0, sigma);
    return hipGetLastError();
}

__global__ void k_synth_normal(float * __restrict__ dst, int64_t count, uint64_t seed, uint64_t stream, float mean, float sigma) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= count) { return; }
    const uint64_t key = stream_key(seed, stream) + 2ull * (uint64_t) i;
    dst[i] = (float) ((double) mean + (double) sigma * gauss(mix64(key), mix64(key + 1)));
}

// fp16 -> fp32 (exact): the F16 router weight (ffn_gate_inp as F16, fl.cu:317-319) widened for the fp32 router kernels
__global__ void k_f16_to_f32(const uint16_t * __restrict__ src, float * __restrict__ dst, int64_t count) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < count) { dst[i] = h2f(src[i]); }
}
hipError_t launch_f16_to_f32(const uint16_t * src, float * dst, int64_t count, hipStream_t st) {
    if (count <= 0) { return hipSuccess; }
    k_f16_to_f32<<<(unsigned) ((count + 255) / 256), 256, 0, st>>>(src, dst, count);
    return hipGetLastError();
}

hipError_t launch_synth_normal(float * dst, int64_t count, uint64_t seed, uint64_t stream, float mean, float sigma, hipStream_t st) {
    if (count <= 0) { return hipSuccess; }
    k_synth_normal<<<(unsigned) ((count + 255) / 256), 256, 0, st>>>(dst, count, seed, stream, mean, sigma);
    return hipGetLastError();
}

}  // namespace lk
