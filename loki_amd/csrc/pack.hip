// pack.hip -- IQ2_XXS layout conversion (ggml <-> tiled) and the synthetic-data generators used by tests and bench.
//
// The reference reads experts in ggml's layout straight from its NVMe-fed arena (expert e of a [K, N, 256] tensor at
// e * N * (K/256) * 66 B, src/fused_layer.cu:604). With every expert resident in HBM the block is repacked once at load
// into the tiled layout of moe_common.h (same bytes per block, regrouped so one wave load covers a 4-row x 4-block unit).
#include "moe_common.h"
#include "moe_kernels.h"

namespace lk {

__device__ __forceinline__ void block_addrs(uint64_t i, int R, int nb, size_t &ggml_off, size_t &tile_qs, size_t &tile_d, int &m) {
    const uint64_t per = (uint64_t) R * nb;
    m = (int) (i / per); const uint64_t rem = i % per; const int r = (int) (rem / nb), j = (int) (rem % nb);
    ggml_off = ((size_t) r * nb + j) * IQ2B;
    const size_t unit = ((size_t) (r / UROWS) * (nb / UBLK) + (size_t) (j / UBLK)) * UNIT;
    const int sub = UBLK * (r % UROWS) + (j % UBLK);
    tile_qs = unit + 64 * sub; tile_d = unit + 1024 + 2 * sub;
}

__global__ void k_pack(const uint8_t * __restrict__ src, size_t sstride, uint8_t * __restrict__ dst, size_t dstride,
                       int R, int nb, int nmat, int to_tiled) {
    const uint64_t i = (uint64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t) nmat * R * nb) { return; }
    size_t go, tq, td; int m; block_addrs(i, R, nb, go, tq, td, m);
    if (to_tiled) {
        const uint16_t * s = reinterpret_cast<const uint16_t *>(src + (size_t) m * sstride + go);
        uint8_t * d = dst + (size_t) m * dstride;
        uint16_t * q = reinterpret_cast<uint16_t *>(d + tq);
#pragma unroll
        for (int k = 0; k < 32; ++k) { q[k] = s[1 + k]; }
        *reinterpret_cast<uint16_t *>(d + td) = s[0];
    } else {
        const uint8_t * s = src + (size_t) m * sstride;
        uint16_t * d = reinterpret_cast<uint16_t *>(dst + (size_t) m * dstride + go);
        const uint16_t * q = reinterpret_cast<const uint16_t *>(s + tq);
#pragma unroll
        for (int k = 0; k < 32; ++k) { d[1 + k] = q[k]; }
        d[0] = *reinterpret_cast<const uint16_t *>(s + td);
    }
}

static hipError_t pack_common(const uint8_t * src, size_t sstride, uint8_t * dst, size_t dstride, int R, int K, int nmat, int to_tiled, hipStream_t st) {
    if (R % UROWS || K % (QK * UBLK) || nmat <= 0) { return hipErrorInvalidValue; }
    const uint64_t tot = (uint64_t) nmat * R * (K / QK);
    k_pack<<<(unsigned) ((tot + 255) / 256), 256, 0, st>>>(src, sstride, dst, dstride, R, K / QK, nmat, to_tiled);
    return hipGetLastError();
}
hipError_t launch_pack_tiled(const uint8_t * src, size_t s, uint8_t * dst, size_t d, int R, int K, int nmat, hipStream_t st) { return pack_common(src, s, dst, d, R, K, nmat, 1, st); }
hipError_t launch_unpack_tiled(const uint8_t * src, size_t s, uint8_t * dst, size_t d, int R, int K, int nmat, hipStream_t st) { return pack_common(src, s, dst, d, R, K, nmat, 0, st); }

// ---------------------------------------------------------------- synthetic data (counter-based, any layout)
// splitmix64's output function (Steele, Lea & Flood 2014) as a counter hash: word w of block (row r, block j) of matrix
// id is mix(key(seed, id) + 16 * (r * nb + j) + w); words 0..7 are the 64 qs bytes, words 8 and 9 feed Box-Muller for d.
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
    if (i >= (uint64_t) nmat * R * nb) { return; }
    size_t go, tq, td; int m; block_addrs(i, R, nb, go, tq, td, m);
    const uint64_t key = stream_key(seed, mat0 + (uint64_t) m) + 16ull * (i % ((uint64_t) R * nb));
    uint64_t wds[8];
#pragma unroll
    for (int w = 0; w < 8; ++w) { wds[w] = mix64(key + (uint64_t) w); }
    const float dv = (float) (fabs(gauss(mix64(key + 8), mix64(key + 9))) * (double) sigma);
    const uint16_t dh = __half_as_ushort(__float2half_rn(dv));
    uint8_t * base = dst + (size_t) m * dstride;
    if (layout == LAYOUT_TILED) {
        uint64_t * q = reinterpret_cast<uint64_t *>(base + tq);
#pragma unroll
        for (int w = 0; w < 8; ++w) { q[w] = wds[w]; }
        *reinterpret_cast<uint16_t *>(base + td) = dh;
    } else {
        uint16_t * b16 = reinterpret_cast<uint16_t *>(base + go);
        b16[0] = dh;
#pragma unroll
        for (int w = 0; w < 8; ++w) { for (int k = 0; k < 4; ++k) { b16[1 + 4 * w + k] = (uint16_t) (wds[w] >> (16 * k)); } }
    }
}

hipError_t launch_synth_iq2(uint8_t * dst, size_t dstride, int R, int K, int nmat, int layout, uint64_t seed, uint64_t mat0, float sigma, hipStream_t st) {
    if (R % UROWS || K % (QK * UBLK) || nmat <= 0) { return hipErrorInvalidValue; }
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

hipError_t launch_synth_normal(float * dst, int64_t count, uint64_t seed, uint64_t stream, float mean, float sigma, hipStream_t st) {
    if (count <= 0) { return hipSuccess; }
    k_synth_normal<<<(unsigned) ((count + 255) / 256), 256, 0, st>>>(dst, count, seed, stream, mean, sigma);
    return hipGetLastError();
}

}  // namespace lk
