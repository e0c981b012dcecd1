// quant.hip -- Q8_K activation quantisation (one wave per 256-value block), ggml rms_norm, exp-contract probes.
//
// Q8_K follows quantize_row_q8_K_ref (ggml-quants.c; the reference quantises per 32 instead, src/fused_layer.cu:40-47):
// amax = max |x| with its first occurrence's signed value `max`; iscale = -127/max; q = min(127, round-half-even(iscale*x));
// d = 1/iscale; an all-zero block gives d = 0, q = 0. rintf is round-half-even, the same integer ggml's 1.5*2^23 trick
// produces for |v| <= 2^22, and the product is rounded on its own (contraction off), so q and d are bit-identical.
#include "moe_common.h"
#include "moe_kernels.h"

namespace lk {

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

__global__ void __launch_bounds__(256) k_quant_q8k(const float * __restrict__ x, int64_t nblk, int8_t * __restrict__ q, float * __restrict__ d) {
    const int64_t b = (int64_t) blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblk) { return; }
    q8k_block_wave(x + b * QK, q + b * QK, d + b);
}

hipError_t launch_quant_q8k(const float * x, int64_t nrows, int K, int8_t * q, float * d, hipStream_t st) {
    const int64_t nblk = nrows * (K / QK);
    if (nblk <= 0) { return hipSuccess; }
    k_quant_q8k<<<(unsigned) ((nblk + 3) / 4), 256, 0, st>>>(x, nblk, q, d);
    return hipGetLastError();
}

// ggml_compute_forward_rms_norm_f32: sum of fp32 squares accumulated in fp64, mean rounded to fp32,
// scale = 1/sqrtf(mean + eps), y = x*scale, then * w (ggml_mul with the norm weight). The fp64 sum is a tree here
// (sequential in ggml): it can differ from ggml's in the last fp64 bits, which only rarely survive the fp32 rounding.
__global__ void __launch_bounds__(256) k_rmsnorm(const float * __restrict__ x, const float * __restrict__ w, float * __restrict__ y, int D, float eps) {
#pragma clang fp contract(off)
    __shared__ double red[4];
    const int row = blockIdx.x; const float * xr = x + (size_t) row * D; double s = 0.0;
    for (int i = threadIdx.x; i < D; i += 256) { const float sq = xr[i] * xr[i]; s += (double) sq; }
    for (int off = 32; off > 0; off >>= 1) { s += __shfl_xor(s, off); }
    if ((threadIdx.x & 63) == 0) { red[threadIdx.x >> 6] = s; }
    __syncthreads();
    const double tot = (red[0] + red[1]) + (red[2] + red[3]);
    const float mean = (float) (tot / (double) D);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int i = threadIdx.x; i < D; i += 256) { y[(size_t) row * D + i] = (xr[i] * scale) * (w ? w[i] : 1.0f); }
}

hipError_t launch_rmsnorm(const float * x, const float * w, float * y, int n, int D, float eps, hipStream_t st) {
    if (n <= 0) { return hipSuccess; }
    k_rmsnorm<<<n, 256, 0, st>>>(x, w, y, D, eps);
    return hipGetLastError();
}

__global__ void k_expf_probe(const float * __restrict__ x, float * __restrict__ y, int64_t n, int which) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) { return; }
    y[i] = which == 0 ? det_expf(x[i]) : which == 1 ? det_sigmoid(x[i]) : det_silu(x[i]);
}

hipError_t launch_expf_probe(const float * x, float * y, int64_t n, int which, hipStream_t st) {
    if (n <= 0) { return hipSuccess; }
    k_expf_probe<<<(unsigned) ((n + 255) / 256), 256, 0, st>>>(x, y, n, which);
    return hipGetLastError();
}

}  // namespace lk
