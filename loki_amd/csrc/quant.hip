// quant.hip -- Q8_K activation quantisation (one wave per 256-value block), ggml rms_norm, exp-contract probes.
//
// Q8_K follows quantize_row_q8_K_ref (ggml-quants.c; the reference quantises per 32 instead, src/fused_layer.cu:40-47):
// amax = max |x| with its first occurrence's signed value `max`; iscale = -127/max; q = min(127, round-half-even(iscale*x));
// d = 1/iscale; an all-zero block gives d = 0, q = 0. rintf is round-half-even, the same integer ggml's 1.5*2^23 trick
// produces for |v| <= 2^22, and the product is rounded on its own (contraction off), so q and d are bit-identical.
#include "moe_device.h"
#include "moe_kernels.h"

namespace lk {

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

// ggml_compute_forward_rms_norm_f32: fp32 squares accumulated in fp64, mean rounded to fp32, scale = 1/sqrtf(mean + eps),
// y = x*scale, then * w (ggml_mul with the norm weight). The fp64 sum follows the chunk contract of sumsq_chunk (256
// in-order chunk sums, pairwise tree) -- the order the decode block's fused pre-norm reproduces; ggml's single
// sequential sum can differ from it in the last fp64 bits, which only rarely survive the fp32 rounding of the mean.
template <int L4>
__global__ void __launch_bounds__(256) k_rmsnorm(const float * __restrict__ x, const float * __restrict__ w, float * __restrict__ y, int D, float eps) {
#pragma clang fp contract(off)
    __shared__ double red[4];
    const int row = blockIdx.x; const float * xr = x + (size_t) row * D;
    const double s = tree64(sumsq_chunk<L4>(xr, threadIdx.x));
    if ((threadIdx.x & 63) == 0) { red[threadIdx.x >> 6] = s; }
    __syncthreads();
    const float scale = rms_scale(red[0], red[1], red[2], red[3], D, eps);
    for (int i = threadIdx.x; i < D; i += 256) { y[(size_t) row * D + i] = (xr[i] * scale) * (w ? w[i] : 1.0f); }
}

hipError_t launch_rmsnorm(const float * x, const float * w, float * y, int n, int D, float eps, hipStream_t st) {
    if (n <= 0) { return hipSuccess; }
    switch (D) {   // chunks of D / 256 values, 16-byte loads
    case 7168: k_rmsnorm<7><<<n, 256, 0, st>>>(x, w, y, D, eps); break;
    case 4096: k_rmsnorm<4><<<n, 256, 0, st>>>(x, w, y, D, eps); break;
    case 2048: k_rmsnorm<2><<<n, 256, 0, st>>>(x, w, y, D, eps); break;
    case 1024: k_rmsnorm<1><<<n, 256, 0, st>>>(x, w, y, D, eps); break;
    default: return hipErrorInvalidValue;
    }
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
