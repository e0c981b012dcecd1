// moe_kernels.h -- host-side launchers of the MoE-block kernels (internal to libloki_moe; the C ABI is include/loki_moe.h).
// Every launcher enqueues on the given stream and returns hipGetLastError() of its launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace lk {

// Q8_K of nrows rows of K floats (K % 256 == 0): q [nrows][K], d [nrows][K/256]
hipError_t launch_quant_q8k(const float * x, int64_t nrows, int K, int8_t * q, float * d, hipStream_t st);

// router logits [n][n_exp] under the fp64 chunk contract (K % 256 == 0)
hipError_t launch_router_logits(const float * W, const float * x, int n, int n_exp, int K, float * logits, hipStream_t st);
// sigmoid, bias, grouped top-k, normalised weights; probs [n][n_exp], sel/wts [n][topk]
hipError_t launch_router_select(const float * logits, const float * bias, int n, int n_exp, int n_group, int topk_group,
                                int topk, float scale, float * probs, int * sel, float * wts, hipStream_t st);

// stable counting sort of the P = n*topk pairs by expert: counts [n_exp], offsets [n_exp+1], perm/inv [P],
// act = used experts ascending, nact = their number (device scalar)
hipError_t launch_dispatch(const int * sel, int P, int n_exp, int * counts, int * offsets, int * perm, int * inv,
                           int * act, int * nact, hipStream_t st);

struct GemvArgs {
    const uint8_t * w0, * w1;        // routed expert bases (tiled layout), expert e at w + e * estride; w1 only for gate/up
    size_t estride;
    const uint8_t * sh0, * sh1;      // shared expert matrices (tiled)
    const int8_t * aq; const float * ad;   // Q8_K activations: gate/up rows = tokens, down rows = slots
    int K, R;                        // columns (activation length) and rows of each matrix
    const int * act, * nact, * offsets, * perm;
    int topk, n, P, max_act;         // max_act: launch bound on used experts (host side)
    int shared;                      // 1: the shared expert runs as the extra slot m == nact (tokens 0..n-1)
    float * out;                     // gate/up: h [P+n][R]; down: o [P+n][R]
    float * dbg0, * dbg1;            // optional gate / up outputs (gate/up launch only)
};
hipError_t launch_gemv_gateup(const GemvArgs & a, hipStream_t st);
hipError_t launch_gemv_down(const GemvArgs & a, hipStream_t st);

// y[t] = sum_k (o[inv[t*topk+k]] * w[t][k]) in k order + o[P+t] (+ resid[t] when given)
hipError_t launch_combine(const float * o, const int * inv, const float * wts, int n, int topk, int E, int P,
                          const float * resid, float * y, float * moe, hipStream_t st);

// ggml-layout IQ2_XXS matrices -> tiled layout (nmat matrices of R x K at the given byte strides)
hipError_t launch_pack_tiled(const uint8_t * src, size_t src_stride, uint8_t * dst, size_t dst_stride, int R, int K, int nmat, hipStream_t st);
hipError_t launch_unpack_tiled(const uint8_t * src, size_t src_stride, uint8_t * dst, size_t dst_stride, int R, int K, int nmat, hipStream_t st);

// synthetic data: IQ2_XXS matrices (qs uniform bytes, d = fp16(|N(0, sigma^2)|)) keyed by (seed, matrix id, row, block)
hipError_t launch_synth_iq2(uint8_t * dst, size_t dst_stride, int R, int K, int nmat, int layout, uint64_t seed,
                            uint64_t mat0, float sigma, hipStream_t st);
hipError_t launch_synth_normal(float * dst, int64_t count, uint64_t seed, uint64_t stream, float mean, float sigma, hipStream_t st);

// ggml rms_norm (fp64 sum of fp32 squares) then the weight (w may be null = ones); one block per row
hipError_t launch_rmsnorm(const float * x, const float * w, float * y, int n, int D, float eps, hipStream_t st);

// element-wise probes of the exp contract (tests)
hipError_t launch_expf_probe(const float * x, float * y, int64_t n, int which, hipStream_t st);

}  // namespace lk
