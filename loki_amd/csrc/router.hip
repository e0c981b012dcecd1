// router.hip -- the DeepSeek-V3/R1 grouped sigmoid router on the device (no host round-trip).
//
// Reference: router_probs / router_topk (src/fused_layer.cu:313-332, launched at :506) and the ggml graph
// (src/server_core_fused.cpp:646-650) compute p = sigmoid(W x), take the top-8 of p + bias with ties to the lower index,
// and weight w_k = p[sel_k] / max(sum p[sel], 2^-14) * 2.5. This build adds the grouped rule the task names (8 groups of
// 32 experts; a group's score is the sum of its two best biased scores; the top-4 groups stay eligible), which reduces
// to the reference's rule with n_group = topk_group = 1.
//
// Logit contract (shared bit for bit with the CPU checker, moe_device.h): 256 chunks of K/256 products, each summed in
// order in fp64 from exact fp32 x fp32 products, a fixed pairwise tree over the chunk sums, one rounding to fp32. The
// sigmoid uses the fp64 exp contract of moe_common.h. Selection and weights are plain fp32 compares, adds and one
// correctly rounded division, so sel and wts are bit-identical to the checker's.
#include "moe_device.h"
#include "moe_kernels.h"

namespace lk {

constexpr int RT = 8;   // tokens per router wave

// one wave per (expert, 8-token tile); every token's logit is a full wave reduction (logit_tree)
__global__ void __launch_bounds__(64) k_router_logits(const float * __restrict__ W, const float * __restrict__ x, int n, int n_exp, int K,
                                                      float * __restrict__ logits) {
    const int e = blockIdx.x, t0 = blockIdx.y * RT;
    const int nt = min(RT, n - t0);
    for (int t = 0; t < nt; ++t) {
        double s[4];
        if (K == 7168) { logit_chunks<7>(W + (size_t) e * K, x + (size_t) (t0 + t) * K, s); }
        else { logit_chunks_any(W + (size_t) e * K, x + (size_t) (t0 + t) * K, K, s); }
        const double tot = logit_tree(s);
        if (threadIdx.x == 0) { logits[(size_t) (t0 + t) * n_exp + e] = (float) tot; }
    }
}

hipError_t launch_router_logits(const float * W, const float * x, int n, int n_exp, int K, float * logits, hipStream_t st) {
    if (n <= 0) { return hipSuccess; }
    if (K % 1024 != 0) { return hipErrorInvalidValue; }
    k_router_logits<<<dim3(n_exp, (n + RT - 1) / RT), 64, 0, st>>>(W, x, n, n_exp, K, logits);
    return hipGetLastError();
}

// one wave per token; lane l holds experts 4l..4l+3 (n_exp <= 256); the rule is select_token's (moe_device.h)
__global__ void __launch_bounds__(64) k_router_select(const float * __restrict__ logits, const float * __restrict__ bias, int n, int n_exp,
                                                      int n_group, int topk_group, int topk, float scale,
                                                      float * __restrict__ probs, int * __restrict__ sel, float * __restrict__ wts) {
    __shared__ float scr[NEXP_MAX + 2 * 64];
    __shared__ int so[MAXK]; __shared__ float wo[MAXK];
    const int t = blockIdx.x, lane = threadIdx.x;
    float lg[4], bv[4];
    load_bias(bias, n_exp, bv);
#pragma unroll
    for (int j = 0; j < 4; ++j) { const int e = 4 * lane + j; lg[j] = e < n_exp ? logits[(size_t) t * n_exp + e] : 0.f; }
    select_token(lg, bv, n_exp, n_group, topk_group, topk, scale, scr, so, wo, probs ? probs + (size_t) t * n_exp : nullptr);
    lds_visible();
    if (lane < topk) { sel[(size_t) t * topk + lane] = so[lane]; wts[(size_t) t * topk + lane] = wo[lane]; }
}

hipError_t launch_router_select(const float * logits, const float * bias, int n, int n_exp, int n_group, int topk_group,
                                int topk, float scale, float * probs, int * sel, float * wts, hipStream_t st) {
    if (n <= 0) { return hipSuccess; }
    if (n_exp > NEXP_MAX || n_exp % n_group || topk > MAXK || topk_group > n_group || topk > topk_group * (n_exp / n_group) || n_exp / n_group < 2 || n_group > 64) {
        return hipErrorInvalidValue;
    }
    k_router_select<<<n, 64, 0, st>>>(logits, bias, n, n_exp, n_group, topk_group, topk, scale, probs, sel, wts);
    return hipGetLastError();
}

}  // namespace lk
