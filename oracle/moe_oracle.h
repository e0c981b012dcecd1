/* moe_oracle.h -- TEST INFRASTRUCTURE ONLY (the checker, never the product).
 *
 * CPU restatement of the DeepSeek-R1 MoE feed-forward block as ggml's CPU backend computes it
 * (quantize_row_q8_K_ref, dequantize_row_iq2_xxs, vec_dot_iq2_xxs_q8_K, mul_mat_id row mapping, swiglu,
 * k-ordered weighted combine + shared expert), plus the grouped sigmoid router named by this build's task.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Layouts are ggml's: an IQ2_XXS matrix [rows][K/256 blocks] of 66-byte blocks {fp16 d; u16 qs[32]};
 * Q8_K activations as struct-of-arrays: q int8 [K], d float [K/256], bsums int16 [K/16].
 */
#pragma once
#include <stdint.h>
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

float or_fp16_to_fp32(uint16_t h);
uint16_t or_fp32_to_fp16(float f);
/* exp contract shared by router sigmoid and SwiGLU: fp64 Cody-Waite reduction + degree-13 Taylor, rounded to fp32 */
float or_expf(float x);
float or_silu(float x);
float or_sigmoid(float x);

void or_quantize_row_q8_K(const float * x, int8_t * q, float * d, int16_t * bsums, int64_t k);
void or_dequantize_row_iq2_xxs(const uint8_t * blocks, float * y, int64_t k);
float or_vec_dot_iq2_xxs_q8_K(int64_t k, const uint8_t * wblocks, const int8_t * q, const float * d);
/* y[r] = vec_dot(row r of an IQ2_XXS matrix [rows][k/256], q8K(x)) for every row (OpenMP over rows) */
void or_matvec_iq2_xxs(const uint8_t * w, int64_t rows, int64_t k, const int8_t * q, const float * d, float * y);

/* router logits contract (K % 1024 == 0): 256 chunks of K/256 consecutive products, each summed in order in fp64 from
 * exact fp32 x fp32 products; the 256 chunk sums combined by a fixed pairwise tree (level by level, entry i of the next
 * level = entries 2i + 2i+1); rounded once to fp32 */
float or_router_logit(const float * w, const float * x, int64_t k);
/* grouped sigmoid router for n rows: probs [n][n_exp] (optional), sel [n][topk] (descending biased score),
 * wts [n][topk] = p[sel] / max(sum p[sel], 2^-14) * scale. Ties go to the lower index (groups and experts). */
int or_router(const float * W, const float * bias, const float * x, int64_t n, int n_exp, int64_t k,
              int n_group, int topk_group, int topk, float scale, float * logits, float * probs, int32_t * sel, float * wts);
/* keep-KE of the engine's narrow dispatch (src/server_core_fused.cpp:793-815): per row the ke largest weights, stably
 * ordered by weight descending, optionally rescaled so they sum to renorm (renorm <= 0: off); rows >= n_pad take row
 * 0's kept experts at weight 0. sel_out / w_out [n][ke]. */
int or_keep_experts(const int32_t * sel, const float * w, int64_t n, int topk, int ke, float renorm, int64_t n_pad,
                    int32_t * sel_out, float * w_out);
/* the same with the engine's --share-experts rule when share != 0 and n > 1 (src/server_core_fused.cpp:798-806): each
 * row keeps its own min(2, ke) heaviest, then prefers experts already in the set U of the rows' own picks (rows below
 * n_pad), then takes the rest in weight order, adding them to U row by row; kept lists in that pick order */
int or_keep_experts_share(const int32_t * sel, const float * w, int64_t n, int topk, int ke, float renorm, int64_t n_pad,
                          int share, int32_t * sel_out, float * w_out);
/* stable counting sort of the n*topk (token, k) pairs by expert; perm[j] = t*topk + k */
int or_dispatch(const int32_t * sel, int64_t n, int topk, int n_exp, int32_t * counts, int32_t * offsets, int32_t * perm);

/* Whole block. gate/up are [H][E/256] and down [E][H/256] IQ2_XXS matrices per expert (pointer per expert,
 * NULL where the expert is never selected), sh_* the shared expert. y [n][E] = sum_k (w_k * o_k) in k order + shared.
 * Optional outputs (NULL to skip): sel/wts [n][topk], g/u/h [n*topk][H] per pair (t*topk+k), o [n*topk][E], sh [n][E].
 * nthreads: OpenMP threads (0 = default). Returns 0, or a negative code on bad arguments / missing experts. */
int or_moe_forward(const float * x, int64_t n, int64_t E, int64_t H,
                   const float * W, const float * bias, int n_exp, int n_group, int topk_group, int topk, float scale,
                   const uint8_t * const * gate, const uint8_t * const * up, const uint8_t * const * down,
                   const uint8_t * sh_gate, const uint8_t * sh_up, const uint8_t * sh_down,
                   float * y, int32_t * sel, float * wts, float * g, float * u, float * o, float * sh, int nthreads);

/* Experts applied to given routing (no router): the same as or_moe_forward after its routing step. */
int or_moe_experts(const float * x, int64_t n, int64_t E, int64_t H, int topk, const int32_t * sel, const float * wts,
                   const uint8_t * const * gate, const uint8_t * const * up, const uint8_t * const * down,
                   const uint8_t * sh_gate, const uint8_t * sh_up, const uint8_t * sh_down,
                   float * y, float * g, float * u, float * o, float * sh, int nthreads);

/* ggml rms_norm then the weight: sum of fp32 squares in fp64, mean as fp32, scale = 1/sqrtf(mean + eps) */
void or_rmsnorm(const float * x, const float * w, float * y, int64_t n, int64_t d, float eps);

/* K-quant formats of the reference's real shards (kquant_oracle.c) */
enum { OR_Q2K = 5, OR_Q3K = 6, OR_Q5K = 3, OR_Q6K = 1, OR_IQ2 = 4 };   /* the FL_* codes of include/loki_moe.h */
int or_kq_block_bytes(int fmt);
void or_dequantize_row_kq(int fmt, const uint8_t * blocks, float * y, int64_t k);
float or_vec_dot_kq_q8_K(int fmt, int64_t k, const uint8_t * w, const int8_t * q8, const float * d8, const int16_t * bsums);
void or_matvec_kq(int fmt, const uint8_t * w, int64_t rows, int64_t k, const int8_t * q, const float * d, const int16_t * bsums,
                  int64_t nt, float * y);
/* or_moe_experts with per-matrix formats: fmts = { routed down, shared gate, shared up, shared down } (OR_IQ2 or a
 * K-quant; routed gate/up stay IQ2_XXS as in the reference's arena), NULL = IQ2_XXS everywhere. Rows are ggml rows of
 * the format (K/256 blocks). */
int or_moe_experts_fmt(const float * x, int64_t n, int64_t E, int64_t H, int topk, const int32_t * sel, const float * wts,
                       const uint8_t * const * gate, const uint8_t * const * up, const uint8_t * const * down,
                       const uint8_t * sh_gate, const uint8_t * sh_up, const uint8_t * sh_down, const int * fmts,
                       float * y, float * g, float * u, float * o, float * sh, int nthreads);

#ifdef __cplusplus
}
#endif
