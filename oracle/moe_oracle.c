/* moe_oracle.c -- TEST INFRASTRUCTURE ONLY: the CPU checker for the MI355X MoE block, never the product.
 *
 * A plain-C restatement of how ggml's CPU backend evaluates the DeepSeek-R1 MoE feed-forward block that
 * the reference builds at src/server_core_fused.cpp:956-979 (mul_mat_id x3, swiglu, x w, k-ordered sum,
 * + shared expert) and routes at src/server_core_fused.cpp:646-650 / src/fused_layer.cu:313-332.
 * ggml itself is not vendored in the reference (build.bat:2-9, README.md:15-16) and no version is pinned,
 * so the ggml functions are restated from their published definitions:
 *   quantize_row_q8_K_ref, dequantize_row_iq2_xxs, ggml_vec_dot_iq2_xxs_q8_K_generic (ggml-quants.c),
 *   ggml_compute_forward_mul_mat_id row mapping, ggml_silu_f32, ggml_compute_forward_rms_norm_f32.
 * Where ggml's SIMD paths leave an order unpinned (router dot, exp), this file fixes an arithmetic contract
 * that the HIP kernels reproduce bit for bit (the router logit and exp contracts below).
 *
 * Build: gcc -O3 -fopenmp -ffp-contract=off (contraction would change the fp32 rounding sequence).
 */
#include "moe_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK_K 256
#define IQ2_BYTES 66

static const uint64_t iq2xxs_grid[256] = {
#include "../loki_amd/csrc/iq2xxs_grid.inc"
};

/* ksigns_iq2xs[i] = i with bit 7 set to the parity of i (reference src/iq2_tables.cuh:70-79): 7 stored sign
 * bits, the 8th sign makes the count of minus signs even. */
static inline uint8_t ksigns(unsigned i) { return (uint8_t) (i | ((__builtin_popcount(i) & 1u) << 7)); }

/* ---------------------------------------------------------------- fp16 <-> fp32 (IEEE binary16, exact) */
float or_fp16_to_fp32(uint16_t h) {
    const uint32_t s = (uint32_t) (h >> 15) << 31, e = (h >> 10) & 31u, m = h & 1023u;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) { bits = s; }
        else {   /* subnormal: value = m * 2^-24, exact in fp32 */
            float f = (float) m * 0x1p-24f; memcpy(&bits, &f, 4); bits |= s;
        }
    } else if (e == 31) { bits = s | 0x7f800000u | (m << 13); }
    else { bits = s | ((e + 112u) << 23) | (m << 13); }
    float f; memcpy(&f, &bits, 4); return f;
}

uint16_t or_fp32_to_fp16(float f) {   /* round to nearest even, with subnormals; used to build fixtures */
    uint32_t x; memcpy(&x, &f, 4);
    const uint32_t s = (x >> 16) & 0x8000u; const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { return (uint16_t) (s | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u)); }
    if (ax >= 0x477ff000u) { return (uint16_t) (s | 0x7c00u); }   /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {   /* below 2^-14: subnormal half, value = round(|f| * 2^24) * 2^-24 */
        float a; memcpy(&a, &ax, 4); const float scaled = a * 0x1p24f;   /* exact: power-of-two scale */
        const float r = rintf(scaled); return (uint16_t) (s | (uint16_t) r);   /* r <= 1024 -> may carry into the smallest normal */
    }
    const uint32_t e = ((ax >> 23) - 112u) << 10, m = (ax >> 13) & 1023u, rest = ax & 0x1fffu;
    uint32_t h = e | m;
    if (rest > 0x1000u || (rest == 0x1000u && (m & 1u))) { h += 1u; }
    return (uint16_t) (s | h);
}

/* ---------------------------------------------------------------- exp contract
 * exp(x) evaluated in fp64: Cody-Waite reduction x = k ln2 + r with ln2 split into a 29-bit head (k*head is
 * exact) and a tail, then the degree-13 Taylor polynomial of e^r on |r| <= ln2/2 (truncation < 5e-18 relative)
 * in Horner form, scaled by 2^k through the exponent field, rounded once to fp32. Only IEEE +,-,*,/ and floor
 * are used, so any IEEE-754 binary64 machine without contraction gives the same bits. */
static double det_exp(double t) {
    if (t < -110.0) { t = -110.0; }
    if (t > 90.0) { t = 90.0; }
    const double inv_ln2 = 0x1.71547652b82fep+0, ln2_hi = 0x1.62e42ffp-1, ln2_lo = -0x1.718432a1b0e26p-35;
    const double kd = floor(t * inv_ln2 + 0.5);
    const double r = (t - kd * ln2_hi) - kd * ln2_lo;
    double p = 0x1.6124613a86d09p-33;          /* 1/13! */
    p = p * r + 0x1.1eed8eff8d898p-29;          /* 1/12! */
    p = p * r + 0x1.ae64567f544e4p-26;          /* 1/11! */
    p = p * r + 0x1.27e4fb7789f5cp-22;          /* 1/10! */
    p = p * r + 0x1.71de3a556c734p-19;          /* 1/9!  */
    p = p * r + 0x1.a01a01a01a01ap-16;          /* 1/8!  */
    p = p * r + 0x1.a01a01a01a01ap-13;          /* 1/7!  */
    p = p * r + 0x1.6c16c16c16c17p-10;          /* 1/6!  */
    p = p * r + 0x1.1111111111111p-7;           /* 1/5!  */
    p = p * r + 0x1.5555555555555p-5;           /* 1/4!  */
    p = p * r + 0x1.5555555555555p-3;           /* 1/3!  */
    p = p * r + 0x1.0p-1;                       /* 1/2!  */
    p = p * r + 1.0;
    p = p * r + 1.0;
    const int k = (int) kd;
    const uint64_t sb = (uint64_t) (k + 1023) << 52; double s; memcpy(&s, &sb, 8);
    return p * s;
}

float or_expf(float x) {
    if (x != x) { return x; }
    return (float) det_exp((double) x);
}
float or_silu(float x) { return x / (1.0f + or_expf(-x)); }          /* ggml_silu_f32 */
float or_sigmoid(float x) { return 1.0f / (1.0f + or_expf(-x)); }    /* ggml_vec_sigmoid_f32 (scalar form) */

/* ---------------------------------------------------------------- Q8_K (quantize_row_q8_K_ref) */
static inline int nearest_int(float fval) {   /* round half to even through the 1.5*2^23 magic constant */
    float val = fval + 12582912.f; int i; memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

void or_quantize_row_q8_K(const float * x, int8_t * q, float * d, int16_t * bsums, int64_t k) {
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; ++i) {
        const float * xb = x + i * QK_K; int8_t * qb = q + i * QK_K;
        float max = 0.f, amax = 0.f;
        for (int j = 0; j < QK_K; ++j) { const float ax = fabsf(xb[j]); if (ax > amax) { amax = ax; max = xb[j]; } }
        if (amax == 0.f) {
            d[i] = 0.f; memset(qb, 0, QK_K);
            if (bsums) { memset(bsums + i * 16, 0, 16 * sizeof(int16_t)); }
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < QK_K; ++j) { const float v = iscale * xb[j]; const int iv = nearest_int(v); qb[j] = (int8_t) (iv < 127 ? iv : 127); }
        if (bsums) { for (int j = 0; j < 16; ++j) { int s = 0; for (int ii = 0; ii < 16; ++ii) { s += qb[j * 16 + ii]; } bsums[i * 16 + j] = (int16_t) s; } }
        d[i] = 1.f / iscale;
    }
}

/* ---------------------------------------------------------------- IQ2_XXS (dequantize_row_iq2_xxs) */
static inline void sub_block_words(const uint8_t * blk, int ib, uint32_t * a0, uint32_t * a1) {
    memcpy(a0, blk + 2 + 8 * ib, 4); memcpy(a1, blk + 2 + 8 * ib + 4, 4);   /* little-endian qs[4ib..4ib+3] */
}

void or_dequantize_row_iq2_xxs(const uint8_t * blocks, float * y, int64_t k) {
    const int64_t nb = k / QK_K;
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t * blk = blocks + i * IQ2_BYTES; uint16_t dh; memcpy(&dh, blk, 2); const float d = or_fp16_to_fp32(dh);
        for (int ib = 0; ib < 8; ++ib) {
            uint32_t a0, a1; sub_block_words(blk, ib, &a0, &a1);
            const float db = d * (0.5f + (float) (a1 >> 28)) * 0.25f;
            for (int l = 0; l < 4; ++l) {
                const uint64_t gv = iq2xxs_grid[(a0 >> (8 * l)) & 255u]; const uint8_t signs = ksigns((a1 >> (7 * l)) & 127u);
                for (int j = 0; j < 8; ++j) {
                    const float g = (float) ((gv >> (8 * j)) & 255u);
                    y[i * QK_K + ib * 32 + l * 8 + j] = db * g * ((signs >> j) & 1u ? -1.f : 1.f);
                }
            }
        }
    }
}

/* ggml_vec_dot_iq2_xxs_q8_K_generic: exact int32 per block (sum over sub-blocks of (2*(a1>>28)+1) * sumi),
 * fp32 accumulation over blocks in order of d_w*d_x*bsum, then * 0.125 */
float or_vec_dot_iq2_xxs_q8_K(int64_t k, const uint8_t * wblocks, const int8_t * q, const float * d) {
    const int64_t nb = k / QK_K; float sumf = 0.f;
    for (int64_t i = 0; i < nb; ++i) {
        const uint8_t * blk = wblocks + i * IQ2_BYTES; uint16_t dh; memcpy(&dh, blk, 2);
        const float dd = or_fp16_to_fp32(dh) * d[i];
        const int8_t * q8 = q + i * QK_K; int32_t bsum = 0;
        for (int ib = 0; ib < 8; ++ib) {
            uint32_t a0, a1; sub_block_words(blk, ib, &a0, &a1);
            const int32_t ls = 2 * (int32_t) (a1 >> 28) + 1; int32_t sumi = 0;
            for (int l = 0; l < 4; ++l) {
                const uint64_t gv = iq2xxs_grid[(a0 >> (8 * l)) & 255u]; const uint8_t signs = ksigns((a1 >> (7 * l)) & 127u);
                for (int j = 0; j < 8; ++j) {
                    const int32_t g = (int32_t) ((gv >> (8 * j)) & 255u);
                    sumi += g * q8[j] * ((signs >> j) & 1u ? -1 : 1);
                }
                q8 += 8;
            }
            bsum += sumi * ls;
        }
        sumf += dd * (float) bsum;
    }
    return 0.125f * sumf;
}

void or_matvec_iq2_xxs(const uint8_t * w, int64_t rows, int64_t k, const int8_t * q, const float * d, float * y) {
    const size_t rb = (size_t) (k / QK_K) * IQ2_BYTES;
    #pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) { y[r] = or_vec_dot_iq2_xxs_q8_K(k, w + (size_t) r * rb, q, d); }
}

/* ---------------------------------------------------------------- router */
float or_router_logit(const float * w, const float * x, int64_t k) {
    const int64_t L = k / 256; double t[256];
    for (int c = 0; c < 256; ++c) {   /* chunk c: K/256 consecutive products summed in order */
        double s = 0.0;
        for (int64_t i = c * L; i < (c + 1) * L; ++i) { s += (double) x[i] * (double) w[i]; }   /* product exact in fp64 */
        t[c] = s;
    }
    for (int m = 256; m > 1; m /= 2) {   /* pairwise tree: entry i of the next level = entries 2i + 2i+1 */
        for (int i = 0; i < m / 2; ++i) { t[i] = t[2 * i] + t[2 * i + 1]; }
    }
    return (float) t[0];
}

/* top-m of v[0..n) over allowed entries: descending value, ties to the lower index (the reference's argmax
 * rule, src/fused_layer.cu:327-329) */
static void topm(const float * v, const unsigned char * allowed, int n, int m, int32_t * out) {
    for (int s = 0; s < m; ++s) {
        int best = -1;
        for (int e = 0; e < n; ++e) {
            if (allowed && !allowed[e]) { continue; }
            int taken = 0; for (int j = 0; j < s; ++j) { if (out[j] == e) { taken = 1; break; } }
            if (taken) { continue; }
            if (best < 0 || v[e] > v[best]) { best = e; }   /* strict: an equal later value never displaces */
        }
        out[s] = best;
    }
}

int or_router(const float * W, const float * bias, const float * x, int64_t n, int n_exp, int64_t k,
              int n_group, int topk_group, int topk, float scale, float * logits, float * probs, int32_t * sel, float * wts) {
    if (n_exp <= 0 || n_exp > 1024 || n_group <= 0 || n_exp % n_group || topk_group <= 0 || topk_group > n_group || topk <= 0 || k % 64) { return -1; }
    const int per = n_exp / n_group; if (topk > topk_group * per || per < 2) { return -1; }
    int rc = 0;
    #pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < n; ++t) {
        float p[1024], c[1024], gs[1024]; unsigned char allow[1024]; int32_t gsel[1024], s8[1024];
        for (int e = 0; e < n_exp; ++e) {
            const float l = or_router_logit(W + (size_t) e * k, x + (size_t) t * k, k);
            if (logits) { logits[t * n_exp + e] = l; }
            p[e] = or_sigmoid(l); c[e] = p[e] + bias[e];
            if (probs) { probs[t * n_exp + e] = p[e]; }
        }
        for (int g = 0; g < n_group; ++g) { int32_t two[2]; topm(c + g * per, NULL, per, 2, two); gs[g] = c[g * per + two[0]] + c[g * per + two[1]]; }
        topm(gs, NULL, n_group, topk_group, gsel);
        memset(allow, 0, (size_t) n_exp);
        for (int j = 0; j < topk_group; ++j) { for (int e = 0; e < per; ++e) { allow[gsel[j] * per + e] = 1; } }
        topm(c, allow, n_exp, topk, s8);
        float sum = 0.f; for (int j = 0; j < topk; ++j) { sum += p[s8[j]]; }
        sum = sum > 6.103515625e-5f ? sum : 6.103515625e-5f;
        for (int j = 0; j < topk; ++j) { sel[t * topk + j] = s8[j]; wts[t * topk + j] = p[s8[j]] / sum * scale; }
    }
    return rc;
}

/* ---------------------------------------------------------------- keep-KE (the engine's narrow host dispatch)
 * src/server_core_fused.cpp:793-815: each row's topk (sel, w) are ordered by weight, descending -- std::sort over 8
 * indices with `w[a] > w[b]`, which for ranges this short is an insertion sort in the standard libraries (libstdc++
 * below 16 elements, MSVC below 32), so equal weights keep their k order -- and the first ke are kept in that order.
 * renorm > 0 (RENORM_EXPERTS, on by default, :811 with the literal 2.5): sw = the kept weights summed in kept order in
 * fp32; if sw > 1e-6f every kept weight is multiplied by f = renorm / sw. Rows >= n_pad (fixed-width pass padding,
 * :815) take row 0's kept experts at weight 0. */
int or_keep_experts(const int32_t * sel, const float * w, int64_t n, int topk, int ke, float renorm, int64_t n_pad,
                    int32_t * sel_out, float * w_out) {
    return or_keep_experts_share(sel, w, n, topk, ke, renorm, n_pad, 0, sel_out, w_out);
}

/* The same with --share-experts (src/server_core_fused.cpp:798-806, the flag at :376; the production client passes it,
 * loki/chat.py:35): when share != 0 and n > 1 every row keeps its own min(2, ke) heaviest experts; U = the set of those
 * experts over the rows below n_pad; then row by row, in row order, the row's remaining slots are filled first by its
 * other picks (weight order) whose expert is in U, then by its remaining picks (weight order), each such expert being
 * added to U as it is taken (so later rows see it). The kept list is in that pick order, and the renorm sums it in
 * that order. */
int or_keep_experts_share(const int32_t * sel, const float * w, int64_t n, int topk, int ke, float renorm, int64_t n_pad,
                          int share, int32_t * sel_out, float * w_out) {
    if (topk <= 0 || topk > 64 || ke <= 0 || ke > topk || n < 0) { return -1; }
    int * ords = (int *) malloc((size_t) (n > 0 ? n : 1) * (size_t) topk * sizeof(int));
    if (!ords) { return -3; }
    for (int64_t i = 0; i < n; ++i) {
        int * ord = ords + i * topk;
        for (int k = 0; k < topk; ++k) { ord[k] = k; }
        for (int a = 1; a < topk; ++a) {   /* insertion sort, strict comparison: stable */
            const int v = ord[a]; int b = a;
            while (b > 0 && w[i * topk + v] > w[i * topk + ord[b - 1]]) { ord[b] = ord[b - 1]; --b; }
            ord[b] = v;
        }
    }
    if (share && n > 1) {
        const int own = ke < 2 ? ke : 2;
        unsigned char inU[65536];
        memset(inU, 0, sizeof inU);
        for (int64_t i = 0; i < n && i < n_pad; ++i) {
            for (int k = 0; k < own; ++k) { const int32_t e = sel[i * topk + ords[i * topk + k]]; if (e < 0 || e > 65535) { free(ords); return -2; } inU[e] = 1; }
        }
        for (int64_t i = 0; i < n; ++i) {
            const int * ord = ords + i * topk;
            int pick[64], np_ = 0;
            for (int k = 0; k < own; ++k) { pick[np_++] = ord[k]; }
            for (int k = own; k < topk && np_ < ke; ++k) {
                const int32_t e = sel[i * topk + ord[k]];
                if (e >= 0 && e <= 65535 && inU[e]) { pick[np_++] = ord[k]; }
            }
            for (int k = own; k < topk && np_ < ke; ++k) {
                int taken = 0;
                for (int j = 0; j < np_; ++j) { if (pick[j] == ord[k]) { taken = 1; break; } }
                if (!taken) {
                    pick[np_++] = ord[k];
                    const int32_t e = sel[i * topk + ord[k]];
                    if (e >= 0 && e <= 65535) { inU[e] = 1; }
                }
            }
            for (int k = 0; k < ke; ++k) { sel_out[i * ke + k] = sel[i * topk + pick[k]]; w_out[i * ke + k] = w[i * topk + pick[k]]; }
        }
    } else {
        for (int64_t i = 0; i < n; ++i) {
            for (int k = 0; k < ke; ++k) { sel_out[i * ke + k] = sel[i * topk + ords[i * topk + k]]; w_out[i * ke + k] = w[i * topk + ords[i * topk + k]]; }
        }
    }
    free(ords);
    for (int64_t i = 0; i < n; ++i) {
        if (renorm > 0.f) {
            float sw = 0.0f;
            for (int k = 0; k < ke; ++k) { sw += w_out[i * ke + k]; }
            if (sw > 1e-6f) { const float f = renorm / sw; for (int k = 0; k < ke; ++k) { w_out[i * ke + k] *= f; } }
        }
    }
    for (int64_t i = n_pad; i < n; ++i) {
        if (i < 1) { continue; }
        for (int k = 0; k < ke; ++k) { sel_out[i * ke + k] = sel_out[k]; w_out[i * ke + k] = 0.0f; }
    }
    return 0;
}

/* ---------------------------------------------------------------- dispatch (mul_mat_id row mapping)
 * For each token t ascending and k ascending, pair (t, k) is appended to its expert's list (the order of
 * ggml_compute_forward_mul_mat_id's matrix_rows and of the reference's byexp, src/server_core_fused.cpp:937). */
int or_dispatch(const int32_t * sel, int64_t n, int topk, int n_exp, int32_t * counts, int32_t * offsets, int32_t * perm) {
    for (int e = 0; e < n_exp; ++e) { counts[e] = 0; }
    for (int64_t i = 0; i < n * topk; ++i) { if (sel[i] < 0 || sel[i] >= n_exp) { return -2; } counts[sel[i]]++; }
    int32_t acc = 0; for (int e = 0; e < n_exp; ++e) { offsets[e] = acc; acc += counts[e]; } offsets[n_exp] = acc;
    int32_t * fill = (int32_t *) calloc((size_t) n_exp, sizeof(int32_t)); if (!fill) { return -3; }
    for (int64_t i = 0; i < n * topk; ++i) { const int e = sel[i]; perm[offsets[e] + fill[e]++] = (int32_t) i; }
    free(fill); return 0;
}

/* ---------------------------------------------------------------- whole block */
static void swiglu_q8(const float * g, const float * u, int64_t H, float * hout, int8_t * q, float * d, int16_t * bs) {
    float * h = hout;
    for (int64_t i = 0; i < H; ++i) { h[i] = or_silu(g[i]) * u[i]; }
    or_quantize_row_q8_K(h, q, d, bs, H);
}

/* one row . Q8_K row in the row's format (IQ2_XXS or a K-quant) */
static float row_dot(int fmt, int64_t k, const uint8_t * w, const int8_t * q, const float * d, const int16_t * bs) {
    return fmt == OR_IQ2 ? or_vec_dot_iq2_xxs_q8_K(k, w, q, d) : or_vec_dot_kq_q8_K(fmt, k, w, q, d, bs);
}
static size_t row_bytes(int fmt, int64_t k) { return (size_t) (k / QK_K) * (size_t) (fmt == OR_IQ2 ? IQ2_BYTES : or_kq_block_bytes(fmt)); }

int or_moe_experts(const float * x, int64_t n, int64_t E, int64_t H, int topk, const int32_t * sel, const float * wts,
                   const uint8_t * const * gate, const uint8_t * const * up, const uint8_t * const * down,
                   const uint8_t * sh_gate, const uint8_t * sh_up, const uint8_t * sh_down,
                   float * y, float * g, float * u, float * o, float * sh, int nthreads) {
    return or_moe_experts_fmt(x, n, E, H, topk, sel, wts, gate, up, down, sh_gate, sh_up, sh_down, NULL, y, g, u, o, sh, nthreads);
}

int or_moe_experts_fmt(const float * x, int64_t n, int64_t E, int64_t H, int topk, const int32_t * sel, const float * wts,
                       const uint8_t * const * gate, const uint8_t * const * up, const uint8_t * const * down,
                       const uint8_t * sh_gate, const uint8_t * sh_up, const uint8_t * sh_down, const int * fmts,
                       float * y, float * g, float * u, float * o, float * sh, int nthreads) {
    if (E % QK_K || H % QK_K || n < 0 || topk <= 0) { return -1; }
    const int fdn = fmts ? fmts[0] : OR_IQ2, fsg = fmts ? fmts[1] : OR_IQ2, fsu = fmts ? fmts[2] : OR_IQ2, fsd = fmts ? fmts[3] : OR_IQ2;
    const int ok[4] = { fdn, fsg, fsu, fsd };
    for (int i = 0; i < 4; ++i) { if (ok[i] != OR_IQ2 && or_kq_block_bytes(ok[i]) == 0) { return -1; } }
#ifdef _OPENMP
    const int saved = omp_get_max_threads(); if (nthreads > 0) { omp_set_num_threads(nthreads); }
#else
    (void) nthreads;
#endif
    const int64_t P = n * topk, nbE = E / QK_K, nbH = H / QK_K;
    for (int64_t p = 0; p < P; ++p) { const int e = sel[p]; if (!gate[e] || !up[e] || !down[e]) { return -4; } }
    int8_t * qx = (int8_t *) malloc((size_t) n * E); float * dx = (float *) malloc((size_t) n * nbE * 4);
    float * gp = g ? g : (float *) malloc((size_t) P * H * 4); float * up_ = u ? u : (float *) malloc((size_t) P * H * 4);
    float * op = o ? o : (float *) malloc((size_t) P * E * 4); float * shp = sh ? sh : (float *) malloc((size_t) n * E * 4);
    int8_t * qh = (int8_t *) malloc((size_t) P * H); float * dh = (float *) malloc((size_t) P * nbH * 4); float * hh = (float *) malloc((size_t) (P > 0 ? P : 1) * H * 4);
    float * gs = (float *) malloc((size_t) n * H * 4), * us = (float *) malloc((size_t) n * H * 4);
    int8_t * qhs = (int8_t *) malloc((size_t) n * H); float * dhs = (float *) malloc((size_t) n * nbH * 4);
    int16_t * bx = (int16_t *) malloc((size_t) (n > 0 ? n : 1) * (E / 16) * 2), * bh = (int16_t *) malloc((size_t) (P > 0 ? P : 1) * (H / 16) * 2);
    int16_t * bhs = (int16_t *) malloc((size_t) (n > 0 ? n : 1) * (H / 16) * 2);
    if (!qx || !dx || !gp || !up_ || !op || !shp || !qh || !dh || !hh || !gs || !us || !qhs || !dhs || !bx || !bh || !bhs) { return -3; }
    const size_t rbE = row_bytes(OR_IQ2, E), rbEg = row_bytes(fsg, E), rbEu = row_bytes(fsu, E), rbH = row_bytes(fdn, H), rbHs = row_bytes(fsd, H);
    #pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < n; ++t) { or_quantize_row_q8_K(x + t * E, qx + t * E, dx + t * nbE, bx + t * (E / 16), E); }
    /* gate / up of every (t, k) pair and of the shared expert per token */
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (P + n) * H; ++i) {
        const int64_t p = i / H, r = i % H;
        if (p < P) {
            const int e = sel[p]; const int64_t t = p / topk;
            gp[p * H + r] = or_vec_dot_iq2_xxs_q8_K(E, gate[e] + r * rbE, qx + t * E, dx + t * nbE);
            up_[p * H + r] = or_vec_dot_iq2_xxs_q8_K(E, up[e] + r * rbE, qx + t * E, dx + t * nbE);
        } else {
            const int64_t t = p - P;
            gs[t * H + r] = row_dot(fsg, E, sh_gate + r * rbEg, qx + t * E, dx + t * nbE, bx + t * (E / 16));
            us[t * H + r] = row_dot(fsu, E, sh_up + r * rbEu, qx + t * E, dx + t * nbE, bx + t * (E / 16));
        }
    }
    #pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < P + n; ++p) {
        if (p < P) { swiglu_q8(gp + p * H, up_ + p * H, H, hh + p * H, qh + p * H, dh + p * nbH, bh + p * (H / 16)); }
        else { const int64_t t = p - P; swiglu_q8(gs + t * H, us + t * H, H, gs + t * H, qhs + t * H, dhs + t * nbH, bhs + t * (H / 16)); }   /* h over g in place */
    }
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (P + n) * E; ++i) {
        const int64_t p = i / E, r = i % E;
        if (p < P) { const int e = sel[p]; op[p * E + r] = row_dot(fdn, H, down[e] + r * rbH, qh + p * H, dh + p * nbH, bh + p * (H / 16)); }
        else { const int64_t t = p - P; shp[t * E + r] = row_dot(fsd, H, sh_down + r * rbHs, qhs + t * H, dhs + t * nbH, bhs + t * (H / 16)); }
    }
    /* combine as the reference's graph: exo * w, then views added in k order, then + shared (eng:970-975) */
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n * E; ++i) {
        const int64_t t = i / E, r = i % E; float m = op[(t * topk) * E + r] * wts[t * topk];
        for (int kk = 1; kk < topk; ++kk) { m = m + op[(t * topk + kk) * E + r] * wts[t * topk + kk]; }
        y[i] = m + shp[i];
    }
    free(qx); free(dx); free(qh); free(dh); free(hh); free(gs); free(us); free(qhs); free(dhs); free(bx); free(bh); free(bhs);
    if (!g) { free(gp); } if (!u) { free(up_); } if (!o) { free(op); } if (!sh) { free(shp); }
#ifdef _OPENMP
    if (nthreads > 0) { omp_set_num_threads(saved); }
#endif
    return 0;
}

int or_moe_forward(const float * x, int64_t n, int64_t E, int64_t H,
                   const float * W, const float * bias, int n_exp, int n_group, int topk_group, int topk, float scale,
                   const uint8_t * const * gate, const uint8_t * const * up, const uint8_t * const * down,
                   const uint8_t * sh_gate, const uint8_t * sh_up, const uint8_t * sh_down,
                   float * y, int32_t * sel, float * wts, float * g, float * u, float * o, float * sh, int nthreads) {
    int32_t * s = sel ? sel : (int32_t *) malloc((size_t) n * topk * 4); float * w = wts ? wts : (float *) malloc((size_t) n * topk * 4);
    if (!s || !w) { return -3; }
#ifdef _OPENMP
    const int saved = omp_get_max_threads(); if (nthreads > 0) { omp_set_num_threads(nthreads); }
#endif
    int rc = or_router(W, bias, x, n, n_exp, E, n_group, topk_group, topk, scale, NULL, NULL, s, w);
#ifdef _OPENMP
    if (nthreads > 0) { omp_set_num_threads(saved); }
#endif
    if (rc == 0) { rc = or_moe_experts(x, n, E, H, topk, s, w, gate, up, down, sh_gate, sh_up, sh_down, y, g, u, o, sh, nthreads); }
    if (!sel) { free(s); } if (!wts) { free(w); }
    return rc;
}

void or_rmsnorm(const float * x, const float * w, float * y, int64_t n, int64_t d, float eps) {
    for (int64_t t = 0; t < n; ++t) {
        const float * xr = x + t * d; double sum = 0.0;
        for (int64_t i = 0; i < d; ++i) { sum += (double) (xr[i] * xr[i]); }
        const float mean = (float) (sum / (double) d); const float scale = 1.0f / sqrtf(mean + eps);
        for (int64_t i = 0; i < d; ++i) { y[t * d + i] = (xr[i] * scale) * (w ? w[i] : 1.0f); }
    }
}
