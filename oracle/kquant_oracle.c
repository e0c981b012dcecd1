/* kquant_oracle.c -- TEST INFRASTRUCTURE ONLY: the CPU checker for the K-quant formats of the reference's real shards,
 * never the product.
 *
 * The reference runs its routed down projection in Q2_K / Q3_K and the shared expert in Q5_K / Q5_K / Q6_K
 * (src/fused_layer.cu:102-158, 203-254; src/server_core_fused.cpp:411-413). ggml is not vendored in the reference and no
 * version is pinned, so ggml's block layouts and scalar reference routines are restated here from their published
 * definitions (ggml-quants.c: dequantize_row_q{2,3,5,6}_K and ggml_vec_dot_q{2,3,5,6}_K_q8_K_generic), with the
 * activations in Q8_K (quantize_row_q8_K_ref, moe_oracle.c). The fp32 accumulation follows those scalar routines:
 *   Q2_K: sumf += dall * isum - dmin * summs per block;
 *   Q3_K, Q6_K: sums[l] += d * aux32[l] per block (l = 0..7), then sumf = sums[0] + .. + sums[7] in order;
 *   Q5_K: as Q3_K / Q6_K, with sumf -= dmin * sumi per block before the final sums[l] are added.
 * Block layouts (bytes): Q2_K 84 = scales[16] qs[64] d dmin; Q3_K 110 = hmask[32] qs[64] scales[12] d;
 * Q5_K 176 = d dmin scales[12] qh[32] qs[128]; Q6_K 210 = ql[128] qh[64] scales[16] d.
 *
 * Build: gcc -O3 -fopenmp -ffp-contract=off (see Makefile).
 */
#include "moe_oracle.h"
#include <string.h>

#define QK_K 256

int or_kq_block_bytes(int fmt) {
    switch (fmt) { case OR_Q2K: return 84; case OR_Q3K: return 110; case OR_Q5K: return 176; case OR_Q6K: return 210; default: return 0; }
}
static float h16(const uint8_t * p) { return or_fp16_to_fp32((uint16_t) (p[0] | (p[1] << 8))); }

/* the 8 6-bit scales and mins of a Q4_K / Q5_K block (get_scale_min_k4) */
static void scale_min_k4(int j, const uint8_t * q, uint8_t * d, uint8_t * m) {
    if (j < 4) { *d = q[j] & 63; *m = q[j + 4] & 63; }
    else { *d = (uint8_t) ((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4)); *m = (uint8_t) ((q[j + 4] >> 4) | ((q[j] >> 6) << 4)); }
}
/* the 16 6-bit scales of a Q3_K block, offset by -32 */
static void q3_scales(const uint8_t * s12, int8_t * sc) {
    const uint32_t kmask1 = 0x03030303u, kmask2 = 0x0f0f0f0fu;
    uint32_t aux[4];
    memcpy(aux, s12, 12);
    const uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
    aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
    aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
    aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
    memcpy(sc, aux, 16);
    for (int j = 0; j < 16; ++j) { sc[j] = (int8_t) (sc[j] - 32); }
}

/* the integer quant values of one block in element order (without scales), and its sub-block scales/mins:
 * Q2_K: q in 0..3, 16 scales (low nibble) and 16 mins (high nibble); Q3_K: q in -4..3, 16 scales (-32..31);
 * Q5_K: q in 0..31, 8 scales and 8 mins; Q6_K: q in -32..31, 16 scales (int8) */
static void kq_unpack(int fmt, const uint8_t * b, int8_t * q, int * sc, int * mn, float * d, float * dmin) {
    if (fmt == OR_Q2K) {
        const uint8_t * scales = b, * qs = b + 16;
        *d = h16(b + 80); *dmin = h16(b + 82);
        for (int j = 0; j < 16; ++j) { sc[j] = scales[j] & 0xF; mn[j] = scales[j] >> 4; }
        int o = 0;
        for (int n = 0; n < 2; ++n) {
            for (int shift = 0; shift < 8; shift += 2) {
                for (int l = 0; l < 32; ++l) { q[o++] = (int8_t) ((qs[32 * n + l] >> shift) & 3); }
            }
        }
    } else if (fmt == OR_Q3K) {
        const uint8_t * hm = b, * qs = b + 32;
        int8_t s8[16]; q3_scales(b + 96, s8);
        *d = h16(b + 108); *dmin = 0.f;
        for (int j = 0; j < 16; ++j) { sc[j] = s8[j]; mn[j] = 0; }
        int o = 0; uint8_t m = 1;
        for (int n = 0; n < 2; ++n) {
            for (int shift = 0; shift < 8; shift += 2) {
                for (int l = 0; l < 32; ++l) { q[o++] = (int8_t) (((qs[32 * n + l] >> shift) & 3) - ((hm[l] & m) ? 0 : 4)); }
                m = (uint8_t) (m << 1);
            }
        }
    } else if (fmt == OR_Q5K) {
        const uint8_t * scales = b + 4, * qh = b + 16, * ql = b + 48;
        *d = h16(b); *dmin = h16(b + 2);
        for (int j = 0; j < 8; ++j) { uint8_t s, m; scale_min_k4(j, scales, &s, &m); sc[j] = s; mn[j] = m; }
        int o = 0; uint8_t u1 = 1, u2 = 2;
        for (int j = 0; j < 4; ++j) {
            for (int l = 0; l < 32; ++l) { q[o++] = (int8_t) ((ql[32 * j + l] & 0xF) + ((qh[l] & u1) ? 16 : 0)); }
            for (int l = 0; l < 32; ++l) { q[o++] = (int8_t) ((ql[32 * j + l] >> 4) + ((qh[l] & u2) ? 16 : 0)); }
            u1 = (uint8_t) (u1 << 2); u2 = (uint8_t) (u2 << 2);
        }
    } else {   /* OR_Q6K */
        const uint8_t * ql = b, * qh = b + 128; const int8_t * scales = (const int8_t *) (b + 192);
        *d = h16(b + 208); *dmin = 0.f;
        for (int j = 0; j < 16; ++j) { sc[j] = scales[j]; mn[j] = 0; }
        for (int n = 0; n < 2; ++n) {
            const uint8_t * l4 = ql + 64 * n, * h = qh + 32 * n; int8_t * a = q + 128 * n;
            for (int l = 0; l < 32; ++l) {
                a[l + 0]  = (int8_t) (((l4[l] & 0xF) | (((h[l] >> 0) & 3) << 4)) - 32);
                a[l + 32] = (int8_t) (((l4[l + 32] & 0xF) | (((h[l] >> 2) & 3) << 4)) - 32);
                a[l + 64] = (int8_t) (((l4[l] >> 4) | (((h[l] >> 4) & 3) << 4)) - 32);
                a[l + 96] = (int8_t) (((l4[l + 32] >> 4) | (((h[l] >> 6) & 3) << 4)) - 32);
            }
        }
    }
}

/* dequantize_row_q*_K: y = d * scale * q (- dmin * min for Q2_K / Q5_K), per 16 (Q2/Q3/Q6) or 32 (Q5) elements */
void or_dequantize_row_kq(int fmt, const uint8_t * blocks, float * y, int64_t k) {
    const int bs = or_kq_block_bytes(fmt);
    for (int64_t i = 0; i < k / QK_K; ++i) {
        int8_t q[QK_K]; int sc[16], mn[16]; float d, dmin;
        kq_unpack(fmt, blocks + i * bs, q, sc, mn, &d, &dmin);
        for (int e = 0; e < QK_K; ++e) {
            float v;
            if (fmt == OR_Q5K) { const int j = e / 32; v = (d * (float) sc[j]) * (float) q[e] - dmin * (float) mn[j]; }
            else if (fmt == OR_Q2K) { const int j = e / 16; v = (d * (float) sc[j]) * (float) q[e] - dmin * (float) mn[j]; }
            else { const int j = e / 16; v = (d * (float) sc[j]) * (float) q[e]; }
            y[i * QK_K + e] = v;
        }
    }
}

/* ggml_vec_dot_q*_K_q8_K (scalar reference order): w = k weights of one row (blocks), q/d/bsums = its Q8_K operand */
float or_vec_dot_kq_q8_K(int fmt, int64_t k, const uint8_t * w, const int8_t * q8, const float * d8, const int16_t * bsums) {
    const int bs = or_kq_block_bytes(fmt);
    float sumf = 0.f, sums[8] = { 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f };
    for (int64_t i = 0; i < k / QK_K; ++i) {
        int8_t a[QK_K]; int sc[16], mn[16]; float d, dmin;
        kq_unpack(fmt, w + i * bs, a, sc, mn, &d, &dmin);
        const int8_t * x = q8 + i * QK_K; const int16_t * bsm = bsums + i * 16;
        if (fmt == OR_Q2K) {
            int summs = 0, isum = 0;
            for (int j = 0; j < 16; ++j) { summs += bsm[j] * mn[j]; }
            for (int j = 0; j < 16; ++j) { int isuml = 0; for (int l = 0; l < 16; ++l) { isuml += x[16 * j + l] * a[16 * j + l]; } isum += sc[j] * isuml; }
            const float dall = d8[i] * d, dm = d8[i] * dmin;
            sumf += dall * (float) isum - dm * (float) summs;
        } else {
            int32_t aux32[8] = { 0, 0, 0, 0, 0, 0, 0, 0 };
            const int per = fmt == OR_Q5K ? 32 : 16;   /* elements per scale */
            for (int j = 0; j < QK_K / 8; ++j) {       /* groups of 8 elements */
                const int s = sc[(8 * j) / per];
                for (int l = 0; l < 8; ++l) { const int16_t p = (int16_t) (x[8 * j + l] * a[8 * j + l]); aux32[l] += s * p; }
            }
            const float dd = d * d8[i];
            for (int l = 0; l < 8; ++l) { sums[l] += dd * (float) aux32[l]; }
            if (fmt == OR_Q5K) {
                int sumi = 0;
                for (int j = 0; j < 16; ++j) { sumi += bsm[j] * mn[j / 2]; }
                sumf -= (dmin * d8[i]) * (float) sumi;
            }
        }
    }
    if (fmt != OR_Q2K) { for (int l = 0; l < 8; ++l) { sumf += sums[l]; } }
    return sumf;
}

/* y[t][r] = row r of w (rows x k, ggml layout) . Q8_K row t (q [nt][k], d [nt][k/256], bsums [nt][k/16]) */
void or_matvec_kq(int fmt, const uint8_t * w, int64_t rows, int64_t k, const int8_t * q, const float * d, const int16_t * bsums,
                  int64_t nt, float * y) {
    const int64_t rb = (k / QK_K) * or_kq_block_bytes(fmt);
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t t = 0; t < nt; ++t) {
        for (int64_t r = 0; r < rows; ++r) {
            y[t * rows + r] = or_vec_dot_kq_q8_K(fmt, k, w + r * rb, q + t * k, d + t * (k / QK_K), bsums + t * (k / 16));
        }
    }
}
