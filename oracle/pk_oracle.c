/*
 * pk_oracle.c -- CPU restatement of pickle's fast-path attention block.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle the HIP path is checked against; see
 * pk_oracle.h).
 *
 * Built with -ffp-contract=off so that every fused multiply-add below is an
 * explicit fmaf() (where the reference uses _mm512_fmadd_ps, or where its
 * build contracts a*b + c) and every other product is rounded on its own.
 * That keeps the oracle's results a property of this source rather than of
 * the compiler's contraction choices.
 */
#include "pk_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* src/pickle_fast.c:1515-1516: half = D/2, capped at 64. */
int pko_rope_half(int head_dim) {
    int half = head_dim / 2;
    return half > 64 ? 64 : half;
}

/* src/pickle_fast.c:1638-1640. */
void pko_rope_inv_freq(float* inv_freq, int head_dim, float theta) {
    int half = pko_rope_half(head_dim);
    for (int i = 0; i < half; i++)
        inv_freq[i] = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
}

/* src/pickle_fast.c:1779-1786: angle is one fp32 multiply of inv_freq by the
 * position converted to float; sin/cos come from libm. */
void pko_rope_fill(float* sin_tab, float* cos_tab, const float* inv_freq,
                   int half, int p_begin, int p_last) {
    for (int p = p_begin; p <= p_last; p++) {
        float* sp = sin_tab + (size_t)p * half;
        float* cp = cos_tab + (size_t)p * half;
        for (int i = 0; i < half; i++) {
            float angle = inv_freq[i] * (float)p;
            sp[i] = sinf(angle);
            cp[i] = cosf(angle);
        }
    }
}

/* src/pickle_fast.c:1916-1935: NeoX pairs (i, i + half) of each head.
 * The reference writes c*a - s*b and s*a + c*b; its default build
 * (-O3 -march=native, FMA targets) contracts each into one fused
 * multiply-add whose addend is the rounded second product, which is the
 * evaluation restated here (checked bit-for-bit against the compiled
 * reference in the CPU tests). */
void pko_rope_apply(float* x, int n_heads, int head_dim, int half,
                    const float* sin_row, const float* cos_row) {
    for (int h = 0; h < n_heads; h++) {
        float* xh = x + (size_t)h * head_dim;
        for (int i = 0; i < half; i++) {
            float a = xh[i];
            float b = xh[i + half];
            float c = cos_row[i], s = sin_row[i];
            float sb = s * b, cb = c * b;
            xh[i]        = fmaf(c, a, -sb);
            xh[i + half] = fmaf(s, a, cb);
        }
    }
}

/* src/pickle_fast.c:1940-1943. */
void pko_kv_append_f32(float* k_layer, float* v_layer, int n_kv_heads,
                       int head_dim, int pos, const float* k, const float* v) {
    size_t row = (size_t)n_kv_heads * head_dim;
    memcpy(k_layer + (size_t)pos * row, k, row * sizeof(float));
    memcpy(v_layer + (size_t)pos * row, v, row * sizeof(float));
}

/* Dot product in the order of the reference's AVX-512 score loop
 * (src/pickle_fast.c:1980-2020): four 16-lane FMA accumulators over 64-float
 * blocks, a 16-float block loop into the first accumulator, the lane-wise sum
 * (a0 + a1) + (a2 + a3), then the 16 -> 8 -> 4 -> 2 -> 1 horizontal tree of
 * _mm512_reduce_add_ps. Requires D % 16 == 0. */
static float dot_lanes16(const float* q, const float* k, int D) {
    float a0[16], a1[16], a2[16], a3[16];
    for (int j = 0; j < 16; j++) a0[j] = a1[j] = a2[j] = a3[j] = 0.0f;
    int d = 0;
    for (; d + 64 <= D; d += 64) {
        for (int j = 0; j < 16; j++) {
            a0[j] = fmaf(q[d + j],      k[d + j],      a0[j]);
            a1[j] = fmaf(q[d + 16 + j], k[d + 16 + j], a1[j]);
            a2[j] = fmaf(q[d + 32 + j], k[d + 32 + j], a2[j]);
            a3[j] = fmaf(q[d + 48 + j], k[d + 48 + j], a3[j]);
        }
    }
    for (; d + 16 <= D; d += 16)
        for (int j = 0; j < 16; j++) a0[j] = fmaf(q[d + j], k[d + j], a0[j]);
    float v[16];
    for (int j = 0; j < 16; j++) v[j] = (a0[j] + a1[j]) + (a2[j] + a3[j]);
    float t8[8], t4[4];
    for (int j = 0; j < 8; j++) t8[j] = v[j + 8] + v[j];
    for (int j = 0; j < 4; j++) t4[j] = t8[j + 4] + t8[j];
    float u0 = t4[2] + t4[0];
    float u1 = t4[3] + t4[1];
    return u0 + u1;
}

/* Scalar score loop (src/pickle_fast.c:2023-2032), used when D % 16 != 0. */
static float dot_scalar(const float* q, const float* k, int D) {
    float acc = 0.0f;
    for (int d = 0; d < D; d++) acc = fmaf(q[d], k[d], acc);
    return acc;
}

/* One head: scores, max-subtracted softmax with expf, the Σ == 0 guard, and
 * the weighted V sum (src/pickle_fast.c:1961-2093). */
static void attend_head(const float* k_layer, const float* v_layer, int HK,
                        int D, size_t attend_n, float scale, const float* qh,
                        int kv_head, float* oh, float* scores) {
    size_t row = (size_t)HK * D;
    for (size_t p = 0; p < attend_n; p++) {
        const float* kp = k_layer + p * row + (size_t)kv_head * D;
        float dot = (D % 16 == 0) ? dot_lanes16(qh, kp, D) : dot_scalar(qh, kp, D);
        scores[p] = dot * scale;
    }
    float maxv = scores[0];
    for (size_t p = 1; p < attend_n; p++)
        if (scores[p] > maxv) maxv = scores[p];
    float sume = 0.0f;
    for (size_t p = 0; p < attend_n; p++) {
        scores[p] = expf(scores[p] - maxv);
        sume += scores[p];
    }
    if (sume == 0.0f) sume = 1.0f;
    float inv_sume = 1.0f / sume;
    for (int d = 0; d < D; d++) oh[d] = 0.0f;
    for (size_t p = 0; p < attend_n; p++) {
        float w = scores[p] * inv_sume;
        const float* vp = v_layer + p * row + (size_t)kv_head * D;
        for (int d = 0; d < D; d++) oh[d] = fmaf(w, vp[d], oh[d]);
    }
}

int pko_attend_f32(const float* k_layer, const float* v_layer, int n_kv_heads,
                   int head_dim, int n_heads, size_t attend_n,
                   const float* q_rot, float* ao, int n_threads) {
    if (!k_layer || !v_layer || !q_rot || !ao) return PKO_ERR_ARG;
    if (n_kv_heads <= 0 || head_dim <= 0 || n_heads <= 0 || attend_n == 0)
        return PKO_ERR_ARG;
    const int H = n_heads, HK = n_kv_heads, D = head_dim;
    const float scale = 1.0f / sqrtf((float)D);
    int failed = 0;
    if (n_threads < 1) n_threads = 1;
#pragma omp parallel num_threads(n_threads) if (n_threads > 1)
    {
        float* scores = (float*)malloc(attend_n * sizeof(float));
        if (!scores) {
#pragma omp atomic write
            failed = 1;
        }
#pragma omp for schedule(static)
        for (int h = 0; h < H; h++) {
            if (!scores) continue;
            attend_head(k_layer, v_layer, HK, D, attend_n, scale,
                        q_rot + (size_t)h * D, h * HK / H,
                        ao + (size_t)h * D, scores);
        }
        free(scores);
    }
    return failed ? PKO_ERR_MEMORY : PKO_OK;
}

/* src/pickle_fast.c:2097-2108. */
void pko_attend_stateless(const float* v, int n_kv_heads, int head_dim,
                          int n_heads, float* ao) {
    for (int h = 0; h < n_heads; h++) {
        const float* vp = v + (size_t)(h * n_kv_heads / n_heads) * head_dim;
        memcpy(ao + (size_t)h * head_dim, vp, (size_t)head_dim * sizeof(float));
    }
}

int pko_decode_step_f32(float* k_layer, float* v_layer, int n_kv_heads,
                        int head_dim, int n_heads, int pos,
                        const float* sin_tab, const float* cos_tab, int half,
                        const float* q, const float* k, const float* v,
                        float* ao, float* q_rot_out, float* k_rot_out,
                        int n_threads) {
    if (pos < 0) return PKO_ERR_RANGE;
    size_t qn = (size_t)n_heads * head_dim, kn = (size_t)n_kv_heads * head_dim;
    float* qr = (float*)malloc(qn * sizeof(float));
    float* kr = (float*)malloc(kn * sizeof(float));
    if (!qr || !kr) { free(qr); free(kr); return PKO_ERR_MEMORY; }
    memcpy(qr, q, qn * sizeof(float));
    memcpy(kr, k, kn * sizeof(float));
    if (half > 0) {
        const float* sp = sin_tab + (size_t)pos * half;
        const float* cp = cos_tab + (size_t)pos * half;
        pko_rope_apply(qr, n_heads, head_dim, half, sp, cp);
        pko_rope_apply(kr, n_kv_heads, head_dim, half, sp, cp);
    }
    pko_kv_append_f32(k_layer, v_layer, n_kv_heads, head_dim, pos, kr, v);
    int rc = pko_attend_f32(k_layer, v_layer, n_kv_heads, head_dim, n_heads,
                            (size_t)pos + 1, qr, ao, n_threads);
    if (q_rot_out) memcpy(q_rot_out, qr, qn * sizeof(float));
    if (k_rot_out) memcpy(k_rot_out, kr, kn * sizeof(float));
    free(qr);
    free(kr);
    return rc;
}

int pko_prefill_f32(float* k_layer, float* v_layer, int n_kv_heads,
                    int head_dim, int n_heads, int pos0, int n_tokens,
                    const float* sin_tab, const float* cos_tab, int half,
                    const float* q, const float* k, const float* v,
                    float* ao, int n_threads) {
    size_t qn = (size_t)n_heads * head_dim, kn = (size_t)n_kv_heads * head_dim;
    for (int i = 0; i < n_tokens; i++) {
        int rc = pko_decode_step_f32(k_layer, v_layer, n_kv_heads, head_dim,
                                     n_heads, pos0 + i, sin_tab, cos_tab, half,
                                     q + i * qn, k + i * kn, v + i * kn,
                                     ao + i * qn, NULL, NULL, n_threads);
        if (rc != PKO_OK) return rc;
    }
    return PKO_OK;
}

/* ---- IEEE binary16 ------------------------------------------------- */

uint16_t pko_f32_to_f16(float x) {
    uint32_t f;
    memcpy(&f, &x, 4);
    uint32_t sign = (f >> 16) & 0x8000u;
    uint32_t absf = f & 0x7fffffffu;
    if (absf >= 0x7f800000u) {                       /* inf / nan */
        uint32_t mant = absf & 0x007fffffu;
        return (uint16_t)(sign | 0x7c00u | (mant ? (0x200u | (mant >> 13)) : 0u));
    }
    int e = (int)(absf >> 23) - 127 + 15;            /* rebiased exponent */
    uint32_t m = absf & 0x007fffffu;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);  /* overflow -> inf */
    if (e <= 0) {                                     /* subnormal or zero */
        if (e < -10) return (uint16_t)sign;
        m |= 0x00800000u;                             /* implicit bit */
        int shift = 14 - e;                           /* 14..24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;  /* may carry into exp */
    return (uint16_t)(sign | q);
}

float pko_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t f;
    if (e == 0) {
        if (m == 0) {
            f = sign;
        } else {                                      /* subnormal */
            int shift = 0;
            while (!(m & 0x400u)) { m <<= 1; shift++; }
            m &= 0x3ffu;
            f = sign | ((uint32_t)(127 - 15 + 1 - shift) << 23) | (m << 13);
        }
    } else if (e == 31) {
        f = sign | 0x7f800000u | (m << 13);
    } else {
        f = sign | ((e + 127 - 15) << 23) | (m << 13);
    }
    float x;
    memcpy(&x, &f, 4);
    return x;
}

void pko_f32_to_f16_n(const float* x, uint16_t* h, size_t n) {
    for (size_t i = 0; i < n; i++) h[i] = pko_f32_to_f16(x[i]);
}

void pko_f16_to_f32_n(const uint16_t* h, float* x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = pko_f16_to_f32(h[i]);
}

int pko_decode_step_f16(uint16_t* k_layer, uint16_t* v_layer, int n_kv_heads,
                        int head_dim, int n_heads, int pos,
                        const float* sin_tab, const float* cos_tab, int half,
                        const float* q, const float* k, const float* v,
                        float* ao, int n_threads) {
    if (pos < 0) return PKO_ERR_RANGE;
    size_t row = (size_t)n_kv_heads * head_dim;
    size_t qn = (size_t)n_heads * head_dim;
    size_t n = ((size_t)pos + 1) * row;
    float* kw = (float*)malloc(n * sizeof(float));
    float* vw = (float*)malloc(n * sizeof(float));
    float* qr = (float*)malloc(qn * sizeof(float));
    float* kr = (float*)malloc(row * sizeof(float));
    if (!kw || !vw || !qr || !kr) {
        free(kw); free(vw); free(qr); free(kr);
        return PKO_ERR_MEMORY;
    }
    memcpy(qr, q, qn * sizeof(float));
    memcpy(kr, k, row * sizeof(float));
    if (half > 0) {
        const float* sp = sin_tab + (size_t)pos * half;
        const float* cp = cos_tab + (size_t)pos * half;
        pko_rope_apply(qr, n_heads, head_dim, half, sp, cp);
        pko_rope_apply(kr, n_kv_heads, head_dim, half, sp, cp);
    }
    pko_f32_to_f16_n(kr, k_layer + (size_t)pos * row, row);
    pko_f32_to_f16_n(v, v_layer + (size_t)pos * row, row);
    pko_f16_to_f32_n(k_layer, kw, n);
    pko_f16_to_f32_n(v_layer, vw, n);
    int rc = pko_attend_f32(kw, vw, n_kv_heads, head_dim, n_heads,
                            (size_t)pos + 1, qr, ao, n_threads);
    free(kw); free(vw); free(qr); free(kr);
    return rc;
}
