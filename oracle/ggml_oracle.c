/*
 * ggml_oracle.c -- CPU restatement of ggml-CPU for the single-token decode
 * path.  TEST INFRASTRUCTURE ONLY: the checker for the HIP kernels and the
 * timed CPU baseline.  The product library never links or calls this file.
 *
 * Upstream functions restated (llama.cpp @ 37b3a9e0, third-party, absent
 * offline) are named in ggml_oracle.h; the reference-side anchors are cited
 * per function below.  Built with -ffp-contract=off so that every fp32
 * operation is rounded exactly where the C source says (explicit fmaf()
 * marks the places where ggml's SIMD code uses a fused multiply-add).
 */
#include "ggml_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ fp16 */

uint16_t orc_fp32_to_fp16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                        /* below 2^-14: half subnormal or zero */
        if (ax <= 0x33000000u) return (uint16_t)sign; /* <= 2^-25 rounds (ties-even) to 0 */
        const uint32_t e = ax >> 23;
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        const uint32_t shift = 126u - e;           /* value / 2^-24 = m * 2^(e-126) */
        uint32_t h = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax >> 13) & 0x3ffu);
    const uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float orc_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {                                   /* subnormal: normalise */
            e = 113;
            while ((m & 0x400u) == 0) { m <<= 1; e--; }
            m &= 0x3ffu;
            x = sign | (e << 23) | (m << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

void orc_fp32_to_fp16_row(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_fp32_to_fp16(x[i]);
}

void orc_fp16_to_fp32_row(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = orc_fp16_to_fp32(x[i]);
}

/* ------------------------------------------------------------------ Q8_0 */

/*
 * ggml quantize_row_q8_0_ref (variant REF) and the ggml-cpu x86 AVX
 * quantize_row_q8_0 (variant X86).  Per 32-block: amax = max|x|,
 * d = amax/127 stored as fp16 (RNE); REF: id = d ? 1/d : 0, q = roundf(x*id);
 * X86: id = amax ? 127/amax : 0, q = round-half-even(x*id).
 * With inv_s != NULL the input is x[j]*inv_s[j] (SmoothQuant divisor folded
 * in as a precomputed fp32 reciprocal).
 */
void orc_quantize_row_q8_0(const float *x, const float *inv_s, orc_block_q8_0 *y, int64_t k, int variant) {
    const int64_t nb = k / ORC_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        float v[ORC_QK8_0];
        float amax = 0.0f;
        for (int j = 0; j < ORC_QK8_0; j++) {
            const int64_t idx = i * ORC_QK8_0 + j;
            v[j] = inv_s ? x[idx] * inv_s[idx] : x[idx];
            const float a = fabsf(v[j]);
            amax = a > amax ? a : amax;
        }
        const float d = amax / 127.0f;
        y[i].d = orc_fp32_to_fp16(d);
        if (variant == ORC_Q8_ROUND_X86) {
            const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
            for (int j = 0; j < ORC_QK8_0; j++) y[i].qs[j] = (int8_t)nearbyintf(v[j] * id);
        } else {
            const float id = d != 0.0f ? 1.0f / d : 0.0f;
            for (int j = 0; j < ORC_QK8_0; j++) y[i].qs[j] = (int8_t)roundf(v[j] * id);
        }
    }
}

void orc_dequantize_row_q8_0(const orc_block_q8_0 *x, float *y, int64_t k) {
    const int64_t nb = k / ORC_QK8_0;
    for (int64_t i = 0; i < nb; i++) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int j = 0; j < ORC_QK8_0; j++) y[i * ORC_QK8_0 + j] = x[i].qs[j] * d;
    }
}

/* ggml_vec_dot_q8_0_q8_0, generic order: sumf += sumi * (dx * dy) */
float orc_vec_dot_q8_0_q8_0(int64_t k, const orc_block_q8_0 *x, const orc_block_q8_0 *y) {
    const int64_t nb = k / ORC_QK8_0;
    float sumf = 0.0f;
    for (int64_t ib = 0; ib < nb; ib++) {
        int32_t sumi = 0;
        for (int j = 0; j < ORC_QK8_0; j++) sumi += (int32_t)x[ib].qs[j] * (int32_t)y[ib].qs[j];
        sumf += (float)sumi * (orc_fp16_to_fp32(x[ib].d) * orc_fp16_to_fp32(y[ib].d));
    }
    return sumf;
}

void orc_q8_0_block_dots(const orc_block_q8_0 *w, const orc_block_q8_0 *xq, int64_t n_rows, int64_t k, int32_t *out) {
    const int64_t nb = k / ORC_QK8_0;
    for (int64_t n = 0; n < n_rows; n++) {
        for (int64_t b = 0; b < nb; b++) {
            const orc_block_q8_0 *wb = &w[n * nb + b];
            int32_t s = 0;
            for (int j = 0; j < ORC_QK8_0; j++) s += (int32_t)wb->qs[j] * (int32_t)xq[b].qs[j];
            out[n * nb + b] = s;
        }
    }
}

void orc_mul_mat_q8_0(const orc_block_q8_0 *w, const float *x, const float *inv_s, float *y,
                      int64_t n_rows, int64_t k, int variant) {
    const int64_t nb = k / ORC_QK8_0;
    orc_block_q8_0 *xq = (orc_block_q8_0 *)malloc((size_t)nb * sizeof(orc_block_q8_0));
    orc_quantize_row_q8_0(x, inv_s, xq, k, variant);
    for (int64_t n = 0; n < n_rows; n++) y[n] = orc_vec_dot_q8_0_q8_0(k, &w[n * nb], xq);
    free(xq);
}

void orc_mul_mat_q8_0_batch(const orc_block_q8_0 *w, const float *x, const float *inv_s, float *y,
                            int64_t n_rows, int64_t k, int64_t m, int variant) {
    for (int64_t i = 0; i < m; i++) orc_mul_mat_q8_0(w, x + i * k, inv_s, y + i * n_rows, n_rows, k, variant);
}

/* host weight quantizer: Q8_0 of W*diag(s) with the ggml reference rounding */
void orc_quantize_weight_q8_0(const float *w, const float *s, orc_block_q8_0 *y, int64_t n_rows, int64_t k) {
    float *row = (float *)malloc((size_t)k * sizeof(float));
    for (int64_t n = 0; n < n_rows; n++) {
        for (int64_t j = 0; j < k; j++) row[j] = s ? w[n * k + j] * s[j] : w[n * k + j];
        orc_quantize_row_q8_0(row, NULL, &y[n * (k / ORC_QK8_0)], k, ORC_Q8_ROUND_REF);
    }
    free(row);
}

/* ------------------------------------------------------------------ Q4_0 */

/* ggml dequantize_row_q4_0: element j = (qs[j] & 15) - 8, element j+16 = (qs[j] >> 4) - 8, times d */
void orc_dequantize_row_q4_0(const orc_block_q4_0 *x, float *y, int64_t k) {
    const int64_t nb = k / ORC_QK4_0;
    for (int64_t i = 0; i < nb; i++) {
        const float d = orc_fp16_to_fp32(x[i].d);
        for (int j = 0; j < ORC_QK4_0 / 2; j++) {
            const int x0 = (x[i].qs[j] & 0x0f) - 8;
            const int x1 = (x[i].qs[j] >> 4) - 8;
            y[i * ORC_QK4_0 + j] = x0 * d;
            y[i * ORC_QK4_0 + j + ORC_QK4_0 / 2] = x1 * d;
        }
    }
}

void orc_mul_mat_q4_0_f16(const orc_block_q4_0 *w, const uint16_t *x_f16, float *y, int64_t n_rows, int64_t k) {
    float *xf = (float *)malloc((size_t)k * sizeof(float));
    float *wf = (float *)malloc((size_t)k * sizeof(float));
    orc_fp16_to_fp32_row(x_f16, xf, k);
    for (int64_t n = 0; n < n_rows; n++) {
        orc_dequantize_row_q4_0(&w[n * (k / ORC_QK4_0)], wf, k);
        float acc = 0.0f;
        for (int64_t j = 0; j < k; j++) acc += wf[j] * xf[j];
        y[n] = acc;
    }
    free(xf);
    free(wf);
}

void orc_mul_mat_q4_0_f16_f64(const orc_block_q4_0 *w, const uint16_t *x_f16, double *y, int64_t n_rows, int64_t k) {
    const int64_t nb = k / ORC_QK4_0;
    for (int64_t n = 0; n < n_rows; n++) {
        double acc = 0.0;
        for (int64_t b = 0; b < nb; b++) {
            const orc_block_q4_0 *blk = &w[n * nb + b];
            const double d = orc_fp16_to_fp32(blk->d);
            for (int j = 0; j < ORC_QK4_0 / 2; j++) {
                acc += (double)((blk->qs[j] & 0x0f) - 8) * d * orc_fp16_to_fp32(x_f16[b * ORC_QK4_0 + j]);
                acc += (double)((blk->qs[j] >> 4) - 8) * d * orc_fp16_to_fp32(x_f16[b * ORC_QK4_0 + j + 16]);
            }
        }
        y[n] = acc;
    }
}

/* ------------------------------------------------------------------ F16 */

/*
 * ggml mul_mat with F16 weights: src1 (fp32) is converted to the vec_dot
 * type F16 (RNE), then ggml_vec_dot_f16 accumulates exact fp16 x fp16
 * products in fp32.  The accumulation here is sequential.
 */
void orc_mul_mat_f16(const uint16_t *w, const float *x, float *y, int64_t n_rows, int64_t k) {
    float *xr = (float *)malloc((size_t)k * sizeof(float));
    for (int64_t j = 0; j < k; j++) xr[j] = orc_fp16_to_fp32(orc_fp32_to_fp16(x[j]));
    for (int64_t n = 0; n < n_rows; n++) {
        float acc = 0.0f;
        for (int64_t j = 0; j < k; j++) acc += orc_fp16_to_fp32(w[n * k + j]) * xr[j];
        y[n] = acc;
    }
    free(xr);
}

void orc_mul_mat_f16_f64(const uint16_t *w, const float *x, double *y, int64_t n_rows, int64_t k) {
    for (int64_t n = 0; n < n_rows; n++) {
        double acc = 0.0;
        for (int64_t j = 0; j < k; j++)
            acc += (double)orc_fp16_to_fp32(w[n * k + j]) * (double)orc_fp16_to_fp32(orc_fp32_to_fp16(x[j]));
        y[n] = acc;
    }
}

/* ------------------------------------------------------- flash_attn_ext */

/*
 * ggml_vec_dot_f16 in the summation order of the x86 F16C/AVX2 build
 * (GGML_F16_STEP 32, GGML_F16_EPR 8: four 8-lane fp32 FMA accumulators,
 * pairwise tree reduction, then hadd of the 8 lanes; leftovers added last).
 */
static float vec_dot_f16_avx2_order(int64_t n, const uint16_t *x, const uint16_t *y) {
    float acc[4][8] = {{0}};
    const int64_t np = n & ~(int64_t)31;
    for (int64_t i = 0; i < np; i += 32)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 8; l++) {
                const int64_t e = i + j * 8 + l;
                acc[j][l] = fmaf(orc_fp16_to_fp32(x[e]), orc_fp16_to_fp32(y[e]), acc[j][l]);
            }
    for (int l = 0; l < 8; l++) { acc[0][l] += acc[2][l]; acc[1][l] += acc[3][l]; }
    for (int l = 0; l < 8; l++) acc[0][l] += acc[1][l];
    float t0[4];
    for (int l = 0; l < 4; l++) t0[l] = acc[0][l] + acc[0][l + 4];
    double sumf = (double)((t0[0] + t0[1]) + (t0[2] + t0[3]));
    for (int64_t i = np; i < n; i++) sumf += (double)(orc_fp16_to_fp32(x[i]) * orc_fp16_to_fp32(y[i]));
    return (float)sumf;
}

static void fa_one_head_ggml(const float *qh, const char *kb, const char *vb, const uint16_t *mask,
                             int64_t kv_len, int64_t d, size_t k_nb1, size_t v_nb1, float scale, float *out) {
    uint16_t *q16 = (uint16_t *)malloc((size_t)d * 2);
    uint16_t *acc16 = (uint16_t *)calloc((size_t)d, 2);
    for (int64_t i = 0; i < d; i++) q16[i] = orc_fp32_to_fp16(qh[i]);
    float S = 0.0f;
    float M = -INFINITY;
    for (int64_t ic = 0; ic < kv_len; ic++) {
        const float mv = mask ? orc_fp16_to_fp32(mask[ic]) : 0.0f;
        if (mv == -INFINITY) continue;
        const uint16_t *krow = (const uint16_t *)(kb + ic * k_nb1);
        const uint16_t *vrow = (const uint16_t *)(vb + ic * v_nb1);
        float s = vec_dot_f16_avx2_order(d, krow, q16);
        s = s * scale;
        s += mv;
        const float Mold = M;
        float ms = 1.0f, vs = 1.0f;
        if (s > M) {
            M = s;
            ms = expf(Mold - M);
            for (int64_t i = 0; i < d; i++) acc16[i] = orc_fp32_to_fp16(orc_fp16_to_fp32(acc16[i]) * ms);
        } else {
            vs = expf(s - M);
        }
        for (int64_t i = 0; i < d; i++)
            acc16[i] = orc_fp32_to_fp16(fmaf(orc_fp16_to_fp32(vrow[i]), vs, orc_fp16_to_fp32(acc16[i])));
        S = S * ms + vs;
    }
    const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
    for (int64_t i = 0; i < d; i++) out[i] = orc_fp16_to_fp32(acc16[i]) * S_inv;
    free(q16);
    free(acc16);
}

static void fa_one_head_f64(const float *qh, const char *kb, const char *vb, const uint16_t *mask,
                            int64_t kv_len, int64_t d, size_t k_nb1, size_t v_nb1, float scale, float *out) {
    double *sc = (double *)malloc((size_t)(kv_len > 0 ? kv_len : 1) * sizeof(double));
    double mx = -INFINITY;
    for (int64_t ic = 0; ic < kv_len; ic++) {
        const double mv = mask ? (double)orc_fp16_to_fp32(mask[ic]) : 0.0;
        const uint16_t *krow = (const uint16_t *)(kb + ic * k_nb1);
        double s = 0.0;
        for (int64_t i = 0; i < d; i++)
            s += (double)orc_fp16_to_fp32(orc_fp32_to_fp16(qh[i])) * (double)orc_fp16_to_fp32(krow[i]);
        sc[ic] = (mv == -INFINITY) ? -INFINITY : s * (double)scale + mv;
        if (sc[ic] > mx) mx = sc[ic];
    }
    double den = 0.0;
    double *acc = (double *)calloc((size_t)d, sizeof(double));
    for (int64_t ic = 0; ic < kv_len; ic++) {
        if (sc[ic] == -INFINITY) continue;
        const double p = exp(sc[ic] - mx);
        den += p;
        const uint16_t *vrow = (const uint16_t *)(vb + ic * v_nb1);
        for (int64_t i = 0; i < d; i++) acc[i] += p * (double)orc_fp16_to_fp32(vrow[i]);
    }
    for (int64_t i = 0; i < d; i++) out[i] = den == 0.0 ? 0.0f : (float)(acc[i] / den);
    free(sc);
    free(acc);
}

void orc_flash_attn_ext_1tok(const float *q, const void *k, const void *v, const uint16_t *mask,
                             int64_t kv_len, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                             size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale,
                             float *out, int mode) {
    const int64_t group = n_q_heads / n_kv_heads;    /* ggml: ik2 = iq2 / (neq2/nek2) */
    for (int64_t h = 0; h < n_q_heads; h++) {
        const int64_t kvh = h / group;
        const char *kb = (const char *)k + kvh * k_nb2;
        const char *vb = (const char *)v + kvh * v_nb2;
        if (mode == 0) fa_one_head_ggml(q + h * d, kb, vb, mask, kv_len, d, k_nb1, v_nb1, scale, out + h * d);
        else           fa_one_head_f64(q + h * d, kb, vb, mask, kv_len, d, k_nb1, v_nb1, scale, out + h * d);
    }
}

/* ------------------------------------------------------------ kv_lengths */

/* patch:2900-2929 set_input_kv_lengths_impl: scan back past non-finite entries, minimum 1 */
void orc_kv_lengths(const void *mask, int mask_is_f16, int64_t n_kv, int64_t n_rows, int32_t *out) {
    for (int64_t r = 0; r < n_rows; r++) {
        int64_t len = n_kv;
        while (len > 0) {
            const float val = mask_is_f16 ? orc_fp16_to_fp32(((const uint16_t *)mask)[r * n_kv + len - 1])
                                          : ((const float *)mask)[r * n_kv + len - 1];
            if (isfinite(val)) break;
            --len;
        }
        out[r] = (int32_t)(len > 1 ? len : 1);
    }
}

/* --------------------------------------------- reference-side A8W8 scheme */

/* patch:1674-1695 ggml_backend_cann_transform_f16_a8w8 (k = ne0, n = ne1; NZ 16x32 scatter) */
void orc_quantize_a8w8_per_channel(const uint16_t *w_f16, int64_t k, int64_t n, int8_t *q_nz, uint16_t *scales) {
    for (int64_t column = 0; column < n; column++) {
        float max_abs = 0.0f;
        for (int64_t row = 0; row < k; row++) {
            const float a = fabsf(orc_fp16_to_fp32(w_f16[column * k + row]));
            max_abs = a > max_abs ? a : max_abs;
        }
        float scale = max_abs / 127.0f;
        if (scale < 1.0e-8f) scale = 1.0e-8f;
        scales[column] = orc_fp32_to_fp16(scale);
        for (int64_t row = 0; row < k; row++) {
            const float value = orc_fp16_to_fp32(w_f16[column * k + row]) / scale;
            const size_t nz = ((((size_t)column / 32) * ((size_t)k / 16) + (size_t)row / 16) * 16 +
                               (size_t)row % 16) * 32 + (size_t)column % 32;
            float r = roundf(value);
            r = r > 127.0f ? 127.0f : (r < -127.0f ? -127.0f : r);
            q_nz[nz] = (int8_t)r;
        }
    }
}

/* experiments/a8w8/w8a8_quantize_custom_vector.cpp:28-57: one scale per token, eps floor, RINT */
void orc_quantize_per_token_i8(const uint16_t *x_f16, int64_t k, int8_t *xq, uint16_t *scale) {
    float max_abs = 0.0f;
    for (int64_t i = 0; i < k; i++) {
        const float a = fabsf(orc_fp16_to_fp32(x_f16[i]));
        max_abs = a > max_abs ? a : max_abs;
    }
    if (max_abs < 0.00000127f) max_abs = 0.00000127f;
    *scale = orc_fp32_to_fp16(max_abs / 127.0f);
    const float inv = 127.0f / max_abs;
    for (int64_t i = 0; i < k; i++) xq[i] = (int8_t)nearbyintf(orc_fp16_to_fp32(x_f16[i]) * inv);
}

/* ============================ timed CPU baseline (SIMD, multithreaded) */

static int cpu_has_vnni(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl") &&
           __builtin_cpu_supports("avx512bw");
}

static int cpu_has_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") && __builtin_cpu_supports("f16c");
}

const char *orc_simd_isa(void) {
    if (cpu_has_vnni()) return "avx512vnni";
    if (cpu_has_avx2()) return "avx2";
    return "scalar";
}

__attribute__((target("avx2,fma,f16c")))
static inline float hsum8(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v);
    __m128 hi = _mm256_extractf128_ps(v, 1);
    lo = _mm_add_ps(lo, hi);
    lo = _mm_hadd_ps(lo, lo);
    lo = _mm_hadd_ps(lo, lo);
    return _mm_cvtss_f32(lo);
}

/* ggml x86 vec_dot_q8_0_q8_0 (AVX2: maddubs on |x| and sign-adjusted y, FMA into 8 lanes) */
__attribute__((target("avx2,fma,f16c")))
static float dot_q8_0_avx2(int64_t nb, const orc_block_q8_0 *x, const orc_block_q8_0 *y) {
    __m256 acc = _mm256_setzero_ps();
    const __m256i ones = _mm256_set1_epi16(1);
    for (int64_t ib = 0; ib < nb; ib++) {
        const __m256 d = _mm256_set1_ps(_cvtsh_ss(x[ib].d) * _cvtsh_ss(y[ib].d));
        const __m256i qx = _mm256_loadu_si256((const __m256i *)x[ib].qs);
        const __m256i qy = _mm256_loadu_si256((const __m256i *)y[ib].qs);
        const __m256i ax = _mm256_sign_epi8(qx, qx);
        const __m256i sy = _mm256_sign_epi8(qy, qx);
        const __m256i s16 = _mm256_maddubs_epi16(ax, sy);
        const __m256i s32 = _mm256_madd_epi16(s16, ones);
        acc = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(s32), acc);
    }
    return hsum8(acc);
}

__attribute__((target("avx2,fma,f16c,avx512f,avx512vl,avx512bw,avx512vnni")))
static float dot_q8_0_vnni(int64_t nb, const orc_block_q8_0 *x, const orc_block_q8_0 *y) {
    __m256 acc = _mm256_setzero_ps();
    for (int64_t ib = 0; ib < nb; ib++) {
        const __m256 d = _mm256_set1_ps(_cvtsh_ss(x[ib].d) * _cvtsh_ss(y[ib].d));
        const __m256i qx = _mm256_loadu_si256((const __m256i *)x[ib].qs);
        const __m256i qy = _mm256_loadu_si256((const __m256i *)y[ib].qs);
        const __m256i ax = _mm256_sign_epi8(qx, qx);
        const __m256i sy = _mm256_sign_epi8(qy, qx);
        const __m256i s32 = _mm256_dpbusd_epi32(_mm256_setzero_si256(), ax, sy);
        acc = _mm256_fmadd_ps(d, _mm256_cvtepi32_ps(s32), acc);
    }
    return hsum8(acc);
}

void orc_mul_mat_q8_0_mt(const orc_block_q8_0 *w, const float *x, const float *inv_s, float *y,
                         int64_t n_rows, int64_t k, int n_threads) {
    orc_mul_mat_q8_0_mt_variant(w, x, inv_s, y, n_rows, k, n_threads, ORC_Q8_ROUND_X86);
}

void orc_mul_mat_q8_0_mt_variant(const orc_block_q8_0 *w, const float *x, const float *inv_s, float *y,
                                 int64_t n_rows, int64_t k, int n_threads, int variant) {
    const int64_t nb = k / ORC_QK8_0;
    orc_block_q8_0 *xq = (orc_block_q8_0 *)malloc((size_t)nb * sizeof(orc_block_q8_0));
    orc_quantize_row_q8_0(x, inv_s, xq, k, variant);
    const int vnni = cpu_has_vnni();
    const int avx2 = cpu_has_avx2();
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t n = 0; n < n_rows; n++) {
        if (vnni) y[n] = dot_q8_0_vnni(nb, &w[n * nb], xq);
        else if (avx2) y[n] = dot_q8_0_avx2(nb, &w[n * nb], xq);
        else y[n] = orc_vec_dot_q8_0_q8_0(k, &w[n * nb], xq);
    }
    free(xq);
}

/* dequantize Q4_0 + fp32 dot with fp16 activations (F16C), 8-lane FMA accumulators */
__attribute__((target("avx2,fma,f16c")))
static float dot_q4_0_f16_avx2(int64_t nb, const orc_block_q4_0 *w, const float *xf) {
    __m256 acc0 = _mm256_setzero_ps(), acc1 = _mm256_setzero_ps();
    const __m128i lowmask = _mm_set1_epi8(0x0f);
    const __m128i eight = _mm_set1_epi8(8);
    for (int64_t b = 0; b < nb; b++) {
        const __m256 d = _mm256_set1_ps(_cvtsh_ss(w[b].d));
        const __m128i q = _mm_loadu_si128((const __m128i *)w[b].qs);
        const __m128i lo = _mm_sub_epi8(_mm_and_si128(q, lowmask), eight);
        const __m128i hi = _mm_sub_epi8(_mm_and_si128(_mm_srli_epi16(q, 4), lowmask), eight);
        const float *xb = xf + b * 32;
        __m256 w0 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(lo)), d);
        __m256 w1 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(lo, 8))), d);
        __m256 w2 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(hi)), d);
        __m256 w3 = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_srli_si128(hi, 8))), d);
        acc0 = _mm256_fmadd_ps(w0, _mm256_loadu_ps(xb + 0), acc0);
        acc1 = _mm256_fmadd_ps(w1, _mm256_loadu_ps(xb + 8), acc1);
        acc0 = _mm256_fmadd_ps(w2, _mm256_loadu_ps(xb + 16), acc0);
        acc1 = _mm256_fmadd_ps(w3, _mm256_loadu_ps(xb + 24), acc1);
    }
    return hsum8(_mm256_add_ps(acc0, acc1));
}

void orc_mul_mat_q4_0_f16_mt(const orc_block_q4_0 *w, const uint16_t *x_f16, float *y,
                             int64_t n_rows, int64_t k, int n_threads) {
    const int64_t nb = k / ORC_QK4_0;
    float *xf = (float *)malloc((size_t)k * sizeof(float));
    orc_fp16_to_fp32_row(x_f16, xf, k);
    const int avx2 = cpu_has_avx2();
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t n = 0; n < n_rows; n++) {
        if (avx2) {
            y[n] = dot_q4_0_f16_avx2(nb, &w[n * nb], xf);
        } else {
            float wf[ORC_QK4_0];
            float acc = 0.0f;
            for (int64_t b = 0; b < nb; b++) {
                orc_dequantize_row_q4_0(&w[n * nb + b], wf, ORC_QK4_0);
                for (int j = 0; j < ORC_QK4_0; j++) acc += wf[j] * xf[b * ORC_QK4_0 + j];
            }
            y[n] = acc;
        }
    }
    free(xf);
}

__attribute__((target("avx2,fma,f16c")))
static float dot_f16_avx2(int64_t k, const uint16_t *w, const uint16_t *x16) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps(), a2 = _mm256_setzero_ps(), a3 = _mm256_setzero_ps();
    int64_t i = 0;
    for (; i + 32 <= k; i += 32) {
        a0 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(w + i))),
                             _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(x16 + i))), a0);
        a1 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(w + i + 8))),
                             _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(x16 + i + 8))), a1);
        a2 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(w + i + 16))),
                             _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(x16 + i + 16))), a2);
        a3 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(w + i + 24))),
                             _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(x16 + i + 24))), a3);
    }
    float s = hsum8(_mm256_add_ps(_mm256_add_ps(a0, a2), _mm256_add_ps(a1, a3)));
    for (; i < k; i++) s += _cvtsh_ss(w[i]) * _cvtsh_ss(x16[i]);
    return s;
}

void orc_mul_mat_f16_mt(const uint16_t *w, const float *x, float *y, int64_t n_rows, int64_t k, int n_threads) {
    uint16_t *x16 = (uint16_t *)malloc((size_t)k * 2);
    orc_fp32_to_fp16_row(x, x16, k);
    const int avx2 = cpu_has_avx2();
#pragma omp parallel for num_threads(n_threads) schedule(static)
    for (int64_t n = 0; n < n_rows; n++) {
        if (avx2) {
            y[n] = dot_f16_avx2(k, w + n * k, x16);
        } else {
            float acc = 0.0f;
            for (int64_t j = 0; j < k; j++) acc += orc_fp16_to_fp32(w[n * k + j]) * orc_fp16_to_fp32(x16[j]);
            y[n] = acc;
        }
    }
    free(x16);
}

/* the same per-head loop as fa_one_head_ggml with F16C/FMA vectors; bit-identical by construction */
__attribute__((target("avx2,fma,f16c")))
static void fa_one_head_ggml_avx2(const float *qh, const char *kb, const char *vb, const uint16_t *mask,
                                  int64_t kv_len, int64_t d, size_t k_nb1, size_t v_nb1, float scale, float *out) {
    uint16_t q16[512];
    uint16_t acc16[512];
    for (int64_t i = 0; i < d; i++) { q16[i] = orc_fp32_to_fp16(qh[i]); acc16[i] = 0; }
    float S = 0.0f;
    float M = -INFINITY;
    for (int64_t ic = 0; ic < kv_len; ic++) {
        const float mv = mask ? _cvtsh_ss(mask[ic]) : 0.0f;
        if (mv == -INFINITY) continue;
        const uint16_t *krow = (const uint16_t *)(kb + ic * k_nb1);
        const uint16_t *vrow = (const uint16_t *)(vb + ic * v_nb1);
        __m256 a[4] = {_mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps(), _mm256_setzero_ps()};
        for (int64_t i = 0; i < d; i += 32)
            for (int j = 0; j < 4; j++)
                a[j] = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(krow + i + 8 * j))),
                                       _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(q16 + i + 8 * j))), a[j]);
        a[0] = _mm256_add_ps(a[0], a[2]);
        a[1] = _mm256_add_ps(a[1], a[3]);
        a[0] = _mm256_add_ps(a[0], a[1]);
        float s = (float)(double)hsum8(a[0]);
        s = s * scale;
        s += mv;
        const float Mold = M;
        float ms = 1.0f, vs = 1.0f;
        if (s > M) {
            M = s;
            ms = expf(Mold - M);
            const __m256 vms = _mm256_set1_ps(ms);
            for (int64_t i = 0; i < d; i += 8) {
                __m256 y = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(acc16 + i)));
                _mm_storeu_si128((__m128i *)(acc16 + i), _mm256_cvtps_ph(_mm256_mul_ps(y, vms), 0));
            }
        } else {
            vs = expf(s - M);
        }
        const __m256 vvs = _mm256_set1_ps(vs);
        for (int64_t i = 0; i < d; i += 8) {
            __m256 y = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(acc16 + i)));
            __m256 x = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(vrow + i)));
            _mm_storeu_si128((__m128i *)(acc16 + i), _mm256_cvtps_ph(_mm256_fmadd_ps(x, vvs, y), 0));
        }
        S = S * ms + vs;
    }
    const float S_inv = S == 0.0f ? 0.0f : 1.0f / S;
    for (int64_t i = 0; i < d; i++) out[i] = _cvtsh_ss(acc16[i]) * S_inv;
}

/* ggml-cpu parallelises single-token flash_attn_ext over q heads */
void orc_flash_attn_ext_1tok_mt(const float *q, const void *k, const void *v, const uint16_t *mask,
                                int64_t kv_len, int64_t n_q_heads, int64_t n_kv_heads, int64_t d,
                                size_t k_nb1, size_t k_nb2, size_t v_nb1, size_t v_nb2, float scale,
                                float *out, int n_threads) {
    const int64_t group = n_q_heads / n_kv_heads;
    const int avx2 = cpu_has_avx2();
#pragma omp parallel for num_threads(n_threads) schedule(dynamic, 1)
    for (int64_t h = 0; h < n_q_heads; h++) {
        const int64_t kvh = h / group;
        if (avx2 && d % 32 == 0 && d <= 512)
            fa_one_head_ggml_avx2(q + h * d, (const char *)k + kvh * k_nb2, (const char *)v + kvh * v_nb2, mask,
                                  kv_len, d, k_nb1, v_nb1, scale, out + h * d);
        else
            fa_one_head_ggml(q + h * d, (const char *)k + kvh * k_nb2, (const char *)v + kvh * v_nb2, mask,
                             kv_len, d, k_nb1, v_nb1, scale, out + h * d);
    }
}
