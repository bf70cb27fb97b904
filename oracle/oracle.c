/*
 * oracle.c — CPU restatement of the reference fomoe expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h). Built with -ffp-contract=off so
 * that its results do not depend on the compiler's FMA contraction choices.
 *
 * Parity pins (all in tests/test_oracle.py):
 *   fp16<->fp32        exhaustive vs IEEE (numpy.float16) and vs oracle/_ref
 *   dequant Q4_K/Q5_K/Q6_K/Q8_0/MXFP4
 *                      bit-exact vs oracle/_ref and vs the committed golden
 *                      fixtures; brute force over all scale/min codes
 *   vec_dot/mat_vec    vs oracle/_ref (within fp32 reordering) and vs an fp64
 *                      dot of the dequantized rows
 *   softmax/top_k      vs oracle/_ref (bit-exact) and textbook properties
 *   Q8_K path          quantize bit-exact vs oracle/_ref; dots vs oracle/_ref
 *   moe layer          vs a composition of oracle/_ref's mat_vec_mul/softmax/
 *                      top_k (golden fixture) and an fp64 re-evaluation
 *   bf16 rounding      vs torch over 1M random bit patterns, 4096 halfway cases
 *                      and the range edges
 *   prefill            fo_moe_prefill_w vs an fp64 numpy recomposition, for
 *                      each bf16 weight-rounding mask; routing vs the decode
 *                      layer's
 *   synth/quantizers   own definition: round-trip error bounds, code ranges
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ------------------------------------------------------------------------
 * fp16 <-> fp32.  Reference src/quant.c:30-67 converts exactly (IEEE binary16
 * to binary32) and rounds to nearest-even the other way, with NaN -> 0x7E00.
 * Restated here by direct field decoding.
 * ------------------------------------------------------------------------ */
float fo_fp16_to_fp32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    const uint32_t m = h & 0x3FFu;
    if (e == 0x1F) return u2f(sign | 0x7F800000u | (m << 13) | (m ? 0x400000u : 0));
    if (e != 0) return u2f(sign | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return u2f(sign);
    return u2f(sign | f2u((float)m * 0x1p-24f));  /* subnormal: m * 2^-24, exact */
}

uint16_t fo_fp32_to_fp16(float f) {
    const uint32_t x = f2u(f);
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return sign | 0x7E00u;        /* NaN */
    if (ax >= 0x477FF000u) return sign | 0x7C00u;       /* rounds to +-inf */
    if (ax >= 0x38800000u) {                            /* normal binary16 */
        uint32_t r = ax + 0xFFFu + ((ax >> 13) & 1u);   /* RNE at bit 13 */
        return sign | (uint16_t)((r - 0x38000000u) >> 13);
    }
    /* subnormal binary16: round(|f| * 2^24) to nearest even */
    float v = u2f(ax) * 0x1p24f;
    float r = (v + 8388608.0f) - 8388608.0f;
    return sign | (uint16_t)r;
}

/* ------------------------------------------------------------------------
 * 6-bit scale/min unpack, reference src/quant.c:72-80.
 * ------------------------------------------------------------------------ */
void fo_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* ------------------------------------------------------------------------
 * Dequantization.
 * ------------------------------------------------------------------------ */

/* Reference src/quant.c:82-105. Element 64g+l: d1*(qs[32g+l]&15)-m1;
 * element 64g+32+l: d2*(qs[32g+l]>>4)-m2 with (d1,m1),(d2,m2) of sub-blocks
 * 2g and 2g+1. */
static void deq_q4_K(const block_q4_K *x, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++, y += QK_K) {
        const float d = fo_fp16_to_fp32(x[i].d), dmin = fo_fp16_to_fp32(x[i].dmin);
        for (int g = 0; g < 4; g++) {
            uint8_t sc, m;
            fo_get_scale_min_k4(2 * g, x[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = dmin * m;
            fo_get_scale_min_k4(2 * g + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = dmin * m;
            const uint8_t *q = x[i].qs + 32 * g;
            for (int l = 0; l < 32; l++) y[64 * g + l] = d1 * (q[l] & 0xF) - m1;
            for (int l = 0; l < 32; l++) y[64 * g + 32 + l] = d2 * (q[l] >> 4) - m2;
        }
    }
}

/* Reference src/quant.c:216-247: Q4_K with a fifth bit per value, bit 2g of
 * qh[l] for element 64g+l and bit 2g+1 for element 64g+32+l. */
static void deq_q5_K(const block_q5_K *x, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++, y += QK_K) {
        const float d = fo_fp16_to_fp32(x[i].d), dmin = fo_fp16_to_fp32(x[i].dmin);
        for (int g = 0; g < 4; g++) {
            uint8_t sc, m;
            fo_get_scale_min_k4(2 * g, x[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = dmin * m;
            fo_get_scale_min_k4(2 * g + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = dmin * m;
            const uint8_t *q = x[i].qs + 32 * g;
            for (int l = 0; l < 32; l++) {
                int hi = (x[i].qh[l] >> (2 * g)) & 1;
                y[64 * g + l] = d1 * ((q[l] & 0xF) + (hi ? 16 : 0)) - m1;
            }
            for (int l = 0; l < 32; l++) {
                int hi = (x[i].qh[l] >> (2 * g + 1)) & 1;
                y[64 * g + 32 + l] = d2 * ((q[l] >> 4) + (hi ? 16 : 0)) - m2;
            }
        }
    }
}

/* Q6_K code of element e (0..255) of one block, in [-32, 31], and its
 * sub-block scale index. Layout per reference src/quant.c:147-175: for half
 * n and l<32, elements 128n+l+32t (t=0..3) take ql[64n+l] low/ql[64n+l+32]
 * low/ql[64n+l] high/ql[64n+l+32] high with qh[32n+l] bits 2t..2t+1. */
static inline int q6_code(const block_q6_K *b, int e) {
    const int n = e >> 7, r = e & 127, t = r >> 5, l = r & 31;
    const uint8_t qlb = b->ql[64 * n + l + ((t & 1) ? 32 : 0)];
    const int lo = (t & 2) ? (qlb >> 4) : (qlb & 0xF);
    const int hi = (b->qh[32 * n + l] >> (2 * t)) & 3;
    return (lo | (hi << 4)) - 32;
}

static void deq_q6_K(const block_q6_K *x, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++, y += QK_K) {
        const float d = fo_fp16_to_fp32(x[i].d);
        for (int e = 0; e < QK_K; e++) y[e] = d * x[i].scales[e >> 4] * q6_code(&x[i], e);
    }
}

/* Reference src/quant.c:266-274. */
static void deq_q8_0(const block_q8_0 *x, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float d = fo_fp16_to_fp32(x[i].d);
        for (int j = 0; j < QK8_0; j++) y[i * QK8_0 + j] = d * x[i].qs[j];
    }
}

/* E2M1 code values and the E8M0 scale, reference src/quant.c:290-315. */
static float e2m1_value(int c) {
    static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    return (c & 8) ? -mag[c & 7] : mag[c & 7];
}
static float e8m0_scale(uint8_t s) { return s == 0xFF ? 0.0f : ldexpf(1.0f, (int)s - 127); }

static void deq_mxfp4(const block_mxfp4 *x, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++) {
        const float s = e8m0_scale(x[i].s);
        for (int j = 0; j < QK_MXFP4 / 2; j++) {
            y[i * QK_MXFP4 + j] = e2m1_value(x[i].qs[j] & 0xF) * s;
            y[i * QK_MXFP4 + j + QK_MXFP4 / 2] = e2m1_value(x[i].qs[j] >> 4) * s;
        }
    }
}

int fo_dequantize_row(int type, const void *x, float *y, int64_t k) {
    const int bv = fomoe_block_values(type);
    if (bv == 0 || k % bv) return -1;
    const int64_t nb = k / bv;
    switch (type) {
        case GGML_TYPE_Q4_K: deq_q4_K((const block_q4_K *)x, y, nb); return 0;
        case GGML_TYPE_Q5_K: deq_q5_K((const block_q5_K *)x, y, nb); return 0;
        case GGML_TYPE_Q6_K: deq_q6_K((const block_q6_K *)x, y, nb); return 0;
        case GGML_TYPE_Q8_0: deq_q8_0((const block_q8_0 *)x, y, nb); return 0;
        case GGML_TYPE_MXFP4: deq_mxfp4((const block_mxfp4 *)x, y, nb); return 0;
        case GGML_TYPE_F32: memcpy(y, x, (size_t)k * 4); return 0;
        case GGML_TYPE_F16:
            for (int64_t i = 0; i < k; i++) y[i] = fo_fp16_to_fp32(((const uint16_t *)x)[i]);
            return 0;
        case GGML_TYPE_BF16:
            for (int64_t i = 0; i < k; i++) y[i] = u2f((uint32_t)((const uint16_t *)x)[i] << 16);
            return 0;
        default: return -1;
    }
}

/* ------------------------------------------------------------------------
 * fp32-activation dots: per super-block partial `sum`, then sumf += sum, in
 * the element order of the reference loops.
 * ------------------------------------------------------------------------ */

/* Reference src/quant.c:109-143. */
static float dot_q4_K(const block_q4_K *x, const float *y, int64_t nb) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; i++, y += QK_K) {
        const float d = fo_fp16_to_fp32(x[i].d), dmin = fo_fp16_to_fp32(x[i].dmin);
        float sum = 0.0f;
        for (int g = 0; g < 4; g++) {
            uint8_t sc, m;
            fo_get_scale_min_k4(2 * g, x[i].scales, &sc, &m);
            const float d1 = d * sc, m1 = dmin * m;
            fo_get_scale_min_k4(2 * g + 1, x[i].scales, &sc, &m);
            const float d2 = d * sc, m2 = dmin * m;
            const uint8_t *q = x[i].qs + 32 * g;
            for (int l = 0; l < 32; l++) sum += (d1 * (q[l] & 0xF) - m1) * y[64 * g + l];
            for (int l = 0; l < 32; l++) sum += (d2 * (q[l] >> 4) - m2) * y[64 * g + 32 + l];
        }
        sumf += sum;
    }
    return sumf;
}

/* Reference src/quant.c:177-212: for each half n and l<32 the four terms
 * ((d*sc)*q)*y of elements l, l+32, l+64, l+96 are added in that order. */
static float dot_q6_K(const block_q6_K *x, const float *y, int64_t nb) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; i++) {
        const float d = fo_fp16_to_fp32(x[i].d);
        const float *yp = y + i * QK_K;
        float sum = 0.0f;
        for (int n = 0; n < 2; n++) {
            for (int l = 0; l < 32; l++) {
                for (int t = 0; t < 4; t++) {
                    const int e = 128 * n + l + 32 * t;
                    sum += d * x[i].scales[e >> 4] * q6_code(&x[i], e) * yp[e];
                }
            }
        }
        sumf += sum;
    }
    return sumf;
}

/* Reference src/quant.c:249-262 (dequantize the block, then dot). */
static float dot_q5_K(const block_q5_K *x, const float *y, int64_t nb) {
    float tmp[QK_K], sumf = 0.0f;
    for (int64_t i = 0; i < nb; i++) {
        deq_q5_K(&x[i], tmp, 1);
        float sum = 0.0f;
        for (int j = 0; j < QK_K; j++) sum += tmp[j] * y[i * QK_K + j];
        sumf += sum;
    }
    return sumf;
}

/* Reference src/quant.c:276-288: d applied per block after the int*fp32 sum. */
static float dot_q8_0(const block_q8_0 *x, const float *y, int64_t nb) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; i++) {
        const float d = fo_fp16_to_fp32(x[i].d);
        float sum = 0.0f;
        for (int j = 0; j < QK8_0; j++) sum += (float)x[i].qs[j] * y[i * QK8_0 + j];
        sumf += d * sum;
    }
    return sumf;
}

/* Reference src/quant.c:317-337. */
static float dot_mxfp4(const block_mxfp4 *x, const float *y, int64_t nb) {
    float sumf = 0.0f;
    for (int64_t i = 0; i < nb; i++) {
        const float s = e8m0_scale(x[i].s);
        float sum = 0.0f;
        for (int j = 0; j < QK_MXFP4 / 2; j++) {
            sum += e2m1_value(x[i].qs[j] & 0xF) * y[i * QK_MXFP4 + j];
            sum += e2m1_value(x[i].qs[j] >> 4) * y[i * QK_MXFP4 + j + QK_MXFP4 / 2];
        }
        sumf += s * sum;
    }
    return sumf;
}

float fo_vec_dot_f32(int type, const void *x, const float *y, int64_t n) {
    const int bv = fomoe_block_values(type);
    if (bv == 0) return NAN;
    const int64_t nb = n / bv;
    switch (type) {
        case GGML_TYPE_Q4_K: return dot_q4_K((const block_q4_K *)x, y, nb);
        case GGML_TYPE_Q5_K: return dot_q5_K((const block_q5_K *)x, y, nb);
        case GGML_TYPE_Q6_K: return dot_q6_K((const block_q6_K *)x, y, nb);
        case GGML_TYPE_Q8_0: return dot_q8_0((const block_q8_0 *)x, y, nb);
        case GGML_TYPE_MXFP4: return dot_mxfp4((const block_mxfp4 *)x, y, nb);
        case GGML_TYPE_F32: {
            float s = 0.0f;
            for (int64_t j = 0; j < n; j++) s += ((const float *)x)[j] * y[j];
            return s;
        }
        case GGML_TYPE_F16: {
            float s = 0.0f;
            for (int64_t j = 0; j < n; j++) s += fo_fp16_to_fp32(((const uint16_t *)x)[j]) * y[j];
            return s;
        }
        case GGML_TYPE_BF16: {
            float s = 0.0f;
            for (int64_t j = 0; j < n; j++) s += u2f((uint32_t)((const uint16_t *)x)[j] << 16) * y[j];
            return s;
        }
        default: return NAN;
    }
}

/* Reference src/tensor.c:102-173: one dot per row, rows in parallel if M>64. */
void fo_mat_vec_mul(float *out, const void *mat, int type, const float *vec,
                    int64_t M, int64_t K) {
    const uint64_t rb = fomoe_row_bytes(type, K);
    if (rb == 0) return;
    #pragma omp parallel for if(M > 64)
    for (int64_t i = 0; i < M; i++)
        out[i] = fo_vec_dot_f32(type, (const uint8_t *)mat + (uint64_t)i * rb, vec, K);
}

/* ------------------------------------------------------------------------
 * Tensor ops, reference src/tensor.c:175-252.
 * ------------------------------------------------------------------------ */
void fo_rms_norm(float *out, const float *x, const float *w, int64_t n, float eps) {
    float ss = 0.0f;
    for (int64_t i = 0; i < n; i++) ss += x[i] * x[i];
    ss = 1.0f / sqrtf(ss / n + eps);
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * ss * w[i];
}

void fo_softmax(float *x, int64_t n) {
    float mx = x[0];
    for (int64_t i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) { x[i] = expf(x[i] - mx); sum += x[i]; }
    const float inv = 1.0f / sum;
    for (int64_t i = 0; i < n; i++) x[i] *= inv;
}

void fo_silu(float *x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = x[i] / (1.0f + expf(-x[i]));
}

/* Insertion into a descending list; a later equal value never displaces an
 * earlier one, so ties keep the lowest index. Slots start at (-1, -1e30). */
void fo_top_k(const float *x, int64_t n, int k, int *indices, float *values) {
    for (int i = 0; i < k; i++) { indices[i] = -1; values[i] = -1e30f; }
    for (int64_t j = 0; j < n; j++) {
        int pos = k;
        while (pos > 0 && x[j] > values[pos - 1]) pos--;
        if (pos < k) {
            for (int i = k - 1; i > pos; i--) { indices[i] = indices[i - 1]; values[i] = values[i - 1]; }
            indices[pos] = (int)j;
            values[pos] = x[j];
        }
    }
}

/* ------------------------------------------------------------------------
 * Q8_K activation path (the reference cpu_expert engine).
 * ------------------------------------------------------------------------ */

/* Reference src/quant.c:343-375: iscale = 127/amax, roundf, clamp +-127,
 * 16-wide block sums, d = 1/iscale. */
void fo_quantize_row_q8_K(const float *x, block_q8_K *y, int64_t k) {
    for (int64_t i = 0; i < k / QK_K; i++, x += QK_K) {
        float amax = 0.0f;
        for (int j = 0; j < QK_K; j++) { float a = fabsf(x[j]); if (a > amax) amax = a; }
        if (amax == 0.0f) { memset(&y[i], 0, sizeof(block_q8_K)); continue; }
        const float iscale = 127.0f / amax;
        for (int j = 0; j < QK_K; j++) {
            int v = (int)roundf(iscale * x[j]);
            y[i].qs[j] = (int8_t)(v > 127 ? 127 : (v < -127 ? -127 : v));
        }
        for (int j = 0; j < QK_K / 16; j++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += y[i].qs[16 * j + l];
            y[i].bsums[j] = (int16_t)s;
        }
        y[i].d = 1.0f / iscale;
    }
}

/* Reference src/quant.c:405-476: integer sums per super-block, scaled by
 * y.d*d (scales) and -y.d*dmin (mins via bsums). The reference spreads the
 * fp32 accumulation over eight SIMD lanes; this restatement sums in block
 * order, so it agrees to fp32 rounding, not bit for bit. */
float fo_vec_dot_q4_K_q8_K(const block_q4_K *x, const block_q8_K *y, int nb) {
    float acc = 0.0f, acc_m = 0.0f;
    for (int i = 0; i < nb; i++) {
        const float d = y[i].d * fo_fp16_to_fp32(x[i].d);
        const float dmin = -y[i].d * fo_fp16_to_fp32(x[i].dmin);
        /* the block's codes in value order, then exact integer sums per
         * sub-block (integer order does not matter: vectorisable) */
        uint8_t q[QK_K];
        for (int c = 0; c < 4; c++)
            for (int l = 0; l < 32; l++) {
                q[64 * c + l] = x[i].qs[32 * c + l] & 0xF;
                q[64 * c + 32 + l] = x[i].qs[32 * c + l] >> 4;
            }
        int32_t sumi = 0, summ = 0;
        for (int j = 0; j < 8; j++) {
            uint8_t sc, m;
            fo_get_scale_min_k4(j, x[i].scales, &sc, &m);
            const int8_t *q8 = y[i].qs + 32 * j;
            int32_t s = 0;
            for (int l = 0; l < 32; l++) s += q[32 * j + l] * q8[l];
            sumi += sc * s;
            summ += m * (y[i].bsums[2 * j] + y[i].bsums[2 * j + 1]);
        }
        acc += d * (float)sumi;
        acc_m += dmin * (float)summ;
    }
    return acc + acc_m;
}

/* Reference src/quant.c:478-607: sum over 16-wide sub-blocks of
 * sc * sum((q-32)*q8), scaled by y.d*d. */
float fo_vec_dot_q6_K_q8_K(const block_q6_K *x, const block_q8_K *y, int nb) {
    float acc = 0.0f;
    for (int i = 0; i < nb; i++) {
        const float d = y[i].d * fo_fp16_to_fp32(x[i].d);
        /* the block's codes in value order (q6_code), then exact integer
         * sums per 16-wide scale group: the order of integer additions does
         * not change them, so these loops may be vectorised freely */
        int8_t q[QK_K];
        for (int n = 0; n < 2; n++)
            for (int l = 0; l < 32; l++) {
                const uint8_t a = x[i].ql[64 * n + l], b = x[i].ql[64 * n + l + 32], h = x[i].qh[32 * n + l];
                q[128 * n + l] = (int8_t)(((a & 0xF) | ((h & 3) << 4)) - 32);
                q[128 * n + l + 32] = (int8_t)(((b & 0xF) | (((h >> 2) & 3) << 4)) - 32);
                q[128 * n + l + 64] = (int8_t)(((a >> 4) | (((h >> 4) & 3) << 4)) - 32);
                q[128 * n + l + 96] = (int8_t)(((b >> 4) | (((h >> 6) & 3) << 4)) - 32);
            }
        int32_t sumi = 0;
        for (int s = 0; s < 16; s++) {
            int32_t p = 0;
            for (int l = 0; l < 16; l++) p += q[16 * s + l] * y[i].qs[16 * s + l];
            sumi += x[i].scales[s] * p;
        }
        acc += d * (float)sumi;
    }
    return acc;
}

/* Reference src/quant.c:588-600 (AVX2 build: dequantize, then fp32 dot
 * against d*q8). */
float fo_vec_dot_q5_K_q8_K(const block_q5_K *x, const block_q8_K *y, int nb) {
    float tmp[QK_K], sumf = 0.0f;
    for (int i = 0; i < nb; i++) {
        deq_q5_K(&x[i], tmp, 1);
        float sum = 0.0f;
        for (int j = 0; j < QK_K; j++) sum += tmp[j] * y[i].d * y[i].qs[j];
        sumf += sum;
    }
    return sumf;
}

/* Reference src/cpu_expert.c:52-72 (Q8_0 and other types are skipped). */
void fo_matvec_q8(float *out, const void *mat, int type, const block_q8_K *q8, int M, int K) {
    const int nb = K / QK_K;
    const uint64_t rb = fomoe_row_bytes(type, K);
    #pragma omp parallel for schedule(static)
    for (int i = 0; i < M; i++) {
        const uint8_t *row = (const uint8_t *)mat + (uint64_t)i * rb;
        if (type == GGML_TYPE_Q4_K) out[i] = fo_vec_dot_q4_K_q8_K((const block_q4_K *)row, q8, nb);
        else if (type == GGML_TYPE_Q6_K) out[i] = fo_vec_dot_q6_K_q8_K((const block_q6_K *)row, q8, nb);
        else if (type == GGML_TYPE_Q5_K) out[i] = fo_vec_dot_q5_K_q8_K((const block_q5_K *)row, q8, nb);
    }
}

/* Reference src/cpu_expert.c:75-116. */
void fo_cpu_expert_ffn(const void *expert, const float *input, float score,
                       int gate_type, int up_type, int down_type,
                       uint64_t gate_size, uint64_t up_size,
                       int n_embd, int inter, float *partial) {
    const uint8_t *e = (const uint8_t *)expert;
    block_q8_K *q8in = (block_q8_K *)malloc(sizeof(block_q8_K) * (size_t)(n_embd / QK_K));
    block_q8_K *q8g = (block_q8_K *)malloc(sizeof(block_q8_K) * (size_t)(inter / QK_K));
    float *g = (float *)malloc(sizeof(float) * (size_t)(2 * inter + n_embd));
    float *u = g + inter, *dn = u + inter;
    fo_quantize_row_q8_K(input, q8in, n_embd);
    fo_matvec_q8(g, e, gate_type, q8in, inter, n_embd);
    fo_matvec_q8(u, e + gate_size, up_type, q8in, inter, n_embd);
    for (int i = 0; i < inter; i++) g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
    fo_quantize_row_q8_K(g, q8g, inter);
    fo_matvec_q8(dn, e + gate_size + up_size, down_type, q8g, n_embd, inter);
    for (int i = 0; i < n_embd; i++) partial[i] += score * dn[i];
    free(q8in); free(q8g); free(g);
}

/* ------------------------------------------------------------------------
 * MoE layer, reference src/inference.c:481-606 (router matvec, softmax,
 * top-k, renormalise, per-expert gate->silu, up, mul, down, scaled add in
 * rank order, shared expert with optional sigmoid gate, residual).
 * Shared expert FFN: reference src/inference.c:361-374.
 * ------------------------------------------------------------------------ */
static void expert_ffn(const uint8_t *blob, int gt, int ut, int dt, uint64_t gs, uint64_t us,
                       const float *h, int H, int F, float *out) {
    float *g = (float *)malloc(sizeof(float) * (size_t)F * 2);
    float *u = g + F;
    fo_mat_vec_mul(g, blob, gt, h, F, H);
    fo_silu(g, F);
    fo_mat_vec_mul(u, blob + gs, ut, h, F, H);
    for (int i = 0; i < F; i++) g[i] = g[i] * u[i];
    fo_mat_vec_mul(out, blob + gs + us, dt, g, H, F);
    free(g);
}

void fo_moe_layer(const fo_moe_desc *L, const float *in, float *out, int flags,
                  int *ids_out, float *w_out) {
    const int H = L->n_embd, E = L->n_experts, k = L->k;
    float *h = (float *)malloc(sizeof(float) * (size_t)H * 3);
    float *ffn = h + H, *dn = ffn + H;
    float *logits = (float *)malloc(sizeof(float) * (size_t)E);
    int ids[64];
    float sc[64];

    if (flags & FO_MOE_NORM) fo_rms_norm(h, in, L->norm_w, H, L->eps);
    else memcpy(h, in, sizeof(float) * (size_t)H);

    fo_mat_vec_mul(logits, L->router, GGML_TYPE_F32, h, E, H);
    if (L->router_bias) for (int e = 0; e < E; e++) logits[e] += L->router_bias[e];
    fo_softmax(logits, E);
    fo_top_k(logits, E, k, ids, sc);
    float ssum = 0.0f;
    for (int i = 0; i < k; i++) ssum += sc[i];
    if (ssum > 0.0f) { const float inv = 1.0f / ssum; for (int i = 0; i < k; i++) sc[i] *= inv; }

    memset(ffn, 0, sizeof(float) * (size_t)H);
    for (int i = 0; i < k; i++) {
        expert_ffn(L->experts + (uint64_t)ids[i] * L->expert_stride, L->gate_type, L->up_type,
                   L->down_type, L->gate_size, L->up_size, h, H, L->inter, dn);
        for (int j = 0; j < H; j++) ffn[j] += sc[i] * dn[j];
    }
    if (L->shared) {
        expert_ffn(L->shared, L->shared_gate_type, L->shared_up_type, L->shared_down_type,
                   L->shared_gate_size, L->shared_up_size, h, H, L->shared_inter, dn);
        if (L->shared_gate_vec) {
            float dot = 0.0f;
            for (int j = 0; j < H; j++) dot += h[j] * L->shared_gate_vec[j];
            const float gsc = 1.0f / (1.0f + expf(-dot));
            for (int j = 0; j < H; j++) dn[j] *= gsc;
        }
        for (int j = 0; j < H; j++) ffn[j] = ffn[j] + dn[j];
    }
    for (int j = 0; j < H; j++) out[j] = (flags & FO_MOE_RESIDUAL) ? in[j] + ffn[j] : ffn[j];
    if (ids_out) memcpy(ids_out, ids, sizeof(int) * (size_t)k);
    if (w_out) memcpy(w_out, sc, sizeof(float) * (size_t)k);
    free(h);
    free(logits);
}

/* ------------------------------------------------------------------------
 * bf16 and the prefill composition.
 * ------------------------------------------------------------------------ */
uint16_t fo_fp32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
float fo_bf16_to_fp32(uint16_t b) { return u2f((uint32_t)b << 16); }
void fo_fp32_to_bf16_n(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = fo_fp32_to_bf16(x[i]);
}

static float f16_round(float v) { return fo_fp16_to_fp32(fo_fp32_to_fp16(v)); }

/* A Q6_K row as the fp16 operands of the GPU prefill's down projection:
 * fp16(q - 32) * fp16(d * sc) rounded to fp16 (both roundings nearest-even;
 * d * sc and the product are exact in fp32 before rounding). Value order
 * and scales as deq_q6_K. */
static void deq_q6_K_f16ops(const block_q6_K *x, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++, y += QK_K) {
        const float d = fo_fp16_to_fp32(x[i].d);
        for (int e = 0; e < QK_K; e++)
            y[e] = f16_round((float)q6_code(&x[i], e) * f16_round(d * (float)x[i].scales[e >> 4]));
    }
}

/* A Q8_0 row as the fp16 operands of the GPU prefill's down projection:
 * fp16(d * q) (the product exact in fp32, one nearest-even rounding). Value
 * order as dequantize_row_q8_0 (reference src/quant.c:266-274). */
static void deq_q8_0_f16ops(const block_q8_0 *x, float *y, int64_t nb) {
    for (int64_t i = 0; i < nb; i++, y += 32) {
        const float d = fo_fp16_to_fp32(x[i].d);
        for (int e = 0; e < 32; e++) y[e] = f16_round(d * (float)x[i].qs[e]);
    }
}

/* rows x cols matrix of `type` dequantized exactly, then rounded to bf16
 * when `round` is 1; round 2: the fp16 operands of the GPU prefill's down
 * projection (Q6_K, Q8_0 as above; other types the exact value rounded to
 * fp16) */
static float *deq_bf16(const uint8_t *w, int type, int rows, int cols, int round) {
    float *m = (float *)malloc(sizeof(float) * (size_t)rows * cols);
    const uint64_t rb = fomoe_row_bytes(type, cols);
#pragma omp parallel for if (rows > 64)
    for (int r = 0; r < rows; r++) {
        float *y = m + (size_t)r * cols;
        if (round == 2 && type == GGML_TYPE_Q6_K) {
            deq_q6_K_f16ops((const block_q6_K *)(w + (uint64_t)r * rb), y, cols / QK_K);
            continue;
        }
        if (round == 2 && type == GGML_TYPE_Q8_0) {
            deq_q8_0_f16ops((const block_q8_0 *)(w + (uint64_t)r * rb), y, cols / 32);
            continue;
        }
        fo_dequantize_row(type, w + (uint64_t)r * rb, y, cols);
        if (round == 2)   /* Q4_K, Q5_K: the exact value rounded once to fp16 */
            for (int c = 0; c < cols; c++) y[c] = f16_round(y[c]);
        else if (round)
            for (int c = 0; c < cols; c++) y[c] = fo_bf16_to_fp32(fo_fp32_to_bf16(y[c]));
    }
    return m;
}

/* The activation row as the fp16 down path carries it: v = hi + lo of its
 * bf16 split, scaled by the power of two 2^-s that brings max|v| into
 * [2^14, 2^15), rounded to fp16; returns s (values stay scaled). */
static int act_f16(float *g, int n) {
    float m = 0.0f;
    for (int i = 0; i < n; i++) {
        const float hi = fo_bf16_to_fp32(fo_fp32_to_bf16(g[i]));
        g[i] = hi + fo_bf16_to_fp32(fo_fp32_to_bf16(g[i] - hi));
        m = fmaxf(m, fabsf(g[i]));
    }
    int e = 0;
    frexpf(m, &e);
    const int s = e - 15;
    for (int i = 0; i < n; i++) g[i] = f16_round(ldexpf(g[i], -s));
    return s;
}

static void matvec_f64(float *out, const float *m, const float *v, int rows, int cols) {
#pragma omp parallel for if (rows > 64)
    for (int r = 0; r < rows; r++) {
        double s = 0.0;
        const float *row = m + (size_t)r * cols;
        for (int c = 0; c < cols; c++) s += (double)row[c] * (double)v[c];
        out[r] = (float)s;
    }
}

/* bf16_mask: bit 0 gate, bit 1 up, bit 2 down weights rounded to bf16;
 * bit 3: the down projection on fp16 operands (deq_bf16 round 2 weights,
 * act_f16 activation) instead; bit 4: bits 0-3 chosen per expert from its
 * types as the GPU prefill does (exact Q4_K/Q4_K gate/up, else bf16; fp16
 * operands for the down projection with F <= 4096, else bf16) */
static void expert_ffn_bf16(const uint8_t *blob, int gt, int ut, int dt, int H, int F, uint64_t gs, uint64_t us,
                            const float *x, float *out, int bf16_mask) {
    if (bf16_mask & 16)
        bf16_mask = ((gt == GGML_TYPE_Q4_K && ut == GGML_TYPE_Q4_K) ? 0 : 3) |
                    (F <= 4096 ? 8 : 4);
    float *g = (float *)malloc(sizeof(float) * (size_t)F * 2), *u = g + F;
    float *wg = deq_bf16(blob, gt, F, H, (bf16_mask & 1) ? 1 : 0);
    matvec_f64(g, wg, x, F, H);
    free(wg);
    float *wu = deq_bf16(blob + gs, ut, F, H, (bf16_mask & 2) ? 1 : 0);
    matvec_f64(u, wu, x, F, H);
    free(wu);
    for (int i = 0; i < F; i++) g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
    const int f16 = (bf16_mask & 8) != 0;
    const int s = f16 ? act_f16(g, F) : 0;
    float *wd = deq_bf16(blob + gs + us, dt, H, F, f16 ? 2 : (bf16_mask & 4) ? 1 : 0);
    matvec_f64(out, wd, g, H, F);
    if (f16)
        for (int r = 0; r < H; r++) out[r] = ldexpf(out[r], s);
    free(wd);
    free(g);
}

void fo_moe_prefill_w(const fo_moe_desc *L, const uint16_t *x, int t0, int nt, float *out, int flags,
                      int *ids_out, float *w_out, int bf16_mask) {
    const int H = L->n_embd, E = L->n_experts, k = L->k;
    float *h = (float *)malloc(sizeof(float) * (size_t)H * 3);
    float *ffn = h + H, *dn = ffn + H;
    float *logits = (float *)malloc(sizeof(float) * (size_t)E);
    int ids[64];
    float sc[64];
    for (int t = t0; t < t0 + nt; t++) {
        for (int j = 0; j < H; j++) h[j] = fo_bf16_to_fp32(x[(size_t)t * H + j]);
        fo_mat_vec_mul(logits, L->router, GGML_TYPE_F32, h, E, H);
        if (L->router_bias) for (int e = 0; e < E; e++) logits[e] += L->router_bias[e];
        fo_softmax(logits, E);
        fo_top_k(logits, E, k, ids, sc);
        float ssum = 0.0f;
        for (int i = 0; i < k; i++) ssum += sc[i];
        if (ssum > 0.0f) { const float inv = 1.0f / ssum; for (int i = 0; i < k; i++) sc[i] *= inv; }
        memset(ffn, 0, sizeof(float) * (size_t)H);
        for (int i = 0; i < k; i++) {
            expert_ffn_bf16(L->experts + (uint64_t)ids[i] * L->expert_stride, L->gate_type, L->up_type,
                            L->down_type, H, L->inter, L->gate_size, L->up_size, h, dn, bf16_mask);
            for (int j = 0; j < H; j++) ffn[j] += sc[i] * dn[j];
        }
        float gsc = 1.0f;
        if (L->shared) {
            expert_ffn_bf16(L->shared, L->shared_gate_type, L->shared_up_type, L->shared_down_type, H,
                            L->shared_inter, L->shared_gate_size, L->shared_up_size, h, dn, bf16_mask);
            if (L->shared_gate_vec) {
                float dot = 0.0f;
                for (int j = 0; j < H; j++) dot += h[j] * L->shared_gate_vec[j];
                gsc = 1.0f / (1.0f + expf(-dot));
                for (int j = 0; j < H; j++) dn[j] *= gsc;
            }
            for (int j = 0; j < H; j++) ffn[j] = ffn[j] + dn[j];
        }
        float *o = out + (size_t)(t - t0) * H;
        for (int j = 0; j < H; j++) o[j] = (flags & FO_MOE_RESIDUAL) ? h[j] + ffn[j] : ffn[j];
        if (ids_out) memcpy(ids_out + (size_t)(t - t0) * k, ids, sizeof(int) * (size_t)k);
        if (w_out) {
            memcpy(w_out + (size_t)(t - t0) * (k + 1), sc, sizeof(float) * (size_t)k);
            w_out[(size_t)(t - t0) * (k + 1) + k] = gsc;
        }
    }
    free(h);
    free(logits);
}

void fo_moe_prefill(const fo_moe_desc *L, const uint16_t *x, int t0, int nt, float *out, int flags,
                    int *ids_out, float *w_out) {
    fo_moe_prefill_w(L, x, t0, nt, out, flags, ids_out, w_out, 7);
}

/* ------------------------------------------------------------------------
 * Synthetic data. Counter-based SplitMix64 (Steele, Lea & Flood 2014): the
 * i-th output for state `key` is mix(key + (i+1)*golden). Normals come from
 * Box-Muller evaluated in float64 with +,-,* only (log, sin/cos, 1/x and
 * 1/sqrt by series and Newton steps with fixed iteration counts), so every
 * IEEE-conforming CPU or GPU produces the same bits; the result is rounded
 * to fp32 once.
 * ------------------------------------------------------------------------ */
#define GOLDEN 0x9E3779B97F4A7C15ull

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t fo_rng_key(uint64_t seed, uint64_t stream) {
    return mix64(seed * GOLDEN + mix64(stream + 0x632BE59BD9B4E019ull));
}

uint64_t fo_rng_u64(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * GOLDEN); }

static inline double d_from_bits(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }
static inline uint64_t d_bits(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }

/* 1/a for a in [1.5, 2.5] by 6 Newton steps from 0.4. */
static double recip_newton(double a) {
    double r = 0.4;
    for (int i = 0; i < 6; i++) r = r * (2.0 - a * r);
    return r;
}

/* ln(u) for u in (0, 1]: u = m*2^e with m in [sqrt(1/2), sqrt(2)),
 * ln m = 2*atanh(s), s = (m-1)/(m+1), series to s^25. */
static double ln_det(double u) {
    uint64_t b = d_bits(u);
    int e = (int)((b >> 52) & 0x7FF) - 1023;
    double m = d_from_bits((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
    if (m > 0x1.6a09e667f3bcdp+0) { m = m * 0.5; e += 1; }
    const double s = (m - 1.0) * recip_newton(m + 1.0);
    const double s2 = s * s;
    static const double c[13] = {
        0x1.0000000000000p+0, 0x1.5555555555555p-2, 0x1.999999999999ap-3, 0x1.2492492492492p-3,
        0x1.c71c71c71c71cp-4, 0x1.745d1745d1746p-4, 0x1.3b13b13b13b14p-4, 0x1.1111111111111p-4,
        0x1.e1e1e1e1e1e1ep-5, 0x1.af286bca1af28p-5, 0x1.8618618618618p-5, 0x1.642c8590b2164p-5,
        0x1.47ae147ae147bp-5};
    double p = c[12];
    for (int i = 11; i >= 0; i--) p = p * s2 + c[i];
    return (double)e * 0x1.62e42fefa39efp-1 + 2.0 * s * p;
}

/* sin and cos of phi in [0, pi/2) by Taylor series to phi^25 / phi^26. */
static void sincos_det(double phi, double *sn, double *cs) {
    static const double ks[13] = {
        0x1.0000000000000p+0, -0x1.5555555555555p-3, 0x1.1111111111111p-7, -0x1.a01a01a01a01ap-13,
        0x1.71de3a556c734p-19, -0x1.ae64567f544e4p-26, 0x1.6124613a86d09p-33, -0x1.ae7f3e733b81fp-41,
        0x1.952c77030ad4ap-49, -0x1.2f49b46814157p-57, 0x1.71b8ef6dcf572p-66, -0x1.761b41316381ap-75,
        0x1.3f3ccdd165fa9p-84};
    static const double kc[14] = {
        0x1.0000000000000p+0, -0x1.0000000000000p-1, 0x1.5555555555555p-5, -0x1.6c16c16c16c17p-10,
        0x1.a01a01a01a01ap-16, -0x1.27e4fb7789f5cp-22, 0x1.1eed8eff8d898p-29, -0x1.93974a8c07c9dp-37,
        0x1.ae7f3e733b81fp-45, -0x1.6827863b97d97p-53, 0x1.e542ba4020225p-62, -0x1.0ce396db7f853p-70,
        0x1.f2cf01972f578p-80, -0x1.88e85fc6a4e5ap-89};
    const double p2 = phi * phi;
    double s = ks[12], c = kc[13];
    for (int i = 11; i >= 0; i--) s = s * p2 + ks[i];
    for (int i = 12; i >= 0; i--) c = c * p2 + kc[i];
    *sn = s * phi;
    *cs = c;
}

/* sqrt(v) for v >= 0 via 1/sqrt(v) (bit-trick seed, 5 Newton steps). */
static double sqrt_det(double v) {
    if (v == 0.0) return 0.0;
    double y = d_from_bits(0x5FE6EB50C7B537A9ull - (d_bits(v) >> 1));
    for (int i = 0; i < 5; i++) y = y * (1.5 - 0.5 * v * y * y);
    return v * y;
}

float fo_normal(uint64_t key, uint64_t i) {
    const uint64_t j = i >> 1;
    const uint64_t r1 = fo_rng_u64(key, 2 * j), r2 = fo_rng_u64(key, 2 * j + 1);
    const double u1 = (double)((r1 >> 11) + 1) * 0x1p-53;   /* (0, 1] */
    const double t = (double)(r2 >> 11) * 0x1p-51;          /* 4*u2 in [0, 4) */
    const int q = (int)t;
    const double phi = (t - (double)q) * 0x1.921fb54442d18p+0;
    const double rad = sqrt_det(-2.0 * ln_det(u1));
    double s, c, cq, sq;
    sincos_det(phi, &s, &c);
    switch (q) {   /* angle = q*pi/2 + phi */
        case 0: cq = c; sq = s; break;
        case 1: cq = -s; sq = c; break;
        case 2: cq = -c; sq = -s; break;
        default: cq = s; sq = -c; break;
    }
    return (float)(rad * ((i & 1) ? sq : cq));
}

void fo_synth_f32(uint64_t seed, uint64_t stream, float std, float *out, int64_t n) {
    const uint64_t key = fo_rng_key(seed, stream);
    #pragma omp parallel for if(n > 65536)
    for (int64_t i = 0; i < n; i++) out[i] = std * fo_normal(key, (uint64_t)i);
}

/* ------------------------------------------------------------------------
 * Quantizers (this build's own; float ops only, round half up via floor).
 * ------------------------------------------------------------------------ */
static inline int nearest_clamp(float v, int lo, int hi) {
    float r = floorf(v + 0.5f);
    if (!(r >= (float)lo)) return lo;   /* also maps NaN to lo */
    if (r > (float)hi) return hi;
    return (int)r;
}

/* Q4_K (and Q5_K when nbits=5): per 32-value sub-block, scale=(max-min)/L and
 * min=-min(0,min); d, dmin = max/63 rounded to fp16; 6-bit sub-scales against
 * those; codes = round((x + dmin*m)/(d*sc)). */
static void quant_kq_block(const float *x, int nbits, uint16_t *dh_out, uint16_t *dmh_out,
                           uint8_t scales[12], uint8_t codes[256]) {
    const float L = (float)((1 << nbits) - 1);
    float sc_f[8], mn_f[8], max_sc = 0.0f, max_mn = 0.0f;
    for (int j = 0; j < 8; j++) {
        float mn = x[32 * j], mx = x[32 * j];
        for (int l = 1; l < 32; l++) {
            const float v = x[32 * j + l];
            if (v < mn) mn = v;
            if (v > mx) mx = v;
        }
        if (mn > 0.0f) mn = 0.0f;
        sc_f[j] = (mx - mn) / L;
        mn_f[j] = -mn;
        if (sc_f[j] > max_sc) max_sc = sc_f[j];
        if (mn_f[j] > max_mn) max_mn = mn_f[j];
    }
    const uint16_t dh = fo_fp32_to_fp16(max_sc / 63.0f), dmh = fo_fp32_to_fp16(max_mn / 63.0f);
    const float df = fo_fp16_to_fp32(dh), dmf = fo_fp16_to_fp32(dmh);
    uint8_t sc[8], m[8];
    for (int j = 0; j < 8; j++) {
        sc[j] = (uint8_t)(df > 0.0f ? nearest_clamp(sc_f[j] / df, 0, 63) : 0);
        m[j] = (uint8_t)(dmf > 0.0f ? nearest_clamp(mn_f[j] / dmf, 0, 63) : 0);
        const float ds = df * (float)sc[j], dm = dmf * (float)m[j];
        for (int l = 0; l < 32; l++)
            codes[32 * j + l] = (uint8_t)(ds > 0.0f ? nearest_clamp((x[32 * j + l] + dm) / ds, 0, (int)L) : 0);
    }
    /* pack per reference src/quant.c:72-80 (inverse of get_scale_min_k4) */
    for (int j = 0; j < 4; j++) {
        scales[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        scales[j + 4] = (uint8_t)((m[j] & 63) | ((m[j + 4] >> 4) << 6));
        scales[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    *dh_out = dh;
    *dmh_out = dmh;
}

static void quant_q4_K(const float *x, block_q4_K *b) {
    uint8_t c[256];
    quant_kq_block(x, 4, &b->d, &b->dmin, b->scales, c);
    for (int g = 0; g < 4; g++)
        for (int l = 0; l < 32; l++)
            b->qs[32 * g + l] = (uint8_t)(c[64 * g + l] | (c[64 * g + 32 + l] << 4));
}

static void quant_q5_K(const float *x, block_q5_K *b) {
    uint8_t c[256];
    quant_kq_block(x, 5, &b->d, &b->dmin, b->scales, c);
    memset(b->qh, 0, sizeof b->qh);
    for (int g = 0; g < 4; g++)
        for (int l = 0; l < 32; l++) {
            const int lo = c[64 * g + l], hi = c[64 * g + 32 + l];
            b->qs[32 * g + l] = (uint8_t)((lo & 0xF) | ((hi & 0xF) << 4));
            b->qh[l] |= (uint8_t)(((lo >> 4) << (2 * g)) | ((hi >> 4) << (2 * g + 1)));
        }
}

/* Q6_K: per 16-value sub-block scale = amax/31; d = max/127 rounded to fp16;
 * signed 8-bit sub-scales; codes round(x/(d*sc)) in [-32,31], stored +32. */
static void quant_q6_K(const float *x, block_q6_K *b) {
    float s_f[16], max_s = 0.0f;
    for (int s = 0; s < 16; s++) {
        float amax = 0.0f;
        for (int l = 0; l < 16; l++) { const float a = fabsf(x[16 * s + l]); if (a > amax) amax = a; }
        s_f[s] = amax / 31.0f;
        if (s_f[s] > max_s) max_s = s_f[s];
    }
    const uint16_t dh = fo_fp32_to_fp16(max_s / 127.0f);
    const float df = fo_fp16_to_fp32(dh);
    uint8_t u[256];
    for (int s = 0; s < 16; s++) {
        const int sc = df > 0.0f ? nearest_clamp(s_f[s] / df, -128, 127) : 0;
        b->scales[s] = (int8_t)sc;
        const float ds = df * (float)sc;
        for (int l = 0; l < 16; l++)
            u[16 * s + l] = (uint8_t)((ds > 0.0f ? nearest_clamp(x[16 * s + l] / ds, -32, 31) : 0) + 32);
    }
    for (int n = 0; n < 2; n++)
        for (int l = 0; l < 32; l++) {
            const int e = 128 * n + l;
            const int q1 = u[e], q2 = u[e + 32], q3 = u[e + 64], q4 = u[e + 96];
            b->ql[64 * n + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
            b->ql[64 * n + l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
            b->qh[32 * n + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    b->d = dh;
}

/* Q8_0: d = amax/127 rounded to fp16, codes round(x/d). */
static void quant_q8_0(const float *x, block_q8_0 *b) {
    float amax = 0.0f;
    for (int l = 0; l < 32; l++) { const float a = fabsf(x[l]); if (a > amax) amax = a; }
    const uint16_t dh = fo_fp32_to_fp16(amax / 127.0f);
    const float df = fo_fp16_to_fp32(dh);
    for (int l = 0; l < 32; l++)
        b->qs[l] = (int8_t)(df > 0.0f ? nearest_clamp(x[l] / df, -127, 127) : 0);
    b->d = dh;
}

int fo_quantize(int type, const float *W, void *dst, int64_t M, int64_t K) {
    const int bv = fomoe_block_values(type);
    if (bv == 0 || K % bv) return -1;
    const int64_t nb = K / bv;
    const uint64_t bb = fomoe_block_bytes(type);
    #pragma omp parallel for if(M > 64)
    for (int64_t r = 0; r < M; r++) {
        for (int64_t i = 0; i < nb; i++) {
            const float *x = W + r * K + i * bv;
            uint8_t *b = (uint8_t *)dst + ((uint64_t)r * nb + i) * bb;
            switch (type) {
                case GGML_TYPE_Q4_K: quant_q4_K(x, (block_q4_K *)b); break;
                case GGML_TYPE_Q5_K: quant_q5_K(x, (block_q5_K *)b); break;
                case GGML_TYPE_Q6_K: quant_q6_K(x, (block_q6_K *)b); break;
                case GGML_TYPE_Q8_0: quant_q8_0(x, (block_q8_0 *)b); break;
                case GGML_TYPE_F32: memcpy(b, x, 4); break;
                default: break;
            }
        }
    }
    return (type == GGML_TYPE_Q4_K || type == GGML_TYPE_Q5_K || type == GGML_TYPE_Q6_K ||
            type == GGML_TYPE_Q8_0 || type == GGML_TYPE_F32) ? 0 : -1;
}

int fo_synth_quant(int type, uint64_t seed, uint64_t stream, float std,
                   int64_t M, int64_t K, void *dst) {
    float *W = (float *)malloc(sizeof(float) * (size_t)(M * K));
    if (!W) return -1;
    fo_synth_f32(seed, stream, std, W, M * K);
    const int rc = fo_quantize(type, W, dst, M, K);
    free(W);
    return rc;
}

/* Zipf(s) bias: Fisher-Yates permutation of experts driven by the stream,
 * rank(e) = 1 + position; bias = -s*ln(rank). */
void fo_zipf_bias(uint64_t seed, uint64_t stream, int n, double s, float *bias) {
    const uint64_t key = fo_rng_key(seed, stream);
    int *perm = (int *)malloc(sizeof(int) * (size_t)n);
    for (int i = 0; i < n; i++) perm[i] = i;
    for (int i = n - 1; i > 0; i--) {
        const int j = (int)(fo_rng_u64(key, (uint64_t)i) % (uint64_t)(i + 1));
        const int t = perm[i]; perm[i] = perm[j]; perm[j] = t;
    }
    for (int r = 0; r < n; r++) bias[perm[r]] = (float)(-s * log((double)(r + 1)));
    free(perm);
}
