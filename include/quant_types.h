/*
 * quant_types.h — GGUF quantization block layouts shared by the host C code
 * and the gfx950 kernels of libfomoe_gfx950.
 *
 * The byte layout of every block is a file format (GGUF / ggml) and must stay
 * byte-compatible with the reference so that expert blobs written for it load
 * unchanged:
 *   block_q4_K  144 B  — reference include/quant_types.h:17-22
 *   block_q5_K  176 B  — reference include/quant_types.h:25-31
 *   block_q6_K  210 B  — reference include/quant_types.h:34-39
 *   block_q8_0   34 B  — reference include/quant_types.h:43-46
 *   block_mxfp4  17 B  — reference include/quant_types.h:50-53
 *   block_q8_K  (host-only activation blocks) — reference include/quant.h:94-98
 * The dtype ids are the ggml ids (reference include/quant_types.h:56-64).
 */
#ifndef FOMOE_QUANT_TYPES_H
#define FOMOE_QUANT_TYPES_H

#include <stdint.h>

#define QK_K 256          /* values per K-quant super-block */
#define K_SCALE_SIZE 12   /* packed 6-bit scale/min bytes in Q4_K / Q5_K */
#define QK8_0 32          /* values per Q8_0 block */
#define QK_MXFP4 32       /* values per MXFP4 block */

/* Q4_K: y = d*sc[j]*q - dmin*m[j], 8 sub-blocks of 32, q in [0,15]. */
typedef struct {
    uint16_t d;                     /* super-block scale, IEEE fp16 bits */
    uint16_t dmin;                  /* super-block min scale, IEEE fp16 bits */
    uint8_t  scales[K_SCALE_SIZE];  /* 8 x (6-bit scale, 6-bit min), packed */
    uint8_t  qs[QK_K / 2];          /* 4-bit codes, two per byte */
} block_q4_K;

/* Q5_K: Q4_K plus one high bit per value, q in [0,31]. */
typedef struct {
    uint16_t d;
    uint16_t dmin;
    uint8_t  scales[K_SCALE_SIZE];
    uint8_t  qh[QK_K / 8];          /* 5th bit of each code */
    uint8_t  qs[QK_K / 2];          /* low 4 bits of each code */
} block_q5_K;

/* Q6_K: y = d*sc[j]*(q-32), 16 sub-blocks of 16, q in [0,63]. */
typedef struct {
    uint8_t  ql[QK_K / 2];          /* low 4 bits of each code */
    uint8_t  qh[QK_K / 4];          /* high 2 bits of each code */
    int8_t   scales[QK_K / 16];     /* signed 8-bit sub-block scales */
    uint16_t d;                     /* super-block scale, IEEE fp16 bits */
} block_q6_K;

/* Q8_0: y = d*q, q in [-127,127]. */
typedef struct {
    uint16_t d;
    int8_t   qs[QK8_0];
} block_q8_0;

/* MXFP4: E8M0 shared exponent + 32 E2M1 codes. */
typedef struct {
    uint8_t s;
    uint8_t qs[QK_MXFP4 / 2];
} block_mxfp4;

/* Q8_K: activation blocks used by the CPU integer-dot baseline. */
typedef struct {
    float   d;
    int8_t  qs[QK_K];
    int16_t bsums[QK_K / 16];
} block_q8_K;

enum ggml_dtype {
    GGML_TYPE_F32   = 0,
    GGML_TYPE_F16   = 1,
    GGML_TYPE_Q8_0  = 8,
    GGML_TYPE_Q4_K  = 12,
    GGML_TYPE_Q5_K  = 13,
    GGML_TYPE_Q6_K  = 14,
    GGML_TYPE_BF16  = 30,
    GGML_TYPE_MXFP4 = 39,
};

#ifdef __cplusplus
#define FOMOE_STATIC_ASSERT static_assert
#else
#define FOMOE_STATIC_ASSERT _Static_assert
#endif
FOMOE_STATIC_ASSERT(sizeof(block_q4_K) == 144, "block_q4_K must be 144 bytes");
FOMOE_STATIC_ASSERT(sizeof(block_q5_K) == 176, "block_q5_K must be 176 bytes");
FOMOE_STATIC_ASSERT(sizeof(block_q6_K) == 210, "block_q6_K must be 210 bytes");
FOMOE_STATIC_ASSERT(sizeof(block_q8_0) == 34, "block_q8_0 must be 34 bytes");
FOMOE_STATIC_ASSERT(sizeof(block_mxfp4) == 17, "block_mxfp4 must be 17 bytes");

/* Bytes of one block and values per block of a dtype; 0 if unsupported. */
static inline uint64_t fomoe_block_bytes(int t) {
    switch (t) {
        case GGML_TYPE_Q4_K:  return 144;
        case GGML_TYPE_Q5_K:  return 176;
        case GGML_TYPE_Q6_K:  return 210;
        case GGML_TYPE_Q8_0:  return 34;
        case GGML_TYPE_MXFP4: return 17;
        case GGML_TYPE_F16:   return 2;
        case GGML_TYPE_BF16:  return 2;
        case GGML_TYPE_F32:   return 4;
        default:              return 0;
    }
}

static inline int fomoe_block_values(int t) {
    switch (t) {
        case GGML_TYPE_Q4_K:
        case GGML_TYPE_Q5_K:
        case GGML_TYPE_Q6_K:  return QK_K;
        case GGML_TYPE_Q8_0:  return QK8_0;
        case GGML_TYPE_MXFP4: return QK_MXFP4;
        case GGML_TYPE_F16:
        case GGML_TYPE_BF16:
        case GGML_TYPE_F32:   return 1;
        default:              return 0;
    }
}

/* Bytes of one row of K values (K a multiple of the block size). */
static inline uint64_t fomoe_row_bytes(int t, int64_t K) {
    int v = fomoe_block_values(t);
    return v ? (uint64_t)(K / v) * fomoe_block_bytes(t) : 0;
}

#endif /* FOMOE_QUANT_TYPES_H */
