/*
 * oracle.h — CPU restatement of the reference fomoe expert hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load liboracle.so, and only as the checker
 * or the timed CPU baseline — never as the computation being measured or
 * shipped. The product library (libfomoe_gfx950.so) does not link it.
 *
 * Every function cites the reference file:line whose behaviour it restates.
 * The synthetic-data generator (fo_rng_*, fo_synth_*, fo_quantize_*) has no
 * reference counterpart: the reference ships no quantizer (its only
 * quantizer is quantize_row_q8_K). It is this build's own definition and the
 * GPU generator must reproduce it bit for bit.
 */
#ifndef FOMOE_ORACLE_H
#define FOMOE_ORACLE_H

#include <stdint.h>
#include <stddef.h>
#include "quant_types.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 <-> fp32 (reference src/quant.c:30-67) ---- */
float    fo_fp16_to_fp32(uint16_t h);
uint16_t fo_fp32_to_fp16(float f);

/* ---- 6-bit scale/min unpack (reference src/quant.c:72-80) ---- */
void fo_get_scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m);

/* ---- row dequantization (reference src/quant.c:82-105, 147-175, 216-247,
 *      266-274, 298-315); k values, k a multiple of the block size ---- */
int fo_dequantize_row(int type, const void *x, float *y, int64_t k);

/* ---- fp32-activation dot products (reference src/quant.c:109-143,
 *      177-212, 249-262, 276-288, 317-337) ---- */
float fo_vec_dot_f32(int type, const void *x, const float *y, int64_t n);

/* ---- mat_vec_mul over fp32 activations (reference src/tensor.c:102-173).
 *      out[M] = W[M x K] . vec[K]; rows in parallel (OpenMP) when M > 64. */
void fo_mat_vec_mul(float *out, const void *mat, int type, const float *vec,
                    int64_t M, int64_t K);

/* ---- tensor ops (reference src/tensor.c:175-252) ---- */
void fo_rms_norm(float *out, const float *x, const float *w, int64_t n, float eps);
void fo_softmax(float *x, int64_t n);
void fo_silu(float *x, int64_t n);
void fo_top_k(const float *x, int64_t n, int k, int *indices, float *values);

/* ---- Q8_K activation path (reference src/quant.c:343-375, 405-607) ---- */
void  fo_quantize_row_q8_K(const float *x, block_q8_K *y, int64_t k);
float fo_vec_dot_q4_K_q8_K(const block_q4_K *x, const block_q8_K *y, int nb);
float fo_vec_dot_q6_K_q8_K(const block_q6_K *x, const block_q8_K *y, int nb);
float fo_vec_dot_q5_K_q8_K(const block_q5_K *x, const block_q8_K *y, int nb);
/* matvec over a pre-quantized Q8_K vector (reference src/cpu_expert.c:52-72) */
void  fo_matvec_q8(float *out, const void *mat, int type, const block_q8_K *q8,
                   int M, int K);
/* one routed expert on the CPU engine, partial += score*down(...)
 * (reference src/cpu_expert.c:75-116). scratch: >= 2*inter + n_embd floats. */
void  fo_cpu_expert_ffn(const void *expert, const float *input, float score,
                        int gate_type, int up_type, int down_type,
                        uint64_t gate_size, uint64_t up_size,
                        int n_embd, int inter, float *partial);

/* ---- MoE layer composition (reference src/inference.c:361-374, 481-606) ----
 * Experts are byte blobs laid out gate | up | down at `expert_stride` apart
 * (reference src/cpu_expert.c:84-88). */
typedef struct {
    int n_embd;            /* H */
    int inter;             /* F, routed expert intermediate */
    int n_experts;         /* E */
    int k;                 /* experts used per token */
    int gate_type, up_type, down_type;
    uint64_t gate_size, up_size, expert_stride;
    const float *router;        /* [E x H] fp32 */
    const float *router_bias;   /* [E] added to logits, or NULL */
    const uint8_t *experts;     /* E blobs, expert_stride apart */
    const uint8_t *shared;      /* shared expert blob (gate|up|down) or NULL */
    int shared_inter;           /* shared expert intermediate */
    uint64_t shared_gate_size, shared_up_size;
    const float *shared_gate_vec; /* [H] sigmoid gate for the shared expert, or NULL */
    const float *norm_w;        /* [H] RMSNorm weight (used with FO_MOE_NORM) */
    float eps;
    /* the shared expert's own tensor types (reference include/model.h:108) */
    int shared_gate_type, shared_up_type, shared_down_type;
} fo_moe_desc;

#define FO_MOE_NORM     1   /* h = rms_norm(x) before routing */
#define FO_MOE_RESIDUAL 2   /* out = x + ffn instead of out = ffn */

/* out[H] from in[H]; ids/weights[k] receive the routing (may be NULL). */
void fo_moe_layer(const fo_moe_desc *L, const float *in, float *out, int flags,
                  int *ids, float *weights);

/* ---- bf16 (round to nearest even; NaN kept quiet) ---- */
uint16_t fo_fp32_to_bf16(float f);
float    fo_bf16_to_fp32(uint16_t b);
void     fo_fp32_to_bf16_n(const float *x, uint16_t *y, int64_t n);

/* ---- multi-token MoE layer (prefill) for tokens t0 .. t0+nt-1 of x [T x H]
 * bf16. Per token the semantics of fo_moe_layer (no norm), with the expert
 * weights rounded to bf16 after exact dequantization, dot products
 * accumulated in double, and the SwiGLU activation kept in fp32 — the
 * arithmetic contract of the bf16 grouped-GEMM prefill.
 * The reference has no prefill GEMM; this composes reference
 * src/inference.c:481-606 per token. out [nt x H]; ids [nt x k];
 * w [nt x (k+1)] (last = shared weight). Only FO_MOE_RESIDUAL is honoured. */
void fo_moe_prefill(const fo_moe_desc *L, const uint16_t *x, int t0, int nt, float *out, int flags,
                    int *ids_out, float *w_out);
/* As fo_moe_prefill with a choice of which weight matrices are rounded to
 * bf16 (bit 0 gate, bit 1 up, bit 2 down; fo_moe_prefill = all three); bit
 * 3: a Q6_K down projection on the GPU's fp16 operands; bit 4 (value 16): the choice
 * made per expert from its own types, as the GPU prefill makes it. */
void fo_moe_prefill_w(const fo_moe_desc *L, const uint16_t *x, int t0, int nt, float *out, int flags,
                      int *ids_out, float *w_out, int bf16_mask);

/* ---- synthetic data (this build's own definition; no reference) ---- */
uint64_t fo_rng_key(uint64_t seed, uint64_t stream);
uint64_t fo_rng_u64(uint64_t key, uint64_t i);
float    fo_normal(uint64_t key, uint64_t i);        /* N(0,1) as fp32 */
void     fo_synth_f32(uint64_t seed, uint64_t stream, float std, float *out, int64_t n);
/* Quantize rows of W (fp32, [M x K] row-major) into `type` blocks. */
int      fo_quantize(int type, const float *W, void *dst, int64_t M, int64_t K);
/* W ~ std*N(0,1) from (seed, stream), quantized to `type`. */
int      fo_synth_quant(int type, uint64_t seed, uint64_t stream, float std,
                        int64_t M, int64_t K, void *dst);
/* Zipf(s) router bias for one layer: bias[e] = log(1/rank(e)^s), with rank a
 * seeded permutation of the experts. */
void     fo_zipf_bias(uint64_t seed, uint64_t stream, int n_experts, double s, float *bias);

#ifdef __cplusplus
}
#endif
#endif
