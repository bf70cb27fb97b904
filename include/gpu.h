/*
 * gpu.h — C-ABI of libfomoe_gfx950.so, the MI355X (gfx950) implementation of
 * fomoe's quantized MoE expert hot path.
 *
 * Drop-in part: gpu_ctx_t, gpu_init, gpu_free and gpu_expert_ffn keep the
 * reference's signatures, ownership and -1 "fall back to CPU" semantics
 * (reference include/gpu.h:10-16, 68-83; implementation
 * src/gpu_kernels.hip:8385-8488). Every other function of the reference's
 * gpu.h is exported too (section "reference lifecycle"), so a -DQMOE_GPU build
 * of the reference links against this library.
 *
 * HBM-resident extensions (no reference counterpart; the reference copies
 * every expert host-to-device per call, which defeats residency): explicit
 * device pointers, int return codes (0 ok, -1 invalid argument / unsupported
 * shape, -2 device error; the message is in gpu_last_error), never exit().
 * All device work is ordered on the context's single stream; calls marked
 * "async" return before the device finishes (use gpu_sync). A context is not
 * re-entrant: one host thread per context, as in the reference.
 */
#ifndef FOMOE_GPU_H
#define FOMOE_GPU_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gpu_ctx gpu_ctx_t;

/* ---------------------------------------------------------------- lifecycle
 * gpu_init: select device 0, create the stream and scratch. NULL when no
 * device is present (reference include/gpu.h:13; gpu_kernels.hip:3774-3777).
 * gpu_free: release everything the context allocated (reference gpu.h:16). */
gpu_ctx_t *gpu_init(void);
void gpu_free(gpu_ctx_t *ctx);

/* ---------------------------------------------------------------- legacy FFN
 * Routed-expert FFN for host buffers (reference include/gpu.h:68-83):
 *   ffn_out = sum_e expert_scores[e] * down_e(silu(gate_e.h) * (up_e.h))
 * expert_buffers[e] points at a host blob gate | up | down (gate at 0, up at
 * expert_gate_size, down at expert_gate_size + expert_up_size). Excludes the
 * shared expert and the residual. Synchronous. Returns 0, or -1 for a NULL
 * ctx, n_experts > 10, n_embd > 4096, expert_intermediate > 2048,
 * expert_stride > 12 MiB, a gate/up/down type outside {Q4_K, Q5_K, Q6_K},
 * or a device error (same limits as reference gpu_kernels.hip:438-441,
 * 8393-8403). */
int gpu_expert_ffn(gpu_ctx_t *ctx,
                   const float *h,
                   void **expert_buffers,
                   const float *expert_scores,
                   int n_experts,
                   int n_embd,
                   int expert_intermediate,
                   uint64_t expert_gate_size,
                   uint64_t expert_up_size,
                   uint64_t expert_stride,
                   int gate_type,
                   int up_type,
                   int down_type,
                   float *ffn_out);

/* ---------------------------------------------------------------- reference lifecycle
 * The rest of the reference's gpu.h, with the same signatures, so that a
 * reference build with -DQMOE_GPU links against this library. This build has
 * no whole-model forward (attention, embeddings, KV cache and the expert cache
 * tiers are outside its scope), so each entry point returns the reference's
 * own "not available" result and the reference's caller takes its CPU path:
 *   gpu_register_buffers / gpu_unregister_buffers (reference gpu.h:19-22):
 *     no-ops; gpu_expert_ffn copies from pageable host memory.
 *   gpu_upload_model (gpu.h:26): -1 (model.c:423 prints "GPU upload failed,
 *     CPU fallback").
 *   gpu_set_ram_cache_mb / gpu_set_vram_cache_mb (gpu.h:30, 34): recorded,
 *     no effect (all experts are HBM-resident through gpu_moe_layer).
 *   gpu_forward (gpu.h:38): NULL (inference.c:427-431 frees the context and
 *     runs the CPU forward).
 *   gpu_reset_state (gpu.h:41): no-op (this build keeps no KV / SSM state).
 *   gpu_seed_vram_cache (gpu.h:46): -1 (model.c:429-431 warns and goes on).
 *   gpu_enable_expert_freq / gpu_get_expert_freq / gpu_get_expert_dims
 *     (gpu.h:50-57): counting is never active; the getter returns NULL and the
 *     dims are 0, which main.c:956 treats as "no profile".
 *   gpu_get_pingpong_relay_stats (gpu.h:61-66): all zero, the reference's
 *     single-GPU answer. */
void gpu_register_buffers(gpu_ctx_t *ctx, void **buffers, int n, uint64_t size);
void gpu_unregister_buffers(gpu_ctx_t *ctx, void **buffers, int n);
int gpu_upload_model(gpu_ctx_t *ctx, const void *model);
void gpu_set_ram_cache_mb(gpu_ctx_t *ctx, int mb);
void gpu_set_vram_cache_mb(gpu_ctx_t *ctx, int mb);
float *gpu_forward(gpu_ctx_t *ctx, void *model, int token_id, int pos);
void gpu_reset_state(gpu_ctx_t *ctx);
int gpu_seed_vram_cache(gpu_ctx_t *ctx, void *model, const char *freq_profile_path);
void gpu_enable_expert_freq(gpu_ctx_t *ctx);
const uint32_t *gpu_get_expert_freq(gpu_ctx_t *ctx);
void gpu_get_expert_dims(gpu_ctx_t *ctx, int *n_layers, int *n_experts);
void gpu_get_pingpong_relay_stats(gpu_ctx_t *ctx, uint64_t *handoffs, uint64_t *payload_bytes,
                                  uint64_t *d2h_bytes, uint64_t *h2d_bytes, uint64_t *dma_bytes);

/* ---------------------------------------------------------------- device memory */
void *gpu_alloc(gpu_ctx_t *ctx, uint64_t bytes);               /* NULL on failure */
void  gpu_dealloc(gpu_ctx_t *ctx, void *d_ptr);
int   gpu_upload(gpu_ctx_t *ctx, void *d_dst, const void *h_src, uint64_t bytes);   /* sync */
int   gpu_download(gpu_ctx_t *ctx, void *h_dst, const void *d_src, uint64_t bytes); /* sync */
int   gpu_sync(gpu_ctx_t *ctx);
/* n_cu, total HBM bytes and the gfx arch name of the context's device. */
int   gpu_device_info(gpu_ctx_t *ctx, int *n_cu, uint64_t *hbm_bytes, char *arch, int arch_len);
const char *gpu_last_error(gpu_ctx_t *ctx);

/* ---------------------------------------------------------------- kernels (async)
 * gpu_dequantize: d_dst[n] = dequantized values of d_src, bit-identical to
 * reference src/quant.c dequantize_row_* (Q4_K, Q5_K, Q6_K, Q8_0, MXFP4, F16,
 * BF16, F32).
 * gpu_matvec_q: d_y[M] = W[M x K] . d_x[K] for quantized W (Q4_K, Q5_K, Q6_K:
 * K % 256 == 0; Q8_0: K % 32 == 0), fp32 activations, exact integer products
 * and fp32 accumulation (replaces reference mat_vec_mul, src/tensor.c:102-173,
 * on the device).
 * gpu_matvec_q_batched: the same for n_mats matrices W_m = d_W + m*mat_stride
 * bytes, x_m = d_x + m*x_stride floats (0: one shared x), y_m = d_y +
 * m*y_stride floats, in one launch. */
int gpu_dequantize(gpu_ctx_t *ctx, int type, const void *d_src, float *d_dst, int64_t n);
int gpu_matvec_q(gpu_ctx_t *ctx, int type, const void *d_W, const float *d_x, float *d_y,
                 int M, int K);
int gpu_matvec_q_batched(gpu_ctx_t *ctx, int type, const void *d_W, uint64_t mat_stride,
                         int n_mats, const float *d_x, uint64_t x_stride, float *d_y,
                         uint64_t y_stride, int M, int K);

/* ---------------------------------------------------------------- MoE layer */
typedef struct {
    int n_embd;                 /* H */
    int inter;                  /* F, routed-expert intermediate */
    int n_experts;              /* E (<= 1024) */
    int k;                      /* experts used per token (<= 16) */
    int gate_type, up_type, down_type;
    uint64_t gate_size, up_size, expert_stride;
    const float *router;        /* device [E x H] fp32 */
    const float *router_bias;   /* device [E] added to the logits, or NULL */
    const void *experts;        /* device, E blobs gate|up|down, expert_stride apart */
    const void *shared;         /* device shared-expert blob gate|up|down, or NULL */
    int shared_inter;           /* F_s, the shared expert's intermediate size */
    uint64_t shared_gate_size, shared_up_size;   /* up at gate_size, down at gate+up */
    const float *shared_gate_vec; /* device [H]: shared output *= sigmoid(h.v); NULL: 1 */
    const float *norm_w;        /* device [H] RMSNorm weight, used with GPU_MOE_NORM */
    float eps;
    /* the shared expert's own tensor types, each of Q4_K/Q5_K/Q6_K/Q8_0
     * (reference include/model.h:108; read from ffn_*_shexp, src/model.c:365-371) */
    int shared_gate_type, shared_up_type, shared_down_type;
} gpu_moe_layer_t;

#define GPU_MOE_NORM     1  /* h = rms_norm(in) * norm_w before routing */
#define GPU_MOE_RESIDUAL 2  /* out = in + ffn (else out = ffn); out may alias in */

/* One MoE layer for one token, everything device-resident (async):
 * router matvec, softmax, top-k (ties to the lowest index), renormalise,
 * routed SwiGLU experts, shared expert, weighted combine (reference
 * src/inference.c:481-606; gpu_kernels.hip 5514-5528, 7405-7435, 7740). */
int gpu_moe_layer(gpu_ctx_t *ctx, const gpu_moe_layer_t *layer, const float *d_in,
                  float *d_out, int flags);
/* gpu_moe_layer without any device allocation: no hipMalloc, hipFree or
 * allocating library call on any path (async, same semantics and kernels as
 * gpu_moe_layer, bit-identical results). No counterpart in the reference; it
 * is for callers that cannot allocate (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation). Its scratch is one static
 * device area of GPU_MOE_NOALLOC_SCRATCH_BYTES (contexts run on device 0),
 * held until the process ends; a layer whose scratch (router logits, routing,
 * prepared h, the k+1 activations, a shared expert's activation and output)
 * does not fit returns -1 with a message. Every call shares that area: calls
 * that overlap (two contexts, or two host threads) race, and the routing that
 * gpu_moe_last_routing reports after a no-allocation call is read from the
 * area, so it is that of the latest no-allocation call of any context. */
#define GPU_MOE_NOALLOC_SCRATCH_BYTES (1u << 20)
int gpu_moe_layer_noalloc(gpu_ctx_t *ctx, const gpu_moe_layer_t *layer, const float *d_in,
                          float *d_out, int flags);
/* Routing of the most recent gpu_moe_layer call (sync): k ids, k weights
 * and the shared-expert weight. */
int gpu_moe_last_routing(gpu_ctx_t *ctx, int32_t *ids, float *weights, float *shared_weight);
/* Router alone (async): d_ids[k], d_weights[k+1] (last = shared weight 1). */
int gpu_router_topk(gpu_ctx_t *ctx, const float *d_router, const float *d_bias,
                    const float *d_x, const float *d_norm_w, float eps, int n_experts,
                    int n_embd, int k, int32_t *d_ids, float *d_weights);

/* n_steps decode steps through n_layers layers, x <- x + moe_l(rms_norm(x))
 * per layer, in place on d_x[n_embd]. The per-step launch sequence is
 * captured into a HIP graph and replayed; the next call with the same
 * descriptors (byte for byte) and d_x replays that graph without capturing
 * again (one call per decoded token costs one graph launch). Async. */
int gpu_moe_stack_decode(gpu_ctx_t *ctx, const gpu_moe_layer_t *layers, int n_layers,
                         float *d_x, int n_steps);

/* ---------------------------------------------------------------- expert store (.qmoe)
 * The reference's expert-store file (reference include/expert_store.h:8-40,
 * src/expert_store.c, tools/prepare_experts.c:116-170): a 64-byte header and
 * one 32-byte entry per MoE layer, then per layer n_experts blobs gate|up|down
 * at expert_stride (4096-aligned) from data_offset; down_type may differ per
 * layer. The layouts below are that file format, byte for byte. */
#define GPU_QMOE_MAGIC   0x454F4D51u   /* "QMOE" */
#define GPU_QMOE_VERSION 2
typedef struct {
    uint32_t magic, version, n_moe_layers, n_experts, quant_type, alignment;
    uint64_t expert_gate_size, expert_up_size, expert_down_size, expert_stride;
    uint8_t reserved[8];
} gpu_qmoe_header_t;                  /* 64 bytes */
typedef struct {
    uint64_t data_offset, expert_stride, down_size;
    uint32_t down_type, pad;
} gpu_qmoe_layer_entry_t;             /* 32 bytes */

/* Host only (no device needed): read and validate the header and up to
 * max_layers index entries. Returns n_moe_layers, or -1 (unreadable file, bad
 * magic, version < 2, inconsistent sizes); *err (may be NULL) gets a message. */
int gpu_qmoe_read_index(const char *path, gpu_qmoe_header_t *hdr, gpu_qmoe_layer_entry_t *layers,
                        int max_layers, const char **err);
/* Copy layer `layer` (n_experts * expert_stride bytes) from the file into
 * device memory d_dst (sync; pinned double-buffered staging). 0 / -1 / -2. */
int gpu_qmoe_upload_layer(gpu_ctx_t *ctx, const char *path, int layer, void *d_dst, uint64_t dst_bytes);
/* Fill the type / size / stride fields of *L for one layer of the store
 * (experts, router and the other pointers are left to the caller). */
int gpu_qmoe_layer_desc(const gpu_qmoe_header_t *hdr, const gpu_qmoe_layer_entry_t *entry,
                        gpu_moe_layer_t *L);

/* ---------------------------------------------------------------- GGUF model files
 * Direct tensor loads from a GGUF model (replaces reference include/gguf.h:
 * gguf_open 121, gguf_close 124, gguf_find_key 127, gguf_get_* 130-140,
 * gguf_find_tensor 143, gguf_read_tensor 147, gguf_tensor_nbytes 150; format
 * and split-file rules of src/gguf.c:10-449). The handle is host-only and
 * read-only after open, so one handle may serve several contexts. */
typedef struct gpu_gguf gpu_gguf_t;
typedef struct {
    const char *name;          /* owned by the handle */
    uint32_t n_dims;
    int32_t type;              /* enum ggml_dtype id */
    int64_t dims[4];           /* ggml order: dims[0] is the contiguous one; unused = 1 */
    uint64_t offset;           /* within its split's data section */
    uint64_t size;             /* bytes, whole blocks (0: type of unknown size) */
    int32_t split;             /* index of the split file holding the data */
    int32_t pad;
} gpu_gguf_tensor_t;
/* Host only. Open and parse a GGUF file; a name with "-00001-of-0000N" also
 * reads the other splits (missing ones are skipped, as the reference does).
 * NULL on an unreadable or malformed file, *err (may be NULL) says why; the
 * message stays valid until the next failing call on this thread. */
gpu_gguf_t *gpu_gguf_open(const char *path, const char **err);
void gpu_gguf_close(gpu_gguf_t *g);
int64_t gpu_gguf_n_tensors(const gpu_gguf_t *g);
int64_t gpu_gguf_n_keys(const gpu_gguf_t *g);
int64_t gpu_gguf_find_tensor(const gpu_gguf_t *g, const char *name);   /* -1: absent */
int gpu_gguf_tensor_info(const gpu_gguf_t *g, int64_t id, gpu_gguf_tensor_t *out);  /* 0 / -1 */
int64_t gpu_gguf_find_key(const gpu_gguf_t *g, const char *key);       /* -1: absent */
/* Key i: name and gguf value type (8 string, 9 array, ...); NULL if out of range. */
const char *gpu_gguf_key(const gpu_gguf_t *g, int64_t i, int *type);
/* Typed getters: 0, or -1 when the key is absent or of another kind (any
 * integer or bool type reads as int, f32/f64 and integers as double). */
int gpu_gguf_get_int(const gpu_gguf_t *g, const char *key, int64_t *v);
int gpu_gguf_get_float(const gpu_gguf_t *g, const char *key, double *v);
const char *gpu_gguf_get_str(const gpu_gguf_t *g, const char *key);      /* NULL: absent */
/* Array key: element type and count, and the raw elements (NULL for a string
 * array; use gpu_gguf_get_arr_str). -1: absent or not an array. */
int gpu_gguf_get_arr(const gpu_gguf_t *g, const char *key, int *elem_type, uint64_t *n,
                     const void **data);
const char *gpu_gguf_get_arr_str(const gpu_gguf_t *g, const char *key, uint64_t i);
/* Bytes of n elements of a ggml type (whole blocks), 0 for an unknown type. */
uint64_t gpu_gguf_type_bytes(int type, uint64_t n);
/* Host only: copy tensor id into h_dst (bytes >= its size). Returns the size
 * read, or -1 (bad id, small buffer, data past the end of its file). */
int64_t gpu_gguf_read_tensor(const gpu_gguf_t *g, int64_t id, void *h_dst, uint64_t bytes);
/* Copy tensor id into device memory d_dst (sync, pinned staging). 0 / -1 / -2. */
int gpu_gguf_upload_tensor(gpu_ctx_t *ctx, const gpu_gguf_t *g, int64_t id, void *d_dst,
                           uint64_t dst_bytes);
/* Upload tensor id as fp32 into d_dst [n elements] (sync): F32 as is, F16 /
 * BF16 widened, Q4_K/Q5_K/Q6_K/Q8_0/MXFP4 dequantized bit-exactly (the
 * conversions of reference src/model.c:42-87). 0 / -1 / -2. */
int gpu_gguf_upload_f32(gpu_ctx_t *ctx, const gpu_gguf_t *g, int64_t id, float *d_dst, int64_t n);
/* Make MoE block `blk` resident (sync): allocates and fills the experts
 * ([E x stride] gate|up|down, stride = gate+up+down rounded up to 4096, the
 * .qmoe layout built by reference tools/prepare_experts.c:107-133, 261-279)
 * from blk.N.ffn_{gate,up,down}_exps.weight, the fp32 router
 * (ffn_gate_inp), the shared expert (ffn_{gate,up,down}_shexp, optional) and
 * its sigmoid gate vector (ffn_gate_inp_shexp, optional), and the RMSNorm
 * weight (post_attention_norm, else ffn_norm; optional), and sets every field
 * of *L: n_embd / inter / n_experts from the tensor shapes, k from
 * {arch}.expert_used_count, eps from {arch}.attention.layer_norm_rms_epsilon
 * (1e-6 if absent) (reference src/model.c:141-162, 349-371). Free with
 * gpu_gguf_free_moe_layer. 0 / -1 (missing tensor, unsupported type or shape)
 * / -2. */
int gpu_gguf_load_moe_layer(gpu_ctx_t *ctx, const gpu_gguf_t *g, int blk, gpu_moe_layer_t *L);
void gpu_gguf_free_moe_layer(gpu_ctx_t *ctx, gpu_moe_layer_t *L);

/* ---------------------------------------------------------------- prefill
 * n_tokens tokens through one MoE layer at once (async): d_x [n_tokens x
 * n_embd] bf16, d_out [n_tokens x n_embd] fp32 (= x + ffn with
 * GPU_MOE_RESIDUAL). Per token the semantics of gpu_moe_layer without the
 * norm (fp32-level router on the bf16 input — bf16 matrix cores with each
 * router weight as three exact bf16 terms when n_embd % 512 == 0, fp32 matrix
 * cores otherwise —, softmax, top-k, renormalise, shared expert); the expert GEMMs are grouped by expert and run on the matrix cores
 * with fp32 accumulation. Operands: Q4_K gate/up weights exactly (fp16 sc*q,
 * the tokens as fp16 under a per-token power of two); a Q6_K down projection
 * as fp16(q - 32) * fp16(d * sc) against the SwiGLU activation as fp16 under
 * a per-pair power of two (within ~6e-4 of the exact layer per token); other
 * types dequantized to bf16 (round to nearest even), with the activation as
 * two bf16 terms (hi + lo, within 2^-18). Types: gate/up Q4_K or Q6_K (any
 * mix), or both Q5_K or both Q8_0; down Q4_K, Q5_K, Q6_K or Q8_0; the same
 * sets for the shared expert: with the routed types and
 * intermediate size it is one more pair per token in the routed pass (with
 * only its down type differing, its down projection is a launch of its
 * own), with gate/up types or an intermediate size of its own it runs first
 * as a one-expert pass whose output the routed pass adds at the shared weight;
 * n_experts <= 1023; with Q4_K gate/up, the experts and shared pointers,
 * expert_stride and the gate sizes must be multiples of 16 bytes (-1 else). A batch larger than the grouping table (n_experts *
 * ceil(n_tokens/32) > 16384) runs as consecutive chunks of
 * (16384 / n_experts) * 32 tokens with the same results per token. No
 * counterpart in the reference, which decodes prompt tokens one at a time
 * (gpu_forward). */
int gpu_moe_prefill(gpu_ctx_t *ctx, const gpu_moe_layer_t *layer, const uint16_t *d_x, int n_tokens,
                    float *d_out, int flags);
/* Routing of the last gpu_moe_prefill (sync): ids [n_tokens x k], weights
 * [n_tokens x (k+1)] (the last per token is the shared-expert weight). */
int gpu_moe_prefill_routing(gpu_ctx_t *ctx, int32_t *ids, float *weights);
/* d_dst[i] = bf16(d_src[i]), round to nearest even (async). */
int gpu_f32_to_bf16(gpu_ctx_t *ctx, const float *d_src, uint16_t *d_dst, int64_t n);

/* ---------------------------------------------------------------- synthetic data
 * This build's own generator (no reference counterpart): counter-based
 * SplitMix64 normals and this build's quantizers; bit-identical to the CPU
 * generator in oracle/. Matrix m of a batch uses stream stream0 + m*step and
 * lands at d_dst + m*dst_stride. K % 256 == 0. Async. */
int gpu_synth_f32(gpu_ctx_t *ctx, uint64_t seed, uint64_t stream, float std, float *d_out,
                  int64_t n);
int gpu_synth_quant(gpu_ctx_t *ctx, int type, uint64_t seed, uint64_t stream0,
                    uint64_t stream_step, float std, int64_t M, int64_t K, int n_mats,
                    void *d_dst, uint64_t dst_stride);
/* Host-side Zipf(s) router bias: bias[e] = -s*ln(rank(e)), rank a seeded
 * permutation. */
void gpu_synth_zipf_bias(uint64_t seed, uint64_t stream, int n, double s, float *h_bias);

/* ---------------------------------------------------------------- timing
 * Events on the context's stream: gpu_timer_start records, gpu_timer_stop
 * records, waits and returns the elapsed milliseconds (< 0 on error). */
int   gpu_timer_start(gpu_ctx_t *ctx);
float gpu_timer_stop(gpu_ctx_t *ctx);

#ifdef __cplusplus
}
#endif

#endif /* FOMOE_GPU_H */
