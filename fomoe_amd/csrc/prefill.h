// prefill.h — argument block and launchers of the multi-token (prefill) MoE
// path: fp32 router GEMM, per-token top-k, deterministic grouping of
// (token, expert) pairs by expert, grouped gate/up and down GEMMs on fp16 /
// bf16 MFMA with the weight operands built in registers, and the per-token
// combine.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "quant_types.h"

namespace fo {

constexpr int kPfMT = 64;        // tokens per GEMM tile (4 MFMA row blocks of 16)
constexpr int kPfThin = 4;       // pairs of a thin tile (integer-MFMA Q6_K down path)
constexpr int kPfGateWaves = 8;                   // gate/up work-group: 4 gate + 4 up waves (two per CU)
constexpr int kPfGateRows = 32 * kPfGateWaves / 2; // F rows per gate/up work-group (32 per wave)

struct PrefillArgs {
    // layer
    int E, k, H, F;
    int gate_type, up_type, down_type;
    const float *router, *router_bias;
    const uint8_t *experts;      // E blobs gate|up|down, stride apart
    uint64_t stride, gate_size, up_size;
    const uint8_t *shared;       // shared blob or NULL
    uint64_t sh_gate_size, sh_up_size;
    const float *shared_gate_vec;  // [H] or NULL
    const float *ys;             // [T x H] or NULL: a shared expert's output computed by a pass of
                                 // its own, combined as the shared pair (weight w[t, k])
    // tokens
    int T;
    const uint16_t *x;           // [T x H] bf16
    float *out;                  // [T x H] fp32
    int residual;                // out = x + ffn
    // workspace (device)
    float *logits;               // [T x E]
    int32_t *ids;                // [T x k]
    float *w;                    // [T x (k+1)]: renormalised weights, then the shared weight
    int32_t *pairpos;            // [T x (k+1)]: pair slot of (token, rank); rank k = shared
    int32_t *pair_tok;           // [P] token of each pair slot, grouped by expert
    int32_t *tiles;              // [max_tiles x 4] {expert (E = shared), first pair, n, order}
    int32_t *dtiles;             // [max_tiles x 4] the same in tiles of up to 2 kPfMT pairs (k_pf_down16)
    int32_t *n_tiles;            // [6]: tiles, tiles before the thin ones, work counter of the gate/up
                                 // kernel, double tiles, double tiles before those of thin experts,
                                 // the shared expert's first tile
    int max_tiles;
    uint16_t *act_hi, *act_lo;   // [P x F] SwiGLU activation as bf16 hi + lo terms (a Q6_K
                                 // down projection rewrites act_hi as fp16 rows, scale in pexp)
    float *xsum;                 // [T x H/32] sums of x over 32-value sub-blocks (Q4_K gate/up path)
    uint16_t *x16;               // [T x H] fp16(x * 2^-xexp[t]) (Q4_K gate/up path)
    int32_t *xexp;               // [T] per-token power-of-two scale of x16
    float *outp;                 // [P x H] fp32, per-pair down output
    int32_t *pexp;               // [P] power-of-two scale of the fp16 activation rows (Q6_K down)
    uint16_t *rsplit;            // bf16 router GEMM operands (prefill_router_ws_elems)
    int thin_down;               // set by launch_prefill: thin tiles take k_pf_down_thin
    int sh_down_type;            // -1: the shared down projection has down_type; else its own type
                                 // (gate/up and F as the routed experts), run by a launch of its own
    int down_sel;                // set by launch_prefill: 0 every expert's down projection, 1 the
                                 // routed experts' only, 2 the shared expert's only
    int dt_sel;                  // set by launch_prefill: 1 leaves the shared expert out of dtiles
    int d16_shared;              // set by launch_prefill: k_pf_down16 runs one expert's T pairs in
                                 // token order (the shared expert's, T*k .. T*k + T, or a one-expert
                                 // pass's) in 32-pair tiles instead of dtiles
    int one_expert;              // every token to expert 0 at weight 1 (E = k = 1, no shared expert):
                                 // no router, top-k or combine; the down projection writes outp rows
                                 // in token order, which are then the output
    int xprep_ready;             // x16 / xsum / xexp already hold these tokens (a pass before this one)
};

// Number of pair slots and an upper bound on the GEMM tiles for T tokens.
// Weight types the prefill runs: gate/up both Q4_K (exact fp16 operands), a
// Q4_K/Q6_K mix, or both Q5_K or both Q8_0 (bf16 operands); down Q4_K, Q5_K,
// Q6_K or Q8_0.
inline bool prefill_types_ok(int gate, int up, int down) {
    auto k46 = [](int t) { return t == GGML_TYPE_Q4_K || t == GGML_TYPE_Q6_K; };
    const bool gu = (k46(gate) && k46(up)) || (gate == up && (gate == GGML_TYPE_Q5_K || gate == GGML_TYPE_Q8_0));
    const bool dn = k46(down) || down == GGML_TYPE_Q5_K || down == GGML_TYPE_Q8_0;
    return gu && dn;
}
inline int prefill_pairs(int T, int k, bool shared) { return T * (k + (shared ? 1 : 0)); }
inline int prefill_max_tiles(int T, int k, int E, bool shared) {
    return (prefill_pairs(T, k, shared) + kPfMT - 1) / kPfMT + E + (shared ? 1 : 0);
}

// Workspace of the bf16 router GEMM (rsplit, uint16 elements): the router's
// three bf16 terms and the token rows, in 32-row x 64-value chunks.
inline uint64_t prefill_router_ws_elems(int E, int T, int H) {
    return ((uint64_t)3 * ((E + 31) / 32) + (uint64_t)((T + 31) / 32)) * 32 * H;
}

hipError_t launch_prefill(const PrefillArgs &a, hipStream_t s);
hipError_t launch_f32_to_bf16(const float *src, uint16_t *dst, int64_t n, hipStream_t s);

}  // namespace fo
