// moe.h — argument blocks of the three-kernel MoE layer (moe.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "shared.h"

namespace fo {

// K1: logits[E] = router . h (+ bias), h = rms_norm(x) * norm_w (norm_w NULL:
// h = x); writes the prepared h (groups of gsz) and *shared_w = sigmoid(h.v)
// (1 when shared_gate_vec is NULL).
struct RouteArgs {
    const float *router, *bias, *x, *norm_w;
    float eps;
    int E, H;
    float *logits;
    uint8_t *xq_h;
    int gsz;
    const float *shared_gate_vec;
    float *shared_w;
};

// K2: top-k of logits, then act_e = silu(gate_e . h) * (up_e . h) for the k
// routed experts (blob = base + id*stride: gate at 0, up at gate_size) and,
// when shared is set, the shared expert (gate at 0, up at sh_gate_size),
// written in prepared form (groups of down_gsz) at xq_act + e*xq_vstride
// (shared: e = k), and as fp32 to act if set. The first work-group with
// nothing else to wait for writes ids[k] / weights[k].
struct ExpandArgs {
    const float *logits;
    int E, k;
    int32_t *ids;
    float *weights;
    const uint8_t *base;
    uint64_t stride, gate_size;
    const uint8_t *shared;
    uint64_t sh_gate_size;
    int F, H;
    uint64_t row_bytes;
    const uint8_t *xq_h;
    uint8_t *xq_act;
    uint64_t xq_vstride;
    int down_gsz;
    float *act;
    int act_only;           // 1: leave xq_act unwritten, act (non-NULL) is the down
                            // kernel's input (ReduceArgs::act_f32)
};

// K3: out[i] = (resid ? resid[i] : 0) + sum_e w_e * down_e[i,:] . act_e over
// the k routed experts in rank order, then the shared expert (weight
// *shared_w, or 1 when NULL) — in the layer's kernels when it has the routed
// types and F (shared != NULL), else from ys[i] (its down projection computed
// by another kernel, weighted here by *shared_w; NULL: none).
struct ReduceArgs {
    const int32_t *ids;
    const float *weights;
    const float *shared_w;
    int k;
    const uint8_t *base;
    uint64_t stride, down_off;
    const uint8_t *shared;
    uint64_t sh_down_off;
    int F, H;
    uint64_t row_bytes;
    const uint8_t *xq_act;
    uint64_t xq_vstride;
    const float *resid;
    float *out;
    const float *ys;
    int sh_type;            // -1: the shared block has the routed down type; else its own
                            // type (F = 1024, reduce_takes_shared_type), from sh_act
    const float *sh_act;    // [F] fp32 shared activation (sh_type >= 0)
    const float *act_f32;   // NULL, or [n_tot x F] fp32 activations, each wave preparing its slot from
                            // them (bit-identical to xq_act's form; the LDS-staged kernel only)
};

hipError_t launch_route(const RouteArgs &a, hipStream_t s);
hipError_t launch_expand(int gate_type, const ExpandArgs &a, hipStream_t s, int n_cu);
hipError_t launch_reduce(int down_type, const ReduceArgs &a, hipStream_t s, int n_cu);
// Whether launch_reduce takes the LDS-staged kernel (the one that can
// prepare its slots from fp32 activations) for this shape.
bool reduce_takes_tile(int down_type, const ReduceArgs &a);
// Whether launch_reduce runs a shared block of type sh_type beside routed
// down projections of down_type for this shape.
bool reduce_takes_shared_type(int down_type, const ReduceArgs &a, int sh_type);
// A shared expert with its own types or intermediate size (shared.h):
// act = silu(gate . h) * (up . h) with h = rms_norm(x) * norm_w (norm_w NULL:
// h = x), then ys = w * down . act (w = a.w, or 1 when NULL).
hipError_t launch_shared(const SharedArgs &a, const float *x, const float *norm_w, float eps, hipStream_t s);

}  // namespace fo
