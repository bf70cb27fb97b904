// kernels.h — argument blocks and launchers of the decode-path kernels.
// Host code (capi.cpp) fills these structs; kernels.hip implements them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fo {

// y[m][r] = W_m[r,:] . x_m for m < n_mats, r < M (batch-1 matvec over many
// matrices in one launch: a layer's experts, or a rotation of them).
struct MatvecArgs {
    const uint8_t *W;       // matrix m at W + m*mat_stride
    uint64_t mat_stride;
    uint64_t row_bytes;
    const uint8_t *xq;      // prepared x_m = xq + m*x_stride bytes (0: shared)
    uint64_t x_stride;
    float *y;               // y_m = y + m*y_stride
    uint64_t y_stride;
    int n_mats, M, K;
    const float *xf;        // fp32 x_m = xf + m*xf_stride, for kernels that prepare it themselves
    uint64_t xf_stride;
};

// True when launch_matvec's kernel for this shape prepares x itself from
// MatvecArgs::xf (no separate activation-prep launch): the Q6_K tile-staged
// kernel always, the general kernel when every matrix shares one x.
bool matvec_self_prep(int type, uint64_t row_bytes, int K, uint64_t x_stride);

// Router: logits = W_r . h (+ bias), h = rms_norm(x)*w when norm_w != NULL,
// then (last work-group) softmax, top-k with lowest-index ties, renormalise,
// and the shared-expert gate sigmoid(h . shared_gate_vec).
struct RouterArgs {
    const float *W;         // [E x H] fp32
    const float *bias;      // [E] or NULL
    const float *x;         // [H]
    const float *norm_w;    // [H] or NULL (no norm)
    float eps;
    int E, H, k;
    float *logits;          // [E] scratch
    unsigned *counter;      // zero before the first launch; reset by the kernel
    int32_t *ids;           // [k]
    float *weights;         // [k + 1]: routed weights, then the shared weight
    const float *shared_gate_vec;  // [H] or NULL (shared weight 1)
};

// act[e][r] = silu(gate_e[r,:].h) * (up_e[r,:].h), e < n_sel routed experts
// (blob = base + ids[e]*stride, or base + e*stride if ids is NULL).
struct GateUpArgs {
    const int32_t *ids;
    int n_sel;
    const uint8_t *base;
    uint64_t stride, gate_off, up_off;
    int F, H;
    uint64_t row_bytes;
    const float *x;
    const float *norm_w;    // h = rms_norm(x)*norm_w when non-NULL, else h = x
    float eps;
    float *act;             // [n_sel x F]
};

// out[i] = (resid ? resid[i] : 0) + (sum_e weights[e] * down_e[i,:].act_e
// + (ys ? ys[i] : 0)); ys = the weighted shared expert's output.
struct DownArgs {
    const int32_t *ids;
    const float *weights;   // [n_sel]
    int n_sel;
    const uint8_t *base;
    uint64_t stride, down_off;
    const float *ys;        // [H] or NULL
    const float *act;       // [n_sel x F]
    int H, F;
    uint64_t row_bytes;
    const float *resid;
    float *out;
};

// Launchers return hipSuccess, or hipErrorInvalidValue for a shape the
// kernels do not cover (checked on the host before any launch).
// Prepare n_vec fp32 vectors of K values (x_stride floats apart) into the
// block-fixed-point form the matvec kernels consume (xq_stride bytes apart).
hipError_t launch_xprep(int gsz, const float *x, uint64_t x_stride, int K, int n_vec,
                        uint8_t *xq, uint64_t xq_stride, hipStream_t s);
hipError_t launch_matvec(int type, const MatvecArgs &a, hipStream_t s, int n_cu);
// xq_h (may be NULL) receives the prepared h in groups of gsz.
hipError_t launch_router(const RouterArgs &a, uint8_t *xq_h, int gsz, hipStream_t s);
hipError_t launch_gateup(int type, const GateUpArgs &a, const uint8_t *xq_h, hipStream_t s,
                         int n_cu);
hipError_t launch_down(int type, const DownArgs &a, const uint8_t *xq_act, uint64_t xq_vstride,
                       hipStream_t s, int n_cu);
hipError_t launch_dequant(int type, const uint8_t *src, float *dst, int64_t n, hipStream_t s);
hipError_t launch_silu_mul(float *g, const float *u, int64_t n, hipStream_t s);
// p[0..n) = 0 with a kernel (usable inside captured graphs, unlike a memset node)
hipError_t launch_zero_u32(uint32_t *p, int n, hipStream_t s);

// Synthetic data (bit-identical to the CPU generator in oracle/).
hipError_t launch_synth_f32(uint64_t seed, uint64_t stream, float std, float *out,
                            int64_t n, hipStream_t s);
hipError_t launch_synth_quant(int type, uint64_t seed, uint64_t stream0, uint64_t stream_step,
                              float std, int64_t M, int64_t K, int n_mats, uint8_t *dst,
                              uint64_t dst_stride, hipStream_t s);
hipError_t launch_quantize(int type, const float *W, int64_t M, int64_t K, uint8_t *dst,
                           hipStream_t s);

// Largest supported K per slot count.
constexpr int kMaxSlotsPerLane = 4;

}  // namespace fo
