// context.h — the gpu_ctx_t behind include/gpu.h and the host-side helpers
// the C-ABI files share (error recording, HIP call checking, scratch growth,
// pinned file-to-device staging).
#pragma once

#include <stdarg.h>
#include <stdio.h>

#include <string>
#include <vector>

#include "common.h"
#include "gpu.h"

struct gpu_ctx {
    int device = 0;
    int n_cu = 0;
    uint64_t hbm = 0;
    char arch[64] = {0};
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::string err;

    // scratch (device)
    float *logits = nullptr;       // [1024]
    unsigned *counter = nullptr;   // router completion counter
    int32_t *ids = nullptr;        // [16]
    float *weights = nullptr;      // [17]
    uint8_t *xq_h = nullptr;       size_t xq_h_cap = 0;
    uint8_t *xq_act = nullptr;     size_t xq_act_cap = 0;
    float *act = nullptr;          size_t act_cap = 0;
    float *act2 = nullptr;         size_t act2_cap = 0;
    float *sh_act = nullptr;       size_t sh_act_cap = 0;   // shared-expert activation [F_s]
    float *sh_ys = nullptr;        size_t sh_ys_cap = 0;    // weighted shared-expert output [H]
    float *vec_in = nullptr;       size_t vec_in_cap = 0;
    float *vec_out = nullptr;      size_t vec_out_cap = 0;
    uint8_t *staging = nullptr;    size_t staging_cap = 0;
    int last_k = 0;
    bool last_fast = false;      // routing of the last layer came from the K1-K3 path
    const int32_t *last_ids = nullptr;   // where the last layer call left its routing
    const float *last_weights = nullptr;

    // prefill workspace (grown on demand)
    float *pf_logits = nullptr;    size_t pf_logits_cap = 0;
    int32_t *pf_ids = nullptr;     size_t pf_ids_cap = 0;
    float *pf_w = nullptr;         size_t pf_w_cap = 0;
    int32_t *pf_pairpos = nullptr; size_t pf_pairpos_cap = 0;
    int32_t *pf_pairtok = nullptr; size_t pf_pairtok_cap = 0;
    int32_t *pf_tiles = nullptr;   size_t pf_tiles_cap = 0;
    int32_t *pf_ntiles = nullptr;  size_t pf_ntiles_cap = 0;
    uint16_t *pf_act = nullptr;    size_t pf_act_cap = 0;   // hi plane then lo plane
    float *pf_outp = nullptr;      size_t pf_outp_cap = 0;
    float *pf_xsum = nullptr;      size_t pf_xsum_cap = 0;
    uint16_t *pf_rsplit = nullptr; size_t pf_rsplit_cap = 0;   // bf16 router GEMM operands
    float *pf_ys = nullptr;        size_t pf_ys_cap = 0;       // shared-expert pass output (own types)
    int pf_T = 0, pf_k = 0;

    // pinned staging for host->device uploads of expert stores
    uint8_t *pin[2] = {nullptr, nullptr};
    hipEvent_t pin_ev[2] = {nullptr, nullptr};

    // values given to gpu_set_{ram,vram}_cache_mb (recorded; no cache tiers here)
    int ram_cache_mb = -1, vram_cache_mb = -1;

    // captured stack-decode graph and the bytes it was captured from
    // (descriptors, x, scratch pointers)
    hipGraphExec_t graph_exec = nullptr;
    std::vector<uint8_t> graph_key;
};

inline int fail(gpu_ctx *c, int code, const char *fmt, ...) {
    if (c) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        c->err = buf;
    }
    return code;
}

#define HIPC(call)                                                                         \
    do {                                                                                   \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess)                                                              \
            return fail(ctx, e_ == hipErrorInvalidValue ? -1 : -2, "%s: %s (%s:%d)", #call, \
                        hipGetErrorString(e_), __FILE__, __LINE__);                        \
    } while (0)

// Grow a device scratch buffer to at least `need` bytes (never inside a
// captured region: callers size everything first).
template <typename Tp>
inline hipError_t ensure(Tp *&p, size_t &cap, size_t need) {
    if (cap >= need) return hipSuccess;
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
    hipError_t e = hipMalloc((void **)&p, need);
    if (e == hipSuccess) cap = need;
    return e;
}

inline bool kquant(int t) { return t == GGML_TYPE_Q4_K || t == GGML_TYPE_Q5_K || t == GGML_TYPE_Q6_K; }
inline bool layer_type(int t) { return kquant(t) || t == GGML_TYPE_Q8_0; }
inline bool matvec_type(int t) { return layer_type(t) || t == GGML_TYPE_MXFP4; }

// Copy `bytes` bytes of an open file, from file_off, to the device through the
// context's two pinned 32 MiB chunks (the read of one overlaps the copy of the
// other), scattering them as segments of `seg` bytes at dst + i * dst_pitch
// (seg = bytes, pitch 0 for a plain copy). Synchronous: the stream is drained
// before returning on every path. 0 / -1 (short read) / -2 (device error).
int file_to_device(gpu_ctx *ctx, int fd, uint64_t file_off, uint64_t bytes, uint8_t *dst, uint64_t seg,
                   uint64_t dst_pitch, const char *what);
