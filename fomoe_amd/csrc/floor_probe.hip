// floor_probe.hip — load-only twins of the decode layer's three kernels, for
// measuring the floor the layer's structure sets (a diagnostic library,
// libfomoe_probe_gfx950.so; the product library does not contain it).
//
// Each probe issues its kernel's memory requests — the same grid, work-group
// shape, LDS staging, load widths, addresses and non-temporal hints, in the
// same order — and replaces the arithmetic by an xor of the loaded words (so
// that no load is dead), with one small store per work-group where the real
// kernel stores its results:
//   k_probe_route    k_route<8>: x (and norm_w) first, then the router rows,
//                    1 KiB spans per instruction; logits written.
//   k_probe_expand   k_expand_q4t: the prepared h staged into LDS by direct
//                    global->LDS loads while wave 0 reads the logits (no
//                    selection arithmetic: the expert ids are read from a
//                    table after the logits), then nine 1 KiB pieces of the
//                    16 gate rows and nine of the 16 up rows per wave, passed
//                    through the wave's LDS area; the prepared activation
//                    bytes of the block written.
//   k_probe_reduce   k_reduce_tile<Q6_K>: per wave (one per expert) the ids,
//                    the activation slot, then fourteen 1 KiB pieces of the
//                    expert's 16 down rows through the wave's LDS area; the
//                    16 outputs written in rank order.
// Shape: the layer of config 3 (Q4_K gate/up at H = 4096, Q6_K down at
// F = 1024, a shared expert in the routed types, k + 1 <= 12).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"
#include "gpu.h"
#include "topk.h"

namespace fo {
namespace {

constexpr int kH = 4096, kF = 1024, kTR = 16;
constexpr int kQ4Row = 2304, kQ6Row = 840;

__global__ void k_probe_empty(uint32_t *sink) {
    if (threadIdx.x == 0 && blockIdx.x == 0 && sink == nullptr) sink[0] = 0;   // never taken
}

struct PRoute {
    const float *router, *x, *norm_w;
    int E;
    float *logits;
    uint8_t *xq_h;
};

// k_route<8>'s requests: 256 threads, two router rows per work-group (a
// half-row per wave), 8 float2 of x and of norm_w per thread, 8 x 16 B of
// router per lane.
__global__ __launch_bounds__(256) void k_probe_route(PRoute a) {
    constexpr int UH = 8;
    __shared__ uint32_t part[4];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int row = 2 * blockIdx.x + (wv >> 1), half = wv & 1;
    uint32_t acc = 0;
    float2 xv[UH], nv[UH];
#pragma unroll
    for (int u = 0; u < UH; u++) xv[u] = ((const float2 *)a.x)[tid + 256 * u];
    if (a.norm_w) {
#pragma unroll
        for (int u = 0; u < UH; u++) nv[u] = ((const float2 *)a.norm_w)[tid + 256 * u];
    }
    uint4 wr[UH];
    const float4 *rp = (const float4 *)(a.router + (uint64_t)min(row, a.E - 1) * kH) + half * (kH / 8);
#pragma unroll
    for (int u = 0; u < UH; u++) wr[u] = ldw16((const uint8_t *)(rp + lane + 64 * u));
#pragma unroll
    for (int u = 0; u < UH; u++) {
        acc ^= __float_as_uint(xv[u].x) ^ __float_as_uint(xv[u].y);
        if (a.norm_w) acc ^= __float_as_uint(nv[u].x) ^ __float_as_uint(nv[u].y);
    }
    // this work-group's share of the prepared h: 12 KiB of limbs + 1 KiB of
    // scales over the grid
    const uint32_t xqb = (uint32_t)xq_bytes(kH, 32), per = (xqb / 16 + gridDim.x - 1) / gridDim.x;
    if ((uint32_t)tid < per && blockIdx.x * per + tid < xqb / 16)
        ((uint4 *)a.xq_h)[blockIdx.x * per + tid] = make_uint4(acc, acc, acc, acc);
#pragma unroll
    for (int u = 0; u < UH; u++) acc ^= wr[u].x ^ wr[u].y ^ wr[u].z ^ wr[u].w;
    for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, 64);
    if (lane == 0) part[wv] = acc;
    __syncthreads();
    if (tid < 2 && 2 * blockIdx.x + tid < a.E)
        a.logits[2 * blockIdx.x + tid] = __uint_as_float((part[2 * tid] ^ part[2 * tid + 1]) & 0x3FFFFFFFu);
}

struct PExpand {
    const float *logits;
    int E, k;
    const int32_t *ids;
    const uint8_t *base, *shared;
    uint64_t stride, gate_size, sh_gate_size;
    const uint8_t *xq_h;
    uint8_t *xq_act;
    uint64_t xq_vstride;
};

__global__ __launch_bounds__(256, 3) void k_probe_expand(PExpand a) {
    constexpr int SPAN = 16 * 576, NP = SPAN / 1024, NW = 4;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    __shared__ int s_ids[kMaxK];
    __shared__ uint32_t s_part[NW];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int tpe = kF / kTR;
    const int e = blockIdx.x / tpe, rb = blockIdx.x - e * tpe;
    const bool routed = e < a.k;
    const uint32_t xqb = (uint32_t)xq_bytes(kH, 32);
    stage_lds(lds, a.xq_h, xqb, wv, NW);
    if (wv == 0 && routed) {   // the selection's reads: every logit once, then the ids
        float m = -3.0e38f;
        for (int i = lane; i < a.E; i += 64) m = fmaxf(m, a.logits[i]);
        m = wave_max(m);
        if (lane <= e) s_ids[lane] = a.ids[lane] + (m == 1.0e30f ? 1 : 0);
    }
    stage_lds_wait();
    const uint8_t *blob;
    uint64_t uo;
    if (routed) { blob = a.base + (uint64_t)s_ids[e] * a.stride; uo = a.gate_size; }
    else { blob = a.shared; uo = a.sh_gate_size; }
    const uint8_t *g0 = blob + (uint64_t)(rb * kTR) * kQ4Row + wv * 576, *u0 = g0 + uo;
    uint4 vg[NP], vu[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const uint32_t o = i * 1024 + lane * 16, go = (o / 576) * kQ4Row + o % 576;
        vg[i] = ldw16(g0 + go);
        vu[i] = ldw16(u0 + go);
    }
    __builtin_amdgcn_sched_barrier(0);
    uint8_t *buf = lds + lds_round(xqb) + 512 + wv * SPAN;
    uint32_t acc = *(const uint32_t *)(lds + 16 * lane);
    auto chunk = [&](uint4 (&p)[NP]) {
#pragma unroll
        for (int i = 0; i < NP; i++) *(uint4 *)(buf + i * 1024 + lane * 16) = p[i];
        const uint4 t = *(const uint4 *)(buf + ((lane * 144) % SPAN));
        acc ^= t.x ^ t.y ^ t.z ^ t.w;
    };
    chunk(vg);
    chunk(vu);
    for (int o = 32; o > 0; o >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, o, 64);
    if (lane == 0) s_part[wv] = acc;
    __syncthreads();
    if (wv == 0) {   // the block's prepared activation: 16 x 3 limb bytes + one {scale, sum}
        const uint32_t v = s_part[0] ^ s_part[1] ^ s_part[2] ^ s_part[3];
        uint8_t *dst = a.xq_act + (uint64_t)e * a.xq_vstride;
        if (lane < 12) ((uint32_t *)(dst + (uint64_t)rb * 48))[lane] = v;
        if (lane == 12) *(float2 *)(dst + xq_limb_bytes(kF) + (uint64_t)rb * 8) = make_float2(__uint_as_float(v & 0x3FFFFFFFu), 0.f);
    }
}

struct PReduce {
    const int32_t *ids;
    const float *weights;
    int k;
    const uint8_t *base, *shared;
    uint64_t stride, down_off, sh_down_off;
    const uint8_t *xq_act;
    uint64_t xq_vstride;
    float *out;
};

__global__ __launch_bounds__(64 * 12) void k_probe_reduce(PReduce a) {
    constexpr uint32_t TB = kTR * kQ6Row, TSTRIDE = (TB + 15) & ~15u;
    constexpr int NV = (TB + 1023) / 1024;
    extern __shared__ __attribute__((aligned(16))) uint8_t tiles[];
    __shared__ uint32_t part[kMaxK + 1][kTR];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int n_tot = a.k + 1, row0 = blockIdx.x * kTR;
    const uint8_t *m = (wv < a.k) ? a.base + (uint64_t)a.ids[wv] * a.stride + a.down_off : a.shared + a.sh_down_off;
    // the lane's activation slot: its 16-value groups' limbs and {scale, sum}
    const uint8_t *xs = a.xq_act + (uint64_t)wv * a.xq_vstride;
    const int slot = lane & 15;
    uint32_t acc = 0;
#pragma unroll
    for (int L = 0; L < 3; L++) {
        const uint4 t = ld16(xs + (uint64_t)L * kF + 64 * slot);
        acc ^= t.x ^ t.y ^ t.z ^ t.w;
    }
    const uint2 ss = *(const uint2 *)(xs + xq_limb_bytes(kF) + 32 * slot);
    acc ^= ss.x ^ ss.y;
    const uint8_t *src = m + (uint64_t)row0 * kQ6Row;
    uint4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] = ldw16(src + min(i * 1024u + lane * 16u, TB - 16));
    __builtin_amdgcn_sched_barrier(0);
    uint8_t *dst = tiles + wv * TSTRIDE;
#pragma unroll
    for (int i = 0; i < NV; i++) *(uint4 *)(dst + min(i * 1024u + lane * 16u, TB - 16)) = v[i];
    const uint4 t = *(const uint4 *)(dst + (lane & 15) * kQ6Row + 16 * (lane >> 4));
    acc ^= t.x ^ t.y ^ t.z ^ t.w;
    acc ^= (uint32_t)__shfl_xor((int)acc, 16, 64);
    acc ^= (uint32_t)__shfl_xor((int)acc, 32, 64);
    if (lane < kTR && wv < n_tot) part[wv][lane] = acc;
    __syncthreads();
    if (tid < kTR) {
        float s = 0.f;
        for (int e = 0; e < n_tot; e++) s = fmaf(e < a.k ? a.weights[e] : 1.f, __uint_as_float(part[e][tid] & 0x3FFFFFFFu), s);
        a.out[row0 + tid] = s;
    }
}

}  // namespace
}  // namespace fo

using namespace fo;

// Times the probes over a rotation of n_layers config-3 layers (layer l
// with routing d_ids[l*k .. l*k+k)), each probe `iters` rotations after one
// warm-up rotation, launches back to back on one stream. us[0..4]: an empty
// kernel, k_probe_route, k_probe_expand, k_probe_reduce (µs per launch), and
// the three probes in sequence (µs per layer). 0 on success, -1 on a layer
// of another shape, a HIP error code otherwise.
extern "C" int fo_probe_layer_floors(const gpu_moe_layer_t *L, int n_layers, const int32_t *d_ids, int iters,
                                     float *us) {
    if (!L || n_layers <= 0 || !d_ids || iters <= 0 || !us) return -1;
    const int E = L[0].n_experts, k = L[0].k;
    for (int l = 0; l < n_layers; l++) {
        const gpu_moe_layer_t &d = L[l];
        if (d.n_embd != kH || d.inter != kF || d.n_experts != E || d.k != k || k + 1 > 12 || !d.shared ||
            d.gate_type != GGML_TYPE_Q4_K || d.up_type != GGML_TYPE_Q4_K || d.down_type != GGML_TYPE_Q6_K ||
            d.shared_inter != kF || d.shared_gate_type != GGML_TYPE_Q4_K || d.shared_down_type != GGML_TYPE_Q6_K ||
            E % 2 || E > kMaxE)
            return -1;
    }
    const uint64_t vstride = xq_stride(kF, 16);
    float *x = nullptr, *logits = nullptr, *w = nullptr, *out = nullptr;
    uint8_t *xq_h = nullptr, *xq_act = nullptr;
    hipStream_t s = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t err = hipSuccess;
#define PC(call) do { err = (call); if (err != hipSuccess) goto done; } while (0)
    PC(hipMalloc(&x, 2 * sizeof(float) * kH));
    PC(hipMalloc(&logits, sizeof(float) * E));
    PC(hipMalloc(&w, sizeof(float) * kMaxK));
    PC(hipMalloc(&out, sizeof(float) * kH));
    PC(hipMalloc(&xq_h, xq_stride(kH, 32) + 1024));
    PC(hipMalloc(&xq_act, vstride * (k + 1)));
    PC(hipMemset(x, 0, 2 * sizeof(float) * kH));
    PC(hipMemset(w, 0, sizeof(float) * kMaxK));
    PC(hipMemset(xq_h, 0, xq_stride(kH, 32) + 1024));
    PC(hipStreamCreate(&s));
    PC(hipEventCreate(&e0));
    PC(hipEventCreate(&e1));
    {
        const uint32_t lds_e = lds_round(xq_bytes(kH, 32)) + 512 + 4 * 16 * 576;
        const uint32_t lds_r = (k + 1) * ((kTR * kQ6Row + 15) & ~15u);
        PC(hipFuncSetAttribute((const void *)k_probe_reduce, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_r));
        PC(hipFuncSetAttribute((const void *)k_probe_expand, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_e));
        auto launch = [&](int which, int l) {
            const gpu_moe_layer_t &d = L[l];
            if (which == 0) {
                k_probe_empty<<<1, 64, 0, s>>>(nullptr);
            } else if (which == 1) {
                PRoute a{d.router, x, x + kH, E, logits, xq_h};
                k_probe_route<<<E / 2, 256, 0, s>>>(a);
            } else if (which == 2) {
                PExpand a{logits, E, k, d_ids + (size_t)l * k, (const uint8_t *)d.experts, (const uint8_t *)d.shared,
                          d.expert_stride, d.gate_size, d.shared_gate_size, xq_h, xq_act, vstride};
                k_probe_expand<<<kF / kTR * (k + 1), 256, lds_e, s>>>(a);
            } else {
                PReduce a{d_ids + (size_t)l * k, w, k, (const uint8_t *)d.experts, (const uint8_t *)d.shared,
                          d.expert_stride, d.gate_size + d.up_size, d.shared_gate_size + d.shared_up_size,
                          xq_act, vstride, out};
                k_probe_reduce<<<kH / kTR, 64 * (k + 1), lds_r, s>>>(a);
            }
        };
        for (int which = 0; which < 5; which++) {
            for (int rep = 0; rep <= iters; rep++) {
                if (rep == 1) PC(hipEventRecord(e0, s));
                for (int l = 0; l < n_layers; l++) {
                    if (which < 4) launch(which, l);
                    else { launch(1, l); launch(2, l); launch(3, l); }
                }
            }
            PC(hipGetLastError());
            PC(hipEventRecord(e1, s));
            PC(hipEventSynchronize(e1));
            float ms = 0.f;
            PC(hipEventElapsedTime(&ms, e0, e1));
            us[which] = ms * 1e3f / (float)(iters * n_layers);
        }
    }
done:
#undef PC
    if (s) (void)hipStreamSynchronize(s);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    if (s) (void)hipStreamDestroy(s);
    (void)hipFree(x); (void)hipFree(logits); (void)hipFree(w);
    (void)hipFree(out); (void)hipFree(xq_h); (void)hipFree(xq_act);
    return err == hipSuccess ? 0 : (int)err;
}
