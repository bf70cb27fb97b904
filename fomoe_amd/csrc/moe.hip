// moe.hip — the batch-1 MoE layer as three kernels with no device-scope
// atomics (on MI355X an agent-scope atomic serialises at ~10 ns, so a 256-WG
// "last block" handshake costs more than a kernel boundary in a graph):
//
//   K1 k_route   router logits = W_r . rms_norm(x) (+ bias); the prepared
//                (block-fixed-point) activation of h for the experts; the
//                shared-expert gate sigmoid(h . v).
//   K2 k_expand  every work-group recomputes top-k + renormalisation from the
//                logits (a few hundred VALU instructions, cheaper than any
//                grid-wide handshake), then streams gate/up rows of the routed
//                experts and the shared expert; each task covers one activation
//                group of rows, so the WG writes silu(g)*u straight into the
//                prepared form the down projection consumes.
//   K3 k_reduce  down projection of all selected experts for a block of output
//                rows with every expert's prepared activation staged in LDS once
//                per WG; the weighted combine and the residual are summed in
//                registers in a fixed order (deterministic).
//
// Semantics follow reference src/inference.c:481-606 (router, softmax, top-k,
// renormalise, SwiGLU experts, scaled add in rank order, shared expert with
// optional sigmoid gate, residual); the reference GPU kernels replaced are
// gpu_kernels.hip kernel_f32_matvec_coop 2127, kernel_softmax 2668,
// kernel_top_k_parallel 2745, kernel_q4k_fused_gate_up_silu 1320,
// kernel_q4k_fused_gus_mw 1474, kernel_q6k_matvec_per_expert 1261,
// kernel_moe_output_residual 1647 and kernel_dot_sigmoid_scale 3648.
#include <float.h>

#include "formats.h"
#include "moe.h"
#include "q4k_mfma.h"
#include "shared.h"
#include "topk.h"

namespace fo {

// ------------------------------------------------------------ wave primitives
FO_DEV float wave_sum_dpp(float v) { return group_sum<kWave>(v); }

// Prepare one group of G values held one per lane in lanes [0, G) of a wave
// (G = 16 or 32): exponent from the group maximum, three balanced int8 limbs
// per value packed four values per dword, {2^-e, group sum} (group_scale_sum). Layout as in
// formats.h. `dst` points at the vector's limb area, `ss` at its {scale,sum}
// area, g is the group index.
template <int G>
FO_DEV void prep_group_lanes(float val, int g, uint8_t *__restrict__ dst, uint8_t *__restrict__ ss) {
    const int lane = threadIdx.x & 63;
    float a = fabsf(val), chk = val * 0.f;
#pragma unroll
    for (int o = 1; o < G; o <<= 1) {
        a = fmaxf(a, __shfl_xor(a, o, 64));
        chk += __shfl_xor(chk, o, 64);
    }
    int E = 0;
    frexpf(a, &E);
    int e = kFixBits - E;
    if (e > 149) e = 149;
    int X = (a > 0.f && chk == 0.f) ? __float2int_rn(ldexpf(val, e)) : 0;
    int isum = X;
#pragma unroll
    for (int o = 1; o < G; o <<= 1) isum += __shfl_xor(isum, o, 64);
    float scale, sum;
    group_scale_sum(a, chk, e, isum, scale, sum);
    uint32_t limb[kLimbs];
#pragma unroll
    for (int L = 0; L < kLimbs - 1; L++) {
        const int b = (int)(int8_t)(X & 0xFF);
        X = (X - b) >> 8;
        limb[L] = (uint32_t)(b & 0xFF);
    }
    limb[kLimbs - 1] = (uint32_t)(X & 0xFF);
    // gather bytes of lanes 4q..4q+3 into lane 4q
#pragma unroll
    for (int L = 0; L < kLimbs; L++) {
        const uint32_t b1 = (uint32_t)__shfl_down((int)limb[L], 1, 64);
        const uint32_t b2 = (uint32_t)__shfl_down((int)limb[L], 2, 64);
        const uint32_t b3 = (uint32_t)__shfl_down((int)limb[L], 3, 64);
        limb[L] = limb[L] | (b1 << 8) | (b2 << 16) | (b3 << 24);
    }
    if (lane < G && (lane & 3) == 0) {
        uint32_t *p = (uint32_t *)(dst + (uint64_t)g * (kLimbs * G));
#pragma unroll
        for (int L = 0; L < kLimbs; L++) p[L * (G / 4) + (lane >> 2)] = limb[L];
    }
    if (lane == 0) *(float2 *)(ss + (uint64_t)g * 8) = make_float2(scale, sum);
}

// ============================================================ K1: route
// WG of 256 threads = 4 waves; WG b handles router rows 2b, 2b+1, each split
// over two waves (half of H each). Every thread first requests its 2*UH
// values of x and norm_w, then its UH float4 of router weights; the norm
// waits only for the first requests (loads retire in issue order), so the
// norm, the activation prep and the shared gate run while the weights are
// in flight.
template <int UH>  // H = 512*UH; a lane holds UH float4 of one half-row
__global__ __launch_bounds__(256) void k_route(RouteArgs a) {
    extern __shared__ float sh[];             // h [H]
    __shared__ float part[4];
    __shared__ float red[4];
    const int H = a.H, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int row = 2 * blockIdx.x + (wv >> 1), half = wv & 1;
    float2 xv[UH], nv[UH];
#pragma unroll
    for (int u = 0; u < UH; u++) xv[u] = ((const float2 *)a.x)[tid + 256 * u];
    if (a.norm_w) {
#pragma unroll
        for (int u = 0; u < UH; u++) nv[u] = ((const float2 *)a.norm_w)[tid + 256 * u];
    }
    float4 wr[UH];
    const bool has_row = row < a.E;
    const float4 *rp = (const float4 *)(a.router + (uint64_t)min(row, a.E - 1) * H) + half * (H / 8);
#pragma unroll
    for (int u = 0; u < UH; u++) {   // whole 1 KiB spans per instruction: non-temporal
        const uint4 t = ldw16((const uint8_t *)(rp + lane + 64 * u));
        wr[u] = make_float4(__uint_as_float(t.x), __uint_as_float(t.y), __uint_as_float(t.z), __uint_as_float(t.w));
    }
    if (a.norm_w) {
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < UH; u++) ss += xv[u].x * xv[u].x + xv[u].y * xv[u].y;
        ss = wave_sum_dpp(ss);
        if (lane == 0) red[wv] = ss;
        __syncthreads();
        const float tot = (red[0] + red[1]) + (red[2] + red[3]);
        const float scale = 1.0f / sqrtf(tot / (float)H + a.eps);
#pragma unroll
        for (int u = 0; u < UH; u++)
            *(float2 *)(sh + 2 * tid + 512 * u) = make_float2(xv[u].x * scale * nv[u].x, xv[u].y * scale * nv[u].y);
    } else {
#pragma unroll
        for (int u = 0; u < UH; u++) *(float2 *)(sh + 2 * tid + 512 * u) = xv[u];
    }
    __syncthreads();
    // this WG's share of the prepared h (groups of a.gsz values, one wave each)
    if (a.xq_h) {
        const int ng = H / a.gsz;
        const int per = (ng + gridDim.x - 1) / gridDim.x;
        for (int j = wv; j < per; j += 4) {
            const int g = blockIdx.x * per + j;
            if (g >= ng) break;
            const float val = lane < a.gsz ? sh[g * a.gsz + lane] : 0.f;
            if (a.gsz == 16) prep_group_lanes<16>(val, g, a.xq_h, a.xq_h + xq_limb_bytes(H));
            else prep_group_lanes<32>(val, g, a.xq_h, a.xq_h + xq_limb_bytes(H));
        }
    }
    // shared-expert gate
    if (blockIdx.x == 0 && wv == 0 && a.shared_w) {
        float g = 1.0f;
        if (a.shared_gate_vec) {
            float d = 0.f;
            for (int i = lane; i < H; i += 64) d += sh[i] * a.shared_gate_vec[i];
            d = wave_sum_dpp(d);
            g = 1.0f / (1.0f + expf(-d));
        }
        if (lane == 0) *a.shared_w = g;
    }
    float acc = 0.f;
    if (has_row) {
        const float *hp = sh + half * (H / 2);
#pragma unroll
        for (int u = 0; u < UH; u++) {
            const float4 hv = *(const float4 *)(hp + 4 * (lane + 64 * u));
            acc = fmaf(wr[u].x, hv.x, acc);
            acc = fmaf(wr[u].y, hv.y, acc);
            acc = fmaf(wr[u].z, hv.z, acc);
            acc = fmaf(wr[u].w, hv.w, acc);
        }
        acc = wave_sum_dpp(acc);
    }
    if (lane == 0) part[wv] = acc;
    __syncthreads();
    if (tid < 2) {
        const int r = 2 * blockIdx.x + tid;
        if (r < a.E) a.logits[r] = (part[2 * tid] + part[2 * tid + 1]) + (a.bias ? a.bias[r] : 0.f);
    }
}

hipError_t launch_route(const RouteArgs &a, hipStream_t s) {
    if (a.E <= 0 || a.E > kMaxE || a.H % 512 || a.H > 8192) return hipErrorInvalidValue;
    const int blocks = (a.E + 1) / 2;
    const size_t lds = (size_t)a.H * 4;
#define FO_K1(U) if (a.H == 512 * U) { k_route<U><<<blocks, 256, lds, s>>>(a); return hipGetLastError(); }
    FO_K1(1) FO_K1(2) FO_K1(3) FO_K1(4) FO_K1(6) FO_K1(8) FO_K1(12) FO_K1(16)
#undef FO_K1
    return hipErrorInvalidValue;
}

// ============================================================ K2: expand
// One work-group of TR/RW waves per task (expert slot e, block of TR rows, TR
// = the activation-group size of the down projection; RW rows per wave); the
// grid is all tasks at once (k=10 + shared, F=1024, TR=16: 704 WGs of 4
// waves, all resident), and every wave issues all its weight loads before any
// arithmetic, so the layer's whole gate/up traffic is in flight together. Routed WGs first compute top-k (wave
// 0) while the other waves stage the prepared h in LDS; the shared expert's
// WGs skip the top-k. The TR results meet in LDS and wave 0 writes them in
// prepared form for K3 (and as fp32 when a.act is set).
// Rows per wave: 4 when a row's raw block is small (Q4_K, Q8_0), else 2, so
// the weight registers of all rows stay resident without scratch.
template <int T, int TR, int U>
struct ExpandShape {
    static constexpr int RW = (U == 1 && sizeof(typename Fmt<T>::Raw) <= 48) ? 4 : 2;
    static constexpr int THREADS = TR / RW * 64;
};

template <int T, int TR, int G, int U>
__global__ __launch_bounds__((ExpandShape<T, TR, U>::THREADS), 3) void k_expand(ExpandArgs a) {
    using F = Fmt<T>;
    constexpr int RW = ExpandShape<T, TR, U>::RW;       // rows per wave
    constexpr int NW = TR / RW;                         // waves
    constexpr int P = kWave / G;                        // rows side by side per pass
    constexpr int PASS = (RW + P - 1) / P;              // passes per wave
    extern __shared__ uint8_t lds[];                    // prepared h
    __shared__ int s_ids[kMaxK];
    __shared__ float s_w[kMaxK], s_val[kMaxK];
    __shared__ float2 s_cand[64];
    __shared__ float s_act[TR];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, sub = lane / G;
    const int H = a.H, F_ = a.F;
    const int tpe = F_ / TR;
    const int e = blockIdx.x / tpe, rb = blockIdx.x - e * tpe;
    const bool routed = e < a.k;
    const uint64_t xqb = xq_bytes(H, F::GSZ);
    // the prepared h streams into LDS while wave 0 selects experts
    stage_lds(lds, a.xq_h, (uint32_t)xqb, wv, NW);
    // A routed WG of rank e needs only the first e+1 selections; the full
    // top-k with weights (for K3) is computed once, by the first WG that has
    // nothing else to wait for (the shared expert's first task, or WG 0).
    const bool full = a.shared ? (e == a.k && rb == 0) : blockIdx.x == 0;
    const int rounds = full ? a.k : (routed ? e + 1 : 0);
    if (wv == 0 && rounds > 0) {
        // one or two selections: arg-max rounds; more: the threshold ranking
        if (rounds <= 2) {
            if (a.E <= 512) wave_topk<8>(a.logits, a.E, rounds, s_ids, full ? s_w : nullptr);
            else wave_topk<16>(a.logits, a.E, rounds, s_ids, full ? s_w : nullptr);
        } else {
            if (a.E <= 512) wave_topk_thr<8>(a.logits, a.E, rounds, s_ids, full ? s_w : nullptr, s_cand, s_val);
            else wave_topk_thr<16>(a.logits, a.E, rounds, s_ids, full ? s_w : nullptr, s_cand, s_val);
        }
        if (full && lane < a.k) { a.ids[lane] = s_ids[lane]; a.weights[lane] = s_w[lane]; }
    }
    stage_lds_wait();
    const uint8_t *blob;
    uint64_t uo;
    if (routed) { blob = a.base + (uint64_t)s_ids[e] * a.stride; uo = a.gate_size; }
    else { blob = a.shared; uo = a.sh_gate_size; }
    // slots past S mirror the last slot (valid addresses) and contribute 0
    const int S = H / F::SLOT;
    int slot[U];
    float live[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int sl = (lane % G) + G * u;
        slot[u] = min(sl, S - 1);
        live[u] = sl < S ? 1.f : 0.f;
    }
    typename F::Raw rg[PASS][U], ru[PASS][U];
#pragma unroll
    for (int p = 0; p < PASS; p++) {
        const int rl = wv * RW + p * P + sub;
        const int row = rb * TR + min(rl, TR - 1);
#pragma unroll
        for (int u = 0; u < U; u++) {
            rg[p][u] = F::load(blob + (uint64_t)row * a.row_bytes, slot[u]);
            ru[p][u] = F::load(blob + uo + (uint64_t)row * a.row_bytes, slot[u]);
        }
    }
    typename F::X X[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        int gi[F::NG];
        F::groups(slot[u], gi);
        load_xslot(X[u], lds, H, gi);
    }
#pragma unroll
    for (int p = 0; p < PASS; p++) {
        float g = 0.f, v = 0.f;
#pragma unroll
        for (int u = 0; u < U; u++) {
            g = fmaf(live[u], F::dot(rg[p][u], slot[u], X[u]), g);
            v = fmaf(live[u], F::dot(ru[p][u], slot[u], X[u]), v);
        }
        g = group_sum<G>(g);
        v = group_sum<G>(v);
        const int rl = wv * RW + p * P + sub;
        if ((lane % G) == 0 && p * P + sub < RW) s_act[rl] = (g / (1.0f + expf(-g))) * v;
    }
    __syncthreads();
    if (wv == 0) {
        const float val = lane < TR ? s_act[lane] : 0.f;
        uint8_t *dst = a.xq_act + (uint64_t)e * a.xq_vstride;
        prep_group_lanes<TR>(val, rb, dst, dst + xq_limb_bytes(F_));
        if (a.act && lane < TR) a.act[(uint64_t)e * F_ + rb * TR + lane] = val;
    }
}

// K2 for Q4_K gate/up at H = 4096 (TR = 16) on the integer MFMA of the Q4_K
// matvec (q4k_mfma.h): wave w takes K-chunk w (4 super-blocks, 576 bytes per
// row) of the work-group's 16 gate rows and 16 up rows, two 9 KiB pieces of
// the 2304-byte rows streamed with non-temporal 1 KiB loads and passed
// through a 9 KiB wave-private LDS area (gate first, then up); the four
// waves' partial row sums meet in LDS for the SwiGLU.
__global__ __launch_bounds__(256, 3) void k_expand_q4t(ExpandArgs a) {
    constexpr int T = GGML_TYPE_Q4_K, TR = 16;
    constexpr int RB = 2304, SPAN = 16 * 576, NP = SPAN / 1024;
    using F = Fmt<T>;
    constexpr int NW = 4;                               // waves: one K-chunk each
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];   // prepared h, then NW row spans
    __shared__ int s_ids[kMaxK];
    __shared__ float s_w[kMaxK], s_val[kMaxK];
    __shared__ float2 s_cand[64];
    __shared__ float s_act[TR];
    __shared__ double s_part[2][4][TR];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int H = a.H, F_ = a.F;
    const int tpe = F_ / TR;
    const int e = blockIdx.x / tpe, rb = blockIdx.x - e * tpe;
    const bool routed = e < a.k;
    const uint64_t xqb = xq_bytes(H, F::GSZ);
    // the prepared h streams into LDS while wave 0 selects experts
    stage_lds(lds, a.xq_h, (uint32_t)xqb, wv, NW);
    // A routed WG of rank e needs only the first e+1 selections; the full
    // top-k with weights (for K3) is computed once, by the first WG that has
    // nothing else to wait for (the shared expert's first task, or WG 0).
    const bool full = a.shared ? (e == a.k && rb == 0) : blockIdx.x == 0;
    const int rounds = full ? a.k : (routed ? e + 1 : 0);
    if (wv == 0 && rounds > 0) {
        // one or two selections: arg-max rounds; more: the threshold ranking
        if (rounds <= 2) {
            if (a.E <= 512) wave_topk<8>(a.logits, a.E, rounds, s_ids, full ? s_w : nullptr);
            else wave_topk<16>(a.logits, a.E, rounds, s_ids, full ? s_w : nullptr);
        } else {
            if (a.E <= 512) wave_topk_thr<8>(a.logits, a.E, rounds, s_ids, full ? s_w : nullptr, s_cand, s_val);
            else wave_topk_thr<16>(a.logits, a.E, rounds, s_ids, full ? s_w : nullptr, s_cand, s_val);
        }
        if (full && lane < a.k) { a.ids[lane] = s_ids[lane]; a.weights[lane] = s_w[lane]; }
    }
    stage_lds_wait();
    const uint8_t *blob;
    uint64_t uo;
    if (routed) { blob = a.base + (uint64_t)s_ids[e] * a.stride; uo = a.gate_size; }
    else { blob = a.shared; uo = a.sh_gate_size; }
    // piece i of chunk wv, lane l: chunk byte o = 1024 i + 16 l of row o / 576
    const uint8_t *g0 = blob + (uint64_t)(rb * TR) * RB + wv * 576, *u0 = g0 + uo;
    uint4 vg[NP], vu[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const uint32_t o = i * 1024 + lane * 16, go = (o / 576) * RB + o % 576;
        vg[i] = ldw16(g0 + go);
        vu[i] = ldw16(u0 + go);
    }
    // keep the scheduler from sinking the up loads below the gate arithmetic
    __builtin_amdgcn_sched_barrier(0);
    uint8_t *zero = lds + lds_round(xqb), *buf = zero + 512 + wv * SPAN;
    if (wv == 0 && lane < 32) *(uint4 *)(zero + 16 * lane) = make_uint4(0, 0, 0, 0);
    const Q4kLane q = q4k_lane(lane);
    const int n = lane & 15, g = lane >> 4;
    const uint8_t *ssl = lds + 3 * 4096 + q.jg * 8;
    __syncthreads();                                   // the zero area
    // the row sums accumulate in fp64 (fp64 fma issues at the fp32 rate here):
    // the layer's parity margin at near-zero outputs is a few per cent
    auto chunk = [&](uint4 (&p)[NP]) {
#pragma unroll
        for (int i = 0; i < NP; i++) *(uint4 *)(buf + i * 1024 + lane * 16) = p[i];
        double y = 0.0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int sb = 4 * wv + b;                 // super-block of the row: groups 8 sb ..
            const uint8_t *xa = lds + sb * 768 + q.aoff;
            y = q4k_sb_dot_mfma(buf + n * 576 + b * 144, q.valid1 ? xa : zero, q.valid2 ? xa : zero,
                                ssl + sb * 64, q, y);
        }
        y += __shfl_xor(y, 16);
        y += __shfl_xor(y, 32);
        return y;
    };
    const double yg = chunk(vg);
    const double yu = chunk(vu);
    if (g == 0) { s_part[0][wv][n] = yg; s_part[1][wv][n] = yu; }
    __syncthreads();
    if (wv == 0 && lane < TR) {
        const float gs = (float)((s_part[0][0][lane] + s_part[0][1][lane]) + (s_part[0][2][lane] + s_part[0][3][lane]));
        const float us = (float)((s_part[1][0][lane] + s_part[1][1][lane]) + (s_part[1][2][lane] + s_part[1][3][lane]));
        s_act[lane] = (gs / (1.0f + expf(-gs))) * us;
    }
    __syncthreads();
    if (wv == 0) {
        const float val = lane < TR ? s_act[lane] : 0.f;
        if (!a.act_only) {   // else the down kernel prepares its groups from act
            uint8_t *dst = a.xq_act + (uint64_t)e * a.xq_vstride;
            prep_group_lanes<TR>(val, rb, dst, dst + xq_limb_bytes(F_));
        }
        if (a.act && lane < TR) a.act[(uint64_t)e * F_ + rb * TR + lane] = val;
    }
}

hipError_t launch_expand(int type, const ExpandArgs &a, hipStream_t s, int n_cu) {
    (void)n_cu;
    const int slot = type == GGML_TYPE_Q8_0 ? 32 : 64;
    const int TR = a.down_gsz;
    if (a.k <= 0 || a.k > kMaxK || a.E <= 0 || a.E > kMaxE || a.F <= 0 || a.F % TR || a.H % slot ||
        (TR != 16 && TR != 32))
        return hipErrorInvalidValue;
    const int S = a.H / slot;
    int G = 4, U = 1;
    while (G < S && G < 64) G <<= 1;
    if (S > 64) U = (S + 63) / 64;
    if (U > 2) return hipErrorInvalidValue;
    const int n_tot = a.k + (a.shared ? 1 : 0);
    const size_t lds = lds_round(xq_bytes(a.H, type == GGML_TYPE_Q6_K ? 16 : 32));
    const int grid = a.F / TR * n_tot;
    // gate/up at H = 4096: row spans through LDS, 16 rows per work-group; a
    // down projection with groups of 32 takes the fp32 activations instead
    if (type == GGML_TYPE_Q4_K && (TR == 16 || (a.act_only && a.act)) && G == 64 && U == 1) {
        k_expand_q4t<<<a.F / 16 * n_tot, 256, lds + 512 + 4 * 16 * 576, s>>>(a);
        return hipGetLastError();
    }
#define FO_K2(TT, RR, GG, UU) \
    if (type == TT && TR == RR && G == GG && U == UU) { k_expand<TT, RR, GG, UU><<<grid, ExpandShape<TT, RR, UU>::THREADS, lds, s>>>(a); return hipGetLastError(); }
#define FO_K2T(TT) \
    FO_K2(TT, 16, 64, 1) FO_K2(TT, 16, 64, 2) FO_K2(TT, 16, 32, 1) FO_K2(TT, 16, 16, 1) FO_K2(TT, 16, 8, 1) FO_K2(TT, 16, 4, 1) \
    FO_K2(TT, 32, 64, 1) FO_K2(TT, 32, 64, 2) FO_K2(TT, 32, 32, 1) FO_K2(TT, 32, 16, 1) FO_K2(TT, 32, 8, 1) FO_K2(TT, 32, 4, 1)
    FO_K2T(GGML_TYPE_Q4_K) FO_K2T(GGML_TYPE_Q5_K) FO_K2T(GGML_TYPE_Q6_K) FO_K2T(GGML_TYPE_Q8_0)
#undef FO_K2T
#undef FO_K2
    return hipErrorInvalidValue;
}

// ============================================================ K3: reduce
// One work-group per block of RB = P*RP output rows with one wave per
// selected expert (routed in rank order, then shared): the wave keeps its
// expert's prepared activation in registers for RP passes of P rows (G lanes
// per row), so it is fetched once per RB rows; every wave issues all its
// weight loads before any arithmetic. Per-expert row sums meet in LDS and
// out = resid + sum_e w_e * dot_e is summed in that fixed order.
template <int T, int G, int RP>
__global__ __launch_bounds__(1024) void k_reduce(ReduceArgs a) {
    using F = Fmt<T>;
    constexpr int P = kWave / G, RB = P * RP;
    __shared__ float part[kMaxK + 1][RB];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, sub = lane / G;
    const int n_tot = a.k + (a.shared ? 1 : 0);
    const int S = a.F / F::SLOT;
    const int slot = min(lane % G, S - 1);          // lanes past S mirror the last slot ...
    const float live = (lane % G) < S ? 1.f : 0.f;  // ... and contribute nothing
    const int row0 = blockIdx.x * RB;
    if (wv < n_tot) {
        const uint8_t *m = (wv < a.k) ? a.base + (uint64_t)a.ids[wv] * a.stride + a.down_off
                                      : a.shared + a.sh_down_off;
        // activation first: the first dot then waits only for it and row 0
        typename F::X X;
        int gi[F::NG];
        F::groups(slot, gi);
        load_xslot(X, a.xq_act + (uint64_t)wv * a.xq_vstride, a.F, gi);
        typename F::Raw raw[RP];
#pragma unroll
        for (int p = 0; p < RP; p++) {
            const int row = min(row0 + p * P + sub, a.H - 1);
            raw[p] = F::load(m + (uint64_t)row * a.row_bytes, slot);
        }
#pragma unroll
        for (int p = 0; p < RP; p++) {
            const float v = group_sum<G>(live * F::dot(raw[p], slot, X));
            if ((lane % G) == 0) part[wv][p * P + sub] = v;
        }
    }
    __syncthreads();
    if (tid < RB && row0 + tid < a.H) {
        float acc = 0.f;
        for (int e = 0; e < a.k; e++) acc = fmaf(a.weights[e], part[e][tid], acc);
        if (a.shared) acc = fmaf(a.shared_w ? *a.shared_w : 1.0f, part[a.k][tid], acc);
        else if (a.ys) acc = fmaf(a.shared_w ? *a.shared_w : 1.0f, a.ys[row0 + tid], acc);
        a.out[row0 + tid] = (a.resid ? a.resid[row0 + tid] : 0.f) + acc;
    }
}

// K3 with the weights staged through LDS: each wave streams its expert's
// 16-row block (16 consecutive rows = 16 * RBYTES contiguous bytes) with
// 1 KiB coalesced loads, writes the pieces to its own LDS area and runs the
// same per-lane slot dots as k_reduce from there, P rows per pass: a pass
// only waits for the pieces that cover its rows (loads retire in issue
// order, and the activation slot is requested before the weights), so the
// arithmetic of early rows overlaps the arrival of later ones. All n_tot
// blocks of a work-group are resident at once (n_tot * 16 * RBYTES <=
// kTileLdsMax).
constexpr int kTileRows = 16;
constexpr uint32_t kTileLdsMax = 152 * 1024;

constexpr int kTileMaxWaves = 12;   // 3 waves per SIMD: room for a whole block in registers

// One wave's 16-row block of matrix m (row0.., RBYTES per row) against the
// prepared activation X: the block streams through the wave's LDS area `dst`
// and its row dots land in part_w[0..16).
template <int T, int G, int RBYTES>
FO_DEV void tile_block_dots(const uint8_t *m, const typename Fmt<T>::X &X, uint8_t *dst, float *part_w, int row0,
                            int H, int slot, float live) {
    using F = Fmt<T>;
    constexpr int P = kWave / G, RP = kTileRows / P;
    constexpr uint32_t TB = kTileRows * RBYTES;
    constexpr int NV = (TB + 1023) / 1024;
    const int lane = threadIdx.x & 63, sub = lane / G;
    const uint8_t *src = m + (uint64_t)row0 * RBYTES;
    const uint32_t nb = (uint32_t)min(kTileRows, H - row0) * RBYTES;
    // a piece that straddles the end is read from the last 16 valid bytes
    // and written to that same position (identical bytes overlap)
    auto pos = [&](uint32_t o) { return o + 16 <= nb ? o : nb - 16; };
    uint4 v[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) v[i] = ldw16(src + pos(i * 1024 + lane * 16));
    // keep the scheduler from sinking weight loads below the arithmetic
    __builtin_amdgcn_sched_barrier(0);
    int written = 0;
#pragma unroll
    for (int p = 0; p < RP; p++) {
        const int need = ((p + 1) * P * RBYTES + 1023) / 1024;   // pieces covering rows < (p+1)*P
#pragma unroll
        for (int i = 0; i < NV; i++)
            if (i >= written && i < need) *(uint4 *)(dst + pos(i * 1024 + lane * 16)) = v[i];
        written = need;
        const int r = p * P + sub;
        const typename F::Raw raw = F::load(dst + r * RBYTES, slot);
        const float d = group_sum<G>(live * F::dot(raw, slot, X));
        if ((lane % G) == 0) part_w[r] = d;
    }
}

// The shared expert's block when its down projection has its own type TS
// (F = 1024): the lane's activation slot is prepared from the fp32 shared
// activation k_expand left (prep_group_regs, bit-identical to the prepared
// form the routed experts read), then the block runs as a routed one.
template <int TS>
FO_DEV void shared_block_dots(const ReduceArgs &a, uint8_t *dst, float *part_w, int row0) {
    using F = Fmt<TS>;
    constexpr int S = 1024 / F::SLOT, G = S, RB = 1024 / (F::SLOT == 64 ? 256 : 32) * F::BLOCK;
    const int slot = (threadIdx.x & 63) % G;
    typename F::X X;
    int gi[F::NG];
    F::groups(slot, gi);
#pragma unroll
    for (int g = 0; g < F::NG; g++) prep_group_regs<F::GSZ>(a.sh_act + gi[g] * F::GSZ, X.l[g], X.sc[g], X.sum[g]);
    tile_block_dots<TS, G, RB>(a.shared + a.sh_down_off, X, dst, part_w, row0, a.H, slot, 1.f);
}

// Tile bytes of a 16-row block of a 1024-wide row in type t.
__host__ __device__ constexpr uint32_t tile_stride_1024(int t) {
    return (uint32_t)kTileRows * (t == GGML_TYPE_Q4_K ? 576u : t == GGML_TYPE_Q5_K ? 704u
                                  : t == GGML_TYPE_Q6_K ? 840u : 1088u);
}

template <int T, int G, int RBYTES>
__global__ __launch_bounds__(64 * kTileMaxWaves) void k_reduce_tile(ReduceArgs a) {
    using F = Fmt<T>;
    constexpr uint32_t TB = kTileRows * RBYTES, TSTRIDE = (TB + 15) & ~15u;
    extern __shared__ __attribute__((aligned(16))) uint8_t tiles[];
    __shared__ float part[kMaxK + 1][kTileRows];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const bool own = a.shared && a.sh_type >= 0;          // shared down in its own type
    const int n_tot = a.k + (a.shared ? 1 : 0);
    const int S = a.F / F::SLOT;
    const int slot = min(lane % G, S - 1);          // lanes past S mirror the last slot ...
    const float live = (lane % G) < S ? 1.f : 0.f;  // ... and contribute nothing
    const int row0 = blockIdx.x * kTileRows;
    if (wv < n_tot && !(own && wv == a.k)) {
        const uint8_t *m = (wv < a.k) ? a.base + (uint64_t)a.ids[wv] * a.stride + a.down_off
                                      : a.shared + a.sh_down_off;
        typename F::X X;
        int gi[F::NG];
        F::groups(slot, gi);
        if (a.act_f32) {   // the slot prepared here from the fp32 activation (as prep_group_lanes would)
#pragma unroll
            for (int g = 0; g < F::NG; g++)
                prep_group_regs<F::GSZ>(a.act_f32 + (uint64_t)wv * a.F + gi[g] * F::GSZ, X.l[g], X.sc[g], X.sum[g]);
        } else {
            load_xslot(X, a.xq_act + (uint64_t)wv * a.xq_vstride, a.F, gi);
        }
        tile_block_dots<T, G, RBYTES>(m, X, tiles + wv * TSTRIDE, part[wv], row0, a.H, slot, live);
    } else if (own && wv == a.k) {
        uint8_t *dst = tiles + a.k * TSTRIDE;
        switch (a.sh_type) {
            case GGML_TYPE_Q4_K: shared_block_dots<GGML_TYPE_Q4_K>(a, dst, part[wv], row0); break;
            case GGML_TYPE_Q5_K: shared_block_dots<GGML_TYPE_Q5_K>(a, dst, part[wv], row0); break;
            case GGML_TYPE_Q6_K: shared_block_dots<GGML_TYPE_Q6_K>(a, dst, part[wv], row0); break;
            default: shared_block_dots<GGML_TYPE_Q8_0>(a, dst, part[wv], row0); break;
        }
    }
    __syncthreads();
    if (tid < kTileRows && row0 + tid < a.H) {
        float acc = 0.f;
        for (int e = 0; e < a.k; e++) acc = fmaf(a.weights[e], part[e][tid], acc);
        if (a.shared) acc = fmaf(a.shared_w ? *a.shared_w : 1.0f, part[a.k][tid], acc);
        else if (a.ys) acc = fmaf(a.shared_w ? *a.shared_w : 1.0f, a.ys[row0 + tid], acc);
        a.out[row0 + tid] = (a.resid ? a.resid[row0 + tid] : 0.f) + acc;
    }
}

// LDS of k_reduce_tile: k routed blocks of tstride bytes, then the shared
// expert's block (its own type's size when sh_type >= 0).
static uint32_t reduce_tile_lds(const ReduceArgs &a, uint32_t tstride) {
    return a.k * tstride + (a.shared ? (a.sh_type >= 0 ? tile_stride_1024(a.sh_type) : tstride) : 0);
}

bool reduce_takes_tile(int type, const ReduceArgs &a) {
    const int n_tot = a.k + (a.shared ? 1 : 0);
    return (type == GGML_TYPE_Q6_K || type == GGML_TYPE_Q4_K || type == GGML_TYPE_Q5_K) && n_tot <= kTileMaxWaves &&
           reduce_tile_lds(a, (uint32_t)(kTileRows * a.row_bytes + 15) & ~15u) <= kTileLdsMax &&
           a.H >= kTileRows && a.F == 1024;
}

bool reduce_takes_shared_type(int down_type, const ReduceArgs &a, int sh_type) {
    if (a.F != 1024 || a.H < kTileRows || a.k + 1 > kTileMaxWaves) return false;
    if (down_type != GGML_TYPE_Q6_K && down_type != GGML_TYPE_Q4_K && down_type != GGML_TYPE_Q5_K) return false;
    if (sh_type != GGML_TYPE_Q4_K && sh_type != GGML_TYPE_Q5_K && sh_type != GGML_TYPE_Q6_K && sh_type != GGML_TYPE_Q8_0)
        return false;
    ReduceArgs b = a;
    b.shared = (const uint8_t *)1;
    b.sh_type = sh_type;
    return reduce_tile_lds(b, tile_stride_1024(down_type)) <= kTileLdsMax;
}

template <int T, int G, int RBYTES>
static hipError_t reduce_tile(const ReduceArgs &a, hipStream_t s) {
    static bool attr = false;   // more than the 64 KiB default of dynamic LDS
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_reduce_tile<T, G, RBYTES>,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)kTileLdsMax);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const int n_tot = a.k + (a.shared ? 1 : 0);
    const uint32_t lds = reduce_tile_lds(a, (kTileRows * RBYTES + 15) & ~15u);
    k_reduce_tile<T, G, RBYTES><<<(a.H + kTileRows - 1) / kTileRows, 64 * n_tot, lds, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_reduce(int type, const ReduceArgs &a, hipStream_t s, int n_cu) {
    (void)n_cu;
    const int slot = type == GGML_TYPE_Q8_0 ? 32 : 64;
    const int n_tot = a.k + (a.shared ? 1 : 0);
    if (a.F % slot || a.F / slot > 64 || a.k <= 0 || n_tot > 16 || a.H <= 0) return hipErrorInvalidValue;
    const int S = a.F / slot;
    int G = 4;
    while (G < S) G <<= 1;
    // the LDS-staged variant when all n_tot 16-row blocks fit at once (and
    // the only one that takes a shared block in its own type)
    if (a.shared && a.sh_type >= 0 && !reduce_takes_shared_type(type, a, a.sh_type)) return hipErrorInvalidValue;
    if (reduce_takes_tile(type, a)) {
        if (type == GGML_TYPE_Q6_K) return reduce_tile<GGML_TYPE_Q6_K, 16, 840>(a, s);
        if (type == GGML_TYPE_Q4_K) return reduce_tile<GGML_TYPE_Q4_K, 16, 576>(a, s);
        if (type == GGML_TYPE_Q5_K) return reduce_tile<GGML_TYPE_Q5_K, 16, 704>(a, s);
    }
    if (a.act_f32) return hipErrorInvalidValue;   // only the LDS-staged kernel prepares from fp32
    constexpr int RP = 4;
    const int RB = (64 / G) * RP;
    const int grid = (a.H + RB - 1) / RB;
    const int threads = 64 * n_tot;
#define FO_K3(TT, GG) \
    if (type == TT && G == GG) { k_reduce<TT, GG, RP><<<grid, threads, 0, s>>>(a); return hipGetLastError(); }
#define FO_K3T(TT) FO_K3(TT, 64) FO_K3(TT, 32) FO_K3(TT, 16) FO_K3(TT, 8) FO_K3(TT, 4)
    FO_K3T(GGML_TYPE_Q4_K) FO_K3T(GGML_TYPE_Q5_K) FO_K3T(GGML_TYPE_Q6_K) FO_K3T(GGML_TYPE_Q8_0)
#undef FO_K3T
#undef FO_K3
    return hipErrorInvalidValue;
}

// ============================================================ shared expert, standalone
// A shared expert whose types or intermediate size differ from the routed
// experts' runs as these two kernels (its weight matrices are not those the
// layer kernels are specialised for): gate/up with its own RMSNorm of x (any
// H = 256 n, 4 rows per work-group), then the down role.
__global__ __launch_bounds__(256) void k_shared_gateup(SharedArgs s, const float *__restrict__ x,
                                                       const float *__restrict__ norm_w, float eps, int split) {
    extern __shared__ __attribute__((aligned(16))) float hs[];   // h [H]
    __shared__ float red[4];
    __shared__ float2 s_gu[4];
    constexpr int PL = 4;   // pieces per lane and round: H / (16 * 64 * split * PL) rounds
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, H = s.H;
    const int r = blockIdx.x * (4 / split) + wv / split, part = wv % split;
    const int rounds = (H / 16 + 64 * split * PL - 1) / (64 * split * PL);
    GateUpRaw<PL> raw;
    shared_gateup_load<PL>(s, r, part, split, 0, raw);
    float scale = 1.0f;
    if (norm_w) {
        float ss = 0.f;
        for (int i = tid; i < H; i += 256) ss += x[i] * x[i];
        ss = wave_sum_dpp(ss);
        if (lane == 0) red[wv] = ss;
        __syncthreads();
        scale = 1.0f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)H + eps);
    }
    for (int i = tid; i < H; i += 256) hs[i] = norm_w ? x[i] * scale * norm_w[i] : x[i];
    __syncthreads();
    float g = 0.f, v = 0.f;
    shared_gateup_finish<PL>(s, part, split, 0, raw, hs, g, v);
    for (int q = 1; q < rounds; q++) {
        shared_gateup_load<PL>(s, r, part, split, q, raw);
        shared_gateup_finish<PL>(s, part, split, q, raw, hs, g, v);
    }
    g = group_sum<kWave>(g);
    v = group_sum<kWave>(v);
    if (lane == 0) s_gu[wv] = make_float2(g, v);
    __syncthreads();
    if (part == 0 && lane == 0 && r < s.F) {
        float gs = s_gu[wv].x, us = s_gu[wv].y;
        for (int q = 1; q < split; q++) { gs += s_gu[wv + q].x; us += s_gu[wv + q].y; }
        s.act[r] = (gs / (1.0f + expf(-gs))) * us;
    }
}

__global__ __launch_bounds__(256) void k_shared_down(SharedArgs s) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sd_lds[];
    shared_down_role(s, blockIdx.x, sd_lds);
}

hipError_t launch_shared(const SharedArgs &a, const float *x, const float *norm_w, float eps, hipStream_t st) {
    if (!a.blob || !a.act || !a.ys || a.H <= 0 || a.H % 256 || a.H > 8192 || a.F <= 0 || a.F % 256 || a.F > 8192 ||
        a.down_rpw <= 0)
        return hipErrorInvalidValue;
    const int split = shared_gateup_split(a.F);
    k_shared_gateup<<<(a.F * split + 3) / 4, 256, (size_t)a.H * 4, st>>>(a, x, norm_w, eps, split);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    SharedArgs b = a;
    b.down_waves = 4;
    k_shared_down<<<shared_down_wgs(b), 256, (size_t)a.F * 4, st>>>(b);
    return hipGetLastError();
}

}  // namespace fo
