// shared.h — the always-active shared expert of a MoE layer, with its own
// gate / up / down types and its own intermediate size F_s (reference
// include/model.h:104-108 per-tensor shared types, src/model.c:164, 359-371;
// shared_expert_ffn at src/inference.c:361-374: gate -> silu, up, mul, down,
// then the sigmoid gate and the add of src/inference.c:585-595).
//
// A shared expert with the routed experts' types and intermediate size rides
// in the layer kernels as one more expert slot; any other runs as the two
// kernels built from the roles below (moe.hip k_shared_gateup, k_shared_down),
// after the router kernel and before the routed down projection, which adds
// ys to its combine:
//   gate/up role  act[r] = silu(gate[r,:] . h) * (up[r,:] . h), one row r per
//                 wave, h = the (normed) layer input, in LDS;
//   down role     ys[i] = w * (down[i,:] . act), w = the shared-expert weight
//                 (sigmoid(h . v), or 1), act staged in LDS.
// A lane holds one 16-value piece per row in flight.
// Both are fp32 dot products over exactly dequantized weights — per value the
// operation of the reference's vec_dot_*_f32 (src/quant.c:109-143, 177-212,
// 249-262, 276-288): w = d1*q - m1 (Q4_K/Q5_K), (d*sc)*q (Q6_K), d*q (Q8_0),
// then sum += w*x, with the partial sums of 16-value pieces added in a
// different order. The shared expert is one matrix set per layer (8 MB at the
// benchmark shape), so this path favours generality (any of the four layer
// types per matrix, any F_s) over the integer-limb decoders of the routed
// experts.
#pragma once

#include "common.h"

namespace fo {

// A row of K values is cut into K/16 pieces of 16 values; a lane decodes one
// piece at a time (at most 8 dwords of raw bytes), so that several rows'
// pieces can be in flight per lane at a modest register cost.
//   Q4_K / Q5_K piece r of super-block b (r = 4m + q): bytes 8q..8q+7 of the
//     32 code bytes of sub-blocks 2m, 2m+1 — values 256b + 64m + 8q + i (low
//     nibbles, sub-block 2m) and 256b + 64m + 32 + 8q + i (high, 2m+1);
//   Q6_K piece r (r = 8n + 4tp + q): ql bytes 64n + 32tp + 8q.., qh bytes
//     32n + 8q.. — values 256b + 128n + 32t + 8q + i for t = tp (low nibbles)
//     and t = tp + 2 (high), scales sc[8n + 2t + q/2];
//   Q8_0 piece: half h of block c — values 32c + 16h + i.
struct PRaw { uint4 a; uint4 b; };

template <int T> FO_DEV PRaw pload(const uint8_t *row, int p);
template <> FO_DEV PRaw pload<GGML_TYPE_Q4_K>(const uint8_t *row, int p) {
    const uint8_t *b = row + (p >> 4) * 144;
    const int r = p & 15;
    const uint2 q = ld8(b + 16 + 32 * (r >> 2) + 8 * (r & 3));
    return PRaw{ld16(b), make_uint4(q.x, q.y, 0, 0)};
}
template <> FO_DEV PRaw pload<GGML_TYPE_Q5_K>(const uint8_t *row, int p) {
    const uint8_t *b = row + (p >> 4) * 176;
    const int r = p & 15;
    const uint2 q = ld8(b + 48 + 32 * (r >> 2) + 8 * (r & 3)), h = ld8(b + 16 + 8 * (r & 3));
    return PRaw{ld16(b), make_uint4(q.x, q.y, h.x, h.y)};
}
template <> FO_DEV PRaw pload<GGML_TYPE_Q6_K>(const uint8_t *row, int p) {
    const uint8_t *b = row + (p >> 4) * 210;
    const int r = p & 15, n = r >> 3, tp = (r >> 2) & 1, q = r & 3;
    const uint2 l = ld8(b + 64 * n + 32 * tp + 8 * q), h = ld8(b + 128 + 32 * n + 8 * q), sc = ld8(b + 192 + 8 * n);
    return PRaw{make_uint4(l.x, l.y, h.x, h.y), make_uint4(sc.x, sc.y, ld2(b + 208), 0)};
}
template <> FO_DEV PRaw pload<GGML_TYPE_Q8_0>(const uint8_t *row, int p) {
    const uint8_t *b = row + (p >> 1) * 34;
    return PRaw{ld16(b + 2 + 16 * (p & 1)), make_uint4(ld2(b), 0, 0, 0)};
}

// Byte i (0..3) of w.
FO_DEV int byte_of(uint32_t w, int i) { return (int)((w >> (8 * i)) & 0xFFu); }

// 6-bit (scale, min) of sub-block j from the 16-byte block header (d, dmin,
// 12 scale bytes; reference src/quant.c:72-80).
FO_DEV void scale_min_k4(const uint4 &h, int j, int &sc, int &mn) {
    const uint32_t q[3] = {h.y, h.z, h.w};
    auto byte = [&](int i) { return byte_of(q[i >> 2], i & 3); };
    if (j < 4) {
        sc = byte(j) & 63;
        mn = byte(j + 4) & 63;
    } else {
        sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
        mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

// acc + sum_i w(code_i) * x_i over 8 values x[0..8) (LDS, 16-byte aligned).
template <typename W>
FO_DEV float dot8(const float *x, float acc, W w) {
    const float4 x0 = *(const float4 *)x, x1 = *(const float4 *)(x + 4);
    acc = fmaf(w(0), x0.x, acc);
    acc = fmaf(w(1), x0.y, acc);
    acc = fmaf(w(2), x0.z, acc);
    acc = fmaf(w(3), x0.w, acc);
    acc = fmaf(w(4), x1.x, acc);
    acc = fmaf(w(5), x1.y, acc);
    acc = fmaf(w(6), x1.z, acc);
    return fmaf(w(7), x1.w, acc);
}

// Dot of piece p with the row's vector x (LDS, plain layout).
template <int T> FO_DEV float pdot(const PRaw &r, int p, const float *x);

template <int T>
FO_DEV float pdot_k45(const PRaw &r, int p, const float *x) {
    const int b = p >> 4, m = (p >> 2) & 3, q = p & 3;
    const float d = h2f(r.a.x), dmin = h2f(r.a.x >> 16);
    const uint32_t c[2] = {r.b.x, r.b.y}, h[2] = {r.b.z, r.b.w};
    const float *xp = x + 256 * b + 64 * m + 8 * q;
    float acc = 0.f;
#pragma unroll
    for (int half = 0; half < 2; half++) {
        const int j = 2 * m + half;
        int sc, mn;
        scale_min_k4(r.a, j, sc, mn);
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        acc = dot8(xp + 32 * half, acc, [&](int i) {
            int code = (byte_of(c[i >> 2], i & 3) >> (4 * half)) & 0xF;
            if (T == GGML_TYPE_Q5_K) code += ((byte_of(h[i >> 2], i & 3) >> j) & 1) << 4;
            return __fsub_rn(__fmul_rn(d1, (float)code), m1);
        });
    }
    return acc;
}
template <> FO_DEV float pdot<GGML_TYPE_Q4_K>(const PRaw &r, int p, const float *x) {
    return pdot_k45<GGML_TYPE_Q4_K>(r, p, x);
}
template <> FO_DEV float pdot<GGML_TYPE_Q5_K>(const PRaw &r, int p, const float *x) {
    return pdot_k45<GGML_TYPE_Q5_K>(r, p, x);
}
template <> FO_DEV float pdot<GGML_TYPE_Q6_K>(const PRaw &r, int p, const float *x) {
    const int b = p >> 4, n = (p >> 3) & 1, tp = (p >> 2) & 1, q = p & 3;
    const float d = h2f(r.b.z);
    const uint32_t l[2] = {r.a.x, r.a.y}, h[2] = {r.a.z, r.a.w};
    float acc = 0.f;
#pragma unroll
    for (int half = 0; half < 2; half++) {
        const int t = tp + 2 * half, sidx = 2 * t + (q >> 1);   // scale byte of the 8 loaded
        const float dsc = d * (float)(int8_t)byte_of(sidx < 4 ? r.b.x : r.b.y, sidx & 3);
        acc = dot8(x + 256 * b + 128 * n + 32 * t + 8 * q, acc, [&](int i) {
            const int lo = (byte_of(l[i >> 2], i & 3) >> (4 * half)) & 0xF;
            const int hb = (byte_of(h[i >> 2], i & 3) >> (2 * t)) & 3;
            return __fmul_rn(dsc, (float)((lo | (hb << 4)) - 32));
        });
    }
    return acc;
}
template <> FO_DEV float pdot<GGML_TYPE_Q8_0>(const PRaw &r, int p, const float *x) {
    const float d = h2f(r.b.x);
    const uint32_t c[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
    const float *xp = x + 16 * p;
    auto w = [&](int i) { return __fmul_rn(d, (float)(int8_t)byte_of(c[i >> 2], i & 3)); };
    const float acc = dot8(xp, 0.f, w);
    return dot8(xp + 8, acc, [&](int i) { return w(8 + i); });
}

// Runtime-typed piece load and dot (wave-uniform type).
FO_DEV PRaw pload_t(int type, const uint8_t *row, int p) {
    switch (type) {
        case GGML_TYPE_Q4_K: return pload<GGML_TYPE_Q4_K>(row, p);
        case GGML_TYPE_Q5_K: return pload<GGML_TYPE_Q5_K>(row, p);
        case GGML_TYPE_Q6_K: return pload<GGML_TYPE_Q6_K>(row, p);
        default: return pload<GGML_TYPE_Q8_0>(row, p);
    }
}
FO_DEV float pdot_t(int type, const PRaw &r, int p, const float *x) {
    switch (type) {
        case GGML_TYPE_Q4_K: return pdot<GGML_TYPE_Q4_K>(r, p, x);
        case GGML_TYPE_Q5_K: return pdot<GGML_TYPE_Q5_K>(r, p, x);
        case GGML_TYPE_Q6_K: return pdot<GGML_TYPE_Q6_K>(r, p, x);
        default: return pdot<GGML_TYPE_Q8_0>(r, p, x);
    }
}

// Shared-expert description for the roles (blob = gate | up | down).
struct SharedArgs {
    const uint8_t *blob;          // NULL: no shared expert
    int gate_type, up_type, down_type;
    uint64_t up_off, down_off;    // byte offsets of up and down in the blob
    uint64_t gate_rb, up_rb, down_rb;   // row bytes
    int F, H;
    float *act;                   // [F] fp32 SwiGLU activation
    const float *w;               // shared-expert weight (sigmoid gate; 1 when NULL)
    float *ys;                    // [H] w * (down . act)
    int down_rpw;                 // down rows per wave
    int down_waves;               // waves per work-group of the down role
};

// Lanes per row for a row of K values: one piece per lane, up to 64.
__host__ __device__ inline int lanes_for(int K) {
    int g = 16;
    while (g < K / 16 && g < 64) g <<= 1;
    return g;
}

// Gate/up role: row r is split over `split` waves (split = 1, 2, 4), wave
// `part` taking pieces part*64 + lane + 64*split*i of the H/16 pieces (at
// most 4*ROUNDS per lane). The rows' pieces are requested by
// shared_gateup_load before the caller stages h in LDS, so they are in flight
// meanwhile; shared_gateup_finish returns this wave's partial gate and up sums
// (the caller adds the parts in order and writes act[r] = silu(g) * u).
template <int PL>
struct GateUpRaw { PRaw g[PL], u[PL]; };

template <int PL>
FO_DEV void shared_gateup_load(const SharedArgs &s, int r, int part, int split, int round, GateUpRaw<PL> &raw) {
    const int lane = threadIdx.x & 63, np = s.H / 16;
    const int rr = min(r, s.F - 1);
    const uint8_t *gr = s.blob + (uint64_t)rr * s.gate_rb, *ur = s.blob + s.up_off + (uint64_t)rr * s.up_rb;
#pragma unroll
    for (int i = 0; i < PL; i++) {
        const int p = min(part * 64 + lane + 64 * split * (PL * round + i), np - 1);
        raw.g[i] = pload_t(s.gate_type, gr, p);
        raw.u[i] = pload_t(s.up_type, ur, p);
    }
}

template <int PL>
FO_DEV void shared_gateup_finish(const SharedArgs &s, int part, int split, int round, const GateUpRaw<PL> &raw,
                                 const float *h_lds, float &g, float &v) {
    const int lane = threadIdx.x & 63, np = s.H / 16;
#pragma unroll
    for (int i = 0; i < PL; i++) {
        const int p = part * 64 + lane + 64 * split * (PL * round + i);
        if (p < np) {
            g += pdot_t(s.gate_type, raw.g[i], p, h_lds);
            v += pdot_t(s.up_type, raw.u[i], p, h_lds);
        }
    }
}

// Down role, work-group `wg` of down_waves waves (= blockDim.x / 64): rows
// [wg*down_waves*down_rpw, +down_waves*down_rpw) of ys, G lanes per row (one
// piece each per pass over the row), four rows' pieces in flight per lane.
template <int G>
FO_DEV void shared_down_rows(const SharedArgs &s, int wg, const float *act_lds) {
    constexpr int P = kWave / G, RQ = 4;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, sub = lane / G, gl = lane % G;
    const int np = s.F / 16, ppl = (np + G - 1) / G;   // pieces per lane and row
    const float w = s.w ? *s.w : 1.0f;
    const int row0 = (wg * s.down_waves + wv) * s.down_rpw;
    for (int r0 = 0; r0 < s.down_rpw; r0 += RQ * P) {
        float acc[RQ] = {};
        for (int c = 0; c < ppl; c++) {
            const int p = min(gl + G * c, np - 1);
            PRaw raw[RQ];
#pragma unroll
            for (int q = 0; q < RQ; q++) {
                const int row = min(row0 + r0 + q * P + sub, s.H - 1);
                raw[q] = pload_t(s.down_type, s.blob + s.down_off + (uint64_t)row * s.down_rb, p);
            }
            if (gl + G * c < np) {
#pragma unroll
                for (int q = 0; q < RQ; q++) acc[q] += pdot_t(s.down_type, raw[q], p, act_lds);
            }
        }
#pragma unroll
        for (int q = 0; q < RQ; q++) {
            const float v = group_sum<G>(acc[q]);
            const int rl = r0 + q * P + sub, row = row0 + rl;
            if (gl == 0 && rl < s.down_rpw && row < s.H) s.ys[row] = w * v;
        }
    }
}

FO_DEV void shared_down_role(const SharedArgs &s, int wg, uint8_t *lds) {
    float *act = (float *)lds;
    for (int i = threadIdx.x; i < s.F; i += blockDim.x) act[i] = s.act[i];
    __syncthreads();
    switch (lanes_for(s.F)) {
        case 16: shared_down_rows<16>(s, wg, act); break;
        case 32: shared_down_rows<32>(s, wg, act); break;
        default: shared_down_rows<64>(s, wg, act); break;
    }
}

// Work-groups of the down role for H rows.
__host__ inline int shared_down_wgs(const SharedArgs &s) {
    const int rows = s.down_waves * s.down_rpw;
    return (s.H + rows - 1) / rows;
}
// Down rows per wave for F_s: one pass of four rows per lane group (the
// work-group count then reaches ~256 at the benchmark H).
__host__ inline int shared_down_rpw(int F) { return 4 * (64 / lanes_for(F)); }
// Waves per gate/up row: ~512 work-groups of 4 waves (two per CU) to spread
// the fp32 dot arithmetic.
__host__ inline int shared_gateup_split(int F) { return F >= 2048 ? 1 : F >= 1024 ? 2 : 4; }

}  // namespace fo
