// formats.h — per-format "slot" decoders for the decode-time (batch-1) kernels.
//
// A row of K values is cut into S = K / SLOT slots. Each lane owns fixed slots
// for every row it touches, so its slice of the activation vector stays in
// registers for the whole kernel (the activation is the only reused operand;
// weight bytes stream through exactly once).
//
// Arithmetic. At batch 1 a plain "byte -> float, fma" unpack costs ~5 VALU
// instructions per Q4_K weight byte, which on gfx950 is as slow as HBM itself.
// Instead the activation is held in block fixed point: each group of GSZ
// values shares an exponent e, X = round(x * 2^e) with |X| < 2^22, split into
// three balanced int8 limbs X = X0 + 2^8 X1 + 2^16 X2. The weight
// codes are small non-negative (or int8) integers, so
//     sum_i q_i * X_i = sum_L 2^(8L) * sum_i q_i * X_{L,i}
// is computed exactly with v_dot4c_i32_i8 (4 products per instruction) and
// only the per-group combination and the scale application use fp32. Each X
// carries an absolute error of at most 2^-23 of the group maximum (2 ulp of
// the largest value) — the size of the fp32 rounding the reference's own
// sequential sum incurs (reference src/quant.c:109-212).
//
// Sub-block scales are applied once per sub-block: sum_i (d*sc*q_i - dmin*m)
// * x_i = d*sc*sum_i q_i x_i - dmin*m*sum_i x_i; the group sums of x are
// prepared with the limbs.
//
// Block layouts follow include/quant_types.h (reference include/quant_types.h
// :17-53) and the value orders of reference src/quant.c:82-105 (Q4_K),
// 147-175 (Q6_K), 216-247 (Q5_K), 266-274 (Q8_0).
#pragma once

#include "common.h"

namespace fo {

constexpr int kLimbs = 3;
constexpr int kFixBits = 22;   // |X| < 2^22: limbs X0, X1 in [-128,127], X2 in [-64,64]

// Prepared activation of one group of GSZ values:
//   limb dwords l[L][k] hold limb L of values 4k..4k+3 (one int8 each),
//   scsum = {2^-e, sum of the group's fp32 values}.
// In memory a vector of K values is [K/GSZ groups][kLimbs][GSZ/4] int32 limb
// dwords followed by K/GSZ float2 {scale, sum} (xq_bytes in common.h).

// a2 * 256 + a1 is formed exactly in int32 (|a| < 2^20 for every format) and
// rounded once on conversion, as fmaf(a2, 256, a1) would round it
FO_DEV float combine(const int a[kLimbs]) {
    return fmaf((float)((a[2] << 8) + a[1]), 256.f, (float)a[0]);
}

FO_DEV int dot4(uint32_t codes, int limbs, int acc) {
    return __builtin_amdgcn_sdot4((int)codes, limbs, acc, false);
}

template <int T> struct Fmt;

// Per-lane prepared activation of one slot: NG groups of GSZ values.
template <int NG, int GSZ> struct XSlot {
    int l[NG][kLimbs][GSZ / 4];
    float sc[NG], sum[NG];
};

// ============================================================ activation prep
// One group of GSZ values: exponent from the group maximum, the balanced int8
// limbs of X = round(x * 2^e) (layout above), the scale 2^-e and the fp32
// sum, in registers. prep_group (kernels.hip) stores them; k_xprep uses one
// thread per group, the tile kernels one lane per group, bit-identically.
// Scale and sum of a prepared group. The sum is that of the quantized values,
// sum_i X_i * 2^-e, from the exact integer sum with one rounding: it enters
// the dots as the Q4_K/Q5_K min term (dmin * m * sum) and the Q6_K offset
// (-32 * sum), where it cancels against the code sums, so a sequential fp32
// sum of x (up to GSZ roundings of partial sums) would cost several times the
// reference's own rounding error. A group holding a NaN or an infinity gets
// NaN for both, so that the non-finite value reaches every output it touches,
// as in the reference's fp32 dot (the limbs of such a group are meaningless).
FO_DEV void group_scale_sum(float M, float chk, int e, int isum, float &scale, float &sum) {
    if (chk != 0.f) {   // chk = sum of v * 0: NaN exactly when some v is NaN or infinite
        scale = sum = __int_as_float(0x7FC00000);
        return;
    }
    scale = (M > 0.f) ? ldexpf(1.0f, -e) : 0.f;
    sum = (float)isum * scale;
}

// One group of GSZ values: exponent from the group maximum, the balanced int8
// limbs of X = round(x * 2^e) (layout above), the scale 2^-e and the group
// sum (group_scale_sum), in registers. prep_group (kernels.hip) stores them;
// k_xprep uses one thread per group, the tile kernels one lane per group,
// bit-identically.
template <int GSZ>
FO_DEV void prep_group_vals(const float (&vals)[GSZ], int (&limb)[kLimbs][GSZ / 4], float &scale, float &sum) {
    float M = 0.f, chk = 0.f;
#pragma unroll
    for (int i = 0; i < GSZ; i++) { M = fmaxf(M, fabsf(vals[i])); chk += vals[i] * 0.f; }
    int E = 0;
    frexpf(M, &E);               // M < 2^E
    int e = kFixBits - E;
    if (e > 149) e = 149;        // keep 2^-e representable
    uint32_t lb[kLimbs][GSZ / 4];
#pragma unroll
    for (int L = 0; L < kLimbs; L++)
#pragma unroll
        for (int k = 0; k < GSZ / 4; k++) lb[L][k] = 0;
    int isum = 0;                // |isum| < GSZ * 2^22: exact in int32
#pragma unroll
    for (int i = 0; i < GSZ; i++) {
        int X = (M > 0.f && chk == 0.f) ? __float2int_rn(ldexpf(vals[i], e)) : 0;
        isum += X;
#pragma unroll
        for (int L = 0; L < kLimbs - 1; L++) {
            const int b = (int)(int8_t)(X & 0xFF);
            X = (X - b) >> 8;
            lb[L][i / 4] |= (uint32_t)(b & 0xFF) << (8 * (i % 4));
        }
        lb[kLimbs - 1][i / 4] |= (uint32_t)(X & 0xFF) << (8 * (i % 4));
    }
    group_scale_sum(M, chk, e, isum, scale, sum);
#pragma unroll
    for (int L = 0; L < kLimbs; L++)
#pragma unroll
        for (int k = 0; k < GSZ / 4; k++) limb[L][k] = (int)lb[L][k];
}

template <int GSZ>
FO_DEV void prep_group_regs(const float *__restrict__ xp, int (&limb)[kLimbs][GSZ / 4], float &scale,
                            float &sum) {
    float vals[GSZ];
#pragma unroll
    for (int i = 0; i < GSZ; i += 4) {
        float4 t = *(const float4 *)(xp + i);
        vals[i] = t.x; vals[i + 1] = t.y; vals[i + 2] = t.z; vals[i + 3] = t.w;
    }
    prep_group_vals<GSZ>(vals, limb, scale, sum);
}

// Load the groups gi[0..NG) of a prepared vector into registers.
template <int NG, int GSZ>
FO_DEV void load_xslot(XSlot<NG, GSZ> &x, const uint8_t *xq, int K, const int gi[NG]) {
    const uint8_t *ss = xq + xq_limb_bytes(K);
#pragma unroll
    for (int g = 0; g < NG; g++) {
        const uint8_t *p = xq + (uint64_t)gi[g] * (kLimbs * GSZ);
#pragma unroll
        for (int L = 0; L < kLimbs; L++)
#pragma unroll
            for (int k = 0; k < GSZ / 4; k += 4) {
                uint4 v = ld16(p + (L * (GSZ / 4) + k) * 4);
                x.l[g][L][k] = (int)v.x; x.l[g][L][k + 1] = (int)v.y;
                x.l[g][L][k + 2] = (int)v.z; x.l[g][L][k + 3] = (int)v.w;
            }
        uint2 s = ld8(ss + (uint64_t)gi[g] * 8);
        x.sc[g] = __uint_as_float(s.x);
        x.sum[g] = __uint_as_float(s.y);
    }
}

// ---------------------------------------------------------------- Q4_K
// Slot = one 64-value group g of super-block b: header (d, dmin, 12 scale
// bytes) + qs[32g .. 32g+31]. Low nibble of qs[32g+l] is value 64g+l, high
// nibble is value 64g+32+l (sub-blocks 2g and 2g+1 = activation groups 2s,
// 2s+1 of 32 values).
template <> struct Fmt<GGML_TYPE_Q4_K> {
    static constexpr int SLOT = 64, BLOCK = 144, NG = 2, GSZ = 32;
    using X = XSlot<NG, GSZ>;
    struct Raw { uint4 hdr, q0, q1; };

    static FO_DEV Raw load(const uint8_t *row, int s) {
        const uint8_t *b = row + (s >> 2) * BLOCK;
        const int g = s & 3;
        return Raw{ld16(b), ld16(b + 16 + 32 * g), ld16(b + 32 + 32 * g)};
    }
    static FO_DEV void groups(int s, int gi[NG]) { gi[0] = 2 * s; gi[1] = 2 * s + 1; }
    // 6-bit (scale, min) pairs of sub-blocks 2g, 2g+1 as two 16-bit byte
    // pairs (reference src/quant.c:72-80 unpacking, two at a time)
    static FO_DEV void scales(const uint4 &h, int g, uint32_t &scp, uint32_t &mp) {
        // branch-free: both encodings are formed and selected, so the header
        // stays in registers and no wait on later loads is forced here
        const int sh = 16 * (g & 1);
        const uint32_t A = (h.w >> sh) & 0xFFFFu;
        const uint32_t B = (h.y >> sh) & 0xFFFFu;
        const uint32_t C = (h.z >> sh) & 0xFFFFu;
        const uint32_t sc_lo = B & 0x3F3Fu, m_lo = C & 0x3F3Fu;
        const uint32_t sc_hi = (A & 0x0F0Fu) | ((B >> 2) & 0x3030u);
        const uint32_t m_hi = ((A >> 4) & 0x0F0Fu) | ((C >> 2) & 0x3030u);
        scp = g < 2 ? sc_lo : sc_hi;
        mp = g < 2 ? m_lo : m_hi;
    }
    static FO_DEV float finish(const uint4 &hdr, int g, float lo, float hi, const X &x) {
        uint32_t scp, mp;
        scales(hdr, g, scp, mp);
        const float d = h2f(hdr.x), dmin = h2f(hdr.x >> 16);
        const float acc = d * (ub0(scp) * lo + ub1(scp) * hi);
        return acc - dmin * (ub0(mp) * x.sum[0] + ub1(mp) * x.sum[1]);
    }
    static FO_DEV float dot(const Raw &r, int s, const X &x) {
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        int a0[kLimbs] = {}, a1[kLimbs] = {};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t lo = q[k] & 0x0F0F0F0Fu, hi = (q[k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int L = 0; L < kLimbs; L++) {
                a0[L] = dot4(lo, x.l[0][L][k], a0[L]);
                a1[L] = dot4(hi, x.l[1][L][k], a1[L]);
            }
        }
        return finish(r.hdr, s & 3, combine(a0) * x.sc[0], combine(a1) * x.sc[1], x);
    }
};

// ---------------------------------------------------------------- Q5_K
// As Q4_K plus qh: bit 2g of qh[l] is the fifth bit of value 64g+l and bit
// 2g+1 that of value 64g+32+l.
template <> struct Fmt<GGML_TYPE_Q5_K> {
    static constexpr int SLOT = 64, BLOCK = 176, NG = 2, GSZ = 32;
    using X = XSlot<NG, GSZ>;
    struct Raw { uint4 hdr, h0, h1, q0, q1; };

    static FO_DEV Raw load(const uint8_t *row, int s) {
        const uint8_t *b = row + (s >> 2) * BLOCK;
        const int g = s & 3;
        return Raw{ld16(b), ld16(b + 16), ld16(b + 32), ld16(b + 48 + 32 * g), ld16(b + 64 + 32 * g)};
    }
    static FO_DEV void groups(int s, int gi[NG]) { gi[0] = 2 * s; gi[1] = 2 * s + 1; }
    static FO_DEV float dot(const Raw &r, int s, const X &x) {
        const int g = s & 3;
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t h[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
        int a0[kLimbs] = {}, a1[kLimbs] = {};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t hb = h[k] >> (2 * g);
            const uint32_t lo = (q[k] & 0x0F0F0F0Fu) | ((hb << 4) & 0x10101010u);
            const uint32_t hi = ((q[k] >> 4) & 0x0F0F0F0Fu) | ((hb << 3) & 0x10101010u);
#pragma unroll
            for (int L = 0; L < kLimbs; L++) {
                a0[L] = dot4(lo, x.l[0][L][k], a0[L]);
                a1[L] = dot4(hi, x.l[1][L][k], a1[L]);
            }
        }
        return Fmt<GGML_TYPE_Q4_K>::finish(r.hdr, g, combine(a0) * x.sc[0], combine(a1) * x.sc[1], x);
    }
};

// ---------------------------------------------------------------- Q6_K
// Slot = (half n, l in [16j, 16j+16)) of super-block b: the 64 values
// 128n + 32t + l for t = 0..3, built from ql[64n+l] (t=0 low, t=2 high),
// ql[64n+32+l] (t=1 low, t=3 high) and bits 2t..2t+1 of qh[32n+l], with
// scales sc[8n + 2t + j]. Activation groups are the 16-value scale groups
// 16b + 8n + 2t + j. Super-blocks are 210 bytes, so these loads are only
// 2-byte aligned.
template <> struct Fmt<GGML_TYPE_Q6_K> {
    static constexpr int SLOT = 64, BLOCK = 210, NG = 4, GSZ = 16;
    using X = XSlot<NG, GSZ>;
    struct Raw { uint4 l0, l1, hh; uint2 sc; uint32_t d; };

    static FO_DEV Raw load(const uint8_t *row, int s) {
        const uint8_t *b = row + (s >> 2) * BLOCK;
        const int n = (s >> 1) & 1, j = s & 1;
        return Raw{ld16(b + 64 * n + 16 * j), ld16(b + 64 * n + 32 + 16 * j),
                   ld16(b + 128 + 32 * n + 16 * j), ld8(b + 192 + 8 * n), ld2(b + 208)};
    }
    static FO_DEV void groups(int s, int gi[NG]) {
        const int base = 16 * (s >> 2) + 8 * ((s >> 1) & 1) + (s & 1);
#pragma unroll
        for (int t = 0; t < NG; t++) gi[t] = base + 2 * t;
    }
    static FO_DEV float dot(const Raw &r, int s, const X &x) {
        const uint32_t L0[4] = {r.l0.x, r.l0.y, r.l0.z, r.l0.w};
        const uint32_t L1[4] = {r.l1.x, r.l1.y, r.l1.z, r.l1.w};
        const uint32_t H[4] = {r.hh.x, r.hh.y, r.hh.z, r.hh.w};
        int a[4][kLimbs] = {};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t q[4] = {
                (L0[k] & 0x0F0F0F0Fu) | ((H[k] << 4) & 0x30303030u),
                (L1[k] & 0x0F0F0F0Fu) | ((H[k] << 2) & 0x30303030u),
                ((L0[k] >> 4) & 0x0F0F0F0Fu) | (H[k] & 0x30303030u),
                ((L1[k] >> 4) & 0x0F0F0F0Fu) | ((H[k] >> 2) & 0x30303030u)};
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int L = 0; L < kLimbs; L++) a[t][L] = dot4(q[t], x.l[t][L][k], a[t][L]);
        }
        // signed scales sc[8n + 2t + j]: bytes j and 2+j of each dword of r.sc
        const int sh = 8 * (s & 1);
        const int s0 = (int)(r.sc.x << (24 - sh)) >> 24, s1 = (int)(r.sc.x << (8 - sh)) >> 24;
        const int s2 = (int)(r.sc.y << (24 - sh)) >> 24, s3 = (int)(r.sc.y << (8 - sh)) >> 24;
        float v = (float)s0 * fmaf(combine(a[0]), x.sc[0], -32.f * x.sum[0]);
        v = fmaf((float)s1, fmaf(combine(a[1]), x.sc[1], -32.f * x.sum[1]), v);
        v = fmaf((float)s2, fmaf(combine(a[2]), x.sc[2], -32.f * x.sum[2]), v);
        v = fmaf((float)s3, fmaf(combine(a[3]), x.sc[3], -32.f * x.sum[3]), v);
        return h2f(r.d) * v;
    }
};

// ---------------------------------------------------------------- Q8_0
// Slot = one 34-byte block: fp16 d + 32 int8 codes (activation group = block).
template <> struct Fmt<GGML_TYPE_Q8_0> {
    static constexpr int SLOT = 32, BLOCK = 34, NG = 1, GSZ = 32;
    using X = XSlot<NG, GSZ>;
    struct Raw { uint4 q0, q1; uint32_t d; };

    static FO_DEV Raw load(const uint8_t *row, int s) {
        const uint8_t *b = row + s * BLOCK;
        return Raw{ld16(b + 2), ld16(b + 18), ld2(b)};
    }
    static FO_DEV void groups(int s, int gi[NG]) { gi[0] = s; }
    static FO_DEV float dot(const Raw &r, int, const X &x) {
        const uint32_t q[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        int a[kLimbs] = {};
#pragma unroll
        for (int k = 0; k < 8; k++)
#pragma unroll
            for (int L = 0; L < kLimbs; L++) a[L] = dot4(q[k], x.l[0][L][k], a[L]);
        return h2f(r.d) * (combine(a) * x.sc[0]);
    }
};

// ---------------------------------------------------------------- MXFP4
// Slot = one 17-byte block: E8M0 exponent s + 32 E2M1 codes (low nibble of
// qs[j] is value j, high nibble value 16+j; reference src/quant.c:290-337).
// Codes are mapped to twice their value as int8 ({0,1,2,3,4,6,8,12} and
// negatives) through v_perm byte tables, so the block scale is 2^(s-128)
// (0 for s = 0xFF, as the reference).
template <> struct Fmt<GGML_TYPE_MXFP4> {
    static constexpr int SLOT = 32, BLOCK = 17, NG = 1, GSZ = 32;
    using X = XSlot<NG, GSZ>;
    struct Raw { uint4 q; uint32_t s; };

    static FO_DEV Raw load(const uint8_t *row, int s) {
        const uint8_t *b = row + s * BLOCK;
        return Raw{ld16(b + 1), ld2(b) & 0xFFu};
    }
    static FO_DEV void groups(int s, int gi[NG]) { gi[0] = s; }
    // four 4-bit codes (one per byte, 0..15) -> 2 * E2M1 value as int8
    static FO_DEV uint32_t e2m1x2(uint32_t c) {
        const uint32_t m = c & 0x07070707u;
        const uint32_t pos = __builtin_amdgcn_perm(0x0C080604u, 0x03020100u, m);
        const uint32_t neg = __builtin_amdgcn_perm(0xF4F8FAFCu, 0xFDFEFF00u, m);
        const uint32_t sgn = ((c >> 3) & 0x01010101u) * 0xFFu;
        return (neg & sgn) | (pos & ~sgn);
    }
    static FO_DEV float dot(const Raw &r, int, const X &x) {
        const uint32_t q[4] = {r.q.x, r.q.y, r.q.z, r.q.w};
        int a[kLimbs] = {};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t lo = e2m1x2(q[k] & 0x0F0F0F0Fu), hi = e2m1x2((q[k] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int L = 0; L < kLimbs; L++) {
                a[L] = dot4(lo, x.l[0][L][k], a[L]);
                a[L] = dot4(hi, x.l[0][L][k + 4], a[L]);
            }
        }
        const float scale = r.s == 0xFFu ? 0.f : ldexpf(1.0f, (int)r.s - 128);
        return scale * (combine(a) * x.sc[0]);
    }
};


}  // namespace fo
