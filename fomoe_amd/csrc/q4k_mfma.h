// q4k_mfma.h — one Q4_K super-block x 16 rows on v_mfma_i32_16x16x64_i8, the
// core of the tile-staged Q4_K matvec (k_matvec_q4k_mfma).
//
// A super-block is 8 sub-blocks of 32 values; byte qs[32c + l] holds value
// 64c + l (low nibble, sub-block 2c) and 64c + 32 + l (high nibble, sub-block
// 2c + 1) (reference src/quant.c:72-105 value order). The super-block runs as
// two MFMA pairs p = 0, 1. Lane (n = lane%16: weight row, g = lane/16) reads
// the 16 bytes qs[32(2p + (g>>1)) + 16(g&1) ..]: their low nibbles are its 16
// codes (B operand) of the pair's first MFMA, their high nibbles those of the
// second. The first MFMA then spans sub-blocks 4p (lane groups 0, 1) and 4p+2
// (groups 2, 3), the second 4p+1 and 4p+3. The A operand routes the three
// activation limbs of each sub-block to its own D rows: sub-block 4p to rows
// 0..2, 4p+2 to rows 4..6 (first MFMA), 4p+1 to rows 8..10 and 4p+3 to rows
// 12..14 (second MFMA, accumulated onto the first), so D lane (n, g) receives
// the three limb sums of row n's sub-block j = 4p + [0, 2, 1, 3][g] and
// applies its scale d*sc_j and min dmin*m_j itself.
#pragma once

#include "formats.h"

namespace fo {

typedef int v4i __attribute__((ext_vector_type(4)));

// Per-lane constants of the MFMA routing (see above).
struct Q4kLane {
    int jg;            // this lane's sub-block within a pair half: 0, 2, 1, 3 for g = 0..3
    uint32_t boff;     // byte offset of the lane's 16 code bytes in the super-block (pair 0)
    uint32_t aoff;     // A-operand offset in the prepared x of the super-block (valid lanes)
    bool valid1, valid2;
};

FO_DEV Q4kLane q4k_lane(int lane) {
    const int n = lane & 15, g = lane >> 4, mb = n >> 2, L = n & 3;
    Q4kLane q;
    q.jg = ((g & 1) << 1) | (g >> 1);
    q.boff = 16 + 32 * (g >> 1) + 16 * (g & 1);
    // A row n = 4 mb + L: limb L of group 2 (mb & 1) + (mb >> 1) of the pair
    q.aoff = (uint32_t)(2 * (mb & 1) + (mb >> 1)) * 96 + 32 * L + 16 * (g & 1);
    q.valid1 = mb == (g >> 1) && L < 3;
    q.valid2 = mb == 2 + (g >> 1) && L < 3;
    return q;
}

// sb: row n's super-block in LDS (16-byte aligned); a1 / a2: the lane's A
// operands of this super-block's first / second MFMAs for pair 0 (pair 1 at
// +384), or a zero area of at least 400 bytes; ssb: {scale, sum} of the
// lane's pair-0 group (pair 1 at +32). Adds the lane's share of
// d * sum_j sc_j (q . x)_j - dmin * sum_j m_j (sum x)_j to y (in float: the
// limb combination rounds once, as the slot dots' does; in double: exact up
// to the accumulation).
template <typename Acc>   // float, or double where a layer's parity margin needs it
FO_DEV Acc q4k_sb_dot_mfma(const uint8_t *sb, const uint8_t *a1, const uint8_t *a2, const uint8_t *ssb,
                           const Q4kLane &q, Acc y) {
    const uint4 hdr = *(const uint4 *)sb;
    const uint4 c0 = *(const uint4 *)(sb + q.boff);
    const uint4 c1 = *(const uint4 *)(sb + q.boff + 64);
    // 6-bit scale / min of sub-blocks jg and 4 + jg (reference src/quant.c:72-80)
    const uint32_t sh = 8 * q.jg;
    const uint32_t b0 = (hdr.y >> sh) & 0xFFu, b4 = (hdr.z >> sh) & 0xFFu, b8 = (hdr.w >> sh) & 0xFFu;
    const float d = h2f(hdr.x), dmin = h2f(hdr.x >> 16);
    const float sc[2] = {d * (float)(b0 & 63), d * (float)((b8 & 0xF) | ((b0 >> 6) << 4))};
    const float mn[2] = {dmin * (float)(b4 & 63), dmin * (float)((b8 >> 4) | ((b4 >> 6) << 4))};
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const uint4 w = p ? c1 : c0;
        const v4i lo = {(int)(w.x & 0x0F0F0F0Fu), (int)(w.y & 0x0F0F0F0Fu), (int)(w.z & 0x0F0F0F0Fu),
                        (int)(w.w & 0x0F0F0F0Fu)};
        const v4i hi = {(int)((w.x >> 4) & 0x0F0F0F0Fu), (int)((w.y >> 4) & 0x0F0F0F0Fu),
                        (int)((w.z >> 4) & 0x0F0F0F0Fu), (int)((w.w >> 4) & 0x0F0F0F0Fu)};
        const v4i A1 = *(const v4i *)(a1 + 384 * p);
        const v4i A2 = *(const v4i *)(a2 + 384 * p);
        v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, lo, (v4i){0, 0, 0, 0}, 0, 0, 0);
        D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A2, hi, D, 0, 0, 0);
        // limb sums of a 32-value sub-block: |D| < 2^16, so D2 * 256 + D1 is exact in fp32
        // (the whole limb combination is exact in fp64); d * sc and dmin * m are exact
        const Acc f = (Acc)((D[2] << 8) + D[1]) * (Acc)256 + (Acc)D[0];
        const float2 ss = *(const float2 *)(ssb + 32 * p);
        y = fma((Acc)sc[p], f * (Acc)ss.x, y);
        y = fma(-(Acc)mn[p], (Acc)ss.y, y);
    }
    return y;
}

// Q5_K super-block (176 bytes: header, qh[32], qs[128]; reference
// src/quant.c:216-262): as Q4_K with a fifth bit per value, bit 2c of qh[l]
// for value 64c + l and bit 2c+1 for value 64c + 32 + l (c = 0..3). The lane
// reads the qh bytes of its 16 code positions (qh[16(g&1) ..]) next to the
// code bytes; the code routing and the per-sub-block scaling are Q4_K's.
FO_DEV float q5k_sb_dot_mfma(const uint8_t *sb, const uint8_t *a1, const uint8_t *a2, const uint8_t *ssb,
                             const Q4kLane &q, int g, float y) {
    const uint4 hdr = *(const uint4 *)sb;
    const uint4 hb = *(const uint4 *)(sb + 16 + 16 * (g & 1));
    const uint4 c0 = *(const uint4 *)(sb + 32 + q.boff);
    const uint4 c1 = *(const uint4 *)(sb + 32 + q.boff + 64);
    const uint32_t sh = 8 * q.jg;
    const uint32_t b0 = (hdr.y >> sh) & 0xFFu, b4 = (hdr.z >> sh) & 0xFFu, b8 = (hdr.w >> sh) & 0xFFu;
    const float d = h2f(hdr.x), dmin = h2f(hdr.x >> 16);
    const float sc[2] = {d * (float)(b0 & 63), d * (float)((b8 & 0xF) | ((b0 >> 6) << 4))};
    const float mn[2] = {dmin * (float)(b4 & 63), dmin * (float)((b8 >> 4) | ((b4 >> 6) << 4))};
    const uint32_t H[4] = {hb.x, hb.y, hb.z, hb.w};
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const uint4 w = p ? c1 : c0;
        const uint32_t W[4] = {w.x, w.y, w.z, w.w};
        const int c = 2 * p + (g >> 1);               // the 64-value chunk of these code bytes
        v4i lo, hi;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t hl = (H[k] >> (2 * c)) & 0x01010101u, hh = (H[k] >> (2 * c + 1)) & 0x01010101u;
            lo[k] = (int)((W[k] & 0x0F0F0F0Fu) | (hl << 4));
            hi[k] = (int)(((W[k] >> 4) & 0x0F0F0F0Fu) | (hh << 4));
        }
        const v4i A1 = *(const v4i *)(a1 + 384 * p);
        const v4i A2 = *(const v4i *)(a2 + 384 * p);
        v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, lo, (v4i){0, 0, 0, 0}, 0, 0, 0);
        D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A2, hi, D, 0, 0, 0);
        const float f = fmaf((float)((D[2] << 8) + D[1]), 256.f, (float)D[0]);
        const float2 ss = *(const float2 *)(ssb + 32 * p);
        y = fmaf(sc[p], f * ss.x, y);
        y = fmaf(-mn[p], ss.y, y);
    }
    return y;
}

}  // namespace fo
