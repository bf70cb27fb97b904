// q6k_mfma.h — one Q6_K super-block x 16 rows on v_mfma_i32_16x16x64_i8, the
// core of the tile-staged Q6_K matvec (k_matvec_q6k_tile).
//
// Lane (r = lane%16, g = lane/16), n = g>>1, j = g&1 owns slot (n, j) of row r:
// the 64 values 128n + 32t + l, l in [16j, 16j+16), t = 0..3 (reference
// src/quant.c:147-175 value order). For each t the 16 codes of lane group g
// form the MFMA B operand (column = weight row r). The A operand routes the
// three activation limbs so that A rows 4g..4g+2 are nonzero only over lane
// group g's k-range and hold limb 0..2 of activation group 16b + 8n + 2t + j
// (lanes of other rows read zeros instead). D layout: lane holds rows
// 4*(lane/16)+i of column lane%16, i.e. lane (r, g) receives the three limb
// sums of its own row's 16-value scale group, to which it applies the group
// scale and offset and the sub-block scale sc[8n + 2t + j] itself.
#pragma once

#include "formats.h"

namespace fo {

typedef int v4i __attribute__((ext_vector_type(4)));

// The lane's bytes of one super-block: ql pieces for t = 0, 2 (lo) and t = 1,
// 3 (hi), the qh piece, the scale pair words of half n and d.
struct Q6kSlot {
    uint4 lo, hi, h;
    uint2 sc;
    uint16_t d;
};

FO_DEV void q6k_slot_load(Q6kSlot &q, const uint8_t *sb, int n, int j) {
    __builtin_memcpy(&q.lo, sb + 64 * n + 16 * j, 16);
    __builtin_memcpy(&q.hi, sb + 64 * n + 32 + 16 * j, 16);
    __builtin_memcpy(&q.h, sb + 128 + 32 * n + 16 * j, 16);
    __builtin_memcpy(&q.sc, sb + 192 + 8 * n, 8);
    __builtin_memcpy(&q.d, sb + 208, 2);
}

// q: the lane's slot bytes (q6k_slot_load); a: the lane's A operand for t = 0
// of this super-block, the operand of t at a + 96 t (a zero area of 304 bytes
// for lanes that carry no limb); ssb: {scale, -32 * sum} of the lane's t = 0
// group, t at ssb + 16 t. Returns the lane's partial of d * sum. The limb
// combination (D2 * 256 + D1 as an exact integer, one rounding to fp32, then
// * 256 + D0 in one fma) rounds exactly as a nested fma of the three exact
// fp32 limb sums would.
FO_DEV float q6k_sb_dot_mfma(const Q6kSlot &q, const uint8_t *a, const uint8_t *ssb, int j) {
    const uint32_t Lo[4] = {q.lo.x, q.lo.y, q.lo.z, q.lo.w};
    const uint32_t Hi[4] = {q.hi.x, q.hi.y, q.hi.z, q.hi.w};
    const uint32_t H[4] = {q.h.x, q.h.y, q.h.z, q.h.w};
    // sc[8n + 2t + j]: byte 0 / byte 2 of the pair word shifted by j
    const uint32_t s01 = q.sc.x >> (8 * j), s23 = q.sc.y >> (8 * j);
    float accb = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        v4i B;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t c;
            if (t == 0) c = (Lo[k] & 0x0F0F0F0Fu) | ((H[k] << 4) & 0x30303030u);
            else if (t == 1) c = (Hi[k] & 0x0F0F0F0Fu) | ((H[k] << 2) & 0x30303030u);
            else if (t == 2) c = ((Lo[k] >> 4) & 0x0F0F0F0Fu) | (H[k] & 0x30303030u);
            else c = ((Hi[k] >> 4) & 0x0F0F0F0Fu) | ((H[k] >> 2) & 0x30303030u);
            B[k] = (int)c;
        }
        const v4i A = *(const v4i *)(a + 96 * t);
        const v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, (v4i){0, 0, 0, 0}, 0, 0, 0);
        const float f = fmaf((float)((D[2] << 8) + D[1]), 256.f, (float)D[0]);
        const float2 ss = *(const float2 *)(ssb + 16 * t);
        const float vv = fmaf(f, ss.x, ss.y);
        const uint32_t sw = (t < 2) ? s01 : s23;
        const float scv = (float)(int8_t)(sw >> (16 * (t & 1)));
        accb = fmaf(scv, vv, accb);
    }
    return h2f(q.d) * accb;
}

}  // namespace fo
