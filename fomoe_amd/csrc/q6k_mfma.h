// q6k_mfma.h — one Q6_K super-block x 16 rows on v_mfma_i32_16x16x64_i8, the
// core of the tile-staged Q6_K matvec (k_matvec_q6k_tile).
//
// Lane (r = lane%16, g = lane/16), n = g>>1, j = g&1 owns slot (n, j) of row r:
// the 64 values 128n + 32t + l, l in [16j, 16j+16), t = 0..3 (reference
// src/quant.c:147-175 value order). For each t the 16 codes of lane group g
// form the MFMA B operand (column = weight row r). The A operand routes the
// three activation limbs so that A rows 4g..4g+2 are nonzero only over lane
// group g's k-range and hold limb 0..2 of activation group 16b + 8n + 2t + j
// (lanes of other rows read a 16-byte zero slot instead). D layout: lane holds rows
// 4*(lane/16)+i of column lane%16, i.e. lane (r, g) receives the three limb
// sums of its own row's 16-value scale group, to which it applies the group
// scale and offset and the sub-block scale sc[8n + 2t + j] itself.
#pragma once

#include "formats.h"

namespace fo {

typedef int v4i __attribute__((ext_vector_type(4)));

// sb: this row's super-block (any alignment, LDS or global); abase / ssb: the
// lane's A-operand / {scale, sum} base for group offset 0; zero16: 16 zero
// bytes, read instead when !valid; g0 = 16 * (index of the super-block in the
// row). Returns the lane's partial of d * sum.
FO_DEV float q6k_sb_dot_mfma(const uint8_t *sb, const uint8_t *abase, const uint8_t *ssb, int g0, int n,
                             int j, bool valid, const uint8_t *zero16) {
    uint4 l0, l1, hh;
    uint2 scb;
    uint16_t d16;
    __builtin_memcpy(&l0, sb + 64 * n + 16 * j, 16);
    __builtin_memcpy(&l1, sb + 64 * n + 32 + 16 * j, 16);
    __builtin_memcpy(&hh, sb + 128 + 32 * n + 16 * j, 16);
    __builtin_memcpy(&scb, sb + 192 + 8 * n, 8);
    __builtin_memcpy(&d16, sb + 208, 2);
    const uint32_t Lo[4] = {l0.x, l0.y, l0.z, l0.w};
    const uint32_t Hi[4] = {l1.x, l1.y, l1.z, l1.w};
    const uint32_t H[4] = {hh.x, hh.y, hh.z, hh.w};
    float accb = 0.f;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        v4i B;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            uint32_t q;
            if (t == 0) q = (Lo[k] & 0x0F0F0F0Fu) | ((H[k] << 4) & 0x30303030u);
            else if (t == 1) q = (Hi[k] & 0x0F0F0F0Fu) | ((H[k] << 2) & 0x30303030u);
            else if (t == 2) q = ((Lo[k] >> 4) & 0x0F0F0F0Fu) | (H[k] & 0x30303030u);
            else q = ((Hi[k] >> 4) & 0x0F0F0F0Fu) | ((H[k] >> 2) & 0x30303030u);
            B[k] = (int)q;
        }
        const int go = g0 + 2 * t;                        // group g0 + 8n + 2t + j
        const v4i A = *(const v4i *)(valid ? abase + go * 48 : zero16);
        const v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, (v4i){0, 0, 0, 0}, 0, 0, 0);
        const float f = fmaf(fmaf((float)D[2], 256.f, (float)D[1]), 256.f, (float)D[0]);
        const float2 ss = *(const float2 *)(ssb + go * 8);
        const float vv = fmaf(f, ss.x, -32.f * ss.y);
        const uint32_t sw = (t < 2) ? scb.x : scb.y;       // sc[8n + 2t + j]
        const int scv = (int)(sw << (24 - 8 * (2 * (t & 1) + j))) >> 24;
        accb = fmaf((float)scv, vv, accb);
    }
    return h2f(d16) * accb;
}

}  // namespace fo
