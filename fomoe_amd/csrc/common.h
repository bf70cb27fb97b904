// common.h — device helpers shared by the gfx950 kernels of libfomoe_gfx950.
//
// Wave64 throughout: every reduction below assumes warpSize == 64 (CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "quant_types.h"

#define FO_DEV __device__ __forceinline__

namespace fo {

constexpr int kWave = 64;

// Prepared-activation layout (see formats.h): K values in groups of gsz take
// K*4 bytes of int8 limbs plus K/gsz float2 {scale, sum}.
__host__ __device__ constexpr int gsz_of(int type) { return type == GGML_TYPE_Q6_K ? 16 : 32; }
__host__ __device__ constexpr uint64_t xq_bytes(int K, int gsz) {
    return (uint64_t)K * 4 + (uint64_t)(K / gsz) * 8;
}
// Per-vector stride of a prepared batch, rounded to 256 bytes.
__host__ __device__ constexpr uint64_t xq_stride(int K, int gsz) {
    return (xq_bytes(K, gsz) + 255) & ~(uint64_t)255;
}

// ---------------------------------------------------------------- loads
// Unaligned-tolerant vector loads. gfx950 runs in unaligned-access mode, so a
// 16-byte load from a 2-byte-aligned Q6_K/Q8_0 field is one global_load_dwordx4.
FO_DEV uint4 ld16(const uint8_t *p) { uint4 v; __builtin_memcpy(&v, p, 16); return v; }
FO_DEV uint2 ld8(const uint8_t *p) { uint2 v; __builtin_memcpy(&v, p, 8); return v; }
FO_DEV uint32_t ld4(const uint8_t *p) { uint32_t v; __builtin_memcpy(&v, p, 4); return v; }
FO_DEV uint32_t ld2(const uint8_t *p) { uint16_t v; __builtin_memcpy(&v, p, 2); return v; }

// Streaming weight loads: every weight byte is read exactly once per call, so
// mark them non-temporal to keep activations resident in L2/MALL.
FO_DEV uint4 ld16_stream(const uint8_t *p) {
    uint4 v;
    v.x = __builtin_nontemporal_load((const uint32_t *)p + 0);
    v.y = __builtin_nontemporal_load((const uint32_t *)p + 1);
    v.z = __builtin_nontemporal_load((const uint32_t *)p + 2);
    v.w = __builtin_nontemporal_load((const uint32_t *)p + 3);
    return v;
}

// fp16 bits -> fp32 (exact; hardware conversion handles subnormals, inf, NaN)
FO_DEV float h2f(uint32_t bits16) {
    return __half2float(__ushort_as_half((unsigned short)(bits16 & 0xFFFFu)));
}

// byte n of a dword as float (v_cvt_f32_ubyteN)
FO_DEV float ub0(uint32_t v) { return (float)(v & 0xFFu); }
FO_DEV float ub1(uint32_t v) { return (float)((v >> 8) & 0xFFu); }
FO_DEV float ub2(uint32_t v) { return (float)((v >> 16) & 0xFFu); }
FO_DEV float ub3(uint32_t v) { return (float)(v >> 24); }

// ---------------------------------------------------------- reductions
// Sum over groups of G consecutive lanes (G a power of two <= 64); every lane
// of the group receives the group sum.
template <int G>
FO_DEV float group_sum(float v) {
#pragma unroll
    for (int o = G / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

FO_DEV float wave_sum(float v) { return group_sum<kWave>(v); }

FO_DEV float wave_max(float v) {
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}

FO_DEV float silu(float g) { return g / (1.0f + __expf(-g)); }

}  // namespace fo
