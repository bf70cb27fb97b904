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
// K*3 bytes of int8 limbs (three per value) plus K/gsz float2 {scale, sum}.
__host__ __device__ constexpr int gsz_of(int type) { return type == GGML_TYPE_Q6_K ? 16 : 32; }
__host__ __device__ constexpr uint64_t xq_limb_bytes(int K) { return (uint64_t)K * 3; }
__host__ __device__ constexpr uint64_t xq_bytes(int K, int gsz) {
    return xq_limb_bytes(K) + (uint64_t)(K / gsz) * 8;
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

// Streaming weight loads (global memory only): every weight byte is read once
// per call, so they carry the non-temporal hint (global_load_* nt). Measured on
// MI355X: a pure 1.77 GB read sustains 7.1 TB/s with nt loads against 6.3 TB/s
// with plain ones. The pointer may be only 2-byte aligned (gfx950 runs in
// unaligned-access mode); never use these on LDS addresses.
typedef uint32_t fo_u32x4a __attribute__((ext_vector_type(4)));
typedef fo_u32x4a fo_u32x4 __attribute__((aligned(1)));   // no alignment promised
FO_DEV uint4 ldw16(const uint8_t *p) {
    const fo_u32x4 t = __builtin_nontemporal_load((const fo_u32x4 *)p);
    return make_uint4(t.x, t.y, t.z, t.w);
}
// Only loads that stream whole cache lines take the hint (the 1 KiB tile
// pieces): the per-lane slot loads of the format decoders read several 16-byte
// pieces of one line from different instructions, and with nt the line is gone
// before the later ones arrive (Q4_K slot matvec: 5.4 -> 4.4 TB/s measured).

// Stage nbytes (a multiple of 16) from global memory into LDS with gfx950's
// direct global->LDS loads (global_load_lds_dwordx4): every wave streams
// 1 KiB pieces, all in flight at once, no VGPRs. The LDS buffer must have room
// up to the next multiple of 1 KiB (the last piece's spare lanes re-read the
// final 16 bytes into that padding). Completion: s_waitcnt vmcnt(0) and a
// barrier, see stage_lds_wait().
FO_DEV void stage_lds(uint8_t *lds_dst, const uint8_t *g, uint32_t nbytes, int wave, int nwaves) {
    const int lane = threadIdx.x & 63;
    for (uint32_t off = (uint32_t)wave * 1024u; off < nbytes; off += (uint32_t)nwaves * 1024u) {
        const uint32_t o = off + (uint32_t)lane * 16u;
        const uint8_t *src = g + (o + 16u <= nbytes ? o : nbytes - 16u);
        __builtin_amdgcn_global_load_lds((const void *)src,
                                         (__attribute__((address_space(3))) void *)(lds_dst + off), 16, 0, 0);
    }
}
// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector-memory
// operations of this wave are outstanding and ignores the other counters.
__host__ __device__ constexpr int vmcnt_le(int n) {
    return (n & 0xF) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8);
}
FO_DEV void stage_lds_wait() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}
// LDS byte address of a pointer into this work-group's LDS.
FO_DEV uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// Direct global->LDS loads (lane l's 16 / 4 bytes land at lds_base + 16 l /
// 4 l; lds_base wave-uniform) issued as inline assembly, so that the compiler
// does not track them: once it knows of an outstanding direct-to-LDS load it
// makes every later LDS read wait for all outstanding loads (vmcnt(0)), which
// serialises a prefetch of the next step with the arithmetic on the current
// one. The caller waits for them itself (s_waitcnt vmcnt, counting the loads
// issued after them); the compiler's own waits for later loads stay correct
// because these are older.
FO_DEV void dma16_untracked(const void *g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off"
                 :: "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_base)) : "memory", "m0");
}
FO_DEV void dma16_untracked_nt(const void *g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :: "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_base)) : "memory", "m0");
}
FO_DEV void dma4_untracked(const void *g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
                 :: "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_base)) : "memory", "m0");
}

// Work-group barrier that orders LDS only: outstanding global loads stay in
// flight (the compiler's LDS fence also waits for them once a direct-to-LDS
// load has been issued). The clobber keeps memory accesses on their side.
FO_DEV void wg_sync_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__host__ __device__ constexpr uint32_t lds_round(uint64_t n) { return (uint32_t)((n + 1023) & ~(uint64_t)1023); }

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
// DPP lane exchanges (gfx9 encodings): quad_perm [1,0,3,2] 0xB1 and
// [2,3,0,1] 0x4E, row_half_mirror 0x141 (lane i <-> 7-i within 8), row_mirror
// 0x140 (lane i <-> 15-i within 16).
template <int CTRL>
FO_DEV float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over groups of G consecutive lanes (G a power of two <= 64); every lane
// of the group receives the group sum. Butterflies inside quads, then the
// 8- and 16-lane mirrors (all DPP, no LDS round trip); 32/64 use permutes.
template <int G>
FO_DEV float group_sum(float v) {
    if (G >= 2) v += dpp<0xB1>(v);
    if (G >= 4) v += dpp<0x4E>(v);
    if (G >= 8) v += dpp<0x141>(v);
    if (G >= 16) v += dpp<0x140>(v);
    if (G >= 32) v += __shfl_xor(v, 16, kWave);
    if (G >= 64) v += __shfl_xor(v, 32, kWave);
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
