// synth.hip — synthetic weights and activations generated in HBM.
//
// This is the build's own data definition (the reference ships no quantizer):
// counter-based SplitMix64 normals via Box-Muller evaluated in float64 with
// +,-,* only (series and fixed Newton steps), then this build's Q4_K / Q5_K /
// Q6_K / Q8_0 quantizers. Every operation is an IEEE basic operation with FMA
// contraction disabled, so the bits equal the CPU generator in oracle/oracle.c
// (the tests compare them on sampled matrices). One wave quantizes one run of
// 256 values: lane l holds values 4l..4l+3 and sub-block statistics are wave
// reductions (min/max are exact in any order).
#include "common.h"
#include "kernels.h"

namespace fo {

#define GOLDEN 0x9E3779B97F4A7C15ull

FO_DEV uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__host__ __device__ inline uint64_t mix64_hd(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__host__ __device__ inline uint64_t rng_key(uint64_t seed, uint64_t stream) {
    return mix64_hd(seed * GOLDEN + mix64_hd(stream + 0x632BE59BD9B4E019ull));
}
FO_DEV uint64_t rng_u64(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * GOLDEN); }

FO_DEV double recip_newton(double a) {
#pragma clang fp contract(off)
    double r = 0.4;
#pragma unroll
    for (int i = 0; i < 6; i++) r = r * (2.0 - a * r);
    return r;
}

FO_DEV double ln_det(double u) {
#pragma clang fp contract(off)
    const uint64_t b = (uint64_t)__double_as_longlong(u);
    int e = (int)((b >> 52) & 0x7FF) - 1023;
    double m = __longlong_as_double((long long)((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull));
    if (m > 0x1.6a09e667f3bcdp+0) { m = m * 0.5; e += 1; }
    const double s = (m - 1.0) * recip_newton(m + 1.0);
    const double s2 = s * s;
    const double c[13] = {
        0x1.0000000000000p+0, 0x1.5555555555555p-2, 0x1.999999999999ap-3, 0x1.2492492492492p-3,
        0x1.c71c71c71c71cp-4, 0x1.745d1745d1746p-4, 0x1.3b13b13b13b14p-4, 0x1.1111111111111p-4,
        0x1.e1e1e1e1e1e1ep-5, 0x1.af286bca1af28p-5, 0x1.8618618618618p-5, 0x1.642c8590b2164p-5,
        0x1.47ae147ae147bp-5};
    double p = c[12];
#pragma unroll
    for (int i = 11; i >= 0; i--) p = p * s2 + c[i];
    return (double)e * 0x1.62e42fefa39efp-1 + 2.0 * s * p;
}

FO_DEV void sincos_det(double phi, double *sn, double *cs) {
#pragma clang fp contract(off)
    const double ks[13] = {
        0x1.0000000000000p+0, -0x1.5555555555555p-3, 0x1.1111111111111p-7, -0x1.a01a01a01a01ap-13,
        0x1.71de3a556c734p-19, -0x1.ae64567f544e4p-26, 0x1.6124613a86d09p-33, -0x1.ae7f3e733b81fp-41,
        0x1.952c77030ad4ap-49, -0x1.2f49b46814157p-57, 0x1.71b8ef6dcf572p-66, -0x1.761b41316381ap-75,
        0x1.3f3ccdd165fa9p-84};
    const double kc[14] = {
        0x1.0000000000000p+0, -0x1.0000000000000p-1, 0x1.5555555555555p-5, -0x1.6c16c16c16c17p-10,
        0x1.a01a01a01a01ap-16, -0x1.27e4fb7789f5cp-22, 0x1.1eed8eff8d898p-29, -0x1.93974a8c07c9dp-37,
        0x1.ae7f3e733b81fp-45, -0x1.6827863b97d97p-53, 0x1.e542ba4020225p-62, -0x1.0ce396db7f853p-70,
        0x1.f2cf01972f578p-80, -0x1.88e85fc6a4e5ap-89};
    const double p2 = phi * phi;
    double s = ks[12], c = kc[13];
#pragma unroll
    for (int i = 11; i >= 0; i--) s = s * p2 + ks[i];
#pragma unroll
    for (int i = 12; i >= 0; i--) c = c * p2 + kc[i];
    *sn = s * phi;
    *cs = c;
}

FO_DEV double sqrt_det(double v) {
#pragma clang fp contract(off)
    if (v == 0.0) return 0.0;
    double y = __longlong_as_double((long long)(0x5FE6EB50C7B537A9ull - ((uint64_t)__double_as_longlong(v) >> 1)));
#pragma unroll
    for (int i = 0; i < 5; i++) y = y * (1.5 - 0.5 * v * y * y);
    return v * y;
}

// Both normals of Box-Muller pair j: values 2j (cos) and 2j+1 (sin).
FO_DEV void normal_pair(uint64_t key, uint64_t j, float &z0, float &z1) {
#pragma clang fp contract(off)
    const uint64_t r1 = rng_u64(key, 2 * j), r2 = rng_u64(key, 2 * j + 1);
    const double u1 = (double)((r1 >> 11) + 1) * 0x1p-53;
    const double t = (double)(r2 >> 11) * 0x1p-51;
    const int q = (int)t;
    const double phi = (t - (double)q) * 0x1.921fb54442d18p+0;
    const double rad = sqrt_det(-2.0 * ln_det(u1));
    double s, c, cq, sq;
    sincos_det(phi, &s, &c);
    switch (q) {
        case 0: cq = c; sq = s; break;
        case 1: cq = -s; sq = c; break;
        case 2: cq = -c; sq = -s; break;
        default: cq = s; sq = -c; break;
    }
    z0 = (float)(rad * cq);
    z1 = (float)(rad * sq);
}

__global__ __launch_bounds__(256) void k_synth_f32(uint64_t key, float std, float *out, int64_t n) {
#pragma clang fp contract(off)
    const int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (2 * j >= n) return;
    float z0, z1;
    normal_pair(key, (uint64_t)j, z0, z1);
    out[2 * j] = std * z0;
    if (2 * j + 1 < n) out[2 * j + 1] = std * z1;
}

FO_DEV int nearest_clamp(float v, int lo, int hi) {
    const float r = floorf(v + 0.5f);
    if (!(r >= (float)lo)) return lo;
    if (r > (float)hi) return hi;
    return (int)r;
}

FO_DEV uint32_t f2h_bits(float f) { return (uint32_t)__half_as_ushort(__float2half_rn(f)); }

template <int G> FO_DEV float gmin(float v) {
#pragma unroll
    for (int o = 1; o < G; o <<= 1) v = fminf(v, __shfl_xor(v, o, 64));
    return v;
}
template <int G> FO_DEV float gmax(float v) {
#pragma unroll
    for (int o = 1; o < G; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
// max over lanes l, l^G, l^2G, ... (across sub-blocks of G lanes)
template <int G> FO_DEV float xmax(float v) {
#pragma unroll
    for (int o = G; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

FO_DEV void st4(uint8_t *p, uint32_t v) { __builtin_memcpy(p, &v, 4); }
FO_DEV void st2(uint8_t *p, uint32_t v) { uint16_t h = (uint16_t)v; __builtin_memcpy(p, &h, 2); }

// Q4_K (NB = 4) / Q5_K (NB = 5) super-block from the wave's 256 values:
// per 32-value sub-block scale (max-min)/L and min -min(0,min); d and dmin
// are max/63 rounded to fp16; 6-bit sub-scales; codes round((x+dmin*m)/(d*sc)).
template <int NB>
FO_DEV void quant_kq(const float v[4], int lane, uint8_t *blk) {
#pragma clang fp contract(off)
    const float L = (float)((1 << NB) - 1);
    float mn = fminf(fminf(v[0], v[1]), fminf(v[2], v[3]));
    float mx = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
    mn = gmin<8>(mn);
    mx = gmax<8>(mx);
    if (mn > 0.0f) mn = 0.0f;
    const float sc_f = (mx - mn) / L, mn_f = -mn;
    const float max_sc = xmax<8>(sc_f), max_mn = xmax<8>(mn_f);
    const uint32_t dh = f2h_bits(max_sc / 63.0f), dmh = f2h_bits(max_mn / 63.0f);
    const float df = h2f(dh), dmf = h2f(dmh);
    const int sc = df > 0.0f ? nearest_clamp(sc_f / df, 0, 63) : 0;
    const int m = dmf > 0.0f ? nearest_clamp(mn_f / dmf, 0, 63) : 0;
    const float ds = df * (float)sc, dm = dmf * (float)m;
    uint32_t c[4];
#pragma unroll
    for (int i = 0; i < 4; i++) c[i] = ds > 0.0f ? (uint32_t)nearest_clamp((v[i] + dm) / ds, 0, (int)L) : 0u;
    // scales of sub-blocks j = 0..7 live in lanes 8j
    int scj[8], mj[8];
#pragma unroll
    for (int j = 0; j < 8; j++) { scj[j] = __shfl(sc, 8 * j, 64); mj[j] = __shfl(m, 8 * j, 64); }
    // codes of value +32 (high nibble partner) live 8 lanes up
    uint32_t hc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) hc[i] = (uint32_t)__shfl_down((int)c[i], 8, 64);
    const int g = lane >> 4, r = lane & 15;
    if (NB == 4) {
        if (r < 8) {
            uint32_t w = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) w |= (c[i] | (hc[i] << 4)) << (8 * i);
            st4(blk + 16 + 32 * g + 4 * r, w);
        }
    } else {
        if (r < 8) {
            uint32_t w = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) w |= ((c[i] & 0xF) | ((hc[i] & 0xF) << 4)) << (8 * i);
            st4(blk + 48 + 32 * g + 4 * r, w);
        }
        // qh byte l collects bit 4 of the codes of value 64g+l (bit 2g) and
        // 64g+32+l (bit 2g+1) for all g: lane k (< 8) gathers dword k
        uint32_t qh = 0;
#pragma unroll
        for (int gg = 0; gg < 4; gg++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t lo = (uint32_t)__shfl((int)c[i], 16 * gg + (lane & 7), 64);
                const uint32_t hi = (uint32_t)__shfl((int)c[i], 16 * gg + 8 + (lane & 7), 64);
                qh |= (((lo >> 4) << (2 * gg)) | ((hi >> 4) << (2 * gg + 1))) << (8 * i);
            }
        }
        if (lane < 8) st4(blk + 16 + 4 * lane, qh);
    }
    if (lane == 0) {
        uint8_t s[12];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            s[j] = (uint8_t)((scj[j] & 63) | ((scj[j + 4] >> 4) << 6));
            s[j + 4] = (uint8_t)((mj[j] & 63) | ((mj[j + 4] >> 4) << 6));
            s[j + 8] = (uint8_t)((scj[j + 4] & 0xF) | ((mj[j + 4] & 0xF) << 4));
        }
        st2(blk, dh);
        st2(blk + 2, dmh);
#pragma unroll
        for (int j = 0; j < 12; j++) blk[4 + j] = s[j];
    }
}

// Q6_K super-block: per 16-value sub-block scale amax/31, d = max/127 in
// fp16, signed 8-bit sub-scales, codes round(x/(d*sc)) in [-32, 31] + 32.
FO_DEV void quant_q6(const float v[4], int lane, uint8_t *blk) {
#pragma clang fp contract(off)
    float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    a = gmax<4>(a);
    const float s_f = a / 31.0f;
    const float max_s = xmax<4>(s_f);
    const uint32_t dh = f2h_bits(max_s / 127.0f);
    const float df = h2f(dh);
    const int sc = df > 0.0f ? nearest_clamp(s_f / df, -128, 127) : 0;
    const float ds = df * (float)sc;
    uint32_t u[4];
#pragma unroll
    for (int i = 0; i < 4; i++) u[i] = (uint32_t)((ds > 0.0f ? nearest_clamp(v[i] / ds, -32, 31) : 0) + 32);
    // lane L: n = L/32, t = (L%32)/8, l = 4(L%8) + i; t=0 lanes gather t=1..3
    uint32_t q2[4], q3[4], q4[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        q2[i] = (uint32_t)__shfl_down((int)u[i], 8, 64);
        q3[i] = (uint32_t)__shfl_down((int)u[i], 16, 64);
        q4[i] = (uint32_t)__shfl_down((int)u[i], 24, 64);
    }
    int scs[16];
#pragma unroll
    for (int s = 0; s < 16; s++) scs[s] = __shfl(sc, 4 * s, 64);
    const int n = lane >> 5, tl = (lane & 31) >> 3, l4 = 4 * (lane & 7);
    if (tl == 0) {
        uint32_t a0 = 0, a1 = 0, h = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t q1 = u[i];
            a0 |= ((q1 & 0xF) | ((q3[i] & 0xF) << 4)) << (8 * i);
            a1 |= ((q2[i] & 0xF) | ((q4[i] & 0xF) << 4)) << (8 * i);
            h |= ((q1 >> 4) | ((q2[i] >> 4) << 2) | ((q3[i] >> 4) << 4) | ((q4[i] >> 4) << 6)) << (8 * i);
        }
        st4(blk + 64 * n + l4, a0);
        st4(blk + 64 * n + 32 + l4, a1);
        st4(blk + 128 + 32 * n + l4, h);
    }
    if (lane == 0) {
#pragma unroll
        for (int s = 0; s < 16; s++) blk[192 + s] = (uint8_t)(int8_t)scs[s];
        st2(blk + 208, dh);
    }
}

// Q8_0: eight 32-value blocks per wave; d = amax/127 in fp16, codes round(x/d).
FO_DEV void quant_q8_0(const float v[4], int lane, uint8_t *run) {
#pragma clang fp contract(off)
    float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
    a = gmax<8>(a);
    const uint32_t dh = f2h_bits(a / 127.0f);
    const float df = h2f(dh);
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 4; i++)
        w |= ((uint32_t)(uint8_t)(int8_t)(df > 0.0f ? nearest_clamp(v[i] / df, -127, 127) : 0)) << (8 * i);
    uint8_t *blk = run + 34 * (lane >> 3);
    st4(blk + 2 + 4 * (lane & 7), w);
    if ((lane & 7) == 0) st2(blk, dh);
}

// Wave-per-256-values generator for n_mats matrices [M x K]: matrix m uses
// stream stream0 + m*stream_step and is written at dst + m*dst_stride.
template <int T>
__global__ __launch_bounds__(256) void k_synth_quant(uint64_t seed, uint64_t stream0, uint64_t stream_step,
                                                     float std, int64_t M, int64_t K, int n_mats,
                                                     uint8_t *dst, uint64_t dst_stride) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int64_t runs_per_row = K / 256, runs_per_mat = M * runs_per_row;
    const int64_t wid = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (wid >= runs_per_mat * n_mats) return;
    const int m = (int)(wid / runs_per_mat);
    const int64_t rr = wid - (int64_t)m * runs_per_mat;
    const int64_t row = rr / runs_per_row, run = rr - row * runs_per_row;
    const uint64_t key = rng_key(seed, stream0 + (uint64_t)m * stream_step);
    const uint64_t i0 = (uint64_t)(row * K + run * 256 + 4 * lane);
    float v[4];
    normal_pair(key, i0 / 2, v[0], v[1]);
    normal_pair(key, i0 / 2 + 1, v[2], v[3]);
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = std * v[i];
    constexpr int bb = T == GGML_TYPE_Q4_K ? 144 : T == GGML_TYPE_Q5_K ? 176 : T == GGML_TYPE_Q6_K ? 210 : 272;
    uint8_t *out = dst + (uint64_t)m * dst_stride + (uint64_t)row * (uint64_t)(runs_per_row * bb) +
                   (uint64_t)run * bb;
    if (T == GGML_TYPE_Q4_K) quant_kq<4>(v, lane, out);
    else if (T == GGML_TYPE_Q5_K) quant_kq<5>(v, lane, out);
    else if (T == GGML_TYPE_Q6_K) quant_q6(v, lane, out);
    else quant_q8_0(v, lane, out);
}

hipError_t launch_synth_f32(uint64_t seed, uint64_t stream, float std, float *out, int64_t n,
                            hipStream_t s) {
    if (n <= 0) return hipErrorInvalidValue;
    const int64_t pairs = (n + 1) / 2;
    k_synth_f32<<<(unsigned)((pairs + 255) / 256), 256, 0, s>>>(rng_key(seed, stream), std, out, n);
    return hipGetLastError();
}

hipError_t launch_synth_quant(int type, uint64_t seed, uint64_t stream0, uint64_t stream_step,
                              float std, int64_t M, int64_t K, int n_mats, uint8_t *dst,
                              uint64_t dst_stride, hipStream_t s) {
    if (M <= 0 || K <= 0 || K % 256 || n_mats <= 0) return hipErrorInvalidValue;
    const int64_t waves = M * (K / 256) * n_mats;
    const unsigned blocks = (unsigned)((waves + 3) / 4);
    switch (type) {
        case GGML_TYPE_Q4_K:
            k_synth_quant<GGML_TYPE_Q4_K><<<blocks, 256, 0, s>>>(seed, stream0, stream_step, std, M, K, n_mats, dst, dst_stride);
            break;
        case GGML_TYPE_Q5_K:
            k_synth_quant<GGML_TYPE_Q5_K><<<blocks, 256, 0, s>>>(seed, stream0, stream_step, std, M, K, n_mats, dst, dst_stride);
            break;
        case GGML_TYPE_Q6_K:
            k_synth_quant<GGML_TYPE_Q6_K><<<blocks, 256, 0, s>>>(seed, stream0, stream_step, std, M, K, n_mats, dst, dst_stride);
            break;
        case GGML_TYPE_Q8_0:
            k_synth_quant<GGML_TYPE_Q8_0><<<blocks, 256, 0, s>>>(seed, stream0, stream_step, std, M, K, n_mats, dst, dst_stride);
            break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace fo
