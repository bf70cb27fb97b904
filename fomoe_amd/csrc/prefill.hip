// prefill.hip — the multi-token MoE path (benchmark config 5: 512 tokens,
// top-10 of 512 experts, Q4_K gate/up and Q6_K down).
//
//   P1 k_pf_router3  logits[T x E] = x . W_r^T (+ bias): bf16 MFMA on x (bf16)
//                    and the fp32 router as three exact bf16 terms, operands
//                    laid out by k_pf_rtile (k_pf_router, fp32 MFMA with LDS
//                    staging, for H not a multiple of 512).
//   P2 k_pf_topk     one wave per token: top-k with lowest-index ties and the
//                    renormalised weights (topk.h), the shared-expert weight
//                    sigmoid(x . v) or 1.
//   P3 k_pf_group    one work-group: (token, rank) pairs grouped by expert in
//                    token order (a per-expert token bitmap in LDS and popcount
//                    prefixes — deterministic, no global atomics), the shared
//                    expert's T pairs after them, and the GEMM tile list
//                    {expert, first pair, n <= 64}.
//   P4 k_pf_gateup   per (tile, 256 rows of F): act = silu(X Wg^T) * (X Wu^T)
//                    with X the tile's gathered bf16 token rows and the weights
//                    dequantized in registers straight into the MFMA B operand
//                    (bf16, round-to-nearest-even of the exact fp32 value);
//                    v_mfma_f32_16x16x32_bf16, fp32 accumulate. The token rows
//                    of super-block kb+1 stream into a second LDS buffer
//                    (direct global->LDS loads) and its weights into registers
//                    while super-block kb is multiplied. act is stored as two
//                    bf16 planes hi = bf16(act), lo = bf16(act - hi)
//                    (|act - hi - lo| <= 2^-18 |act|).
//   P5 k_pf_down     per (tile, 256 rows of H): outp = act Wd^T, same scheme,
//                    two MFMAs (hi, lo) per weight operand, so the intermediate
//                    keeps ~fp32 precision and no result hinges on which side of
//                    a bf16 rounding boundary an fp32 sum landed.
//   P6 k_pf_combine  out[t] = (x[t]) + sum_r w[t,r] outp[pair(t,r)] in rank
//                    order, then the shared expert's pair.
//
// Per-token semantics are those of the batch-1 layer (reference
// src/inference.c:481-606); the reference has no prefill GEMM (its prompt
// tokens go one by one through the decode path), so this path is pinned by
// the oracle's per-token composition with bf16-rounded weights and activations
// (oracle/oracle.c fo_moe_prefill: bf16 weights, fp32 activation).
#include <float.h>

#include <algorithm>
#include <type_traits>

#include "common.h"
#include "prefill.h"
#include "q6k_mfma.h"
#include "topk.h"

namespace fo {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

FO_DEV float bf2f(uint32_t b16) { return __uint_as_float(b16 << 16); }
FO_DEV uint32_t pack_bf16(float lo, float hi) {   // round to nearest even, lo in bits 0..15
    const __bf16 a = (__bf16)lo, b = (__bf16)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// ============================================================ P1 router GEMM
// 32 tokens x 32 experts per work-group on v_mfma_f32_32x32x2_f32: fp32
// operands (x widened exactly from bf16), fp32 accumulate. K runs in chunks
// of 256 staged in LDS k-major (x as [k][token], router as [k][expert]:
// every operand read is 64 consecutive floats), double-buffered, the next
// chunk held in registers while the current one is multiplied; each of the
// four waves accumulates the whole 32 x 32 tile over its quarter of every
// chunk, and the quarters are summed in a fixed order at the end.
constexpr int kRT = 32, kRK = 256;
constexpr uint32_t kRLds = 2u * 2u * kRK * kRT * 4u;    // 128 KiB
typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void k_pf_router(PrefillArgs a) {
    extern __shared__ __attribute__((aligned(16))) float rl_lds[];   // [2][2][kRK][kRT]
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    const int t0 = blockIdx.y * kRT, e0 = blockIdx.x * kRT;
    // loader: row lr (token / expert) of the tile, values 32 c .. 32 c + 31 of the chunk
    const int lr = tid & 31, c = tid >> 5;
    const uint16_t *xp = a.x + (uint64_t)min(t0 + lr, a.T - 1) * a.H + 32 * c;
    const float *rp = a.router + (uint64_t)min(e0 + lr, a.E - 1) * a.H + 32 * c;
    uint4 xv[4];
    float4 rv[8];
    auto fetch = [&](int k0) {
#pragma unroll
        for (int q = 0; q < 4; q++) xv[q] = *(const uint4 *)(xp + k0 + 8 * q);
#pragma unroll
        for (int q = 0; q < 8; q++) rv[q] = *(const float4 *)(rp + k0 + 4 * q);
    };
    auto put = [&](int b) {
        float *xs = rl_lds + b * (2 * kRK * kRT), *rs = xs + kRK * kRT;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t w[4] = {xv[q].x, xv[q].y, xv[q].z, xv[q].w};
#pragma unroll
            for (int h = 0; h < 4; h++) {
                const int k = 32 * c + 8 * q + 2 * h;
                xs[k * kRT + lr] = bf2f(w[h] & 0xFFFFu);
                xs[(k + 1) * kRT + lr] = bf2f(w[h] >> 16);
            }
        }
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int k = 32 * c + 4 * q;
            rs[k * kRT + lr] = rv[q].x;
            rs[(k + 1) * kRT + lr] = rv[q].y;
            rs[(k + 2) * kRT + lr] = rv[q].z;
            rs[(k + 3) * kRT + lr] = rv[q].w;
        }
    };
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.f;
    fetch(0);
    put(0);
    __syncthreads();
    const int NKC = a.H / kRK;
    // A operand: x[token lane % 32][k + lane / 32]; B: router[expert lane % 32][k + lane / 32]
    const int m = lane & 31, kh = lane >> 5;
    for (int kc = 0; kc < NKC; kc++) {
        const int b = kc & 1;
        if (kc + 1 < NKC) fetch((kc + 1) * kRK);
        const float *xs = rl_lds + b * (2 * kRK * kRT), *rs = xs + kRK * kRT;
#pragma unroll
        for (int kk = 64 * wv; kk < 64 * wv + 64; kk += 2) {
            const float av = xs[(kk + kh) * kRT + m];
            const float bv = rs[(kk + kh) * kRT + m];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
        }
        if (kc + 1 < NKC) put(b ^ 1);
        __syncthreads();
    }
    // D layout: lane holds rows 8 (i / 4) + 4 (lane / 32) + i % 4 (tokens) of
    // column lane % 32 (expert); waves 1-3 hand their quarters to wave 0
    float *red = rl_lds;                                   // [3][16][64]
    if (wv > 0) {
#pragma unroll
        for (int i = 0; i < 16; i++) red[((wv - 1) * 16 + i) * 64 + lane] = acc[i];
    }
    __syncthreads();
    if (wv == 0) {
        const int e = e0 + m;
        const float bias = (a.router_bias && e < a.E) ? a.router_bias[e] : 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const float v = ((acc[i] + red[i * 64 + lane]) + red[(16 + i) * 64 + lane]) + red[(32 + i) * 64 + lane];
            const int t = t0 + 8 * (i >> 2) + 4 * kh + (i & 3);
            if (t < a.T && e < a.E) a.logits[(uint64_t)t * a.E + e] = v + bias;
        }
    }
}

// The router GEMM on bf16 MFMA (H % 512 == 0). The tokens are bf16 already;
// each fp32 router weight w is written as three bf16 terms hi = bf16(w),
// mid = bf16(w - hi), lo = bf16(w - hi - mid) (each subtraction exact; hi +
// mid + lo = w to within 2^-24 |w|), so every product x * term is exact in
// fp32 and v_mfma_f32_32x32x16_bf16 accumulates the three partial GEMMs in
// fp32 — fp32-level products at the bf16 matrix rate.
//
// Operand layout (k_pf_rtile, once per call): a 32-row x 64-value block of x
// or of one router term is a 4 KiB chunk ordered [q][lane][8 values], lane
// (r = lane % 32, h = lane / 32) holding values 32h + 8q .. +7 of row r, so
// every load instruction of the GEMM reads 1 KiB contiguous (per-lane 16-byte
// pieces of 32 different rows touch 32-64 cache lines per instruction and
// left the router GEMM bound by the address unit: 30-36 us). MFMA q of a
// block takes the lane's piece q on both operands (the same K permutation on
// A and B leaves the sum unchanged). Chunks: x [T/32][H/64], router
// [E/32][H/64][3 terms]; rows past T or E are zero.
//
// k_pf_router3: 32 tokens x 32 experts per work-group, eight waves, each over
// an eighth of the K blocks, two blocks in flight ahead of the one
// multiplied; the eight partial tiles are summed in wave order at the end.
constexpr int kR3Waves = 8, kR3Ahead = 2;

// One thread per 16-byte piece of the chunks: consecutive threads write
// consecutive pieces, each reading its 8 values (32 bytes of router, 16 of
// x) from its row. (Row-contiguous reads with scattered 16-byte writes, or a
// per-tile transpose through LDS, measured slower: 25 and 15 us against 9.)
FO_DEV void pf_rtile_body(const PrefillArgs &a, uint32_t blk, uint32_t nblk) {
    const int NB = a.H / 64, ET = (a.E + 31) / 32, TT = (a.T + 31) / 32;
    const uint64_t nr = (uint64_t)ET * NB * 256, nx = (uint64_t)TT * NB * 256;   // 16-byte pieces
    uint4 *xt = (uint4 *)(a.rsplit + (uint64_t)3 * ET * 32 * a.H);
    for (uint64_t i = blk * (uint64_t)blockDim.x + threadIdx.x; i < nr + nx; i += (uint64_t)nblk * blockDim.x) {
        const bool isx = i >= nr;
        const uint64_t pi = isx ? i - nr : i;
        const uint64_t chunk = pi >> 8;                  // (row tile, K block)
        const int q = (int)((pi >> 6) & 3), lane = (int)(pi & 63);
        const int kb = (int)(chunk % NB), tile = (int)(chunk / NB);
        const int row = 32 * tile + (lane & 31), k = 64 * kb + 32 * (lane >> 5) + 8 * q;
        if (isx) {
            uint4 v = make_uint4(0, 0, 0, 0);
            if (row < a.T) v = *(const uint4 *)(a.x + (uint64_t)row * a.H + k);
            xt[pi] = v;
        } else {
            float f[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            if (row < a.E) {
                const float4 v0 = *(const float4 *)(a.router + (uint64_t)row * a.H + k);
                const float4 v1 = *(const float4 *)(a.router + (uint64_t)row * a.H + k + 4);
                f[0] = v0.x; f[1] = v0.y; f[2] = v0.z; f[3] = v0.w;
                f[4] = v1.x; f[5] = v1.y; f[6] = v1.z; f[7] = v1.w;
            }
            uint32_t t[3][4];
#pragma unroll
            for (int p = 0; p < 4; p++) {
                uint32_t hw[3] = {0, 0, 0};
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const float fv = f[2 * p + e];
                    const __bf16 th = (__bf16)fv;
                    const float r1 = fv - (float)th;
                    const __bf16 tm = (__bf16)r1;
                    const __bf16 tl = (__bf16)(r1 - (float)tm);
                    hw[0] |= (uint32_t)__builtin_bit_cast(uint16_t, th) << (16 * e);
                    hw[1] |= (uint32_t)__builtin_bit_cast(uint16_t, tm) << (16 * e);
                    hw[2] |= (uint32_t)__builtin_bit_cast(uint16_t, tl) << (16 * e);
                }
#pragma unroll
                for (int j = 0; j < 3; j++) t[j][p] = hw[j];
            }
            uint4 *rt = (uint4 *)a.rsplit + (chunk * 3) * 256 + (pi & 255);
#pragma unroll
            for (int j = 0; j < 3; j++) rt[j * 256] = make_uint4(t[j][0], t[j][1], t[j][2], t[j][3]);
        }
    }
}

__global__ __launch_bounds__(256) void k_pf_rtile(PrefillArgs a) { pf_rtile_body(a, blockIdx.x, gridDim.x); }

__global__ __launch_bounds__(64 * kR3Waves) void k_pf_router3(PrefillArgs a) {
    __shared__ float red[kR3Waves - 1][16][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int NB = a.H / 64, ET = (a.E + 31) / 32;
    const int t0 = blockIdx.y * kRT, e0 = blockIdx.x * kRT;
    const int r = lane & 31, h = lane >> 5;
    const int nb = NB / kR3Waves, kb0 = wv * nb;
    const uint4 *xc = (const uint4 *)(a.rsplit + (uint64_t)3 * ET * 32 * a.H) + ((uint64_t)blockIdx.y * NB + kb0) * 256 + lane;
    const uint4 *wc = (const uint4 *)a.rsplit + ((uint64_t)blockIdx.x * NB + kb0) * 768 + lane;
    struct Blk { uint4 x[4], w[3][4]; };
    auto fetch = [&](Blk &b, int i) {
#pragma unroll
        for (int q = 0; q < 4; q++) b.x[q] = xc[i * 256 + 64 * q];
#pragma unroll
        for (int j = 0; j < 3; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) b.w[j][q] = wc[i * 768 + j * 256 + 64 * q];
    };
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; i++) acc[i] = 0.f;
    Blk ring[kR3Ahead + 1];
#pragma unroll
    for (int i = 0; i < kR3Ahead; i++)
        if (i < nb) fetch(ring[i], i);
    for (int i0 = 0; i0 < nb; i0 += kR3Ahead + 1) {
#pragma unroll
        for (int u = 0; u <= kR3Ahead; u++) {   // ring slot u: block i0 + u
            const int i = i0 + u;
            if (i >= nb) break;
            if (i + kR3Ahead < nb) fetch(ring[(u + kR3Ahead) % (kR3Ahead + 1)], i + kR3Ahead);
            const Blk &b = ring[u];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const bf16x8 xa = __builtin_bit_cast(bf16x8, b.x[q]);
#pragma unroll
                for (int j = 2; j >= 0; j--)   // lo, mid, hi
                    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa, __builtin_bit_cast(bf16x8, b.w[j][q]), acc, 0, 0, 0);
            }
        }
    }
    // D layout: lane holds rows 8 (i / 4) + 4 (lane / 32) + i % 4 (tokens) of column lane % 32
    if (wv > 0) {
#pragma unroll
        for (int i = 0; i < 16; i++) red[wv - 1][i][lane] = acc[i];
    }
    __syncthreads();
    if (wv == 0) {
        const int e = e0 + r;
        const float bias = (a.router_bias && e < a.E) ? a.router_bias[e] : 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            float v = acc[i];
#pragma unroll
            for (int w = 0; w < kR3Waves - 1; w++) v += red[w][i][lane];
            const int t = t0 + 8 * (i >> 2) + 4 * h + (i & 3);
            if (t < a.T && e < a.E) a.logits[(uint64_t)t * a.E + e] = v + bias;
        }
    }
}

// ============================================================ P2 top-k
__global__ __launch_bounds__(256) void k_pf_topk(PrefillArgs a) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= a.T) return;
    const int K1 = a.k + 1;
    if (a.E <= 512) wave_topk<8>(a.logits + (uint64_t)t * a.E, a.E, a.k, a.ids + (uint64_t)t * a.k, a.w + (uint64_t)t * K1);
    else wave_topk<16>(a.logits + (uint64_t)t * a.E, a.E, a.k, a.ids + (uint64_t)t * a.k, a.w + (uint64_t)t * K1);
    float sw = 1.f;
    if (a.shared_gate_vec) {
        float d = 0.f;
        const uint16_t *xp = a.x + (uint64_t)t * a.H;
        for (int i = lane; i < a.H; i += 64) d = fmaf(bf2f(xp[i]), a.shared_gate_vec[i], d);
        d = wave_sum(d);
        sw = 1.0f / (1.0f + expf(-d));
    }
    if (lane == 0) a.w[(uint64_t)t * K1 + a.k] = sw;
}

// ============================================================ P3 grouping
// LDS: per-expert token bitmap bm[e][W] and popcount prefixes pre[e][W],
// W = ceil(T/32) words; counts and offsets over E+1 entries (entry E is the
// shared expert, all T tokens).
constexpr int kPfGroupLds = 16384;     // E*W words of each table
// Row stride of k_pf_group's tables: W rounded up to odd
__host__ __device__ constexpr int pf_group_stride(int W) { return W | 1; }

// Exclusive prefixes over the 1024 threads of 64-bit packed fields:
// inclusive scans within each wave by shuffles, then the 16 wave totals
// summed by every thread.
// Four of them at once (two barriers for all four); buf holds 4 x 16 wave
// totals.
FO_DEV void block_exclusive_scan64x4(uint64_t v0, uint64_t v1, uint64_t v2, uint64_t v3, uint64_t &e0,
                                     uint64_t &e1, uint64_t &e2, uint64_t &e3, uint64_t *buf) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    uint64_t x[4] = {v0, v1, v2, v3};
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        uint64_t y[4];
#pragma unroll
        for (int q = 0; q < 4; q++) y[q] = (uint64_t)__shfl_up((long long)x[q], o, 64);
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (lane >= o) x[q] += y[q];
    }
    if (lane == 63) {
#pragma unroll
        for (int q = 0; q < 4; q++) buf[16 * q + wv] = x[q];
    }
    __syncthreads();
    uint64_t base[4] = {0, 0, 0, 0};
    for (int w = 0; w < wv; w++) {
#pragma unroll
        for (int q = 0; q < 4; q++) base[q] += buf[16 * q + w];
    }
    __syncthreads();
    e0 = base[0] + x[0] - v0; e1 = base[1] + x[1] - v1; e2 = base[2] + x[2] - v2; e3 = base[3] + x[3] - v3;
}

// Bit fields of the packed scans (each field holds its total over all experts:
// pairs < 2^21, full tiles < 2^16, per-expert-at-most-one classes < 2^12).
FO_DEV uint32_t fld(uint64_t v, int lo, int bits) { return (uint32_t)((v >> lo) & ((1ull << bits) - 1)); }

__global__ __launch_bounds__(1024) void k_pf_group(PrefillArgs a) {
    extern __shared__ uint32_t lds[];
    const int tid = threadIdx.x;
    const int W = (a.T + 31) / 32, E = a.E, k = a.k, K1 = k + 1;
    const int Ws = pf_group_stride(W);   // odd: thread e's row walk below is free of bank conflicts
    uint32_t *bm = lds, *pre = lds + E * Ws;
    for (int i = tid; i < E * Ws; i += 1024) bm[i] = 0;
    __syncthreads();
    for (int i = tid; i < a.T * k; i += 1024) {
        const int t = i / k, e = a.one_expert ? 0 : a.ids[i];
        atomicOr(&bm[e * Ws + (t >> 5)], 1u << (t & 31));
    }
    __syncthreads();
    const bool sh = a.shared != nullptr;
    int cnt = 0;
    if (tid < E) {
        for (int w = 0; w < W; w++) { pre[tid * Ws + w] = cnt; cnt += __popc(bm[tid * Ws + w]); }
    } else if (tid == E && sh) {
        cnt = a.T;
    }
    // every prefix the tables need in four scans of packed fields
    constexpr int DT = 2 * kPfMT;
    const int nt = (cnt + kPfMT - 1) / kPfMT;                                 // 64-pair tiles
    // 128-pair tiles of the experts k_pf_down16 runs (dt_sel: all, routed, shared)
    const bool in_dt = a.dt_sel == 0 || tid != E;
    const int dn = in_dt ? (cnt + DT - 1) / DT : 0;
    // The GEMMs take tiles in decreasing cost: entry i's fourth word is the
    // i-th tile by token-block count (4, 3, 2, 1; expert order within a
    // count), so the last work handed out is the cheapest; the one tile of an
    // expert of at most kPfThin pairs comes last of all (the thin experts,
    // whose Q6_K down projection runs on the integer path). Per expert: its
    // full tiles (count 4) and its last, partial tile (count cb).
    const int nfull = cnt / kPfMT, rem = cnt - kPfMT * nfull, cb = (rem + 15) >> 4;   // cb = 0: no partial tile
    // (a shared expert whose down projection runs in its own type is never thin)
    const int thin = cnt > 0 && cnt <= kPfThin && !(tid == E && a.sh_down_type >= 0);
    const int c4 = nfull + (cb == 4), c3 = cb == 3, c2 = cb == 2, c1 = cb == 1 && !thin;
    // Double tiles for k_pf_down16: per expert ceil(cnt / 128) tiles of up to
    // 2 kPfMT pairs (its weights are read and decoded once per 128 pairs), in
    // decreasing token-block count (8 .. 1), those of thin experts last.
    const int dcnt = in_dt ? cnt : 0;
    const int dfull = dcnt / DT, drem = dcnt - DT * dfull, dcb = (drem + 15) >> 4;
    const int dthin = thin && in_dt;
    auto cls = [&](int b) { return b == 8 ? dfull + (dcb == 8) : (dcb == b && !dthin ? 1 : 0); };
    __shared__ uint64_t scan64[4 * 16];
    const uint64_t p1 = (uint64_t)cnt | ((uint64_t)nt << 21) | ((uint64_t)dn << 42);
    const uint64_t p2 = (uint64_t)c4 | ((uint64_t)c3 << 16) | ((uint64_t)c2 << 28) | ((uint64_t)c1 << 40) |
                        ((uint64_t)thin << 52);
    const uint64_t p5 = (uint64_t)dthin;   // thin experts among the double tiles
    const uint64_t p3 = (uint64_t)cls(8) | ((uint64_t)cls(7) << 16) | ((uint64_t)cls(6) << 28) |
                        ((uint64_t)cls(5) << 40) | ((uint64_t)cls(4) << 52);
    const uint64_t p4 = (uint64_t)cls(3) | ((uint64_t)cls(2) << 12) | ((uint64_t)cls(1) << 24);
    uint64_t s1, s2, s3, s4;
    block_exclusive_scan64x4(p1, p2, p3, p4 | (p5 << 36), s1, s2, s3, s4, scan64);
    const int off = (int)fld(s1, 0, 21), toff = (int)fld(s1, 21, 21), doff = (int)fld(s1, 42, 21);
    __shared__ uint64_t s_tot[4];
    if (tid == 1023) { s_tot[0] = s1 + p1; s_tot[1] = s2 + p2; s_tot[2] = s3 + p3; s_tot[3] = s4 + (p4 | (p5 << 36)); }
    if (tid == E && sh) a.n_tiles[5] = toff;   // the shared expert's first 64-pair tile
    __syncthreads();
    const uint64_t t1 = s_tot[0], t2 = s_tot[1], t3 = s_tot[2], t4 = s_tot[3];
    const int T4 = (int)fld(t2, 0, 16), T3 = (int)fld(t2, 16, 12), T2 = (int)fld(t2, 28, 12), T1 = (int)fld(t2, 40, 12);
    const int Tthin = (int)fld(t2, 52, 12), Tdthin = (int)fld(t4, 36, 12);
    const int b4 = (int)fld(s2, 0, 16);                                       // this expert's first rank per count
    const int bpart = cb == 4 ? b4 + nfull : cb == 3 ? T4 + (int)fld(s2, 16, 12)
                    : cb == 2 ? T4 + T3 + (int)fld(s2, 28, 12) : thin ? T4 + T3 + T2 + T1 + (int)fld(s2, 52, 12)
                    : T4 + T3 + T2 + (int)fld(s2, 40, 12);
    if (tid <= E) {
        for (int i = 0; i < nt; i++) {
            int32_t *tp = a.tiles + 4 * (toff + i);
            tp[0] = tid; tp[1] = off + kPfMT * i; tp[2] = min(kPfMT, cnt - kPfMT * i);
            a.tiles[4 * (i < nfull ? b4 + i : bpart) + 3] = toff + i;
        }
    }
    // [0]: tiles, [1]: tiles before the thin ones, [2]: k_pf_gateup_f16 work
    // counter, [3]: double tiles, [4]: double tiles before the thin experts'
    const int NT = (int)fld(t1, 21, 21), ND = (int)fld(t1, 42, 21);
    if (tid == 1023) { a.n_tiles[0] = NT; a.n_tiles[1] = NT - Tthin; a.n_tiles[2] = 0; a.n_tiles[3] = ND; a.n_tiles[4] = ND - Tdthin; }
    {
        int tot[9], base[9];   // per class count and first rank, classes in order 8, 7, .., 1
        tot[8] = (int)fld(t3, 0, 16); tot[7] = (int)fld(t3, 16, 12); tot[6] = (int)fld(t3, 28, 12);
        tot[5] = (int)fld(t3, 40, 12); tot[4] = (int)fld(t3, 52, 12);
        tot[3] = (int)fld(t4, 0, 12); tot[2] = (int)fld(t4, 12, 12); tot[1] = (int)fld(t4, 24, 12);
        base[8] = 0;
        for (int b = 7; b >= 1; b--) base[b] = base[b + 1] + tot[b + 1];
        const int thin_base = base[1] + tot[1];
        const int mine[9] = {0, (int)fld(s4, 24, 12), (int)fld(s4, 12, 12), (int)fld(s4, 0, 12), (int)fld(s3, 52, 12),
                             (int)fld(s3, 40, 12), (int)fld(s3, 28, 12), (int)fld(s3, 16, 12), (int)fld(s3, 0, 16)};
        if (tid <= E) {
            for (int i = 0; i < dn; i++) {
                int32_t *tp = a.dtiles + 4 * (doff + i);
                tp[0] = tid; tp[1] = off + DT * i; tp[2] = min(DT, cnt - DT * i);
                int rank;
                if (dthin) rank = thin_base + (int)fld(s4, 36, 12);
                else if (i < dfull) rank = base[8] + mine[8] + i;
                else rank = dcb == 8 ? base[8] + mine[8] + dfull : base[dcb] + mine[dcb];
                a.dtiles[4 * rank + 3] = doff + i;
            }
        }
    }
    // pair offsets of each expert for the placement pass
    __shared__ int s_off[1025];
    if (tid <= E) s_off[tid] = off;
    __syncthreads();
    for (int i = tid; i < a.T * k; i += 1024) {
        const int t = i / k, r = i - t * k, e = a.one_expert ? 0 : a.ids[i];
        const uint32_t word = bm[e * Ws + (t >> 5)];
        const int pos = s_off[e] + (int)pre[e * Ws + (t >> 5)] + __popc(word & ((1u << (t & 31)) - 1u));
        a.pair_tok[pos] = t;
        a.pairpos[t * K1 + r] = pos;
    }
    if (sh)
        for (int t = tid; t < a.T; t += 1024) {
            const int pos = s_off[E] + t;
            a.pair_tok[pos] = t;
            a.pairpos[t * K1 + k] = pos;
        }
}

// ============================================================ weight decode
// Eight consecutive values k = 32*ch + 8*kg .. +7 of one row's super-block,
// dequantized exactly in fp32 (as reference src/quant.c:82-105, 147-175) and
// rounded to bf16, packed for the MFMA B operand.
template <int T> struct PfDec;

template <> struct PfDec<GGML_TYPE_Q4_K> {
    static constexpr int TYPE = GGML_TYPE_Q4_K, BLOCK = 144;
    struct Sb { uint4 hdr; uint2 q[4]; };
    static FO_DEV Sb load(const uint8_t *sb, int kg) {
        Sb s;
        s.hdr = ld16(sb);
#pragma unroll
        for (int c = 0; c < 4; c++) s.q[c] = ld8(sb + 16 + 32 * c + 8 * kg);
        return s;
    }
    // group j (0..7) = 32-value chunk ch: scale/min per reference src/quant.c:72-80
    static FO_DEV u32x4 decode(const Sb &s, int ch) {
        const uint32_t sc4[3] = {s.hdr.y, s.hdr.z, s.hdr.w};
        const int j = ch;
        auto byte = [&](int i) -> uint32_t { return (sc4[i >> 2] >> (8 * (i & 3))) & 0xFFu; };
        uint32_t sc, mn;
        if (j < 4) { sc = byte(j) & 63; mn = byte(j + 4) & 63; }
        else {
            sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
            mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
        }
        const float d1 = h2f(s.hdr.x) * (float)sc, m1 = h2f(s.hdr.x >> 16) * (float)mn;
        const uint2 q = s.q[ch >> 1];
        const int sh = 4 * (ch & 1);
        const uint32_t w0 = (q.x >> sh) & 0x0F0F0F0Fu, w1 = (q.y >> sh) & 0x0F0F0F0Fu;
        u32x4 r;
        r[0] = pack_bf16(fmaf(d1, ub0(w0), -m1), fmaf(d1, ub1(w0), -m1));
        r[1] = pack_bf16(fmaf(d1, ub2(w0), -m1), fmaf(d1, ub3(w0), -m1));
        r[2] = pack_bf16(fmaf(d1, ub0(w1), -m1), fmaf(d1, ub1(w1), -m1));
        r[3] = pack_bf16(fmaf(d1, ub2(w1), -m1), fmaf(d1, ub3(w1), -m1));
        return r;
    }
};

template <> struct PfDec<GGML_TYPE_Q6_K> {
    static constexpr int TYPE = GGML_TYPE_Q6_K, BLOCK = 210;
    struct Sb { uint2 ql[4], qh[2]; uint4 sc; uint32_t d; };
    static FO_DEV Sb load(const uint8_t *sb, int kg) {
        Sb s;
#pragma unroll
        for (int n = 0; n < 2; n++) {
            s.ql[2 * n] = ld8(sb + 64 * n + 8 * kg);
            s.ql[2 * n + 1] = ld8(sb + 64 * n + 32 + 8 * kg);
            s.qh[n] = ld8(sb + 128 + 32 * n + 8 * kg);
        }
        s.sc = ld16(sb + 192);
        s.d = ld2(sb + 208);
        return s;
    }
    // chunk ch = 4n + t: values 128n + 32t + l, l = 8kg..8kg+7; scale sc[8n + 2t + kg/2]
    static FO_DEV u32x4 decode(const Sb &s, int ch, int kg) {
        const int n = ch >> 2, t = ch & 3;
        const uint2 l = s.ql[2 * n + (t & 1)];
        const uint2 h = s.qh[n];
        const int ls = 4 * (t >> 1), hs = 2 * t;
        const uint32_t c0 = ((l.x >> ls) & 0x0F0F0F0Fu) | (((h.x >> hs) & 0x03030303u) << 4);
        const uint32_t c1 = ((l.y >> ls) & 0x0F0F0F0Fu) | (((h.y >> hs) & 0x03030303u) << 4);
        const int si = 8 * n + 2 * t + (kg >> 1);
        const uint32_t scw = si < 4 ? s.sc.x : si < 8 ? s.sc.y : si < 12 ? s.sc.z : s.sc.w;
        const int scv = (int)(int8_t)((scw >> (8 * (si & 3))) & 0xFFu);
        const float d1 = h2f(s.d) * (float)scv;
        u32x4 r;
        r[0] = pack_bf16(d1 * (ub0(c0) - 32.f), d1 * (ub1(c0) - 32.f));
        r[1] = pack_bf16(d1 * (ub2(c0) - 32.f), d1 * (ub3(c0) - 32.f));
        r[2] = pack_bf16(d1 * (ub0(c1) - 32.f), d1 * (ub1(c1) - 32.f));
        r[3] = pack_bf16(d1 * (ub2(c1) - 32.f), d1 * (ub3(c1) - 32.f));
        return r;
    }
};

// Q5_K (reference src/quant.c:216-247): Q4_K's header and nibbles plus a
// fifth bit per value, bit j of qh[l] for value l of sub-block j.
template <> struct PfDec<GGML_TYPE_Q5_K> {
    static constexpr int TYPE = GGML_TYPE_Q5_K, BLOCK = 176;
    struct Sb { uint4 hdr; uint2 qh; uint2 q[4]; };
    static FO_DEV Sb load(const uint8_t *sb, int kg) {
        Sb s;
        s.hdr = ld16(sb);
        s.qh = ld8(sb + 16 + 8 * kg);
#pragma unroll
        for (int c = 0; c < 4; c++) s.q[c] = ld8(sb + 48 + 32 * c + 8 * kg);
        return s;
    }
    // chunk ch = sub-block ch, values 8kg..8kg+7 of it
    static FO_DEV u32x4 decode(const Sb &s, int ch, int) {
        const uint32_t sc4[3] = {s.hdr.y, s.hdr.z, s.hdr.w};
        const int j = ch;
        auto byte = [&](int i) -> uint32_t { return (sc4[i >> 2] >> (8 * (i & 3))) & 0xFFu; };
        uint32_t sc, mn;
        if (j < 4) { sc = byte(j) & 63; mn = byte(j + 4) & 63; }
        else {
            sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
            mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
        }
        const float d1 = h2f(s.hdr.x) * (float)sc, m1 = h2f(s.hdr.x >> 16) * (float)mn;
        const uint2 q = s.q[ch >> 1];
        const int sh = 4 * (ch & 1);
        const uint32_t w0 = ((q.x >> sh) & 0x0F0F0F0Fu) | (((s.qh.x >> ch) & 0x01010101u) << 4);
        const uint32_t w1 = ((q.y >> sh) & 0x0F0F0F0Fu) | (((s.qh.y >> ch) & 0x01010101u) << 4);
        u32x4 r;
        r[0] = pack_bf16(fmaf(d1, ub0(w0), -m1), fmaf(d1, ub1(w0), -m1));
        r[1] = pack_bf16(fmaf(d1, ub2(w0), -m1), fmaf(d1, ub3(w0), -m1));
        r[2] = pack_bf16(fmaf(d1, ub0(w1), -m1), fmaf(d1, ub1(w1), -m1));
        r[3] = pack_bf16(fmaf(d1, ub2(w1), -m1), fmaf(d1, ub3(w1), -m1));
        return r;
    }
};

// Q8_0 (reference src/quant.c:266-274) in groups of eight 34-byte blocks
// (256 values, the unit the grouped GEMMs step by): chunk ch = block ch.
template <> struct PfDec<GGML_TYPE_Q8_0> {
    static constexpr int TYPE = GGML_TYPE_Q8_0, BLOCK = 8 * 34;
    struct Sb { uint32_t d[4]; uint2 q[8]; };   // d: the blocks' fp16 scales, two per word
    static FO_DEV Sb load(const uint8_t *sb, int kg) {
        Sb s;
#pragma unroll
        for (int c = 0; c < 4; c++) s.d[c] = ld2(sb + 68 * c) | (ld2(sb + 68 * c + 34) << 16);
#pragma unroll
        for (int c = 0; c < 8; c++) s.q[c] = ld8(sb + 34 * c + 2 + 8 * kg);
        return s;
    }
    static FO_DEV u32x4 decode(const Sb &s, int ch, int) {
        const float d = h2f(s.d[ch >> 1] >> (16 * (ch & 1)));
        const uint2 q = s.q[ch];
        auto v = [&](uint32_t w, int i) { return d * (float)(int8_t)((w >> (8 * i)) & 0xFFu); };
        u32x4 r;
        r[0] = pack_bf16(v(q.x, 0), v(q.x, 1));
        r[1] = pack_bf16(v(q.x, 2), v(q.x, 3));
        r[2] = pack_bf16(v(q.y, 0), v(q.y, 1));
        r[3] = pack_bf16(v(q.y, 2), v(q.y, 3));
        return r;
    }
};

// Eight values of chunk ch (lane group kg) of a Q4_K or Q5_K super-block as
// fp16 operands: the exact fp32 dequantized value d1 * q - m1 (the product is
// exact, one rounding for the difference, as the reference's dequantization)
// rounded once more to fp16 (nearest even).
template <int T>
FO_DEV f16x8 pf_decode_f16_k(const typename PfDec<T>::Sb &s, int ch) {
    const uint32_t sc4[3] = {s.hdr.y, s.hdr.z, s.hdr.w};
    const int j = ch;
    auto byte = [&](int i) -> uint32_t { return (sc4[i >> 2] >> (8 * (i & 3))) & 0xFFu; };
    uint32_t sc, mn;
    if (j < 4) { sc = byte(j) & 63; mn = byte(j + 4) & 63; }
    else {
        sc = (byte(j + 4) & 0xF) | ((byte(j - 4) >> 6) << 4);
        mn = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
    const float d1 = h2f(s.hdr.x) * (float)sc, m1 = h2f(s.hdr.x >> 16) * (float)mn;
    const uint2 q = s.q[ch >> 1];
    const int sh = 4 * (ch & 1);
    uint32_t w0 = (q.x >> sh) & 0x0F0F0F0Fu, w1 = (q.y >> sh) & 0x0F0F0F0Fu;
    if constexpr (T == GGML_TYPE_Q5_K) {
        w0 |= ((s.qh.x >> ch) & 0x01010101u) << 4;
        w1 |= ((s.qh.y >> ch) & 0x01010101u) << 4;
    }
    f16x8 r;
    r[0] = (_Float16)fmaf(d1, ub0(w0), -m1); r[1] = (_Float16)fmaf(d1, ub1(w0), -m1);
    r[2] = (_Float16)fmaf(d1, ub2(w0), -m1); r[3] = (_Float16)fmaf(d1, ub3(w0), -m1);
    r[4] = (_Float16)fmaf(d1, ub0(w1), -m1); r[5] = (_Float16)fmaf(d1, ub1(w1), -m1);
    r[6] = (_Float16)fmaf(d1, ub2(w1), -m1); r[7] = (_Float16)fmaf(d1, ub3(w1), -m1);
    return r;
}

template <int T>
FO_DEV u32x4 pf_decode(const typename PfDec<T>::Sb &s, int ch, int kg) {
    if constexpr (T == GGML_TYPE_Q4_K) return PfDec<T>::decode(s, ch);
    else return PfDec<T>::decode(s, ch, kg);
}

FO_DEV bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// ============================================================ P4/P5 grouped GEMMs
// Work-group placement: a 1-D grid of nrb * ceil8(max_tiles) work-groups,
// numbered so that the nrb row-block work-groups of one tile have ids equal
// mod 8. Work-group i runs on XCD i % 8 (round-robin dispatch), so all of a
// tile's row blocks share one XCD, whose L2 serves the tile's staged
// activation rows to every one of them (with (row block, tile) as a 2-D grid
// each XCD held one row block of every tile and fetched every tile's rows).
FO_DEV void pf_tile_of(int nrb, int &tile, int &rb) {
    const int i = blockIdx.x, c = i / (8 * nrb), j = i - c * 8 * nrb;
    tile = 8 * c + (j & 7);
    rb = j >> 3;
}
inline unsigned pf_grid(int nrb, int max_tiles) { return (unsigned)(nrb * ((max_tiles + 7) & ~7)); }
// Work-group: 4 waves, tile of <= 64 pairs (token rows) x 64 weight rows; wave
// w owns weight rows 16w..16w+15 (MFMA columns: lane % 16) for every token
// block. The tile's activations for one 256-value super-block sit in LDS
// (row stride 264 bf16: 16-byte aligned, rows spread over banks).

// Activation tile in LDS: 64 token rows x 256 bf16 (32 chunks of 16 B), no
// padding; chunk c of row m sits at slot c ^ (m & 15) so that the 16 rows an
// MFMA A-operand read touches fall on 16 different 16-byte bank groups.
// Filled with gfx950's direct global->LDS loads (one wave instruction = two
// rows), so the next super-block's tile streams in while the current one is
// multiplied, without holding it in registers.
constexpr int kPfTile = kPfMT * 256;              // bf16 elements per tile buffer
FO_DEV int pf_swz(int m, int c) { return m * 256 + 8 * (c ^ (m & 15)); }

template <typename RowPtr>
FO_DEV void pf_stage_async(uint16_t *buf, int n, int k0, RowPtr src_row) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int rows = (n + 15) & ~15;                           // the MFMA row blocks in use
    for (int q = wave; q < rows / 2; q += nw) {
        const int m = 2 * q + (lane >> 5), cs = lane & 31;      // LDS slot (m, cs)
        const int c = cs ^ (m & 15);                            // global chunk stored there
        const uint16_t *src = src_row(m < n ? m : 0) + k0 + 8 * c;
        __builtin_amdgcn_global_load_lds((const void *)src,
                                         (__attribute__((address_space(3))) void *)(buf + q * 512), 16, 0, 0);
    }
}

// Token rows of a tile: lane m of `tok` holds the token of tile row m (rows
// past n repeat the last one). The row addresses come from it by readlane, so
// no staging load waits for an index load (waiting for the newest load is
// waiting for every load in flight: each row load used to drain the wave).
FO_DEV void pf_stage_tokens(uint16_t *buf, int n, int k0, const uint16_t *x, int H, int tok) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int rows = (n + 15) & ~15;
    for (int q = wave; q < rows / 2; q += nw) {
        const int m = 2 * q + (lane >> 5), cs = lane & 31;
        const int c = cs ^ (m & 15);
        const int ta = __builtin_amdgcn_readlane(tok, 2 * q), tb = __builtin_amdgcn_readlane(tok, 2 * q + 1);
        const uint16_t *src = x + (uint64_t)(lane < 32 ? ta : tb) * H + k0 + 8 * c;
        __builtin_amdgcn_global_load_lds((const void *)src,
                                         (__attribute__((address_space(3))) void *)(buf + q * 512), 16, 0, 0);
    }
}

#pragma clang fp contract(off)
// Work-group: kPfGateWaves waves over kPfGateRows rows of F: the first half
// computes the gate rows, the second half the same up rows, for every token
// block of the tile; the up sums meet the gate sums in LDS for the SwiGLU
// epilogue. Wide work-groups share one staged token tile among many rows.
template <int GT, int UT>
__global__ __launch_bounds__(kPfGateWaves * 64, 4) void k_pf_gateup(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t xs[2 * kPfTile];
    int tile, rbk;
    pf_tile_of(a.F / kPfGateRows, tile, rbk);
    if (tile >= *a.n_tiles) return;
    const int4 tl = *(const int4 *)(a.tiles + 4 * tile);
    const int e = tl.x, p0 = tl.y, n = tl.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, col = lane & 15, kg = lane >> 4;
    const bool shared = e == a.E;
    const uint8_t *blob = shared ? a.shared : a.experts + (uint64_t)e * a.stride;
    constexpr int HW = kPfGateWaves / 2;
    const bool is_up = wave >= HW;
    const int rl = 32 * (wave % HW) + col;                // rows rl, rl + 16 within the WG's kPfGateRows
    const int row = rbk * kPfGateRows + rl;
    const int nb = (n + 15) >> 4, NK = a.H / 256;
    const int32_t *toks = a.pair_tok + p0;
    const int my_tok = toks[min(lane, n - 1)];
    f32x4 acc[2][4];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[h][b] = (f32x4){0, 0, 0, 0};
    auto run = [&](auto dec, const uint8_t *w0, uint64_t rowb) {
        using D = decltype(dec);
        const uint8_t *w1 = w0 + 16 * rowb;
        pf_stage_tokens(xs, n, 0, a.x, a.H, my_tok);
        auto s0_next = D::load(w0, kg);
        auto s1_next = D::load(w1, kg);
        for (int kb = 0; kb < NK; kb++) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();                              // tile kb in LDS; buffer kb-1 free
            const auto s0 = s0_next;
            const auto s1 = s1_next;
            if (kb + 1 < NK) {
                pf_stage_tokens(xs + ((kb + 1) & 1) * kPfTile, n, (kb + 1) * 256, a.x, a.H, my_tok);
                s0_next = D::load(w0 + (uint64_t)(kb + 1) * D::BLOCK, kg);
                s1_next = D::load(w1 + (uint64_t)(kb + 1) * D::BLOCK, kg);
            }
            const uint16_t *xb = xs + (kb & 1) * kPfTile;
#pragma unroll
            for (int ch = 0; ch < 8; ch++) {
                const bf16x8 b0 = as_bf16x8(pf_decode<D::TYPE>(s0, ch, kg));
                const bf16x8 b1 = as_bf16x8(pf_decode<D::TYPE>(s1, ch, kg));
#pragma unroll
                for (int b = 0; b < 4; b++)
                    if (b < nb) {
                        const bf16x8 av = *(const bf16x8 *)(xb + pf_swz(16 * b + col, 4 * ch + kg));
                        acc[0][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b0, acc[0][b], 0, 0, 0);
                        acc[1][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, b1, acc[1][b], 0, 0, 0);
                    }
            }
        }
    };
    if (!is_up) {
        const uint64_t rb = (uint64_t)NK * PfDec<GT>::BLOCK;
        run(PfDec<GT>{}, blob + (uint64_t)row * rb, rb);
    } else {
        const uint64_t up_off = shared ? a.sh_gate_size : a.gate_size;
        const uint64_t rb = (uint64_t)NK * PfDec<UT>::BLOCK;
        run(PfDec<UT>{}, blob + up_off + (uint64_t)row * rb, rb);
    }
    __syncthreads();                                      // all reads of xs done: reuse it
    float *ub = (float *)xs;                              // [64 tokens][kPfGateRows] up sums
    if (is_up) {
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int b = 0; b < 4; b++)
#pragma unroll
                for (int i = 0; i < 4; i++) ub[(16 * b + 4 * kg + i) * kPfGateRows + rl + 16 * h] = acc[h][b][i];
    }
    __syncthreads();
    if (!is_up) {
        // D layout: lane holds rows 4*(lane/16)+i (tokens) of column lane%16 (weight row);
        // the activation is stored as hi/lo bf16 planes for the down projection
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int b = 0; b < 4; b++) {
                if (b >= nb) break;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int m = 16 * b + 4 * kg + i;
                    if (m < n) {
                        const float g = acc[h][b][i], u = ub[m * kPfGateRows + rl + 16 * h];
                        const float v = (g / (1.0f + expf(-g))) * u;
                        const __bf16 hi = (__bf16)v;
                        const __bf16 lo = (__bf16)(v - (float)hi);
                        const uint64_t o = (uint64_t)(p0 + m) * a.F + row + 16 * h;
                        a.act_hi[o] = __builtin_bit_cast(uint16_t, hi);
                        a.act_lo[o] = __builtin_bit_cast(uint16_t, lo);
                    }
                }
            }
    }
}

// ------------------------------------------------------------ Q4_K gate/up on exact fp16 MFMA operands
// A Q4_K weight is d * sc_j * q - dmin * m_j (q 4-bit, sc_j / m_j 6-bit
// per 32-value sub-block j, d / dmin fp16 per super-block). sc_j * q <= 945
// is an exact fp16 integer, so the B operand of v_mfma_f32_16x16x32_f16 is
// built as fp16(sc_j * q) (v_perm of the code bytes under 0x64 gives
// 1024 + q, one v_pk_fma_f16 (1024 + q) * sc - 1024 * sc gives sc * q
// exactly) and the MFMA accumulates a whole super-block: per output
// acc += d * D with D = sum_k x_k sc_j q_k, one fma per super-block instead
// of one scale per 32 values. The min term -sum_j (dmin m_j) S_j (S_j the
// token's sub-block sums, fp32) runs on v_mfma_f32_16x16x4_f32 into the same
// accumulator. The token rows (and their sums) enter scaled by a per-token
// power of two (k_pf_xprep: the row maximum lands in [2^14, 2^15), so the
// fp16 rows are exact for every value above 2^-28 of the row maximum and off
// by at most 2^-39 of it below), which the epilogue undoes.
//
// Work item = (tile, 128 rows of F); work-group = 8 waves, wave w owns the
// 16 gate and 16 up rows 16w..16w+15 of the item. K runs in steps of one
// super-block: per step each wave's rows (2 x 16 x 144 bytes) go from HBM
// straight into its own LDS area by direct global->LDS loads (1 KiB
// coalesced pieces, no registers), and the work-group shares the step's token
// rows (<= 64 x 256 fp16, swizzled) and sub-block sums, staged the same way.
// 74 KiB of LDS and <= 128 VGPRs: two work-groups share a CU, and the loads
// of one overlap the arithmetic of the other. Work-groups take items from a
// counter (reset by k_pf_group).
constexpr int kWsWaves = 8;
constexpr int kWsRows = 16 * kWsWaves;                // F rows per item

// Token prep for the fp16 path, one work-group per token: s = the power of
// two that brings max|x| into [2^14, 2^15) (large and tiny rows alike),
// x16 = fp16(x * 2^-s), the fp32 sums of the bf16 values over 32-value
// sub-blocks (sequential) times 2^-s, and s.
__global__ __launch_bounds__(256) void k_pf_xprep(PrefillArgs a) {
    __shared__ float red[4];
    const int t = blockIdx.x, tid = threadIdx.x, H = a.H;
    const uint16_t *xr = a.x + (uint64_t)t * H;
    float m = 0.f;
    for (int i = tid; i < H; i += 256) m = fmaxf(m, fabsf(bf2f(xr[i])));
    m = wave_max(m);
    if ((tid & 63) == 0) red[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int E = 0;
    frexpf(m, &E);                                         // 2^(E-1) <= m < 2^E (m finite, nonzero)
    const int sx = E - 15;
    uint16_t *x16 = a.x16 + (uint64_t)t * H;
    for (int i = tid; i < H; i += 256)
        x16[i] = __builtin_bit_cast(uint16_t, (_Float16)ldexpf(bf2f(xr[i]), -sx));
    const int nsb = H / 32;
    for (int j = tid; j < nsb; j += 256) {
        const uint16_t *p = xr + 32 * j;
        float sum = 0.f;
        for (int q = 0; q < 32; q++) sum = sum + bf2f(p[q]);
        a.xsum[(uint64_t)t * nsb + j] = ldexpf(sum, -sx);
    }
    if (tid == 0) a.xexp[t] = sx;
}

// k_pf_xprep with one wave per token (H % 2048 == 0): lane l owns values
// V l .. V l + V - 1 (V = H / 64, whole 32-value sub-blocks), so the same
// maximum, scale and sequential sub-block sums as k_pf_xprep come out of
// shuffles and registers instead of barriers and 2-byte loads; the row is
// read twice (the second time from the caches).
constexpr int kXpWaves = 4;

FO_DEV void pf_xprep_body(const PrefillArgs &a, uint32_t blk) {
    const int lane = threadIdx.x & 63, t = blk * kXpWaves + (threadIdx.x >> 6);
    if (t >= a.T) return;
    const int H = a.H, V = H / 64, nc = V / 8;          // 16-byte chunks per lane
    const uint16_t *xr = a.x + (uint64_t)t * H + (uint64_t)lane * V;
    float m = 0.f;
    for (int c = 0; c < nc; c++) {
        const uint4 w = *(const uint4 *)(xr + 8 * c);
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int i = 0; i < 4; i++) m = fmaxf(m, fmaxf(fabsf(bf2f(u[i] & 0xFFFFu)), fabsf(bf2f(u[i] >> 16))));
    }
    m = wave_max(m);
    int E = 0;
    frexpf(m, &E);                                         // 2^(E-1) <= m < 2^E (m finite, nonzero)
    const int sx = E - 15;
    uint16_t *x16 = a.x16 + (uint64_t)t * H + (uint64_t)lane * V;
    float *xs = a.xsum + (uint64_t)t * (H / 32) + lane * (V / 32);
    float sum = 0.f;
    for (int c = 0; c < nc; c++) {
        const uint4 w = *(const uint4 *)(xr + 8 * c);
        const uint32_t u[4] = {w.x, w.y, w.z, w.w};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float f0 = bf2f(u[i] & 0xFFFFu), f1 = bf2f(u[i] >> 16);
            sum = sum + f0;
            sum = sum + f1;
            o[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)ldexpf(f0, -sx)) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)ldexpf(f1, -sx)) << 16);
        }
        *(uint4 *)(x16 + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
        if ((c & 3) == 3) {
            xs[c >> 2] = ldexpf(sum, -sx);
            sum = 0.f;
        }
    }
    if (lane == 0) a.xexp[t] = sx;
}

__global__ __launch_bounds__(64 * kXpWaves) void k_pf_xprep_w(PrefillArgs a) { pf_xprep_body(a, blockIdx.x); }

// The router operand layout and the token prep in one launch (neither reads
// what the other writes): work-groups [0, n_rt) lay out the router GEMM's
// operands, the rest prepare the tokens for the fp16 gate/up kernel.
__global__ __launch_bounds__(256) void k_pf_prep(PrefillArgs a, uint32_t n_rt) {
    if (blockIdx.x < n_rt) pf_rtile_body(a, blockIdx.x, n_rt);
    else pf_xprep_body(a, blockIdx.x - n_rt);
}

// 6-bit (scale, min) of sub-block j from the 12 scale bytes (words y, z, w
// of a Q4_K header; reference src/quant.c:72-80)
FO_DEV void q4_scale_min(const uint4 &hdr, int j, uint32_t &sc, uint32_t &mn) {
    const int jj = j & 3;
    const uint32_t b0 = (hdr.y >> (8 * jj)) & 0xFFu, b4 = (hdr.z >> (8 * jj)) & 0xFFu, b8 = (hdr.w >> (8 * jj)) & 0xFFu;
    const bool lo = j < 4;
    sc = lo ? (b0 & 63) : ((b8 & 0xF) | ((b0 >> 2) & 0x30));
    mn = lo ? (b4 & 63) : ((b8 >> 4) | ((b4 >> 2) & 0x30));
}

// Eight codes of nibble h (0: low, 1: high) of q times the sub-block scale as
// exact fp16. A byte b = code (h = 0) or 16 code (h = 1, the nibble masked in
// place, no shift) becomes the fp16 1024 + b through byte permutes with 0x64;
// with (sc, nsc) = q4_scale_f16(scale, h) one fma per pair gives code * scale:
// (1024 + b) s - 1024 s with s = scale / 16^h, exact with one rounding
// (|code * scale| <= 945).
FO_DEV f16x8 q4_codes_f16(uint2 q, int h, f16x2 sc, f16x2 nsc) {
    const uint32_t m = h ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
    const uint32_t w0 = q.x & m, w1 = q.y & m;
    const uint32_t p[4] = {__builtin_amdgcn_perm(0x64646464u, w0, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, w0, 0x04030402u),
                           __builtin_amdgcn_perm(0x64646464u, w1, 0x04010400u),
                           __builtin_amdgcn_perm(0x64646464u, w1, 0x04030402u)};
    u32x4 r;
#pragma unroll
    for (int i = 0; i < 4; i++)
        r[i] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(f16x2, p[i]), sc, nsc));
    return __builtin_bit_cast(f16x8, r);
}
// (scale / 16^h, -1024 scale / 16^h) as fp16 pairs, exact: the bits 0x6400 |
// scale are 1024 + scale, 0x5400 | scale are 64 + scale / 16
FO_DEV void q4_scale_f16(uint32_t scale, int h, f16x2 &sc, f16x2 &nsc) {
    const f16x2 m1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
    const f16x2 off = h ? (f16x2){(_Float16)-64.f, (_Float16)-64.f} : m1024;
    sc = __builtin_bit_cast(f16x2, (scale * 0x10001u) | (h ? 0x54005400u : 0x64006400u)) + off;
    nsc = sc * m1024;
}

constexpr int kGbKC = 256;                            // K values per step
constexpr uint32_t kGbHalf = 16 * 144;                // a wave's 16 rows of one matrix per step
constexpr uint32_t kGbW = 2 * kGbHalf;                // 4608 bytes: gate | up
constexpr int kGbPieces = (kGbW + 1023) / 1024;       // 5 (the last one partial)
constexpr uint32_t kGbArea = kGbPieces * 1024;        // a wave's LDS area (the partial piece lands whole)
constexpr uint32_t kGbA = kPfMT * kGbKC * 2;          // 32 KiB token rows
constexpr uint32_t kGbS = 8 * kPfMT * 4;              // 2 KiB sub-block sums
constexpr uint32_t kGbLds = kGbA + kGbS + kWsWaves * kGbArea;   // 74 KiB

__global__ __launch_bounds__(64 * kWsWaves, 4) void k_pf_gateup_f16(PrefillArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t gb_lds[];
    __shared__ int s_item;
    __shared__ int s_exp[kPfMT];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, col = lane & 15, kg = lane >> 4;
    uint16_t *ab = (uint16_t *)gb_lds;
    float *sb = (float *)(gb_lds + kGbA);
    uint8_t *wb = gb_lds + kGbA + kGbS + w * kGbArea;    // [gate 16 x 144 | up 16 x 144]
    const int H = a.H, nsb = H / 32, NQ = H / kGbKC, nfg = a.F / kWsRows;
    const uint32_t rowb = (uint32_t)(H / 256) * 144;
    const int n_items = *a.n_tiles * nfg;
    for (;;) {
        if (tid == 0) s_item = atomicAdd(a.n_tiles + 2, 1);
        __syncthreads();
        const int item = s_item;
        if (item >= n_items) break;
        const int ti = item / nfg, fg = item - ti * nfg;
        const int tile = a.tiles[4 * ti + 3];                    // tiles in decreasing cost
        const int4 tl = *(const int4 *)(a.tiles + 4 * tile);
        const bool shared = tl.x == a.E;
        const uint8_t *blob = shared ? a.shared : a.experts + (uint64_t)tl.x * a.stride;
        const uint8_t *w0 = blob + (uint64_t)(fg * kWsRows + 16 * w) * rowb;
        const uint32_t up_off = (uint32_t)(shared ? a.sh_gate_size : a.gate_size);
        const int p0 = tl.y, n = tl.z, nb = (n + 15) >> 4;
        const int tok = a.pair_tok[p0 + min(lane, n - 1)];    // token of tile row lane
        if (w == 0) s_exp[lane] = a.xexp[tok];
        // step q: this wave's weights, then the token rows and their sub-block sums
        auto issue_w = [&](int q) {
#pragma unroll
            for (int i = 0; i < kGbPieces; i++) {   // piece i, lane l: byte o = 1024 i + 16 l of [gate | up],
                // row (o mod 2304) / 144; lanes past the step's bytes re-read its last 16
                const uint32_t o = min(i * 1024u + lane * 16u, kGbW - 16);
                const uint32_t oo = o < kGbHalf ? o : o - kGbHalf;
                const uint32_t off = (oo / 144) * rowb + oo % 144 + (o >= kGbHalf ? up_off : 0u) + 144u * q;
                __builtin_amdgcn_global_load_lds((const void *)(w0 + off),
                                                 (__attribute__((address_space(3))) void *)(wb + i * 1024), 16, 0, 0);
            }
        };
        auto issue_x = [&](int q) {
            for (int q2 = w; q2 < 8 * nb; q2 += kWsWaves) {      // two token rows per wave instruction
                const int m = 2 * q2 + (lane >> 5), c = (lane & 31) ^ (m & 15);
                const uint16_t *src = a.x16 + (uint64_t)__builtin_amdgcn_ds_bpermute(4 * m, tok) * H + q * kGbKC + 8 * c;
                __builtin_amdgcn_global_load_lds((const void *)src,
                                                 (__attribute__((address_space(3))) void *)(ab + 2 * q2 * kGbKC), 16, 0, 0);
            }
            if (w < 8)                                           // one sub-block's token sums per instruction
                __builtin_amdgcn_global_load_lds((const void *)(a.xsum + (uint64_t)tok * nsb + q * 8 + w),
                                                 (__attribute__((address_space(3))) void *)(sb + w * kPfMT), 4, 0, 0);
        };
        auto run = [&](auto NBC) {
            constexpr int NB = decltype(NBC)::value;
            f32x4 gA[NB], uA[NB];
#pragma unroll
            for (int b = 0; b < NB; b++) { gA[b] = (f32x4){0.f, 0.f, 0.f, 0.f}; uA[b] = gA[b]; }
            for (int q = 0; q < NQ; q++) {
                issue_w(q);
                issue_x(q);
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();                               // everyone's loads of step q have landed
                // Lane group kg owns sub-blocks 2 kg and 2 kg + 1 of the super-block
                // (MFMA (c, h): lane group kg's 8 values are values 8c..8c+7 of
                // sub-block 2 kg + h; the token operand is read in the same
                // order), so each lane decodes two (scale, min) pairs instead of
                // all eight.
                auto pass = [&](const uint8_t *rw, f32x4 (&acc)[NB]) {
                    const uint4 hw = *(const uint4 *)rw;
                    f16x2 sp[2], nsp[2];
                    float bm[2];                               // -dmin * m of sub-block 2 kg + h of row col
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        uint32_t sc, mn;
                        q4_scale_min(hw, 2 * kg + h, sc, mn);
                        // sc as an fp16 pair: bits 0x6400 | sc = 1024 + sc, minus 1024
                        q4_scale_f16(sc, h, sp[h], nsp[h]);
                        bm[h] = -h2f(hw.x >> 16) * (float)mn;
                    }
                    f32x4 dd[NB];
#pragma unroll
                    for (int tb = 0; tb < NB; tb++) dd[tb] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const uint2 qw = *(const uint2 *)(rw + 16 + 32 * kg + 8 * c);   // sub-blocks 2 kg, 2 kg + 1
#pragma unroll
                        for (int h = 0; h < 2; h++) {
                            const f16x8 bw = q4_codes_f16(qw, h, sp[h], nsp[h]);
                            const int chunk = 8 * kg + 4 * h + c;  // values 32 (2 kg + h) + 8 c
#pragma unroll
                            for (int tb = 0; tb < NB; tb++) {
                                const int m = 16 * tb + col;
                                const f16x8 av = *(const f16x8 *)(ab + m * kGbKC + 8 * (chunk ^ (m & 15)));
                                dd[tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bw, dd[tb], 0, 0, 0);
                            }
                        }
                        __builtin_amdgcn_sched_barrier(0);
                    }
                    const float d = h2f(hw.x);
#pragma unroll
                    for (int tb = 0; tb < NB; tb++) {
#pragma unroll
                        for (int i = 0; i < 4; i++) acc[tb][i] = fmaf(d, dd[tb][i], acc[tb][i]);
#pragma unroll
                        for (int h = 0; h < 2; h++) {   // A: S of token 16 tb + col, sub-block 2 kg + h
                            const float sa = sb[(2 * kg + h) * kPfMT + 16 * tb + col];
                            acc[tb] = __builtin_amdgcn_mfma_f32_16x16x4f32(sa, bm[h], acc[tb], 0, 0, 0);
                        }
                    }
                };
                pass(wb + col * 144, gA);
                pass(wb + kGbHalf + col * 144, uA);
                __syncthreads();                               // the step's LDS is free for the next one
            }
            const int row = fg * kWsRows + 16 * w + col;
#pragma unroll
            for (int tb = 0; tb < NB; tb++) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int m = 16 * tb + 4 * kg + i;
                    if (m < n) {
                        const int sx = s_exp[m];
                        const float g = ldexpf(gA[tb][i], sx), u = ldexpf(uA[tb][i], sx);
                        const float val = (g / (1.0f + expf(-g))) * u;
                        const __bf16 hi = (__bf16)val;
                        const __bf16 lo = (__bf16)(val - (float)hi);
                        const uint64_t o = (uint64_t)(p0 + m) * a.F + row;
                        a.act_hi[o] = __builtin_bit_cast(uint16_t, hi);
                        a.act_lo[o] = __builtin_bit_cast(uint16_t, lo);
                    }
                }
            }
        };
        switch (nb) {
            case 1: run(std::integral_constant<int, 1>{}); break;
            case 2: run(std::integral_constant<int, 2>{}); break;
            case 3: run(std::integral_constant<int, 3>{}); break;
            default: run(std::integral_constant<int, 4>{}); break;
        }
        __syncthreads();                                       // s_item and s_exp are free
    }
}

constexpr int kPfDownWaves = 8;                   // 8 waves x 32 rows = 256 weight rows per work-group

template <int DT, int NW = kPfDownWaves>
__global__ __launch_bounds__(NW * 64) void k_pf_down(PrefillArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t dxs[];   // 2 buffers x {hi, lo} tiles
    int tile, rbk;
    pf_tile_of(a.H / (32 * NW), tile, rbk);
    if (a.down_sel == 2) {   // the shared expert's tiles only: a grid over ceil(T / kPfMT) of them
        if (tile >= (a.T + kPfMT - 1) / kPfMT) return;
        tile += a.n_tiles[5];
    } else if (tile >= *a.n_tiles) {
        return;
    }
    const int4 tl = *(const int4 *)(a.tiles + 4 * tile);
    const int e = tl.x, p0 = tl.y, n = tl.z;
    if (a.down_sel == 1 && e == a.E) return;                // the routed experts only
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, col = lane & 15, kg = lane >> 4;
    const bool shared = e == a.E;
    const uint8_t *blob = shared ? a.shared : a.experts + (uint64_t)e * a.stride;
    const uint64_t down_off = shared ? a.sh_gate_size + a.sh_up_size : a.gate_size + a.up_size;
    const int row = rbk * (32 * NW) + 32 * wave + col;   // rows row, row + 16
    const uint64_t db = (uint64_t)(a.F / 256) * PfDec<DT>::BLOCK;
    const uint8_t *drow = blob + down_off + (uint64_t)row * db, *drow1 = drow + 16 * db;
    const int nb = (n + 15) >> 4, NK = a.F / 256;
    f32x4 acc[2][4];
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int b = 0; b < 4; b++) acc[h][b] = (f32x4){0, 0, 0, 0};
    auto stage = [&](int kb) {   // first half of the waves stages hi, second half lo
        constexpr int HW = NW / 2;
        uint16_t *buf = dxs + (kb & 1) * 2 * kPfTile + (wave / HW) * kPfTile;
        const uint16_t *plane = (wave / HW) ? a.act_lo : a.act_hi;
        const int lane_ = threadIdx.x & 63, w4 = wave % HW;
        for (int q = w4; q < nb * 8; q += HW) {
            const int m = 2 * q + (lane_ >> 5), cs = lane_ & 31;
            const int c = cs ^ (m & 15);
            const uint16_t *src = plane + (uint64_t)(p0 + (m < n ? m : 0)) * a.F + kb * 256 + 8 * c;
            __builtin_amdgcn_global_load_lds((const void *)src,
                                             (__attribute__((address_space(3))) void *)(buf + q * 512), 16, 0, 0);
        }
    };
    stage(0);
    auto s0_next = PfDec<DT>::load(drow, kg);
    auto s1_next = PfDec<DT>::load(drow1, kg);
    for (int kb = 0; kb < NK; kb++) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        const auto s0 = s0_next;
        const auto s1 = s1_next;
        if (kb + 1 < NK) {
            stage(kb + 1);
            s0_next = PfDec<DT>::load(drow + (uint64_t)(kb + 1) * PfDec<DT>::BLOCK, kg);
            s1_next = PfDec<DT>::load(drow1 + (uint64_t)(kb + 1) * PfDec<DT>::BLOCK, kg);
        }
        const uint16_t *xh = dxs + (kb & 1) * 2 * kPfTile, *xl = xh + kPfTile;
#pragma unroll
        for (int ch = 0; ch < 8; ch++) {
            const bf16x8 b0 = as_bf16x8(pf_decode<DT>(s0, ch, kg));
            const bf16x8 b1 = as_bf16x8(pf_decode<DT>(s1, ch, kg));
#pragma unroll
            for (int b = 0; b < 4; b++) {
                if (b < nb) {
                    const int o = pf_swz(16 * b + col, 4 * ch + kg);
                    const bf16x8 ah = *(const bf16x8 *)(xh + o), al = *(const bf16x8 *)(xl + o);
                    acc[0][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, b0, acc[0][b], 0, 0, 0);
                    acc[0][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, b0, acc[0][b], 0, 0, 0);
                    acc[1][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, b1, acc[1][b], 0, 0, 0);
                    acc[1][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, b1, acc[1][b], 0, 0, 0);
                }
            }
        }
    }
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int b = 0; b < 4; b++) {
            if (b >= nb) break;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 16 * b + 4 * kg + i;
                if (m < n) a.outp[(uint64_t)(p0 + m) * a.H + row + 16 * h] = acc[h][b][i];
            }
        }
}

// ------------------------------------------------------------ Q6_K down on fp16 operands
// Activation prep, one wave per pair row: v = hi + lo (the fp32 SwiGLU value
// as the gate/up kernels store it, exactly), s = the power of two that brings
// max|v| into [2^14, 2^15), and the row is rewritten in place (over the hi
// plane) as fp16(v * 2^-s); s goes to pexp. Lane l owns the 8-value chunks l,
// l + 64, ... (every load and store instruction covers 1 KiB contiguous),
// held in registers between the maximum (shuffles) and the rewrite.
constexpr int kApWaves = 4;

__global__ __launch_bounds__(64 * kApWaves) void k_pf_actprep_w(PrefillArgs a, int n_pairs) {
    const int lane = threadIdx.x & 63, p = blockIdx.x * kApWaves + (threadIdx.x >> 6);
    if (p >= n_pairs) return;
    const int F = a.F, nc = F / 8;                         // 8-value chunks; lane takes lane + 64 i
    uint16_t *hi = a.act_hi + (uint64_t)p * F;
    const uint16_t *lo = a.act_lo + (uint64_t)p * F;
    constexpr int kMaxI = 8;                               // F <= 4096
    float v[kMaxI][8];
    float m = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxI; i++) {
        const int c = lane + 64 * i;
        if (c < nc) {
            const uint4 h4 = *(const uint4 *)(hi + 8 * c), l4 = *(const uint4 *)(lo + 8 * c);
            const uint32_t hw[4] = {h4.x, h4.y, h4.z, h4.w}, lw[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                v[i][2 * q] = bf2f(hw[q] & 0xFFFFu) + bf2f(lw[q] & 0xFFFFu);
                v[i][2 * q + 1] = bf2f(hw[q] >> 16) + bf2f(lw[q] >> 16);
            }
#pragma unroll
            for (int e = 0; e < 8; e++) m = fmaxf(m, fabsf(v[i][e]));
        }
    }
    m = wave_max(m);
    int E = 0;
    frexpf(m, &E);
    const int sx = E - 15;
#pragma unroll
    for (int i = 0; i < kMaxI; i++) {
        const int c = lane + 64 * i;
        if (c < nc) {
            uint32_t o[4];
#pragma unroll
            for (int q = 0; q < 4; q++)
                o[q] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)ldexpf(v[i][2 * q], -sx)) |
                       ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)ldexpf(v[i][2 * q + 1], -sx)) << 16);
            *(uint4 *)(hi + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
    if (lane == 0) a.pexp[p] = sx;
}

// The Q6_K down projection with B = fp16(q - 32) * fp16(d * sc) (one v_perm,
// one v_pk_add_f16 and one v_pk_mul_f16 per two codes; both roundings are
// nearest-even, 2^-11 relative at most) against the fp16 activation rows of
// k_pf_actprep, one MFMA per operand; the epilogue applies the pair's 2^s.
// One activation plane halves the LDS of k_pf_down (64 KiB for two buffers).
// One persistent work-group per CU (up to 256 VGPRs, two waves per SIMD) loops over the
// items (tile, 256 rows) of its XCD: the next step's activation rows and
// weights are requested before the current step is multiplied — the last
// step of an item requests the next item's first, so no item starts on an
// empty pipeline — and with untracked direct-to-LDS loads and no spill
// reloads nothing in the step waits for them (config 5: 0.807 ms per
// prefill against 0.817 ms for one work-group per item; that kernel, 341 µs,
// against 358 µs for two work-groups per CU at 128 VGPRs, whose spill
// reloads waited for every outstanding load).
constexpr int kPfD16Waves = 8, kPfD16PerCU = 1;   // waves per work-group (32 rows each), work-groups per CU
constexpr int kPfD16Tile = 2 * kPfTile;           // activation rows of a double tile (128 pairs) per step
// A super-block's register image for either down type of a launch (the
// routed RT, the shared ST), so that one item's loads can be in flight while
// an item of the other type is multiplied.
struct PfRaw { uint32_t r[20]; };
template <int T>
FO_DEV void pf_load_raw(PfRaw &w, const uint8_t *p, int kg) {
    const typename PfDec<T>::Sb s = PfDec<T>::load(p, kg);
    static_assert(sizeof(s) <= sizeof(PfRaw), "super-block image too large");
    __builtin_memcpy(&w, &s, sizeof(s));
}
template <int T>
FO_DEV typename PfDec<T>::Sb pf_sb(const PfRaw &w) {
    typename PfDec<T>::Sb s;
    __builtin_memcpy(&s, &w, sizeof(s));
    return s;
}

template <int RT, int ST>   // Q6_K: fp16(q - 32) * fp16(d * sc); Q8_0: fp16(d * q); Q4_K / Q5_K: fp16(exact value)
__global__ __launch_bounds__(kPfD16Waves * 64, kPfD16PerCU * kPfD16Waves / 4) void k_pf_down16(PrefillArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint16_t d16s[];   // 2 buffers x double tile
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), col = lane & 15, kg = lane >> 4;
    // items (double tile of up to 128 pairs of one expert, block of 256
    // rows: the expert's weights are read and decoded once per 128 pairs;
    // 188 -> 164 us at config 5 against 64-pair tiles) of this work-group's
    // XCD (work-group i
    // runs on XCD i % 8): the XCD takes row blocks x, x + 8 of every tile, in
    // decreasing tile cost (the order k_pf_group records), so the XCDs get like
    // work and all tiles of one expert read a row block through the same L2
    // (an expert's tiles are neighbours in that order; down16 HBM reads -15 %
    // against every eighth tile per XCD); its work-groups take its items
    // u = i / 8, + G8, ..., the costliest first
    // thin experts: k_pf_down_thin; the shared expert alone: tiles of 32
    // pairs, so that its items (16 row blocks each) reach every work-group
    constexpr int kShTile = 32;
    const int nt = a.d16_shared ? (a.T + kShTile - 1) / kShTile : a.n_tiles[a.thin_down ? 4 : 3];
    const int nrb = a.H / (32 * kPfD16Waves);
    const int x = blockIdx.x & 7, G8 = gridDim.x >> 3;
    const int nrbx = (nrb - x + 7) >> 3, n_u = nt * nrbx;     // row blocks x, x + 8, ... of every tile
    const uint64_t dbR = (uint64_t)(a.F / 256) * PfDec<RT>::BLOCK, dbS = (uint64_t)(a.F / 256) * PfDec<ST>::BLOCK;
    const int NK = a.F / 256;
    struct Item { int p0, n, row; const uint8_t *drow; uint64_t db; bool ok, sh; };
    auto item_at = [&](int u) {
        Item it;
        const int tl = u / nrbx, rbk = x + 8 * (u - tl * nrbx);
        it.ok = u < n_u;
        int4 t4;
        if (a.d16_shared) {   // one expert's T pairs in token order: the shared expert's follow the
                              // T * k routed ones; a one-expert pass's are all of them
            const int i = it.ok ? tl : 0;
            const int e0 = a.one_expert ? 0 : a.E, base = a.one_expert ? 0 : a.T * a.k;
            t4 = make_int4(e0, base + kShTile * i, min(kShTile, a.T - kShTile * i), 0);
        } else {
            const int tile = a.dtiles[4 * (it.ok ? tl : 0) + 3];
            t4 = *(const int4 *)(a.dtiles + 4 * tile);
        }
        const bool shared = t4.x == a.E;
        const uint8_t *blob = shared ? a.shared : a.experts + (uint64_t)t4.x * a.stride;
        const uint64_t down_off = shared ? a.sh_gate_size + a.sh_up_size : a.gate_size + a.up_size;
        it.p0 = t4.y; it.n = t4.z;
        it.row = rbk * (32 * kPfD16Waves) + 32 * wave + col;   // rows row, row + 16
        it.sh = shared;
        it.db = shared ? dbS : dbR;
        it.drow = blob + down_off + (uint64_t)it.row * it.db;
        return it;
    };
    // a step's activation rows land while the previous step is multiplied:
    // the direct-to-LDS loads are untracked by the compiler (a tracked one
    // makes every LDS read of the current step wait for them); the wait at
    // the top of each step covers them
    auto stage = [&](const Item &it, int kb, int buf_i) {
        const uint32_t buf = lds_addr(d16s + buf_i * kPfD16Tile);
        const int nb = (it.n + 15) >> 4;
        for (int q = wave; q < nb * 8; q += kPfD16Waves) {
            const int m = 2 * q + (lane >> 5), cs = lane & 31;
            const int c = cs ^ (m & 15);
            const uint16_t *src = a.act_hi + (uint64_t)(it.p0 + (m < it.n ? m : 0)) * a.F + kb * 256 + 8 * c;
            dma16_untracked(src, buf + q * 1024);
        }
    };
    // fp16 operand of chunk ch (values 128n + 32t + 8kg .. +7, scale group
    // 8n + 2t + kg/2) of one super-block
    const f16x2 m1056 = {(_Float16)-1056.f, (_Float16)-1056.f};
    const f16x2 m1152 = {(_Float16)-1152.f, (_Float16)-1152.f};
    auto dec = [&](auto TC, const auto &sb, int ch) {
      if constexpr (decltype(TC)::value == GGML_TYPE_Q4_K || decltype(TC)::value == GGML_TYPE_Q5_K) {
        return pf_decode_f16_k<decltype(TC)::value>(sb, ch);
      } else if constexpr (decltype(TC)::value == GGML_TYPE_Q8_0) {
        // block ch, codes 8 kg .. 8 kg + 7: byte b ^ 0x80 = q + 128 becomes the
        // fp16 1024 + q + 128 by a byte permute; minus 1152 is q exactly; times d
        // (fp16) is the one rounding
        const uint2 q = sb.q[ch];
        const uint32_t u0 = q.x ^ 0x80808080u, u1 = q.y ^ 0x80808080u;
        const uint32_t dh = (sb.d[ch >> 1] >> (16 * (ch & 1))) & 0xFFFFu;
        const f16x2 d2 = __builtin_bit_cast(f16x2, dh | (dh << 16));
        const uint32_t pw[4] = {__builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u),
                                __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u),
                                __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u),
                                __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)};
        u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; i++)
            r[i] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, pw[i]) + m1152) * d2);
        return __builtin_bit_cast(f16x8, r);
      } else {
        const int nn = ch >> 2, t = ch & 3;
        const uint2 l = sb.ql[2 * nn + (t & 1)];
        const uint2 h = sb.qh[nn];
        const int ls = 4 * (t >> 1), hs = 2 * t;
        const uint32_t c0 = ((l.x >> ls) & 0x0F0F0F0Fu) | (((h.x >> hs) & 0x03030303u) << 4);
        const uint32_t c1 = ((l.y >> ls) & 0x0F0F0F0Fu) | (((h.y >> hs) & 0x03030303u) << 4);
        const int si = 8 * nn + 2 * t + (kg >> 1);
        const uint32_t scw = si < 4 ? sb.sc.x : si < 8 ? sb.sc.y : si < 12 ? sb.sc.z : sb.sc.w;
        const int scv = (int)(int8_t)((scw >> (8 * (si & 3))) & 0xFFu);
        const _Float16 dsc = (_Float16)(h2f(sb.d) * (float)scv);   // exact product, one rounding
        const f16x2 ds2 = {dsc, dsc};
        const uint32_t pw[4] = {__builtin_amdgcn_perm(0x64646464u, c0, 0x04010400u),
                                __builtin_amdgcn_perm(0x64646464u, c0, 0x04030402u),
                                __builtin_amdgcn_perm(0x64646464u, c1, 0x04010400u),
                                __builtin_amdgcn_perm(0x64646464u, c1, 0x04030402u)};
        u32x4 r;
#pragma unroll
        for (int i = 0; i < 4; i++)   // (1024 + q) - 1056 = q - 32 exactly, then one rounding
            r[i] = __builtin_bit_cast(uint32_t, (__builtin_bit_cast(f16x2, pw[i]) + m1056) * ds2);
        return __builtin_bit_cast(f16x8, r);
      }
    };
    int u = blockIdx.x >> 3;
    Item cur = item_at(u);
    if (!cur.ok) return;
    int gs = 0;                                       // steps done: LDS buffer gs & 1
    stage(cur, 0, 0);
    PfRaw s0_next, s1_next;
    auto load2 = [&](const Item &it, int kb) {   // the item's two row blocks, super-block kb
        const uint8_t *p = it.drow + (uint64_t)kb * (it.sh ? PfDec<ST>::BLOCK : PfDec<RT>::BLOCK);
        if (it.sh) { pf_load_raw<ST>(s0_next, p, kg); pf_load_raw<ST>(s1_next, p + 16 * it.db, kg); }
        else { pf_load_raw<RT>(s0_next, p, kg); pf_load_raw<RT>(s1_next, p + 16 * it.db, kg); }
    };
    load2(cur, 0);
    // the token-block count is a compile-time constant of an item's steps
    // (fewer live registers for small tiles: no spill reloads, whose waits
    // would also wait for the next step's loads); the last step requests the
    // next item's first
    auto run = [&](auto NBC, auto TC, const Item &nxt) {
        constexpr int NB = decltype(NBC)::value, T = decltype(TC)::value;
        f32x4 acc[2][NB];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int b = 0; b < NB; b++) acc[h][b] = (f32x4){0, 0, 0, 0};
        for (int kb = 0; kb < NK; kb++) {
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
            const auto s0 = pf_sb<T>(s0_next);
            const auto s1 = pf_sb<T>(s1_next);
            if (kb + 1 < NK) {
                stage(cur, kb + 1, (gs + 1) & 1);
                load2(cur, kb + 1);
            } else if (nxt.ok) {
                stage(nxt, 0, (gs + 1) & 1);
                load2(nxt, 0);
            }
            const uint16_t *xh = d16s + (gs & 1) * kPfD16Tile;
#pragma unroll
            for (int ch = 0; ch < 8; ch++) {
                const f16x8 b0 = dec(TC, s0, ch), b1 = dec(TC, s1, ch);
#pragma unroll
                for (int b = 0; b < NB; b++) {
                    const f16x8 av = *(const f16x8 *)(xh + pf_swz(16 * b + col, 4 * ch + kg));
                    acc[0][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b0, acc[0][b], 0, 0, 0);
                    acc[1][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, b1, acc[1][b], 0, 0, 0);
                }
            }
            gs++;
        }
#pragma unroll
        for (int b = 0; b < NB; b++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = 16 * b + 4 * kg + i;
                if (m < cur.n) {
                    const int sx = a.pexp[cur.p0 + m];
#pragma unroll
                    for (int h = 0; h < 2; h++)
                        a.outp[(uint64_t)(cur.p0 + m) * a.H + cur.row + 16 * h] = ldexpf(acc[h][b][i], sx);
                }
            }
        }
    };
    for (;;) {
        u += G8;
        const Item nxt = item_at(u);
        auto by_nb = [&](auto TC) {
            switch ((cur.n + 15) >> 4) {
                case 1: run(std::integral_constant<int, 1>{}, TC, nxt); break;
                case 2: run(std::integral_constant<int, 2>{}, TC, nxt); break;
                case 3: run(std::integral_constant<int, 3>{}, TC, nxt); break;
                case 4: run(std::integral_constant<int, 4>{}, TC, nxt); break;
                case 5: run(std::integral_constant<int, 5>{}, TC, nxt); break;
                case 6: run(std::integral_constant<int, 6>{}, TC, nxt); break;
                case 7: run(std::integral_constant<int, 7>{}, TC, nxt); break;
                default: run(std::integral_constant<int, 8>{}, TC, nxt); break;
            }
        };
        if constexpr (RT == ST) by_nb(std::integral_constant<int, RT>{});
        else if (cur.sh) by_nb(std::integral_constant<int, ST>{});
        else by_nb(std::integral_constant<int, RT>{});
        if (!nxt.ok) break;
        cur = nxt;
    }
}
#pragma clang fp contract(on)

// ------------------------------------------------------------ Q6_K down of the thin tiles
// Tiles of at most kPfThin pairs (k_pf_group orders them last) run the
// decode matvec's integer path instead of k_pf_down16: a 16-row weight tile
// streamed with 1 KiB loads into LDS (the next tile in flight) and, per pair,
// the Q6_K super-block dot on v_mfma_i32_16x16x64_i8 against the pair's
// activation as int8 limbs (q6k_mfma.h, as k_matvec_q6k_tile). The limbs are
// prepared from the fp16 activation rows k_pf_actprep_w wrote (exactly: a
// fp16 value needs 11 of the 22 fixed-point bits), and the pair's 2^s is
// applied to the result. The code building is shared by the tile's pairs, so
// a weight costs ~0.75 + 0.5 n VALU instructions per code against ~3.4 for
// the fp16 operand decode of k_pf_down16, whose 16-token MFMA blocks a thin
// tile leaves mostly empty. Work unit = (thin tile, kPfThinWaves *
// kPfThinTPW * 16 rows): the work-group's waves prepare one pair's
// activation each into LDS shared by all of them (one copy per work-group,
// so that 8 waves per CU fit in LDS: with a copy per one-wave work-group
// only 5 did: 121.5 -> 109.3 us at config 5), then each wave streams its
// kPfThinTPW tiles; units dealt round-robin; F == 1024. (4 waves x 4 tiles,
// 8 x 4, 8 x 2, 2 x 8: 115 / 119 / 127 / 122 us; the results held in LDS
// and stored once per unit: no change.)
constexpr int kPfThinTPW = 8, kPfThinWaves = 4;
constexpr int kPfThinF = 1024;                                     // the one F this kernel is built for
constexpr uint32_t kPfThinRow = kPfThinF / 256 * 210;              // Q6_K row: 840 bytes
constexpr uint32_t kPfThinX = 3 * kPfThinF + kPfThinF / 16 * 8;    // one pair's prepared activation
constexpr uint32_t kPfThinZero = 304;                              // zero A operands (as kT6Zero)
constexpr uint32_t kPfThinTile = 16 * kPfThinRow;                  // 13,440 bytes
constexpr int kPfThinUnitRows = 16 * kPfThinTPW * kPfThinWaves;    // 512 rows
// 64 lanes x 16 activation values = one F = 1024 row per pair (lane = 16-value group)
static_assert(kPfThinF == 64 * 16 && kPfThinRow == 840, "k_pf_down_thin's lane layout covers F = 1024 only");
static_assert(kPfThin <= kPfThinWaves, "one wave prepares each pair's activation");

// Whether the Q6_K down projection's thin tiles take k_pf_down_thin (the one
// place that decides; k_pf_group orders thin tiles last whatever it says).
__host__ inline bool pf_thin_down(const PrefillArgs &a) {
    return a.down_type == GGML_TYPE_Q6_K && a.F == kPfThinF && a.H % kPfThinUnitRows == 0;
}
constexpr uint32_t kPfThinLds = kPfThin * kPfThinX + kPfThinZero + kPfThinWaves * kPfThinTile;   // 68.3 KiB

__global__ __launch_bounds__(64 * kPfThinWaves) void k_pf_down_thin(PrefillArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sx[];
    // the pairs' 2^s, read with the activations: a global load inside the
    // tile loop would wait for the next tile's loads (issued before it)
    __shared__ int s_pe[kPfThin];
    constexpr int NV = (kPfThinTile + 1023) / 1024;
    constexpr uint32_t rb = kPfThinRow, limb_bytes = 3 * kPfThinF;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    uint8_t *zero = sx + kPfThin * kPfThinX;
    uint8_t *tb = zero + kPfThinZero + wv * kPfThinTile;
    const int n_thick = a.n_tiles[1], n_thin = a.n_tiles[0] - n_thick;
    const int upt = a.H / kPfThinUnitRows, nunits = n_thin * upt;
    if ((int)threadIdx.x < kPfThinZero / 16) *(uint4 *)(zero + 16 * threadIdx.x) = make_uint4(0, 0, 0, 0);
    const int r = lane & 15, g = lane >> 4, n = g >> 1, j = g & 1, L = r & 3;
    const bool valid = (r >> 2) == g && L < 3;
    const uint32_t aoff = (8 * n + j) * 48 + 16 * L, soff = limb_bytes + (8 * n + j) * 8;
    for (int u = blockIdx.x; u < nunits; u += gridDim.x) {
        const int ti = n_thick + u / upt, row0 = (u % upt) * kPfThinUnitRows + wv * 16 * kPfThinTPW;
        const int tile = a.tiles[4 * ti + 3];
        const int4 t4 = *(const int4 *)(a.tiles + 4 * tile);
        const bool shared = t4.x == a.E;
        const uint8_t *blob = shared ? a.shared : a.experts + (uint64_t)t4.x * a.stride;
        const uint64_t down_off = shared ? a.sh_gate_size + a.sh_up_size : a.gate_size + a.up_size;
        const uint8_t *W = blob + down_off + (uint64_t)row0 * rb;
        const int p0 = t4.y, np = t4.z;                  // np <= kPfThin
        uint4 v[NV];
        auto issue = [&](int tt) {
            const uint8_t *tp = W + (uint64_t)tt * kPfThinTile;
#pragma unroll
            for (int i = 0; i < NV; i++) v[i] = ldw16(tp + min(i * 1024u + lane * 16u, kPfThinTile - 16));
        };
        issue(0);
        __syncthreads();                                 // the previous unit's LDS reads are done
        if (wv < np) {                                   // wave m prepares pair m (lane = 16-value group)
            const uint16_t *src = a.act_hi + (uint64_t)(p0 + wv) * a.F + 16 * lane;
            const uint4 h0 = *(const uint4 *)src, h1 = *(const uint4 *)(src + 8);
            const uint32_t w[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
            float vals[16];
#pragma unroll
            for (int q = 0; q < 8; q++) {
                vals[2 * q] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[q] & 0xFFFFu));
                vals[2 * q + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[q] >> 16));
            }
            int limb[kLimbs][4];
            float scale, sum;
            prep_group_vals<16>(vals, limb, scale, sum);
            uint8_t *xm = sx + wv * kPfThinX;
#pragma unroll
            for (int Lq = 0; Lq < kLimbs; Lq++)
                *(uint4 *)(xm + lane * 48 + 16 * Lq) = make_uint4(limb[Lq][0], limb[Lq][1], limb[Lq][2], limb[Lq][3]);
            *(float2 *)(xm + limb_bytes + lane * 8) = make_float2(scale, -32.f * sum);
            if (lane == 0) s_pe[wv] = a.pexp[p0 + wv];
        }
        __syncthreads();
        for (int tt = 0; tt < kPfThinTPW; tt++) {
#pragma unroll
            for (int i = 0; i < NV; i++) *(uint4 *)(tb + min(i * 1024u + lane * 16u, kPfThinTile - 16)) = v[i];
            if (tt + 1 < kPfThinTPW) issue(tt + 1);
            Q6kSlot qs[4];
#pragma unroll
            for (int b = 0; b < 4; b++) q6k_slot_load(qs[b], tb + r * rb + b * 210, n, j);
#pragma unroll 1
            for (int m = 0; m < np; m++) {
                const uint8_t *xm = sx + m * kPfThinX;
                float acc = 0.f;
#pragma unroll
                for (int b = 0; b < 4; b++)
                    acc += q6k_sb_dot_mfma(qs[b], valid ? xm + aoff + 768 * b : zero, xm + soff + 128 * b, j);
                acc += __shfl_xor(acc, 16);
                acc += __shfl_xor(acc, 32);
                if (g == 0)
                    a.outp[(uint64_t)(p0 + m) * a.H + row0 + 16 * tt + r] = ldexpf(acc, s_pe[m]);
            }
        }
    }
}

// ============================================================ P6 combine
// One work-group per (token, kCombCols columns); each thread owns float4 columns and requests all
// of the token's pair rows for a column before summing them in rank order. The pair rows are read
// once: non-temporal loads (20.7 against 21.8 us at config 5; 512 or 2048 columns per work-group
// 25.7 / 23.0 us).
constexpr int kCombCols = 1024;   // columns of one token per work-group

__global__ __launch_bounds__(256) void k_pf_combine(PrefillArgs a) {
    __shared__ int s_pp[kMaxK + 1];
    __shared__ float s_w[kMaxK + 1];
    const int t = blockIdx.x, K1 = a.k + 1, n = a.k + (a.shared ? 1 : 0);
    const int c0 = blockIdx.y * kCombCols / 4, c1 = min(a.H / 4, c0 + kCombCols / 4);   // float4 columns
    if ((int)threadIdx.x < K1) {
        s_pp[threadIdx.x] = a.pairpos[(uint64_t)t * K1 + threadIdx.x];
        s_w[threadIdx.x] = a.w[(uint64_t)t * K1 + threadIdx.x];
    }
    __syncthreads();
    for (int i4 = c0 + threadIdx.x; i4 < c1; i4 += 256) {
        float4 o[kMaxK + 1];
#pragma unroll
        for (int r = 0; r <= kMaxK; r++)
            if (r < n) {
                const uint4 u = ldw16((const uint8_t *)(a.outp + (uint64_t)s_pp[r] * a.H + 4 * i4));
                o[r] = make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
            }
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int r = 0; r < kMaxK; r++)
            if (r < a.k) {
                acc.x = acc.x + s_w[r] * o[r].x; acc.y = acc.y + s_w[r] * o[r].y;
                acc.z = acc.z + s_w[r] * o[r].z; acc.w = acc.w + s_w[r] * o[r].w;
            }
        if (a.shared || a.ys) {
            float4 sh = make_float4(0.f, 0.f, 0.f, 0.f);
            if (a.ys) sh = *(const float4 *)(a.ys + (uint64_t)t * a.H + 4 * i4);
#pragma unroll
            for (int r = 0; r <= kMaxK; r++)
                if (r == a.k && a.shared) sh = o[r];
            const float ws = s_w[a.k];
            acc.x = acc.x + sh.x * ws; acc.y = acc.y + sh.y * ws;
            acc.z = acc.z + sh.z * ws; acc.w = acc.w + sh.w * ws;
        }
        if (a.residual) {
            const uint2 xb = *(const uint2 *)(a.x + (uint64_t)t * a.H + 4 * i4);
            acc.x = bf2f(xb.x & 0xFFFFu) + acc.x; acc.y = bf2f(xb.x >> 16) + acc.y;
            acc.z = bf2f(xb.y & 0xFFFFu) + acc.z; acc.w = bf2f(xb.y >> 16) + acc.w;
        }
        *(float4 *)(a.out + (uint64_t)t * a.H + 4 * i4) = acc;
    }
}

__global__ void k_f32_to_bf16(const float *src, uint16_t *dst, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = __builtin_bit_cast(uint16_t, (__bf16)src[i]);
}

hipError_t launch_f32_to_bf16(const float *src, uint16_t *dst, int64_t n, hipStream_t s) {
    if (n <= 0) return hipErrorInvalidValue;
    k_f32_to_bf16<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(src, dst, n);
    return hipGetLastError();
}

// ============================================================ launcher
template <int GT, int UT>
static hipError_t launch_gateup_t(const PrefillArgs &a, hipStream_t s) {
    k_pf_gateup<GT, UT><<<pf_grid(a.F / kPfGateRows, a.max_tiles), kPfGateWaves * 64, 0, s>>>(a);
    return hipGetLastError();
}

// The k_pf_down16 type pairs built: each down type alone, and a shared Q6_K
// or Q8_0 down projection beside any routed type.
#define FO_D16_ALL \
    FO_D16(GGML_TYPE_Q4_K, GGML_TYPE_Q4_K) FO_D16(GGML_TYPE_Q5_K, GGML_TYPE_Q5_K) \
    FO_D16(GGML_TYPE_Q6_K, GGML_TYPE_Q6_K) FO_D16(GGML_TYPE_Q8_0, GGML_TYPE_Q8_0) \
    FO_D16(GGML_TYPE_Q4_K, GGML_TYPE_Q6_K) FO_D16(GGML_TYPE_Q4_K, GGML_TYPE_Q8_0) \
    FO_D16(GGML_TYPE_Q5_K, GGML_TYPE_Q6_K) FO_D16(GGML_TYPE_Q5_K, GGML_TYPE_Q8_0) \
    FO_D16(GGML_TYPE_Q6_K, GGML_TYPE_Q8_0) FO_D16(GGML_TYPE_Q8_0, GGML_TYPE_Q6_K)

hipError_t launch_prefill(const PrefillArgs &a_, hipStream_t s) {
    PrefillArgs a = a_;
    // A shared expert whose down projection has a type of its own (gate/up
    // and F as the routed experts) shares the routed gate/up GEMM as expert
    // E; the down projections run per type: bf16-operand launches first
    // (they read the hi/lo activation planes), then the fp16 Q6_K path.
    auto fp16_down = [&](int t) { (void)t; return a.F <= 4096; };   // every down type of the prefill
    const int RT = a.down_type, ST = a.sh_down_type;
    const bool sep = a.shared && ST >= 0 && ST != RT;
    // k_pf_down16 runs one type per launch: the routed experts' (its tile
    // table, the shared expert left out when its type differs) and then the
    // shared expert's pairs when its own type takes the fp16 path too
    const bool rt16 = fp16_down(RT), st16 = sep && fp16_down(ST);
    // one launch takes routed and shared tiles when its type pair is built
    // (a shared Q6_K or Q8_0 down beside any routed type)
    const bool joint = rt16 && st16 && (ST == GGML_TYPE_Q6_K || ST == GGML_TYPE_Q8_0);
    a.down_sel = 0;
    a.d16_shared = 0;
    a.dt_sel = sep && !joint ? 1 : 0;
    const bool okt = prefill_types_ok(a.gate_type, a.up_type, a.down_type);
    const int W = (a.T + 31) / 32;
    if (!okt || a.T <= 0 || a.E <= 0 || a.E > 1023 || a.k <= 0 || a.k > a.E || a.k > kMaxK ||
        a.H <= 0 || a.H % 256 || a.H % (32 * kPfDownWaves) || a.H % (32 * kPfD16Waves) || a.F <= 0 || a.F % 256 || a.F % kPfGateRows || a.E * W > kPfGroupLds ||
        a.max_tiles < prefill_max_tiles(a.T, a.k, a.E, a.shared != nullptr))
        return hipErrorInvalidValue;
    const bool fp16_gateup = a.gate_type == GGML_TYPE_Q4_K && a.up_type == GGML_TYPE_Q4_K;
    if (a.one_expert && (a.E != 1 || a.k != 1 || a.shared)) return hipErrorInvalidValue;
    bool xprep_done = a.xprep_ready != 0;
    if (a.one_expert) {
        // no router: the grouping places every token on expert 0
    } else if (a.H % (64 * kR3Waves) == 0 && a.rsplit) {
        const uint64_t pieces = prefill_router_ws_elems(a.E, a.T, a.H) / 8;   // upper bound
        const unsigned n_rt = (unsigned)std::min<uint64_t>((pieces + 255) / 256, 8192);
        if (fp16_gateup && !xprep_done && a.H % 2048 == 0) {
            k_pf_prep<<<n_rt + (a.T + kXpWaves - 1) / kXpWaves, 256, 0, s>>>(a, n_rt);
            xprep_done = true;
        } else {
            k_pf_rtile<<<n_rt, 256, 0, s>>>(a);
        }
        k_pf_router3<<<dim3((a.E + kRT - 1) / kRT, (a.T + kRT - 1) / kRT), 64 * kR3Waves, 0, s>>>(a);
    } else {
        static bool router_attr = false;   // above the 64 KiB default of dynamic LDS
        if (!router_attr) {
            hipError_t e = hipFuncSetAttribute((const void *)k_pf_router, hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)kRLds);
            if (e != hipSuccess) return e;
            router_attr = true;
        }
        k_pf_router<<<dim3((a.E + kRT - 1) / kRT, (a.T + kRT - 1) / kRT), 256, kRLds, s>>>(a);
    }
    if (!a.one_expert) k_pf_topk<<<(a.T + 3) / 4, 256, 0, s>>>(a);
    static bool lds_attr = false;   // the grouping tables may exceed the 64 KiB default
    if (!lds_attr) {
        hipError_t e = hipFuncSetAttribute((const void *)k_pf_group, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           2 * (kPfGroupLds + kMaxE) * (int)sizeof(uint32_t));
        if (e != hipSuccess) return e;
        lds_attr = true;
    }
    k_pf_group<<<1, 1024, 2 * (size_t)a.E * pf_group_stride(W) * sizeof(uint32_t), s>>>(a);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    if (fp16_gateup) {   // exact fp16 operands
        if (xprep_done) {
        } else if (a.H % 2048 == 0) {
            k_pf_xprep_w<<<(a.T + kXpWaves - 1) / kXpWaves, 64 * kXpWaves, 0, s>>>(a);
        } else {
            k_pf_xprep<<<a.T, 256, 0, s>>>(a);
        }
        static bool gb_attr = false;   // above the 64 KiB default of dynamic LDS
        if (!gb_attr) {
            hipError_t e = hipFuncSetAttribute((const void *)k_pf_gateup_f16,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)kGbLds);
            if (e != hipSuccess) return e;
            gb_attr = true;
        }
        int dev = 0, n_cu = 256;
        if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev);
        k_pf_gateup_f16<<<2 * n_cu, 64 * kWsWaves, kGbLds, s>>>(a);
        err = hipGetLastError();
    }
#define FO_GU(G, U) if (a.gate_type == G && a.up_type == U) err = launch_gateup_t<G, U>(a, s);
    FO_GU(GGML_TYPE_Q4_K, GGML_TYPE_Q6_K)
    FO_GU(GGML_TYPE_Q6_K, GGML_TYPE_Q4_K) FO_GU(GGML_TYPE_Q6_K, GGML_TYPE_Q6_K)
    FO_GU(GGML_TYPE_Q5_K, GGML_TYPE_Q5_K) FO_GU(GGML_TYPE_Q8_0, GGML_TYPE_Q8_0)
#undef FO_GU
    if (err != hipSuccess) return err;
    {
        const size_t lds = 4 * (size_t)kPfTile * sizeof(uint16_t);       // 128 KiB
        const unsigned grid = pf_grid(a.H / (32 * kPfDownWaves), a.max_tiles);
        static bool down_attr = false;
        if (!down_attr) {
            const void *fns[8] = {(const void *)k_pf_down<GGML_TYPE_Q4_K>, (const void *)k_pf_down<GGML_TYPE_Q5_K>,
                                  (const void *)k_pf_down<GGML_TYPE_Q6_K>, (const void *)k_pf_down<GGML_TYPE_Q8_0>,
                                  (const void *)k_pf_down<GGML_TYPE_Q4_K, 4>, (const void *)k_pf_down<GGML_TYPE_Q5_K, 4>,
                                  (const void *)k_pf_down<GGML_TYPE_Q6_K, 4>, (const void *)k_pf_down<GGML_TYPE_Q8_0, 4>};
            for (const void *f : fns) {
                const hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
                if (e != hipSuccess) return e;
            }
            down_attr = true;
        }
        auto down_bf16 = [&](int type, int sel) {
            PrefillArgs d = a;
            d.down_sel = sel;
            if (sel == 2) {   // one expert's tiles: 4-wave work-groups of 128 rows, so that they fill the CUs
                const unsigned g = pf_grid(a.H / (32 * 4), (a.T + kPfMT - 1) / kPfMT);
                if (type == GGML_TYPE_Q4_K) k_pf_down<GGML_TYPE_Q4_K, 4><<<g, 256, lds, s>>>(d);
                else if (type == GGML_TYPE_Q5_K) k_pf_down<GGML_TYPE_Q5_K, 4><<<g, 256, lds, s>>>(d);
                else if (type == GGML_TYPE_Q8_0) k_pf_down<GGML_TYPE_Q8_0, 4><<<g, 256, lds, s>>>(d);
                else k_pf_down<GGML_TYPE_Q6_K, 4><<<g, 256, lds, s>>>(d);
                return;
            }
            if (type == GGML_TYPE_Q4_K) k_pf_down<GGML_TYPE_Q4_K><<<grid, kPfDownWaves * 64, lds, s>>>(d);
            else if (type == GGML_TYPE_Q5_K) k_pf_down<GGML_TYPE_Q5_K><<<grid, kPfDownWaves * 64, lds, s>>>(d);
            else if (type == GGML_TYPE_Q8_0) k_pf_down<GGML_TYPE_Q8_0><<<grid, kPfDownWaves * 64, lds, s>>>(d);
            else k_pf_down<GGML_TYPE_Q6_K><<<grid, kPfDownWaves * 64, lds, s>>>(d);
        };
        if (!rt16) down_bf16(RT, sep ? 1 : 0);
        if (sep && !st16) down_bf16(ST, 2);
        if (rt16 || st16) {   // fp16 operands, one activation plane
            const size_t lds16 = 2 * (size_t)kPfD16Tile * sizeof(uint16_t);   // 128 KiB
            static bool d16_attr = false;
            if (!d16_attr) {
#define FO_D16(R, S) \
                if (hipFuncSetAttribute((const void *)k_pf_down16<R, S>, hipFuncAttributeMaxDynamicSharedMemorySize, \
                                        (int)lds16) != hipSuccess) return hipErrorInvalidValue;
                FO_D16_ALL
#undef FO_D16
                if (hipFuncSetAttribute((const void *)k_pf_down_thin, hipFuncAttributeMaxDynamicSharedMemorySize,
                                        (int)kPfThinLds) != hipSuccess) return hipErrorInvalidValue;
                d16_attr = true;
            }
            const int np = prefill_pairs(a.T, a.k, a.shared != nullptr);
            k_pf_actprep_w<<<(np + kApWaves - 1) / kApWaves, 64 * kApWaves, 0, s>>>(a, np);
            a.thin_down = rt16 && pf_thin_down(a);   // thin routed Q6_K experts (never the shared one here)
            int dev = 0, n_cu = 256;
            if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev);
            const unsigned g16 = (kPfD16PerCU * n_cu + 7) & ~7;   // persistent
            auto down16 = [&](int rt, int st, int shared_only) {
                PrefillArgs d = a;
                d.d16_shared = shared_only;
#define FO_D16(R, S) if (rt == R && st == S) { k_pf_down16<R, S><<<g16, kPfD16Waves * 64, lds16, s>>>(d); return; }
                FO_D16_ALL
#undef FO_D16
            };
            if (rt16) down16(RT, joint ? ST : RT, a.one_expert);   // (one expert: its pairs in 32-pair tiles)
            if (st16 && !joint) down16(ST, ST, 1);      // the shared expert alone
            if (a.thin_down) k_pf_down_thin<<<2 * n_cu, 64 * kPfThinWaves, kPfThinLds, s>>>(a);
        }
    }
    if (!a.one_expert) k_pf_combine<<<dim3(a.T, (a.H + kCombCols - 1) / kCombCols), 256, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace fo
