// kernels.hip — gfx950 decode-path kernels: activation prep, batched quantized
// matvec, router + softmax + top-k, fused gate/up/SiLU, down + weighted
// combine, and the bit-exact dequantizer.
//
// Reference counterparts (replaced, not ported): gpu_kernels.hip
// kernel_q4k_matvec_coop 1858, kernel_q6k_matvec_coop 1747,
// kernel_q8_0_matvec_coop 1901, kernel_f32_matvec_coop 2127, kernel_softmax
// 2668, kernel_top_k_parallel 2745, kernel_q4k_fused_gate_up_silu 1320,
// kernel_q6k_matvec_per_expert 1261, kernel_weighted_sum 1631,
// kernel_moe_output_residual 1647, kernel_silu_mul 1306.
#include <float.h>

#include "formats.h"
#include "kernels.h"
#include "q4k_mfma.h"
#include "q6k_mfma.h"

namespace fo {

// ============================================================ activation prep
// One group of GSZ values prepared (prep_group_regs, formats.h) and stored:
// limbs to `lp8` (kLimbs * GSZ bytes), {scale, sum} to `ss`.
template <int GSZ>
FO_DEV void prep_group(const float *__restrict__ xp, uint8_t *lp8, uint8_t *ss) {
    int limb[kLimbs][GSZ / 4];
    float scale, sum;
    prep_group_regs<GSZ>(xp, limb, scale, sum);
    uint32_t *lp = (uint32_t *)lp8;
#pragma unroll
    for (int L = 0; L < kLimbs; L++)
#pragma unroll
        for (int k = 0; k < GSZ / 4; k += 4)
            *(uint4 *)(lp + L * (GSZ / 4) + k) = make_uint4(limb[L][k], limb[L][k + 1], limb[L][k + 2], limb[L][k + 3]);
    *(float2 *)ss = make_float2(scale, sum);
}

template <int GSZ>
__global__ __launch_bounds__(256) void k_xprep(const float *__restrict__ x, uint64_t x_stride,
                                               int K, int n_vec, uint8_t *__restrict__ xq,
                                               uint64_t xq_stride) {
    const int ng = K / GSZ;
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (int64_t)ng * n_vec) return;
    const int v = (int)(gid / ng), g = (int)(gid % ng);
    uint8_t *out = xq + (uint64_t)v * xq_stride;
    prep_group<GSZ>(x + (uint64_t)v * x_stride + (uint64_t)g * GSZ, out + (uint64_t)g * (kLimbs * GSZ),
                    out + xq_limb_bytes(K) + (uint64_t)g * 8);
}

hipError_t launch_xprep(int gsz, const float *x, uint64_t x_stride, int K, int n_vec,
                        uint8_t *xq, uint64_t xq_stride_b, hipStream_t s) {
    if (K % gsz || n_vec <= 0) return hipErrorInvalidValue;
    const int64_t n = (int64_t)(K / gsz) * n_vec;
    const int blocks = (int)((n + 255) / 256);
    if (gsz == 16) k_xprep<16><<<blocks, 256, 0, s>>>(x, x_stride, K, n_vec, xq, xq_stride_b);
    else if (gsz == 32) k_xprep<32><<<blocks, 256, 0, s>>>(x, x_stride, K, n_vec, xq, xq_stride_b);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

// ============================================================ lane state
// A lane's slots: G lanes share one row (G = 64 when a row has >= 64 slots,
// else the next power of two >= S) and P = 64/G rows are processed side by
// side per pass; lane l owns slots (l % G) + G*u, u < U.
template <int U, int G>
struct Slots {
    int slot[U];
    bool ok[U];
    FO_DEV void init(int lane, int S) {
#pragma unroll
        for (int u = 0; u < U; u++) { slot[u] = (lane % G) + G * u; ok[u] = slot[u] < S; }
    }
};

// The prepared activation of a lane's slots, held in registers.
template <int T, int U>
struct XRegs {
    typename Fmt<T>::X x[U];
    template <int G>
    FO_DEV void load(const Slots<U, G> &sl, const uint8_t *xq, int K) {
#pragma unroll
        for (int u = 0; u < U; u++)
            if (sl.ok[u]) {
                int gi[Fmt<T>::NG];
                Fmt<T>::groups(sl.slot[u], gi);
                load_xslot(x[u], xq, K, gi);
            }
    }
};

template <int T, int U>
struct RowRaw { typename Fmt<T>::Raw r[U]; };

template <int T, int U, int G>
FO_DEV void load_row(RowRaw<T, U> &rr, const uint8_t *row, const Slots<U, G> &sl) {
#pragma unroll
    for (int u = 0; u < U; u++)
        if (sl.ok[u]) rr.r[u] = Fmt<T>::load(row, sl.slot[u]);
}

template <int T, int U, int G>
FO_DEV float dot_row(const RowRaw<T, U> &rr, const Slots<U, G> &sl, const XRegs<T, U> &X) {
    float a = 0.f;
#pragma unroll
    for (int u = 0; u < U; u++)
        if (sl.ok[u]) a += Fmt<T>::dot(rr.r[u], sl.slot[u], X.x[u]);
    return a;
}

// Contiguous share [t0, t1) of `total` tasks for wave w of nw.
FO_DEV void wave_share(int64_t total, int w, int nw, int64_t &t0, int64_t &t1) {
    t0 = total * w / nw;
    t1 = total * (w + 1) / nw;
}

// ============================================================ batched matvec
// y_m[r] = W_m[r,:] . x_m. Tasks are (matrix, block of P*R rows); each wave
// takes a contiguous run of tasks and issues all loads of a task before any
// arithmetic.
template <int T, int U, int G, int R>
__global__ __launch_bounds__(256) void k_matvec(MatvecArgs a) {
    constexpr int P = kWave / G, ROWS = P * R;
    const int lane = threadIdx.x & 63, sub = lane / G;
    const int w = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nw = (int)((gridDim.x * blockDim.x) >> 6);
    const int S = a.K / Fmt<T>::SLOT;
    const int64_t tpm = (a.M + ROWS - 1) / ROWS;
    int64_t t0, t1;
    wave_share(tpm * a.n_mats, w, nw, t0, t1);
    Slots<U, G> L;
    L.init(lane, S);
    XRegs<T, U> X;
    int64_t cur = -1;
    // With a shared fp32 x (xf, xf_stride 0) the work-group prepares it in LDS
    // itself (one thread per group, bit-identical to k_xprep); otherwise x
    // comes prepared from global memory.
    extern __shared__ __attribute__((aligned(16))) uint8_t xs_lds[];
    const uint8_t *xq = a.xq;
    if (a.xf) {
        constexpr int GSZ = Fmt<T>::GSZ;
        const int ng = a.K / GSZ;
        for (int g = threadIdx.x; g < ng; g += blockDim.x)
            prep_group<GSZ>(a.xf + g * GSZ, xs_lds + g * (kLimbs * GSZ), xs_lds + xq_limb_bytes(a.K) + g * 8);
        __syncthreads();
        xq = xs_lds;
    }
    // Outputs collect in LDS (a wave's tasks are consecutive rows) and leave
    // as one coalesced store per 64 rows: a 4-byte write per row between the
    // weight reads costs read bandwidth (read/write turnarounds).
    __shared__ float ybuf[4][kWave];
    const int wv = threadIdx.x >> 6;
    int64_t ym = -1;
    int ybase = 0, ycount = 0;
    auto flush = [&]() {
        if (ycount > 0 && lane < ycount) a.y[ym * a.y_stride + ybase + lane] = ybuf[wv][lane];
        ycount = 0;
    };
    for (int64_t t = t0; t < t1; t++) {
        const int64_t m = t / tpm;
        const int rb = (int)(t - m * tpm);
        if (m != cur && (cur < 0 || a.x_stride)) X.load(L, xq + m * a.x_stride, a.K);
        cur = m;
        const uint8_t *W = a.W + m * a.mat_stride;
        RowRaw<T, U> raw[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(rb * ROWS + r * P + sub, a.M - 1);
            load_row(raw[r], W + (uint64_t)row * a.row_bytes, L);
        }
        const int row0 = rb * ROWS;
        if (m != ym || row0 != ybase + ycount || ycount + ROWS > kWave) {
            flush();
            ym = m;
            ybase = row0;
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float v = group_sum<G>(dot_row(raw[r], L, X));
            const int row = row0 + r * P + sub;
            if ((lane % G) == 0 && row < a.M) ybuf[wv][row - ybase] = v;
        }
        ycount += min(ROWS, a.M - row0);
    }
    flush();
}

// Slot geometry of a K-wide row: lanes per row G and slots per lane U.
static bool geometry(int type, int K, int &G, int &U) {
    const int slot = (type == GGML_TYPE_Q8_0 || type == GGML_TYPE_MXFP4) ? 32 : 64;
    if (K <= 0 || K % slot) return false;
    if ((type == GGML_TYPE_Q4_K || type == GGML_TYPE_Q5_K || type == GGML_TYPE_Q6_K) && K % 256)
        return false;
    const int S = K / slot;
    if (S >= 64) { G = 64; U = (S + 63) / 64; return U <= kMaxSlotsPerLane; }
    G = 4;                      // at least 4 lanes per row (extra lanes idle)
    while (G < S) G <<= 1;
    U = 1;
    return true;
}

static int waves_for(int64_t tasks, int n_cu, int per_cu) {
    const int64_t cap = (int64_t)n_cu * per_cu;
    return (int)(tasks < cap ? (tasks > 0 ? tasks : 1) : cap);
}

template <int T, int R>
static hipError_t matvec_t(const MatvecArgs &a, hipStream_t s, int n_cu) {
    int G, U;
    if (!geometry(T, a.K, G, U)) return hipErrorInvalidValue;
    const int P = 64 / G;
    const int64_t tasks = (int64_t)((a.M + P * R - 1) / (P * R)) * a.n_mats;
    const int blocks = (waves_for(tasks, n_cu, 16) + 3) / 4;
    const size_t lds = a.xf ? lds_round(xq_bytes(a.K, Fmt<T>::GSZ)) : 0;
#define FO_MV(GG, UU) \
    if (G == GG && U == UU) { k_matvec<T, UU, GG, R><<<blocks, 256, lds, s>>>(a); return hipGetLastError(); }
    FO_MV(64, 1) FO_MV(64, 2) FO_MV(64, 3) FO_MV(64, 4)
    FO_MV(32, 1) FO_MV(16, 1) FO_MV(8, 1) FO_MV(4, 1)
#undef FO_MV
    return hipErrorInvalidValue;
}


// ============================================================ Q6_K matvec, tile-staged MFMA
// For Q6_K rows of K <= 1024 (the expert down-projection shape). One wave
// per work-group streams a tile of 16 consecutive rows (16 * row_bytes
// contiguous bytes) with 1 KiB coalesced loads, the next tile's loads in
// flight while the current one is computed, writes it to its LDS area and
// reads every lane's pieces back from there. The integer dots run on
// v_mfma_i32_16x16x64_i8: B (weights) = lane (row = lane%16, lane group g)
// with the 64 codes of slot (n = g>>1, j = g&1) for one t; A = the activation
// limbs routed so that D lane (row, g) receives the three limb sums of its own
// 16-value scale group, rows 4g..4g+2 of A being nonzero only over lane group
// g's k-range (other lanes read zeros). D layout: lane holds
// rows 4*(lane/16)+i of column lane%16. Group scales / offsets / sub-block
// scales are then applied per lane as in Fmt<Q6_K>.
constexpr int kT6Rows = 16;                  // 16 rows x 840 B <= 14 KiB per tile
constexpr uint32_t kT6Zero = 304;            // zero A operands: 16 bytes at offsets 0, 96, 192, 288

template <int NSB, int TPW>
__global__ __launch_bounds__(64) void k_matvec_q6k_tile(MatvecArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sx[];
    constexpr int NV = (kT6Rows * NSB * 210 + 1023) / 1024;
    constexpr uint32_t TBYTES = (kT6Rows * NSB * 210 + 15) & ~15u;   // the tile's LDS area
    constexpr int K = NSB * 256;
    const int lane = threadIdx.x;
    const int mat = blockIdx.y;
    constexpr uint32_t limb_bytes = 3u * K, xbytes = limb_bytes + (K / 16) * 8;
    constexpr uint32_t zoff = (xbytes + 15) & ~15u;    // zero A operands for the rows of other groups
    uint8_t *tb = sx + zoff + kT6Zero;
    float *ys = (float *)(tb + TBYTES);                // [TPW * 16] results
    const uint8_t *Wm = a.W + mat * a.mat_stride;
    constexpr uint32_t rb = NSB * 210;                 // launched only for contiguous rows
    constexpr uint32_t full_bytes = kT6Rows * rb;
    const int tile0 = blockIdx.x * TPW;
    const int ntiles = (a.M + kT6Rows - 1) / kT6Rows;
    // A piece that straddles the end of a partial tile (16*rows*rb need not be a
    // multiple of 16) is read from the last 16 valid bytes and written to that
    // same LDS position (overlapping its neighbour with identical bytes). A
    // whole tile is a multiple of 16 bytes: only its last piece is clamped,
    // on the read and on the write (lanes past the end of the tile write the
    // tile's last 16 bytes again, so the LDS area is just the tile's size).
    auto tile_bytes = [&](int tile) { return (uint32_t)min(kT6Rows, a.M - tile * kT6Rows) * rb; };
    auto pos = [&](uint32_t o, uint32_t nb) { return o + 16 <= nb ? o : nb - 16; };
    auto issue = [&](uint4 (&v)[NV], int tile) {
        const uint8_t *tp = Wm + (uint64_t)tile * kT6Rows * rb;
        const uint32_t nb = tile_bytes(tile);
        if (nb == full_bytes) {
#pragma unroll
            for (int i = 0; i < NV; i++) v[i] = ldw16(tp + min(i * 1024u + lane * 16u, full_bytes - 16));
        } else {
#pragma unroll
            for (int i = 0; i < NV; i++) v[i] = ldw16(tp + pos(i * 1024 + lane * 16, nb));
        }
    };
    // one register buffer: tile t+1 is requested right after tile t has been
    // copied to LDS, so its loads overlap tile t's arithmetic (measured faster
    // than two buffers, which need more registers for no more overlap)
    uint4 v[NV];
    if (tile0 < ntiles) issue(v, tile0);
    // the activation is prepared here, one lane per 16-value group (K <= 1024);
    // the group's {scale, -32 * sum} folds the Q6_K code offset into one fma
    if (lane < K / 16) {
        int limb[kLimbs][4];
        float scale, sum;
        prep_group_regs<16>(a.xf + mat * a.xf_stride + lane * 16, limb, scale, sum);
#pragma unroll
        for (int L = 0; L < kLimbs; L++)
            *(uint4 *)(sx + lane * 48 + 16 * L) = make_uint4(limb[L][0], limb[L][1], limb[L][2], limb[L][3]);
        *(float2 *)(sx + limb_bytes + lane * 8) = make_float2(scale, -32.f * sum);
    }
    if (lane < kT6Zero / 16) *(uint4 *)(sx + zoff + 16 * lane) = make_uint4(0, 0, 0, 0);
    __syncthreads();
    const int r = lane & 15, g = lane >> 4, n = g >> 1, j = g & 1, L = r & 3;
    const bool valid = (r >> 2) == g && L < 3;
    const uint8_t *abase = sx + (8 * n + j) * 48 + 16 * L;
    const uint8_t *ssb = sx + limb_bytes + (8 * n + j) * 8;
#pragma unroll
    for (int tt = 0; tt < TPW; tt++) {
        const int tile = tile0 + tt;
        if (tile >= ntiles) break;
        {
            const uint32_t nb = tile_bytes(tile);
            if (nb == full_bytes) {
#pragma unroll
                for (int i = 0; i < NV; i++) *(uint4 *)(tb + min(i * 1024u + lane * 16u, full_bytes - 16)) = v[i];
            } else {
#pragma unroll
                for (int i = 0; i < NV; i++) *(uint4 *)(tb + pos(i * 1024 + lane * 16, nb)) = v[i];
            }
        }
        if (tt + 1 < TPW && tile + 1 < ntiles) issue(v, tile + 1);
        const uint8_t *rp = tb + r * rb;
        float acc = 0.f;
        // every super-block's bytes requested before the first MFMA
        Q6kSlot qs[NSB];
#pragma unroll
        for (int b = 0; b < NSB; b++) q6k_slot_load(qs[b], rp + b * 210, n, j);
#pragma unroll
        for (int b = 0; b < NSB; b++)   // group 16b + 8n + 2t + j: limbs at +768 b, {scale, offset} at +128 b
            acc += q6k_sb_dot_mfma(qs[b], valid ? abase + 768 * b : sx + zoff, ssb + 128 * b, j);
        acc += __shfl_xor(acc, 16);
        acc += __shfl_xor(acc, 32);
        if (g == 0) ys[tt * kT6Rows + r] = acc;
    }
    // the work-group's TPW*16 outputs leave as one contiguous store at the end:
    // a 64-byte write per tile between the weight reads costs ~8 % of the
    // read bandwidth (read/write turnarounds)
    for (int q = lane; q < TPW * kT6Rows; q += 64) {
        const int row = tile0 * kT6Rows + q;
        if (row < a.M) a.y[mat * a.y_stride + row] = ys[q];
    }
}

// TPW = 4 tiles per wave: per-launch p50 0.7-2.2 % below TPW = 8 in same-box
// alternating runs on two boxes (TPW = 2, 3 slower; 6 between)
template <int NSB, int TPW = 4>
static hipError_t matvec_q6k_tile(const MatvecArgs &a, hipStream_t s) {
    constexpr int K = NSB * 256;
    const int ntiles = (a.M + kT6Rows - 1) / kT6Rows;
    const uint32_t lds = ((xq_bytes(K, 16) + 15) & ~15u) + kT6Zero +
                         ((kT6Rows * NSB * 210 + 15) & ~15u) + TPW * kT6Rows * 4;
    k_matvec_q6k_tile<NSB, TPW><<<dim3((ntiles + TPW - 1) / TPW, a.n_mats), 64, lds, s>>>(a);
    return hipGetLastError();
}

// ============================================================ Q8_0 matvec, tile-staged MFMA (K = 1024)
// The Q6_K tile kernel's stream (one wave per work-group, tiles of 16 rows =
// 16 x 1088 contiguous bytes = 17 KiB, 1 KiB non-temporal loads, the next
// tile in flight) with the codes fed to v_mfma_i32_16x16x64_i8 as they are
// (int8): per pair of MFMAs, lane (n = row, g) reads the 16 codes of block
// 4p + (g>>1) (first) and 4p + 2 + (g>>1) (second), half g&1; the A operand
// routes the 32-value groups' limbs so that D lane group g receives the three
// limb sums of block 4p + g of row n, scaled by its d. ~70 VALU instructions
// per tile and lane against ~280 for the slot dots.
constexpr uint32_t kQ8Row = 1088, kQ8X = 3 * 1024 + (1024 / 32) * 8, kQ8Zero = 416;

template <int TPW>
__global__ __launch_bounds__(64) void k_matvec_q80_mfma(MatvecArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sx[];
    constexpr uint32_t TB = 16 * kQ8Row;
    constexpr int NV = TB / 1024;                               // 17 pieces, whole
    const int lane = threadIdx.x, mat = blockIdx.y;
    uint8_t *zero = sx + kQ8X, *tb = zero + kQ8Zero;
    float *ys = (float *)(tb + NV * 1024);                      // [TPW * 16]
    const uint8_t *Wm = a.W + mat * a.mat_stride;
    const int tile0 = blockIdx.x * TPW, ntiles = (a.M + 15) / 16;
    // a partial last tile (M >= 16) is read as rows M-16 .. M-1, its results shifted
    auto first_row = [&](int tile) { return min(tile * 16, a.M - 16); };
    auto issue = [&](uint4 (&v)[NV], int tile) {
        const uint8_t *tp = Wm + (uint64_t)first_row(tile) * kQ8Row;
#pragma unroll
        for (int i = 0; i < NV; i++) v[i] = ldw16(tp + i * 1024 + lane * 16);
    };
    uint4 v[NV];
    if (tile0 < ntiles) issue(v, tile0);
    if (lane < 1024 / 32) {   // the wave's x: one lane per 32-value group
        int limb[kLimbs][8];
        float scale, sum;
        prep_group_regs<32>(a.xf + mat * a.xf_stride + lane * 32, limb, scale, sum);
#pragma unroll
        for (int L = 0; L < kLimbs; L++) {
            *(uint4 *)(sx + lane * 96 + 32 * L) = make_uint4(limb[L][0], limb[L][1], limb[L][2], limb[L][3]);
            *(uint4 *)(sx + lane * 96 + 32 * L + 16) = make_uint4(limb[L][4], limb[L][5], limb[L][6], limb[L][7]);
        }
        *(float2 *)(sx + 3 * 1024 + lane * 8) = make_float2(scale, sum);
    } else if (lane < 32 + kQ8Zero / 16) {
        *(uint4 *)(zero + 16 * (lane - 32)) = make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
    const int n = lane & 15, g = lane >> 4, mb = n >> 2, L = n & 3;
    const bool valid1 = mb == (g >> 1) && L < 3, valid2 = mb == 2 + (g >> 1) && L < 3;
    const uint8_t *xa = sx + mb * 96 + 32 * L + 16 * (g & 1);   // + 384 p: group 4p + mb
    const uint8_t *a1 = valid1 ? xa : zero, *a2 = valid2 ? xa : zero;
    const int s1 = valid1 ? 384 : 0, s2 = valid2 ? 384 : 0;   // zero lanes stay on the zero area
    const float2 *ssl = (const float2 *)(sx + 3 * 1024) + g;  // group 4p + g
#pragma unroll
    for (int tt = 0; tt < TPW; tt++) {
        const int tile = tile0 + tt;
        if (tile >= ntiles) break;
#pragma unroll
        for (int i = 0; i < NV; i++) *(uint4 *)(tb + i * 1024 + lane * 16) = v[i];
        if (tt + 1 < TPW && tile + 1 < ntiles) issue(v, tile + 1);
        const uint8_t *rp = tb + n * kQ8Row;
        float y = 0.f;
#pragma unroll
        for (int p = 0; p < 8; p++) {
            v4i B1, B2;
            __builtin_memcpy(&B1, rp + 34 * (4 * p + (g >> 1)) + 2 + 16 * (g & 1), 16);
            __builtin_memcpy(&B2, rp + 34 * (4 * p + 2 + (g >> 1)) + 2 + 16 * (g & 1), 16);
            uint16_t d16;
            __builtin_memcpy(&d16, rp + 34 * (4 * p + g), 2);
            const v4i A1 = *(const v4i *)(a1 + s1 * p), A2 = *(const v4i *)(a2 + s2 * p);
            v4i D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1, (v4i){0, 0, 0, 0}, 0, 0, 0);
            D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A2, B2, D, 0, 0, 0);
            const float f = fmaf((float)((D[2] << 8) + D[1]), 256.f, (float)D[0]);
            y = fmaf(h2f(d16), f * ssl[4 * p].x, y);
        }
        y += __shfl_xor(y, 16);
        y += __shfl_xor(y, 32);
        const int shift = tile * 16 - first_row(tile);
        if (g == 0 && n >= shift) ys[tt * 16 + n - shift] = y;
    }
    for (int q = lane; q < TPW * 16; q += 64) {
        const int row = tile0 * 16 + q;
        if (row < a.M) a.y[mat * a.y_stride + row] = ys[q];
    }
}

// 4 tiles per wave (as the Q6_K tile kernel): per-launch p50 3 % (Q8_0) and 4 %
// (Q5_K) below 8 tiles per wave in alternating same-box runs
template <int TPW>
static hipError_t matvec_q80_mfma_t(const MatvecArgs &a, hipStream_t s) {
    const int ntiles = (a.M + 15) / 16;
    const uint32_t lds = kQ8X + kQ8Zero + 16 * kQ8Row + TPW * 16 * 4;
    k_matvec_q80_mfma<TPW><<<dim3((ntiles + TPW - 1) / TPW, a.n_mats), 64, lds, s>>>(a);
    return hipGetLastError();
}

static hipError_t matvec_q80_mfma(const MatvecArgs &a, hipStream_t s) { return matvec_q80_mfma_t<4>(a, s); }

// ============================================================ Q5_K matvec, tile-staged MFMA (K = 1024)
// The Q8_0 MFMA kernel's stream (one wave per work-group, 16-row tiles =
// 16 x 704 contiguous bytes = 11 KiB, the next tile in flight) with the Q5_K
// super-block dot of q4k_mfma.h (Q4_K's code routing plus the fifth bit).
constexpr uint32_t kQ5Row = 704, kQ5X = 3 * 1024 + (1024 / 32) * 8, kQ5Zero = 416;

template <int TPW>
__global__ __launch_bounds__(64) void k_matvec_q5k_mfma(MatvecArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t sx[];
    constexpr uint32_t TB = 16 * kQ5Row;
    constexpr int NV = TB / 1024;                               // 11 pieces, whole
    const int lane = threadIdx.x, mat = blockIdx.y;
    uint8_t *zero = sx + kQ5X, *tb = zero + kQ5Zero;
    float *ys = (float *)(tb + NV * 1024);                      // [TPW * 16]
    const uint8_t *Wm = a.W + mat * a.mat_stride;
    const int tile0 = blockIdx.x * TPW, ntiles = (a.M + 15) / 16;
    auto first_row = [&](int tile) { return min(tile * 16, a.M - 16); };
    auto issue = [&](uint4 (&v)[NV], int tile) {
        const uint8_t *tp = Wm + (uint64_t)first_row(tile) * kQ5Row;
#pragma unroll
        for (int i = 0; i < NV; i++) v[i] = ldw16(tp + i * 1024 + lane * 16);
    };
    uint4 v[NV];
    if (tile0 < ntiles) issue(v, tile0);
    if (lane < 1024 / 32) {   // the wave's x: one lane per 32-value group
        int limb[kLimbs][8];
        float scale, sum;
        prep_group_regs<32>(a.xf + mat * a.xf_stride + lane * 32, limb, scale, sum);
#pragma unroll
        for (int L = 0; L < kLimbs; L++) {
            *(uint4 *)(sx + lane * 96 + 32 * L) = make_uint4(limb[L][0], limb[L][1], limb[L][2], limb[L][3]);
            *(uint4 *)(sx + lane * 96 + 32 * L + 16) = make_uint4(limb[L][4], limb[L][5], limb[L][6], limb[L][7]);
        }
        *(float2 *)(sx + 3 * 1024 + lane * 8) = make_float2(scale, sum);
    } else if (lane < 32 + kQ5Zero / 16) {
        *(uint4 *)(zero + 16 * (lane - 32)) = make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
    const Q4kLane q = q4k_lane(lane);
    const int n = lane & 15, g = lane >> 4;
    const uint8_t *ssl = sx + 3 * 1024 + q.jg * 8;
#pragma unroll
    for (int tt = 0; tt < TPW; tt++) {
        const int tile = tile0 + tt;
        if (tile >= ntiles) break;
#pragma unroll
        for (int i = 0; i < NV; i++) *(uint4 *)(tb + i * 1024 + lane * 16) = v[i];
        if (tt + 1 < TPW && tile + 1 < ntiles) issue(v, tile + 1);
        const uint8_t *rp = tb + n * kQ5Row;
        float y = 0.f;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const uint8_t *xa = sx + b * 768 + q.aoff;
            y = q5k_sb_dot_mfma(rp + b * 176, q.valid1 ? xa : zero, q.valid2 ? xa : zero, ssl + b * 64, q, g, y);
        }
        y += __shfl_xor(y, 16);
        y += __shfl_xor(y, 32);
        const int shift = tile * 16 - first_row(tile);
        if (g == 0 && n >= shift) ys[tt * 16 + n - shift] = y;
    }
    for (int r = lane; r < TPW * 16; r += 64) {
        const int row = tile0 * 16 + r;
        if (row < a.M) a.y[mat * a.y_stride + row] = ys[r];
    }
}

// 4 tiles per wave: see matvec_q80_mfma_t
template <int TPW>
static hipError_t matvec_q5k_mfma_t(const MatvecArgs &a, hipStream_t s) {
    const int ntiles = (a.M + 15) / 16;
    const uint32_t lds = kQ5X + kQ5Zero + 16 * kQ5Row + TPW * 16 * 4;
    k_matvec_q5k_mfma<TPW><<<dim3((ntiles + TPW - 1) / TPW, a.n_mats), 64, lds, s>>>(a);
    return hipGetLastError();
}

static hipError_t matvec_q5k_mfma(const MatvecArgs &a, hipStream_t s) { return matvec_q5k_mfma_t<4>(a, s); }

// ============================================================ Q4_K matvec, tile-staged MFMA
// For Q4_K rows of K = 4096 (the expert gate/up shape). Four-wave work-groups
// share one prepared x (13 KiB of LDS); each wave streams its own blocks of
// 16 rows in chunks of 4 super-blocks (16 x 576 bytes = 9 KiB loaded as nine
// 1 KiB wave pieces; each lane's 16 bytes lie within one row's 576-byte
// segment, row segments 2304 bytes apart), the next chunk's loads in flight
// while the current one is multiplied, writes each chunk to its LDS area and
// runs the integer dots of all 16 rows on v_mfma_i32_16x16x64_i8 (q4k_mfma.h):
// 16 MFMAs and ~300 VALU instructions per chunk against ~370 VALU for the same
// bytes as per-lane slot dots. 51 KiB of LDS per work-group: 12 waves per CU. One block per
// wave (the work-group's four blocks = 64 consecutive rows) measured fastest:
// 6.50 TB/s against 6.34 / 6.27 / 6.24 with 2 / 4 / 8 blocks per wave. Chunks
// 0 and 2 of a row end in the middle of a 128-byte line that chunks 1 and 3
// begin with: those chunks load without the non-temporal hint, so the line
// stays in L2 for the next chunk (HBM fetch 1.084 -> 1.000 x the algorithmic
// bytes, 6.50 -> 6.85 TB/s).
constexpr int kQ4Waves = 4, kQ4Tpw = 1;             // blocks of 16 rows per wave (2, 4, 8: slower)
constexpr uint32_t kQ4K = 4096, kQ4Row = 2304, kQ4Chunk = 576, kQ4ChunkBytes = 16 * kQ4Chunk;
constexpr uint32_t kQ4X = 3 * kQ4K + (kQ4K / 32) * 8;   // prepared x: limbs, then {scale, sum}
constexpr uint32_t kQ4Zero = 416;                       // zero A operands (>= 384 + 16)
constexpr uint32_t kQ4Lds = kQ4X + kQ4Zero + kQ4Waves * kQ4ChunkBytes + kQ4Waves * kQ4Tpw * 16 * 4;

__global__ __launch_bounds__(64 * kQ4Waves, 3) void k_matvec_q4k_mfma(MatvecArgs a) {   // 3 WGs per CU
    extern __shared__ __attribute__((aligned(16))) uint8_t sx[];
    constexpr int NP = kQ4ChunkBytes / 1024;             // 9 pieces per chunk
    constexpr int NC = kQ4K / 1024;                      // 4 chunks per block (4 super-blocks each)
    // wv through readfirstlane: the compiler then treats the wave's block
    // addresses as uniform (SGPR base + per-lane 32-bit offset)
    const int lane = threadIdx.x & 63, wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), mat = blockIdx.y;
    uint8_t *zero = sx + kQ4X;
    uint8_t *tb = zero + kQ4Zero + wv * kQ4ChunkBytes;
    float *ys = (float *)(sx + kQ4X + kQ4Zero + kQ4Waves * kQ4ChunkBytes);   // [waves][kQ4Tpw * 16]
    const uint8_t *Wm = a.W + mat * a.mat_stride;
    const int nblk = (a.M + 15) / 16;
    const int blk0 = (blockIdx.x * kQ4Waves + wv) * kQ4Tpw;
    // piece i of a chunk, lane l: chunk byte o = 1024 i + 16 l of row o / 576
    uint32_t goff[NP];
#pragma unroll
    for (int i = 0; i < NP; i++) {
        const uint32_t o = i * 1024 + lane * 16;
        goff[i] = (o / kQ4Chunk) * kQ4Row + o % kQ4Chunk;
    }
    // unit u = (block t = u / NC, chunk c = u % NC) of this wave; a partial
    // last block (M >= 16) is read as rows M-16 .. M-1, its results shifted
    auto first_row = [&](int blk) { return min(blk * 16, a.M - 16); };
    auto issue = [&](uint4 (&v)[NP], int u) {
        const int blk = blk0 + u / NC, c = u % NC;
        const uint8_t *base = Wm + (uint64_t)first_row(blk) * kQ4Row + c * kQ4Chunk;
        if (c & 1) {
#pragma unroll
            for (int i = 0; i < NP; i++) v[i] = ldw16(base + goff[i]);
        } else {   // chunks 0, 2 end mid-line: plain loads keep that line in L2 for chunks 1, 3
#pragma unroll
            for (int i = 0; i < NP; i++) v[i] = ld16(base + goff[i]);
        }
    };
    const int nunits = min(kQ4Tpw, nblk - blk0) * NC;
    uint4 v[NP];
    if (nunits > 0) issue(v, 0);
    // the work-group's x, prepared by threads 0..127 (one 32-value group each)
    if (threadIdx.x < kQ4K / 32) {
        const int gi = threadIdx.x;
        int limb[kLimbs][8];
        float scale, sum;
        prep_group_regs<32>(a.xf + mat * a.xf_stride + gi * 32, limb, scale, sum);
#pragma unroll
        for (int L = 0; L < kLimbs; L++) {
            *(uint4 *)(sx + gi * 96 + 32 * L) = make_uint4(limb[L][0], limb[L][1], limb[L][2], limb[L][3]);
            *(uint4 *)(sx + gi * 96 + 32 * L + 16) = make_uint4(limb[L][4], limb[L][5], limb[L][6], limb[L][7]);
        }
        *(float2 *)(sx + 3 * kQ4K + gi * 8) = make_float2(scale, sum);
    } else if (threadIdx.x < kQ4K / 32 + kQ4Zero / 16) {
        *(uint4 *)(zero + 16 * (threadIdx.x - kQ4K / 32)) = make_uint4(0, 0, 0, 0);
    }
    __syncthreads();
    const Q4kLane q = q4k_lane(lane);
    const int n = lane & 15, g = lane >> 4;
    const uint8_t *ssl = sx + 3 * kQ4K + q.jg * 8;
#pragma unroll 1
    for (int t = 0; t < kQ4Tpw; t++) {
        if (t * NC >= nunits) break;
        float y = 0.f;
#pragma unroll 1
        for (int c = 0; c < NC; c++) {
            const int u = t * NC + c;
#pragma unroll
            for (int i = 0; i < NP; i++) *(uint4 *)(tb + i * 1024 + lane * 16) = v[i];
            if (u + 1 < nunits) issue(v, u + 1);
            const uint8_t *rp = tb + n * kQ4Chunk;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int sb = 4 * c + b;                    // super-block of the row: groups 8 sb ..
                const uint8_t *xa = sx + sb * 768 + q.aoff;
                y = q4k_sb_dot_mfma(rp + b * 144, q.valid1 ? xa : zero, q.valid2 ? xa : zero, ssl + sb * 64, q, y);
            }
        }
        y += __shfl_xor(y, 16);
        y += __shfl_xor(y, 32);
        const int shift = (blk0 + t) * 16 - first_row(blk0 + t);
        if (g == 0 && n >= shift) ys[(wv * kQ4Tpw + t) * 16 + n - shift] = y;
    }
    __syncthreads();
    // the work-group's rows [16 * blk0(wave 0), + 16 * kQ4Waves * kQ4Tpw) leave as one store
    const int row0 = blockIdx.x * kQ4Waves * kQ4Tpw * 16;
    for (int r = threadIdx.x; r < kQ4Waves * kQ4Tpw * 16; r += 64 * kQ4Waves)
        if (row0 + r < a.M) a.y[mat * a.y_stride + row0 + r] = ys[r];
}

static hipError_t matvec_q4k_mfma(const MatvecArgs &a, hipStream_t s) {
    static bool attr = false;   // more than the 64 KiB default of dynamic LDS
    if (!attr) {
        const hipError_t e = hipFuncSetAttribute((const void *)k_matvec_q4k_mfma,
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)kQ4Lds);
        if (e != hipSuccess) return e;
        attr = true;
    }
    const int nblk = (a.M + 15) / 16, per_wg = kQ4Waves * kQ4Tpw;
    k_matvec_q4k_mfma<<<dim3((nblk + per_wg - 1) / per_wg, a.n_mats), 64 * kQ4Waves, kQ4Lds, s>>>(a);
    return hipGetLastError();
}

// ============================================================ tile-staged slot matvec
// k_matvec_tile<T, K, RT>: rows of K values, RT consecutive rows per
// tile (RT * row_bytes contiguous bytes). One wave per work-group streams its
// tiles with non-temporal 1 KiB loads (the next tile in flight while the
// current one is computed), writes each to its LDS area and reads every lane's
// slots back from there; lane l owns slots l%G + G*u of P = 64/G rows per pass
// (Fmt<T> slot dots on the exact int8 limbs) and prepares its own activation
// groups from fp32 x (prep_group_regs, bit-identical to k_xprep). Used for
// Q4_K at K = 8192 (and K = 4096 with fewer than 16 rows; RT * row_bytes =
// 18 KiB), Q8_0 at K = 4096 (17 KiB tiles), Q5_K at K = 4096 (11 KiB), MXFP4
// at K = 4096 (17 KiB), and the K = 1024 Q8_0 / Q5_K shapes with fewer than 16
// rows; the MFMA kernels above serve the rest. Over the per-lane-load
// k_matvec this scheme took Q4_K at K = 4096 from 5.5 to 5.8-6.0 TB/s; for
// Q6_K at K = 1024 it measured 5.0 TB/s against 5.6 for the MFMA tile kernel.
// With G = 64 the RT row partials of a lane are reduced across the wave
// together, halving the live values at each xor step.
template <int N>
FO_DEV float rows_sum(float (&v)[N], int lane) {   // lane ends with row (lane >> (6 - log2 N)) & (N-1)
    int m = 32;
#pragma unroll
    for (int w = N; w > 1; w >>= 1, m >>= 1) {
        const bool up = lane & m;
#pragma unroll
        for (int i = 0; i < w / 2; i++) {
            const float keep = up ? v[i + w / 2] : v[i], send = up ? v[i] : v[i + w / 2];
            v[i] = keep + __shfl_xor(send, m, kWave);
        }
    }
#pragma unroll
    for (; m >= 1; m >>= 1) v[0] += __shfl_xor(v[0], m, kWave);
    return v[0];
}

template <int T, int K, int RT, int TPW>
__global__ __launch_bounds__(64) void k_matvec_tile(MatvecArgs a) {
    using F = Fmt<T>;
    constexpr int S = K / F::SLOT;                    // slots per row
    constexpr int G = S >= 64 ? 64 : S, P = 64 / G, U = S / G;
    constexpr int BV = F::SLOT == 64 ? 256 : 32;      // values per format block
    constexpr int RB = K / BV * F::BLOCK, TB = RT * RB, NV = (TB + 1023) / 1024;
    static_assert(S % G == 0 && RT % P == 0, "tile geometry");
    extern __shared__ __attribute__((aligned(16))) uint8_t tb[];   // [NV KiB] tile + [TPW*RT] results
    float *ys = (float *)(tb + NV * 1024);
    const int lane = threadIdx.x, mat = blockIdx.y, sub = lane / G;
    const uint8_t *Wm = a.W + mat * a.mat_stride;
    const int tile0 = blockIdx.x * TPW;
    const int ntiles = (a.M + RT - 1) / RT;
    // a piece that straddles the end of a tile is read from the last 16 valid
    // bytes and written to that same LDS position (identical bytes overlap)
    auto tile_bytes = [&](int tile) { return (uint32_t)min(RT, a.M - tile * RT) * RB; };
    auto pos = [&](uint32_t o, uint32_t nb) { return o + 16 <= nb ? o : nb - 16; };
    auto issue = [&](uint4 (&v)[NV], int tile) {
        const uint32_t nb = tile_bytes(tile);
        const uint8_t *tp = Wm + (uint64_t)tile * TB;
#pragma unroll
        for (int i = 0; i < NV; i++) v[i] = ldw16(tp + pos(i * 1024 + lane * 16, nb));
    };
    uint4 v[NV];
    if (tile0 < ntiles) issue(v, tile0);
    // the lane's activation slots, prepared from fp32 x while the tile loads
    typename F::X X[U];
    const float *xm = a.xf + mat * a.xf_stride;
#pragma unroll
    for (int u = 0; u < U; u++) {
        int gi[F::NG];
        F::groups(lane % G + G * u, gi);
#pragma unroll
        for (int g = 0; g < F::NG; g++)
            prep_group_regs<F::GSZ>(xm + gi[g] * F::GSZ, X[u].l[g], X[u].sc[g], X[u].sum[g]);
    }
#pragma unroll
    for (int tt = 0; tt < TPW; tt++) {
        const int tile = tile0 + tt;
        if (tile >= ntiles) break;
        const uint32_t nb = tile_bytes(tile);
#pragma unroll
        for (int i = 0; i < NV; i++) {
            const uint32_t o = i * 1024 + lane * 16;
            *(uint4 *)(tb + (o < nb ? pos(o, nb) : o)) = v[i];
        }
        if (tt + 1 < TPW && tile + 1 < ntiles) issue(v, tile + 1);
        constexpr int PASS = RT / P;
        float part[PASS];
#pragma unroll
        for (int p = 0; p < PASS; p++) {
            const uint8_t *row = tb + (p * P + sub) * RB;
            part[p] = 0.f;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int s = lane % G + G * u;
                part[p] += F::dot(F::load(row, s), s, X[u]);
            }
        }
        if (G == 64) {
            const float y = rows_sum<PASS>(part, lane);
            constexpr int SH = PASS == 8 ? 3 : PASS == 4 ? 2 : PASS == 2 ? 1 : 0;
            if ((lane & ((64 >> SH) - 1)) == 0) ys[tt * RT + (lane >> (6 - SH))] = y;
        } else {
#pragma unroll
            for (int p = 0; p < PASS; p++) {
                const float y = group_sum<G>(part[p]);
                if (lane % G == 0) ys[tt * RT + p * P + sub] = y;
            }
        }
    }
    // outputs leave as one contiguous store per work-group
    for (int q = lane; q < TPW * RT; q += 64) {
        const int row = tile0 * RT + q;
        if (row < a.M) a.y[mat * a.y_stride + row] = ys[q];
    }
}

template <int T, int K, int RT>
static hipError_t matvec_tile(const MatvecArgs &a, hipStream_t s) {
    constexpr int TPW = 8, BV = Fmt<T>::SLOT == 64 ? 256 : 32;
    const int ntiles = (a.M + RT - 1) / RT;
    const uint32_t lds = (RT * (K / BV) * Fmt<T>::BLOCK + 1023) / 1024 * 1024 + TPW * RT * 4;
    k_matvec_tile<T, K, RT, TPW><<<dim3((ntiles + TPW - 1) / TPW, a.n_mats), 64, lds, s>>>(a);
    return hipGetLastError();
}

// shapes served by k_matvec_tile (contiguous rows)
static bool tile_shape(int type, uint64_t row_bytes, int K) {
    if (type == GGML_TYPE_Q4_K) return (K == 4096 || K == 8192) && row_bytes == (uint64_t)K / 256 * 144;
    if (type == GGML_TYPE_Q8_0) return (K == 1024 || K == 4096) && row_bytes == (uint64_t)K / 32 * 34;
    if (type == GGML_TYPE_Q5_K) return (K == 1024 || K == 4096) && row_bytes == (uint64_t)K / 256 * 176;
    if (type == GGML_TYPE_MXFP4) return K == 4096 && row_bytes == (uint64_t)K / 32 * 17;
    return false;
}

bool matvec_self_prep(int type, uint64_t row_bytes, int K, uint64_t x_stride) {
    if (type == GGML_TYPE_Q6_K && row_bytes == (uint64_t)K / 256 * 210 && K % 256 == 0 && K <= 1024)
        return true;   // tile-staged kernel: one matrix per work-group, any x_stride
    if (tile_shape(type, row_bytes, K)) return true;
    return x_stride == 0 && (type == GGML_TYPE_Q4_K || type == GGML_TYPE_Q5_K || type == GGML_TYPE_Q6_K ||
                             type == GGML_TYPE_Q8_0 || type == GGML_TYPE_MXFP4);
}

hipError_t launch_matvec(int type, const MatvecArgs &a, hipStream_t s, int n_cu) {
    if (a.M <= 0 || a.n_mats <= 0) return hipErrorInvalidValue;
    switch (type) {
        case GGML_TYPE_Q4_K:
            if (a.xf && tile_shape(type, a.row_bytes, a.K)) {   // tile-staged path
                if (a.K == 4096 && a.M >= 16) return matvec_q4k_mfma(a, s);
                if (a.K == 4096) return matvec_tile<GGML_TYPE_Q4_K, 4096, 8>(a, s);
                return matvec_tile<GGML_TYPE_Q4_K, 8192, 4>(a, s);
            }
            return matvec_t<GGML_TYPE_Q4_K, 2>(a, s, n_cu);
        case GGML_TYPE_Q5_K:
            if (a.xf && tile_shape(type, a.row_bytes, a.K)) {   // tile-staged path
                if (a.K == 1024 && a.M >= 16) return matvec_q5k_mfma(a, s);
                if (a.K == 1024) return matvec_tile<GGML_TYPE_Q5_K, 1024, 16>(a, s);
                return matvec_tile<GGML_TYPE_Q5_K, 4096, 4>(a, s);
            }
            return matvec_t<GGML_TYPE_Q5_K, 2>(a, s, n_cu);
        case GGML_TYPE_Q6_K:
            if (a.xf && a.row_bytes == (uint64_t)a.K / 256 * 210 && a.K % 256 == 0 && a.K <= 1024) {   // tile-staged path
                if (a.K == 1024) return matvec_q6k_tile<4>(a, s);
                if (a.K == 768) return matvec_q6k_tile<3>(a, s);
                if (a.K == 512) return matvec_q6k_tile<2>(a, s);
                if (a.K == 256) return matvec_q6k_tile<1>(a, s);
            }
            return matvec_t<GGML_TYPE_Q6_K, 2>(a, s, n_cu);
        case GGML_TYPE_Q8_0:
            if (a.xf && tile_shape(type, a.row_bytes, a.K)) {   // tile-staged path
                if (a.K == 1024 && a.M >= 16) return matvec_q80_mfma(a, s);
                if (a.K == 1024) return matvec_tile<GGML_TYPE_Q8_0, 1024, 16>(a, s);
                return matvec_tile<GGML_TYPE_Q8_0, 4096, 4>(a, s);
            }
            return matvec_t<GGML_TYPE_Q8_0, 2>(a, s, n_cu);
        case GGML_TYPE_MXFP4:
            if (a.xf && tile_shape(type, a.row_bytes, a.K)) return matvec_tile<GGML_TYPE_MXFP4, 4096, 8>(a, s);
            return matvec_t<GGML_TYPE_MXFP4, 2>(a, s, n_cu);
        default: return hipErrorInvalidValue;
    }
}

// ============================================================ router
// Work-group of 4 waves, one router row per wave. The input is staged in LDS
// (RMS-normalised when norm_w is set: h = x * (1/sqrt(mean(x^2)+eps)) * w, in
// the operation order of reference src/tensor.c:175-184), each work-group
// also writes its share of the prepared activation of h for the expert
// kernels, and the last work-group to finish runs softmax, top-k and
// renormalisation (reference src/inference.c:486-502, src/tensor.c:186-252).
constexpr int kRouterMaxE = 1024;

template <int UH>  // H = 256*UH; a lane holds 4*UH values of h (UH = 0: any H, a multiple of 256)
__global__ __launch_bounds__(256) void k_router(RouterArgs a, uint8_t *__restrict__ xq_h, int gsz) {
    extern __shared__ float sh[];  // H floats
    __shared__ float red[4];
    __shared__ int last;
    const int H = a.H, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    for (int i = tid * 4; i < H; i += 1024) *(float4 *)(sh + i) = *(const float4 *)(a.x + i);
    __syncthreads();
    if (a.norm_w) {
        float ss = 0.f;
        for (int i = tid; i < H; i += 256) ss += sh[i] * sh[i];
        ss = wave_sum(ss);
        if (lane == 0) red[wv] = ss;
        __syncthreads();
        const float tot = (red[0] + red[1]) + (red[2] + red[3]);
        const float scale = 1.0f / sqrtf(tot / (float)H + a.eps);
        __syncthreads();
        for (int i = tid; i < H; i += 256) sh[i] = sh[i] * scale * a.norm_w[i];
        __syncthreads();
    }
    // this work-group's share of the prepared activation of h
    if (xq_h) {
        const int ng = H / gsz, per = (ng + gridDim.x - 1) / gridDim.x;
        for (int j = tid; j < per; j += 256) {
            const int g = blockIdx.x * per + j;
            if (g >= ng) break;
            const float *xp = sh + g * gsz;
            float M = 0.f, chk = 0.f;
            for (int i = 0; i < gsz; i++) { M = fmaxf(M, fabsf(xp[i])); chk += xp[i] * 0.f; }
            int E = 0;
            frexpf(M, &E);
            int e = kFixBits - E;
            if (e > 149) e = 149;
            uint32_t *lp = (uint32_t *)(xq_h + (uint64_t)g * (kLimbs * gsz));
            int isum = 0;
            for (int k = 0; k < gsz / 4; k++) {
                uint32_t lb[kLimbs] = {};
                for (int b = 0; b < 4; b++) {
                    int X = (M > 0.f && chk == 0.f) ? __float2int_rn(ldexpf(xp[4 * k + b], e)) : 0;
                    isum += X;
                    for (int L = 0; L < kLimbs - 1; L++) {
                        const int v = (int)(int8_t)(X & 0xFF);
                        X = (X - v) >> 8;
                        lb[L] |= (uint32_t)(v & 0xFF) << (8 * b);
                    }
                    lb[kLimbs - 1] |= (uint32_t)(X & 0xFF) << (8 * b);
                }
                for (int L = 0; L < kLimbs; L++) lp[L * (gsz / 4) + k] = lb[L];
            }
            float scale, sum;
            group_scale_sum(M, chk, e, isum, scale, sum);
            *(float2 *)(xq_h + xq_limb_bytes(H) + (uint64_t)g * 8) = make_float2(scale, sum);
        }
    }
    // one row per wave
    const int e = blockIdx.x * 4 + wv;
    if (e < a.E) {
        const float *row = a.W + (uint64_t)e * H;
        float acc = 0.f;
        if constexpr (UH > 0) {   // all of the row's loads in flight at once
            float4 wv4[UH];
#pragma unroll
            for (int u = 0; u < UH; u++) wv4[u] = *((const float4 *)row + lane + 64 * u);
#pragma unroll
            for (int u = 0; u < UH; u++) {
                const float4 hv = *(const float4 *)(sh + 4 * (lane + 64 * u));
                acc = fmaf(wv4[u].x, hv.x, acc);
                acc = fmaf(wv4[u].y, hv.y, acc);
                acc = fmaf(wv4[u].z, hv.z, acc);
                acc = fmaf(wv4[u].w, hv.w, acc);
            }
        } else {                  // any H = 256 * n: the same sums, one float4 at a time
            for (int u = 0; u < H / 256; u++) {
                const float4 w4 = *((const float4 *)row + lane + 64 * u);
                const float4 hv = *(const float4 *)(sh + 4 * (lane + 64 * u));
                acc = fmaf(w4.x, hv.x, acc);
                acc = fmaf(w4.y, hv.y, acc);
                acc = fmaf(w4.z, hv.z, acc);
                acc = fmaf(w4.w, hv.w, acc);
            }
        }
        acc = wave_sum(acc);
        if (lane == 0) a.logits[e] = acc + (a.bias ? a.bias[e] : 0.f);
    }
    // last work-group: softmax, top-k, renormalise
    __syncthreads();
    if (tid == 0) {
        __threadfence();
        const unsigned prev = atomicAdd(a.counter, 1u);
        last = (prev == gridDim.x - 1);
    }
    __syncthreads();
    if (!last || wv != 0) return;
    __threadfence();
    constexpr int NV = kRouterMaxE / 64;
    float v[NV];
    float mx = -FLT_MAX;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = lane + 64 * j;
        v[j] = (i < a.E) ? __hip_atomic_load(a.logits + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                         : -FLT_MAX;
        mx = fmaxf(mx, v[j]);
    }
    mx = wave_max(mx);
    float ls = 0.f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = lane + 64 * j;
        v[j] = (i < a.E) ? expf(v[j] - mx) : 0.f;
        ls += v[j];
    }
    const float inv = 1.0f / wave_sum(ls);
#pragma unroll
    for (int j = 0; j < NV; j++) v[j] = (lane + 64 * j < a.E) ? v[j] * inv : -FLT_MAX;
    // top-k: k rounds of wave argmax, ties to the lowest index
    float selv[16];
    int seli[16];
    for (int kk = 0; kk < a.k; kk++) {
        float best = -FLT_MAX;
        int bi = 0x7FFFFFFF;
#pragma unroll
        for (int j = 0; j < NV; j++)
            if (v[j] > best) { best = v[j]; bi = lane + 64 * j; }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(best, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (ov > best || (ov == best && oi < bi)) { best = ov; bi = oi; }
        }
        if (bi < 0 || bi >= a.E) { bi = 0; best = 0.f; }  // non-finite logits: never index out of range
        selv[kk] = best;
        seli[kk] = bi;
        if (lane == (bi & 63)) {
#pragma unroll
            for (int j = 0; j < NV; j++)
                if (j == (bi >> 6)) v[j] = -FLT_MAX;
        }
    }
    // shared-expert gate sigmoid(h . g)
    float gate = 1.0f;
    if (a.shared_gate_vec) {
        float d = 0.f;
        for (int i = lane; i < H; i += 64) d += sh[i] * a.shared_gate_vec[i];
        d = wave_sum(d);
        gate = 1.0f / (1.0f + expf(-d));
    }
    if (lane == 0) {
        float ssum = 0.f;
        for (int kk = 0; kk < a.k; kk++) ssum += selv[kk];
        const float rinv = ssum > 0.f ? 1.0f / ssum : 1.0f;
        for (int kk = 0; kk < a.k; kk++) {
            a.ids[kk] = seli[kk];
            a.weights[kk] = ssum > 0.f ? selv[kk] * rinv : selv[kk];
        }
        a.weights[a.k] = gate;
        __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

hipError_t launch_router(const RouterArgs &a, uint8_t *xq_h, int gsz, hipStream_t s) {
    if (a.E <= 0 || a.E > kRouterMaxE || a.k <= 0 || a.k > 16 || a.k > a.E || a.H % 256)
        return hipErrorInvalidValue;
    const int blocks = (a.E + 3) / 4;
    const size_t lds = (size_t)a.H * 4;
#define FO_RT(UU) \
    if (a.H == 256 * UU) { k_router<UU><<<blocks, 256, lds, s>>>(a, xq_h, gsz); return hipGetLastError(); }
    FO_RT(1) FO_RT(2) FO_RT(4) FO_RT(8) FO_RT(12) FO_RT(16) FO_RT(24) FO_RT(32)
#undef FO_RT
    if (a.H <= 8192) {
        k_router<0><<<blocks, 256, lds, s>>>(a, xq_h, gsz);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

// ============================================================ gate/up/SiLU
// Tasks are (expert slot, block of P*R rows); gate and up rows of a task are
// loaded together and act = silu(gate.h) * (up.h) (reference
// src/inference.c:555-566 order: silu of gate, then multiply by up).
template <int T, int U, int G, int R>
__global__ __launch_bounds__(256) void k_gateup(GateUpArgs a, const uint8_t *__restrict__ xq_h) {
    constexpr int P = kWave / G, ROWS = P * R;
    const int lane = threadIdx.x & 63, sub = lane / G;
    const int w = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nw = (int)((gridDim.x * blockDim.x) >> 6);
    const int S = a.H / Fmt<T>::SLOT;
    const int n_tot = a.n_sel;
    const int tpe = (a.F + ROWS - 1) / ROWS;
    int64_t t0, t1;
    wave_share((int64_t)tpe * n_tot, w, nw, t0, t1);
    if (t0 >= t1) return;
    Slots<U, G> L;
    L.init(lane, S);
    XRegs<T, U> X;
    X.load(L, xq_h, a.H);
    for (int64_t t = t0; t < t1; t++) {
        const int e = (int)(t / tpe), rb = (int)(t - (int64_t)e * tpe);
        const uint8_t *blob = a.base + (uint64_t)(a.ids ? a.ids[e] : e) * a.stride;
        const uint64_t go = a.gate_off, uo = a.up_off;
        RowRaw<T, U> rg[R], ru[R];
#pragma unroll
        for (int r = 0; r < R; r++) {
            const int row = min(rb * ROWS + r * P + sub, a.F - 1);
            load_row(rg[r], blob + go + (uint64_t)row * a.row_bytes, L);
            load_row(ru[r], blob + uo + (uint64_t)row * a.row_bytes, L);
        }
#pragma unroll
        for (int r = 0; r < R; r++) {
            const float g = group_sum<G>(dot_row(rg[r], L, X));
            const float u = group_sum<G>(dot_row(ru[r], L, X));
            const int row = rb * ROWS + r * P + sub;
            if ((lane % G) == 0 && row < a.F) a.act[(uint64_t)e * a.F + row] = (g / (1.0f + expf(-g))) * u;
        }
    }
}

template <int T, int R>
static hipError_t gateup_t(const GateUpArgs &a, const uint8_t *xq_h, hipStream_t s, int n_cu) {
    int G, U;
    if (!geometry(T, a.H, G, U)) return hipErrorInvalidValue;
    const int P = 64 / G, n_tot = a.n_sel;
    const int64_t tasks = (int64_t)((a.F + P * R - 1) / (P * R)) * n_tot;
    const int blocks = (waves_for(tasks, n_cu, 16) + 3) / 4;
#define FO_GU(GG, UU) \
    if (G == GG && U == UU) { k_gateup<T, UU, GG, R><<<blocks, 256, 0, s>>>(a, xq_h); return hipGetLastError(); }
    FO_GU(64, 1) FO_GU(64, 2) FO_GU(32, 1) FO_GU(16, 1) FO_GU(8, 1) FO_GU(4, 1)
#undef FO_GU
    return hipErrorInvalidValue;
}

hipError_t launch_gateup(int type, const GateUpArgs &a, const uint8_t *xq_h, hipStream_t s, int n_cu) {
    if (a.F <= 0 || a.n_sel <= 0) return hipErrorInvalidValue;
    switch (type) {
        case GGML_TYPE_Q4_K: return gateup_t<GGML_TYPE_Q4_K, 2>(a, xq_h, s, n_cu);
        case GGML_TYPE_Q5_K: return gateup_t<GGML_TYPE_Q5_K, 2>(a, xq_h, s, n_cu);
        case GGML_TYPE_Q6_K: return gateup_t<GGML_TYPE_Q6_K, 2>(a, xq_h, s, n_cu);
        case GGML_TYPE_Q8_0: return gateup_t<GGML_TYPE_Q8_0, 2>(a, xq_h, s, n_cu);
        default: return hipErrorInvalidValue;
    }
}

// ============================================================ down + combine
// Tasks are blocks of P rows of the output; for each routed expert e (in rank
// order) the wave loads NE experts' rows at a time and accumulates weights[e]
// * down_e[row,:].act_e in the lanes before a single group reduction per row;
// out = resid + (sum + ys) (reference src/inference.c: 574 vec_scaled_add in
// rank order, 595 shared add, 606 residual).
template <int T, int U, int G, int NE>
__global__ __launch_bounds__(256) void k_down(DownArgs a, const uint8_t *__restrict__ xq_act,
                                              uint64_t xq_vstride) {
    constexpr int P = kWave / G;
    const int lane = threadIdx.x & 63, sub = lane / G;
    const int w = (int)((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const int nw = (int)((gridDim.x * blockDim.x) >> 6);
    const int S = a.F / Fmt<T>::SLOT;
    const int n_tot = a.n_sel;
    const int tasks = (a.H + P - 1) / P;
    int64_t t0, t1;
    wave_share(tasks, w, nw, t0, t1);
    Slots<U, G> L;
    L.init(lane, S);
    for (int64_t t = t0; t < t1; t++) {
        const int row_u = (int)t * P + sub;
        const int row = min(row_u, a.H - 1);
        float acc = 0.f;
        for (int e0 = 0; e0 < n_tot; e0 += NE) {
            RowRaw<T, U> raw[NE];
#pragma unroll
            for (int i = 0; i < NE; i++) {
                const int e = e0 + i;
                if (e < n_tot) {
                    const uint8_t *m = a.base + (uint64_t)(a.ids ? a.ids[e] : e) * a.stride + a.down_off;
                    load_row(raw[i], m + (uint64_t)row * a.row_bytes, L);
                }
            }
#pragma unroll
            for (int i = 0; i < NE; i++) {
                const int e = e0 + i;
                if (e < n_tot) {
                    XRegs<T, U> X;
                    X.load(L, xq_act + (uint64_t)e * xq_vstride, a.F);
                    acc = fmaf(a.weights[e], dot_row(raw[i], L, X), acc);
                }
            }
        }
        const float v = group_sum<G>(acc);
        if ((lane % G) == 0 && row_u < a.H)
            a.out[row_u] = (a.resid ? a.resid[row_u] : 0.f) + (a.ys ? v + a.ys[row_u] : v);
    }
}

template <int T>
static hipError_t down_t(const DownArgs &a, const uint8_t *xq_act, uint64_t xq_vstride, hipStream_t s,
                         int n_cu) {
    int G, U;
    if (!geometry(T, a.F, G, U)) return hipErrorInvalidValue;
    const int P = 64 / G;
    const int64_t tasks = (a.H + P - 1) / P;
    const int blocks = (waves_for(tasks, n_cu, 16) + 3) / 4;
#define FO_DN(GG, UU) \
    if (G == GG && U == UU) { k_down<T, UU, GG, 4><<<blocks, 256, 0, s>>>(a, xq_act, xq_vstride); return hipGetLastError(); }
    FO_DN(64, 1) FO_DN(64, 2) FO_DN(32, 1) FO_DN(16, 1) FO_DN(8, 1) FO_DN(4, 1)
#undef FO_DN
    return hipErrorInvalidValue;
}

hipError_t launch_down(int type, const DownArgs &a, const uint8_t *xq_act, uint64_t xq_vstride,
                       hipStream_t s, int n_cu) {
    if (a.H <= 0 || a.n_sel < 0) return hipErrorInvalidValue;
    switch (type) {
        case GGML_TYPE_Q4_K: return down_t<GGML_TYPE_Q4_K>(a, xq_act, xq_vstride, s, n_cu);
        case GGML_TYPE_Q5_K: return down_t<GGML_TYPE_Q5_K>(a, xq_act, xq_vstride, s, n_cu);
        case GGML_TYPE_Q6_K: return down_t<GGML_TYPE_Q6_K>(a, xq_act, xq_vstride, s, n_cu);
        case GGML_TYPE_Q8_0: return down_t<GGML_TYPE_Q8_0>(a, xq_act, xq_vstride, s, n_cu);
        default: return hipErrorInvalidValue;
    }
}

// ============================================================ dequantize
// One thread per value, with the exact operation order of the reference
// dequantizers (reference src/quant.c:82-105, 147-175, 216-247, 266-274,
// 298-315); results are bit-identical (the products are exact, see the
// oracle's pins).
__global__ __launch_bounds__(256) void k_dequant(int type, const uint8_t *__restrict__ src,
                                                 float *__restrict__ dst, int64_t n) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float y = 0.f;
    if (type == GGML_TYPE_Q4_K || type == GGML_TYPE_Q5_K) {
        const int bb = type == GGML_TYPE_Q4_K ? 144 : 176;
        const uint8_t *b = src + (i >> 8) * bb;
        const int e = (int)(i & 255), g = e >> 6, hi = (e >> 5) & 1, l = e & 31;
        const int j = 2 * g + hi;
        const uint8_t *sc = b + 4;
        int s6, m6;
        if (j < 4) { s6 = sc[j] & 63; m6 = sc[j + 4] & 63; }
        else { s6 = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4); m6 = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4); }
        const float d = h2f(ld2(b)), dmin = h2f(ld2(b + 2));
        const uint8_t *qs = b + (type == GGML_TYPE_Q4_K ? 16 : 48);
        int q = hi ? (qs[32 * g + l] >> 4) : (qs[32 * g + l] & 0xF);
        if (type == GGML_TYPE_Q5_K) q += ((b[16 + l] >> (2 * g + hi)) & 1) ? 16 : 0;
        const float d1 = d * (float)s6, m1 = dmin * (float)m6;
        y = d1 * (float)q - m1;
    } else if (type == GGML_TYPE_Q6_K) {
        const uint8_t *b = src + (i >> 8) * 210;
        const int e = (int)(i & 255), n = e >> 7, r = e & 127, t = r >> 5, l = r & 31;
        const uint8_t qlb = b[64 * n + l + ((t & 1) ? 32 : 0)];
        const int lo = (t & 2) ? (qlb >> 4) : (qlb & 0xF);
        const int hbits = (b[128 + 32 * n + l] >> (2 * t)) & 3;
        const int q = (lo | (hbits << 4)) - 32;
        const float d = h2f(ld2(b + 208));
        y = d * (float)(int8_t)b[192 + (e >> 4)] * (float)q;
    } else if (type == GGML_TYPE_Q8_0) {
        const uint8_t *b = src + (i >> 5) * 34;
        y = h2f(ld2(b)) * (float)(int8_t)b[2 + (i & 31)];
    } else if (type == GGML_TYPE_MXFP4) {
        const uint8_t *b = src + (i >> 5) * 17;
        const int e = (int)(i & 31);
        const int c = (e < 16) ? (b[1 + e] & 0xF) : (b[1 + e - 16] >> 4);
        const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
        const float v = (c & 8) ? -mag[c & 7] : mag[c & 7];
        const float s = (b[0] == 0xFF) ? 0.0f : ldexpf(1.0f, (int)b[0] - 127);
        y = v * s;
    } else if (type == GGML_TYPE_F16) {
        y = h2f(ld2(src + 2 * i));
    } else if (type == GGML_TYPE_BF16) {
        y = __uint_as_float(ld2(src + 2 * i) << 16);
    } else {
        y = ((const float *)src)[i];
    }
    dst[i] = y;
}

hipError_t launch_dequant(int type, const uint8_t *src, float *dst, int64_t n, hipStream_t s) {
    if (n <= 0) return hipErrorInvalidValue;
    k_dequant<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(type, src, dst, n);
    return hipGetLastError();
}

__global__ void k_silu_mul(float *g, const float *u, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { const float v = g[i]; g[i] = (v / (1.0f + expf(-v))) * u[i]; }
}

hipError_t launch_silu_mul(float *g, const float *u, int64_t n, hipStream_t s) {
    k_silu_mul<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(g, u, n);
    return hipGetLastError();
}

__global__ void k_zero_u32(uint32_t *p, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

hipError_t launch_zero_u32(uint32_t *p, int n, hipStream_t s) {
    k_zero_u32<<<(n + 255) / 256, 256, 0, s>>>(p, n);
    return hipGetLastError();
}

}  // namespace fo
