// topk.h — single-wave top-k with renormalised weights, shared by the
// batch-1 layer (moe.hip) and the prefill path (prefill.hip).
#pragma once

#include <float.h>

#include "common.h"

namespace fo {

// Top-k of E logits (<= 1024) as the reference selects them: over the fp32
// probabilities p_i = expf(l_i - l_max) * (1 / sum) (reference
// src/tensor.c:186-200), largest first, ties to the lowest index
// (src/tensor.c:226-252), with the selected p renormalised
// (src/inference.c:496-502). p is monotone in l, so the selection runs on the
// logits and the weights are exp(l_i - l_1) / sum over the selection (the
// same quantity), unless the last selected logit lies more than kSatGap below
// the first: then p of the selection or of its rivals can underflow, distinct
// logits can share p = 0 and the reference's ties apply, so the selection
// runs again on p itself and the weights renormalise p as the reference does.
// One wave: k rounds of "largest (value, lowest index)" over its lanes; the
// results go to LDS s_ids[k], s_w[k] (visible after the caller's barrier).
// Each round costs ~500 cycles of dependent VALU/SGPR latency, so the whole
// selection is ~2 us of single-wave latency; splitting it over four waves
// measured slower (the merge round-trip through LDS costs more than it saves).
constexpr int kMaxE = 1024, kMaxK = 16;
// exp(-80) / 1024 is still a normal float: above this gap p of every
// selected expert is positive and normal and no unselected one can tie with it
constexpr float kSatGap = 80.f;

// One round of "take the largest (value, lowest index)" over the wave: lb/li
// are this lane's best; returns the winner's value and index (uniform).
FO_DEV void wave_argmax(float lb, int li, float &m, int &idx) {
    float t = lb;
    t = fmaxf(t, dpp<0xB1>(t));
    t = fmaxf(t, dpp<0x4E>(t));
    t = fmaxf(t, dpp<0x141>(t));
    t = fmaxf(t, dpp<0x140>(t));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(t), 48));
    m = fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
    const uint64_t ball = __ballot(lb == m);
    if (__popcll(ball) == 1) {
        idx = __builtin_amdgcn_readlane(li, __ffsll((unsigned long long)ball) - 1);
    } else {  // tie: lowest index among the lanes holding m
        int c = lb == m ? li : 0x7FFFFFFF;
        c = min(c, __builtin_amdgcn_update_dpp(c, c, 0xB1, 0xF, 0xF, false));
        c = min(c, __builtin_amdgcn_update_dpp(c, c, 0x4E, 0xF, 0xF, false));
        c = min(c, __builtin_amdgcn_update_dpp(c, c, 0x141, 0xF, 0xF, false));
        c = min(c, __builtin_amdgcn_update_dpp(c, c, 0x140, 0xF, 0xF, false));
        idx = min(min(__builtin_amdgcn_readlane(c, 0), __builtin_amdgcn_readlane(c, 16)),
                  min(__builtin_amdgcn_readlane(c, 32), __builtin_amdgcn_readlane(c, 48)));
    }
}

// This lane's logits 64j + lane (-FLT_MAX past E).
template <int NV>
FO_DEV void wave_logits(const float *__restrict__ logits, int E, float (&v)[NV]) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = 64 * j + lane;
        v[j] = i < E ? logits[i] : -FLT_MAX;
    }
}

// Logits (from wave_logits) to softmax probabilities in place, -1 past E
// (below every probability); NaN logits drop out of the max.
template <int NV>
FO_DEV void wave_probs(float (&v)[NV], int E) {
    const int lane = threadIdx.x & 63;
    float mx = -FLT_MAX;
#pragma unroll
    for (int j = 0; j < NV; j++) mx = fmaxf(mx, v[j]);
    mx = wave_max(mx);
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < NV; j++) {
        v[j] = 64 * j + lane < E ? expf(v[j] - mx) : 0.f;
        sum += v[j];
    }
    const float inv = 1.0f / group_sum<kWave>(sum);
#pragma unroll
    for (int j = 0; j < NV; j++) v[j] = 64 * j + lane < E ? v[j] * inv : -1.f;
}

// Weight of the selection held by lanes 0..k-1 (value v). Probabilities:
// v * (1 / their sum in rank order) when the sum is positive, else v.
// Logits: exp(v - v_0) / the sum of those.
FO_DEV float select_weight(float v, int k, bool prob) {
    if (prob) {
        float s = 0.f;
        for (int r = 0; r < k; r++) s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), r));
        return s > 0.f ? v * (1.0f / s) : v;
    }
    const int lane = threadIdx.x & 63;
    const float m0 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
    const float e = lane < k ? expf(v - m0) : 0.f;
    return e * (1.0f / group_sum<kWave>(e));
}

// Whether a logit selection from `first` down to `last` needs no rerun on p
// (false for non-finite values as well).
FO_DEV bool logit_selection_exact(float first, float last) { return last - first > -kSatGap; }

// Whether the logit order of the kr values held by lanes 0..kr-1 (largest
// first, equal values in index order; the last is the best value left out of
// a selection of kr-1) is also the order of their fp32 probabilities. Two
// distinct logits a > b can round to the same p = expf(l - l_max) * inv, and
// the reference then takes the lower index first. With d = l - l_max, p's
// relative change is a - b, while the rounding of d (half an ulp of |d|),
// expf (about an ulp) and the product with inv (half an ulp) move p by less
// than 2^-21 max(1, |d|) relative; so adjacent logits that are equal or
// further apart than 2^-20 max(1, |d|) keep their order in p, and any other
// pair sends the selection to the rerun on p.
FO_DEV bool logit_order_exact(float v, int kr, float first) {
    const int lane = threadIdx.x & 63;
    const float nx = __shfl_down(v, 1, kWave);
    bool ok = true;
    if (lane + 1 < kr) ok = v == nx || v - nx > 0x1p-20f * fmaxf(1.0f, fabsf(nx - first));
    return __ballot(!ok) == 0;
}

// Selection of k over v (logits, or probabilities when prob; E <= 64*NV;
// consumed); returns false when a logit selection must rerun on p. Over
// logits one more value is taken, the best one left out, for the order check
// at the selection's boundary.
template <int NV>
FO_DEV bool wave_topk_v(float (&v)[NV], int E, int k, int *s_ids, float *s_w, bool prob) {
    const int lane = threadIdx.x & 63;
    const int kr = (!prob && k < E) ? k + 1 : k;
    float my_v = -FLT_MAX;   // lane kk keeps selection kk (no indexed private arrays:
    int my_i = 0;            // those would put the kernel on scratch, which throttles residency)
    for (int kk = 0; kk < kr; kk++) {
        float lb = v[0];
        int lj = 0;
#pragma unroll
        for (int j = 1; j < NV; j++)
            if (v[j] > lb) { lb = v[j]; lj = j; }
        float m;
        int idx;
        wave_argmax(lb, 64 * lj + lane, m, idx);
        if (idx < 0 || idx >= E) idx = 0;   // non-finite logits: never index outside the table
        if (lane == kk) { my_v = m; my_i = idx; }
        if (lane == (idx & 63)) {
#pragma unroll
            for (int j = 0; j < NV; j++)
                if (j == (idx >> 6)) v[j] = -FLT_MAX;
        }
    }
    const float first = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_v), 0));
    const float last = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_v), k - 1));
    if (!prob && (!logit_selection_exact(first, last) || !logit_order_exact(my_v, kr, first))) return false;
    const float wv = s_w ? select_weight(my_v, k, prob) : 0.f;
    if (lane < k) { s_ids[lane] = my_i; if (s_w) s_w[lane] = wv; }
    return true;
}

template <int NV>
FO_DEV void wave_topk(const float *__restrict__ logits, int E, int k, int *s_ids, float *s_w) {
    float v[NV];
    wave_logits<NV>(logits, E, v);
    if (wave_topk_v<NV>(v, E, k, s_ids, s_w, false)) return;
    wave_logits<NV>(logits, E, v);
    wave_probs<NV>(v, E);
    wave_topk_v<NV>(v, E, k, s_ids, s_w, true);
}

// Same selection through a threshold: the 64 lane maxima are sorted across
// the wave (a 21-step flip / half-cleaner network: DPP inside 16-lane rows,
// three permutes across rows), so T = the k-th largest lane maximum; k lane
// maxima are >= T, hence the top k of all E values are all >= T. The
// candidates (every value >= T: k plus the few second-best values of the
// same lanes) are compacted to LDS, twice in a row, and ranked exactly by
// (value desc, index asc) against the next n-1 entries of that doubled list
// with wave-wide DPP shifts. Falls back to k arg-max rounds when k > 16 or
// more than 32 values tie in at T (or NaNs leave fewer than k candidates).
// Over logits it ranks k+1 values (the boundary check of logit_order_exact;
// s_ids and s_val then receive k+1 entries). s_cand: 64 (value, index)
// slots, s_val: k + 1 values, both in LDS.
template <int CTRL>
FO_DEV float dpp_keep(float v) {   // lanes whose source is outside the row keep v
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
FO_DEV int dpp_keep_i(int v) { return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xF, 0xF, false); }

template <int NV>
FO_DEV bool wave_topk_thr_v(float (&v)[NV], int E, int k, int *s_ids, float *s_w, float2 *s_cand,
                            float *s_val, bool prob) {
    const int lane = threadIdx.x & 63, r = lane & 15;
    const int kr = (!prob && k < E) ? k + 1 : k;   // logits: also the best one left out
    float mx = -FLT_MAX;
#pragma unroll
    for (int j = 0; j < NV; j++) mx = fmaxf(mx, v[j]);   // NaNs drop out
    // descending sort of the lane maxima (lower lane = larger value)
    auto cx = [&](float p, bool lo) { mx = lo ? fmaxf(mx, p) : fminf(mx, p); };
    auto x4 = [&]() { const float u = dpp_keep<0x104>(mx), d = dpp_keep<0x114>(mx); cx((r & 4) ? d : u, !(r & 4)); };
    auto x8 = [&]() { const float u = dpp_keep<0x108>(mx), d = dpp_keep<0x118>(mx); cx((r & 8) ? d : u, !(r & 8)); };
    auto x2 = [&]() { cx(dpp_keep<0x4E>(mx), !(r & 2)); };
    auto x1 = [&]() { cx(dpp_keep<0xB1>(mx), !(r & 1)); };
    x1();                                                      // size 2
    cx(dpp_keep<0x1B>(mx), !(r & 2)); x1();                    // size 4 (flip = quad mirror)
    cx(dpp_keep<0x141>(mx), !(r & 4)); x2(); x1();             // size 8 (flip = half-row mirror)
    cx(dpp_keep<0x140>(mx), !(r & 8)); x4(); x2(); x1();       // size 16 (flip = row mirror)
    cx(__shfl_xor(mx, 31, kWave), !(lane & 16)); x8(); x4(); x2(); x1();                     // size 32
    cx(__shfl_xor(mx, 63, kWave), !(lane & 32)); cx(__shfl_xor(mx, 16, kWave), !(lane & 16));
    x8(); x4(); x2(); x1();                                    // size 64
    bool ok = kr <= 16;
    int n = 0;
    if (ok) {
        const float T = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), kr - 1));
        uint64_t m[NV];
#pragma unroll
        for (int j = 0; j < NV; j++) { m[j] = __ballot(v[j] >= T); n += __popcll(m[j]); }
        ok = n >= kr && n <= 32;
        if (ok) {   // candidates in (j, lane) order at [0, n) and again at [n, 2n)
            int base = 0;
#pragma unroll
            for (int j = 0; j < NV; j++) {
                const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m[j] >> 32),
                                                                      __builtin_amdgcn_mbcnt_lo((uint32_t)m[j], 0u));
                if (v[j] >= T) {
                    const float2 cv = make_float2(v[j], __int_as_float(64 * j + lane));
                    s_cand[pos] = cv;
                    s_cand[pos + n] = cv;
                }
                base += __popcll(m[j]);
            }
        }
    }
    if (!ok) return wave_topk_v<NV>(v, E, k, s_ids, s_w, prob);
    // lane l < n ranks candidate l against entries l+1 .. l+n-1 of the doubled list
    const float2 c = lane < 2 * n ? s_cand[lane] : make_float2(-FLT_MAX, __int_as_float(0x7FFFFFFF));
    const int ci = __float_as_int(c.y);
    float ov = c.x;
    int oi = ci, rank = 0;
    for (int q = 1; q < n; q++) {
        ov = dpp_keep<0x130>(ov);      // wave_shl:1 — lane l now sees entry l+q
        oi = dpp_keep_i<0x130>(oi);
        rank += (ov > c.x || (ov == c.x && oi < ci)) ? 1 : 0;
    }
    if (lane < n && rank < kr) {
        s_ids[rank] = (ci >= 0 && ci < E) ? ci : 0;
        s_val[rank] = c.x;
    }
    if (!prob && (!logit_selection_exact(s_val[0], s_val[k - 1]) ||
                  !logit_order_exact(lane < kr ? s_val[lane] : 0.f, kr, s_val[0])))
        return false;
    if (s_w) {
        const float wv = select_weight(lane < k ? s_val[lane] : 0.f, k, prob);
        if (lane < k) s_w[lane] = wv;
    }
    return true;
}

template <int NV>
FO_DEV void wave_topk_thr(const float *__restrict__ logits, int E, int k, int *s_ids, float *s_w,
                          float2 *s_cand, float *s_val) {
    float v[NV];
    wave_logits<NV>(logits, E, v);
    if (wave_topk_thr_v<NV>(v, E, k, s_ids, s_w, s_cand, s_val, false)) return;
    wave_logits<NV>(logits, E, v);
    wave_probs<NV>(v, E);
    wave_topk_thr_v<NV>(v, E, k, s_ids, s_w, s_cand, s_val, true);
}

}  // namespace fo
