// topk.h — single-wave top-k with renormalised weights, shared by the
// batch-1 layer (moe.hip) and the prefill path (prefill.hip).
#pragma once

#include <float.h>

#include "common.h"

namespace fo {

// Top-k of E logits (<= 1024) with ties to the lowest index — the order of
// reference src/tensor.c:226-252 applied to softmax(logits), which is
// monotone — and the renormalised weights exp(l_i - l_max) / sum over the
// selection (= softmax then renormalise, reference src/inference.c:488-502).
// One wave: k rounds of "largest (value, lowest index)" over its lanes; the
// results go to LDS s_ids[k], s_w[k] (visible after the caller's barrier).
// Each round costs ~500 cycles of dependent VALU/SGPR latency, so the whole
// selection is ~2 us of single-wave latency; splitting it over four waves
// measured slower (the merge round-trip through LDS costs more than it saves).
constexpr int kMaxE = 1024, kMaxK = 16;

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

template <int NV>  // logits per lane: E <= 64*NV
FO_DEV void wave_topk(const float *__restrict__ logits, int E, int k, int *s_ids, float *s_w) {
    const int lane = threadIdx.x & 63;
    float v[NV];
#pragma unroll
    for (int j = 0; j < NV; j++) {
        const int i = 64 * j + lane;
        v[j] = i < E ? logits[i] : -FLT_MAX;
    }
    float my_v = -FLT_MAX;   // lane kk keeps selection kk (no indexed private arrays:
    int my_i = 0;            // those would put the kernel on scratch, which throttles residency)
    for (int kk = 0; kk < k; kk++) {
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
    const float m0 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(my_v)));
    const float e = lane < k ? expf(my_v - m0) : 0.f;
    const float inv = 1.0f / group_sum<kWave>(e);
    if (lane < k) { s_ids[lane] = my_i; if (s_w) s_w[lane] = e * inv; }
}

}  // namespace fo
