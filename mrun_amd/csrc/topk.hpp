// Softmax + top-k of one token's router logits, shared by the router and the decode kernels so
// that every kernel derives bit-identical expert choices and scores (moe.rs:151-159).
//
// One wave per token; lane l holds experts l, l + 64, ... Keys are (gate << 16) | (0xffff - id),
// so the k largest keys are the k largest gates with equal gates ranked by ascending id (the tie
// rule argpartition leaves open, nuvec.rs:558-562), listed in rank order. Each of the k rounds is
// one wave-wide maximum (DPP within rows, row broadcasts across them, one readlane). The scores
// are computed by lanes 0..k-1 in parallel.
#pragma once

#include "common.hpp"

namespace mrun {

constexpr int kMaxExpertsPerLane = 8;  // E <= 512
constexpr int kMaxTopK = 16;

// Maximum over the wave, left in a scalar: four DPP steps inside each 16-lane row, then the row
// broadcasts (lane 15 into rows 1 and 3, lane 31 into rows 2 and 3), so lane 63 holds the result.
__device__ __forceinline__ uint32_t wave_max_u32_b(uint32_t v) {
    v = umax_(v, dpp_u32<0xB1>(v));
    v = umax_(v, dpp_u32<0x4E>(v));
    v = umax_(v, dpp_u32<0x141>(v));
    v = umax_(v, dpp_u32<0x140>(v));
    v = umax_(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x142, 0xA, 0xF, false));
    v = umax_(v, (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, 0x143, 0xC, 0xF, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// bf16(RN32(a / b)) for finite a >= 0, b > 0. A reciprocal and one Newton step land within a few
// ulp of the correctly rounded quotient. That already decides the bf16 rounding unless the
// quotient's low 16 bits lie near the bf16 midpoint 0x8000; only then the IEEE division runs.
__device__ __forceinline__ uint32_t bf16_quotient(float a, float b) {
    const float r = __builtin_amdgcn_rcpf(b);
    float q = a * r;
    q = __builtin_fmaf(__builtin_fmaf(-q, b, a), r, q);
    if ((__float_as_uint(q) & 0xFFFFu) - 0x7FF0u <= 0x20u) q = a / b;
    return f2bf(q);
}

// NPER = experts per lane (E <= 64 * NPER).
template <int NPER>
__device__ __forceinline__ void topk_token_n(const bf16_t *__restrict__ lrow, int E, int k,
                                             bool norm, bf16_t *__restrict__ grow,
                                             uint32_t *__restrict__ idrow,
                                             bf16_t *__restrict__ srow) {
    const int lane = threadIdx.x & 63;
    // every load is issued before any is used (clamped indices, no loads under a condition)
    uint32_t raw[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) raw[i] = lrow[min(lane + 64 * i, E - 1)];
    float lv[NPER];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        lv[i] = lane + 64 * i < E ? bf2f(raw[i]) : -INFINITY;
        m = fmaxf(m, lv[i]);
    }
    m = wave_max(m);
    float s = 0.f, ex[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        ex[i] = lane + 64 * i < E ? expf(lv[i] - m) : 0.f;
        s += ex[i];
    }
    s = group_sum<64>(s);
    uint32_t key[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
        const int e = lane + 64 * i;
        const uint32_t g = bf16_quotient(ex[i], s);  // R(softmax), as nuvec.rs:593-598
        if (grow && e < E) grow[e] = (bf16_t)g;
        key[i] = e < E ? (g << 16) | (uint32_t)(0xffff - e) : 0u;
    }
    uint32_t best[kMaxTopK];
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
        best[j] = 0;
        if (j < k) {
            uint32_t b = key[0];
#pragma unroll
            for (int i = 1; i < NPER; ++i) b = umax_(b, key[i]);
            b = wave_max_u32_b(b);
#pragma unroll
            for (int i = 0; i < NPER; ++i) key[i] = key[i] == b ? 0u : key[i];
            best[j] = b;
        }
    }
    float sum = 0.f;
    if (norm) {
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            if (j < k) sum += bf2f(best[j] >> 16);  // in rank order, as the reference sums
        sum = rbf(sum);
    }
    uint32_t mine = 0;
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) mine = lane == j ? best[j] : mine;
    if (lane < k) {
        idrow[lane] = 0xffffu - (mine & 0xffffu);
        srow[lane] = (bf16_t)(norm ? bf16_quotient(bf2f(mine >> 16), sum) : (mine >> 16));
    }
}

__device__ __forceinline__ void topk_token(const bf16_t *__restrict__ lrow, int E, int k, bool norm,
                                           bf16_t *__restrict__ grow, uint32_t *__restrict__ idrow,
                                           bf16_t *__restrict__ srow) {
    if (E <= 256) topk_token_n<4>(lrow, E, k, norm, grow, idrow, srow);
    else topk_token_n<8>(lrow, E, k, norm, grow, idrow, srow);
}

}  // namespace mrun
