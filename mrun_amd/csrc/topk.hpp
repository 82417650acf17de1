// Softmax + top-k of one token's router logits, shared by the router and the decode kernels so
// that every kernel derives bit-identical expert choices and scores (moe.rs:151-159).
#pragma once

#include "common.hpp"

namespace mrun {

constexpr int kMaxExpertsPerLane = 8;  // E <= 512
constexpr int kMaxTopK = 16;

// NPER = experts per lane (E <= 64 * NPER).
template <int NPER>
__device__ __forceinline__ void topk_token_n(const bf16_t *__restrict__ lrow, int E, int k,
                                             bool norm, bf16_t *__restrict__ grow,
                                             uint32_t *__restrict__ idrow,
                                             bf16_t *__restrict__ srow) {
    constexpr int kMaxExpertsPerLane = NPER;
    const int lane = threadIdx.x & 63;
    float lv[kMaxExpertsPerLane];
    uint32_t key[kMaxExpertsPerLane];
    // every load is issued before any is used (clamped indices, no loads under a condition)
    uint32_t raw[kMaxExpertsPerLane];
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i) raw[i] = lrow[min(lane + 64 * i, E - 1)];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i) {
        lv[i] = lane + 64 * i < E ? bf2f(raw[i]) : -INFINITY;
        m = fmaxf(m, lv[i]);
    }
    m = wave_max(m);
    float s = 0.f, ex[kMaxExpertsPerLane];
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i) {
        const int e = lane + 64 * i;
        ex[i] = e < E ? expf(lv[i] - m) : 0.f;
        s += ex[i];
    }
    s = group_sum<64>(s);
#pragma unroll
    for (int i = 0; i < kMaxExpertsPerLane; ++i) {
        const int e = lane + 64 * i;
        if (e < E) {
            const uint32_t g = f2bf(ex[i] / s);
            if (grow) grow[e] = (bf16_t)g;
            key[i] = (g << 16) | (uint32_t)(0xffff - e);
        } else {
            key[i] = 0;
        }
    }
    float gsel[kMaxTopK];
#pragma unroll
    for (int j = 0; j < kMaxTopK; ++j) {
        if (j < k) {
            uint32_t best = 0;
#pragma unroll
            for (int i = 0; i < kMaxExpertsPerLane; ++i) best = key[i] > best ? key[i] : best;
            best = wave_max_u32(best);
#pragma unroll
            for (int i = 0; i < kMaxExpertsPerLane; ++i)
                if (key[i] == best) key[i] = 0;
            gsel[j] = bf2f(best >> 16);
            if (lane == 0) idrow[j] = 0xffffu - (best & 0xffffu);
        }
    }
    if (lane == 0) {
        float sum = 0.f;
        if (norm) {
#pragma unroll
            for (int j = 0; j < kMaxTopK; ++j)
                if (j < k) sum += gsel[j];
            sum = rbf(sum);
        }
#pragma unroll
        for (int j = 0; j < kMaxTopK; ++j)
            if (j < k) srow[j] = (bf16_t)f2bf(norm ? gsel[j] / sum : gsel[j]);
    }
}

__device__ __forceinline__ void topk_token(const bf16_t *__restrict__ lrow, int E, int k, bool norm,
                                           bf16_t *__restrict__ grow, uint32_t *__restrict__ idrow,
                                           bf16_t *__restrict__ srow) {
    if (E <= 128) topk_token_n<2>(lrow, E, k, norm, grow, idrow, srow);
    else if (E <= 192) topk_token_n<3>(lrow, E, k, norm, grow, idrow, srow);
    else if (E <= 256) topk_token_n<4>(lrow, E, k, norm, grow, idrow, srow);
    else topk_token_n<8>(lrow, E, k, norm, grow, idrow, srow);
}

}  // namespace mrun
