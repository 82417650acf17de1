// The packed A operand of the prefill grouped GEMM (moe_gemm.hip): rows re-paired block by block
// in the order the MFMA fragments read them, and each 64-wide group's sum split exactly into three
// bf16. Shared by the packing launch and the router launch's packing workgroups (dense.hip).
#pragma once

#include "common.hpp"

namespace mrun {

// X split exactly into three bf16: hi + mid + lo == x (truncations of f32)
__device__ __forceinline__ void split3(float x, uint32_t &hi, uint32_t &mid, uint32_t &lo) {
    const float h = __uint_as_float(__float_as_uint(x) & 0xFFFF0000u);
    const float r1 = x - h;
    const float m = __uint_as_float(__float_as_uint(r1) & 0xFFFF0000u);
    hi = __float_as_uint(h) >> 16;
    mid = __float_as_uint(m) >> 16;
    lo = __float_as_uint(r1 - m) >> 16;
}

// One 8-element block v of a row (block blk): re-paired into its packed position, and its group's
// sum (the 8 blocks of a group are 8 aligned consecutive lanes) split into the three bf16.
// (store = false: the lane only takes part in the group sum)
__device__ __forceinline__ void pack_block_v(uint4 v, int row, bool store, int K, int blk,
                                             bf16_t *__restrict__ xp, int ldp,
                                             bf16_t *__restrict__ xs) {
    const int g = blk >> 3, w = blk & 7;
    const uint4 p = make_uint4(__builtin_amdgcn_perm(v.z, v.x, 0x05040100u),
                               __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                               __builtin_amdgcn_perm(v.w, v.y, 0x05040100u),
                               __builtin_amdgcn_perm(v.w, v.y, 0x07060302u));
    const int pos = 2 * (w & 3) + (w >> 2);
    if (store) *(uint4 *)(xp + (size_t)row * ldp + g * 64 + pos * 8) = p;
    float s = bf_lo(v.x) + bf_hi(v.x);
    s += bf_lo(v.y) + bf_hi(v.y);
    s += bf_lo(v.z) + bf_hi(v.z);
    s += bf_lo(v.w) + bf_hi(v.w);
    s = group_sum<8>(s);
    if (store && w == 0) {
        uint32_t hi, mid, lo;
        split3(s, hi, mid, lo);
        const int G = K / 64;
        bf16_t *d = xs + (size_t)row * 3 * G + g;
        d[0] = (bf16_t)hi;
        d[G] = (bf16_t)mid;
        d[2 * G] = (bf16_t)lo;
    }
}

__device__ __forceinline__ void pack_block(const bf16_t *__restrict__ x, int lda, int row,
                                           bool store, int K, int blk, bf16_t *__restrict__ xp,
                                           int ldp, bf16_t *__restrict__ xs) {
    pack_block_v(*(const uint4 *)(x + (size_t)row * lda + (size_t)blk * 8), row, store, K, blk, xp,
                 ldp, xs);
}

}  // namespace mrun
