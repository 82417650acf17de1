// Device helpers shared by the MoE kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint16_t bf16_t;

namespace mrun {

// Workgroup barrier that waits for this wave's LDS (and scalar) operations only: global loads
// issued before it stay in flight. __syncthreads also waits for every outstanding vector memory
// operation (vmcnt(0)), which turns loads issued several steps ahead into loads waited for at the
// next barrier. The "memory" clobber keeps the compiler from moving memory accesses across it; the
// compiler still waits for each prefetched register before its first use.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// bf16 bits <-> f32. Rounding is to nearest even; NaN stays NaN (quiet). The conversion is
// gfx950's v_cvt_pk_bf16_f32, which gives the integer round-to-nearest-even
//   u += 0x7fff + ((u >> 16) & 1); u >> 16
// for every non-NaN f32 (checked on the device over all 2^32 inputs), in one instruction.
__device__ __forceinline__ float bf2f(uint32_t h) { return __uint_as_float(h << 16); }
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ uint32_t f2bf(float f) {
    return (uint32_t)__builtin_bit_cast(unsigned short, (__bf16)f);
}
// two values into one packed word (a in the low half)
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
    typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
    const bf16x2_t v = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, v);
}
// f rounded to the nearest bf16 value, kept as f32.
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

__device__ __forceinline__ float sigmoidf_(float z) { return 1.0f / (1.0f + expf(-z)); }

// Cross-lane reductions without the LDS crossbar: DPP moves combine lanes inside each 16-lane row
// (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror: every lane of a row
// ends with the row's total), then v_readlane gathers the rows' totals into scalars. The order of
// the additions is fixed, so results are deterministic.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __uint_as_float(dpp_u32<CTRL>(__float_as_uint(v)));
}
__device__ __forceinline__ float lane_f32(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// v + (a row broadcast of v) in some rows; the other rows keep v. One v_add_f32 with the DPP
// control (the DPP source is the first operand; disabled rows leave the destination, which is v).
// The s_nops cover the DPP read of a just-written VGPR and a read of the result right after.
//   bcast15: rows 1 and 3 add lanes 15 and 47;  bcast31: rows 2 and 3 add lane 31.
__device__ __forceinline__ float add_row_bcast15(float v) {
    asm("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\ts_nop 1"
        : "+v"(v));
    return v;
}
__device__ __forceinline__ float add_row_bcast31(float v) {
    asm("s_nop 1\n\tv_add_f32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf\n\ts_nop 1"
        : "+v"(v));
    return v;
}

__device__ __forceinline__ float row_sum16(float v) {
    v += dpp_f32<0xB1>(v);
    v += dpp_f32<0x4E>(v);
    v += dpp_f32<0x141>(v);
    v += dpp_f32<0x140>(v);
    return v;
}

// Sum over groups of WIDTH consecutive lanes (16, 32 or 64); every lane of a group receives its
// group's total.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(WIDTH == 1 || WIDTH == 2 || WIDTH == 4 || WIDTH == 8 || WIDTH == 16 ||
                      WIDTH == 32 || WIDTH == 64,
                  "group width");
    if (WIDTH == 1) return v;
    if (WIDTH == 2) return v + dpp_f32<0xB1>(v);
    if (WIDTH == 4) {
        v += dpp_f32<0xB1>(v);
        return v + dpp_f32<0x4E>(v);
    }
    if (WIDTH == 8) {
        v += dpp_f32<0xB1>(v);
        v += dpp_f32<0x4E>(v);
        return v + dpp_f32<0x141>(v);
    }
    v = row_sum16(v);
    if (WIDTH == 16) return v;
    // row totals r0..r3 -> (r0 + r1) and (r2 + r3) in rows 1 and 3 (row_bcast:15 adds lane 15's
    // value into row 1 and lane 47's into row 3; the other rows keep theirs), then
    // (r0 + r1) + (r2 + r3) in row 3 (row_bcast:31 adds lane 31's value into rows 2 and 3).
    // Addition commutes exactly, so the sums are bit for bit those of (r0 + r1) + (r2 + r3).
    v = add_row_bcast15(v);
    if (WIDTH == 32) return (threadIdx.x & 32) ? lane_f32(v, 63) : lane_f32(v, 31);
    v = add_row_bcast31(v);
    return lane_f32(v, 63);
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f32<0xB1>(v));
    v = fmaxf(v, dpp_f32<0x4E>(v));
    v = fmaxf(v, dpp_f32<0x141>(v));
    v = fmaxf(v, dpp_f32<0x140>(v));
    return fmaxf(fmaxf(lane_f32(v, 0), lane_f32(v, 16)), fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

__device__ __forceinline__ uint32_t umax_(uint32_t a, uint32_t b) { return a > b ? a : b; }

// Eight bf16 (one uint4) dotted with eight f32 codes.
__device__ __forceinline__ void unpack8(const uint4 &v, float *f) {
    f[0] = bf_lo(v.x); f[1] = bf_hi(v.x);
    f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
    f[4] = bf_lo(v.z); f[5] = bf_hi(v.z);
    f[6] = bf_lo(v.w); f[7] = bf_hi(v.w);
}

// ss + f[0]^2 + ... + f[7]^2 in that order, and 1 / sqrt(sum / D + eps): the two steps every
// RMSNorm here shares, so that all of them round alike.
__device__ __forceinline__ float sumsq8(const float *f, float ss) {
#pragma unroll
    for (int k = 0; k < 8; ++k) ss += f[k] * f[k];
    return ss;
}
__device__ __forceinline__ float rms_inv_of(float sum, int D, float eps) {
    return 1.0f / sqrtf(sum / (float)D + eps);
}

// 1 / sqrt(mean(x^2) + eps) of one bf16 row of D elements (D % 8 == 0), computed by one wave in a
// fixed order — lane l sums elements 8 l + 512 i + j (i, then j) over 2048-element passes, then a
// butterfly over the wave — so every kernel that normalises a row gets the same bits (RMSNorm,
// fast::rms_norm nuvec.rs:796-798). With res, the row is R(x + res) (add_rms_norm).
__device__ __forceinline__ float row_rms_inv(const bf16_t *x, const bf16_t *res, int D, float eps,
                                             int lane) {
    float ss = 0.f;
    for (int d = lane * 8; d < D; d += 2048) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (d + 512 * i < D) {
                const uint4 v = *(const uint4 *)(x + d + 512 * i);
                float f[8];
                f[0] = bf_lo(v.x), f[1] = bf_hi(v.x), f[2] = bf_lo(v.y), f[3] = bf_hi(v.y);
                f[4] = bf_lo(v.z), f[5] = bf_hi(v.z), f[6] = bf_lo(v.w), f[7] = bf_hi(v.w);
                if (res) {
                    const uint4 r = *(const uint4 *)(res + d + 512 * i);
                    f[0] = rbf(f[0] + bf_lo(r.x)), f[1] = rbf(f[1] + bf_hi(r.x));
                    f[2] = rbf(f[2] + bf_lo(r.y)), f[3] = rbf(f[3] + bf_hi(r.y));
                    f[4] = rbf(f[4] + bf_lo(r.z)), f[5] = rbf(f[5] + bf_hi(r.z));
                    f[6] = rbf(f[6] + bf_lo(r.w)), f[7] = rbf(f[7] + bf_hi(r.w));
                }
                ss = sumsq8(f, ss);
            }
        }
    }
    return rms_inv_of(group_sum<64>(ss), D, eps);
}

}  // namespace mrun
