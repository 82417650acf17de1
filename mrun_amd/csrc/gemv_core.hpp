// Inner loop of the decode-shaped 4-bit products: one wave streams weight rows with 128-bit loads
// and dots them with a few activation rows, dequantizing in registers.
//
// Dequant: nibble q sits in the low mantissa bits of bf16 128.0 (0x4300 | q == 128 + q exactly),
// so two codes of a word become a bf16 pair with one and-or. The pair holds codes (i, i + 4) of
// the word, and the activations are re-paired the same way once per row (v_perm_b32); v_dot2
// then accumulates x * (128 + q) in f32 and the affine map folds the offset back:
//     sum_k x_k (q_k s + b) = s * sum_k x_k (128 + q_k) + (b - 128 s) * sum_k x_k.
// A lane owns 32-code chunks li, li + LPR, ...; a chunk lies in one quant group (32 | group). The
// LPR lanes of a row are summed by a fixed butterfly, so a row's bits depend on K only.
//
// 8-bit codes (B = 8; a chunk is two uint4): each byte's low and high nibble take the same bf16
// trick, so a word of four codes gives the pairs (lo q_i, lo q_{i+2}), (lo q_{i+1}, lo q_{i+3}) and
// the same for the high nibbles; the activations are re-paired as (x_i, x_{i+2}), (x_{i+1}, x_{i+3})
// and with q = lo + 16 hi:
//     sum_k x_k (q_k s + b) = s * (P'_lo + 16 P'_hi) + (b - 2176 s) * sum_k x_k,
// P'_lo = sum x (128 + lo), P'_hi = sum x (128 + hi), 2176 = 128 * 17.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

namespace mrun {

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

// 32 activations re-paired as (x[8w+i], x[8w+i+4]) in dword 4w+i, and their sum.
struct XChunk {
    uint32_t v[16];
    float sum;
};

// 32 activations as loaded (4 x 128 bits).
struct XRaw {
    uint4 a[4];
};

__device__ __forceinline__ void load_xraw(const bf16_t *src, XRaw &r) {
    const uint4 *p = (const uint4 *)src;
#pragma unroll
    for (int w = 0; w < 4; ++w) r.a[w] = p[w];
}

// 32 activations re-paired for 8-bit codes, the order dot_chunk8 reads: dword 2i holds
// (x[4i], x[4i+2]), dword 2i + 1 holds (x[4i+1], x[4i+3]); and their sum.
__device__ __forceinline__ void pair_x8(const XRaw &r, XChunk &c) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint4 a = r.a[w];
        c.v[4 * w + 0] = __builtin_amdgcn_perm(a.y, a.x, 0x05040100u);  // x0, x2
        c.v[4 * w + 1] = __builtin_amdgcn_perm(a.y, a.x, 0x07060302u);  // x1, x3
        c.v[4 * w + 2] = __builtin_amdgcn_perm(a.w, a.z, 0x05040100u);  // x4, x6
        c.v[4 * w + 3] = __builtin_amdgcn_perm(a.w, a.z, 0x07060302u);  // x5, x7
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s = dot2(c.v[i], 0x3F803F80u, s);
    c.sum = s;
}

__device__ __forceinline__ void pair_x(const XRaw &r, XChunk &c) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const uint4 a = r.a[w];
        c.v[4 * w + 0] = __builtin_amdgcn_perm(a.z, a.x, 0x05040100u);
        c.v[4 * w + 1] = __builtin_amdgcn_perm(a.z, a.x, 0x07060302u);
        c.v[4 * w + 2] = __builtin_amdgcn_perm(a.w, a.y, 0x05040100u);
        c.v[4 * w + 3] = __builtin_amdgcn_perm(a.w, a.y, 0x07060302u);
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s = dot2(c.v[i], 0x3F803F80u, s);
    c.sum = s;
}

// The code mask and the bf16 128.0 pair in VGPRs: with them as operands an and-or is one
// v_and_or_b32 (a three-operand instruction takes no literal constant here). The asm has no side
// effects, so the compiler computes the two values once and keeps them.
__device__ __forceinline__ void code_consts(uint32_t &cm, uint32_t &cx) {
    asm("v_mov_b32 %0, 0x000F000F" : "=v"(cm));
    asm("v_mov_b32 %0, 0x43004300" : "=v"(cx));
}

// sum_k x_k (128 + q_k) over the 32 codes of one uint4.
__device__ __forceinline__ float dot_chunk(const uint4 &q, const XChunk &x) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    uint32_t cm, cx;
    code_consts(cm, cx);
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc = dot2(x.v[4 * i + 0], (w[i] & cm) | cx, acc);
        acc = dot2(x.v[4 * i + 1], ((w[i] >> 4) & cm) | cx, acc);
        acc = dot2(x.v[4 * i + 2], ((w[i] >> 8) & cm) | cx, acc);
        acc = dot2(x.v[4 * i + 3], ((w[i] >> 12) & cm) | cx, acc);
    }
    return acc;
}

// sum_k x_k (128 + lo_k) and sum_k x_k (128 + hi_k) over the 32 codes of two uint4 (8-bit codes)
__device__ __forceinline__ float2 dot_chunk8(const uint4 *q, const XChunk &x) {
    const uint32_t w[8] = {q[0].x, q[0].y, q[0].z, q[0].w, q[1].x, q[1].y, q[1].z, q[1].w};
    uint32_t cm, cx;
    code_consts(cm, cx);
    float lo = 0.f, hi = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        lo = dot2(x.v[2 * i], (w[i] & cm) | cx, lo);
        lo = dot2(x.v[2 * i + 1], ((w[i] >> 8) & cm) | cx, lo);
        hi = dot2(x.v[2 * i], ((w[i] >> 4) & cm) | cx, hi);
        hi = dot2(x.v[2 * i + 1], ((w[i] >> 12) & cm) | cx, hi);
    }
    return make_float2(lo, hi);
}

// One weight row's chunks for one lane: codes (B / 4 uint4 per chunk) and the raw bf16 scale and
// bias. Loads use clamped addresses and are never followed by a use inside a condition, so all of
// a wave's loads are in flight together; `ok` bit c masks the chunks that lie past the row or the
// matrix, bit 31 says whether the weight has biases.
template <int CPL, int B = 4>
struct WRow {
    static constexpr int kBits = B, kQ = B / 4;
    uint4 q[CPL * kQ];
    uint32_t s[CPL], b[CPL];
    uint32_t ok;
};

template <int CPL, int B = 4>
__device__ __forceinline__ void load_wrow(const QW &w, int e, int row, int li, int lpr,
                                          WRow<CPL, B> &r) {
    constexpr int QC = B / 4;  // uint4 of codes per chunk
    const int n_ch = w.in >> 5;
    const int gshift = __builtin_ctz((unsigned)w.group);  // groups of 32, 64 or 128
    const int groups = w.in >> gshift;
    const size_t rr = (size_t)e * w.out + min(row, w.out - 1);
    const uint32_t *codes = w.codes + rr * (size_t)(w.in * B / 32);
    // without biases the scales stand in, so the load is unconditional; row_part zeroes the term
    const bf16_t *biases = w.biases ? w.biases : w.scales;
    r.ok = w.biases ? 0x80000000u : 0u;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const int ch = li + c * lpr;
        const int chc = min(ch, n_ch - 1);
#pragma unroll
        for (int u = 0; u < QC; ++u) r.q[c * QC + u] = *(const uint4 *)(codes + (size_t)chc * 4 * QC + 4 * u);
        const size_t gi = rr * groups + ((chc * 32) >> gshift);
        r.s[c] = w.scales[gi];
        r.b[c] = biases[gi];
        r.ok |= (row < w.out && ch < n_ch) ? (1u << c) : 0u;
    }
}

// Lane's part of row . x over its chunks: s * sum x (128 + q) + (b - 128 s) * sum x. FULL: the
// caller's shape puts every chunk and row in range, so the `ok` masks are all set (same values).
template <int CPL, bool FULL = false, int B = 4>
__device__ __forceinline__ float row_part(const WRow<CPL, B> &r, const XChunk *x) {
    float a = 0.f;
    const bool has_b = (r.ok >> 31) & 1u;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        const bool ok = FULL || ((r.ok >> c) & 1u);
        const float s = ok ? bf2f(r.s[c]) : 0.f;
        if constexpr (B == 8) {
            const float bp = ok ? (has_b ? bf2f(r.b[c]) : 0.f) - 2176.f * s : 0.f;
            const float2 lh = dot_chunk8(&r.q[2 * c], x[c]);
            a += s * (lh.x + 16.f * lh.y) + bp * x[c].sum;
        } else {
            const float bp = ok ? (has_b ? bf2f(r.b[c]) : 0.f) - 128.f * s : 0.f;
            a += s * dot_chunk(r.q[c], x[c]) + bp * x[c].sum;
        }
    }
    return a;
}

// Keeps a row's raw loads opaque inside a loop, so their conversions are not hoisted next to the
// loads (where a conversion would wait for the load before the loads that follow are issued).
template <int CPL, int B>
__device__ __forceinline__ void opaque_row(WRow<CPL, B> &r) {
#pragma unroll
    for (int c = 0; c < CPL * (B / 4); ++c)
        asm volatile("" : "+v"(r.q[c].x), "+v"(r.q[c].y), "+v"(r.q[c].z), "+v"(r.q[c].w));
#pragma unroll
    for (int c = 0; c < CPL; ++c) asm volatile("" : "+v"(r.s[c]), "+v"(r.b[c]));
}

// The lane's chunks of one activation row (clamped: chunks past the row are masked by the
// weights' `ok`, so their values never count).
template <int CPL>
__device__ __forceinline__ void load_xrow_raw(const bf16_t *row, int li, int lpr, int n_ch,
                                              XRaw *x) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) load_xraw(row + min(li + c * lpr, n_ch - 1) * 32, x[c]);
}

template <int CPL, int B = 4>
__device__ __forceinline__ void pair_xrow(const XRaw *raw, XChunk *x) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
        if constexpr (B == 8) pair_x8(raw[c], x[c]);
        else pair_x(raw[c], x[c]);
    }
}

// Rows that one GEMV writes for another to read (the decode's gate/up activations) are stored
// already re-paired: element e of a row sits at paired_index(e), so that a chunk loads as the
// XChunk words pair_x would build (dword 4w + i of a 32-element chunk holds elements 8w + i and
// 8w + i + 4).
__host__ __device__ constexpr int paired_index(int e) {
    return (e & ~31) | (e & 24) | ((e & 3) << 1) | ((e >> 2) & 1);
}
// the same for chunks that 8-bit weights read (pair_x8's order: elements 4i + j at 4i + 2 (j % 2)
// + j / 2, i.e. bits 0 and 1 of the index swapped)
template <int B>
__host__ __device__ constexpr int paired_index_b(int e) {
    if constexpr (B == 8) return (e & ~3) | ((e & 1) << 1) | ((e >> 1) & 1);
    else return paired_index(e);
}

// A chunk stored re-paired: the words as loaded, and their sum in pair_x's order (same bits).
__device__ __forceinline__ void chunk_of_paired(const XRaw &r, XChunk &c) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        c.v[4 * w + 0] = r.a[w].x;
        c.v[4 * w + 1] = r.a[w].y;
        c.v[4 * w + 2] = r.a[w].z;
        c.v[4 * w + 3] = r.a[w].w;
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s = dot2(c.v[i], 0x3F803F80u, s);
    c.sum = s;
}

template <int CPL>
__device__ __forceinline__ void chunks_of_paired(const XRaw *raw, XChunk *x) {
#pragma unroll
    for (int c = 0; c < CPL; ++c) chunk_of_paired(raw[c], x[c]);
}

}  // namespace mrun
