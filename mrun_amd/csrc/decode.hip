// Decode schedule of the MoE block (T <= 16 tokens, T*k <= 128 pairs): three launches, no global
// routing round trip and no permutation (SparseMoe::forward, moe.rs:149-174).
//
//   K1 router  : router logits (+ bias) and the shared expert's gate logit, one wave per row.
//   K2 gate/up : the shared expert's gate/up + SwiGLU (it does not depend on the routing, so those
//                workgroups stream from the first cycle), and the routed experts: every routed
//                workgroup re-derives the top-k of all T tokens from the logits (the same code as
//                the router op, so the same bits; T > 4 reads them from a top-k launch instead),
//                picks the slot-th active expert (experts in ascending order) and streams that
//                expert's gate/up rows for its pairs. The first routed workgroup publishes the
//                routing for K3.
//   K3 down    : prefetches the shared expert's down rows, reads the routing, computes the routed
//                down rows of every active expert for its 4 or 8 output rows and its group of
//                tokens (two groups from T = 2, four from T = 8), then the combine of those tokens:
//                out = R(R(sum_j R(y[t,j] * s[t,j])) + R(R(sigmoid(g_t)) * shared[t])).
// Rows wider than 2048 (the Coder shape): a K2 workgroup streams several row blocks pair by pair
// with the next rows loaded before the current ones are computed, and without a shared expert K3
// takes one wave per pair streaming that expert's down rows. Every row keeps the same bits.
// Pair p = t*k + j indexes the activations (act [T*k, I]), so no argsort is needed at decode; the
// results are the same as the sorted dispatch's, row by row.
#include <hip/hip_ext.h>

#include "common.hpp"
#include "gemv_core.hpp"
#include "kernels.hpp"
#include "topk.hpp"

namespace mrun {

constexpr int kMaxT = 32, kMaxP = 256;

// A set of pair indices below kMaxP = 256 (one bit each), taken in ascending order. Four named
// words rather than an array, so that the set stays in scalar registers (an indexed array went
// to scratch memory).
struct PairSet {
    uint64_t m0, m1, m2, m3;
    // the lowest pair left, removed from the set; -1 when the set is empty
    __device__ __forceinline__ int next() {
        if (m0) return take(m0, 0);
        if (m1) return take(m1, 64);
        if (m2) return take(m2, 128);
        if (m3) return take(m3, 192);
        return -1;
    }
    __device__ __forceinline__ static int take(uint64_t &w, int base) {
        const int p = base + __ffsll((unsigned long long)w) - 1;
        w &= w - 1;
        return p;
    }
};
static_assert(kMaxP == 256, "PairSet holds 256 pairs");

// Lane l + d's value of v for d = 16 and 32 (permlane swaps of v with itself) and l ^ 8, l ^ 4,
// l ^ 2, l ^ 1 (DPP), each added to v: a butterfly level on lane bit 5, 4, 3, 2, 1 or 0.
__device__ __forceinline__ float swap_add32(float a, float b) {  // lanes < 32: a; >= 32: b
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                    false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float swap_add16(float a, float b) {  // even rows: a; odd rows: b
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false,
                                                    false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float butterfly_low4(float v) {  // lane bits 3, 2, 1, 0
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x128, 0xF, 0xF, false));
    int m = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x104, 0xF, 0x5, false);  // l + 4
    m = __builtin_amdgcn_update_dpp(m, __float_as_int(v), 0x114, 0xF, 0xA, false);      // l - 4
    v += __int_as_float(m);
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}

// Sums over the wave of RG (2 or 4) rows' gate values g and up values u, scattered: the lanes of
// row r's range [64 r / RG, 64 (r + 1) / RG) end with its two sums in gs and us. Whatever RG, a
// sum pairs lanes by bit 5 of their index first, then bits 4, 3, 2, 1 and 0, so a row's sums
// have the same bits for every RG.
template <int RG>
__device__ __forceinline__ void rows_reduce_scatter(const float (&g)[RG], const float (&u)[RG],
                                                    float &gs, float &us) {
    static_assert(RG == 2 || RG == 4, "two or four rows");
    float g16, u16;
    if constexpr (RG == 4) {
        // bit 5: rows 0, 1 stay in lanes < 32, rows 2, 3 in lanes >= 32; bit 4: rows 0, 2 in the
        // even 16-lane rows, 1, 3 in the odd ones
        const float g32a = swap_add32(g[0], g[2]), g32b = swap_add32(g[1], g[3]);
        const float u32a = swap_add32(u[0], u[2]), u32b = swap_add32(u[1], u[3]);
        g16 = swap_add16(g32a, g32b);
        u16 = swap_add16(u32a, u32b);
    } else {
        const float g32 = swap_add32(g[0], g[1]), u32 = swap_add32(u[0], u[1]);
        g16 = swap_add16(g32, g32);  // bit 4 of one row: every lane adds lane l ^ 16's value
        u16 = swap_add16(u32, u32);
    }
    gs = butterfly_low4(g16);
    us = butterfly_low4(u16);
}

// Rows [row_base + g*RPI + rsub] of w0 (and w1 with glu), g < RG, for the pairs in ps (pair p
// reads A row p / a_div and writes output row p). The next pair's activations are loaded while
// the current pair is computed.
// FULL: every row of the wave and every chunk of its lanes is in range (no masking).
template <int LPR, int CPL, int RG, bool GLU, bool FULL = false, int B = 4>
__device__ __forceinline__ void gemv_wave(const QW &w0, const QW &w1, int e, int row_base,
                                          const bf16_t *A, int lda, int a_div, PairSet ps,
                                          bf16_t *out, int ldo, int lane) {
    constexpr int RPI = 64 / LPR;
    const int li = lane % LPR, rsub = lane / LPR;
    const int n_ch = w0.in >> 5;
    WRow<CPL, B> r0[RG], r1[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) {
        const int row = row_base + g * RPI + rsub;
        load_wrow<CPL, B>(w0, e, row, li, LPR, r0[g]);
        if (GLU) load_wrow<CPL, B>(w1, e, row, li, LPR, r1[g]);
    }
    int p = ps.next();
    if (p < 0) return;
    XRaw cur[CPL], nxt[CPL];
    load_xrow_raw<CPL>(A + (size_t)(p / a_div) * lda, li, LPR, n_ch, cur);
    while (p >= 0) {
        const int pn = ps.next();
        load_xrow_raw<CPL>(A + (size_t)((pn >= 0 ? pn : p) / a_div) * lda, li, LPR, n_ch, nxt);
        XChunk xc[CPL];
        pair_xrow<CPL, B>(cur, xc);
#pragma unroll
        for (int g = 0; g < RG; ++g) {
            opaque_row(r0[g]);
            if (GLU) opaque_row(r1[g]);
        }
        if constexpr (GLU && LPR == 64 && RG > 1) {
            // the wave's RG gate and up sums by a reduce-scatter: row u's two sums end in lanes
            // [64 u / RG, 64 (u + 1) / RG), and one lane of them evaluates its SwiGLU
            float s0[RG], s1[RG];
#pragma unroll
            for (int g = 0; g < RG; ++g) {
                s0[g] = row_part<CPL, FULL>(r0[g], xc);
                s1[g] = row_part<CPL, FULL>(r1[g], xc);
            }
            float a0, a1;
            rows_reduce_scatter<RG>(s0, s1, a0, a1);
            const int u = lane / (64 / RG), row = row_base + u;
            if (lane % (64 / RG) == 0 && row < w0.out) {
                const float gt = rbf(a0), up = rbf(a1);
                out[(size_t)p * ldo + paired_index_b<B>(row)] = (bf16_t)f2bf((gt * sigmoidf_(gt)) * up);
            }
        } else {
#pragma unroll
            for (int g = 0; g < RG; ++g) {
                const int row = row_base + g * RPI + rsub;
                const float a0 = group_sum<LPR>(row_part<CPL, FULL>(r0[g], xc));
                const float a1 = GLU ? group_sum<LPR>(row_part<CPL, FULL>(r1[g], xc)) : 0.f;
                if (li == 0 && row < w0.out) {
                    float v = a0;
                    if (GLU) {
                        const float gt = rbf(a0), up = rbf(a1);
                        v = (gt * sigmoidf_(gt)) * up;
                    }
                    out[(size_t)p * ldo + paired_index_b<B>(row)] = (bf16_t)f2bf(v);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < CPL; ++c) cur[c] = nxt[c];
        p = pn;
    }
}

// One pair, rows row0 + l * row_step (l < L) of w0 and w1 with GLU: the activation row is loaded
// and re-paired once, and the next rows' weights are loaded before the current rows are computed
// (the last iteration is peeled, so no load sits under a condition). One row per wave (LPR = 64).
template <int CPL>
__device__ __forceinline__ void gemv_wave_stream1(const QW &w0, const QW &w1, int e, int row0,
                                                  int row_step, int L, const bf16_t *arow,
                                                  bf16_t *orow, int lane) {
    const int n_ch = w0.in >> 5;
    XRaw xr[CPL];
    load_xrow_raw<CPL>(arow, lane, 64, n_ch, xr);
    WRow<CPL> c0, c1, n0, n1;
    load_wrow<CPL>(w0, e, row0, lane, 64, c0);
    load_wrow<CPL>(w1, e, row0, lane, 64, c1);
    XChunk xc[CPL];
    pair_xrow<CPL>(xr, xc);
    auto emit = [&](const WRow<CPL> &g, const WRow<CPL> &u, int row) __attribute__((always_inline)) {
        const float a0 = group_sum<64>(row_part(g, xc)), a1 = group_sum<64>(row_part(u, xc));
        if (lane == 0 && row < w0.out) {
            const float gt = rbf(a0), up = rbf(a1);
            orow[paired_index(row)] = (bf16_t)f2bf((gt * sigmoidf_(gt)) * up);
        }
    };
    int row = row0;
    for (int l = 0; l + 1 < L; ++l, row += row_step) {
        load_wrow<CPL>(w0, e, row + row_step, lane, 64, n0);
        load_wrow<CPL>(w1, e, row + row_step, lane, 64, n1);
        opaque_row(c0);
        opaque_row(c1);
        emit(c0, c1, row);
        c0 = n0;
        c1 = n1;
    }
    opaque_row(c0);
    opaque_row(c1);
    emit(c0, c1, row);
}

// Eight bf16 of a raw row through the RMSNorm: R(R(x * inv) * w), w eight bf16 (or ones).
__device__ __forceinline__ uint4 norm8(uint4 x, float inv, uint4 w) {
    const uint32_t xs[4] = {x.x, x.y, x.z, x.w}, ws[4] = {w.x, w.y, w.z, w.w};
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t ww = ws[k];
        const uint32_t lo = f2bf(rbf(bf_lo(xs[k]) * inv) * bf_lo(ww));
        const uint32_t hi = f2bf(rbf(bf_hi(xs[k]) * inv) * bf_hi(ww));
        o[k] = lo | (hi << 16);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// A lane's four 8-element pieces of a 2048-element pass of a row: elements [d + 512 i, +8),
// clamped to the row's last 8 (the clamped pieces are never used).
struct Row4 {
    uint4 v[4];
};
__device__ __forceinline__ Row4 load_row4(const bf16_t *p, int d, int D) {
    Row4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.v[i] = *(const uint4 *)(p + min(d + 512 * i, D - 8));
    return r;
}

// One dense row for T <= 16 tokens (one wave): R(x[t] . w) then R(. + bias). Lane l owns
// elements [8l + 512i, +8); tokens go in groups of 4 whose loads are issued together. `first` is
// the lane's first pass of w (load_row4(w, 8 lane, D)), loaded by the caller as early as it can;
// each later pass of w is loaded before the current one is used.
template <int MAXT>
__device__ __forceinline__ void router_row(const bf16_t *x, int T, int D, const bf16_t *w,
                                           Row4 first, const bf16_t *bias, bf16_t *out, int ldo,
                                           int lane) {
    constexpr int TG = MAXT < 4 ? MAXT : 4;
    float acc[MAXT];
#pragma unroll
    for (int t = 0; t < MAXT; ++t) acc[t] = 0.f;
    const uint32_t braw = bias ? (uint32_t)*bias : 0u;
    Row4 cur = first;
    for (int d = lane * 8; d < D; d += 2048) {
        const Row4 wr = cur;
        if (d + 2048 < D) cur = load_row4(w, d + 2048, D);
        const uint4 *wv = wr.v;
#pragma unroll
        for (int t0 = 0; t0 < MAXT; t0 += TG) {
            if (t0 < T) {
                uint4 xv[TG][4];
#pragma unroll
                for (int tt = 0; tt < TG; ++tt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        xv[tt][i] = *(const uint4 *)(x + (size_t)min(t0 + tt, T - 1) * D +
                                                     min(d + 512 * i, D - 8));
#pragma unroll
                for (int tt = 0; tt < TG; ++tt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (d + 512 * i < D) {
                            float a = acc[t0 + tt];
                            a = dot2(xv[tt][i].x, wv[i].x, a);
                            a = dot2(xv[tt][i].y, wv[i].y, a);
                            a = dot2(xv[tt][i].z, wv[i].z, a);
                            a = dot2(xv[tt][i].w, wv[i].w, a);
                            acc[t0 + tt] = a;
                        }
                    }
            }
        }
    }
#pragma unroll
    for (int t = 0; t < MAXT; ++t) {
        if (t < T) {
            const float v = group_sum<64>(acc[t]);
            if (lane == 0) {
                float l = rbf(v);
                if (bias) l = rbf(l + bf2f(braw));
                out[(size_t)t * ldo] = (bf16_t)f2bf(l);
            }
        }
    }
}

// Dense rows kernel (Linear::forward for T <= 16): one wave per output row.
template <int MAXT>
__global__ __launch_bounds__(256) void rows_kernel(const bf16_t *__restrict__ x, int T, int D,
                                                   const bf16_t *__restrict__ W,
                                                   const bf16_t *__restrict__ bias, int N,
                                                   bf16_t *__restrict__ out) {
    const int lane = threadIdx.x & 63, r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= N) return;
    const bf16_t *w = W + (size_t)r * D;
    router_row<MAXT>(x, T, D, w, load_row4(w, lane * 8, D), bias ? bias + r : nullptr, out + r, N,
                     lane);
}

hipError_t launch_rows(const bf16_t *x, int T, int D, const bf16_t *W, const bf16_t *bias, int N,
                       bf16_t *out, hipStream_t stream) {
    dim3 grid((N + 3) / 4);
    if (T <= 4) rows_kernel<4><<<grid, 256, 0, stream>>>(x, T, D, W, bias, N, out);
    else rows_kernel<16><<<grid, 256, 0, stream>>>(x, T, D, W, bias, N, out);
    return hipGetLastError();
}

// One quantized Linear row (4 or 8 bits, expert 0 of w; groups of 32 to 128) for T <= 16 tokens:
// R(x[t] . w) then R(. + bias), the weight dequantized as q s + b in f32 (Quantized::dequantize,
// nuvec.rs:1173-1204) and dotted in f32. Lane l owns the 8-element chunks [8l + 512i, +8) of each
// 2048-wide pass (a chunk lies in one group); all of a pass's loads are issued before any is used.
template <int MAXT>
__device__ __forceinline__ void qrouter_row(const bf16_t *x, int T, int D, const QW w, int row,
                                            const bf16_t *bias, bf16_t *out, int ldo, int lane) {
    float acc[MAXT];
#pragma unroll
    for (int t = 0; t < MAXT; ++t) acc[t] = 0.f;
    // group sizes are powers of two (32, 64 or 128): a shift, not a division per chunk
    const int gshift = __builtin_ctz((unsigned)w.group);
    const int groups = D >> gshift, wpr = D * w.bits / 32;  // code words per row
    const uint32_t *codes = w.codes + (size_t)row * wpr;
    const bf16_t *sc = w.scales + (size_t)row * groups;
    const bf16_t *bi = w.biases ? w.biases + (size_t)row * groups : nullptr;
    for (int d0 = lane * 8; d0 < D; d0 += 2048) {
        uint2 cw[4];
        uint32_t sraw[4], braw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = min(d0 + 512 * i, D - 8);  // clamped; chunks past D are not used
            if (w.bits == 8) cw[i] = *(const uint2 *)(codes + d / 4);
            else cw[i] = make_uint2(codes[d / 8], 0u);
            sraw[i] = sc[d >> gshift];
            braw[i] = bi ? bi[d >> gshift] : 0u;
        }
        float wv[4][8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float s = bf2f(sraw[i]), b = bf2f(braw[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t q = w.bits == 8 ? ((e < 4 ? cw[i].x : cw[i].y) >> (8 * (e & 3))) & 0xFFu
                                               : (cw[i].x >> (4 * e)) & 0xFu;
                wv[i][e] = __builtin_fmaf((float)q, s, b);
            }
        }
        // tokens in groups of 4 whose activation loads are issued together (one at a time made
        // every token a round trip: T = 16 took 11 us longer than the dense router)
        constexpr int TG = MAXT < 4 ? MAXT : 4;
#pragma unroll
        for (int t0 = 0; t0 < MAXT; t0 += TG) {
            if (t0 < T) {
                uint4 xv[TG][4];
#pragma unroll
                for (int tt = 0; tt < TG; ++tt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        xv[tt][i] = *(const uint4 *)(x + (size_t)min(t0 + tt, T - 1) * D +
                                                     min(d0 + 512 * i, D - 8));
#pragma unroll
                for (int tt = 0; tt < TG; ++tt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if (d0 + 512 * i < D) {
                            float xf[8];
                            unpack8(xv[tt][i], xf);
                            float a = acc[t0 + tt];
#pragma unroll
                            for (int e = 0; e < 8; ++e) a = __builtin_fmaf(xf[e], wv[i][e], a);
                            acc[t0 + tt] = a;
                        }
                    }
            }
        }
    }
    const uint32_t braw = bias ? (uint32_t)*bias : 0u;
#pragma unroll
    for (int t = 0; t < MAXT; ++t) {
        if (t < T) {
            const float v = group_sum<64>(acc[t]);
            if (lane == 0) {
                float l = rbf(v);
                if (bias) l = rbf(l + bf2f(braw));
                out[(size_t)t * ldo] = (bf16_t)f2bf(l);
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// K1: router logits + the shared expert's gate logit

// QUANT: some rows are quantized (a separate instantiation, so the dense-router kernel keeps its
// registers and schedule). Four rows per workgroup, one per wave; TSPLIT waves (T > 2, no fused
// norm; 4 up to 16 tokens, 8 up to 32):
// one row per workgroup, and wave w takes tokens [4w, 4w + 4) of it.
template <int MAXT, bool NORM, bool QUANT, int TSPLIT = 0>
__global__ __launch_bounds__(TSPLIT > 4 ? 512 : 256) void decode_router_kernel(DecodeJob j) {
    // the wave index in a scalar register: the row, its weights and the branches below are the
    // wave's own (per-lane values would make every field of a quantized row a per-lane load)
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = TSPLIT ? (int)blockIdx.x : (int)blockIdx.x * 4 + wave;
    const int D = j.D;
    const bf16_t *w = nullptr, *bias = nullptr;
    bool quant = false;  // a quantized row instead (row qr of qw)
    QW qw{};
    int qr = 0;
    bf16_t *out = nullptr;
    int ldo = 1;
    if (r < j.E) {
        if (!QUANT || j.router) w = j.router + (size_t)r * D;
        else quant = true, qw = j.router_q, qr = r;
        out = j.logits + r, ldo = j.E;
        bias = j.router_bias ? j.router_bias + r : nullptr;
    } else if (r == j.E && j.S) {
        if (!QUANT || j.sh_gate_w) w = j.sh_gate_w;
        else quant = true, qw = j.sh_gate_q;
        bias = j.sh_gate_b, out = j.sh_logit;
    }
    // the weight row's first pass is loaded before anything waits (the norm below, in particular)
    Row4 first{};
    if (w) first = load_row4(w, lane * 8, D);
    const bf16_t *x = j.x;
    if (NORM) {
        // fused RMSNorm: the workgroup normalises the T rows of norm_src into LDS (wave v takes
        // rows v, v + 4, ...; row_rms_inv's order and rounding, so the bits of the norm kernel), and
        // workgroup 0 also writes them to j.x for K2. A row of D <= 2048 is read once.
        extern __shared__ __align__(16) bf16_t hs[];
        const uint4 ones = make_uint4(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);
        for (int t = wave; t < j.T; t += 4) {
            const bf16_t *src = j.norm_src + (size_t)t * D;
            bf16_t *hrow = &hs[(size_t)t * D], *grow = (bf16_t *)j.x + (size_t)t * D;
            if (D <= 2048) {
                const Row4 xv = load_row4(src, lane * 8, D);
                const Row4 nv = j.norm_w ? load_row4(j.norm_w, lane * 8, D) : Row4{{ones, ones, ones, ones}};
                float ss = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (lane * 8 + 512 * i < D) {
                        float f[8];
                        unpack8(xv.v[i], f);
                        ss = sumsq8(f, ss);
                    }
                const float inv = rms_inv_of(group_sum<64>(ss), D, j.eps);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int d = lane * 8 + 512 * i;
                    if (d < D) {
                        const uint4 h = norm8(xv.v[i], inv, nv.v[i]);
                        *(uint4 *)(hrow + d) = h;
                        if (blockIdx.x == 0) *(uint4 *)(grow + d) = h;
                    }
                }
            } else {
                const float inv = row_rms_inv(src, nullptr, D, j.eps, lane);
                for (int d = lane * 8; d < D; d += 512) {
                    const uint4 nv = j.norm_w ? *(const uint4 *)(j.norm_w + d) : ones;
                    const uint4 h = norm8(*(const uint4 *)(src + d), inv, nv);
                    *(uint4 *)(hrow + d) = h;
                    if (blockIdx.x == 0) *(uint4 *)(grow + d) = h;
                }
            }
        }
        __syncthreads();
        x = hs;
    }
    if (TSPLIT) {
        const int tb = wave * 4;
        if (tb >= j.T) return;
        const int tn = min(4, j.T - tb);
        x += (size_t)tb * D;
        if (out) out += (size_t)tb * ldo;
        if (w) router_row<4>(x, tn, D, w, first, bias, out, ldo, lane);
        else if (QUANT && quant) qrouter_row<4>(x, tn, D, qw, qr, bias, out, ldo, lane);
        return;
    }
    if (w) router_row<MAXT>(x, j.T, D, w, first, bias, out, ldo, lane);
    else if (QUANT && quant) qrouter_row<MAXT>(x, j.T, D, qw, qr, bias, out, ldo, lane);
}

// ---------------------------------------------------------------------------------------------
// shared by K2 and K3: the top-k of every token into LDS, and the active-expert mask

template <int NW, bool MASK = true>
__device__ __forceinline__ void all_topk(const DecodeJob &j, bool compute, uint32_t *sid,
                                         bf16_t *ssc, uint32_t *mask) {
    // token t goes to wave (t + blockIdx.x) % NW: the workgroups sharing a CU spread their top-k
    // over its four SIMDs
    const int wave = (int)((threadIdx.x >> 6) + NW - (blockIdx.x & 3)) % NW;
    if (threadIdx.x < 16) mask[threadIdx.x] = 0;
    if (compute) {
        for (int t = wave; t < j.T; t += NW)
            topk_token(j.logits + (size_t)t * j.E, j.E, j.k, j.norm != 0, nullptr, sid + t * j.k,
                       ssc + t * j.k);
    } else {
        const int P = j.T * j.k;
        if ((int)threadIdx.x < P) {
            sid[threadIdx.x] = j.ids[threadIdx.x];
            ssc[threadIdx.x] = j.scores[threadIdx.x];
        }
    }
    __syncthreads();
    if (!MASK) return;
    for (int p = threadIdx.x; p < j.T * j.k; p += 64 * NW) atomicOr(&mask[sid[p] >> 5], 1u << (sid[p] & 31));
    __syncthreads();
}

// The slot-th set bit of the expert mask (words mask[0..nw), nw <= 16), i.e. the slot-th active
// expert in ascending order, or -1 past the last; one wave, all words at once: lane l holds word l
// and the inclusive count of set bits up to it (a scan over the 16 lanes of DPP row 0), the word
// is the number of words whose count is <= slot, and the bit within it is found by halving.
__device__ __forceinline__ int slot_expert(const uint32_t *mask, int nw, int slot, int lane) {
    const uint32_t mw = mask[lane & 15];
    const int cnt = lane < nw ? __popc(mw) : 0;
    int inc = cnt;
    inc += __builtin_amdgcn_mov_dpp(inc, 0x111, 0xF, 0xF, true);  // row_shr:1 (0 past the row)
    inc += __builtin_amdgcn_mov_dpp(inc, 0x112, 0xF, 0xF, true);  // row_shr:2
    inc += __builtin_amdgcn_mov_dpp(inc, 0x114, 0xF, 0xF, true);  // row_shr:4
    inc += __builtin_amdgcn_mov_dpp(inc, 0x118, 0xF, 0xF, true);  // row_shr:8
    const int w = __popcll(__ballot(lane < nw && inc <= slot));
    if (w >= nw) return -1;
    uint32_t m = mw;
    int r = slot - (inc - cnt), pos = 0;  // rank of the bit within this lane's word
#pragma unroll
    for (int h = 16; h >= 1; h >>= 1) {
        const int c = __popc(m & ((1u << h) - 1u));
        const bool up = r >= c;
        r = up ? r - c : r;
        m = up ? m >> h : m;
        pos = up ? pos + h : pos;
    }
    const int bit = __builtin_amdgcn_readlane(pos, w);
    // the bit is set by construction; checked so that an index past the experts cannot come out
    const uint32_t word = (uint32_t)__builtin_amdgcn_readlane((int)mw, w);
    return ((word >> bit) & 1u) ? w * 32 + bit : -1;
}

// Pairs choosing expert e (one wave, from LDS).
__device__ __forceinline__ PairSet pairs_of(const uint32_t *sid, int P, int e, int lane) {
    PairSet ps;
    ps.m0 = __ballot(lane < P && (int)sid[lane] == e);
    ps.m1 = __ballot(lane + 64 < P && (int)sid[lane + 64] == e);
    ps.m2 = ps.m3 = 0;
    if (P > 128) {  // uniform: batches of more than 16 tokens
        ps.m2 = __ballot(lane + 128 < P && (int)sid[lane + 128] == e);
        ps.m3 = __ballot(lane + 192 < P && (int)sid[lane + 192] == e);
    }
    return ps;
}

// ---------------------------------------------------------------------------------------------
// K2: shared + routed gate/up

// K2 workgroups: NW waves x RG rows of one projection pair each, up to 4 tokens for the shared
// expert, for gu_loop consecutive row blocks in turn (a routed workgroup derives the routing once
// for all of them). Few rows per wave keep several waves per SIMD, so their dependent reductions
// overlap; the loop keeps the workgroup count near one resident round for wide experts.
__host__ __device__ inline int shared_gateup_blocks(const DecodeJob &j, int rows) {
    return j.S ? (j.S / rows) * ((j.T + 3) / 4) : 0;
}

// (the streaming kernel with 3 chunks per lane is held to 168 registers, 3 waves per SIMD: at 171
// it ran 2, and T = 1 took 4 us longer on the Coder shape)
// FULL: D is exactly LPR * CPL chunks of 32 (rows are whole by construction: I and S are
// multiples of the rows per workgroup).
template <int LPR, int CPL, int RG, int NW, bool LOOP, bool SH_LAST, bool FULL = false, int B = 4>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(LOOP && CPL == 3 ? 3 : 1))) void decode_gateup_kernel(
    DecodeJob j) {
    __shared__ uint32_t sid[kMaxP], mask[16];
    __shared__ bf16_t ssc[kMaxP];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int RPI = 64 / LPR;
    const int L = LOOP ? j.gu_loop : 1;
    const int n_sh = shared_gateup_blocks(j, NW * RG * RPI * L);
    // one gemv_wave call for both kinds of workgroup (its code is large): pick its operands
    // Workgroup order. A CU hosts two or three K2 workgroups (i, i + #CUs, ...), and its later ones
    // run slower. SH_LAST (T <= 2) puts the routed workgroups first, so that the shared ones (no
    // routing to wait for, done early) take the CUs' third places; above, where the shared
    // expert's share is larger, they go first.
    const int n_ro = (int)gridDim.x - n_sh;
    const bool sh = SH_LAST ? (int)blockIdx.x >= n_ro : (int)blockIdx.x < n_sh;
    const int bid = !SH_LAST ? (int)blockIdx.x : sh ? (int)blockIdx.x - n_ro : (int)blockIdx.x + n_sh;
    auto pick = [&](const QW &a, const QW &b) {  // field by field: no copy of the arguments
        QW q;
        q.codes = sh ? a.codes : b.codes;
        q.scales = sh ? a.scales : b.scales;
        q.biases = sh ? a.biases : b.biases;
        q.experts = sh ? a.experts : b.experts;
        q.out = sh ? a.out : b.out;
        q.in = sh ? a.in : b.in;
        q.group = sh ? a.group : b.group;
        q.bits = sh ? a.bits : b.bits;
        return q;
    };
    // benchmark instrumentation (j.clock set): the device wall clock at each workgroup's start and
    // at each wave's end, whichever way the wave leaves, folded into pair blockIdx % 64 of the 64
    // (start min, end max) pairs (one address for every workgroup serialises its atomics)
    unsigned long long *const clk = j.clock ? j.clock + 2 * (blockIdx.x & 63) : nullptr;
    struct ClockEnd {
        unsigned long long *c;
        __device__ ~ClockEnd() {
            if (c && (threadIdx.x & 63) == 0) atomicMax(c + 1, __builtin_amdgcn_s_memrealtime());
        }
    } clock_end{clk};
    if (clk && threadIdx.x == 0) atomicMin(clk, __builtin_amdgcn_s_memrealtime());
    const QW w0 = pick(j.sg, j.wg), w1 = pick(j.su, j.wu);
    int e = 0, rb, a_div, ldo;
    PairSet ps{};
    bf16_t *out;
    if (sh) {  // shared expert gate/up: 4 * RG * RPI rows x up to 4 tokens
        const int n_row_blocks = j.S / (NW * RG * RPI * L);
        rb = bid % n_row_blocks;
        const int t0 = (bid / n_row_blocks) * 4;
        const int tn = min(4, j.T - t0);
        a_div = 1, ldo = j.S, out = j.sh_act;
        ps.m0 = ((1ull << tn) - 1) << t0;  // t0 + tn <= T <= 32
    } else {
        const int r = bid - n_sh, row_blocks = j.I / (NW * RG * RPI * L);
        const int slot = r / row_blocks;
        rb = r % row_blocks;
        // one token (the T = 1 decode): its k experts are distinct, so slot s takes the s-th ranked
        // one, pair s; no expert mask and no search of it on the way to the expert rows
        const bool one = j.T == 1 && j.topk_in_kernel;
        if (one) all_topk<NW, false>(j, true, sid, ssc, mask);
        else all_topk<NW>(j, j.topk_in_kernel != 0, sid, ssc, mask);
        if (r == 0 && j.topk_in_kernel) {  // publish the routing for K3
            const int P = j.T * j.k;
            if ((int)threadIdx.x < P) {
                j.ids[threadIdx.x] = sid[threadIdx.x];
                j.scores[threadIdx.x] = ssc[threadIdx.x];
            }
        }
        if (one) {
            if (slot >= j.k) return;
            e = __builtin_amdgcn_readfirstlane((int)sid[slot]);
            ps.m0 = 1ull << slot;
        } else {
            e = slot_expert(mask, (j.E + 31) / 32, slot, lane);
            if (e < 0) return;
            ps = pairs_of(sid, j.T * j.k, e, lane);
        }
        a_div = j.k, ldo = j.I, out = j.act;
    }
    if (LOOP) {  // RG = 1, LPR = 64: rows rb * L * NW + wave + NW * l, pair by pair
        static_assert(!LOOP || (RG == 1 && LPR == 64), "the streaming loop takes one row per wave");
        // (two pairs' activations held at a time measured slower: 256 registers, one wave per SIMD)
        for (;;) {
            const int p = ps.next();
            if (p < 0) break;
            // opaque, so nothing of one pair's pass (row addresses) is held over for the next
            int row0 = rb * L * NW + wave;
            asm volatile("" : "+v"(row0));
            gemv_wave_stream1<CPL>(w0, w1, e, row0, NW, L, j.x + (size_t)(p / a_div) * j.D,
                                   out + (size_t)p * ldo, lane);
        }
    } else {
        gemv_wave<LPR, CPL, RG, true, FULL, B>(w0, w1, e, (rb * NW + wave) * RG * RPI, j.x, j.D,
                                               a_div, ps, out, ldo, lane);
    }
}

// ---------------------------------------------------------------------------------------------
// K3: down + combine

template <int LPR, int CPL, int SLPR, int SCPL, int PB, int kDownRowsPerWG, int B = 4>
__global__ __launch_bounds__(256) void decode_down_kernel(DecodeJob j) {
    constexpr int RPI = 64 / LPR, NRG = kDownRowsPerWG / RPI;
    constexpr int SRPI = 64 / SLPR, SNRG = kDownRowsPerWG / SRPI, SG = (SNRG + 3) / 4;
    __shared__ uint32_t sid[kMaxP];
    __shared__ bf16_t ssc[kMaxP];
    __shared__ float yv[kMaxP][kDownRowsPerWG];
    __shared__ float ysh[kMaxT][kDownRowsPerWG];
    __shared__ bf16_t shl[kMaxT];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // workgroup = (token group, row block); the token group's pairs are a contiguous range, and a
    // token's combine needs only its own pairs
    const int n_rb = j.D / kDownRowsPerWG;
    const int d0 = (blockIdx.x % n_rb) * kDownRowsPerWG;
    const int t0 = (blockIdx.x / n_rb) * j.down_tokens, t1 = min(j.T, t0 + j.down_tokens);

    // the routing is loaded first (loads complete in issue order), then what does not depend on
    // it: the shared expert's rows and first activation row, the shared gate logits, this wave's
    // first activation rows
    const int P = j.T * j.k;
    const uint32_t my_id = j.ids[min((int)threadIdx.x, P - 1)];
    const uint32_t my_sc = j.scores[min((int)threadIdx.x, P - 1)];
    WRow<SCPL, B> sr[SG];
    const int sli = lane % SLPR;
    XRaw scur[SCPL];
    {
        // unconditional: without a shared expert the routed down weights and activations stand in
        // (never used), so no load sits under a condition
        const bool has_s = j.S != 0;
        QW sd;
        sd.codes = has_s ? j.sd.codes : j.wd.codes;
        sd.scales = has_s ? j.sd.scales : j.wd.scales;
        sd.biases = has_s ? j.sd.biases : j.wd.biases;
        sd.experts = has_s ? j.sd.experts : j.wd.experts;
        sd.out = has_s ? j.sd.out : j.wd.out;
        sd.in = has_s ? j.sd.in : j.wd.in;
        sd.group = has_s ? j.sd.group : j.wd.group;
        sd.bits = has_s ? j.sd.bits : j.wd.bits;
#pragma unroll
        for (int i = 0; i < SG; ++i) {
            const int g = wave + 4 * i;
            load_wrow<SCPL, B>(sd, 0, g < SNRG ? d0 + g * SRPI + lane / SLPR : j.D, sli, SLPR, sr[i]);
        }
        load_xrow_raw<SCPL>(has_s ? j.sh_act + (size_t)t0 * j.S : j.act, sli, SLPR,
                            (has_s ? j.S : j.I) >> 5, scur);
    }
    // clamped indices and unconditional LDS writes (threads past the end repeat the last value):
    // a load used under a condition would make the wait there cover every load issued before
    const bf16_t *shl_src = j.S ? j.sh_logit : j.scores;  // any valid pointer without a shared expert
    const uint32_t my_shl = shl_src[min((int)threadIdx.x, j.T - 1)];
    const int li = lane % LPR, rsub = lane / LPR;
    const int per_wave = ((t1 - t0) * j.k + 3) / 4;
    const int p_lo = t0 * j.k + wave * per_wave, p_hi = min(t1 * j.k, p_lo + per_wave);
    XRaw xr[PB][CPL];
    auto load_act = [&](int pb) {  // rows clamped into [0, P): also a wave without pairs loads
#pragma unroll
        for (int b = 0; b < PB; ++b)
            load_xrow_raw<CPL>(j.act + (size_t)max(0, min(pb + b, p_hi - 1)) * j.I, li, LPR,
                               j.I >> 5, xr[b]);
    };
    load_act(p_lo);
    sid[min((int)threadIdx.x, P - 1)] = my_id;
    ssc[min((int)threadIdx.x, P - 1)] = (bf16_t)my_sc;
    // LDS only: the loads above stay in flight, so the routed weight rows (which need sid) are
    // issued as soon as the routing has arrived, not after the activations and shared rows
    lds_barrier();

    // work: for each pair p (expert sid[p]) its NRG row groups of this workgroup's rows; a wave
    // takes PB pairs at a time and issues all their loads before computing
    for (int pb = p_lo; pb < p_hi; pb += PB) {
        if (pb != p_lo) load_act(pb);
        WRow<CPL, B> wr[PB][NRG];
#pragma unroll
        for (int b = 0; b < PB; ++b) {
            const int e = (int)sid[min(pb + b, p_hi - 1)];
#pragma unroll
            for (int g = 0; g < NRG; ++g)
                load_wrow<CPL, B>(j.wd, e, d0 + g * RPI + rsub, li, LPR, wr[b][g]);
        }
#pragma unroll
        for (int b = 0; b < PB; ++b) {
            const int p = pb + b;
            if (p >= p_hi) break;
            XChunk xc[CPL];
            chunks_of_paired<CPL>(xr[b], xc);
#pragma unroll
            for (int g = 0; g < NRG; ++g) {
                const float y = group_sum<LPR>(row_part(wr[b][g], xc));
                if (li == 0) yv[p][g * RPI + rsub] = rbf(y);
            }
        }
    }
    if (j.S) {
        XRaw nxt[SCPL];
        for (int t = t0; t < t1; ++t) {
            load_xrow_raw<SCPL>(j.sh_act + (size_t)min(t + 1, t1 - 1) * j.S, sli, SLPR, j.S >> 5,
                                nxt);
            XChunk xc[SCPL];
            chunks_of_paired<SCPL>(scur, xc);
#pragma unroll
            for (int c = 0; c < SCPL; ++c) scur[c] = nxt[c];
#pragma unroll
            for (int i = 0; i < SG; ++i) {
                const int g = wave + 4 * i;
                opaque_row(sr[i]);
                const float y = group_sum<SLPR>(row_part(sr[i], xc));
                if (g < SNRG && sli == 0) ysh[t][g * SRPI + lane / SLPR] = rbf(y);
            }
        }
    }
    shl[min((int)threadIdx.x, kMaxT - 1)] = (bf16_t)my_shl;
    __syncthreads();
    for (int i = threadIdx.x; i < (t1 - t0) * kDownRowsPerWG; i += 256) {
        const int t = t0 + i / kDownRowsPerWG, dd = i % kDownRowsPerWG;
        float acc = 0.f;
        for (int jj = 0; jj < j.k; ++jj) {
            const int p = t * j.k + jj;
            acc += rbf(yv[p][dd] * bf2f(ssc[p]));
        }
        float r = rbf(acc);
        if (j.S) {
            const float sg = rbf(sigmoidf_(bf2f(shl[t])));
            r = rbf(r + rbf(sg * ysh[t][dd]));
        }
        bf16_t *o = j.out + (size_t)t * j.D + d0 + dd;
        if (j.residual) r = rbf(bf2f(j.residual[(size_t)t * j.D + d0 + dd]) + r);  // R(x + MoE(h))
        *o = (bf16_t)f2bf(r);
    }
}

// K3 without a shared expert and down rows of more than 2048 inputs: wave w takes pairs w, w + 8,
// ... (each pair's expert's down rows for the workgroup's drs output rows): it loads and pairs the
// pair's activation row once and streams the rows in batches of RB, the next batch loaded before
// the current one is computed; then the combine of the workgroup's rows for every token from
// LDS. Each row's dot and every rounding are those of decode_down_kernel with LPR = 64 (the same
// bits).
constexpr int kStreamMaxRows = 32, kStreamBatch = 2;

template <int CPL, int RB>
__global__ __launch_bounds__(512) void decode_down_stream_kernel(DecodeJob j, int drs) {
    __shared__ float yv[kMaxP][kStreamMaxRows];
    __shared__ bf16_t ssc[kMaxP];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int P = j.T * j.k;
    const int d0 = blockIdx.x * drs;
    for (int p = wave; p < P; p += 8) {
        const int e = (int)j.ids[p];
        XRaw xr[CPL];
        load_xrow_raw<CPL>(j.act + (size_t)p * j.I, lane, 64, j.I >> 5, xr);
        WRow<CPL> cur[RB], nxt[RB];
#pragma unroll
        for (int b = 0; b < RB; ++b) load_wrow<CPL>(j.wd, e, d0 + b, lane, 64, cur[b]);
        const uint32_t sc = j.scores[p];
        XChunk xc[CPL];
        chunks_of_paired<CPL>(xr, xc);
        auto emit = [&](int r) __attribute__((always_inline)) {
#pragma unroll
            for (int b = 0; b < RB; ++b) opaque_row(cur[b]);
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                const float y = group_sum<64>(row_part(cur[b], xc));
                if (lane == 0) yv[p][r + b] = rbf(y);
            }
        };
        int r = 0;
        for (; r + RB < drs; r += RB) {
#pragma unroll
            for (int b = 0; b < RB; ++b) load_wrow<CPL>(j.wd, e, d0 + r + RB + b, lane, 64, nxt[b]);
            emit(r);
#pragma unroll
            for (int b = 0; b < RB; ++b) cur[b] = nxt[b];
        }
        emit(r);
        if (lane == 0) ssc[p] = (bf16_t)sc;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < j.T * drs; i += blockDim.x) {
        const int t = i / drs, dd = i % drs;
        float acc = 0.f;
        for (int jj = 0; jj < j.k; ++jj) {
            const int p = t * j.k + jj;
            acc += rbf(yv[p][dd] * bf2f(ssc[p]));
        }
        float r = rbf(acc);
        const size_t o = (size_t)t * j.D + d0 + dd;
        if (j.residual) r = rbf(bf2f(j.residual[o]) + r);  // R(x + MoE(h))
        j.out[o] = (bf16_t)f2bf(r);
    }
}

// whether the streaming K3 takes the job: rows per workgroup D / 512 (two workgroups per CU), a
// multiple of the batch of 2 rows (measured against D / 256 and batches of 4 or 8: 24.9 against
// 26.5 to 28.6 us on the Coder shape)
static int stream_k3_rows(const DecodeJob &j) {
    const int ich = j.I >> 5;
    // (at most 3 chunks of 32 per lane: 4 would spill)
    if (j.S != 0 || ich <= 64 || ich > 192 || j.D % 512 != 0) return 0;
    const int drs = j.D / 512;
    return (drs % kStreamBatch == 0 && drs <= kStreamMaxRows) ? drs : 0;
}

// ---------------------------------------------------------------------------------------------

template <int MAXT>
static void launch_k1(const DecodeJob &j, hipStream_t s) {
    dim3 grid((j.E + (j.S ? 1 : 0) + 3) / 4);
    const size_t lds = j.norm_src ? 2 * (size_t)j.T * j.D : 0;
    if (j.T > 2 && !j.norm_src) {
        // one row per workgroup from T = 3, a wave per 4 tokens: every wave reads its tokens'
        // activation rows, so spreading the rows over all CUs spreads those reads, and splitting
        // the tokens over waves issues them at once (one row per single-wave workgroup: T = 16
        // 66.75 -> 65.5 us per block, T = 8 40.8 -> 40.1, T = 4 26.35 -> 25.85; at T = 1 and 2,
        // where the rows are one or two reads, four rows per workgroup stay faster: 14.1 -> 14.6
        // and 18.3 -> 18.6)
        dim3 g1(j.E + (j.S ? 1 : 0));
        const int nt = 64 * ((j.T + 3) / 4);
        const bool q = !j.router || (j.S && !j.sh_gate_w);
        if (j.T > 16) {
            if (q) decode_router_kernel<4, false, true, 8><<<g1, nt, 0, s>>>(j);
            else decode_router_kernel<4, false, false, 8><<<g1, nt, 0, s>>>(j);
        } else if (q) {
            decode_router_kernel<4, false, true, 4><<<g1, nt, 0, s>>>(j);
        } else {
            decode_router_kernel<4, false, false, 4><<<g1, nt, 0, s>>>(j);
        }
        return;
    }
    if (!j.router || (j.S && !j.sh_gate_w)) {  // a quantized router or shared gate
        if (j.norm_src) decode_router_kernel<MAXT, true, true><<<grid, 256, lds, s>>>(j);
        else decode_router_kernel<MAXT, false, true><<<grid, 256, 0, s>>>(j);
    } else if (j.norm_src) {
        decode_router_kernel<MAXT, true, false><<<grid, 256, lds, s>>>(j);
    } else {
        decode_router_kernel<MAXT, false, false><<<grid, 256, 0, s>>>(j);
    }
}

template <int LPR, int CPL, int PB, int DR, int B>
static void launch_k3_pb(const DecodeJob &j, hipStream_t s);

// K3 token groups: from T = 2 the tokens are split into groups, each with its own workgroups for
// every row block (more workgroups, fewer pairs each, so each wave's chain of pair batches is
// shorter). The split keeps every row's bits. Two groups: T = 16 71.7 -> 66.7 us per block,
// T = 4 28.3 -> 27.5, T = 2 18.8 -> 18.5. From T = 8 four groups with one pair per load batch
// (fewer registers, so more waves per SIMD hide the batches' round trips): T = 16 63.15 -> 59.2,
// T = 8 39.4 -> 38.8 (four groups with batches of 4 at T = 16: 68.4; eight groups: 60.4; one
// pair per batch at T = 4: 25.55 -> 25.85).
static int k3_token_groups(int T) { return T >= 8 ? 4 : (T >= 2 ? 2 : 1); }

// K2 with RG rows per wave and NW waves per workgroup (I and S multiples of NW * RG). With rows
// wider than 2048 (one row per wave), each workgroup streams gu_loop row blocks, the smallest
// power of two that keeps the routed workgroups at 1024 per token or fewer (I and S multiples of
// NW * RG * gu_loop): a workgroup per row block derived the routing once per block, ran in several
// rounds and had one block's loads in flight at a time. (On the 6144 x 2560 Coder shape this is 8
// row blocks at T = 1 to 16; caps of 512, 2048 and 4096 per token measured slower.) Narrower rows
// (one round already) take one row block per workgroup (the loop measured slower there).
template <int RG, int NW, bool LOOP, int B>
static void launch_k2_l(const DecodeJob &j, int n_ch, dim3 g2, hipStream_t s) {
    auto go1 = [&](auto kernel) { kernel<<<g2, 64 * NW, 0, s>>>(j); };
    // the shared expert's workgroups last at T <= 2 (T = 1: 14.9 -> 14.2 us per block, T = 2:
    // 20.8 -> 19.3), first above (last measured 4 and 7 us slower at T = 4 and 16)
    auto go = [&](auto first, auto last) {
        if (j.T <= 2) go1(last);
        else go1(first);
    };
    // whole rows of 2048 from T = 2: the unmasked row math (T = 16 59.3 -> 58.15 us per block,
    // T = 4 25.75 -> 25.55, T = 2 18.15 -> 18.0; at T = 1 within the noise)
    if constexpr (B == 8) {  // 8-bit experts: rows of at most 2048 (one chunk per lane)
        if (n_ch == 64 && (RG == 4 || j.T == 2)) go(decode_gateup_kernel<64, 1, RG, NW, false, false, true, 8>, decode_gateup_kernel<64, 1, RG, NW, false, true, true, 8>);
        else go(decode_gateup_kernel<64, 1, RG, NW, false, false, false, 8>, decode_gateup_kernel<64, 1, RG, NW, false, true, false, 8>);
        return;
    }
    if (n_ch == 64 && !LOOP && (RG == 4 || j.T == 2)) go(decode_gateup_kernel<64, 1, RG, NW, false, false, true>, decode_gateup_kernel<64, 1, RG, NW, false, true, true>);
    else if (n_ch <= 64) go(decode_gateup_kernel<64, 1, RG, NW, LOOP, false>, decode_gateup_kernel<64, 1, RG, NW, LOOP, true>);
    else if (n_ch <= 128) go(decode_gateup_kernel<64, 2, RG, NW, LOOP, false>, decode_gateup_kernel<64, 2, RG, NW, LOOP, true>);
    else if (n_ch <= 192) go(decode_gateup_kernel<64, 3, RG, NW, LOOP, false>, decode_gateup_kernel<64, 3, RG, NW, LOOP, true>);
    else go(decode_gateup_kernel<64, 4, RG, NW, LOOP, false>, decode_gateup_kernel<64, 4, RG, NW, LOOP, true>);
}

template <int RG, int NW, int B>
static void launch_k2(DecodeJob j, int n_ch, hipStream_t s) {
    const int per_slot = j.I / (NW * RG), sh_blocks = j.S / (NW * RG);
    int L = 1;
    while (RG == 1 && n_ch > 64 && j.max_slots * per_slot / L > 1024 * j.T &&
           per_slot % (2 * L) == 0 && sh_blocks % (2 * L) == 0)
        L *= 2;
    j.gu_loop = L;
    dim3 g2(shared_gateup_blocks(j, NW * RG * L) + (j.I / (NW * RG * L)) * j.max_slots);
    if (RG == 1 && L > 1) launch_k2_l<1, NW, true, B>(j, n_ch, g2, s);
    else launch_k2_l<RG, NW, false, B>(j, n_ch, g2, s);
}

template <int LPR, int CPL, int B>
static void launch_k3_s(DecodeJob j, hipStream_t s) {
    j.down_tokens = (j.T + k3_token_groups(j.T) - 1) / k3_token_groups(j.T);
    // output rows per workgroup: two row groups per wave, at least 4 rows (8 with 16-lane rows,
    // where 4, 16 and 32 measured slower: T = 1 18.3, 18.1, 20.7 against 17.4 us per block; fewer
    // workgroups re-read the pairs' activation rows fewer times, until each wave's chain of pair
    // batches grows too long). Pairs per load batch keep a batch's activations and weight rows
    // within ~128 registers; batches of 4 only for waves of more than 8 pairs (a wave takes a
    // quarter of its group's pairs): with 2 to 8 pairs a wave, batches of 2 measured faster
    // (T = 4, 4 pairs a wave: 27.1 -> 26.75 us per block) and no slower at T = 1 and 8
    constexpr int DR = 2 * (64 / LPR) > 4 ? 2 * (64 / LPR) : 4;
    constexpr int NRG = DR / (64 / LPR) > 0 ? DR / (64 / LPR) : 1;
    constexpr int PB = (NRG * CPL <= 2) ? 4 : (NRG * CPL <= 4 ? 2 : 1);
    if (j.T >= 8) launch_k3_pb<LPR, CPL, 1, DR, B>(j, s);
    else if (PB == 4 && (j.down_tokens * j.k + 3) / 4 <= 8) launch_k3_pb<LPR, CPL, 2, DR, B>(j, s);
    else launch_k3_pb<LPR, CPL, PB, DR, B>(j, s);
}

template <int LPR, int CPL, int PB, int DR, int B>
static void launch_k3_pb(const DecodeJob &j, hipStream_t s) {
    dim3 grid(j.D / DR * ((j.T + j.down_tokens - 1) / j.down_tokens));
    const int sch = j.S ? j.S >> 5 : 16;
    if (sch == 16) decode_down_kernel<LPR, CPL, 16, 1, PB, DR, B><<<grid, 256, 0, s>>>(j);
    else if (sch < 64) decode_down_kernel<LPR, CPL, 32, 2, PB, DR, B><<<grid, 256, 0, s>>>(j);
    else if (sch <= 64 || B == 8) decode_down_kernel<LPR, CPL, 64, 1, PB, DR, B><<<grid, 256, 0, s>>>(j);
    else if (sch <= 128) decode_down_kernel<LPR, CPL, 64, 2, PB, DR, B><<<grid, 256, 0, s>>>(j);
    else decode_down_kernel<LPR, CPL, 64, 4, PB, DR, B><<<grid, 256, 0, s>>>(j);
}

// 8-bit experts take the same kernels with rows of at most 2048 inputs (one chunk of codes per
// lane) and at most 2048 intermediate and shared outputs (the down kernel's chunk layouts)
bool decode_supported_bits(int D, int I, int S, int bits) {
    if (bits == 4) return true;
    return bits == 8 && D <= 2048 && I <= 2048 && S <= 2048;
}

bool decode_supported(int D, int I, int S, int T, int k, int E) {
    auto ok = [](int K) { return K >= 512 && K <= 8192 && K % 32 == 0; };
    return T >= 1 && T <= kMaxT && T * k <= kMaxP && E <= 512 && ok(D) && ok(I) &&
           (S == 0 || (ok(S) && S % 16 == 0)) && D % 4 == 0 && I % 16 == 0 && D >= 2048;
}

hipError_t launch_decode(const DecodeJob &j, hipStream_t s, StageMarks *marks) {
    // the fused norm keeps the block input in the router launch's LDS: 16 tokens at most
    if (j.norm_src && (j.T > 16 || 2 * (size_t)j.T * j.D > 65536)) return hipErrorInvalidValue;
    if (!j.router_done) {
        if (j.T == 1) launch_k1<1>(j, s);
        else if (j.T <= 4) launch_k1<4>(j, s);
        else launch_k1<16>(j, s);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (!j.topk_in_kernel) {
        e = launch_topk(j.logits, j.T, j.E, j.k, j.norm != 0, nullptr, j.ids, j.scores, s);
        if (e != hipSuccess) return e;
    }
    if (marks) marks->mark(s);

    const int n_ch = j.D >> 5;
    // rows per wave: 2 at T = 2 (1024 routed waves-of-rows over 16 expert slots), 4 otherwise; at
    // T = 1 four rows (256 routed workgroups instead of 512, so that with the shared expert's the
    // grid takes about one workgroup per CU) took the launch from 6.0 to 5.5 us (timed from
    // inside) at the same bits; rows wider than 2048 take one row per wave and the streaming loop
    // at every T
    const int rg = n_ch > 64 ? 1 : (j.T == 2 ? 2 : 4);
    // 4 waves per workgroup: 8 and 16 (fewer redundant top-ks per CU) measured slower
    const bool b8 = j.wg.bits == 8;
    if (b8 && rg == 2) launch_k2<2, 4, 8>(j, n_ch, s);
    else if (b8) launch_k2<4, 4, 8>(j, n_ch, s);
    else if (rg == 1) launch_k2<1, 4, 4>(j, n_ch, s);
    else if (rg == 2) launch_k2<2, 4, 4>(j, n_ch, s);
    else launch_k2<4, 4, 4>(j, n_ch, s);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (marks) marks->mark(s);

    const int ich = j.I >> 5;
    if (const int drs = stream_k3_rows(j)) {
        const dim3 g3(j.D / drs), b3(512);
        if (ich <= 128) decode_down_stream_kernel<2, kStreamBatch><<<g3, b3, 0, s>>>(j, drs);
        else decode_down_stream_kernel<3, kStreamBatch><<<g3, b3, 0, s>>>(j, drs);
    } else if (b8) {  // 8-bit experts: I of at most 2048
        if (ich == 16) launch_k3_s<16, 1, 8>(j, s);
        else if (ich < 64) launch_k3_s<32, 2, 8>(j, s);
        else launch_k3_s<64, 1, 8>(j, s);
    } else if (ich == 16) launch_k3_s<16, 1, 4>(j, s);
    else if (ich < 64) launch_k3_s<32, 2, 4>(j, s);
    else if (ich <= 64) launch_k3_s<64, 1, 4>(j, s);
    else if (ich <= 128) launch_k3_s<64, 2, 4>(j, s);
    else if (ich <= 192) launch_k3_s<64, 3, 4>(j, s);
    else launch_k3_s<64, 4, 4>(j, s);
    e = hipGetLastError();
    if (e == hipSuccess && marks) marks->mark(s);
    return e;
}

}  // namespace mrun
