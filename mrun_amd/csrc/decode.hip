// Decode schedule of the MoE block (T <= 16 tokens, T*k <= 128 pairs): three launches, no global
// routing round trip and no permutation (SparseMoe::forward, moe.rs:149-174).
//
//   K1 router  : router logits (+ bias), the shared expert's gate logit and its gate/up + SwiGLU.
//                The shared expert does not depend on the routing, so it runs beside the router.
//   K2 gate/up : every workgroup re-derives the top-k of all T tokens from the L2-resident logits
//                (the same code as the router op, so the same bits), picks the slot-th active expert
//                (experts in ascending order), and streams that expert's gate/up rows for its pairs.
//   K3 down    : prefetches the shared expert's down rows, re-derives top-k and scores, computes the
//                routed down rows of every active expert for its 8 output rows, then the combine:
//                out = R(R(sum_j R(y[t,j] * s[t,j])) + R(R(sigmoid(g_t)) * shared[t])).
// Pair p = t*k + j indexes the activations (act [T*k, I]), so no argsort is needed at decode; the
// results are the same as the sorted dispatch's, row by row.
#include "common.hpp"
#include "gemv_core.hpp"
#include "kernels.hpp"
#include "topk.hpp"

namespace mrun {

constexpr int kMaxT = 16, kMaxP = 128, kDownRowsPerWG = 8;

// Rows [row_base + g*RPI + rsub] of w0 (and w1 with glu), g < RG, for the pairs set in pm0|pm1
// (bit p: pair p reads A row p / a_div and writes output row p). The next pair's activations are
// loaded while the current pair is computed.
template <int LPR, int CPL, int RG, bool GLU>
__device__ __forceinline__ void gemv_wave(const QW &w0, const QW &w1, int e, int row_base,
                                          const bf16_t *A, int lda, int a_div, uint64_t pm0,
                                          uint64_t pm1, bf16_t *out, int ldo, int lane) {
    constexpr int RPI = 64 / LPR;
    const int li = lane % LPR, rsub = lane / LPR;
    const int n_ch = w0.in >> 5;
    WRow<CPL> r0[RG], r1[RG];
#pragma unroll
    for (int g = 0; g < RG; ++g) {
        const int row = row_base + g * RPI + rsub;
        load_wrow<CPL>(w0, e, row, li, LPR, r0[g]);
        if (GLU) load_wrow<CPL>(w1, e, row, li, LPR, r1[g]);
    }
    auto next = [&](uint64_t &m0, uint64_t &m1) -> int {
        if (m0) {
            const int p = __ffsll((unsigned long long)m0) - 1;
            m0 &= m0 - 1;
            return p;
        }
        if (m1) {
            const int p = 64 + __ffsll((unsigned long long)m1) - 1;
            m1 &= m1 - 1;
            return p;
        }
        return -1;
    };
    int p = next(pm0, pm1);
    if (p < 0) return;
    XRaw cur[CPL], nxt[CPL];
    load_xrow_raw<CPL>(A + (size_t)(p / a_div) * lda, li, LPR, n_ch, cur);
    while (p >= 0) {
        const int pn = next(pm0, pm1);
        load_xrow_raw<CPL>(A + (size_t)((pn >= 0 ? pn : p) / a_div) * lda, li, LPR, n_ch, nxt);
        XChunk xc[CPL];
        pair_xrow<CPL>(cur, xc);
#pragma unroll
        for (int g = 0; g < RG; ++g) {
            opaque_row(r0[g]);
            if (GLU) opaque_row(r1[g]);
        }
#pragma unroll
        for (int g = 0; g < RG; ++g) {
            const int row = row_base + g * RPI + rsub;
            const float a0 = group_sum<LPR>(row_part(r0[g], xc));
            const float a1 = GLU ? group_sum<LPR>(row_part(r1[g], xc)) : 0.f;
            if (li == 0 && row < w0.out) {
                float v = a0;
                if (GLU) {
                    const float gt = rbf(a0), up = rbf(a1);
                    v = (gt * sigmoidf_(gt)) * up;
                }
                out[(size_t)p * ldo + row] = (bf16_t)f2bf(v);
            }
        }
#pragma unroll
        for (int c = 0; c < CPL; ++c) cur[c] = nxt[c];
        p = pn;
    }
}

// One dense row for T <= 16 tokens (one wave): R(x[t] . w) then R(. + bias). Lane l owns
// elements [8l + 512i, +8); tokens go in groups of 4 whose loads are issued together.
template <int MAXT>
__device__ __forceinline__ void router_row(const bf16_t *x, int T, int D, const bf16_t *w,
                                           const bf16_t *bias, bf16_t *out, int ldo, int lane) {
    constexpr int TG = 4;
    float acc[MAXT];
#pragma unroll
    for (int t = 0; t < MAXT; ++t) acc[t] = 0.f;
    const uint32_t braw = bias ? (uint32_t)*bias : 0u;
    for (int d = lane * 8; d < D; d += 2048) {
        uint4 wv[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) wv[i] = *(const uint4 *)(w + min(d + 512 * i, D - 8));
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
    router_row<MAXT>(x, T, D, W + (size_t)r * D, bias ? bias + r : nullptr, out + r, N, lane);
}

hipError_t launch_rows(const bf16_t *x, int T, int D, const bf16_t *W, const bf16_t *bias, int N,
                       bf16_t *out, hipStream_t stream) {
    dim3 grid((N + 3) / 4);
    if (T <= 4) rows_kernel<4><<<grid, 256, 0, stream>>>(x, T, D, W, bias, N, out);
    else rows_kernel<16><<<grid, 256, 0, stream>>>(x, T, D, W, bias, N, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// K1: router + shared gate logit + shared gate/up

template <int MAXT, int LPR, int CPL>
__global__ __launch_bounds__(256) void decode_router_kernel(DecodeJob j) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n_rows = j.E + (j.S ? 1 : 0);
    const int n_rb = (n_rows + 3) / 4;
    if ((int)blockIdx.x < n_rb) {
        const int r = blockIdx.x * 4 + wave;
        if (r < j.E)
            router_row<MAXT>(j.x, j.T, j.D, j.router + (size_t)r * j.D,
                             j.router_bias ? j.router_bias + r : nullptr, j.logits + r, j.E, lane);
        else if (r == j.E)
            router_row<MAXT>(j.x, j.T, j.D, j.sh_gate_w, j.sh_gate_b, j.sh_logit, 1, lane);
        return;
    }
    // shared expert gate/up: 16 rows x up to 4 tokens per workgroup
    constexpr int RPI = 64 / LPR, RG = 4;
    const int sb = blockIdx.x - n_rb, n_row_blocks = j.S / 16;
    const int rb = sb % n_row_blocks, t0 = (sb / n_row_blocks) * 4;
    const int tn = min(4, j.T - t0);
    const uint64_t toks = ((1ull << tn) - 1) << t0;
    gemv_wave<LPR, CPL, RG, true>(j.sg, j.su, 0, (rb * 4 + wave) * RG * RPI, j.x, j.D, 1, toks, 0,
                                  j.sh_act, j.S, lane);
}

// ---------------------------------------------------------------------------------------------
// shared by K2 and K3: the top-k of every token into LDS, and the active-expert mask

__device__ __forceinline__ void all_topk(const DecodeJob &j, uint32_t *sid, bf16_t *ssc,
                                         uint32_t *mask) {
    const int wave = threadIdx.x >> 6;
    if (threadIdx.x < 16) mask[threadIdx.x] = 0;
    if (j.topk_in_kernel) {
        for (int t = wave; t < j.T; t += 4)
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
    for (int p = threadIdx.x; p < j.T * j.k; p += 256) atomicOr(&mask[sid[p] >> 5], 1u << (sid[p] & 31));
    __syncthreads();
}

// Pairs choosing expert e, as a 128-bit set (one wave, from LDS).
__device__ __forceinline__ void pairs_of(const uint32_t *sid, int P, int e, int lane,
                                         uint64_t &pm0, uint64_t &pm1) {
    pm0 = __ballot(lane < P && (int)sid[lane] == e);
    pm1 = __ballot(lane + 64 < P && (int)sid[lane + 64] == e);
}

// ---------------------------------------------------------------------------------------------
// K2: routed gate/up

template <int LPR, int CPL>
__global__ __launch_bounds__(256) void decode_gateup_kernel(DecodeJob j) {
    __shared__ uint32_t sid[kMaxP], mask[16];
    __shared__ bf16_t ssc[kMaxP];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    all_topk(j, sid, ssc, mask);
    // the slot-th active expert, experts in ascending order
    const int slot = blockIdx.y;
    int e = -1, n = 0;
    for (int w = 0; w < (j.E + 31) / 32; ++w) {
        const uint32_t mw = mask[w];
        const int c = __popc(mw);
        if (e < 0 && slot < n + c) {
            uint32_t m = mw;
            for (int i = 0; i < slot - n; ++i) m &= m - 1;
            e = w * 32 + __ffs(m) - 1;
        }
        n += c;
    }
    if (e < 0) return;
    uint64_t pm0, pm1;
    pairs_of(sid, j.T * j.k, e, lane, pm0, pm1);
    constexpr int RPI = 64 / LPR, RG = 4;
    gemv_wave<LPR, CPL, RG, true>(j.wg, j.wu, e, (blockIdx.x * 4 + wave) * RG * RPI, j.x, j.D, j.k,
                                  pm0, pm1, j.act, j.I, lane);
}

// ---------------------------------------------------------------------------------------------
// K3: down + combine

template <int LPR, int CPL, int SLPR, int SCPL, int PB>
__global__ __launch_bounds__(256) void decode_down_kernel(DecodeJob j) {
    constexpr int RPI = 64 / LPR, NRG = kDownRowsPerWG / RPI;
    constexpr int SRPI = 64 / SLPR, SNRG = kDownRowsPerWG / SRPI, SG = (SNRG + 3) / 4;
    __shared__ uint32_t sid[kMaxP], mask[16];
    __shared__ bf16_t ssc[kMaxP];
    __shared__ float yv[kMaxP][kDownRowsPerWG];
    __shared__ float ysh[kMaxT][kDownRowsPerWG];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int d0 = blockIdx.x * kDownRowsPerWG;

    // the shared expert's rows do not depend on the routing: start their loads first
    WRow<SCPL> sr[SG];
    if (j.S) {
#pragma unroll
        for (int i = 0; i < SG; ++i) {
            const int g = wave + 4 * i;
            load_wrow<SCPL>(j.sd, 0, g < SNRG ? d0 + g * SRPI + lane / SLPR : j.D, lane % SLPR,
                            SLPR, sr[i]);
        }
    }
    all_topk(j, sid, ssc, mask);

    // work: for each pair p (expert sid[p]) its NRG row groups of this workgroup's rows; a wave
    // takes PB pairs at a time and issues all their loads before computing
    const int P = j.T * j.k, li = lane % LPR, rsub = lane / LPR;
    const int per_wave = (P + 3) / 4;
    const int p_lo = wave * per_wave, p_hi = min(P, p_lo + per_wave);
    for (int pb = p_lo; pb < p_hi; pb += PB) {
        XRaw xr[PB][CPL];
        WRow<CPL> wr[PB][NRG];
#pragma unroll
        for (int b = 0; b < PB; ++b) {
            const int p = min(pb + b, p_hi - 1);
            const int e = (int)sid[p];
            load_xrow_raw<CPL>(j.act + (size_t)p * j.I, li, LPR, j.I >> 5, xr[b]);
#pragma unroll
            for (int g = 0; g < NRG; ++g)
                load_wrow<CPL>(j.wd, e, d0 + g * RPI + rsub, li, LPR, wr[b][g]);
        }
#pragma unroll
        for (int b = 0; b < PB; ++b) {
            const int p = pb + b;
            if (p >= p_hi) break;
            XChunk xc[CPL];
            pair_xrow<CPL>(xr[b], xc);
#pragma unroll
            for (int g = 0; g < NRG; ++g) {
                const float y = group_sum<LPR>(row_part(wr[b][g], xc));
                if (li == 0) yv[p][g * RPI + rsub] = rbf(y);
            }
        }
    }
    if (j.S) {
        const int sli = lane % SLPR;
        XRaw cur[SCPL], nxt[SCPL];
        load_xrow_raw<SCPL>(j.sh_act, sli, SLPR, j.S >> 5, cur);
        for (int t = 0; t < j.T; ++t) {
            load_xrow_raw<SCPL>(j.sh_act + (size_t)min(t + 1, j.T - 1) * j.S, sli, SLPR, j.S >> 5,
                                nxt);
            XChunk xc[SCPL];
            pair_xrow<SCPL>(cur, xc);
#pragma unroll
            for (int c = 0; c < SCPL; ++c) cur[c] = nxt[c];
#pragma unroll
            for (int i = 0; i < SG; ++i) {
                const int g = wave + 4 * i;
                opaque_row(sr[i]);
                const float y = group_sum<SLPR>(row_part(sr[i], xc));
                if (g < SNRG && sli == 0) ysh[t][g * SRPI + lane / SLPR] = rbf(y);
            }
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < j.T * kDownRowsPerWG; i += 256) {
        const int t = i / kDownRowsPerWG, dd = i % kDownRowsPerWG;
        float acc = 0.f;
        for (int jj = 0; jj < j.k; ++jj) {
            const int p = t * j.k + jj;
            acc += rbf(yv[p][dd] * bf2f(ssc[p]));
        }
        float r = rbf(acc);
        if (j.S) {
            const float sg = rbf(sigmoidf_(bf2f(j.sh_logit[t])));
            r = rbf(r + rbf(sg * ysh[t][dd]));
        }
        j.out[(size_t)t * j.D + d0 + dd] = (bf16_t)f2bf(r);
    }
}

// ---------------------------------------------------------------------------------------------

template <int MAXT>
static void launch_k1(const DecodeJob &j, hipStream_t s) {
    const int n_rb = (j.E + (j.S ? 1 : 0) + 3) / 4;
    // LPR 64 (D >= 2048): 16 rows x 4 tokens per workgroup
    const int sh_blocks = j.S ? (j.S / 16) * ((j.T + 3) / 4) : 0;
    const int n_ch = j.D >> 5;
    dim3 grid(n_rb + sh_blocks);
    if (n_ch <= 64) decode_router_kernel<MAXT, 64, 1><<<grid, 256, 0, s>>>(j);
    else if (n_ch <= 128) decode_router_kernel<MAXT, 64, 2><<<grid, 256, 0, s>>>(j);
    else if (n_ch <= 192) decode_router_kernel<MAXT, 64, 3><<<grid, 256, 0, s>>>(j);
    else decode_router_kernel<MAXT, 64, 4><<<grid, 256, 0, s>>>(j);
}

template <int LPR, int CPL>
static void launch_k3_s(const DecodeJob &j, hipStream_t s) {
    // pairs per load batch: keep a batch's activations and weight rows within ~128 registers
    constexpr int NRG = kDownRowsPerWG / (64 / LPR);
    constexpr int PB = (NRG * CPL <= 2) ? 4 : (NRG * CPL <= 4 ? 2 : 1);
    dim3 grid(j.D / kDownRowsPerWG);
    const int sch = j.S ? j.S >> 5 : 16;
    if (sch == 16) decode_down_kernel<LPR, CPL, 16, 1, PB><<<grid, 256, 0, s>>>(j);
    else if (sch < 64) decode_down_kernel<LPR, CPL, 32, 2, PB><<<grid, 256, 0, s>>>(j);
    else if (sch <= 64) decode_down_kernel<LPR, CPL, 64, 1, PB><<<grid, 256, 0, s>>>(j);
    else if (sch <= 128) decode_down_kernel<LPR, CPL, 64, 2, PB><<<grid, 256, 0, s>>>(j);
    else decode_down_kernel<LPR, CPL, 64, 4, PB><<<grid, 256, 0, s>>>(j);
}

bool decode_supported(int D, int I, int S, int T, int k, int E) {
    auto ok = [](int K) { return K >= 512 && K <= 8192 && K % 32 == 0; };
    return T >= 1 && T <= kMaxT && T * k <= kMaxP && E <= 512 && ok(D) && ok(I) &&
           (S == 0 || (ok(S) && S % 16 == 0)) && D % kDownRowsPerWG == 0 && I % 16 == 0 &&
           D >= 2048;
}

hipError_t launch_decode(const DecodeJob &j, hipStream_t s, StageMarks *marks) {
    if (j.T <= 4) launch_k1<4>(j, s);
    else launch_k1<16>(j, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (!j.topk_in_kernel) {
        e = launch_topk(j.logits, j.T, j.E, j.k, j.norm != 0, nullptr, j.ids, j.scores, s);
        if (e != hipSuccess) return e;
    }
    if (marks) marks->mark(s);

    const int n_ch = j.D >> 5;
    dim3 g2(j.I / 16, j.max_slots);
    if (n_ch <= 64) decode_gateup_kernel<64, 1><<<g2, 256, 0, s>>>(j);
    else if (n_ch <= 128) decode_gateup_kernel<64, 2><<<g2, 256, 0, s>>>(j);
    else if (n_ch <= 192) decode_gateup_kernel<64, 3><<<g2, 256, 0, s>>>(j);
    else decode_gateup_kernel<64, 4><<<g2, 256, 0, s>>>(j);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (marks) marks->mark(s);

    const int ich = j.I >> 5;
    if (ich == 16) launch_k3_s<16, 1>(j, s);
    else if (ich < 64) launch_k3_s<32, 2>(j, s);
    else if (ich <= 64) launch_k3_s<64, 1>(j, s);
    else if (ich <= 128) launch_k3_s<64, 2>(j, s);
    else if (ich <= 192) launch_k3_s<64, 3>(j, s);
    else launch_k3_s<64, 4>(j, s);
    e = hipGetLastError();
    if (e == hipSuccess && marks) marks->mark(s);
    return e;
}

}  // namespace mrun
