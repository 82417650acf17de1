// Prefill-shaped products on the matrix cores (gfx950 v_mfma_f32_32x32x16_bf16):
//  - grouped 4-bit expert GEMM over expert-sorted row tiles (gather_qmm with sorted indices,
//    nuvec.rs:670-686), optionally with the gate/up pair and SwiGLU fused in the epilogue
//    (moe.rs:79-83, activations.rs:55-59);
//  - dense bf16 GEMM (the router's Linear, load.rs:294-306).
//
// Affine dequant folded around the MFMA: a code q sits in the low mantissa bits of bf16 128.0
// (0x4300 | q == 128 + q exactly), so the B tile is built with one and-or per two codes; the MFMA
// chain over a quant group (64 k) accumulates P' = sum_k x_k (128 + q_k) in f32, and the group is
// applied on the VALU as  acc += s * P' + (b - 128 s) * X  with X = sum_k x_k of the group. Each
// dword of B holds codes (i, i + 4) of its word, so the A tile is staged re-paired the same way.
// Dense B (the router's bf16 weights) goes to the MFMAs unchanged.
//
#include "common.hpp"
#include "kernels.hpp"

namespace mrun {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

constexpr int BM = kGemmTileM, BN = kGemmTileN, BK = 64, LDK = BK + 8;

__device__ __forceinline__ bf16x8_t lds_frag(const bf16_t *p) {
    return __builtin_bit_cast(bf16x8_t, *(const uint4 *)p);
}

// Eight 4-bit codes of one word -> bf16 (128 + q) pairs (q_i, q_{i+4}), i = 0..3.
__device__ __forceinline__ uint4 codes_to_pairs(uint32_t w) {
    return make_uint4((w & 0x000F000Fu) | 0x43004300u, ((w >> 4) & 0x000F000Fu) | 0x43004300u,
                      ((w >> 8) & 0x000F000Fu) | 0x43004300u, ((w >> 12) & 0x000F000Fu) | 0x43004300u);
}

// Eight bf16 x_0..x_7 (one uint4) re-paired as (x_i, x_{i+4}).
__device__ __forceinline__ uint4 pair8(const uint4 &a) {
    return make_uint4(__builtin_amdgcn_perm(a.z, a.x, 0x05040100u),
                      __builtin_amdgcn_perm(a.z, a.x, 0x07060302u),
                      __builtin_amdgcn_perm(a.w, a.y, 0x05040100u),
                      __builtin_amdgcn_perm(a.w, a.y, 0x07060302u));
}

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
__device__ __forceinline__ float dot2_(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
}

template <bool QUANT, bool GLU, int SUB>
__global__ __launch_bounds__(256) void gemm_kernel(GemmJob j) {
    constexpr int NP = GLU ? 2 : 1;
    constexpr int TPR = GLU ? 2 : 4;           // B threads per output row (quantized)
    constexpr int WPT = 8 / TPR;               // code words per B thread per step
    __shared__ __align__(16) bf16_t As[BM * LDK];
    __shared__ __align__(16) bf16_t Bs[NP * BN * LDK];
    __shared__ float Sc[NP][SUB][BN], Bi[NP][SUB][BN];
    __shared__ float Xs[SUB][BM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (j.zero && blockIdx.x == 0 && blockIdx.y == 0)
        for (int i = tid; i < j.n_zero; i += 256) j.zero[i] = 0;
    int e, row0, mrows;
    if (j.has_routing) {
        if (blockIdx.x >= *j.routing.n_tiles) return;
        const uint32_t *t3 = j.routing.tiles + 3 * (size_t)blockIdx.x;
        e = (int)t3[0];
        row0 = (int)t3[1];
        mrows = (int)t3[2];
    } else {
        e = 0;
        row0 = blockIdx.x * BM;
        if (row0 >= j.M) return;
        mrows = min(BM, j.M - row0);
    }
    const int n0 = blockIdx.y * BN;
    const int K = j.K;

    // A: row ar, 16 elements from ak
    const int ar = tid >> 2, ak = (tid & 3) * 16;
    const int apos = row0 + min(ar, mrows - 1);
    const int arow = j.a_map ? (int)(j.a_map[apos] / (uint32_t)j.a_div) : apos;
    const bf16_t *aptr = j.A + (size_t)arow * j.lda + ak;

    // B
    const int bp = QUANT ? tid / (BN * TPR) : 0;
    const int bn = QUANT ? (tid % (BN * TPR)) / TPR : tid >> 2;
    const int bq = QUANT ? tid % TPR : tid & 3;
    const QW &wq = (GLU && bp) ? j.w1 : j.w0;
    const uint32_t *bcodes = nullptr;
    const bf16_t *bdense = nullptr;
    const int brow = min(n0 + bn, j.N - 1);  // columns past N load a valid row, never stored
    if (QUANT) bcodes = wq.codes + ((size_t)e * wq.out + brow) * (K >> 3) + bq * WPT;
    else bdense = j.bd + (size_t)brow * K + bq * 16;
    // scales: thread -> (p, sub, n)
    const bool sthread = QUANT && tid < NP * SUB * BN;
    const int sp = tid / (SUB * BN), ss = (tid / BN) % SUB, sn = tid % BN;
    const QW &wsq = (GLU && sp == 1) ? j.w1 : j.w0;
    const size_t srow =
        ((size_t)e * wsq.out + min(n0 + sn, j.N - 1)) * (size_t)(K / wsq.group);

    uint4 ra0, ra1, rb0, rb1;
    uint32_t rw[WPT];
    uint32_t rs = 0, rbias = 0;  // raw bf16: converted when staged, a step after the load
    auto gload = [&](int k0) {
        ra0 = ((const uint4 *)(aptr + k0))[0];
        ra1 = ((const uint4 *)(aptr + k0))[1];
        if (QUANT) {
#pragma unroll
            for (int i = 0; i < WPT; ++i) rw[i] = bcodes[(k0 >> 3) + i];
            const int g = (k0 + ss * (BK / SUB)) / wsq.group;
            rs = wsq.scales[srow + g];
            rbias = wsq.biases ? (uint32_t)wsq.biases[srow + g] : 0u;
        } else {
            rb0 = ((const uint4 *)(bdense + k0))[0];
            rb1 = ((const uint4 *)(bdense + k0))[1];
        }
    };

    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 31, fk = (lane >> 5) * 8;
    f32x16_t acc[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[p][i] = 0.f;

    gload(0);
    for (int k0 = 0; k0 < K; k0 += BK) {
        __syncthreads();
        // stage A (and its group sums) and B into LDS
        if (QUANT) {
            const uint4 pa0 = pair8(ra0), pa1 = pair8(ra1);
            *(uint4 *)&As[ar * LDK + ak] = pa0;
            *(uint4 *)&As[ar * LDK + ak + 8] = pa1;
            const uint32_t av[8] = {pa0.x, pa0.y, pa0.z, pa0.w, pa1.x, pa1.y, pa1.z, pa1.w};
            float xs = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) xs = dot2_(av[i], 0x3F803F80u, xs);
            xs += dpp_f32<0xB1>(xs);  // the 4 threads of a row are one quad
            if (SUB == 1) {
                xs += dpp_f32<0x4E>(xs);
                if ((tid & 3) == 0) Xs[0][ar] = xs;
            } else {
                if ((tid & 1) == 0) Xs[(tid & 3) >> 1][ar] = xs;
            }
            bf16_t *bdst = &Bs[(bp * BN + bn) * LDK + bq * WPT * 8];
#pragma unroll
            for (int i = 0; i < WPT; ++i) *(uint4 *)(bdst + 8 * i) = codes_to_pairs(rw[i]);
            if (sthread) {
                const float sc = bf2f(rs);
                Sc[sp][ss][sn] = sc;
                Bi[sp][ss][sn] = bf2f(rbias) - 128.f * sc;
            }
        } else {
            *(uint4 *)&As[ar * LDK + ak] = ra0;
            *(uint4 *)&As[ar * LDK + ak + 8] = ra1;
            *(uint4 *)&Bs[bn * LDK + bq * 16] = rb0;
            *(uint4 *)&Bs[bn * LDK + bq * 16 + 8] = rb1;
        }
        __syncthreads();
        if (k0 + BK < K) gload(k0 + BK);

#pragma unroll
        for (int sub = 0; sub < SUB; ++sub) {
            f32x16_t part[NP];
#pragma unroll
            for (int p = 0; p < NP; ++p)
#pragma unroll
                for (int i = 0; i < 16; ++i) part[p][i] = 0.f;
#pragma unroll
            for (int s = 0; s < BK / SUB / 16; ++s) {
                const int kk = sub * (BK / SUB) + s * 16 + fk;
                const bf16x8_t a = lds_frag(&As[(wm * 32 + fr) * LDK + kk]);
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    const bf16x8_t b = lds_frag(&Bs[(p * BN + wn * 32 + fr) * LDK + kk]);
                    if (QUANT)
                        part[p] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, part[p], 0, 0, 0);
                    else
                        acc[p] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[p], 0, 0, 0);
                }
            }
            if (QUANT) {
#pragma unroll
                for (int p = 0; p < NP; ++p) {
                    const float sc = Sc[p][sub][wn * 32 + fr], bi = Bi[p][sub][wn * 32 + fr];
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int r = wm * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
                        acc[p][i] += sc * part[p][i] + bi * Xs[sub][r];
                    }
                }
            }
        }
    }

    const int col = n0 + wn * 32 + fr;
    const float bias = (!GLU && j.bias && col < j.N) ? bf2f(j.bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = wm * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (r < mrows && col < j.N) {
            const int pos = row0 + r;
            const int orow = j.o_map ? (int)j.o_map[pos] : pos;
            float v;
            if (GLU) {
                const float g = rbf(acc[0][i]), u = rbf(acc[GLU ? 1 : 0][i]);
                v = (g * sigmoidf_(g)) * u;
            } else {
                v = acc[0][i];
                if (j.bias) v = rbf(v) + bias;
            }
            j.out[(size_t)orow * j.ldo + col] = (bf16_t)f2bf(v);
        }
    }
}

hipError_t launch_gemm(const GemmJob &j, hipStream_t stream) {
    const int tiles = j.has_routing ? j.max_tiles : (j.M + BM - 1) / BM;
    if (tiles <= 0) return hipSuccess;
    dim3 grid(tiles, (j.N + BN - 1) / BN);
    if (!j.bd) {
        const bool sub2 = j.w0.group == 32;
        if (j.glu) {
            if (sub2) gemm_kernel<true, true, 2><<<grid, 256, 0, stream>>>(j);
            else gemm_kernel<true, true, 1><<<grid, 256, 0, stream>>>(j);
        } else {
            if (sub2) gemm_kernel<true, false, 2><<<grid, 256, 0, stream>>>(j);
            else gemm_kernel<true, false, 1><<<grid, 256, 0, stream>>>(j);
        }
    } else {
        gemm_kernel<false, false, 1><<<grid, 256, 0, stream>>>(j);
    }
    return hipGetLastError();
}

}  // namespace mrun
