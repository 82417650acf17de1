// Prefill-shaped products on the matrix cores (gfx950 v_mfma_f32_32x32x16_bf16):
//  - grouped 4-bit expert GEMM over expert-sorted row tiles (gather_qmm with sorted indices,
//    nuvec.rs:670-686), optionally with the gate/up pair and SwiGLU fused in the epilogue
//    (moe.rs:79-83, activations.rs:55-59);
//  - dense bf16 GEMM (the router's Linear, load.rs:294-306).
//
// Exact affine dequant: out = sum_g [ s_g * sum_{k in g} x_k q_k + b_g * sum_{k in g} x_k ].
// The codes 0..15 are exact in bf16, so each group's sum_k x_k q_k is an MFMA chain with f32
// accumulation; the group's scale and bias are applied in f32 on the VALU. No bf16 rounding of
// dequantized weights happens anywhere (q*s+b is generally not a bf16 value).
//
// Tile: 64 rows x 64 columns (per projection) x 64 k per step, 4 waves in 2 x 2, each wave one
// 32 x 32 accumulator per projection. A rows are gathered through a row map (sorted position ->
// token row); B codes are dequantized once per step into LDS and shared by the 4 waves. Global
// loads of step k+1 are issued before the MFMAs of step k.
#include "common.hpp"
#include "kernels.hpp"

namespace mrun {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

constexpr int BM = kGemmTileM, BN = kGemmTileN, BK = 64, LDK = BK + 8;

__device__ __forceinline__ bf16x8_t lds_frag(const bf16_t *p) {
    return __builtin_bit_cast(bf16x8_t, *(const uint4 *)p);
}

// Eight 4-bit codes of one word -> eight exact bf16 (code order preserved).
__device__ __forceinline__ uint4 codes_to_bf16(uint32_t w) {
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = __float_as_uint((float)((w >> (4 * i)) & 15u)) >> 16;
    return make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16),
                      b[6] | (b[7] << 16));
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
    const QW &wsq = (GLU && sp) ? j.w1 : j.w0;
    const size_t srow =
        ((size_t)e * wsq.out + min(n0 + sn, j.N - 1)) * (size_t)(K / wsq.group);

    uint4 ra0, ra1, rb0, rb1;
    uint32_t rw[WPT];
    float rs = 0.f, rbias = 0.f;
    auto gload = [&](int k0) {
        ra0 = ((const uint4 *)(aptr + k0))[0];
        ra1 = ((const uint4 *)(aptr + k0))[1];
        if (QUANT) {
#pragma unroll
            for (int i = 0; i < WPT; ++i) rw[i] = bcodes[(k0 >> 3) + i];
            if (sthread) {
                const int g = (k0 + ss * (BK / SUB)) / wsq.group;
                rs = bf2f(wsq.scales[srow + g]);
                rbias = wsq.biases ? bf2f(wsq.biases[srow + g]) : 0.f;
            }
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
        *(uint4 *)&As[ar * LDK + ak] = ra0;
        *(uint4 *)&As[ar * LDK + ak + 8] = ra1;
        if (QUANT) {
            float xs = 0.f;
            const uint32_t av[8] = {ra0.x, ra0.y, ra0.z, ra0.w, ra1.x, ra1.y, ra1.z, ra1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) xs += bf_lo(av[i]) + bf_hi(av[i]);
            xs += __shfl_xor(xs, 1, 64);
            if (SUB == 1) {
                xs += __shfl_xor(xs, 2, 64);
                if ((tid & 3) == 0) Xs[0][ar] = xs;
            } else {
                if ((tid & 1) == 0) Xs[(tid & 3) >> 1][ar] = xs;
            }
            bf16_t *bdst = &Bs[(bp * BN + bn) * LDK + bq * WPT * 8];
#pragma unroll
            for (int i = 0; i < WPT; ++i) *(uint4 *)(bdst + 8 * i) = codes_to_bf16(rw[i]);
            if (sthread) {
                Sc[sp][ss][sn] = rs;
                Bi[sp][ss][sn] = rbias;
            }
        } else {
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
