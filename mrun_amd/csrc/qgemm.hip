// Prefill-shaped products on the matrix cores (gfx950 v_mfma_f32_32x32x16_bf16):
//  - grouped 4- or 8-bit expert GEMM over expert-sorted row tiles (gather_qmm with sorted indices,
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

constexpr int BM = 64, BN = kGemmTileN, BK = 64, LDK = BK + 8;

__device__ __forceinline__ bf16x8_t lds_frag(const bf16_t *p) {
    return __builtin_bit_cast(bf16x8_t, *(const uint4 *)p);
}

// Eight 4-bit codes of one word -> bf16 (128 + q) pairs (q_i, q_{i+4}), i = 0..3.
__device__ __forceinline__ uint4 codes_to_pairs(uint32_t w) {
    return make_uint4((w & 0x000F000Fu) | 0x43004300u, ((w >> 4) & 0x000F000Fu) | 0x43004300u,
                      ((w >> 8) & 0x000F000Fu) | 0x43004300u, ((w >> 12) & 0x000F000Fu) | 0x43004300u);
}

// Four 8-bit codes of one word -> bf16 pairs (q0, q1), (q2, q3): integers below 256 are exact in
// bf16, so the top half of their f32 conversion is their bf16.
__device__ __forceinline__ uint2 codes8_to_pairs(uint32_t w) {
    const uint32_t f0 = __float_as_uint((float)(w & 0xffu));
    const uint32_t f1 = __float_as_uint((float)((w >> 8) & 0xffu));
    const uint32_t f2 = __float_as_uint((float)((w >> 16) & 0xffu));
    const uint32_t f3 = __float_as_uint((float)(w >> 24));
    return make_uint2(__builtin_amdgcn_perm(f1, f0, 0x07060302u),
                      __builtin_amdgcn_perm(f3, f2, 0x07060302u));
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

// QB: 0 = dense bf16 B (j.bd, no experts), 4 or 8 = affine-quantized B with that many bits per
// code, 16 = dense bf16 experts (QW with bits 16: gather_mm). 8-bit codes convert to exact bf16
// integers (no offset, A in natural order).
template <int QB, bool GLU, int SUB>
__global__ __launch_bounds__(256) void gemm_kernel(GemmJob j) {
    constexpr bool QUANT = QB == 4 || QB == 8;
    constexpr bool DEXP = QB == 16;
    constexpr int NB4 = DEXP ? (GLU ? 4 : 2) : 2;  // 16-byte B loads per thread per step (dense)
    constexpr int NP = GLU ? 2 : 1;
    constexpr int TPR = GLU ? 2 : 4;           // B threads per output row (quantized)
    constexpr int WPS = BK * (QB ? QB : 4) / 32;  // code words of a row per K step
    constexpr int WPT = WPS / TPR;             // code words per B thread per step
    constexpr int EPW = QB ? 32 / QB : 8;      // codes per word
    constexpr float OFF = QB == 4 ? 128.f : 0.f;  // code offset of the B values
    __shared__ __align__(16) bf16_t As[BM * LDK];
    __shared__ __align__(16) bf16_t Bs[NP * BN * LDK];
    __shared__ float Sc[NP][SUB][BN], Bi[NP][SUB][BN];
    __shared__ float Xs[SUB][BM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (j.zero && blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0)
        for (int i = tid; i < j.n_zero; i += 256) j.zero[i] = 0;
    int e, row0, mrows;
    if (j.has_routing) {
        if (blockIdx.x >= *j.routing.n_tiles) return;
        const uint32_t *t3 = j.routing.tiles + 3 * (size_t)blockIdx.x;
        e = (int)t3[0];
        row0 = (int)t3[1] + BM * (int)blockIdx.z;
        mrows = (int)t3[2] - BM * (int)blockIdx.z;
        if (mrows <= 0) return;
        mrows = min(mrows, BM);
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
    const int bp = (QUANT || DEXP) ? tid / (BN * TPR) : 0;
    const int bn = (QUANT || DEXP) ? (tid % (BN * TPR)) / TPR : tid >> 2;
    const int bq = (QUANT || DEXP) ? tid % TPR : tid & 3;
    const QW &wq = (GLU && bp) ? j.w1 : j.w0;
    const uint32_t *bcodes = nullptr;
    const bf16_t *bdense = nullptr;
    const int brow = min(n0 + bn, j.N - 1);  // columns past N load a valid row, never stored
    if (QUANT) bcodes = wq.codes + ((size_t)e * wq.out + brow) * (size_t)(K / EPW) + bq * WPT;
    else if (DEXP) bdense = (const bf16_t *)wq.codes + ((size_t)e * wq.out + brow) * K + bq * 8 * NB4;
    else bdense = j.bd + (size_t)brow * K + bq * 16;
    // scales: thread -> (p, sub, n)
    const bool sthread = QUANT && tid < NP * SUB * BN;
    const int sp = tid / (SUB * BN), ss = (tid / BN) % SUB, sn = tid % BN;
    const QW &wsq = (GLU && sp == 1) ? j.w1 : j.w0;
    const size_t srow =
        QUANT ? ((size_t)e * wsq.out + min(n0 + sn, j.N - 1)) * (size_t)(K / wsq.group) : 0;

    uint4 ra0, ra1, rb[NB4];
    uint32_t rw[WPT];
    uint32_t rs = 0, rbias = 0;  // raw bf16: converted when staged, a step after the load
    auto gload = [&](int k0) {
        ra0 = ((const uint4 *)(aptr + k0))[0];
        ra1 = ((const uint4 *)(aptr + k0))[1];
        if (QUANT) {
#pragma unroll
            for (int i = 0; i < WPT; ++i) rw[i] = bcodes[k0 / EPW + i];
            const int g = (k0 + ss * (BK / SUB)) / wsq.group;
            rs = wsq.scales[srow + g];
            rbias = wsq.biases ? (uint32_t)wsq.biases[srow + g] : 0u;
        } else {
#pragma unroll
            for (int i = 0; i < NB4; ++i) rb[i] = ((const uint4 *)(bdense + k0))[i];
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
            const uint4 pa0 = QB == 4 ? pair8(ra0) : ra0, pa1 = QB == 4 ? pair8(ra1) : ra1;
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
            bf16_t *bdst = &Bs[(bp * BN + bn) * LDK + bq * WPT * EPW];
#pragma unroll
            for (int i = 0; i < WPT; ++i) {
                if (QB == 4) *(uint4 *)(bdst + 8 * i) = codes_to_pairs(rw[i]);
                else *(uint2 *)(bdst + 4 * i) = codes8_to_pairs(rw[i]);
            }
            if (sthread) {
                const float sc = bf2f(rs);
                Sc[sp][ss][sn] = sc;
                Bi[sp][ss][sn] = bf2f(rbias) - OFF * sc;
            }
        } else {
            *(uint4 *)&As[ar * LDK + ak] = ra0;
            *(uint4 *)&As[ar * LDK + ak + 8] = ra1;
            bf16_t *bdst = &Bs[(bp * BN + bn) * LDK + bq * 8 * NB4];
#pragma unroll
            for (int i = 0; i < NB4; ++i) *(uint4 *)(bdst + 8 * i) = rb[i];
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
    // output rows and bias before any store, in one batch of loads: a load inside each element's
    // bounds check made every store wait for all outstanding memory operations
    float bias = 0.f;
    if (!GLU && j.bias) bias = bf2f(j.bias[min(col, j.N - 1)]);
    int orow[16];
#pragma unroll
    for (int i = 0; i < 16; ++i)
        orow[i] = row0 + min(wm * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3), mrows - 1);
    if (j.o_map) {
#pragma unroll
        for (int i = 0; i < 16; ++i) orow[i] = (int)j.o_map[orow[i]];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = wm * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (r < mrows && col < j.N) {
            float v;
            if (GLU) {
                const float g = rbf(acc[0][i]), u = rbf(acc[GLU ? 1 : 0][i]);
                v = (g * sigmoidf_(g)) * u;
            } else {
                v = acc[0][i];
                if (j.bias) v = rbf(v) + bias;
            }
            j.out[(size_t)orow[i] * j.ldo + col] = (bf16_t)f2bf(v);
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Quantized grouped GEMM, group size 64: workgroup tile 64 WM rows x 256 B rows (glu: 128 gate +
// 128 up columns), 4 WM waves as WM (rows) x 4 (columns); each wave owns 64 rows x two 32-column
// fragments, 16 MFMAs per K step of 64. The launcher builds WM = 1: 64-row tiles of 4 waves, two
// workgroups per CU.
//  - Global loads: A per K step (128 bytes of a row, 8 lanes to a line), the packed codes per SS
//    K steps (a "super-step": 32 SS bytes of a B row, 64 with SS = 2), scales and biases per 16 K
//    steps (a "chunk": 32 bytes of a row each). They pass through registers into LDS; A is
//    re-paired on the way, codes stay packed (XOR-swizzled 16-byte units so fragment reads are
//    conflict-free).
//  - Each lane expands the 32 codes of a fragment and K step in registers. The K step's k are
//    assigned to MFMA slots so that lane half h, sub-step s holds code word 4h + s of the step;
//    the A tile is written in the same order (k block w at position 16 (w % 4) + 8 (w / 4)).
//  - One barrier per K step (A, codes, scales are double-buffered); loads run 2 K steps (A),
//    one super-step (codes) and one chunk (scales) ahead. The barrier waits for LDS operations
//    only, so those loads stay in flight across it.
//  - The VALU does one FMA per output element and K step (acc += s * P', P' the MFMA chain of the
//    step started from zero); the affine bias  sum_k (b - 128 s) x_k = b X - 128 s X  is a small
//    GEMM over the chunk, [rows x 6 C] x [6 C x cols], run on the MFMAs with X = sum_k x_k of a
//    step split into three bf16 (hi + mid + lo == X exactly) against b and -128 s (exact).
//  - A wave whose 64 rows are all past the tile only stages.
//  - The hardware deals workgroups to the 8 XCDs round-robin (workgroup L to XCD L % 8). Blocks
//    of G_TG consecutive tiles go to one XCD, dispatched one after the other: the column blocks of a
//    tile share that XCD's L2 for the tile's A rows, and consecutive tiles of one expert (its rows
//    beyond the first tile) share it for the expert's weights.
//  - Optional shared tiles (a non-routed product of the same N, the shared expert) come first.

constexpr int G_BNB = 256, G_KSC = 16, G_TG = 4;
// tile rows = 64 WM (WM = 1, or 2 with 128-row routed tiles), codes staged per G_SS K steps,
// G_SBUF buffers of scales
constexpr int G_SS = 2, G_SBUF = 1;

struct GTile {
    const bf16_t *A;
    int lda;
    const uint32_t *a_map;
    int a_div;
    int e, row0, mrows, K;
    const uint32_t *o_map;
    bf16_t *out;
    int ldo;
};

__device__ __forceinline__ uint4 expand_codes(uint32_t w, uint32_t cm, uint32_t cx) {
    return make_uint4((w & cm) | cx, ((w >> 4) & cm) | cx, ((w >> 8) & cm) | cx,
                      ((w >> 12) & cm) | cx);
}

// -128 s for a pair of bf16 scales (exact: a power-of-two scaling)
__device__ __forceinline__ uint32_t neg128_pair(uint32_t w) {
    const uint32_t lo = __float_as_uint(-128.f * bf_lo(w)) >> 16;
    const uint32_t hi = __float_as_uint(-128.f * bf_hi(w)) & 0xFFFF0000u;
    return lo | hi;
}

template <bool GLU, int WM, int SS, int SBUF>
__global__ __launch_bounds__(256 * WM, 2 / WM) void qgemm_kernel(GemmJob j) {
    constexpr int G_BM = 64 * WM, G_THREADS = 256 * WM, CU = 2 * SS;  // CU: 16-byte code units per row
    __shared__ __align__(16) bf16_t As[2][G_BM * LDK];
    __shared__ __align__(16) uint4 Bc[2][G_BNB * CU];           // codes of a super-step
    __shared__ __align__(16) bf16_t Sb[SBUF][2][G_BNB][G_KSC];  // scales, biases of a chunk
    __shared__ __align__(16) bf16_t Xs[2][3][G_BM][G_KSC];      // X splits of a chunk

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (j.zero && blockIdx.x == 0)
        for (int i = tid; i < j.n_zero; i += G_THREADS) j.zero[i] = 0;

    constexpr int NCOLS = GLU ? G_BNB / 2 : G_BNB;
    const int nblk = (j.N + NCOLS - 1) / NCOLS;
    // XCD x = L % 8 takes blocks of G_TG consecutive tiles (b % 8 == x); within a block, the G_TG
    // tiles of column block 0 come first, then column block 1, ...
    const int L = blockIdx.x, slot = L >> 3, xcd = L & 7;
    const int r = slot % (G_TG * nblk);
    const int t = G_TG * (8 * (slot / (G_TG * nblk)) + xcd) + r % G_TG, nb = r / G_TG;
    const int s_tiles = j.has_shared ? (j.sh.M + G_BM - 1) / G_BM : 0;
    const bool shared_tile = t < s_tiles;
    GTile g;
    if (shared_tile) {
        g.A = j.sh.A, g.lda = j.sh.lda, g.a_map = nullptr, g.a_div = 1, g.e = 0;
        g.row0 = t * G_BM, g.mrows = min(G_BM, j.sh.M - g.row0), g.K = j.sh.K;
        g.o_map = nullptr, g.out = j.sh.out, g.ldo = j.sh.ldo;
    } else {
        const int rt = t - s_tiles;
        g.A = j.A, g.lda = j.lda, g.a_map = j.a_map, g.a_div = j.a_div;
        g.K = j.K, g.o_map = j.o_map, g.out = j.out, g.ldo = j.ldo;
        if (j.has_routing) {
            if (rt >= j.max_tiles || rt >= (int)*j.routing.n_tiles) return;
            const uint32_t *t3 = j.routing.tiles + 3 * (size_t)rt;
            g.e = (int)t3[0], g.row0 = (int)t3[1], g.mrows = (int)t3[2];
        } else {
            g.e = 0, g.row0 = rt * G_BM;
            if (g.row0 >= j.M) return;
            g.mrows = min(G_BM, j.M - g.row0);
        }
    }
    const int n0 = nb * NCOLS;
    const int K = g.K, nks = K / BK, groups = K / 64;

    // ---- staging roles
    // A: row ar, k blocks 2q and 2q + 1 of each step
    const int ar = tid >> 2, q = tid & 3;
    const int apos = g.row0 + min(ar, g.mrows - 1);
    const int arow = g.a_map ? (int)(g.a_map[apos] / (uint32_t)g.a_div) : apos;
    const bf16_t *aptr = g.A + (size_t)arow * g.lda + 16 * q;
    const int pw0 = 16 * ((2 * q) & 3) + 8 * ((2 * q) >> 2);
    const int pw1 = 16 * ((2 * q + 1) & 3) + 8 * ((2 * q + 1) >> 2);
    // weights of this tile (selected field by field: a pointer into the kernel arguments would go
    // to scratch); under glu B rows 0..127 are gate columns, 128..255 up columns
    const uint32_t *codes0 = shared_tile ? j.sh.w0.codes : j.w0.codes;
    const uint32_t *codes1 = shared_tile ? (GLU ? j.sh.w1.codes : j.sh.w0.codes) : (GLU ? j.w1.codes : j.w0.codes);
    const bf16_t *scales0 = shared_tile ? j.sh.w0.scales : j.w0.scales;
    const bf16_t *scales1 = shared_tile ? (GLU ? j.sh.w1.scales : j.sh.w0.scales) : (GLU ? j.w1.scales : j.w0.scales);
    const bf16_t *biases0 = shared_tile ? j.sh.w0.biases : j.w0.biases;
    const bf16_t *biases1 = shared_tile ? (GLU ? j.sh.w1.biases : j.sh.w0.biases) : (GLU ? j.w1.biases : j.w0.biases);
    const int wout = shared_tile ? j.sh.w0.out : j.w0.out;
    const int wexp = shared_tile ? j.sh.w0.experts : j.w0.experts;
    auto weight_row = [&](int r) __attribute__((always_inline)) -> uint32_t {  // B row r of the tile -> row of the weight tensors
        const int col = min(n0 + (GLU ? (r % NCOLS) : r), j.N - 1);
        return (uint32_t)(g.e * wout + col);
    };
    // codes: units u = tid + G_THREADS i (i < 4) of a super-step, B row u / CU, 16-byte unit u % CU;
    // the unit sits at position (u % CU) ^ swz(row) of its row, so fragment reads are free of
    // bank conflicts; byte offsets are 32-bit (the tensors stay below 4 GiB, checked by the host)
    auto swz = [](int r) { return CU == 8 ? ((r & 7) ^ ((r >> 3) & 1)) : (((r >> 1) & 3) ^ ((r >> 3) & 1)); };
    constexpr int RPU = G_THREADS / CU;  // B rows covered by one unit index i
    const int cr = tid / CU, cu = tid % CU;
    const uint32_t coff0 = weight_row(cr) * (uint32_t)(K >> 1) + 16u * cu;
    const uint32_t coff1 = weight_row(cr + RPU) * (uint32_t)(K >> 1) + 16u * cu;
    // NCU = 4 / WM units per thread cover the 256 B rows: unit i is B row cr + RPU i, whose weight is
    // the gate (codes0) for rows below NCOLS and the up projection (codes1) above, under glu
    constexpr int NCU = 4 / WM;
    static_assert(CU == 4 && NCU * G_THREADS == G_BNB * CU, "code units must cover the B rows once");
    const uint32_t coff2 = NCU > 2 ? weight_row(cr + 2 * RPU) * (uint32_t)(K >> 1) + 16u * cu : 0u;
    const uint32_t coff3 = NCU > 2 ? weight_row(cr + 3 * RPU) * (uint32_t)(K >> 1) + 16u * cu : 0u;
    const int cdst = cr * CU + (cu ^ swz(cr));  // + RPU * CU i (swz(cr + RPU i) == swz(cr))
    // scales / biases of a chunk: units u = tid + G_THREADS i (i < 4 / WM): array u / 512, B row
    // (u / 2) % 256, 16-byte half u % 2; offsets are clamped inside the tensor (a partial last
    // chunk reads unused values)
    constexpr int NSB = 4 / WM;
    // unit i: array i / (NSB / 2) (scales, biases), B row (tid / 2) % 256 + 128 (i % (NSB / 2)) with
    // WM = 1, (tid / 2) with WM = 2; two row offsets serve all units (named registers: arrays
    // captured by the lambdas below would live in scratch)
    const int sr0 = (tid >> 1) & 255, sr1 = NSB > 2 ? sr0 + 128 : sr0;
    const uint32_t so0 = weight_row(sr0) * (uint32_t)groups + 8u * (tid & 1);  // in elements
    const uint32_t so1 = weight_row(sr1) * (uint32_t)groups + 8u * (tid & 1);
    const bool up0 = GLU && sr0 >= NCOLS, up1 = GLU && sr1 >= NCOLS;
    const int sd0 = (sr0 * G_KSC + 8 * (tid & 1)) / 8, sd1 = (sr1 * G_KSC + 8 * (tid & 1)) / 8;
    constexpr int SB_ARR = G_BNB * G_KSC / 8;  // uint4 per array
    const uint32_t slast = (uint32_t)wexp * (uint32_t)wout * (uint32_t)groups - 8u;
    struct ARegs {
        uint4 a0, a1;
    };
    uint4 rc0, rc1, rc2, rc3;  // codes of the next super-step
    uint4 rs0, rs1, rb0, rb1;  // scales and biases of the next chunk (rows sr0, sr1)
    auto load_a = [&](int ks, ARegs &r) __attribute__((always_inline)) {
        const uint4 *pa = (const uint4 *)(aptr + ks * BK);
        r.a0 = pa[0];
        r.a1 = pa[1];
    };
    auto load_codes = [&](int ss) __attribute__((always_inline)) {  // super-step ss (clamped by the caller)
        const uint32_t o = 32u * SS * (uint32_t)ss;
        rc0 = *(const uint4 *)((const char *)codes0 + coff0 + o);
        if (NCU > 2) {  // rows cr, cr + 64 gate; cr + 128, cr + 192 up
            rc1 = *(const uint4 *)((const char *)codes0 + coff1 + o);
            rc2 = *(const uint4 *)((const char *)codes1 + coff2 + o);
            rc3 = *(const uint4 *)((const char *)codes1 + coff3 + o);
        } else {        // rows cr gate, cr + 128 up
            rc1 = *(const uint4 *)((const char *)codes1 + coff1 + o);
        }
    };
    auto load_scales = [&](int ch) __attribute__((always_inline)) {  // chunk ch (clamped by the caller)
        const uint32_t o = (uint32_t)(ch * G_KSC);
        rs0 = *(const uint4 *)((up0 ? scales1 : scales0) + min(so0 + o, slast));
        rb0 = *(const uint4 *)((up0 ? biases1 : biases0) + min(so0 + o, slast));
        if (NSB > 2) {
            rs1 = *(const uint4 *)((up1 ? scales1 : scales0) + min(so1 + o, slast));
            rb1 = *(const uint4 *)((up1 ? biases1 : biases0) + min(so1 + o, slast));
        }
    };
    auto store_codes = [&](int ss) __attribute__((always_inline)) {
        uint4 *d = &Bc[ss & 1][cdst];
        d[0] = rc0;
        d[RPU * CU] = rc1;
        if (NCU > 2) {
            d[2 * RPU * CU] = rc2;
            d[3 * RPU * CU] = rc3;
        }
    };
    auto store_scales = [&](int ch) __attribute__((always_inline)) {
        uint4 *d = (uint4 *)&Sb[ch % SBUF][0][0][0];
        d[sd0] = rs0;
        d[SB_ARR + sd0] = rb0;
        if (NSB > 2) {
            d[sd1] = rs1;
            d[SB_ARR + sd1] = rb1;
        }
    };
    auto stage_a = [&](const ARegs &r, int ks) __attribute__((always_inline)) {
        const int kc = ks % G_KSC, par = (ks / G_KSC) & 1, buf = ks & 1;
        const uint4 pa0 = pair8(r.a0), pa1 = pair8(r.a1);
        *(uint4 *)&As[buf][ar * LDK + pw0] = pa0;
        *(uint4 *)&As[buf][ar * LDK + pw1] = pa1;
        float xs = 0.f;
        xs = dot2_(pa0.x, 0x3F803F80u, xs);
        xs = dot2_(pa0.y, 0x3F803F80u, xs);
        xs = dot2_(pa0.z, 0x3F803F80u, xs);
        xs = dot2_(pa0.w, 0x3F803F80u, xs);
        xs = dot2_(pa1.x, 0x3F803F80u, xs);
        xs = dot2_(pa1.y, 0x3F803F80u, xs);
        xs = dot2_(pa1.z, 0x3F803F80u, xs);
        xs = dot2_(pa1.w, 0x3F803F80u, xs);
        xs += dpp_f32<0xB1>(xs);
        xs += dpp_f32<0x4E>(xs);
        // exact three-way split by truncation: hi + mid + lo == xs
        const float hi = __uint_as_float(__float_as_uint(xs) & 0xFFFF0000u);
        const float r1 = xs - hi;
        const float mid = __uint_as_float(__float_as_uint(r1) & 0xFFFF0000u);
        const float lo = r1 - mid;
        if (q < 3) {
            const float v = q == 0 ? hi : (q == 1 ? mid : lo);
            Xs[par][q][ar][kc] = (bf16_t)(__float_as_uint(v) >> 16);
        }
        if (kc == 0 && nks - ks < G_KSC) {  // last chunk is partial: clear its unused columns
#pragma unroll
            for (int cc = 0; cc < G_KSC / 4; ++cc) {
                const int c = 4 * cc + q;
                if (c >= nks - ks) Xs[par][0][ar][c] = Xs[par][1][ar][c] = Xs[par][2][ar][c] = 0;
            }
        }
    };

    // ---- compute role: rows wm*64.., fragments ni at B rows bro[ni]
    const int wm = wave >> 2, wn = wave & 3;
    const int fr = lane & 31, fh = lane >> 5, fk = fh * 8;
    const bool active = wm * 64 < g.mrows;
    int bro[2];
    bro[0] = GLU ? wn * 32 : wn * 64;
    bro[1] = GLU ? NCOLS + wn * 32 : wn * 64 + 32;
    const int arow0 = wm * 64 + fr;
    uint32_t cm = 0x000F000Fu, cx = 0x43004300u;  // kept in VGPRs so and-or fuses
    asm volatile("" : "+v"(cm), "+v"(cx));
    f32x16_t acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mi][ni][i] = 0.f;

    auto compute = [&](int ks) __attribute__((always_inline)) {
        const int kc = ks % G_KSC, buf = ks & 1, sb = (ks / SS) & 1, par = (ks / G_KSC) & 1;
        const int sbb = (ks / G_KSC) % SBUF;
        const bf16_t *as = As[buf];
        uint4 cw[2];
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const int R = bro[ni] + fr, c = 2 * (ks % SS) + fh;
            cw[ni] = Bc[sb][R * CU + (c ^ swz(R))];
        }
        f32x16_t part[2][2];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            bf16x8_t a[2], b[2];
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) a[mi] = lds_frag(&as[(arow0 + mi * 32) * LDK + 16 * s + fk]);
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const uint32_t w = s == 0 ? cw[ni].x : s == 1 ? cw[ni].y : s == 2 ? cw[ni].z : cw[ni].w;
                b[ni] = __builtin_bit_cast(bf16x8_t, expand_codes(w, cm, cx));
            }
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int ni = 0; ni < 2; ++ni) {
                    if (s == 0) {
                        const f32x16_t z = {};
                        part[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mi], b[ni], z, 0, 0, 0);
                    } else {
                        part[mi][ni] =
                            __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mi], b[ni], part[mi][ni], 0, 0, 0);
                    }
                }
        }
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) {
            const float sc = bf2f(Sb[sbb][0][bro[ni] + fr][kc]);
#pragma unroll
            for (int mi = 0; mi < 2; ++mi)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[mi][ni][i] += sc * part[mi][ni][i];
        }
        if (kc == G_KSC - 1 || ks == nks - 1) {  // bias GEMM over the chunk's K steps
            bf16x8_t bv[2][2];
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const int R = bro[ni] + fr;
                const uint4 sv = *(const uint4 *)&Sb[sbb][0][R][fk];
                bv[ni][0] = lds_frag(&Sb[sbb][1][R][fk]);
                bv[ni][1] = __builtin_bit_cast(
                    bf16x8_t, make_uint4(neg128_pair(sv.x), neg128_pair(sv.y), neg128_pair(sv.z),
                                         neg128_pair(sv.w)));
            }
#pragma unroll
            for (int mi = 0; mi < 2; ++mi) {
                bf16x8_t xa[3];
#pragma unroll
                for (int tt = 0; tt < 3; ++tt) xa[tt] = lds_frag(&Xs[par][tt][arow0 + mi * 32][fk]);
#pragma unroll
                for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                    for (int u = 0; u < 2; ++u)
#pragma unroll
                        for (int tt = 0; tt < 3; ++tt)
                            acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xa[tt], bv[ni][u],
                                                                                  acc[mi][ni], 0, 0, 0);
            }
        }
    };

    // ---- pipeline (nks is a multiple of 4)
    const int nss = nks / SS, nch = (nks + G_KSC - 1) / G_KSC;
    ARegs ra0, ra1;
    load_codes(0);
    load_scales(0);
    load_a(0, ra0);
    load_a(1, ra1);
    store_codes(0);
    store_scales(0);
    load_codes(min(1, nss - 1));
    load_scales(min(1, nch - 1));
    stage_a(ra0, 0);
    load_a(2, ra0);
    lds_barrier();
    // K step k: compute k, stage k + 1 from `next` (loaded two steps ago), refill `next` with k + 3.
    // pf_a / pf_c (constants at each call) turn off the A / code prefetches of the last four steps,
    // which would load past the end: the epilogue would wait for them, and a wave keeps its slot
    // until its loads have returned.
    auto step = [&](int k, bool super_end, ARegs &next, bool pf_a, bool pf_c)
                    __attribute__((always_inline)) {
        if (active) compute(k);
        if (k + 1 < nks) {
            if (super_end) {  // next super-step: its codes were loaded one super-step ago
                store_codes((k + 1) / SS);
                if (pf_c) load_codes(min((k + 1) / SS + 1, nss - 1));
                if ((k + 1) % G_KSC == 0) {
                    if (SBUF == 1) lds_barrier();  // every wave is done with the chunk's scales
                    store_scales((k + 1) / G_KSC);
                    load_scales(min((k + 1) / G_KSC + 1, nch - 1));
                }
            }
            stage_a(next, k + 1);
        }
        if (pf_a) load_a(min(k + 3, nks - 1), next);
        lds_barrier();
    };
    int ks = 0;
    for (; ks + 4 < nks; ks += 4) {
        step(ks, SS == 1, ra1, true, true);
        step(ks + 1, SS <= 2, ra0, true, true);
        step(ks + 2, SS == 1, ra1, true, true);
        step(ks + 3, true, ra0, true, true);
    }
    // the last four steps (nks is a multiple of 8): only step nks - 4 still loads (A of nks - 1);
    // no chunk of scales starts inside them
    static_assert(SS <= 2, "the code prefetch of the last steps assumes super-steps of <= 2");
    step(ks, SS == 1, ra1, true, SS == 1);
    step(ks + 1, SS <= 2, ra0, false, false);
    step(ks + 2, SS == 1, ra1, false, false);
    step(ks + 3, true, ra0, false, false);
    if (!active) return;

    // epilogue: glu -> R(silu(R(gate)) * R(up)); else R(.) (+ bias: R(R(.) + b)). The output rows
    // of all 32 elements come first, in one batch of index loads (none without o_map): a load
    // inside each element's bounds check made every store wait for all outstanding memory
    // operations, the K loop's last prefetches included.
    int orow[2][16];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int i = 0; i < 16; ++i)
            orow[mi][i] = g.row0 + min(wm * 64 + mi * 32 + 8 * (i >> 2) + 4 * fh + (i & 3),
                                       g.mrows - 1);
    if (g.o_map) {
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int i = 0; i < 16; ++i) orow[mi][i] = (int)g.o_map[orow[mi][i]];
    }
    float bias_v[2] = {0.f, 0.f};  // R(.) + bias of the two column fragments (no glu)
    if (!GLU && j.bias) {
#pragma unroll
        for (int ni = 0; ni < 2; ++ni) bias_v[ni] = bf2f(j.bias[min(n0 + wn * 64 + ni * 32 + fr, j.N - 1)]);
    }
#pragma unroll
    for (int mi = 0; mi < 2; ++mi) {
        if (GLU) {
            const int col = n0 + wn * 32 + fr;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = wm * 64 + mi * 32 + 8 * (i >> 2) + 4 * fh + (i & 3);
                if (r < g.mrows && col < j.N) {
                    const float gt = rbf(acc[mi][0][i]), u = rbf(acc[mi][1][i]);
                    g.out[(size_t)orow[mi][i] * g.ldo + col] =
                        (bf16_t)f2bf((gt * sigmoidf_(gt)) * u);
                }
            }
        } else {
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const int col = n0 + wn * 64 + ni * 32 + fr;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int r = wm * 64 + mi * 32 + 8 * (i >> 2) + 4 * fh + (i & 3);
                    if (r < g.mrows && col < j.N) {
                        float v = acc[mi][ni][i];
                        if (j.bias) v = rbf(v) + bias_v[ni];
                        g.out[(size_t)orow[mi][i] * g.ldo + col] = (bf16_t)f2bf(v);
                    }
                }
            }
        }
    }
}

bool qgemm_supported(const GemmJob &j) {
    auto ok = [](const QW &w, int K) {
        // 16-byte units of codes and of scales per row; 32-bit byte offsets into the codes
        return w.codes && w.scales && w.biases && w.bits == 4 && w.group == 64 && K % 512 == 0 &&
               (size_t)w.experts * w.out * (size_t)(K / 2) < ((size_t)1 << 32);
    };
    if (j.bd || !ok(j.w0, j.K) || (j.glu && !ok(j.w1, j.K))) return false;
    if (j.has_shared && (!ok(j.sh.w0, j.sh.K) || (j.glu && !ok(j.sh.w1, j.sh.K)))) return false;
    return true;
}

// 64-row tiles (WM = 1). The kernel also builds with WM = 2 (128-row tiles of 512 threads, one
// workgroup per CU); measured at T = 4096 (experts averaging 128 rows) that was 12 % slower, so the
// launcher keeps WM = 1.
constexpr int G_WM = 1;

hipError_t launch_gemm(const GemmJob &j, hipStream_t stream) {
    if (qgemm_supported(j)) {
        constexpr int bm = 64 * G_WM;
        const int ncols = j.glu ? G_BNB / 2 : G_BNB;
        const int nblk = (j.N + ncols - 1) / ncols;
        const int s_tiles = j.has_shared ? (j.sh.M + bm - 1) / bm : 0;
        const int r_tiles = j.has_routing ? j.max_tiles : (j.M + bm - 1) / bm;
        const int tiles8 = (s_tiles + r_tiles + 8 * G_TG - 1) / (8 * G_TG) * (8 * G_TG);
        if (tiles8 == 0) return hipSuccess;
        const dim3 grid(tiles8 * nblk);
        if (j.glu) qgemm_kernel<true, G_WM, G_SS, G_SBUF><<<grid, 256 * G_WM, 0, stream>>>(j);
        else qgemm_kernel<false, G_WM, G_SS, G_SBUF><<<grid, 256 * G_WM, 0, stream>>>(j);
        return hipGetLastError();
    }
    if (j.has_shared) return hipErrorInvalidValue;  // only the kernel above takes shared tiles
    // routed tiles hold up to kGemmTileM rows: grid.z walks them in steps of BM
    const int tiles = j.has_routing ? j.max_tiles : (j.M + BM - 1) / BM;
    if (tiles <= 0) return hipSuccess;
    dim3 grid(tiles, (j.N + BN - 1) / BN, j.has_routing ? kGemmTileM / BM : 1);
    if (!j.bd) {
        // the gate/up pair shares one quantization
        if (j.glu && (j.w1.bits != j.w0.bits || j.w1.group != j.w0.group)) return hipErrorInvalidValue;
        const bool sub2 = j.w0.group == 32, b8 = j.w0.bits == 8;
        if (j.w0.bits == 16) {
            if (j.glu) gemm_kernel<16, true, 1><<<grid, 256, 0, stream>>>(j);
            else gemm_kernel<16, false, 1><<<grid, 256, 0, stream>>>(j);
            return hipGetLastError();
        }
        if (j.glu) {
            if (b8) {
                if (sub2) gemm_kernel<8, true, 2><<<grid, 256, 0, stream>>>(j);
                else gemm_kernel<8, true, 1><<<grid, 256, 0, stream>>>(j);
            } else {
                if (sub2) gemm_kernel<4, true, 2><<<grid, 256, 0, stream>>>(j);
                else gemm_kernel<4, true, 1><<<grid, 256, 0, stream>>>(j);
            }
        } else {
            if (b8) {
                if (sub2) gemm_kernel<8, false, 2><<<grid, 256, 0, stream>>>(j);
                else gemm_kernel<8, false, 1><<<grid, 256, 0, stream>>>(j);
            } else {
                if (sub2) gemm_kernel<4, false, 2><<<grid, 256, 0, stream>>>(j);
                else gemm_kernel<4, false, 1><<<grid, 256, 0, stream>>>(j);
            }
        }
    } else {
        gemm_kernel<0, false, 1><<<grid, 256, 0, stream>>>(j);
    }
    return hipGetLastError();
}

}  // namespace mrun
