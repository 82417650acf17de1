// Dense bf16 Linear on the matrix cores for prefill-sized inputs: the router and the shared
// expert's gate (Linear::forward with a dense weight, load.rs:294-306): y = R(x W^T), then
// R(y + bias). Both products read the same x, so they run as one launch (the gate is one more
// column block).
//
// Workgroup tile 64 rows x 64 columns, K steps of 64, v_mfma_f32_32x32x16_bf16. KG groups of 4
// waves split K into KG consecutive ranges; each group stages its own range through its own
// double-buffered LDS tiles (no operand is read twice), each wave of a group owns 32 x 32 of the
// tile, and at the end the groups' partial sums meet in LDS and are added in group order. The
// router's products are small (T x 257 outputs: a few hundred workgroups at most, one per CU),
// so the K steps wait on latency: the groups put KG waves on each SIMD and shorten the chain of
// dependent steps KG times. Each thread keeps NST K steps of loads in flight in registers (a ring
// unrolled by NST); one barrier per K step, which waits for LDS only, so the loads stay in flight
// across it. A step issues its MFMAs first and then stages the next step's tile, so the matrix
// cores run while the stores and the barrier wait.
//
// With pack_a set, extra workgroups of the launch (column blocks past the product's, one per row
// block and quarter of K) write A in the grouped GEMM's packed layout with launch_apack's code, bit
// for bit. They run beside the product on the CUs it leaves idle; folded into the product's own
// staging, their stores would share the load counter and every K step would wait for all loads.
#include <type_traits>

#include "apack.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace mrun {

namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;

// K quarters of the packing workgroups: 4 when the quarters hold whole 64-wide groups
__host__ __device__ inline int dense_pack_quarters(int K) { return K % 256 == 0 ? 4 : 1; }
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;

constexpr int DBM = 64, DBN = 64, DBK = 64, DLDK = DBK + 8;

struct Stage {
    uint4 a0, a1, b0, b1;
};

template <int NST, int KG>
__global__ __launch_bounds__(256 * KG) void dense_gemm_kernel(DenseJob j) {
    // per group: A and B tiles, double-buffered; after the K loop the first KG - 1 groups' 4 x 64
    // x 16 partial sums reuse the space (KG - 1 groups x 16 KB <= KG x 36 KB)
    __shared__ __align__(16) bf16_t stage_lds[KG][2][2][DBM * DLDK];
    const int kg = threadIdx.x >> 8, tid = threadIdx.x & 255, lane = tid & 63, wave = tid >> 6;
    bf16_t(*As)[DBM * DLDK] = stage_lds[kg][0];
    bf16_t(*Bs)[DBN * DLDK] = stage_lds[kg][1];
    if (j.zero && blockIdx.x == 0 && blockIdx.y == 0)
        for (int i = threadIdx.x; i < j.n_zero; i += 256 * KG) j.zero[i] = 0;

    // column block -> weight (W0's blocks first, then W1's, then the packing blocks)
    const int nb0 = (j.N0 + DBN - 1) / DBN;
    const int nbw = nb0 + (j.W1 ? (j.N1 + DBN - 1) / DBN : 0);
    if ((int)blockIdx.y >= nbw) {  // pack rows [64 x, +64) of K quarter y - nbw (apack's code)
        const int nq = dense_pack_quarters(j.K), kq = (int)blockIdx.y - nbw;
        const int bpr = j.K / nq / 8, r0 = (int)blockIdx.x * DBM;  // blocks per row and quarter
        // every thread takes the same number of blocks (DBM * bpr is a multiple of 512, since
        // bpr is a multiple of 8), so whole 64-lane waves take part in each DPP sum; rows past M
        // are clamped for the loads and skipped for the stores. The loads of PB blocks are issued
        // before any is used: one round trip per PB blocks, not one per block.
        constexpr int PB = 8;
        const int step = 256 * KG;
        for (int i0 = threadIdx.x; i0 < DBM * bpr; i0 += PB * step) {
            uint4 v[PB];
#pragma unroll
            for (int u = 0; u < PB; ++u) {
                const int i = min(i0 + u * step, DBM * bpr - 1);
                const int row = r0 + i / bpr, blk = kq * bpr + i % bpr;
                v[u] = *(const uint4 *)(j.A + (size_t)min(row, j.M - 1) * j.lda + (size_t)blk * 8);
            }
#pragma unroll
            for (int u = 0; u < PB; ++u) {
                const int i = i0 + u * step;
                if (i >= DBM * bpr) break;  // uniform: the same count for every thread
                const int row = r0 + i / bpr, blk = kq * bpr + i % bpr;
                pack_block_v(v[u], min(row, j.M - 1), row < j.M, j.K, blk, j.pack_a, j.K, j.pack_x);
            }
        }
        return;
    }
    const bool second = (int)blockIdx.y >= nb0;
    const bf16_t *W = second ? j.W1 : j.W0;
    const bf16_t *bias = second ? j.bias1 : j.bias0;
    const int N = second ? j.N1 : j.N0;
    bf16_t *out = second ? j.out1 : j.out0;
    const int ldo = second ? j.ldo1 : j.ldo0;
    const int n0 = (second ? (int)blockIdx.y - nb0 : (int)blockIdx.y) * DBN;
    const int row0 = blockIdx.x * DBM;
    const int mrows = min(DBM, j.M - row0);
    const int K = j.K, nks = K / DBK / KG;  // K steps of each group (K a multiple of 64 KG)

    // staging: row tid / 4, 16 elements from k = 16 (tid % 4); rows past the end load the last
    // row (never stored)
    const int sr = tid >> 2, sk = (tid & 3) * 16;
    const bf16_t *ap = j.A + (size_t)(row0 + min(sr, mrows - 1)) * j.lda + sk + kg * nks * DBK;
    const bf16_t *bp = W + (size_t)min(n0 + sr, N - 1) * K + sk + kg * nks * DBK;
    // stages pass by value (a reference into them would put the ring in scratch)
    auto load = [&](int ks) __attribute__((always_inline)) -> Stage {
        const uint4 *pa = (const uint4 *)(ap + ks * DBK), *pb = (const uint4 *)(bp + ks * DBK);
        return Stage{pa[0], pa[1], pb[0], pb[1]};
    };
    auto store = [&](int ks, Stage st) __attribute__((always_inline)) {
        bf16_t *a = &As[ks & 1][sr * DLDK + sk], *b = &Bs[ks & 1][sr * DLDK + sk];
        *(uint4 *)a = st.a0, *(uint4 *)(a + 8) = st.a1;
        *(uint4 *)b = st.b0, *(uint4 *)(b + 8) = st.b1;
    };

    const int wm = wave >> 1, wn = wave & 1, fr = lane & 31, fk = (lane >> 5) * 8;
    f32x16_t acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    auto compute = [&](int ks) __attribute__((always_inline)) {
        const bf16_t *a = &As[ks & 1][(wm * 32 + fr) * DLDK + fk];
        const bf16_t *b = &Bs[ks & 1][(wn * 32 + fr) * DLDK + fk];
#pragma unroll
        for (int s = 0; s < 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(bf16x8_t, *(const uint4 *)(a + 16 * s)),
                __builtin_bit_cast(bf16x8_t, *(const uint4 *)(b + 16 * s)), acc, 0, 0, 0);
    };
    // ring slot i holds the loads of the steps = i (mod NST). Step ks (its tile in LDS buffer
    // ks & 1) issues its MFMAs, then stores step ks + 1's loads into the other buffer and refills
    // their slot with step ks + 1 + NST (clamped: the tail reloads a valid step), then the barrier.
    Stage ring[NST];
#pragma unroll
    for (int i = 0; i < NST; ++i) ring[i] = load(min(i, nks - 1));
    store(0, ring[0]);
    ring[0] = load(min(NST, nks - 1));
    lds_barrier();
    auto step = [&](int ks, auto ic) __attribute__((always_inline)) {
        constexpr int I1 = (decltype(ic)::value + 1) % NST;  // slot of step ks + 1
        compute(ks);
        if (ks + 1 < nks) {
            store(ks + 1, ring[I1]);
            ring[I1] = load(min(ks + 1 + NST, nks - 1));
        }
        lds_barrier();
    };
    int ks = 0;
    for (; ks + NST <= nks; ks += NST) {
        step(ks, std::integral_constant<int, 0>{});
        if constexpr (NST > 1) step(ks + 1, std::integral_constant<int, 1>{});
        if constexpr (NST > 2) step(ks + 2, std::integral_constant<int, 2>{});
        static_assert(NST <= 3, "ring of at most 3 steps");
    }
    if (ks < nks) step(ks, std::integral_constant<int, 0>{});
    if constexpr (NST > 2)
        if (ks + 1 < nks) step(ks + 1, std::integral_constant<int, 1>{});

    if (KG > 1) {  // group g > 0 leaves its sums in LDS; group 0 adds them in group order
        float *red = (float *)&stage_lds[0][0][0][0];
        __syncthreads();
        if (kg > 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) red[(((kg - 1) * 4 + wave) * 16 + i) * 64 + lane] = acc[i];
        }
        __syncthreads();
        if (kg > 0) return;
#pragma unroll
        for (int g = 0; g < KG - 1; ++g)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] += red[((g * 4 + wave) * 16 + i) * 64 + lane];
    }
    const int col = n0 + wn * 32 + fr;
    const float bv = (bias && col < N) ? bf2f(bias[col]) : 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int r = wm * 32 + 8 * (i >> 2) + 4 * (lane >> 5) + (i & 3);
        if (r < mrows && col < N) {
            float v = rbf(acc[i]);
            if (bias) v = rbf(v + bv);
            out[(size_t)(row0 + r) * ldo + col] = (bf16_t)f2bf(v);
        }
    }
}

}  // namespace

bool dense_gemm_supported(int M, int K) { return M > 16 && K % DBK == 0 && K >= DBK; }

// K groups of the launch: 2 measured best in the configs[2] prefill (router stage 18.0 against
// 19.3 us with 1 group, 19.2 and 20.6 with 4 groups of 2- and 3-step rings) and with x in the
// last-level cache (10.9 against 11.8 us, 4 groups 10.8); the steps wait on load latency, which
// more waves per SIMD shorten only a little.
constexpr int kDenseKG = 2;

hipError_t launch_dense_gemm(const DenseJob &j, hipStream_t stream) {
    if (!dense_gemm_supported(j.M, j.K) || j.N0 <= 0 || (j.W1 && j.N1 <= 0))
        return hipErrorInvalidValue;
    int nb = (j.N0 + DBN - 1) / DBN + (j.W1 ? (j.N1 + DBN - 1) / DBN : 0);
    if (j.pack_a) nb += dense_pack_quarters(j.K);
    dim3 grid((j.M + DBM - 1) / DBM, nb);
    // a deeper ring (4, 6, 8 steps) measured no faster
    if (j.K % (DBK * kDenseKG) == 0)
        dense_gemm_kernel<3, kDenseKG><<<grid, 256 * kDenseKG, 0, stream>>>(j);
    else dense_gemm_kernel<3, 1><<<grid, 256, 0, stream>>>(j);
    return hipGetLastError();
}

}  // namespace mrun
