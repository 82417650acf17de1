// The prefill forward's expert products on the matrix cores (gfx950 v_mfma_f32_32x32x16_bf16):
// SwitchGlu's gate/up with SwiGLU, and down (moe.rs:79-83; gather_qmm with sorted indices,
// nuvec.rs:670-686), with the shared expert's products as extra tiles of the same launches.
//
// The affine dequant is folded around the MFMA. A code q sits in the low mantissa bits of bf16
// 128.0 (0x4300 | q == 128 + q exactly), so one and-or turns a code word into the B operand; the
// MFMA chain over one quant group (64 k) gives P' = sum x (128 + q) in f32, and the group enters
// the result as  s * P' + (b - 128 s) * X  with X = sum x over the group. No weight is rounded.
//
// Operand layout (prepared once per row, outside the K loop):
//  - A rows are "packed": in each 64-wide group the eight 8-element k blocks are stored in the
//    order the MFMA fragments read them (block 4h + s at position 2s + h: K sub-step s, lane half
//    h) and each block is re-paired (x0, x4, x1, x5, x2, x6, x3, x7) to match the code expansion
//    (dword i of an expanded word holds codes i and i + 4). The GEMM copies A into LDS unchanged.
//  - X is stored split exactly into three bf16 (hi + mid + lo == X, truncation) per group:
//    XS [rows][3][K / 64]. apack_kernel writes those of x; the gate/up epilogue those of act (the
//    two waves covering a 64-column group add their half sums, handed over through LDS).
//  - The bias term  sum_g X_g (b_g - 128 s_g)  is a small MFMA product per tile: K entries of
//    X splits against b (lane half 0) and -128 s (lane half 1; exact), 3 MFMAs per 8 entries.
//
// Schedule: persistent workgroups (two per CU, 4 waves) walk a list of items (64-row tile x
// column block of 256 B rows; under glu 128 gate + 128 up rows). The list is cut into eight
// contiguous segments, one per XCD (the hardware deals workgroup L to XCD L % 8), so the column
// blocks of a row tile run side by side on one XCD and share its L2 for the A rows. The K steps
// of consecutive items form one stream: A and codes go from global memory straight into LDS
// (global_load_lds, no VGPRs, no VALU), four K steps in flight, the next item's first steps
// loading during this item's epilogue. Each wave owns 64 rows x 64 B rows (2 x 2 fragments) and
// per K step issues 16 MFMAs, expands 8 code words and applies the group scale with 64 FMAs.
// LDS reads are inline ds_read with explicit lgkmcnt waits, and the DMA waits are explicit
// vmcnt counts, so the compiler inserts no wait of its own on the LDS that the DMA fills.
#include <type_traits>

#include "apack.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace mrun {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 mg_bf16x8;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float mg_f32x16;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;

namespace mg {
constexpr int BM = 64, BK = 64, BNR = 256, NT = 256;
constexpr int KS = 2;                          // K steps per LDS stage
constexpr int NSTG = 2;                        // stages in the ring
constexpr int A_STEP = BM * BK * 2;            // one K step of A: 64 rows x 128 B
constexpr int A_BYTES = KS * A_STEP;
constexpr int C_BYTES = BNR * 32 * KS;         // codes of a stage: 256 B rows x 64 B
constexpr int STAGE = A_BYTES + C_BYTES;       // 32 KB
constexpr int S_BYTES = BNR * 16;              // scales of 8 groups per B row
constexpr int R_BYTES = BM * 4;                // A rows (tokens) of a routed tile
constexpr int T_BYTES = 256;                   // a routed tile's record (copied as 64 dwords)
constexpr int X_BYTES = BM * 3 * 16;           // bias term: X splits of 8 entries per row
constexpr int B_BYTES = BNR * 16;              // bias term: biases of 8 groups per B row
constexpr int OFF_S = NSTG * STAGE, OFF_R = OFF_S + 2 * S_BYTES, OFF_T = OFF_R + 2 * R_BYTES;
constexpr int OFF_X = OFF_T + 2 * T_BYTES;
constexpr int OFF_B = OFF_X + X_BYTES;
constexpr int LDS_BYTES = OFF_B + B_BYTES;     // 81,920: two workgroups per CU
static_assert(LDS_BYTES <= 81920, "two workgroups per CU");
}  // namespace mg

__device__ __forceinline__ uint32_t lds_offset(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)p;
}
// An LDS read whose wait comes later (an lgkmcnt asm taking the destination as "+v"). The compiler
// takes the destination as written at issue, so any copy or spill of it before the wait would read
// a register the load has not yet filled: the kernels that use it must build without VGPR spills
// (tests/test_isa.py checks the built code for both).
template <int OFF>
__device__ __forceinline__ u32x4 ds_read16(uint32_t a) {
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
    return v;
}
// Reads whose results become addresses or counts: the reads and their wait are one statement, so
// that no copy or spill of a destination register can come between a read and its arrival.
__device__ __forceinline__ void ds_read3_now(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t &v0,
                                             uint32_t &v1, uint32_t &v2) {
    asm volatile("ds_read_b32 %0, %3\n\tds_read_b32 %1, %4\n\tds_read_b32 %2, %5\n\ts_waitcnt lgkmcnt(0)"
                 : "=&v"(v0), "=&v"(v1), "=&v"(v2)
                 : "v"(a0), "v"(a1), "v"(a2));
}
// Global memory goes to LDS through buffer loads (buffer_load ... lds): a raw resource per
// tensor (base address in scalar registers), a per-lane 32-bit byte offset and a scalar one, so
// that no per-lane 64-bit address arithmetic is needed. 16 (or 4) bytes per lane land at
// lds + 16 * lane (4 * lane); the LDS address is the same for the whole wave.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t rsrc_of(const void *p, uint32_t bytes = 0xFFFFFFFFu) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void dma16(rsrc_t r, uint32_t voff, uint32_t soff, char *lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)lds, 16, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma4(rsrc_t r, uint32_t voff, uint32_t soff, char *lds) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)lds, 4, voff, soff, 0, 0);
}
// Wait until at most N of this wave's global loads are outstanding, then a workgroup barrier.
template <int N>
__device__ __forceinline__ void vm_wait_barrier() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"i"(N) : "memory");
}

// a code word (8 codes) into the bf16 pairs (128 + q_i, 128 + q_{i+4}), in two halves
__device__ __forceinline__ void mg_expand_lo(u32x4 &r, uint32_t w, uint32_t cm, uint32_t cx) {
    r.x = (w & cm) | cx;
    r.y = ((w >> 4) & cm) | cx;
}
__device__ __forceinline__ void mg_expand_hi(u32x4 &r, uint32_t w, uint32_t cm, uint32_t cx) {
    r.z = ((w >> 8) & cm) | cx;
    r.w = ((w >> 12) & cm) | cx;
}

// -128 s for a pair of bf16 scales (exact: a power-of-two scaling)
__device__ __forceinline__ uint32_t mg_neg128(uint32_t w) {
    const uint32_t lo = __float_as_uint(-128.f * bf_lo(w)) >> 16;
    const uint32_t hi = __float_as_uint(-128.f * bf_hi(w)) & 0xFFFF0000u;
    return lo | hi;
}

// ---------------------------------------------------------------------------------------------
// A packing: x [rows][K] (row stride lda) -> packed rows [rows][K] (stride ldp) and the X splits
// [rows][3][K / 64]. One thread per 8-element block; the 8 threads of a group are adjacent lanes.

__global__ __launch_bounds__(256) void apack_kernel(const bf16_t *__restrict__ x, int lda, int rows,
                                                    int K, bf16_t *__restrict__ xp, int ldp,
                                                    bf16_t *__restrict__ xs) {
    const int nb = K / 8;
    const long long b = (long long)blockIdx.x * 256 + threadIdx.x;
    if (b >= (long long)rows * nb) return;  // whole groups only: rows * nb is a multiple of 8
    pack_block(x, lda, (int)(b / nb), true, K, (int)(b % nb), xp, ldp, xs);
}

hipError_t launch_apack(const bf16_t *x, int lda, int rows, int K, bf16_t *xp, int ldp,
                        bf16_t *xs, hipStream_t stream) {
    const long long n = (long long)rows * (K / 8);
    if (n == 0) return hipSuccess;
    apack_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(x, lda, rows, K, xp, ldp, xs);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------
// the grouped GEMM

// A value the whole wave holds, moved to a scalar register: integer divisions by runtime values
// run on the VALU, and without this the compiler would treat their results (and the loads and
// branches that depend on them) as per-lane.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
// A pointer the whole wave holds, in scalar registers (so that a per-lane choice between two such
// pointers is a select of values, not a per-lane load of the kernel argument holding them).
template <class T>
__device__ __forceinline__ const T *unip(const T *p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const T *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

// LDS swizzles (16-byte units). A rows are 128 B (8 units): rows r and r + 8 (same bank window
// at 256 B per cycle) and rows of one parity in 16 get distinct masks. B rows are 64 B (4 units,
// two K steps of codes): the 4 rows of a 256-byte window... rows r, r + 4, r + 8, r + 12 (which
// share a position in a 256-byte window) get distinct masks, and so do r, r + 2, r + 4, r + 6
// (a 128-byte window).
__device__ __forceinline__ int swz_a(int r) { return (r & 7) ^ ((r >> 3) & 1); }
__device__ __forceinline__ int swz_c(int r) { return ((r >> 2) ^ (r >> 1)) & 3; }

// The tile row whose act column sum lane `l` holds after the gate/up epilogue's reduce-scatter:
// with fr = l % 32, bit 4 of fr chose the row fragment (32 rows), bits 3-2 the 8-row block,
// bits 1-0 the row in a block of 4, and the lane half (l / 32) the block of 4 within 8 (the
// MFMA's C layout: value i of lane l is row 8 (i / 4) + 4 (l / 32) + i % 4 of its fragment).
__device__ __forceinline__ int xrow_of(int l) {
    const int fr = l & 31;
    return 32 * (fr >> 4) + 8 * ((fr >> 2) & 3) + 4 * (l >> 5) + (fr & 3);
}

// HALF: tiles of at most 32 rows (the batch's routed tiles cut to 32 rows, the shared expert's
// rows in tiles of 32): the second row fragment's MFMAs, scale FMAs, bias term and epilogue are
// left out, and so are the copies of A rows 32-63 (their LDS fragment reads stay, unused, so
// every LDS wait count is the same in both instantiations).
template <bool GLU, bool HALF = false>
__global__ __launch_bounds__(mg::NT, 2) void moe_gemm_kernel(MoeGemmJob j) {
    using namespace mg;
    __shared__ __align__(16) char smem[LDS_BYTES];
    const int tid = threadIdx.x, lane = tid & 63, wave = uni(tid >> 6);
    const int fr = lane & 31, fh = lane >> 5;
    const uint32_t lds0 = lds_offset(smem);
    char *const rowbuf = smem + OFF_R;

    constexpr int NCOLS = GLU ? 128 : 256;
    const int NB = j.N / NCOLS;
    constexpr int TM = HALF ? 32 : BM;  // rows per tile
    constexpr int NMI = HALF ? 1 : 2;   // row fragments of 32 rows
    const int s_tiles = j.has_shared ? (j.sh.M + TM - 1) / TM : 0;
    const int r_tiles =
        j.has_routing ? min((int)*j.routing.n_tiles, j.max_tiles) : (j.M + TM - 1) / TM;
    const int total = (s_tiles + r_tiles) * NB;
    const int G8 = (int)(gridDim.x >> 3), xcd = (int)(blockIdx.x & 7), slot = (int)(blockIdx.x >> 3);
    const int seg_lo = (int)((long long)total * xcd / 8);
    const int seg_hi = (int)((long long)total * (xcd + 1) / 8);
    const int n_items = uni(seg_hi - seg_lo > slot ? (seg_hi - seg_lo - slot + G8 - 1) / G8 : 0);
    if (n_items == 0) return;
    const int K = j.K, nks = K / BK, G = K / 64;
    const int total_steps = n_items * nks;  // a multiple of 8

    // item n of this workgroup: (row tile, column block); shared tiles come first
    struct Item {
        int e, row0, mrows, n0, tile;  // tile: routed tile index (rows from the table), or -1
        bool sh;
    };
    // item n's row tile (shared tiles first) and column block
    auto item_pos = [&](int n, int &rt, int &cb) __attribute__((always_inline)) {
        const int i = seg_lo + slot + G8 * n;
        rt = uni(i / NB), cb = i - rt * NB;
    };
    // A routed tile's record (expert, first row, rows) and token rows reach LDS through copies
    // that wave 0 issues one item ahead (fetch_rows), into slot n % 2: no scalar-cache miss and
    // no wait on a global load at an item switch.
    auto item_of = [&](int n) __attribute__((always_inline)) {
        int rt, cb;
        item_pos(n, rt, cb);
        Item it;
        it.n0 = cb * NCOLS;
        if (rt < s_tiles) {
            it.sh = true, it.e = 0, it.row0 = rt * TM, it.mrows = min(TM, j.sh.M - it.row0);
            it.tile = -1;
        } else {
            it.sh = false;
            const int r = rt - s_tiles;
            if (j.has_routing) {
                const uint32_t rec = lds0 + OFF_T + (uint32_t)(n & 1) * T_BYTES;
                uint32_t e, row0, mrows;
                ds_read3_now(rec, rec + 4, rec + 8, e, row0, mrows);
                it.e = uni((int)e), it.row0 = uni((int)row0), it.mrows = uni((int)mrows);
                it.tile = j.tile_rows ? r : -1;
            } else {
                it.e = 0, it.row0 = r * TM, it.mrows = min(TM, j.M - it.row0), it.tile = -1;
            }
        }
        return it;
    };

    // ---- load role: A rows ra, ra + 32 (16-byte unit ua), B rows rb, rb + 128 (unit uc), scale
    // row tid. Units are XOR-swizzled (swz_a, swz_c) so that the 16-byte fragment reads of 16
    // adjacent lanes fall on distinct 16-byte bank groups of a 256-byte window, and those of 8
    // adjacent lanes on distinct ones of a 128-byte window.
    const int ra = wave * 8 + (lane >> 3);
    const uint32_t ua16 = 16u * (uint32_t)((lane & 7) ^ swz_a(ra));
    // codes: copy i moves B rows 64 i + 16 wave + lane / 4, 16-byte unit lane % 4 of each
    const int rb = 16 * wave + (lane >> 2);
    const uint32_t uc16 = 16u * (uint32_t)((lane & 3) ^ swz_c(rb));  // swz_c(rb + 64 i) == swz_c(rb)
    // the item's sources and this lane's byte offsets in them
    rsrc_t r_a, r_c0, r_c1, r_s;
    uint32_t la0 = 0, la1 = 0, lc[4] = {0u, 0u, 0u, 0u}, ls = 0;
    int l_item = 0, l_ks = 0;
    Item li{};     // the load cursor's item, taken over by the compute cursor at its switch
    int lx = 0;    // the load cursor's A row of tile row `lane` (the bias term's X splits)

    // the A rows (tokens) of tile rows r0, r1, r2 of item n
    auto a_rows = [&](const Item &it, int n, int r0, int r1, int r2, int &v0, int &v1, int &v2)
                      __attribute__((always_inline)) {
        r0 = min(r0, it.mrows - 1), r1 = min(r1, it.mrows - 1), r2 = min(r2, it.mrows - 1);
        if (it.tile >= 0) {
            const uint32_t rb = lds0 + OFF_R + (uint32_t)(n & 1) * R_BYTES;
            uint32_t u0, u1, u2;
            ds_read3_now(rb + 4 * r0, rb + 4 * r1, rb + 4 * r2, u0, u1, u2);
            v0 = (int)u0, v1 = (int)u1, v2 = (int)u2;
        } else {
            v0 = it.row0 + r0, v1 = it.row0 + r1, v2 = it.row0 + r2;
        }
    };
    // copy item n's tile record and token rows into LDS slot n % 2 (wave 0; routed tiles)
    auto fetch_rows = [&](int n) __attribute__((always_inline)) {
        if (n >= n_items || wave != 0 || !j.has_routing) return;
        int rt, cb;
        item_pos(n, rt, cb);
        if (rt < s_tiles) return;
        const int r = rt - s_tiles;
        dma4(rsrc_of(j.routing.tiles, 12u * (uint32_t)j.max_tiles), 4u * (uint32_t)lane,
             12u * (uint32_t)r, smem + OFF_T + (n & 1) * T_BYTES);
        // 64 entries from tile r's first (those past the table read as 0: its resource's size)
        if (j.tile_rows)
            dma4(rsrc_of(j.tile_rows, 4u * (uint32_t)j.max_tiles * (uint32_t)TM),
                 4u * (uint32_t)lane, 4u * (uint32_t)(r * TM), rowbuf + (n & 1) * R_BYTES);
    };
    auto setup_load = [&](int n) __attribute__((always_inline)) {
        const Item it = item_of(n);
        int r0, r1, x0;
        a_rows(it, n, ra, ra + 32, lane, r0, r1, x0);
        li = it, lx = x0;
        const int lda = it.sh ? j.sh.lda : j.lda;
        r_a = rsrc_of(it.sh ? j.sh.A : j.A);
        la0 = (uint32_t)r0 * (uint32_t)lda * 2u + ua16;
        la1 = (uint32_t)r1 * (uint32_t)lda * 2u + ua16;
        r_c0 = rsrc_of(it.sh ? j.sh.w0.codes : j.w0.codes);
        r_c1 = GLU ? rsrc_of(it.sh ? j.sh.w1.codes : j.w1.codes) : r_c0;
        const uint32_t wrow = (uint32_t)it.e * (uint32_t)(it.sh ? j.sh.w0.out : j.w0.out);
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // under glu, rows 0-127 are gate (w0), 128-255 up (w1)
            const int R = 64 * i + rb;
            const uint32_t col = (uint32_t)(it.n0 + (GLU ? (R & 127) : R));
            lc[i] = (wrow + col) * (uint32_t)(K / 2) + uc16;
        }
        const bool up = GLU && wave >= 2;  // waves 2, 3 load the up rows' scales
        r_s = rsrc_of(up ? (it.sh ? j.sh.w1.scales : j.w1.scales) : (it.sh ? j.sh.w0.scales : j.w0.scales));
        ls = (wrow + (uint32_t)(GLU ? it.n0 + (tid & 127) : it.n0 + tid)) * (uint32_t)G * 2u;
        fetch_rows(n + 1);  // one item ahead
    };
    // issue the DMA of global step gl (the load cursor's item and K step) into ring stage ST
    // copy `part` of the load cursor's stage (its item, K steps l_ks, l_ks + 1) into ring slot
    // SLOT: parts 0-3 A (K step part / 2, rows ra + 32 (part % 2)), parts 4-7 codes copy part - 4
    auto issue_part = [&](int part, auto slot_c) __attribute__((always_inline)) {
        constexpr int SLOT = decltype(slot_c)::value;
        char *sa = smem + SLOT * STAGE, *sc = sa + A_BYTES;
        if (part < 4) {
            if (HALF && (part & 1)) return;  // A rows 32-63: no MFMA of a 32-row tile reads them
            const int kk = part >> 1;
            dma16(r_a, (part & 1) ? la1 : la0, 128u * (l_ks + kk),
                  sa + kk * A_STEP + (part & 1) * 4096 + wave * 1024);
        } else {
            const int i = part - 4;
            dma16(GLU && i >= 2 ? r_c1 : r_c0, lc[i], 32u * l_ks, sc + i * 4096 + wave * 1024);
        }
    };
    // the scale chunk of K steps l_ks .. l_ks + 7 (global K step gl): items have a multiple of 8 K
    // steps, so a chunk starts with a ring slot 0 stage
    auto issue_scales = [&](int gl) __attribute__((always_inline)) {
        dma16(r_s, ls, 2u * l_ks, smem + OFF_S + ((gl >> 3) & 1) * S_BYTES + wave * 1024);
    };
    // the load cursor's next stage (and item)
    auto advance = [&]() __attribute__((always_inline)) {
        l_ks += KS;
        if (l_ks == nks) {
            l_ks = 0;
            if (++l_item < n_items) setup_load(l_item);
        }
    };

    // ---- compute role: rows mi * 32 + fr, B rows bro[ni] + fr
    uint32_t a_off[4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
        a_off[s] = lds0 + (uint32_t)(fr * 128 + 16 * ((2 * s + fh) ^ swz_a(fr)));
    const int bro0 = GLU ? wave * 32 : wave * 64, bro1 = GLU ? 128 + wave * 32 : wave * 64 + 32;
    // code words of fragment ni at K step kk of a stage: unit 2 kk + fh of B row bro + fr
    uint32_t c_addr[2][2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
        const uint32_t off = (uint32_t)(fr * 64 + 16 * ((2 * kk + fh) ^ swz_c(fr)));
        c_addr[0][kk] = lds0 + A_BYTES + (uint32_t)bro0 * 64 + off;
        c_addr[1][kk] = lds0 + A_BYTES + (uint32_t)bro1 * 64 + off;
    }
    const uint32_t s_addr0 = lds0 + OFF_S + (uint32_t)(bro0 + fr) * 16;
    const uint32_t s_addr1 = lds0 + OFF_S + (uint32_t)(bro1 + fr) * 16;
    uint32_t cm = 0x000F000Fu, cx = 0x43004300u;  // in VGPRs, so that and-or fuses
    asm volatile("" : "+v"(cm), "+v"(cx));

    mg_f32x16 acc[2][2];
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int ni = 0; ni < 2; ++ni)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mi][ni][i] = 0.f;

    // ---- prologue: rows of item 0, then the first stage
    fetch_rows(0);
    vm_wait_barrier<0>();
    setup_load(0);
    issue_scales(0);
    for (int part = 0; part < 8; ++part) issue_part(part, std::integral_constant<int, 0>{});
    advance();

    Item ci{};     // the compute cursor's item
    int xrow = 0;  // A row of tile row `lane` (the bias term's X splits)
    bool no_bias = false;
    int cn = 0, ks = -1;  // the compute cursor's item and K step
    u32x4 sch0 = {0u, 0u, 0u, 0u}, sch1 = sch0;  // scales of the current 8-step chunk
    mg_f32x16 part0[2], part1[2];  // the K step's group products P' of fragments 0 and 1
    float sc_pend = 0.f;           // scale still to apply to part1
#pragma unroll
    for (int mi = 0; mi < 2; ++mi)
#pragma unroll
        for (int i = 0; i < 16; ++i) part0[mi][i] = part1[mi][i] = 0.f;

    // The gate/up epilogue's group sums of act: the odd wave of each pair writes its half sums to
    // LDS after the next stage's barrier (every wave is then done with the bias operands there),
    // the even wave adds them to its own after the barrier that follows and stores the splits.
    // x_state: 0 nothing pending, 1 the write, 2 the read.
    int x_state = 0;
    float x_pend = 0.f;
    bf16_t *x_dst = nullptr;  // this lane's row entry, or null past the tile's rows
    const int x_oxe = j.N / 64;
    const uint32_t x_slot = lds0 + OFF_X + 256u * (uint32_t)(wave >> 1) + 4u * (uint32_t)lane;
    auto x_write = [&]() __attribute__((always_inline)) {
        if (wave & 1) {
            asm volatile("ds_write_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" ::"v"(x_slot), "v"(x_pend)
                         : "memory");
        }
        x_state = 2;
    };
    auto x_read_store = [&]() __attribute__((always_inline)) {
        if (!(wave & 1)) {
            uint32_t o;
            asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(o) : "v"(x_slot));
            if (x_dst) {
                uint32_t hi, mid, lo;
                split3(x_pend + __uint_as_float(o), hi, mid, lo);
                x_dst[0] = (bf16_t)hi;
                x_dst[x_oxe] = (bf16_t)mid;
                x_dst[2 * x_oxe] = (bf16_t)lo;
            }
        }
        x_state = 0;
    };

    auto step = [&](int gs, auto st_c) __attribute__((always_inline)) {
        constexpr int ST = decltype(st_c)::value;
        if (++ks == nks) ks = 0, ++cn;
        // K steps ST = 0, 1 read ring slot 0, ST = 2, 3 slot 1. A stage starts at even ST: its
        // copies (issued during the previous stage) must have landed, and every wave must be done
        // with the slot that the next stage's copies, issued between this K step's MFMAs, fill.
        constexpr int SLOT = ST >> 1;
        constexpr bool SS = (ST & 1) == 0;
        // After the last stage the copies go on, in bounds (the load cursor stays on the last
        // item), into the slot that is no longer read: the MFMA loop then has no branch.
        if constexpr (SS) {
            vm_wait_barrier<0>();
            if (SLOT == 1 && (l_ks & 7) == 0 && gs + KS < total_steps) issue_scales(gs + KS);
            if constexpr (GLU) {
                if (ST == 0 && x_state == 1) x_write();
                else if (ST == 2 && x_state == 2) x_read_store();
            }
        }
        constexpr auto SLOT_N = std::integral_constant<int, 1 - SLOT>{};
        // the load cursor moves on at the start of the K step after the one that issued its copies
        // (a branch right after the MFMA loop lets the compiler sink the loop's FMAs past it)
        if constexpr (!SS) advance();

        if (ST == 0 && ks == 0) {  // the load cursor is on this item (it is at least 4 K steps long)
            ci = li, xrow = lx;
            no_bias = ci.sh ? j.sh.w0.biases == nullptr : j.w0.biases == nullptr;
        }
        // the bias term: chunk c (groups 8c .. 8c + 7 of this item) runs at the last K step of its
        // groups, 8 (c + 1) - 1, and loads its operands 3 steps before
        constexpr int per = 8;  // K steps per chunk
        const int axe = G;
        const int c_now = (ks + 1) % per == 0 ? (ks + 1) / per - 1 : -1;
        const int c_pre = ST == 0 && (ks + 4) % per == 0 ? (ks + 4) / per - 1 : -1;
        if (c_pre >= 0) {  // the chunk's X splits (waves 0-2) and biases into LDS
            if (wave < 3)
                dma16(rsrc_of(ci.sh ? j.sh.AX : j.AX), 2u * (uint32_t)((xrow * 3 + wave) * axe),
                      16u * (uint32_t)c_pre, smem + OFF_X + wave * 1024);
            if (!no_bias) {
                const int R = tid;  // B row
                const bool upr = GLU && wave >= 2;
                const int col = ci.n0 + (GLU ? (R & 127) : R);
                const uint32_t wrow = (uint32_t)ci.e * (uint32_t)(ci.sh ? j.sh.w0.out : j.w0.out) + col;
                const bf16_t *bg = ci.sh ? j.sh.w0.biases : j.w0.biases;
                const bf16_t *bu = GLU ? (ci.sh ? j.sh.w1.biases : j.w1.biases) : bg;
                // the chunk's 8 groups (16 bytes)
                dma16(rsrc_of(upr ? bu : bg), 2u * wrow * (uint32_t)G, 16u * (uint32_t)c_pre,
                      smem + OFF_B + wave * 1024);
            }
        }

        // ---- the K step: fragments from LDS (stage ST: immediate offsets). The wave raises its
        // issue priority for the MFMA loop, so that the other workgroup's wave on this SIMD fills
        // the matrix core's gaps with its bookkeeping rather than competing with the loop.
        __builtin_amdgcn_s_setprio(1);
        constexpr int SA = SLOT * STAGE + (ST & 1) * A_STEP, SC = SLOT * STAGE;
        const uint32_t spar = ((gs >> 3) & 1) * S_BYTES;
        // Reads in the order they are needed; LDS reads complete in order, so a partial lgkmcnt
        // wait covers the oldest ones (scalar loads in flight only make such waits stricter).
        u32x4 cw0 = ds_read16<SC>(c_addr[0][ST & 1]);
        u32x4 a00 = ds_read16<SA>(a_off[0]), a10 = ds_read16<SA + 4096>(a_off[0]);
        u32x4 a01 = ds_read16<SA>(a_off[1]), a11 = ds_read16<SA + 4096>(a_off[1]);
        u32x4 a02 = ds_read16<SA>(a_off[2]), a12 = ds_read16<SA + 4096>(a_off[2]);
        u32x4 a03 = ds_read16<SA>(a_off[3]), a13 = ds_read16<SA + 4096>(a_off[3]);
        u32x4 cw1 = ds_read16<SC>(c_addr[1][ST & 1]);
        if (ST == 0) {  // the scales of this 8-step chunk: 8 groups per B row
            sch0 = ds_read16<0>(s_addr0 + spar);
            sch1 = ds_read16<0>(s_addr1 + spar);
        }
        constexpr int NR = ST == 0 ? 12 : 10;
        // the group's scale: ks % 4 == ST (items have a multiple of 8 K steps)
        const int gi = (ks & 4) | ST;
        auto scale_of = [&](const u32x4 &sw) __attribute__((always_inline)) {
            const uint32_t w2 = (gi & 4) ? ((ST & 2) ? sw.w : sw.z) : ((ST & 2) ? sw.y : sw.x);
            return (ST & 1) ? bf_hi(w2) : bf_lo(w2);
        };
        // The matrix cores run fragment 0's chains, then fragment 1's (4 K sub-steps x 2 row
        // fragments each). Between two MFMAs the wave issues about 7 VALU: the expansion of the
        // next code word and 4 scale FMAs, those of fragment 1 of the previous K step (pend)
        // under fragment 0's chains, and fragment 0's under fragment 1's, so that no FMA waits
        // for the chain it reads. sched_barrier pins the interleave.
        u32x4 e = {0u, 0u, 0u, 0u}, en = e;
        float sc0 = 0.f;
        asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(cw0), "+v"(a00), "+v"(a10) : "i"(NR - 3));
        mg_expand_lo(e, cw0[0], cm, cx);
        mg_expand_hi(e, cw0[0], cm, cx);
#pragma unroll
        for (int q = 0; q < 16; ++q) {  // MFMA slot q: fragment q / 8, sub-step (q / 2) % 4, rows q % 2
            const int ni = q >> 3, s = (q >> 1) & 3, mi = q & 1;
            if (q == 2) asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a01), "+v"(a11) : "i"(NR - 5));
            if (q == 4) asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a02), "+v"(a12) : "i"(NR - 7));
            if (q == 6) asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(a03), "+v"(a13) : "i"(NR - 9));
            const u32x4 af = mi ? (s == 0 ? a10 : s == 1 ? a11 : s == 2 ? a12 : a13)
                                : (s == 0 ? a00 : s == 1 ? a01 : s == 2 ? a02 : a03);
            mg_f32x16 &pt = ni ? part1[mi] : part0[mi];
            const mg_f32x16 z = {};
            if (!(HALF && mi))  // (HALF: no second row fragment; its A reads keep the wait counts)
                pt = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(mg_bf16x8, af),
                                                            __builtin_bit_cast(mg_bf16x8, e),
                                                            s ? pt : z, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if (SS && (q & 1)) issue_part(q >> 1, SLOT_N);
            // 4 scale FMAs: slot q's share of pend (q < 8) or of fragment 0 (q >= 8)
            if (q == 8) {
                if (ST == 0) asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(sch0), "+v"(sch1));
                sc0 = scale_of(sch0);
            }
#pragma unroll
            for (int i = 4 * (q & 3); i < 4 * (q & 3) + 4; ++i) {
                const int fm = (q & 7) >> 2;
                if (HALF && fm) continue;
                if (q < 8) acc[fm][1][i] += sc_pend * part1[fm][i];
                else acc[fm][0][i] += sc0 * part0[fm][i];
            }
            // half of the code word of the next (fragment, sub-step) pair nn: the low half after
            // the pair's first MFMA, the high half after its second, then it becomes the operand
            const int nn = (q >> 1) + 1;
            if (nn < 8) {
                if (q == 6) asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(cw1) : "i"(NR - 10));
                const uint32_t w = (nn < 4 ? cw0 : cw1)[nn & 3];
                if ((q & 1) == 0) {
                    mg_expand_lo(en, w, cm, cx);
                } else {
                    mg_expand_hi(en, w, cm, cx);
                    e = en;
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        sc_pend = scale_of(sch1);
        __builtin_amdgcn_s_setprio(0);
        if (c_now >= 0) {  // bias term of chunk c_now: X splits against b (lane half 0), -128 s (1)
            const uint32_t xo = lds0 + OFF_X + 16 * fr;
            u32x4 xa00 = ds_read16<0>(xo), xa01 = ds_read16<1024>(xo), xa02 = ds_read16<2048>(xo);
            u32x4 xa10 = ds_read16<512>(xo), xa11 = ds_read16<1536>(xo), xa12 = ds_read16<2560>(xo);
            u32x4 bv0 = ds_read16<0>(lds0 + OFF_B + (uint32_t)(bro0 + fr) * 16);
            u32x4 bv1 = ds_read16<0>(lds0 + OFF_B + (uint32_t)(bro1 + fr) * 16);
            asm volatile("s_waitcnt lgkmcnt(0)"
                         : "+v"(xa00), "+v"(xa01), "+v"(xa02), "+v"(xa10), "+v"(xa11), "+v"(xa12),
                           "+v"(bv0), "+v"(bv1));
            const u32x4 xa[2][3] = {{xa00, xa01, xa02}, {xa10, xa11, xa12}};
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                // lane half 0: the biases; lane half 1: -128 x the scales of this K chunk
                u32x4 v = fh == 0 ? (ni ? bv1 : bv0) : (ni ? sch1 : sch0);
                if (fh == 1) {
                    v.x = mg_neg128(v.x), v.y = mg_neg128(v.y);
                    v.z = mg_neg128(v.z), v.w = mg_neg128(v.w);
                } else if (no_bias) {
                    v = u32x4{0u, 0u, 0u, 0u};
                }
#pragma unroll
                for (int mi = 0; mi < NMI; ++mi)
#pragma unroll
                    for (int tt = 0; tt < 3; ++tt)
                        acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(mg_bf16x8, xa[mi][tt]),
                            __builtin_bit_cast(mg_bf16x8, v), acc[mi][ni], 0, 0, 0);
            }
        }
        if (ST != 3 || ks != nks - 1) return;
        // the item's last fragment-1 scale
#pragma unroll
        for (int mi = 0; mi < NMI; ++mi)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[mi][1][i] += sc_pend * part1[mi][i];
        sc_pend = 0.f;

        // ---- epilogue of item ci. Stores are widened by exchanging values between lanes (DPP):
        // a 2-byte store per lane and value costs about as much as a 16-byte one. They go through
        // a buffer resource over the tile's own rows (from row0, mrows rows), so that the stores
        // of the rows past mrows fall outside it and are dropped: no branch per store.
        bf16_t *out = ci.sh ? j.sh.out : j.out;
        const int ldo = ci.sh ? j.sh.ldo : j.ldo;
        const rsrc_t r_out = rsrc_of(out + (size_t)ci.row0 * ldo, (uint32_t)ci.mrows * (uint32_t)ldo * 2u);
        if (GLU) {
            // act = R(silu(R(gate)) * R(up)), stored packed; and this wave's half of the act rows'
            // group sums (the down product's X)
            bf16_t *OX = ci.sh ? j.sh.OX : j.OX;
            const int col = ci.n0 + wave * 32 + fr;
            const int c64 = col & 63, kb = c64 >> 3, jj = c64 & 7;
            // lanes with jj < 4 store packed pair (jj, jj + 4) of rows i (i even); lanes jj >= 4
            // the pair of row i + 1: both at the packed position of jj & 3
            const int pcol = (col & ~63) + 8 * (2 * (kb & 3) + (kb >> 2)) + 2 * (jj & 3);
            const bool hi4 = (jj & 4) != 0;
            float va[2][16];  // the act values (rounded) of rows mi * 32 + 8 (i / 4) + 4 fh + i % 4
            if (HALF)
#pragma unroll
                for (int i = 0; i < 16; ++i) va[1][i] = 0.f;
#pragma unroll
            for (int mi = 0; mi < NMI; ++mi)
#pragma unroll
                for (int i = 0; i < 16; i += 2) {
                    float v[2];
#pragma unroll
                    for (int d = 0; d < 2; ++d) {
                        const uint32_t gu = f2bf2(acc[mi][0][i + d], acc[mi][1][i + d]);
                        const float g = bf_lo(gu), u = bf_hi(gu);
                        // silu(g) = g / (1 + exp(-g)): v_exp and v_rcp (within 2 f32 ulp)
                        const float e = __builtin_amdgcn_exp2f(-1.44269504088896f * g);
                        v[d] = (g * __builtin_amdgcn_rcpf(1.f + e)) * u;
                    }
                    const uint32_t hv = f2bf2(v[0], v[1]);  // row i in the low half, i + 1 high
                    va[mi][i] = bf_lo(hv), va[mi][i + 1] = bf_hi(hv);
                    // lane l (jj < 4) keeps row i of (jj, jj + 4); lane l + 4 row i + 1
                    const uint32_t send = hi4 ? (hv & 0xFFFFu) : (hv >> 16);
                    const uint32_t from_up = (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0x104, 0xF, 0xF, false);   // lane l + 4
                    const uint32_t from_dn = (uint32_t)__builtin_amdgcn_mov_dpp((int)send, 0x114, 0xF, 0xF, false);   // lane l - 4
                    const uint32_t pair = hi4 ? (from_dn | (hv & 0xFFFF0000u)) : ((hv & 0xFFFFu) | (from_up << 16));
                    const int r = mi * 32 + 8 * (i >> 2) + 4 * fh + (i & 3) + (hi4 ? 1 : 0);
                    __builtin_amdgcn_raw_buffer_store_b32(pair, r_out, (r * ldo + pcol) * 2, 0, 0);
                }
            // this wave's sums of the 32 act columns for each row, by a reduce-scatter over the
            // 32 lanes of each lane half (their columns): every step pairs lane l with lane l ^ d,
            // each keeps the half of its values that its bit d selects and adds the partner's
            // copy of it. After d = 16 (permlane16_swap), 8 (row_ror:8), 4 (row_shl/shr:4 by
            // banks), 2 and 1 (quad_perm) the lane holds the sum of row xrow_of(lane).
            float w16[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {  // d = 16: lanes of even rows keep mi = 0, odd rows 1
                const auto sw = __builtin_amdgcn_permlane16_swap(__float_as_uint(va[0][i]),
                                                                __float_as_uint(va[1][i]), false, false);
                w16[i] = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
            }
            const bool b3 = (lane & 8) != 0, b2 = (lane & 4) != 0, b1 = (lane & 2) != 0, b0 = (lane & 1) != 0;
            float w8[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {  // d = 8: keep i + 8 b3
                const float keep = b3 ? w16[i + 8] : w16[i], send = b3 ? w16[i] : w16[i + 8];
                w8[i] = keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), 0x128, 0xF, 0xF, false));
            }
            float w4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {  // d = 4: keep i + 4 b2
                const float keep = b2 ? w8[i + 4] : w8[i], send = b2 ? w8[i] : w8[i + 4];
                int m = __builtin_amdgcn_update_dpp(0, __float_as_int(send), 0x104, 0xF, 0x5, false);  // banks 0, 2: lane l + 4
                m = __builtin_amdgcn_update_dpp(m, __float_as_int(send), 0x114, 0xF, 0xA, false);      // banks 1, 3: lane l - 4
                w4[i] = keep + __int_as_float(m);
            }
            float w2[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {  // d = 2: keep i + 2 b1
                const float keep = b1 ? w4[i + 2] : w4[i], send = b1 ? w4[i] : w4[i + 2];
                w2[i] = keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), 0x4E, 0xF, 0xF, false));
            }
            {  // d = 1: keep b0
                const float keep = b0 ? w2[1] : w2[0], send = b0 ? w2[0] : w2[1];
                x_pend = keep + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(send), 0xB1, 0xF, 0xF, false));
            }
            // the group sum is this wave's half plus its partner's (waves 2h, 2h + 1 cover group
            // n0 / 64 + h, with the same lane-to-row map); the hand-over runs after the next
            // barriers
            const int xr = xrow_of(lane);
            x_dst = xr < ci.mrows
                        ? OX + (size_t)(ci.row0 + xr) * 3 * x_oxe + (ci.n0 >> 6) + (wave >> 1)
                        : nullptr;
            x_state = 1;
        } else {
            // each 4 x 4 block (4 rows of a lane, 4 columns of a lane quad) is transposed within
            // the quad (every lane then holds 4 adjacent columns of one row), and lanes l, l ^ 4
            // (the two quads of 8 adjacent columns) trade halves of two such blocks, so that every
            // lane stores 8 adjacent columns of one row (16 bytes)
            const int q = fr & 3;
            const bool hq = (fr & 4) != 0;  // keeps the odd block of each pair
            typedef unsigned u32x4s __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int ni = 0; ni < 2; ++ni) {
                const int col8 = ci.n0 + (ni ? bro1 : bro0) + (fr & ~7);
#pragma unroll
                for (int mi = 0; mi < NMI; ++mi) {
                    uint2 w4[4];
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const uint32_t p02 = f2bf2(acc[mi][ni][4 * b], acc[mi][ni][4 * b + 2]);
                        const uint32_t p13 = f2bf2(acc[mi][ni][4 * b + 1], acc[mi][ni][4 * b + 3]);
                        // lanes q, q ^ 1: even lanes gather rows 0 and 2, odd lanes rows 1 and 3
                        const uint32_t own = (q & 1) ? p13 : p02;
                        const uint32_t rcv = (uint32_t)__builtin_amdgcn_mov_dpp((int)((q & 1) ? p02 : p13), 0xB1, 0xF, 0xF, false);
                        const uint32_t lo_src = (q & 1) ? rcv : own, hi_src = (q & 1) ? own : rcv;
                        const uint32_t A = __builtin_amdgcn_perm(hi_src, lo_src, 0x05040100u);  // row q & 1
                        const uint32_t B = __builtin_amdgcn_perm(hi_src, lo_src, 0x07060302u);  // row 2 + (q & 1)
                        // lanes q, q ^ 2: lanes 0, 1 complete rows 0, 1; lanes 2, 3 rows 2, 3
                        const uint32_t r2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)((q & 2) ? A : B), 0x4E, 0xF, 0xF, false);
                        w4[b] = (q & 2) ? make_uint2(r2, B) : make_uint2(A, r2);
                    }
#pragma unroll
                    for (int bp = 0; bp < 2; ++bp) {
                        const uint2 keep = hq ? w4[2 * bp + 1] : w4[2 * bp];
                        const uint2 send = hq ? w4[2 * bp] : w4[2 * bp + 1];
                        // lane ^ 4 within each row of 16 lanes: banks 0, 2 read lane + 4, banks 1, 3 lane - 4
                        int rx = __builtin_amdgcn_update_dpp(0, (int)send.x, 0x104, 0xF, 0x5, false);
                        rx = __builtin_amdgcn_update_dpp(rx, (int)send.x, 0x114, 0xF, 0xA, false);
                        int ry = __builtin_amdgcn_update_dpp(0, (int)send.y, 0x104, 0xF, 0x5, false);
                        ry = __builtin_amdgcn_update_dpp(ry, (int)send.y, 0x114, 0xF, 0xA, false);
                        const u32x4s v = hq ? u32x4s{(uint32_t)rx, (uint32_t)ry, keep.x, keep.y}
                                            : u32x4s{keep.x, keep.y, (uint32_t)rx, (uint32_t)ry};
                        const int r = mi * 32 + 8 * (2 * bp + (hq ? 1 : 0)) + 4 * fh + q;
                        __builtin_amdgcn_raw_buffer_store_b128(v, r_out, (r * ldo + col8) * 2, 0, 0);
                    }
                }
            }
        }
#pragma unroll
        for (int mi = 0; mi < 2; ++mi)
#pragma unroll
            for (int ni = 0; ni < 2; ++ni)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[mi][ni][i] = 0.f;
    };
    // each K step is scheduled on its own (sched_barrier): interleaving neighbouring steps only
    // lengthens live ranges past the register budget of two waves per SIMD
    for (int gs = 0; gs < total_steps; gs += 4) {
        step(gs, std::integral_constant<int, 0>{});
        __builtin_amdgcn_sched_barrier(0);
        step(gs + 1, std::integral_constant<int, 1>{});
        __builtin_amdgcn_sched_barrier(0);
        step(gs + 2, std::integral_constant<int, 2>{});
        __builtin_amdgcn_sched_barrier(0);
        step(gs + 3, std::integral_constant<int, 3>{});
        __builtin_amdgcn_sched_barrier(0);
    }
    if (GLU && x_state == 1) {  // the last item's group sums
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        x_write();
        asm volatile("s_barrier" ::: "memory");
        x_read_store();
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the trailing copies
}

bool moe_gemm_supported(const MoeGemmJob &j) {
    auto ok = [](const QW &w, int K) {
        // byte offsets from the tensors' bases are 32-bit
        return w.codes && w.scales && w.bits == 4 && w.group == 64 && K % 512 == 0 &&
               (size_t)w.experts * (size_t)w.out * (size_t)(K / 2) < ((size_t)1 << 32) &&
               ((uintptr_t)w.codes & 15) == 0 && ((uintptr_t)w.scales & 15) == 0 &&
               (!w.biases || ((uintptr_t)w.biases & 15) == 0);
    };
    const int ncols = j.glu ? 128 : 256;
    if (j.N <= 0 || j.N % ncols != 0 || !ok(j.w0, j.K) || (j.glu && !ok(j.w1, j.K))) return false;
    if (j.tile_m != 0 && j.tile_m != 32 && j.tile_m != 64) return false;  // rows per tile
    // A row offsets (row * lda * 2 bytes, through a buffer resource) are 32-bit
    auto a_fits = [](long long rows, int lda) { return rows > 0 && rows * lda * 2 < (1LL << 32); };
    if (!a_fits(j.a_rows, j.lda) || (j.has_shared && !a_fits(j.sh.M, j.sh.lda))) return false;
    // A rows and the X splits go to LDS in 16-byte copies
    auto a_aligned = [](const bf16_t *a, int lda, const bf16_t *ax) {
        return a && ax && lda % 8 == 0 && ((uintptr_t)a & 15) == 0 && ((uintptr_t)ax & 15) == 0;
    };
    if (!a_aligned(j.A, j.lda, j.AX) || (j.has_shared && !a_aligned(j.sh.A, j.sh.lda, j.sh.AX)))
        return false;
    if (j.w0.out != j.N || (j.glu && j.w1.out != j.N)) return false;
    // epilogue stores: 16 bytes per lane (down: 8 adjacent columns) or 4 (gate/up: a packed
    // pair), at row offsets from the output's base
    auto out_ok = [&](const bf16_t *p, int ldo) {
        const int a = j.glu ? 2 : 8;  // elements per store
        return p && ldo > 0 && ldo % a == 0 && ((uintptr_t)p & (uintptr_t)(2 * a - 1)) == 0;
    };
    if (!out_ok(j.out, j.ldo) || (j.has_shared && !out_ok(j.sh.out, j.sh.ldo))) return false;
    // X splits: one entry per group of x (gate/up) or of act (down)
    const int axe = j.K / 64;
    if (j.ax_e != axe) return false;
    if (j.has_shared) {
        if (!ok(j.sh.w0, j.K) || (j.glu && !ok(j.sh.w1, j.K))) return false;
        if (j.sh.w0.out != j.N || (j.glu && j.sh.w1.out != j.N)) return false;
        if (j.sh.ax_e != axe) return false;
    }
    return true;
}

static int cu_count() {
    static int cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (!cached[dev]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        cached[dev] = n;
    }
    return cached[dev];
}

hipError_t launch_moe_gemm(const MoeGemmJob &j, hipStream_t stream) {
    if (!moe_gemm_supported(j)) return hipErrorInvalidValue;
    const int ncols = j.glu ? 128 : 256;
    const int nb = j.N / ncols;
    const int tm = j.tile_m == 32 ? 32 : mg::BM;
    const int s_tiles = j.has_shared ? (j.sh.M + tm - 1) / tm : 0;
    const int r_tiles = j.has_routing ? j.max_tiles : (j.M + tm - 1) / tm;
    const long long items = (long long)(s_tiles + r_tiles) * nb;
    if (items == 0) return hipSuccess;
    long long grid = 2LL * cu_count();
    if (grid > items) grid = items;
    grid = (grid + 7) / 8 * 8;
    if (tm == 32) {
        if (j.glu) moe_gemm_kernel<true, true><<<(unsigned)grid, mg::NT, 0, stream>>>(j);
        else moe_gemm_kernel<false, true><<<(unsigned)grid, mg::NT, 0, stream>>>(j);
    } else if (j.glu) {
        moe_gemm_kernel<true><<<(unsigned)grid, mg::NT, 0, stream>>>(j);
    } else {
        moe_gemm_kernel<false><<<(unsigned)grid, mg::NT, 0, stream>>>(j);
    }
    return hipGetLastError();
}

}  // namespace mrun
