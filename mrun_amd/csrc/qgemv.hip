// Decode-shaped gathered 4- and 8-bit products (gather_qmm at few rows, nuvec.rs:670-686) and dense
// bf16 ones (bits 16: gather_mm, nuvec.rs:688-697) for the facade ops and the block's generic path.
//
// Layout: a weight row of K codes is K*BITS/32 u32 words; LPR lanes share a row, each lane owning
// 128-bit code chunks (32 codes at 4 bits, 16 at 8) li, li+LPR, ...; a chunk always lies in one
// quant group (chunk codes | group). Per (row, pair) a lane computes scale*sum(x*q) + bias*sum(x)
// over its chunks in f32, then the LPR lanes are summed by a fixed butterfly: the order depends on
// K only, never on how many rows or pairs are in flight (rows of a batch keep their one-row bits).
#include "common.hpp"
#include "kernels.hpp"

namespace mrun {

// Rows of one pair chunk per extra (shared-expert) slot.
constexpr int kExtraRowsPerSlot = 4;

struct Chunk {
    uint4 q;
    float s, b;
};

// Keeps the packed codes opaque inside a loop, so the compiler does not hoist their conversion
// to f32 (8x the registers) out of the per-pair loop.
__device__ __forceinline__ void opaque(uint4 &q) {
    asm volatile("" : "+v"(q.x), "+v"(q.y), "+v"(q.z), "+v"(q.w));
}

// sum_i x[i] * q[i] over 32 codes of a chunk; xs = sum of the 32 x values.
__device__ __forceinline__ float dot32(const uint4 &q, const uint4 *xv) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float acc = 0.f;
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
        const uint32_t lo = w[wi] & 0x0f0f0f0fu, hi = (w[wi] >> 4) & 0x0f0f0f0fu;
        const uint4 xx = xv[wi];
        // codes 8wi..8wi+7 pair with x bf16 values 8wi..8wi+7 (xx.x holds x0,x1; ...)
        acc += bf_lo(xx.x) * (float)(lo & 0xffu);
        acc += bf_hi(xx.x) * (float)(hi & 0xffu);
        acc += bf_lo(xx.y) * (float)((lo >> 8) & 0xffu);
        acc += bf_hi(xx.y) * (float)((hi >> 8) & 0xffu);
        acc += bf_lo(xx.z) * (float)((lo >> 16) & 0xffu);
        acc += bf_hi(xx.z) * (float)((hi >> 16) & 0xffu);
        acc += bf_lo(xx.w) * (float)(lo >> 24);
        acc += bf_hi(xx.w) * (float)(hi >> 24);
    }
    return acc;
}

// sum_i x[i] * q[i] over the 16 8-bit codes of a chunk (codes 4wi..4wi+3 in word wi, LSB first).
__device__ __forceinline__ float dot16_8(const uint4 &q, const uint4 *xv) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float acc = 0.f;
#pragma unroll
    for (int wi = 0; wi < 4; ++wi) {
        const uint4 xx = xv[wi >> 1];
        const uint32_t xa = (wi & 1) ? xx.z : xx.x, xb = (wi & 1) ? xx.w : xx.y;
        acc += bf_lo(xa) * (float)(w[wi] & 0xffu);
        acc += bf_hi(xa) * (float)((w[wi] >> 8) & 0xffu);
        acc += bf_lo(xb) * (float)((w[wi] >> 16) & 0xffu);
        acc += bf_hi(xb) * (float)(w[wi] >> 24);
    }
    return acc;
}

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_v;

// sum_i x[i] * w[i] over the 8 dense bf16 weights of a chunk (f32 accumulation).
__device__ __forceinline__ float dot8_16(const uint4 &q, const uint4 &x) {
    auto d2 = [](uint32_t a, uint32_t b, float c) {
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_v, a),
                                               __builtin_bit_cast(bf16x2_v, b), c, false);
    };
    return d2(x.w, q.w, d2(x.z, q.z, d2(x.y, q.y, d2(x.x, q.x, 0.f))));
}

// sum of the x values of a chunk (XQ x 8 bf16)
template <int XQ>
__device__ __forceinline__ float sum_x(const uint4 *xv) {
    float s = 0.f;
#pragma unroll
    for (int wi = 0; wi < XQ; ++wi) {
        s += bf_lo(xv[wi].x) + bf_hi(xv[wi].x);
        s += bf_lo(xv[wi].y) + bf_hi(xv[wi].y);
        s += bf_lo(xv[wi].z) + bf_hi(xv[wi].z);
        s += bf_lo(xv[wi].w) + bf_hi(xv[wi].w);
    }
    return s;
}

template <int BITS>
__device__ __forceinline__ Chunk load_chunk(const QW &w, int e, int row, int ch) {
    constexpr int CPC = 128 / BITS;  // codes per chunk
    Chunk c;
    const size_t r = (size_t)e * w.out + row;
    const int words = w.in * BITS / 32;
    c.q = *(const uint4 *)(w.codes + r * words + (size_t)ch * 4);
    if (BITS == 16) {  // dense bf16: no affine map
        c.s = 1.f, c.b = 0.f;
        return c;
    }
    const int gshift = __builtin_ctz((unsigned)w.group);  // groups of 32, 64 or 128
    const int groups = w.in >> gshift;
    const int g = (ch * CPC) >> gshift;
    c.s = bf2f(w.scales[r * groups + g]);
    c.b = w.biases ? bf2f(w.biases[r * groups + g]) : 0.f;
    return c;
}

// ---------------------------------------------------------------------------------------------

template <bool GLU, int LPR, int CPL, int RG, int PCH, int BITS>
__global__ __launch_bounds__(256) void gemv_kernel(GemvJob j) {
    constexpr int CPC = 128 / BITS;    // codes per 128-bit chunk
    constexpr int XQ = CPC / 8;        // 128-bit activation loads per chunk
    constexpr int RPI = 64 / LPR;      // rows per load instruction
    constexpr int ROWS_W = RG * RPI;   // rows per wave
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int li = lane % LPR, rsub = lane / LPR;
    const int slot = blockIdx.y;

    const bf16_t *A;
    int lda, a_div, e, lo, hi, ldo;
    const uint32_t *a_map, *o_map;
    QW w0, w1;
    bf16_t *out;
    if (slot < j.max_slots) {
        if (j.has_routing) {
            if ((uint32_t)slot >= *j.routing.n_active) return;
            e = (int)j.routing.active[slot];
            lo = (int)j.routing.offsets[e];
            hi = (int)j.routing.offsets[e + 1];
        } else {
            if (slot > 0) return;
            e = 0;
            lo = 0;
            hi = j.rows;
        }
        A = j.A, lda = j.lda, a_map = j.a_map, a_div = j.a_div;
        w0 = j.w0, w1 = j.w1, o_map = j.o_map, out = j.out, ldo = j.ldo;
    } else {
        const int xs = slot - j.max_slots;
        lo = xs * kExtraRowsPerSlot;
        hi = min(j.x_rows, lo + kExtraRowsPerSlot);
        if (lo >= hi) return;
        e = 0;
        A = j.xA, lda = j.x_lda, a_map = nullptr, a_div = 1;
        w0 = j.xw0, w1 = j.xw1, o_map = nullptr, out = j.xout, ldo = j.x_ldo;
    }
    const int n_ch = w0.in / CPC;
    const int row_base = (blockIdx.x * 4 + wave) * ROWS_W;

    Chunk c0[RG][CPL], c1[RG][CPL];
#pragma unroll
    for (int g = 0; g < RG; ++g) {
        const int row = row_base + g * RPI + rsub;
#pragma unroll
        for (int c = 0; c < CPL; ++c) {
            const int ch = li + c * LPR;
            if (row < w0.out && ch < n_ch) {
                c0[g][c] = load_chunk<BITS>(w0, e, row, ch);
                if (GLU) c1[g][c] = load_chunk<BITS>(w1, e, row, ch);
            } else {
                c0[g][c] = Chunk{make_uint4(0, 0, 0, 0), 0.f, 0.f};
                c1[g][c] = c0[g][c];
            }
        }
    }

    for (int p0 = lo; p0 < hi; p0 += PCH) {
        uint4 xv[PCH][CPL][XQ];
        float xs[PCH][CPL];
#pragma unroll
        for (int pp = 0; pp < PCH; ++pp) {
            const int pos = p0 + pp;
            const int arow = pos < hi ? (a_map ? (int)(a_map[pos] / (uint32_t)a_div) : pos) : -1;
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                const int ch = li + c * LPR;
                if (arow >= 0 && ch < n_ch) {
                    const uint4 *src = (const uint4 *)(A + (size_t)arow * lda + ch * CPC);
#pragma unroll
                    for (int q = 0; q < XQ; ++q) xv[pp][c][q] = src[q];
                    xs[pp][c] = BITS == 16 ? 0.f : sum_x<XQ>(xv[pp][c]);
                } else {
#pragma unroll
                    for (int q = 0; q < XQ; ++q) xv[pp][c][q] = make_uint4(0, 0, 0, 0);
                    xs[pp][c] = 0.f;
                }
            }
        }
#pragma unroll
        for (int g = 0; g < RG; ++g) {
#pragma unroll
            for (int c = 0; c < CPL; ++c) {
                opaque(c0[g][c].q);
                if (GLU) opaque(c1[g][c].q);
            }
        }
#pragma unroll
        for (int g = 0; g < RG; ++g) {
            const int row = row_base + g * RPI + rsub;
#pragma unroll
            for (int pp = 0; pp < PCH; ++pp) {
                float a0 = 0.f, a1 = 0.f;
#pragma unroll
                for (int c = 0; c < CPL; ++c) {
                    if (BITS == 16) {
                        a0 += dot8_16(c0[g][c].q, xv[pp][c][0]);
                        if (GLU) a1 += dot8_16(c1[g][c].q, xv[pp][c][0]);
                        continue;
                    }
                    const float d0 = BITS == 4 ? dot32(c0[g][c].q, xv[pp][c])
                                               : dot16_8(c0[g][c].q, xv[pp][c]);
                    a0 += c0[g][c].s * d0 + c0[g][c].b * xs[pp][c];
                    if (GLU) {
                        const float d1 = BITS == 4 ? dot32(c1[g][c].q, xv[pp][c])
                                                   : dot16_8(c1[g][c].q, xv[pp][c]);
                        a1 += c1[g][c].s * d1 + c1[g][c].b * xs[pp][c];
                    }
                }
                a0 = group_sum<LPR>(a0);
                if (GLU) a1 = group_sum<LPR>(a1);
                const int pos = p0 + pp;
                if (li == 0 && row < w0.out && pos < hi) {
                    const int orow = o_map ? (int)o_map[pos] : pos;
                    float v;
                    if (GLU) {
                        const float gt = rbf(a0), up = rbf(a1);
                        v = (gt * sigmoidf_(gt)) * up;
                    } else {
                        v = a0;
                    }
                    out[(size_t)orow * ldo + row] = (bf16_t)f2bf(v);
                }
            }
        }
    }
}

template <bool GLU, int BITS, int LPR, int CPL>
static void launch_gemv_t(const GemvJob &j, hipStream_t stream) {
    constexpr int RG = GLU ? 4 : 8;
    constexpr int RPI = 64 / LPR;
    constexpr int ROWS_B = 4 * RG * RPI;
    const int extra = j.x_rows > 0 ? (j.x_rows + kExtraRowsPerSlot - 1) / kExtraRowsPerSlot : 0;
    const int rows = (extra && j.xw0.out > j.w0.out) ? j.xw0.out : j.w0.out;
    dim3 grid((rows + ROWS_B - 1) / ROWS_B, j.max_slots + extra);
    gemv_kernel<GLU, LPR, CPL, RG, 1, BITS><<<grid, 256, 0, stream>>>(j);
}

// lanes per row from the chunks per row (the routed and the extra weights share K's chunking)
template <bool GLU, int BITS>
static hipError_t launch_gemv_bits(const GemvJob &j, hipStream_t stream) {
    const int n_ch = j.max_slots > 0 ? j.w0.in / (128 / BITS) : j.xw0.in / (128 / BITS);
    if (n_ch >= 64) {
        const int cpl = (n_ch + 63) / 64;
        if (cpl == 1) launch_gemv_t<GLU, BITS, 64, 1>(j, stream);
        else if (cpl == 2) launch_gemv_t<GLU, BITS, 64, 2>(j, stream);
        else if (cpl == 3) launch_gemv_t<GLU, BITS, 64, 3>(j, stream);
        else if (cpl == 4) launch_gemv_t<GLU, BITS, 64, 4>(j, stream);
        else if (BITS >= 8 && cpl <= 8) launch_gemv_t<GLU, BITS, 64, 8>(j, stream);
        else return hipErrorInvalidValue;
    } else if (n_ch >= 32) {
        launch_gemv_t<GLU, BITS, 32, 2>(j, stream);
    } else if (n_ch >= 16) {
        launch_gemv_t<GLU, BITS, 16, 2>(j, stream);
    } else if (n_ch >= 8) {
        launch_gemv_t<GLU, BITS, 8, 2>(j, stream);
    } else if (n_ch >= 4) {
        launch_gemv_t<GLU, BITS, 4, 2>(j, stream);
    } else if (n_ch >= 2) {
        launch_gemv_t<GLU, BITS, 2, 2>(j, stream);
    } else {
        launch_gemv_t<GLU, BITS, 1, 1>(j, stream);
    }
    return hipGetLastError();
}

template <bool GLU>
static hipError_t launch_gemv_one(const GemvJob &j, hipStream_t stream) {
    const int bits = j.max_slots > 0 ? j.w0.bits : j.xw0.bits;
    if (bits == 16) return launch_gemv_bits<GLU, 16>(j, stream);
    return bits == 8 ? launch_gemv_bits<GLU, 8>(j, stream) : launch_gemv_bits<GLU, 4>(j, stream);
}

hipError_t launch_gemv(const GemvJob &j, hipStream_t stream) {
    // routed and extra (shared) weights of different widths or bit counts go in two launches
    const bool split = j.max_slots > 0 && j.x_rows > 0 &&
                       (j.xw0.bits != j.w0.bits || j.xw0.in != j.w0.in);
    if (!split) return j.glu ? launch_gemv_one<true>(j, stream) : launch_gemv_one<false>(j, stream);
    GemvJob a = j, b = j;
    a.x_rows = 0;
    b.max_slots = 0;
    hipError_t e = j.glu ? launch_gemv_one<true>(a, stream) : launch_gemv_one<false>(a, stream);
    if (e != hipSuccess) return e;
    return j.glu ? launch_gemv_one<true>(b, stream) : launch_gemv_one<false>(b, stream);
}

}  // namespace mrun
