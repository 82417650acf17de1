// Element-wise parts of the MoE block: swiglu (activations.rs:55-59), the weighted combine with the
// sigmoid-gated shared expert (moe.rs:84-93, 161-171), rms_norm / add_rms_norm around the block
// (nuvec.rs:796-811), and a Linear's bias add (load.rs:302-305). All HBM-bound: 128-bit loads and
// stores of 8 bf16 per thread, f32 inside, one bf16 rounding per reference op.
#include "common.hpp"
#include "kernels.hpp"

namespace mrun {

__global__ __launch_bounds__(256) void swiglu_kernel(const bf16_t *__restrict__ g,
                                                     const bf16_t *__restrict__ u, int64_t n,
                                                     bf16_t *__restrict__ out) {
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (i + 8 <= n) {
        float gf[8], uf[8];
        unpack8(*(const uint4 *)(g + i), gf);
        unpack8(*(const uint4 *)(u + i), uf);
        uint32_t o[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] = f2bf((gf[k] * sigmoidf_(gf[k])) * uf[k]);
        *(uint4 *)(out + i) =
            make_uint4(o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16),
                       o[6] | (o[7] << 16));
    } else {
        for (int64_t k = i; k < n; ++k) {
            const float gv = bf2f(g[k]);
            out[k] = (bf16_t)f2bf((gv * sigmoidf_(gv)) * bf2f(u[k]));
        }
    }
}

hipError_t launch_swiglu(const bf16_t *g, const bf16_t *u, int64_t n, bf16_t *out,
                         hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    const int64_t blocks = (n + 256 * 8 - 1) / (256 * 8);
    swiglu_kernel<<<dim3((unsigned)blocks), 256, 0, stream>>>(g, u, n, out);
    return hipGetLastError();
}

// One workgroup per (token, 2048-column slab); thread = 8 columns. All k row indices, then all k
// rows, are loaded before the first is used (the rows' loads overlap instead of following each
// other); the sum stays in j order.
//
// POST (rows of at most 2048, one slab): the layer stack's residual add and the next layer's
// RMSNorm on the combined row, in the order of rms_norm_row_kernel (lane l of that kernel's wave
// sums chunks l, l + 64, ... in turn: here chunk l + 64 w sits with wave w's lane l, so the waves
// pass each lane's running sum on through LDS in wave order), so the bits are those of the
// separate kernel.
template <int KMAX, bool POST>
__global__ __launch_bounds__(256) void combine_kernel(const bf16_t *__restrict__ y,
                                                      const uint32_t *__restrict__ inverse,
                                                      const bf16_t *__restrict__ scores, int T,
                                                      int k, int D, const bf16_t *__restrict__ sh_y,
                                                      const bf16_t *__restrict__ sh_logit,
                                                      bf16_t *__restrict__ out, PostNorm post) {
    const int t = blockIdx.x;
    const int d = (blockIdx.y * 256 + threadIdx.x) * 8;
    if (!POST && d >= D) return;
    const bool on = d < D;
    const int dc = min(d, D - 8);  // clamped (POST: threads past the row keep to the barriers)
    uint32_t row[KMAX];
    uint32_t sraw[KMAX];
#pragma unroll
    for (int jj = 0; jj < KMAX; ++jj) {
        const int p = t * k + min(jj, k - 1);
        row[jj] = inverse ? inverse[p] : (uint32_t)p;
        sraw[jj] = scores[p];
    }
    uint4 yv[KMAX];
#pragma unroll
    for (int jj = 0; jj < KMAX; ++jj) yv[jj] = *(const uint4 *)(y + (size_t)row[jj] * D + dc);
    uint4 rv = make_uint4(0u, 0u, 0u, 0u);
    if (POST) rv = *(const uint4 *)(post.resid + (size_t)t * D + dc);
    const float sg = sh_y ? rbf(sigmoidf_(bf2f(sh_logit[t]))) : 0.f;
    uint4 sv = make_uint4(0, 0, 0, 0);
    if (sh_y) sv = *(const uint4 *)(sh_y + (size_t)t * D + dc);
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.f;
#pragma unroll
    for (int jj = 0; jj < KMAX; ++jj) {
        if (jj < k) {
            const float s = bf2f(sraw[jj]);
            float yf[8];
            unpack8(yv[jj], yf);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] += rbf(yf[i] * s);
        }
    }
    uint32_t o[8];
    if (sh_y) {
        float sf[8];
        unpack8(sv, sf);
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = f2bf(rbf(acc[i]) + rbf(sg * sf[i]));
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = f2bf(acc[i]);
    }
    if (!POST) {
        *(uint4 *)(out + (size_t)t * D + d) = make_uint4(o[0] | (o[1] << 16), o[2] | (o[3] << 16),
                                                         o[4] | (o[5] << 16), o[6] | (o[7] << 16));
        return;
    }
    // resid = R(resid + o); the running sum of squares of chunk (lane, wave) continues wave by wave
    __shared__ float chain[64];
    __shared__ float inv_s;
    float f[8];
    unpack8(rv, f);
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = rbf(f[i] + bf2f(o[i]));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int w = 0; w < 4; ++w) {
        if (wave == w) {
            float ss = w == 0 ? 0.f : chain[lane];
            if (on) ss = sumsq8(f, ss);
            chain[lane] = ss;
        }
        __syncthreads();
    }
    if (wave == 0) {
        const float v = group_sum<64>(chain[lane]);
        if (lane == 0) inv_s = rms_inv_of(v, D, post.eps);
    }
    __syncthreads();
    if (!on) return;
    const float inv = inv_s;
    uint32_t hv[8], rn[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float wv = post.w ? bf2f(post.w[d + i]) : 1.0f;
        hv[i] = f2bf(rbf(f[i] * inv) * wv);
        rn[i] = f2bf(f[i]);
    }
    *(uint4 *)(post.resid + (size_t)t * D + d) = make_uint4(
        rn[0] | (rn[1] << 16), rn[2] | (rn[3] << 16), rn[4] | (rn[5] << 16), rn[6] | (rn[7] << 16));
    *(uint4 *)(post.h + (size_t)t * D + d) = make_uint4(
        hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16), hv[6] | (hv[7] << 16));
}

hipError_t launch_combine(const bf16_t *y, const uint32_t *inverse, const bf16_t *scores, int T,
                          int k, int D, const bf16_t *sh_y, const bf16_t *sh_logit, bf16_t *out,
                          hipStream_t stream, const PostNorm *post) {
    dim3 grid(T, (D + 2047) / 2048);
    if (post) {
        if (D > 2048 || D % 8 != 0 || k > 16) return hipErrorInvalidValue;
        if (k <= 8) combine_kernel<8, true><<<grid, 256, 0, stream>>>(y, inverse, scores, T, k, D, sh_y, sh_logit, out, *post);
        else combine_kernel<16, true><<<grid, 256, 0, stream>>>(y, inverse, scores, T, k, D, sh_y, sh_logit, out, *post);
        return hipGetLastError();
    }
    const PostNorm none{};
    if (k <= 8) combine_kernel<8, false><<<grid, 256, 0, stream>>>(y, inverse, scores, T, k, D, sh_y, sh_logit, out, none);
    else combine_kernel<16, false><<<grid, 256, 0, stream>>>(y, inverse, scores, T, k, D, sh_y, sh_logit, out, none);
    return hipGetLastError();
}

// One workgroup per row. With res: h = R(x + res) is written and normalised; else x is. h may
// alias x or res (each thread writes only the elements it has just read), so neither is restrict.
__global__ __launch_bounds__(256) void rms_norm_kernel(const bf16_t *x,
                                                       const bf16_t *res,
                                                       const bf16_t *__restrict__ w, int D,
                                                       float eps, bf16_t *h,
                                                       bf16_t *__restrict__ y) {
    const int r = blockIdx.x;
    const bf16_t *xr = x + (size_t)r * D;
    const bf16_t *rr = res ? res + (size_t)r * D : nullptr;
    // every wave forms the row's 1/rms itself, in the order the fused decode router uses
    const float inv = row_rms_inv(xr, rr, D, eps, threadIdx.x & 63);
    // the row is read in full before any element is written (h may alias x or res)
    __syncthreads();
    for (int d = threadIdx.x * 8; d < D; d += 2048) {
        float xf[8];
        unpack8(*(const uint4 *)(xr + d), xf);
        if (rr) {
            float rf[8];
            unpack8(*(const uint4 *)(rr + d), rf);
#pragma unroll
            for (int i = 0; i < 8; ++i) xf[i] = rbf(xf[i] + rf[i]);
        }
        uint32_t o[8], hv[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float wv = w ? bf2f(w[d + i]) : 1.0f;
            o[i] = f2bf(rbf(xf[i] * inv) * wv);
            hv[i] = f2bf(xf[i]);
        }
        if (rr && h)
            *(uint4 *)(h + (size_t)r * D + d) =
                make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16),
                           hv[6] | (hv[7] << 16));
        *(uint4 *)(y + (size_t)r * D + d) = make_uint4(
            o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16));
    }
}

// Rows of at most 2048: one wave per row (four rows per workgroup). The wave reads its row once
// into registers (lane l: elements [8l + 512i, +8)), forms 1/rms with row_rms_inv's order and
// rounding (the same bits as the kernel above and the fused decode router) and writes the elements
// it read, so h may alias x or res.
__global__ __launch_bounds__(256) void rms_norm_row_kernel(const bf16_t *x, const bf16_t *res,
                                                           const bf16_t *__restrict__ w, int rows,
                                                           int D, float eps, bf16_t *h,
                                                           bf16_t *__restrict__ y) {
    const int lane = threadIdx.x & 63, r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const bf16_t *xr = x + (size_t)r * D;
    const bf16_t *rr = res ? res + (size_t)r * D : nullptr;
    uint4 xv[4], rv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = min(lane * 8 + 512 * i, D - 8);  // clamped; chunks past D are not used
        xv[i] = *(const uint4 *)(xr + d);
        rv[i] = rr ? *(const uint4 *)(rr + d) : make_uint4(0u, 0u, 0u, 0u);
    }
    float f[4][8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        unpack8(xv[i], f[i]);
        if (rr) {
            float rf[8];
            unpack8(rv[i], rf);
#pragma unroll
            for (int k = 0; k < 8; ++k) f[i][k] = rbf(f[i][k] + rf[k]);
        }
        if (lane * 8 + 512 * i < D) ss = sumsq8(f[i], ss);
    }
    const float inv = rms_inv_of(group_sum<64>(ss), D, eps);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane * 8 + 512 * i;
        if (d >= D) continue;
        uint32_t o[8], hv[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float wv = w ? bf2f(w[d + k]) : 1.0f;
            o[k] = f2bf(rbf(f[i][k] * inv) * wv);
            hv[k] = f2bf(f[i][k]);
        }
        if (rr && h)
            *(uint4 *)(h + (size_t)r * D + d) =
                make_uint4(hv[0] | (hv[1] << 16), hv[2] | (hv[3] << 16), hv[4] | (hv[5] << 16),
                           hv[6] | (hv[7] << 16));
        *(uint4 *)(y + (size_t)r * D + d) = make_uint4(
            o[0] | (o[1] << 16), o[2] | (o[3] << 16), o[4] | (o[5] << 16), o[6] | (o[7] << 16));
    }
}

hipError_t launch_rms_norm(const bf16_t *x, const bf16_t *res, const bf16_t *w, int rows, int D,
                           float eps, bf16_t *h, bf16_t *y, hipStream_t stream) {
    if (D <= 2048) rms_norm_row_kernel<<<(rows + 3) / 4, 256, 0, stream>>>(x, res, w, rows, D, eps, h, y);
    else rms_norm_kernel<<<rows, 256, 0, stream>>>(x, res, w, D, eps, h, y);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void add_bias_kernel(bf16_t *y, const bf16_t *__restrict__ b,
                                                       int64_t total, int n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < total) y[i] = (bf16_t)f2bf(bf2f(y[i]) + bf2f(b[i % n]));
}

hipError_t launch_add_bias(bf16_t *y, const bf16_t *bias, int rows, int n, hipStream_t stream) {
    const int64_t total = (int64_t)rows * n;
    add_bias_kernel<<<dim3((unsigned)((total + 255) / 256)), 256, 0, stream>>>(y, bias, total, n);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t *dst, uint32_t v, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) dst[i] = v;
}

hipError_t launch_fill_u32(uint32_t *dst, uint32_t v, int n, hipStream_t stream) {
    if (n <= 0) return hipSuccess;
    fill_u32_kernel<<<dim3((n + 255) / 256), 256, 0, stream>>>(dst, v, n);
    return hipGetLastError();
}

// dst[r] = src[map[r]] for rows of `width` bf16 (a multiple of 8), 16 bytes per thread.
__global__ __launch_bounds__(256) void rows_gather_kernel(const bf16_t *__restrict__ src,
                                                          const uint32_t *__restrict__ map,
                                                          int rows, int width,
                                                          bf16_t *__restrict__ dst) {
    const int chunks = width / 8;
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long long)rows * chunks) return;
    const int r = (int)(i / chunks), c = (int)(i % chunks);
    *(uint4 *)(dst + (size_t)r * width + (size_t)c * 8) =
        *(const uint4 *)(src + (size_t)map[r] * width + (size_t)c * 8);
}

hipError_t launch_rows_gather(const bf16_t *src, const uint32_t *map, int rows, int width,
                              bf16_t *dst, hipStream_t stream) {
    const long long n = (long long)rows * (width / 8);
    if (n <= 0) return hipSuccess;
    if (width % 8 != 0) return hipErrorInvalidValue;
    rows_gather_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stream>>>(src, map, rows, width, dst);
    return hipGetLastError();
}

// y[t][n] = R(x[t] . W[n]) (then R(. + bias[n])) for narrow outputs (a Linear with few rows, e.g.
// the shared expert's gate): one wave per token, the rows of W in turn.
__global__ __launch_bounds__(256) void rowdot_kernel(const bf16_t *__restrict__ x, int T, int D,
                                                     const bf16_t *__restrict__ W, int N,
                                                     const bf16_t *__restrict__ bias,
                                                     bf16_t *__restrict__ y) {
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (t >= T) return;
    const bf16_t *xr = x + (size_t)t * D;
    for (int n = 0; n < N; ++n) {
        const bf16_t *wr = W + (size_t)n * D;
        float acc = 0.f;
        for (int d = lane * 8; d < D; d += 512) {
            float xf[8], wf[8];
            unpack8(*(const uint4 *)(xr + d), xf);
            unpack8(*(const uint4 *)(wr + d), wf);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc += xf[i] * wf[i];
        }
        acc = group_sum<64>(acc);
        if (lane == 0) {
            float v = rbf(acc);
            if (bias) v = rbf(v + bf2f(bias[n]));
            y[(size_t)t * N + n] = (bf16_t)f2bf(v);
        }
    }
}

hipError_t launch_rowdot(const bf16_t *x, int T, int D, const bf16_t *W, int N,
                         const bf16_t *bias, bf16_t *y, hipStream_t stream) {
    rowdot_kernel<<<dim3((T + 3) / 4), 256, 0, stream>>>(x, T, D, W, N, bias, y);
    return hipGetLastError();
}

}  // namespace mrun
