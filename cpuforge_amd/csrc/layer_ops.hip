// The ops around the attention in a cpuforge training step, on gfx950:
// RMSNorm, the SwiGLU gate, cross-entropy with its gradient and AdamW.  All
// are HBM-bound: rows are read with coalesced 16-byte loads, kept in LDS or
// registers while a row statistic is formed, and written once.
//
// Where the reference fixes an order of f32 operations (RMSNorm's sum of
// squares, AdamW's update), the kernels keep it with explicitly rounded
// operations (no fused multiply-add), so those results equal the reference
// algorithm's bit for bit.  Row reductions over a vocabulary (cross-entropy)
// and over many rows (the RMSNorm gain gradient) run in a fixed parallel
// order instead: deterministic, and within a few ulp of the sequential sum.
#include <limits.h>

#include "cfattn_common.hpp"
#include "cfops_kernels.hpp"

// No multiply-add contraction in this file: the helpers below round every
// product, sum, quotient and square root on its own (correctly rounded, as
// hipcc's default f32 division and sqrt are).  HIP's own __fadd_rn and
// __fmul_rn are plain operators defined where contraction is on, so after
// inlining they could still be fused.
#pragma clang fp contract(off)

namespace cfattn {

namespace {
__device__ __forceinline__ float radd(float a, float b) { return a + b; }
__device__ __forceinline__ float rsub(float a, float b) { return a - b; }
__device__ __forceinline__ float rmul(float a, float b) { return a * b; }
__device__ __forceinline__ float rdiv(float a, float b) { return a / b; }
__device__ __forceinline__ float rsqrt_cr(float a) { return sqrtf(a); }
}  // namespace

namespace {

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// Rows per RMSNorm workgroup and the LDS row stride (an odd number of floats,
// so the one-lane-per-row sums read distinct banks).
constexpr int kRmsThreads = 256;
constexpr int kRmsMaxRows = 16;
constexpr size_t kRmsLdsFloats = 16384;  // 64 KiB per staged tensor
inline int rms_ld(size_t dim) { return (int)(dim | 1); }
inline int rms_rows(size_t dim) {
    const size_t r = kRmsLdsFloats / (size_t)rms_ld(dim);
    return (int)(r < 1 ? 1 : r > kRmsMaxRows ? kRmsMaxRows : r);
}
inline bool rms_staged(size_t dim) { return (size_t)rms_ld(dim) <= kRmsLdsFloats; }

}  // namespace

// ------------------------------------------------------------------ RMSNorm
// Stage `nr` rows of `dim` floats into LDS rows `ld` apart.
template <bool VEC>
__device__ __forceinline__ void stage_f32_rows(float* __restrict__ s, const float* __restrict__ g, int nr, int dim,
                                               int ld) {
    const int n = nr * dim;
    if (VEC) {
        for (int i = threadIdx.x; i < n / 4; i += blockDim.x) {
            const float4 v = reinterpret_cast<const float4*>(g)[i];
            const int e = i * 4, rr = e / dim, c = e - rr * dim;
            float* d = s + rr * ld + c;
            d[0] = v.x;
            d[1] = v.y;
            d[2] = v.z;
            d[3] = v.w;
        }
    } else {
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const int rr = i / dim;
            s[rr * ld + i - rr * dim] = g[i];
        }
    }
}

// rmsnorm_forward (rmsnorm.rs:4-28): per row, the sum of squares in element
// order (one lane per row, over LDS), inv = 1 / sqrt(sum / dim + eps), then
// y = (x * inv) * w over the whole block.
template <bool VEC>
__global__ __launch_bounds__(kRmsThreads) void rmsnorm_fwd_kernel(const float* __restrict__ x,
                                                                  const float* __restrict__ w, float* __restrict__ y,
                                                                  float* __restrict__ rstd, long rows, int dim, int rpb,
                                                                  float eps) {
    extern __shared__ float smem[];
    const int ld = dim | 1;
    float* sx = smem;
    float* sinv = smem + rpb * ld;
    const long r0 = (long)blockIdx.x * rpb;
    const int nr = (int)min((long)rpb, rows - r0);
    stage_f32_rows<VEC>(sx, x + r0 * dim, nr, dim, ld);
    __syncthreads();
    if ((int)threadIdx.x < nr) {
        const float* row = sx + threadIdx.x * ld;
        float ss = 0.0f;
        // Eight LDS reads issued ahead of each eight in-order adds: the sum's
        // order stays the element order, the reads leave the add chain.
        int i = 0;
        for (; i + 8 <= dim; i += 8) {
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = row[i + j];
#pragma unroll
            for (int j = 0; j < 8; j++) ss = radd(ss, rmul(v[j], v[j]));
        }
        for (; i < dim; i++) ss = radd(ss, rmul(row[i], row[i]));
        const float ms = rdiv(ss, (float)dim);
        const float inv = rdiv(1.0f, rsqrt_cr(radd(ms, eps)));
        sinv[threadIdx.x] = inv;
        rstd[r0 + threadIdx.x] = inv;
    }
    __syncthreads();
    float* yb = y + r0 * dim;
    const int n = nr * dim;
    if (VEC) {
        for (int i = threadIdx.x; i < n / 4; i += blockDim.x) {
            const int e = i * 4, rr = e / dim, c = e - rr * dim;
            const float* s = sx + rr * ld + c;
            const float inv = sinv[rr];
            const float4 wv = *reinterpret_cast<const float4*>(w + c);
            reinterpret_cast<float4*>(yb)[i] =
                make_float4(rmul(rmul(s[0], inv), wv.x), rmul(rmul(s[1], inv), wv.y),
                            rmul(rmul(s[2], inv), wv.z), rmul(rmul(s[3], inv), wv.w));
        }
    } else {
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const int rr = i / dim, c = i - rr * dim;
            yb[i] = rmul(rmul(sx[rr * ld + c], sinv[rr]), w[c]);
        }
    }
}

// Rows wider than the LDS budget: one thread per row, straight from memory.
__global__ __launch_bounds__(256) void rmsnorm_fwd_rowwise_kernel(const float* __restrict__ x,
                                                                  const float* __restrict__ w, float* __restrict__ y,
                                                                  float* __restrict__ rstd, long rows, long dim,
                                                                  float eps) {
    const long r = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const float* row = x + r * dim;
    float ss = 0.0f;
    for (long i = 0; i < dim; i++) ss = radd(ss, rmul(row[i], row[i]));
    const float inv = rdiv(1.0f, rsqrt_cr(radd(rdiv(ss, (float)dim), eps)));
    rstd[r] = inv;
    for (long i = 0; i < dim; i++) y[r * dim + i] = rmul(rmul(row[i], inv), w[i]);
}

// rmsnorm_backward (rmsnorm.rs:33-67), rows of one workgroup:
//   dot  = sum_i ((dy_i * w_i) * x_i) * inv   (element order, one lane per row)
//   mean = dot / dim,  xhat = x * inv
//   dx  += inv * (dy * w - xhat * mean)
// and, with `partial` non-null, the block's gain-gradient partial sums
// partial[block][i] = sum over the block's rows, in row order, of dy_i * xhat_i.
template <bool VEC>
__global__ __launch_bounds__(kRmsThreads) void rmsnorm_bwd_kernel(const float* __restrict__ dy,
                                                                  const float* __restrict__ x,
                                                                  const float* __restrict__ w,
                                                                  const float* __restrict__ rstd,
                                                                  float* __restrict__ dx, float* __restrict__ partial,
                                                                  long rows, int dim, int rpb) {
    extern __shared__ float smem[];
    const int ld = dim | 1;
    float* sx = smem;
    float* sdy = sx + rpb * ld;
    float* sw = sdy + rpb * ld;
    float* sinv = sw + dim;
    float* smean = sinv + rpb;
    const long r0 = (long)blockIdx.x * rpb;
    const int nr = (int)min((long)rpb, rows - r0);
    stage_f32_rows<VEC>(sx, x + r0 * dim, nr, dim, ld);
    stage_f32_rows<VEC>(sdy, dy + r0 * dim, nr, dim, ld);
    for (int i = threadIdx.x; i < dim; i += blockDim.x) sw[i] = w[i];
    if ((int)threadIdx.x < nr) sinv[threadIdx.x] = rstd[r0 + threadIdx.x];
    __syncthreads();
    if ((int)threadIdx.x < nr) {
        const float* xr = sx + threadIdx.x * ld;
        const float* gr = sdy + threadIdx.x * ld;
        const float inv = sinv[threadIdx.x];
        float dot = 0.0f;
        int i = 0;
        for (; i + 8 <= dim; i += 8) {
            float t[8];
#pragma unroll
            for (int j = 0; j < 8; j++) t[j] = rmul(rmul(rmul(gr[i + j], sw[i + j]), xr[i + j]), inv);
#pragma unroll
            for (int j = 0; j < 8; j++) dot = radd(dot, t[j]);
        }
        for (; i < dim; i++) dot = radd(dot, rmul(rmul(rmul(gr[i], sw[i]), xr[i]), inv));
        smean[threadIdx.x] = rdiv(dot, (float)dim);
    }
    __syncthreads();
    float* dxb = dx + r0 * dim;
    const int n = nr * dim;
    auto grad = [&](int rr, int c) {
        const float inv = sinv[rr];
        const float xh = rmul(sx[rr * ld + c], inv);
        return rmul(inv, rsub(rmul(sdy[rr * ld + c], sw[c]), rmul(xh, smean[rr])));
    };
    if (VEC) {
        for (int i = threadIdx.x; i < n / 4; i += blockDim.x) {
            const int e = i * 4, rr = e / dim, c = e - rr * dim;
            float4 d = reinterpret_cast<float4*>(dxb)[i];
            d.x = radd(d.x, grad(rr, c));
            d.y = radd(d.y, grad(rr, c + 1));
            d.z = radd(d.z, grad(rr, c + 2));
            d.w = radd(d.w, grad(rr, c + 3));
            reinterpret_cast<float4*>(dxb)[i] = d;
        }
    } else {
        for (int i = threadIdx.x; i < n; i += blockDim.x) {
            const int rr = i / dim, c = i - rr * dim;
            dxb[i] = radd(dxb[i], grad(rr, c));
        }
    }
    if (partial) {
        for (int c = threadIdx.x; c < dim; c += blockDim.x) {
            float acc = 0.0f;
            for (int rr = 0; rr < nr; rr++)
                acc = radd(acc, rmul(sdy[rr * ld + c], rmul(sx[rr * ld + c], sinv[rr])));
            partial[(long)blockIdx.x * dim + c] = acc;
        }
    }
}

// Rows wider than the LDS budget: one thread per row; the gain gradient goes
// through one partial row per row.
__global__ __launch_bounds__(256) void rmsnorm_bwd_rowwise_kernel(const float* __restrict__ dy,
                                                                  const float* __restrict__ x,
                                                                  const float* __restrict__ w,
                                                                  const float* __restrict__ rstd,
                                                                  float* __restrict__ dx, float* __restrict__ partial,
                                                                  long rows, long dim) {
    const long r = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    const float* xr = x + r * dim;
    const float* gr = dy + r * dim;
    const float inv = rstd[r];
    float dot = 0.0f;
    for (long i = 0; i < dim; i++) dot = radd(dot, rmul(rmul(rmul(gr[i], w[i]), xr[i]), inv));
    const float mean = rdiv(dot, (float)dim);
    for (long i = 0; i < dim; i++) {
        const float xh = rmul(xr[i], inv);
        dx[r * dim + i] = radd(dx[r * dim + i], rmul(inv, rsub(rmul(gr[i], w[i]), rmul(xh, mean))));
        if (partial) partial[r * dim + i] = rmul(gr[i], xh);
    }
}

// dw[i] += the partial rows, in a fixed two-level order: a workgroup covers
// 32 columns with eight threads per column; thread j adds the partial rows
// j*per .. j*per + per - 1 in order, and the eight sums are then added to dw
// in j order.  Deterministic, and the loads of one thread are independent
// of its adds, so they stay in flight together.
__global__ __launch_bounds__(256) void rmsnorm_dw_reduce_kernel(const float* __restrict__ partial,
                                                                float* __restrict__ dw, long nblk, long dim) {
    __shared__ float ssum[8][32];
    const int cl = threadIdx.x & 31, j = threadIdx.x >> 5;
    const long c = (long)blockIdx.x * 32 + cl;
    const long per = (nblk + 7) / 8;
    const long b0 = j * per, b1 = min(nblk, b0 + per);
    float s = 0.0f;
    if (c < dim) {
#pragma unroll 8
        for (long b = b0; b < b1; b++) s = radd(s, partial[b * dim + c]);
    }
    ssum[j][cl] = s;
    __syncthreads();
    if (j == 0 && c < dim) {
        float t = dw[c];
        for (int i = 0; i < 8; i++) t = radd(t, ssum[i][cl]);
        dw[c] = t;
    }
}

size_t rmsnorm_bwd_partial_floats(size_t rows, size_t dim) {
    if (rows == 0 || dim == 0) return 0;
    if (!rms_staged(dim)) return rows * dim;
    const size_t rpb = (size_t)rms_rows(dim);
    return (rows + rpb - 1) / rpb * dim;
}

hipError_t launch_rmsnorm_fwd(const float* x, const float* w, float* y, float* rstd, size_t rows, size_t dim, float eps,
                              hipStream_t st) {
    if (rows == 0 || dim == 0) return hipSuccess;
    if (!rms_staged(dim)) {
        hipLaunchKernelGGL(rmsnorm_fwd_rowwise_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, x, w,
                           y, rstd, (long)rows, (long)dim, eps);
        return hipGetLastError();
    }
    const int rpb = rms_rows(dim);
    const size_t nblk = (rows + rpb - 1) / rpb;
    if (nblk > 0x7fffffffu) return hipErrorInvalidConfiguration;
    const size_t lds = ((size_t)rpb * rms_ld(dim) + rpb) * sizeof(float);
    const bool vec = dim % 4 == 0 && aligned16(x) && aligned16(w) && aligned16(y);
    if (vec)
        hipLaunchKernelGGL(rmsnorm_fwd_kernel<true>, dim3((unsigned)nblk), dim3(kRmsThreads), lds, st, x, w, y, rstd,
                           (long)rows, (int)dim, rpb, eps);
    else
        hipLaunchKernelGGL(rmsnorm_fwd_kernel<false>, dim3((unsigned)nblk), dim3(kRmsThreads), lds, st, x, w, y, rstd,
                           (long)rows, (int)dim, rpb, eps);
    return hipGetLastError();
}

hipError_t launch_rmsnorm_bwd(const float* dy, const float* x, const float* w, const float* rstd, float* dx, float* dw,
                              float* partial, size_t rows, size_t dim, hipStream_t st) {
    if (rows == 0 || dim == 0) return hipSuccess;
    float* part = dw ? partial : nullptr;
    size_t nblk;
    if (!rms_staged(dim)) {
        hipLaunchKernelGGL(rmsnorm_bwd_rowwise_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, dy, x,
                           w, rstd, dx, part, (long)rows, (long)dim);
        nblk = rows;
    } else {
        const int rpb = rms_rows(dim);
        nblk = (rows + rpb - 1) / rpb;
        if (nblk > 0x7fffffffu) return hipErrorInvalidConfiguration;
        const size_t lds = ((size_t)2 * rpb * rms_ld(dim) + dim + 2 * rpb) * sizeof(float);
        const bool vec = dim % 4 == 0 && aligned16(dy) && aligned16(x) && aligned16(dx);
        if (vec)
            hipLaunchKernelGGL(rmsnorm_bwd_kernel<true>, dim3((unsigned)nblk), dim3(kRmsThreads), lds, st, dy, x, w,
                               rstd, dx, part, (long)rows, (int)dim, rpb);
        else
            hipLaunchKernelGGL(rmsnorm_bwd_kernel<false>, dim3((unsigned)nblk), dim3(kRmsThreads), lds, st, dy, x, w,
                               rstd, dx, part, (long)rows, (int)dim, rpb);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !dw) return e;
    hipLaunchKernelGGL(rmsnorm_dw_reduce_kernel, dim3((unsigned)((dim + 31) / 32)), dim3(256), 0, st, part, dw,
                       (long)nblk, (long)dim);
    return hipGetLastError();
}

// ------------------------------------------------------------------ SwiGLU
// sigmoid(x) = 1 / (1 + exp(-x)) (swiglu.rs:6-8).
__device__ __forceinline__ float sigmoid_ref(float x) { return rdiv(1.0f, radd(1.0f, expf(-x))); }

__device__ __forceinline__ float silu_mul_one(float g, float u) {
    return rmul(rmul(g, sigmoid_ref(g)), u);
}
// d/dg [g * s(g)] = s * (1 + g * (1 - s)); dg += (dh * u) * dsilu, du += dh * silu.
__device__ __forceinline__ void silu_mul_grad(float dh, float g, float u, float& dg, float& du) {
    const float s = sigmoid_ref(g);
    const float silu = rmul(g, s);
    const float dsilu = rmul(s, radd(1.0f, rmul(g, rsub(1.0f, s))));
    dg = radd(dg, rmul(rmul(dh, u), dsilu));
    du = radd(du, rmul(dh, silu));
}

template <bool VEC>
__global__ __launch_bounds__(256) void silu_mul_fwd_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                           float* __restrict__ h, long n) {
    const long stride = (long)gridDim.x * blockDim.x;
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC) {
        for (; i < n / 4; i += stride) {
            const float4 a = reinterpret_cast<const float4*>(g)[i];
            const float4 b = reinterpret_cast<const float4*>(u)[i];
            reinterpret_cast<float4*>(h)[i] =
                make_float4(silu_mul_one(a.x, b.x), silu_mul_one(a.y, b.y), silu_mul_one(a.z, b.z), silu_mul_one(a.w, b.w));
        }
    } else {
        for (; i < n; i += stride) h[i] = silu_mul_one(g[i], u[i]);
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void silu_mul_bwd_kernel(const float* __restrict__ dh, const float* __restrict__ g,
                                                           const float* __restrict__ u, float* __restrict__ dg,
                                                           float* __restrict__ du, long n) {
    const long stride = (long)gridDim.x * blockDim.x;
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC) {
        for (; i < n / 4; i += stride) {
            const float4 d = reinterpret_cast<const float4*>(dh)[i];
            const float4 a = reinterpret_cast<const float4*>(g)[i];
            const float4 b = reinterpret_cast<const float4*>(u)[i];
            float4 x = reinterpret_cast<float4*>(dg)[i];
            float4 y = reinterpret_cast<float4*>(du)[i];
            silu_mul_grad(d.x, a.x, b.x, x.x, y.x);
            silu_mul_grad(d.y, a.y, b.y, x.y, y.y);
            silu_mul_grad(d.z, a.z, b.z, x.z, y.z);
            silu_mul_grad(d.w, a.w, b.w, x.w, y.w);
            reinterpret_cast<float4*>(dg)[i] = x;
            reinterpret_cast<float4*>(du)[i] = y;
        }
    } else {
        for (; i < n; i += stride) silu_mul_grad(dh[i], g[i], u[i], dg[i], du[i]);
    }
}

// Elementwise grid: enough workgroups to fill 256 CUs several times over.
static unsigned ew_blocks(size_t items) {
    const size_t b = (items + 255) / 256;
    return (unsigned)(b < 1 ? 1 : b > 8192 ? 8192 : b);
}

hipError_t launch_silu_mul_fwd(const float* g, const float* u, float* h, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    if (n % 4 == 0 && aligned16(g) && aligned16(u) && aligned16(h))
        hipLaunchKernelGGL(silu_mul_fwd_kernel<true>, dim3(ew_blocks(n / 4)), dim3(256), 0, st, g, u, h, (long)n);
    else
        hipLaunchKernelGGL(silu_mul_fwd_kernel<false>, dim3(ew_blocks(n)), dim3(256), 0, st, g, u, h, (long)n);
    return hipGetLastError();
}

hipError_t launch_silu_mul_bwd(const float* dh, const float* g, const float* u, float* dg, float* du, size_t n,
                               hipStream_t st) {
    if (n == 0) return hipSuccess;
    if (n % 4 == 0 && aligned16(dh) && aligned16(g) && aligned16(u) && aligned16(dg) && aligned16(du))
        hipLaunchKernelGGL(silu_mul_bwd_kernel<true>, dim3(ew_blocks(n / 4)), dim3(256), 0, st, dh, g, u, dg, du,
                           (long)n);
    else
        hipLaunchKernelGGL(silu_mul_bwd_kernel<false>, dim3(ew_blocks(n)), dim3(256), 0, st, dh, g, u, dg, du,
                           (long)n);
    return hipGetLastError();
}

// ----------------------------------------------------------- cross-entropy
constexpr long kIgnoreIndex = -100;  // crates/core/src/ops/loss.rs:4
constexpr int kCeThreads = 512;

// Block-wide max / sum over kCeThreads threads in a fixed order: within each
// wave by xor shuffles, then the eight wave results in wave order.
__device__ __forceinline__ float block_reduce(float v, bool is_max, float* sred) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float w = __shfl_xor(v, o);
        v = is_max ? fmaxf(v, w) : radd(v, w);
    }
    __syncthreads();  // sred is free (an earlier reduction's readers are done)
    if ((threadIdx.x & 63) == 0) sred[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = sred[0];
    for (int i = 1; i < kCeThreads / 64; i++) r = is_max ? fmaxf(r, sred[i]) : radd(r, sred[i]);
    return r;
}

__global__ __launch_bounds__(256) void ce_begin_kernel(const int64_t* __restrict__ targets, long rows,
                                                       CeMisc* __restrict__ m) {
    __shared__ int sc[4];
    int cnt = 0;
    for (long r = threadIdx.x; r < rows; r += blockDim.x) cnt += targets[r] != kIgnoreIndex;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) cnt += __shfl_xor(cnt, o);
    if ((threadIdx.x & 63) == 0) sc[threadIdx.x >> 6] = cnt;
    __syncthreads();
    if (threadIdx.x == 0) {
        m->n_valid = sc[0] + sc[1] + sc[2] + sc[3];
        m->bad_row = INT_MAX;
        m->loss = 0.0f;
    }
}

// One row per workgroup (loss.rs:27-53).  With NV4 > 0 the row stays in
// registers (NV4 float4 per thread) between the max, the exp sum and the
// write, so it is read from memory once; NV4 == 0 streams it three times.
template <int NV4>
__global__ __launch_bounds__(kCeThreads) void ce_rows_kernel(const float* logits, const int64_t* __restrict__ targets,
                                                             float* dlogits, float* __restrict__ row_loss, long row0,
                                                             long vocab, CeMisc* __restrict__ m) {
    __shared__ float sred[kCeThreads / 64];
    const long r = row0 + blockIdx.x;
    const int64_t t = targets[r];
    const float* lr = logits + (long)blockIdx.x * vocab;
    float* dr = dlogits + (long)blockIdx.x * vocab;
    const int tid = threadIdx.x;
    if (t == kIgnoreIndex || t < 0 || t >= vocab) {
        if (t != kIgnoreIndex && tid == 0) atomicMin(&m->bad_row, (int)r);
        for (long i = tid; i < vocab; i += kCeThreads) dr[i] = 0.0f;
        if (tid == 0) row_loss[r] = 0.0f;
        return;
    }
    const float inv_n = rdiv(1.0f, (float)m->n_valid);
    const float lt = lr[t];
    float mx = -INFINITY;
    if constexpr (NV4 > 0) {
        const long nv = vocab / 4;
        float4 v[NV4];
#pragma unroll
        for (int i = 0; i < NV4; i++) {
            const long idx = (long)i * kCeThreads + tid;
            if (idx < nv) {
                v[i] = reinterpret_cast<const float4*>(lr)[idx];
                mx = fmaxf(mx, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
            }
        }
        mx = block_reduce(mx, true, sred);
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < NV4; i++) {
            const long idx = (long)i * kCeThreads + tid;
            if (idx < nv) {
                v[i].x = expf(rsub(v[i].x, mx));
                v[i].y = expf(rsub(v[i].y, mx));
                v[i].z = expf(rsub(v[i].z, mx));
                v[i].w = expf(rsub(v[i].w, mx));
                sum = radd(sum, radd(radd(v[i].x, v[i].y), radd(v[i].z, v[i].w)));
            }
        }
        sum = block_reduce(sum, false, sred);
        const float sc = rmul(rdiv(1.0f, sum), inv_n);
#pragma unroll
        for (int i = 0; i < NV4; i++) {
            const long idx = (long)i * kCeThreads + tid;
            if (idx < nv) {
                float4 d = make_float4(rmul(v[i].x, sc), rmul(v[i].y, sc), rmul(v[i].z, sc),
                                       rmul(v[i].w, sc));
                const long e = idx * 4;
                if (t >= e && t < e + 4) {
                    const int k = (int)(t - e);
                    if (k == 0) d.x = rsub(d.x, inv_n);
                    if (k == 1) d.y = rsub(d.y, inv_n);
                    if (k == 2) d.z = rsub(d.z, inv_n);
                    if (k == 3) d.w = rsub(d.w, inv_n);
                }
                reinterpret_cast<float4*>(dr)[idx] = d;
            }
        }
        if (tid == 0) row_loss[r] = rsub(radd(logf(sum), mx), lt);
    } else {
        for (long i = tid; i < vocab; i += kCeThreads) mx = fmaxf(mx, lr[i]);
        mx = block_reduce(mx, true, sred);
        float sum = 0.0f;
        for (long i = tid; i < vocab; i += kCeThreads) sum = radd(sum, expf(rsub(lr[i], mx)));
        sum = block_reduce(sum, false, sred);
        const float sc = rmul(rdiv(1.0f, sum), inv_n);
        // Every thread has read all of its elements before any is written,
        // and each element is read and written by the same thread, so dr
        // may alias lr.
        for (long i = tid; i < vocab; i += kCeThreads) {
            float d = rmul(expf(rsub(lr[i], mx)), sc);
            if (i == t) d = rsub(d, inv_n);
            dr[i] = d;
        }
        if (tid == 0) row_loss[r] = rsub(radd(logf(sum), mx), lt);
    }
}

// Mean loss: per-row losses summed in f64 in row order (64 contiguous runs,
// then the runs in order), divided by the number of scored rows.
__global__ __launch_bounds__(64) void ce_finish_kernel(const int64_t* __restrict__ targets,
                                                       const float* __restrict__ row_loss, long rows,
                                                       CeMisc* __restrict__ m) {
    __shared__ double sp[64];
    const long per = (rows + 63) / 64;
    const long a = threadIdx.x * per, b = min(rows, a + per);
    double s = 0.0;
    for (long r = a; r < b; r++)
        if (targets[r] != kIgnoreIndex) s += (double)row_loss[r];
    sp[threadIdx.x] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double tot = 0.0;
        for (int i = 0; i < 64; i++) tot += sp[i];
        const int n = m->n_valid;
        m->loss = n > 0 ? (float)(tot / (double)n) : 0.0f;
    }
}

hipError_t launch_ce_begin(const int64_t* targets, size_t rows, void* misc, hipStream_t st) {
    hipLaunchKernelGGL(ce_begin_kernel, dim3(1), dim3(256), 0, st, targets, (long)rows, static_cast<CeMisc*>(misc));
    return hipGetLastError();
}

hipError_t launch_ce_rows(const float* logits, const int64_t* targets, float* dlogits, float* row_loss, size_t row0,
                          size_t nrows, size_t vocab, void* misc, hipStream_t st) {
    if (nrows == 0 || vocab == 0) return hipSuccess;
    if (nrows > 0x7fffffffu) return hipErrorInvalidConfiguration;
    CeMisc* m = static_cast<CeMisc*>(misc);
    const dim3 grid((unsigned)nrows), block(kCeThreads);
    const bool vec = vocab % 4 == 0 && aligned16(logits) && aligned16(dlogits);
    const size_t v4 = (vocab / 4 + kCeThreads - 1) / kCeThreads;  // float4 per thread
    if (vec && v4 <= 8)
        hipLaunchKernelGGL(ce_rows_kernel<8>, grid, block, 0, st, logits, targets, dlogits, row_loss, (long)row0,
                           (long)vocab, m);
    else if (vec && v4 <= 16)
        hipLaunchKernelGGL(ce_rows_kernel<16>, grid, block, 0, st, logits, targets, dlogits, row_loss, (long)row0,
                           (long)vocab, m);
    else if (vec && v4 <= 32)
        hipLaunchKernelGGL(ce_rows_kernel<32>, grid, block, 0, st, logits, targets, dlogits, row_loss, (long)row0,
                           (long)vocab, m);
    else
        hipLaunchKernelGGL(ce_rows_kernel<0>, grid, block, 0, st, logits, targets, dlogits, row_loss, (long)row0,
                           (long)vocab, m);
    return hipGetLastError();
}

hipError_t launch_ce_finish(const int64_t* targets, const float* row_loss, size_t rows, void* misc, hipStream_t st) {
    hipLaunchKernelGGL(ce_finish_kernel, dim3(1), dim3(64), 0, st, targets, row_loss, (long)rows,
                       static_cast<CeMisc*>(misc));
    return hipGetLastError();
}

// ------------------------------------------------------------------- AdamW
// optim.rs:21-29 with every product and sum rounded on its own:
//   m = b1*m + (1-b1)*g,  v = b2*v + ((1-b2)*g)*g,
//   p -= lr * ((m/bc1) / (sqrt(v/bc2) + eps) + wd*p).
__device__ __forceinline__ void adamw_one(float& p, float g, float& m, float& v, float lr, float b1, float b2, float ob1,
                                          float ob2, float eps, float wd, float bc1, float bc2) {
    m = radd(rmul(b1, m), rmul(ob1, g));
    v = radd(rmul(b2, v), rmul(rmul(ob2, g), g));
    const float mhat = rdiv(m, bc1);
    const float vhat = rdiv(v, bc2);
    const float upd = radd(rdiv(mhat, radd(rsqrt_cr(vhat), eps)), rmul(wd, p));
    p = rsub(p, rmul(lr, upd));
}

template <bool VEC>
__global__ __launch_bounds__(256) void adamw_kernel(float* __restrict__ p, const float* __restrict__ g,
                                                    float* __restrict__ m, float* __restrict__ v, long n, float lr,
                                                    float b1, float b2, float eps, float wd, float bc1, float bc2) {
    const float ob1 = rsub(1.0f, b1), ob2 = rsub(1.0f, b2);
    const long stride = (long)gridDim.x * blockDim.x;
    long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    if (VEC) {
        for (; i < n / 4; i += stride) {
            float4 pp = reinterpret_cast<float4*>(p)[i];
            const float4 gg = reinterpret_cast<const float4*>(g)[i];
            float4 mm = reinterpret_cast<float4*>(m)[i];
            float4 vv = reinterpret_cast<float4*>(v)[i];
            adamw_one(pp.x, gg.x, mm.x, vv.x, lr, b1, b2, ob1, ob2, eps, wd, bc1, bc2);
            adamw_one(pp.y, gg.y, mm.y, vv.y, lr, b1, b2, ob1, ob2, eps, wd, bc1, bc2);
            adamw_one(pp.z, gg.z, mm.z, vv.z, lr, b1, b2, ob1, ob2, eps, wd, bc1, bc2);
            adamw_one(pp.w, gg.w, mm.w, vv.w, lr, b1, b2, ob1, ob2, eps, wd, bc1, bc2);
            reinterpret_cast<float4*>(p)[i] = pp;
            reinterpret_cast<float4*>(m)[i] = mm;
            reinterpret_cast<float4*>(v)[i] = vv;
        }
    } else {
        for (; i < n; i += stride) adamw_one(p[i], g[i], m[i], v[i], lr, b1, b2, ob1, ob2, eps, wd, bc1, bc2);
    }
}

hipError_t launch_adamw(float* p, const float* g, float* m, float* v, size_t n, float lr, float beta1, float beta2,
                        float eps, float weight_decay, float bc1, float bc2, hipStream_t st) {
    if (n == 0) return hipSuccess;
    if (n % 4 == 0 && aligned16(p) && aligned16(g) && aligned16(m) && aligned16(v))
        hipLaunchKernelGGL(adamw_kernel<true>, dim3(ew_blocks(n / 4)), dim3(256), 0, st, p, g, m, v, (long)n, lr,
                           beta1, beta2, eps, weight_decay, bc1, bc2);
    else
        hipLaunchKernelGGL(adamw_kernel<false>, dim3(ew_blocks(n)), dim3(256), 0, st, p, g, m, v, (long)n, lr, beta1,
                           beta2, eps, weight_decay, bc1, bc2);
    return hipGetLastError();
}

}  // namespace cfattn
