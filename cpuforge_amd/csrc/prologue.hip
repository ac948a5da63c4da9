// Attention prologue and its backward on gfx950, plus small elementwise
// helpers.
//
// Forward (crates/model/src/layer.rs:104-116): for every (token, head) row of
// q_pre [.., n_heads, D] and k_pre [.., n_kv, D]
//   [Qwen3 only] rstd = 1/sqrt(mean(x^2) + eps), x = x * rstd * w
//                 (crates/core/src/ops/rmsnorm.rs:4-26)
//   RoPE rotate-half at position pos0 + t: lo' = x1 c - x2 s, hi' = x2 c + x1 s
//                 (crates/core/src/ops/rope.rs:71-89)
// then the row is written in the attention's compute dtype.  One thread per
// row keeps the reference's sequential f32 order, and contraction is off, so
// in fp32 mode the rows equal the reference's bit for bit.
//
// Backward (layer.rs:191-206): inverse RoPE of dq/dk (sine negated), then
// [Qwen3] dx += rstd (dy w - xhat mean(dy w xhat)),  dw += sum_rows dy xhat
// (rmsnorm.rs:32-67).  dw is reduced without atomics: per-chunk partial sums
// in a fixed row order, then a fixed-order sum over chunks.
#include "cfattn_common.hpp"
#include "cfattn_kernels.hpp"

namespace cfattn {

struct ProParams {
    const float* q_pre;
    const float* k_pre;
    void* q_out;
    void* k_out;
    float* q_rstd;
    float* k_rstd;
    const float* qw;
    const float* kw;
    float eps;
    const float* cos;
    const float* sin;
    int half, pos0;
    int seq, nh, nkv, hd;
    long rows_q, rows_k;
};

template <typename T>
__global__ __launch_bounds__(256) void prologue_fwd_kernel(const ProParams p) {
#pragma clang fp contract(off)
    long r = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const bool isq = r < p.rows_q;
    if (!isq) r -= p.rows_q;
    if (r >= (isq ? p.rows_q : p.rows_k)) return;
    const int heads = isq ? p.nh : p.nkv;
    const int t = (int)((r / heads) % p.seq);
    const float* x = (isq ? p.q_pre : p.k_pre) + r * p.hd;
    T* y = static_cast<T*>(isq ? p.q_out : p.k_out) + r * p.hd;
    const float* w = isq ? p.qw : p.kw;
    float inv = 1.0f;
    if (w) {
        float ss = 0.0f;
        for (int i = 0; i < p.hd; i++) ss += x[i] * x[i];
        const float ms = ss / (float)p.hd;
        inv = 1.0f / sqrtf(ms + p.eps);
        (isq ? p.q_rstd : p.k_rstd)[r] = inv;
    }
    const float* cs = p.cos + (long)(p.pos0 + t) * p.half;
    const float* sn = p.sin + (long)(p.pos0 + t) * p.half;
    for (int i = 0; i < p.half; i++) {
        float x1 = x[i], x2 = x[i + p.half];
        if (w) {
            x1 = x1 * inv * w[i];
            x2 = x2 * inv * w[i + p.half];
        }
        const float c = cs[i], s = sn[i];
        y[i] = from_f32<T>(x1 * c - x2 * s);
        y[i + p.half] = from_f32<T>(x2 * c + x1 * s);
    }
}

struct ProBwdParams {
    const float* dq;
    const float* dk;
    const float* q_pre;
    const float* k_pre;
    const float* q_rstd;
    const float* k_rstd;
    const float* qw;
    const float* kw;
    float* dq_pre;
    float* dk_pre;
    float* dqw;
    float* dkw;
    float* partial;  // [2][n_chunks][hd]
    const float* cos;
    const float* sin;
    int half, pos0;
    int seq, nh, nkv, hd;
    long rows_q, rows_k;
    int chunk_rows, n_chunks_q, n_chunks_k;
};

// Inverse rotation of element i of a gradient row (sine negated, as
// RopeCache::apply with inverse=true).
__device__ __forceinline__ float unrotate(const float* g, const float* cs, const float* sn, int i, int half) {
#pragma clang fp contract(off)
    if (i < half) {
        const float c = cs[i], s = -1.0f * sn[i];
        return g[i] * c - g[i + half] * s;
    }
    const int j = i - half;
    const float c = cs[j], s = -1.0f * sn[j];
    return g[i] * c + g[j] * s;
}

__global__ __launch_bounds__(256) void prologue_bwd_rows_kernel(const ProBwdParams p) {
#pragma clang fp contract(off)
    long r = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const bool isq = r < p.rows_q;
    if (!isq) r -= p.rows_q;
    if (r >= (isq ? p.rows_q : p.rows_k)) return;
    const int heads = isq ? p.nh : p.nkv;
    const int t = (int)((r / heads) % p.seq);
    const float* g = (isq ? p.dq : p.dk) + r * p.hd;
    float* dx = (isq ? p.dq_pre : p.dk_pre) + r * p.hd;
    const float* w = isq ? p.qw : p.kw;
    const float* cs = p.cos + (long)(p.pos0 + t) * p.half;
    const float* sn = p.sin + (long)(p.pos0 + t) * p.half;
    if (!w) {
        for (int i = 0; i < p.hd; i++) dx[i] += unrotate(g, cs, sn, i, p.half);
        return;
    }
    const float* x = (isq ? p.q_pre : p.k_pre) + r * p.hd;
    const float inv = (isq ? p.q_rstd : p.k_rstd)[r];
    float dot = 0.0f;
    for (int i = 0; i < p.hd; i++) dot += unrotate(g, cs, sn, i, p.half) * w[i] * x[i] * inv;
    const float mean = dot / (float)p.hd;
    for (int i = 0; i < p.hd; i++) {
        const float dy = unrotate(g, cs, sn, i, p.half);
        const float xhat = x[i] * inv;
        dx[i] += inv * (dy * w[i] - xhat * mean);
    }
}

// partial[which][chunk][i] = sum over the chunk's rows of dy[row][i] * xhat[row][i].
__global__ __launch_bounds__(256) void prologue_bwd_dw_partial_kernel(const ProBwdParams p) {
#pragma clang fp contract(off)
    const int i = threadIdx.x;
    if (i >= p.hd) return;
    int chunk = blockIdx.x;
    const bool isq = chunk < p.n_chunks_q;
    if (!isq) chunk -= p.n_chunks_q;
    const long rows = isq ? p.rows_q : p.rows_k;
    const int heads = isq ? p.nh : p.nkv;
    const float* gbase = isq ? p.dq : p.dk;
    const float* xbase = isq ? p.q_pre : p.k_pre;
    const float* rstd = isq ? p.q_rstd : p.k_rstd;
    const long r0 = (long)chunk * p.chunk_rows;
    const long r1 = r0 + p.chunk_rows < rows ? r0 + p.chunk_rows : rows;
    float acc = 0.0f;
    for (long r = r0; r < r1; r++) {
        const int t = (int)((r / heads) % p.seq);
        const float* cs = p.cos + (long)(p.pos0 + t) * p.half;
        const float* sn = p.sin + (long)(p.pos0 + t) * p.half;
        const float dy = unrotate(gbase + r * p.hd, cs, sn, i, p.half);
        const float xhat = xbase[r * p.hd + i] * rstd[r];
        acc += dy * xhat;
    }
    const long slot = isq ? chunk : (long)p.n_chunks_q + chunk;
    p.partial[slot * p.hd + i] = acc;
}

__global__ __launch_bounds__(256) void prologue_bwd_dw_reduce_kernel(const ProBwdParams p) {
    const int i = threadIdx.x;
    if (i >= p.hd) return;
    const bool isq = blockIdx.x == 0;
    const int n = isq ? p.n_chunks_q : p.n_chunks_k;
    const long base = isq ? 0 : p.n_chunks_q;
    float acc = 0.0f;
    for (int c = 0; c < n; c++) acc += p.partial[(base + c) * p.hd + i];
    float* dw = isq ? p.dqw : p.dkw;
    dw[i] += acc;
}

__global__ __launch_bounds__(256) void f32_to_bf16_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst,
                                                          size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = f32_to_bf16(src[i]);
}

__global__ __launch_bounds__(256) void fill_zero_kernel(float* __restrict__ dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = 0.0f;
}

static unsigned grid_for(size_t n) {
    size_t g = (n + 255) / 256;
    if (g > 65536) g = 65536;
    return (unsigned)(g ? g : 1);
}

hipError_t launch_prologue_fwd(Dtype dt, const Dims& d, const Prologue& pr, const float* q_pre, const float* k_pre,
                               void* q_out, void* k_out, float* q_rstd, float* k_rstd, hipStream_t st,
                               KernelTimer* timer) {
    ProParams p{};
    p.q_pre = q_pre;
    p.k_pre = k_pre;
    p.q_out = q_out;
    p.k_out = k_out;
    p.q_rstd = q_rstd;
    p.k_rstd = k_rstd;
    p.qw = pr.qw;
    p.kw = pr.kw;
    p.eps = pr.eps;
    p.cos = pr.cos;
    p.sin = pr.sin;
    p.half = d.hd / 2;
    p.pos0 = pr.pos0;
    p.seq = d.seq;
    p.nh = d.nh;
    p.nkv = d.nkv;
    p.hd = d.hd;
    p.rows_q = (long)d.batch * d.seq * d.nh;
    p.rows_k = (long)d.batch * d.seq * d.nkv;
    const long rows = p.rows_q + p.rows_k;
    if (rows == 0) return hipSuccess;
    const unsigned grid = (unsigned)((rows + 255) / 256);
    TimedLaunch tl(timer, kKernProFwd, st);
    if (dt == kBF16)
        hipLaunchKernelGGL(prologue_fwd_kernel<bf16_bits>, dim3(grid), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(prologue_fwd_kernel<float>, dim3(grid), dim3(256), 0, st, p);
    return hipGetLastError();
}

static constexpr int kChunkRows = 256;

size_t prologue_bwd_scratch_floats(const Dims& d) {
    const long rq = (long)d.batch * d.seq * d.nh, rk = (long)d.batch * d.seq * d.nkv;
    const long nq = (rq + kChunkRows - 1) / kChunkRows, nk = (rk + kChunkRows - 1) / kChunkRows;
    return (size_t)((nq + nk) * d.hd);
}

hipError_t launch_prologue_bwd(const Dims& d, const Prologue& pr, const float* dq, const float* dk,
                               const float* q_pre, const float* k_pre, const float* q_rstd, const float* k_rstd,
                               float* dq_pre, float* dk_pre, float* dqw, float* dkw, float* partial, hipStream_t st,
                               KernelTimer* timer) {
    ProBwdParams p{};
    p.dq = dq;
    p.dk = dk;
    p.q_pre = q_pre;
    p.k_pre = k_pre;
    p.q_rstd = q_rstd;
    p.k_rstd = k_rstd;
    p.qw = pr.qw;
    p.kw = pr.kw;
    p.dq_pre = dq_pre;
    p.dk_pre = dk_pre;
    p.dqw = dqw;
    p.dkw = dkw;
    p.partial = partial;
    p.cos = pr.cos;
    p.sin = pr.sin;
    p.half = d.hd / 2;
    p.pos0 = pr.pos0;
    p.seq = d.seq;
    p.nh = d.nh;
    p.nkv = d.nkv;
    p.hd = d.hd;
    p.rows_q = (long)d.batch * d.seq * d.nh;
    p.rows_k = (long)d.batch * d.seq * d.nkv;
    p.chunk_rows = kChunkRows;
    p.n_chunks_q = (int)((p.rows_q + kChunkRows - 1) / kChunkRows);
    p.n_chunks_k = (int)((p.rows_k + kChunkRows - 1) / kChunkRows);
    const long rows = p.rows_q + p.rows_k;
    if (rows == 0) return hipSuccess;
    TimedLaunch tl(timer, kKernProBwd, st);
    hipLaunchKernelGGL(prologue_bwd_rows_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !pr.qw) return e;
    hipLaunchKernelGGL(prologue_bwd_dw_partial_kernel, dim3(p.n_chunks_q + p.n_chunks_k), dim3(256), 0, st, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(prologue_bwd_dw_reduce_kernel, dim3(2), dim3(256), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_f32_to_bf16(const float* src, uint16_t* dst, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(f32_to_bf16_kernel, dim3(grid_for(n)), dim3(256), 0, st, src, dst, n);
    return hipGetLastError();
}

hipError_t launch_fill_zero(float* dst, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(n)), dim3(256), 0, st, dst, n);
    return hipGetLastError();
}

}  // namespace cfattn
