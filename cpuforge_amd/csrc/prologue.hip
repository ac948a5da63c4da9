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
    int srows;  // rows per block of the staged kernel
    int vec4;   // 4-column accesses: D % 8 == 0, D/8 divides 256, 16-byte aligned rows and tables
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

// The same rows, restructured for bandwidth: a block of srows rows of q or k
// (a contiguous range of memory) per workgroup of 256 threads.
//   - Qwen3 only: the rows are staged in LDS with coalesced loads and one lane
//     per row runs the sequential sum of squares above (LDS rows are D+1
//     floats apart, D even, so those lanes hit distinct banks); rstd goes to
//     LDS and to global memory.
//   - The rotation is elementwise: each thread takes column pairs (i, i+D/2)
//     of the block's rows, consecutive threads consecutive i, reading x (from
//     LDS or straight from global memory) and writing y with coalesced
//     accesses.  Every element's expression is the one above, so the result
//     is unchanged bit for bit.
constexpr int kStageMaxRows = 64;
constexpr int kStageMaxD = 256;
// Rows per block of the forward: 32 rows (17 KiB of LDS with the Qwen3 norm
// at head_dim 128) let eight workgroups share a CU instead of four (C4
// prologue forward 0.070 -> 0.059 ms); each row's expressions are unchanged.
constexpr int kFwdStageRows = 32;
// Rows per block, keeping a block's LDS within 64 KiB.
static int stage_rows(int hd, int nbuf) {
    const int r = 65536 / (nbuf * (hd + 1) * (int)sizeof(float));
    return r < kStageMaxRows ? r : kStageMaxRows;
}

// Copy n consecutive floats of `src` (rows of D) into LDS rows LD apart, 256
// threads, eight loads in flight per thread before their stores.  With
// `vec` (src 16-byte aligned, D a multiple of 4) the loads are 16 bytes
// each: a block of 64 rows of 128 floats is then one round of loads.
__device__ __forceinline__ void stage_rows_to_lds(float* dst, const float* src, int n, int D, int LD, int tid,
                                                  bool vec = false) {
    if (vec) {
        const float4* s4 = reinterpret_cast<const float4*>(src);
        const int n4 = n / 4;
        for (int j0 = 0; j0 < n4; j0 += 256 * 8) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int j = j0 + u * 256 + tid;
                v[u] = j < n4 ? s4[j] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int j = j0 + u * 256 + tid;
                if (j < n4) {
                    float* d = dst + (j * 4 / D) * LD + (j * 4) % D;
                    d[0] = v[u].x, d[1] = v[u].y, d[2] = v[u].z, d[3] = v[u].w;
                }
            }
        }
        return;
    }
    for (int j0 = 0; j0 < n; j0 += 256 * 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u * 256 + tid;
            v[u] = j < n ? src[j] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u * 256 + tid;
            if (j < n) dst[(j / D) * LD + j % D] = v[u];
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void prologue_fwd_staged_kernel(const ProParams p) {
#pragma clang fp contract(off)
    extern __shared__ float stage[];  // Qwen3: [srows][hd + 1] rows, then [srows] rstd
    const int tid = threadIdx.x;
    const long nbq = (p.rows_q + p.srows - 1) / p.srows;
    long blk = blockIdx.x;
    const bool isq = blk < nbq;
    if (!isq) blk -= nbq;
    const long rows = isq ? p.rows_q : p.rows_k;
    const long r0 = blk * p.srows;
    const int nr = (int)min((long)p.srows, rows - r0);
    const int D = p.hd, LD = p.hd + 1, half = p.half;
    const int heads = isq ? p.nh : p.nkv;
    const float* x = (isq ? p.q_pre : p.k_pre) + r0 * D;
    const float* w = isq ? p.qw : p.kw;
    float* srstd = stage + p.srows * LD;
    if (w) {
        stage_rows_to_lds(stage, x, nr * D, D, LD, tid, p.vec4);
        __syncthreads();
        if (tid < nr) {
            const float* xr = stage + tid * LD;
            float ss = 0.0f;
            for (int i = 0; i < D; i++) ss += xr[i] * xr[i];
            const float ms = ss / (float)D;
            const float inv = 1.0f / sqrtf(ms + p.eps);
            srstd[tid] = inv;
            (isq ? p.q_rstd : p.k_rstd)[r0 + tid] = inv;
        }
        __syncthreads();
    }
    T* y = static_cast<T*>(isq ? p.q_out : p.k_out) + r0 * D;
    if (p.vec4) {
        // Four consecutive columns per thread: half/4 threads per row, the
        // position (one division) per row; same expressions per element.
        const int cpr = half / 4, rpi = 256 / cpr;
        const int i = (tid % cpr) * 4;
        for (int row = tid / cpr; row < nr; row += rpi) {
            const int t = (int)(((r0 + row) / heads) % p.seq);
            const float4 c4 = *reinterpret_cast<const float4*>(p.cos + (long)(p.pos0 + t) * half + i);
            const float4 s4 = *reinterpret_cast<const float4*>(p.sin + (long)(p.pos0 + t) * half + i);
            float a[4], b[4];
            if (w) {
                const float inv = srstd[row];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    a[u] = stage[row * LD + i + u] * inv * w[i + u];
                    b[u] = stage[row * LD + i + half + u] * inv * w[i + half + u];
                }
            } else {
                const float4 a4 = *reinterpret_cast<const float4*>(x + (long)row * D + i);
                const float4 b4 = *reinterpret_cast<const float4*>(x + (long)row * D + i + half);
                a[0] = a4.x, a[1] = a4.y, a[2] = a4.z, a[3] = a4.w;
                b[0] = b4.x, b[1] = b4.y, b[2] = b4.z, b[3] = b4.w;
            }
            const float c[4] = {c4.x, c4.y, c4.z, c4.w}, sv[4] = {s4.x, s4.y, s4.z, s4.w};
            T lo[4], hi[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                lo[u] = from_f32<T>(a[u] * c[u] - b[u] * sv[u]);
                hi[u] = from_f32<T>(b[u] * c[u] + a[u] * sv[u]);
            }
            T* yr = y + (long)row * D + i;
            if constexpr (sizeof(T) == 2) {
                *reinterpret_cast<uint2*>(yr) = make_uint2((uint32_t)lo[0] | ((uint32_t)lo[1] << 16),
                                                           (uint32_t)lo[2] | ((uint32_t)lo[3] << 16));
                *reinterpret_cast<uint2*>(yr + half) = make_uint2((uint32_t)hi[0] | ((uint32_t)hi[1] << 16),
                                                                  (uint32_t)hi[2] | ((uint32_t)hi[3] << 16));
            } else {
                *reinterpret_cast<float4*>(yr) = make_float4(lo[0], lo[1], lo[2], lo[3]);
                *reinterpret_cast<float4*>(yr + half) = make_float4(hi[0], hi[1], hi[2], hi[3]);
            }
        }
        return;
    }
    for (int j = tid; j < nr * half; j += 256) {
        const int row = j / half, i = j % half;
        const int t = (int)(((r0 + row) / heads) % p.seq);
        float x1, x2;
        if (w) {
            const float inv = srstd[row];
            x1 = stage[row * LD + i] * inv * w[i];
            x2 = stage[row * LD + i + half] * inv * w[i + half];
        } else {
            x1 = x[(long)row * D + i];
            x2 = x[(long)row * D + i + half];
        }
        const float c = p.cos[(long)(p.pos0 + t) * half + i], sn = p.sin[(long)(p.pos0 + t) * half + i];
        y[(long)row * D + i] = from_f32<T>(x1 * c - x2 * sn);
        y[(long)row * D + i + half] = from_f32<T>(x2 * c + x1 * sn);
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
    int srows;  // rows per block of the staged kernel
    int unrot;  // 0: dq/dk are already unrotated (the backward's kEpiUnrotStore epilogue)
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
    auto dyv = [&](int i) { return p.unrot ? unrotate(g, cs, sn, i, p.half) : g[i]; };
    if (!w) {
        for (int i = 0; i < p.hd; i++) dx[i] += dyv(i);
        return;
    }
    const float* x = (isq ? p.q_pre : p.k_pre) + r * p.hd;
    const float inv = (isq ? p.q_rstd : p.k_rstd)[r];
    float dot = 0.0f;
    for (int i = 0; i < p.hd; i++) dot += dyv(i) * w[i] * x[i] * inv;
    const float mean = dot / (float)p.hd;
    for (int i = 0; i < p.hd; i++) {
        const float dy = dyv(i);
        const float xhat = x[i] * inv;
        dx[i] += inv * (dy * w[i] - xhat * mean);
    }
}

// The same rows restructured like prologue_fwd_staged_kernel, elementwise
// over column pairs (i, i+D/2) with the expressions above and a coalesced +=
// into dq_pre/dk_pre.  Qwen3 first writes the unrotated gradient dy and stages
// the input rows and w in LDS, then runs the sequential dot product with one
// lane per row reading only LDS.
__global__ __launch_bounds__(256) void prologue_bwd_rows_staged_kernel(const ProBwdParams p) {
#pragma clang fp contract(off)
    // Qwen3: [srows][hd + 1] dy rows, [srows][hd + 1] input rows, [srows] mean, [hd] w
    extern __shared__ float stage[];
    const int tid = threadIdx.x;
    const long nbq = (p.rows_q + p.srows - 1) / p.srows;
    long blk = blockIdx.x;
    const bool isq = blk < nbq;
    if (!isq) blk -= nbq;
    const long rows = isq ? p.rows_q : p.rows_k;
    const long r0 = blk * p.srows;
    const int nr = (int)min((long)p.srows, rows - r0);
    const int D = p.hd, LD = p.hd + 1, half = p.half;
    const int heads = isq ? p.nh : p.nkv;
    const float* w = isq ? p.qw : p.kw;
    const float* g = (isq ? p.dq : p.dk) + r0 * D;
    const float* x = (isq ? p.q_pre : p.k_pre) + r0 * D;
    const float* rstd = w ? (isq ? p.q_rstd : p.k_rstd) + r0 : nullptr;
    float* sdy = stage;
    float* sx = stage + p.srows * LD;
    float* smean = stage + 2 * p.srows * LD;
    float* sw = smean + p.srows;
    float* dx = (isq ? p.dq_pre : p.dk_pre) + r0 * D;
    auto dy_pair = [&](int row, int i, float& dy1, float& dy2) {
        const int t = (int)(((r0 + row) / heads) % p.seq);
        const float* cs = p.cos + (long)(p.pos0 + t) * half;
        const float* sn = p.sin + (long)(p.pos0 + t) * half;
        const float* gr = g + (long)row * D;
        if (p.unrot) {
            dy1 = unrotate(gr, cs, sn, i, half);
            dy2 = unrotate(gr, cs, sn, i + half, half);
        } else {
            dy1 = gr[i];
            dy2 = gr[i + half];
        }
    };
    if (!w) {
        for (int j = tid; j < nr * half; j += 256) {
            const int row = j / half, i = j % half;
            float dy1, dy2;
            dy_pair(row, i, dy1, dy2);
            dx[(long)row * D + i] += dy1;
            dx[(long)row * D + i + half] += dy2;
        }
        return;
    }
    stage_rows_to_lds(sx, x, nr * D, D, LD, tid);
    for (int i = tid; i < D; i += 256) sw[i] = w[i];
    for (int j = tid; j < nr * half; j += 256) {
        const int row = j / half, i = j % half;
        float dy1, dy2;
        dy_pair(row, i, dy1, dy2);
        sdy[row * LD + i] = dy1;
        sdy[row * LD + i + half] = dy2;
    }
    __syncthreads();
    if (tid < nr) {
        const float* dyr = sdy + tid * LD;
        const float* xr = sx + tid * LD;
        const float inv = rstd[tid];
        float dot = 0.0f;
        for (int i = 0; i < D; i++) dot += dyr[i] * sw[i] * xr[i] * inv;
        smean[tid] = dot / (float)D;
    }
    // This block's share of the norm-gain gradient, in row order:
    // partial[block][i] = sum over its rows of dy * xhat (reduced over blocks
    // by prologue_bwd_dw_reduce_kernel).
    for (int i = tid; i < D; i += 256) {
        float acc = 0.0f;
        for (int row = 0; row < nr; row++) acc += sdy[row * LD + i] * (sx[row * LD + i] * rstd[row]);
        p.partial[(isq ? blk : nbq + blk) * D + i] = acc;
    }
    __syncthreads();
    for (int j = tid; j < nr * half; j += 256) {
        const int row = j / half, i = j % half;
        const float inv = rstd[row], mean = smean[row];
        const float dy1 = sdy[row * LD + i], dy2 = sdy[row * LD + i + half];
        const float xh1 = sx[row * LD + i] * inv, xh2 = sx[row * LD + i + half] * inv;
        dx[(long)row * D + i] += inv * (dy1 * sw[i] - xh1 * mean);
        dx[(long)row * D + i + half] += inv * (dy2 * sw[i + half] - xh2 * mean);
    }
}

// The norm backward of the staged kernel, vectorised, for head dims D = 8 G
// (G a power of two up to 32) with 16-byte aligned rows and tables: G lanes
// own a row, lane j of the group holding head dims 8j .. 8j+7 in registers
// (two 16-byte loads of each operand), so a workgroup covers 256 / G rows per
// pass and p.chunk_rows rows in all.  Per element the expressions are the
// staged kernel's; the row dot of dy w x rstd is summed over the lane's
// eight dims in order and then over the G lanes by a fixed xor-shuffle tree,
// so results are reproducible bit for bit (the staged kernel sums each row
// left to right: the two differ in the last bits of the dot).  The lane also
// keeps the gain-gradient sums of its eight dims over its rows, and the
// workgroup adds its 256 / G row slots in slot order into partial[chunk],
// which prologue_bwd_dw_reduce_kernel reduces over chunks as before.  The
// inverse RoPE reads the partner half of the gradient row (dims i +- D/2) from
// the cache lines the neighbouring lanes load.
template <int G>
__global__ __launch_bounds__(256) void prologue_bwd_norm_vec_kernel(const ProBwdParams p) {
#pragma clang fp contract(off)
    constexpr int D = 8 * G, SLOTS = 256 / G;
    __shared__ float red[SLOTS][D];
    const int tid = threadIdx.x, j = tid % G, slot = tid / G;
    const long nbq = (p.rows_q + p.chunk_rows - 1) / p.chunk_rows;
    long blk = blockIdx.x;
    const bool isq = blk < nbq;
    if (!isq) blk -= nbq;
    const long rows = isq ? p.rows_q : p.rows_k;
    const long r_begin = blk * p.chunk_rows, r_end = min(rows, r_begin + p.chunk_rows);
    const int heads = isq ? p.nh : p.nkv, half = D / 2;
    const float* gbase = isq ? p.dq : p.dk;
    const float* xbase = isq ? p.q_pre : p.k_pre;
    const float* rstd = isq ? p.q_rstd : p.k_rstd;
    float* dxbase = isq ? p.dq_pre : p.dk_pre;
    const int d0 = 8 * j;                   // the lane's first head dim
    const int dp = d0 < half ? d0 + half : d0 - half;  // its partner dims under the rotation
    const int dc = d0 < half ? d0 : d0 - half;         // its cos/sin index
    float w[8], acc[8];
    {
        const float* wp = (isq ? p.qw : p.kw) + d0;
        const float4 a = *reinterpret_cast<const float4*>(wp), b = *reinterpret_cast<const float4*>(wp + 4);
        w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = b.x, w[5] = b.y, w[6] = b.z, w[7] = b.w;
    }
#pragma unroll
    for (int i = 0; i < 8; i++) acc[i] = 0.0f;
    auto load8 = [](const float* s, float (&v)[8]) {
        const float4 a = *reinterpret_cast<const float4*>(s), b = *reinterpret_cast<const float4*>(s + 4);
        v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
    };
    for (long r0 = r_begin; r0 < r_end; r0 += SLOTS) {
        const long r = r0 + slot;
        const bool ok = r < r_end;
        float dy[8], x[8], inv = 0.0f;
        if (ok) {
            const float* g = gbase + r * D;
            if (p.unrot) {
                const int t = (int)((r / heads) % p.seq);
                float gs[8], gp[8], c[8], sn[8];
                load8(g + d0, gs);
                load8(g + dp, gp);
                load8(p.cos + (long)(p.pos0 + t) * half + dc, c);
                load8(p.sin + (long)(p.pos0 + t) * half + dc, sn);
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    // unrotate(): element i < half is g[i] c - g[i + half] s,
                    // element i >= half g[i] c + g[i - half] s, s = -sin.
                    const float s = -1.0f * sn[i];
                    dy[i] = d0 < half ? gs[i] * c[i] - gp[i] * s : gs[i] * c[i] + gp[i] * s;
                }
            } else {
                load8(g + d0, dy);
            }
            load8(xbase + r * D + d0, x);
            inv = rstd[r];
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) dy[i] = 0.0f, x[i] = 0.0f;
        }
        float dot = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) dot += dy[i] * w[i] * x[i] * inv;
#pragma unroll
        for (int off = G / 2; off >= 1; off >>= 1) dot += __shfl_xor(dot, off, G);
        if (ok) {
            const float mean = dot / (float)D;
            float* dx = dxbase + r * D + d0;
            float o[8];
            load8(dx, o);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float xh = x[i] * inv;
                o[i] += inv * (dy[i] * w[i] - xh * mean);
                acc[i] += dy[i] * (x[i] * inv);
            }
            *reinterpret_cast<float4*>(dx) = make_float4(o[0], o[1], o[2], o[3]);
            *reinterpret_cast<float4*>(dx + 4) = make_float4(o[4], o[5], o[6], o[7]);
        }
    }
    // The gain-gradient sums of the workgroup's row slots, added in slot order.
#pragma unroll
    for (int i = 0; i < 8; i++) red[slot][d0 + i] = acc[i];
    __syncthreads();
    for (int d = tid; d < D; d += 256) {
        float s = 0.0f;
        for (int k = 0; k < SLOTS; k++) s += red[k][d];
        p.partial[(isq ? blk : nbq + blk) * D + d] = s;
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
        const float dy = p.unrot ? unrotate(gbase + r * p.hd, cs, sn, i, p.half) : gbase[r * p.hd + i];
        const float xhat = xbase[r * p.hd + i] * rstd[r];
        acc += dy * xhat;
    }
    const long slot = isq ? chunk : (long)p.n_chunks_q + chunk;
    p.partial[slot * p.hd + i] = acc;
}

// dw[i] += sum over chunks of partial[..][chunk][i]: one workgroup per (q or k,
// i).  Thread t adds chunks t, t+256, ... in order, then a fixed tree over the
// 256 thread sums, so the result does not depend on scheduling.
__global__ __launch_bounds__(256) void prologue_bwd_dw_reduce_kernel(const ProBwdParams p) {
#pragma clang fp contract(off)
    __shared__ float red[256];
    const int tid = threadIdx.x;
    const int i = blockIdx.x % p.hd;
    const bool isq = blockIdx.x < p.hd;
    const int n = isq ? p.n_chunks_q : p.n_chunks_k;
    if (n == 0) return;  // no rows of this side in the launch: its gradient is left as it is
    const long base = isq ? 0 : p.n_chunks_q;
    float acc = 0.0f;
    for (int c = tid; c < n; c += 256) acc += p.partial[(base + c) * p.hd + i];
    red[tid] = acc;
    __syncthreads();
#pragma unroll
    for (int w = 128; w >= 1; w >>= 1) {
        if (tid < w) red[tid] = red[tid] + red[tid + w];
        __syncthreads();
    }
    if (tid == 0) (isq ? p.dqw : p.dkw)[i] += red[0];
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
    const uintptr_t al = 16;
    p.vec4 = d.hd % 8 == 0 && 256 % (d.hd / 8) == 0 && (uintptr_t)q_pre % al == 0 && (uintptr_t)k_pre % al == 0 &&
             (uintptr_t)q_out % al == 0 && (uintptr_t)k_out % al == 0 && (uintptr_t)pr.cos % al == 0 &&
             (uintptr_t)pr.sin % al == 0;
    TimedLaunch tl(timer, kKernProFwd, st);
    if (d.hd <= kStageMaxD) {
        // The rstd column counted as one more float per row.
        p.srows = stage_rows(d.hd + 1, 1);
        if (p.srows > kFwdStageRows) p.srows = kFwdStageRows;
        const long blocks = (p.rows_q + p.srows - 1) / p.srows + (p.rows_k + p.srows - 1) / p.srows;
        if (blocks > 0x7fffffffL) return hipErrorInvalidConfiguration;
        const size_t lds = pr.qw ? (size_t)p.srows * (d.hd + 2) * sizeof(float) : 0;
        if (dt == kBF16)
            hipLaunchKernelGGL(prologue_fwd_staged_kernel<bf16_bits>, dim3((unsigned)blocks), dim3(256), lds, st, p);
        else
            hipLaunchKernelGGL(prologue_fwd_staged_kernel<float>, dim3((unsigned)blocks), dim3(256), lds, st, p);
        return hipGetLastError();
    }
    const unsigned grid = (unsigned)((rows + 255) / 256);
    if (dt == kBF16)
        hipLaunchKernelGGL(prologue_fwd_kernel<bf16_bits>, dim3(grid), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(prologue_fwd_kernel<float>, dim3(grid), dim3(256), 0, st, p);
    return hipGetLastError();
}

static constexpr int kChunkRows = 32;  // rows per partial sum of the norm-gain gradient (row-per-thread path)
static constexpr int kVecRows = 256;  // rows per workgroup (and gain-gradient chunk) of the vectorised norm backward

static bool aligned16(std::initializer_list<const void*> ptrs) {
    for (const void* q : ptrs)
        if (reinterpret_cast<uintptr_t>(q) % 16 != 0) return false;
    return true;
}
template <typename... T>
static bool aligned16(const T*... ptrs) {
    return aligned16({static_cast<const void*>(ptrs)...});
}

// Rows per partial sum of the norm-gain gradient: the staged kernel's block,
// else kChunkRows.
static int dw_chunk_rows(int hd) { return hd <= kStageMaxD ? stage_rows(hd + 2, 2) : kChunkRows; }

size_t prologue_bwd_scratch_floats(const Dims& d) {
    const long rq = (long)d.batch * d.seq * d.nh, rk = (long)d.batch * d.seq * d.nkv;
    const long cr = dw_chunk_rows(d.hd);
    const long nq = (rq + cr - 1) / cr, nk = (rk + cr - 1) / cr;
    return (size_t)((nq + nk) * d.hd);
}

hipError_t launch_prologue_bwd(const Dims& d, const Prologue& pr, const float* dq, const float* dk,
                               const float* q_pre, const float* k_pre, const float* q_rstd, const float* k_rstd,
                               float* dq_pre, float* dk_pre, float* dqw, float* dkw, float* partial, hipStream_t st,
                               KernelTimer* timer, bool unrotated, bool k_only) {
    ProBwdParams p{};
    p.unrot = unrotated ? 0 : 1;
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
    p.rows_q = k_only ? 0 : (long)d.batch * d.seq * d.nh;
    p.rows_k = (long)d.batch * d.seq * d.nkv;
    p.chunk_rows = dw_chunk_rows(d.hd);
    p.n_chunks_q = (int)((p.rows_q + p.chunk_rows - 1) / p.chunk_rows);
    p.n_chunks_k = (int)((p.rows_k + p.chunk_rows - 1) / p.chunk_rows);
    const long rows = p.rows_q + p.rows_k;
    if (rows == 0) return hipSuccess;
    TimedLaunch tl(timer, kKernProBwd, st);
    const int G = d.hd / 8;
    const bool vec = pr.qw && d.hd % 8 == 0 && (G == 4 || G == 8 || G == 16 || G == 32) &&
                     aligned16(dq, dk, q_pre, k_pre, dq_pre, dk_pre, pr.qw, pr.kw, pr.cos, pr.sin) &&
                     (d.hd / 2) % 4 == 0;
    if (vec) {
        // kVecRows rows per workgroup (a chunk of the gain-gradient sum);
        // fewer chunks than the staged kernel's, so the scratch suffices.
        p.chunk_rows = kVecRows;
        p.n_chunks_q = (int)((p.rows_q + p.chunk_rows - 1) / p.chunk_rows);
        p.n_chunks_k = (int)((p.rows_k + p.chunk_rows - 1) / p.chunk_rows);
        const long blocks = (long)p.n_chunks_q + p.n_chunks_k;
        if (blocks > 0x7fffffffL) return hipErrorInvalidConfiguration;
        switch (G) {
            case 4: hipLaunchKernelGGL(prologue_bwd_norm_vec_kernel<4>, dim3((unsigned)blocks), dim3(256), 0, st, p); break;
            case 8: hipLaunchKernelGGL(prologue_bwd_norm_vec_kernel<8>, dim3((unsigned)blocks), dim3(256), 0, st, p); break;
            case 16: hipLaunchKernelGGL(prologue_bwd_norm_vec_kernel<16>, dim3((unsigned)blocks), dim3(256), 0, st, p); break;
            default: hipLaunchKernelGGL(prologue_bwd_norm_vec_kernel<32>, dim3((unsigned)blocks), dim3(256), 0, st, p); break;
        }
    } else if (d.hd <= kStageMaxD) {
        p.srows = p.chunk_rows;  // stage_rows(hd + 2, 2): the mean column and w counted as more floats per row
        const long blocks = (p.rows_q + p.srows - 1) / p.srows + (p.rows_k + p.srows - 1) / p.srows;
        if (blocks > 0x7fffffffL) return hipErrorInvalidConfiguration;
        const size_t lds = pr.qw ? (2 * (size_t)p.srows * (d.hd + 1) + p.srows + d.hd) * sizeof(float) : 0;
        hipLaunchKernelGGL(prologue_bwd_rows_staged_kernel, dim3((unsigned)blocks), dim3(256), lds, st, p);
    } else {
        hipLaunchKernelGGL(prologue_bwd_rows_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, p);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !pr.qw) return e;
    if (d.hd > kStageMaxD) {  // the staged kernel writes the partial sums itself
        hipLaunchKernelGGL(prologue_bwd_dw_partial_kernel, dim3(p.n_chunks_q + p.n_chunks_k), dim3(256), 0, st, p);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(prologue_bwd_dw_reduce_kernel, dim3(2 * d.hd), dim3(256), 0, st, p);
    return hipGetLastError();
}

hipError_t launch_norm_gain_reduce(float* part, int nq, int nk, int hd, float* dqw, float* dkw, hipStream_t st) {
    if (hd <= 0) return hipSuccess;
    ProBwdParams p{};
    p.partial = part;
    p.n_chunks_q = nq;
    p.n_chunks_k = nk;
    p.hd = hd;
    p.dqw = dqw;
    p.dkw = dkw;
    hipLaunchKernelGGL(prologue_bwd_dw_reduce_kernel, dim3(2 * hd), dim3(256), 0, st, p);
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
