// LoRA adapter products of Linear::forward / Linear::backward
// (crates/model/src/linear.rs:56-91) as f32 kernels.  Every product here has
// the adapter rank R (4, 8 or 16) as one of its dimensions, so as a GEMM it
// is a thin, memory-bound shape a library tiles poorly (about 15 us a call
// for a few MB of traffic at the SmolLM-135M shapes).  Here each is a
// streaming pass over its big operand, split so that thousands of waves keep
// many loads in flight:
//   forward   xs = scale * x A^T      rowdot partials over chunks of `in`, then
//             y += xs B^T             the update kernel sums them in chunk order
//   backward  dxa = scale * dy B      (the same pair of kernels)
//             dx += dxa A
//             gb += dy^T xs,  ga += dxa^T x: per-chunk partial sums over the
//             tokens, then a reduction of the chunks in order.
// Every sum runs in a fixed order (no atomics): results are reproducible bit
// for bit.  The caller guarantees 16-byte aligned rows (in and out multiples
// of four, aligned base pointers).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "cfops_kernels.hpp"

namespace cfattn {
namespace {

constexpr int kDotRows = 64;   // rows per rowdot workgroup
constexpr int kDotChunk = 64;  // k values per rowdot partial
constexpr int kUpdRows = 16;   // rows per update workgroup (4 per wave)
constexpr int kUpdCols = 256;  // columns per update workgroup (4 per lane)
constexpr int kGradCols = 64;  // columns per gradient workgroup (1 per lane)

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// P[c][row][j] = sum over k in chunk c of src[row][k] * m(j, k), where
// m(j, k) = M[j*K + k] (MROW: M is [R x K], the forward's A) or M[k*R + j]
// (the backward's B, [K x R]).  Four lanes share a row, 16 values of the
// chunk each, and add their sums pairwise (the same order in every lane).
template <int R, bool MROW>
__global__ __launch_bounds__(256) void lora_rowdot_kernel(const float* __restrict__ src, const float* __restrict__ M,
                                                          int t, int K, float* __restrict__ P) {
    // m(j, k) of the chunk, k-major with rows padded to R + 4 floats: lane kq
    // of a row takes k = 16q + 4kq + s, so the four lanes of a row read rows
    // 4 apart, which the padding puts on distinct banks.
    constexpr int MS = R + 4;
    __shared__ __attribute__((aligned(16))) float sm[kDotChunk * MS];
    const int c = blockIdx.y, k0 = c * kDotChunk;
    const int tid = threadIdx.x;
    const int r = tid >> 2, kq = tid & 3;
    const int row = blockIdx.x * kDotRows + r;
    // The row's values first: their latency overlaps the staging below.
    float xv[16];
    const float* sp = src + (size_t)min(row, t - 1) * K + k0 + kq * 4;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 v = (k0 + q * 16 + kq * 4 < K) ? ld4(sp + q * 16) : make_float4(0.f, 0.f, 0.f, 0.f);
        xv[4 * q] = v.x, xv[4 * q + 1] = v.y, xv[4 * q + 2] = v.z, xv[4 * q + 3] = v.w;
    }
    for (int e = tid; e < R * kDotChunk; e += 256) {
        const int j = MROW ? e / kDotChunk : e % R;
        const int kk = MROW ? e % kDotChunk : e / R;
        const int k = k0 + kk;
        sm[kk * MS + j] = k < K ? (MROW ? M[(size_t)j * K + k] : M[(size_t)k * R + j]) : 0.0f;
    }
    __syncthreads();
    float acc[R];
#pragma unroll
    for (int j = 0; j < R; j++) acc[j] = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
        for (int s4 = 0; s4 < 4; s4++) {
            const float xe = xv[4 * q + s4];
            const float* mk = &sm[(16 * q + 4 * kq + s4) * MS];
#pragma unroll
            for (int j = 0; j < R; j += 4) {
                const float4 m4 = *reinterpret_cast<const float4*>(mk + j);
                acc[j] = __builtin_fmaf(xe, m4.x, acc[j]);
                acc[j + 1] = __builtin_fmaf(xe, m4.y, acc[j + 1]);
                acc[j + 2] = __builtin_fmaf(xe, m4.z, acc[j + 2]);
                acc[j + 3] = __builtin_fmaf(xe, m4.w, acc[j + 3]);
            }
        }
#pragma unroll
    for (int j = 0; j < R; j++) {
        acc[j] += __shfl_xor(acc[j], 1);
        acc[j] += __shfl_xor(acc[j], 2);
    }
    if (kq == 0 && row < t) {
        float* o = P + ((size_t)c * t + row) * R;
#pragma unroll
        for (int j = 0; j < R; j += 4)
            *reinterpret_cast<float4*>(o + j) = make_float4(acc[j], acc[j + 1], acc[j + 2], acc[j + 3]);
    }
}

// v[row][j] = scale * (sum over the nkc chunks, in order, of P[c][row][j]),
// then (ADD) dst[row][n] += sum_j v[row][j] * nmat(j, n), with nmat(j, n) =
// N[n*R + j] (NCOLR: N is [ncol x R], the forward's B) or N[j*ncol + n] (the
// backward's A, [R x ncol]).  The workgroups of column block 0 also write v
// to vout (xs, or dxa).  Each lane updates four columns of four rows.
template <int R, bool NCOLR, bool ADD = true>
__global__ __launch_bounds__(256) void lora_update_kernel(const float* __restrict__ P, int nkc, float scale,
                                                          const float* __restrict__ N, int t, int ncol,
                                                          float* __restrict__ dst, float* __restrict__ vout) {
    __shared__ float vs[kUpdRows][R];
    const int row0 = blockIdx.x * kUpdRows;
    const int tid = threadIdx.x;
    const int n = blockIdx.y * kUpdCols + (tid & 63) * 4;
    const int rq = (tid >> 6) * 4;
    const bool col_ok = ADD && n < ncol;
    // The lane's destination values and N columns first: they do not
    // depend on v, so their latency overlaps the sums below.
    float nb[4][R];
    float4 d[4];
    if (col_ok) {
        if (NCOLR) {
#pragma unroll
            for (int q = 0; q < 4; q++)
#pragma unroll
                for (int j = 0; j < R; j += 4) {
                    const float4 v = ld4(N + (size_t)(n + q) * R + j);
                    nb[q][j] = v.x, nb[q][j + 1] = v.y, nb[q][j + 2] = v.z, nb[q][j + 3] = v.w;
                }
        } else {
#pragma unroll
            for (int j = 0; j < R; j++) {
                const float4 v = ld4(N + (size_t)j * ncol + n);
                nb[0][j] = v.x, nb[1][j] = v.y, nb[2][j] = v.z, nb[3][j] = v.w;
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int row = row0 + rq + i;
            d[i] = row < t ? ld4(dst + (size_t)row * ncol + n) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    if (tid < kUpdRows * R) {
        const int r = tid / R, j = tid % R, row = row0 + r;
        float s = 0.0f;
        if (row < t) {
            const float* pp = P + (size_t)row * R + j;
            const size_t cs = (size_t)t * R;
            int c = 0;
            for (; c + 8 <= nkc; c += 8) {  // eight loads in flight, added in chunk order
                float q[8];
#pragma unroll
                for (int u = 0; u < 8; u++) q[u] = pp[(size_t)(c + u) * cs];
#pragma unroll
                for (int u = 0; u < 8; u++) s += q[u];
            }
            for (; c < nkc; c++) s += pp[(size_t)c * cs];
        }
        const float v = s * scale;
        vs[r][j] = v;
        if (blockIdx.y == 0 && row < t) vout[(size_t)row * R + j] = v;
    }
    __syncthreads();
    if (!col_ok) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int row = row0 + rq + i;
        if (row >= t) break;
        float s[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float a = 0.0f;
#pragma unroll
            for (int j = 0; j < R; j++) a = __builtin_fmaf(vs[rq + i][j], nb[q][j], a);
            s[q] = a;
        }
        *reinterpret_cast<float4*>(dst + (size_t)row * ncol + n) =
            make_float4(d[i].x + s[0], d[i].y + s[1], d[i].z + s[2], d[i].w + s[3]);
    }
}

// Gradient partial sums over one chunk of kLoraChunk tokens:
//   column blocks [0, nb_gb):        Pgb[c][n][j] = sum_i dy[i][n] * xs[i][j]   (n < out)
//   column blocks [nb_gb, + nb_ga):  Pga[c][k][j] = sum_i x[i][k] * dxa[i][j]   (k < in)
// A workgroup takes 64 columns (one per lane) of one chunk; its four waves
// sum rows 16w .. 16w + 15 of the chunk, the small operand's rows staged in
// LDS, and the four wave sums are added in wave order.
template <int R>
__global__ __launch_bounds__(256) void lora_grad_part_kernel(const float* __restrict__ dy,
                                                            const float* __restrict__ xs,
                                                            const float* __restrict__ x,
                                                            const float* __restrict__ dxa, int t, int in, int out,
                                                            int nb_gb, float* __restrict__ pgb,
                                                            float* __restrict__ pga) {
    constexpr int kSub = kLoraChunk / 4;
    __shared__ __attribute__((aligned(16))) float ssm[kLoraChunk][R];
    __shared__ float wsum[3][64][R + 1];
    const int c = blockIdx.y;
    const int i0 = c * kLoraChunk, i1 = min(t, i0 + kLoraChunk);
    const bool is_gb = (int)blockIdx.x < nb_gb;
    const float* big = is_gb ? dy : x;
    const float* small = is_gb ? xs : dxa;
    const int ncol = is_gb ? out : in;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int col = (is_gb ? blockIdx.x : blockIdx.x - nb_gb) * 64 + lane;
    const int cl = min(col, ncol - 1);
    const int r0 = wave * kSub;
    // The big operand's column first: its latency overlaps the staging.
    float b[kSub];
#pragma unroll
    for (int u = 0; u < kSub; u++) b[u] = i0 + r0 + u < i1 ? big[(size_t)(i0 + r0 + u) * ncol + cl] : 0.0f;
    for (int e = tid; e < kLoraChunk * R; e += 256) {
        const int i = i0 + e / R;
        ssm[e / R][e % R] = i < i1 ? small[(size_t)i * R + e % R] : 0.0f;
    }
    __syncthreads();
    float acc[R];
#pragma unroll
    for (int j = 0; j < R; j++) acc[j] = 0.0f;
#pragma unroll
    for (int u = 0; u < kSub; u++) {
#pragma unroll
        for (int j = 0; j < R; j += 4) {
            const float4 s4 = *reinterpret_cast<const float4*>(&ssm[r0 + u][j]);
            acc[j] = __builtin_fmaf(b[u], s4.x, acc[j]);
            acc[j + 1] = __builtin_fmaf(b[u], s4.y, acc[j + 1]);
            acc[j + 2] = __builtin_fmaf(b[u], s4.z, acc[j + 2]);
            acc[j + 3] = __builtin_fmaf(b[u], s4.w, acc[j + 3]);
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int j = 0; j < R; j++) wsum[wave - 1][lane][j] = acc[j];
    }
    __syncthreads();
    if (wave != 0 || col >= ncol) return;
#pragma unroll
    for (int w = 0; w < 3; w++)
#pragma unroll
        for (int j = 0; j < R; j++) acc[j] += wsum[w][lane][j];
    float* o = (is_gb ? pgb + (size_t)c * out * R : pga + (size_t)c * in * R) + (size_t)col * R;
#pragma unroll
    for (int j = 0; j < R; j += 4)
        *reinterpret_cast<float4*>(o + j) = make_float4(acc[j], acc[j + 1], acc[j + 2], acc[j + 3]);
}

// gb[n][j] += sum over chunks (in chunk order) of Pgb[c][n][j]; then
// ga[j][k] += sum over chunks of Pga[c][k][j].
__global__ __launch_bounds__(256) void lora_grad_reduce_kernel(const float* __restrict__ pgb,
                                                               const float* __restrict__ pga, int nch, int R, int n_gb,
                                                               int n_ga, int in, float* __restrict__ gb,
                                                               float* __restrict__ ga) {
    const int e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e < n_gb) {
        float s = 0.0f;
#pragma unroll 8
        for (int c = 0; c < nch; c++) s += pgb[(size_t)c * n_gb + e];
        gb[e] = gb[e] + s;
    } else if (e < n_gb + n_ga) {
        const int f = e - n_gb;  // = k*R + j
        float s = 0.0f;
#pragma unroll 8
        for (int c = 0; c < nch; c++) s += pga[(size_t)c * n_ga + f];
        const int k = f / R, j = f % R;
        float* g = ga + (size_t)j * in + k;
        *g = *g + s;
    }
}

// Weff[o][i] = W[o][i] + scale * sum_j B[o][j] A[j][i]: the base weight with
// the adapter merged in, so that x Weff^T = x W^T + (scale x A^T) B^T and
// dy Weff = dy W + (scale dy B) A in one GEMM each.  The j sum is one FMA
// chain in j order.  Each lane writes four consecutive columns of one row.
template <int R>
__global__ __launch_bounds__(256) void lora_merge_kernel(const float* __restrict__ W, const float* __restrict__ A,
                                                         const float* __restrict__ B, float scale, int out, int in,
                                                         float* __restrict__ Weff) {
    const long e = ((long)blockIdx.x * 256 + threadIdx.x) * 4;
    if (e >= (long)out * in) return;
    const int o = (int)(e / in), i = (int)(e % in);
    float b[R];
#pragma unroll
    for (int j = 0; j < R; j += 4) {
        const float4 v = ld4(B + (size_t)o * R + j);
        b[j] = v.x, b[j + 1] = v.y, b[j + 2] = v.z, b[j + 3] = v.w;
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < R; j++) {
        const float4 a = ld4(A + (size_t)j * in + i);
        acc.x = __builtin_fmaf(b[j], a.x, acc.x);
        acc.y = __builtin_fmaf(b[j], a.y, acc.y);
        acc.z = __builtin_fmaf(b[j], a.z, acc.z);
        acc.w = __builtin_fmaf(b[j], a.w, acc.w);
    }
    const float4 w = ld4(W + e);
    const float4 r = make_float4(__builtin_fmaf(scale, acc.x, w.x), __builtin_fmaf(scale, acc.y, w.y),
                                 __builtin_fmaf(scale, acc.z, w.z), __builtin_fmaf(scale, acc.w, w.w));
    *reinterpret_cast<float4*>(Weff + e) = r;
}

int nchunks(int n, int c) { return (n + c - 1) / c; }

template <int R>
hipError_t lora_fwd_r(const float* x, const float* a, const float* b, float scale, int t, int in, int out, float* y,
                      float* xs, float* part, hipStream_t st) {
    const int nkc = nchunks(in, kDotChunk);
    lora_rowdot_kernel<R, true><<<dim3(nchunks(t, kDotRows), nkc), 256, 0, st>>>(x, a, t, in, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (y)
        lora_update_kernel<R, true><<<dim3(nchunks(t, kUpdRows), nchunks(out, kUpdCols)), 256, 0, st>>>(
            part, nkc, scale, b, t, out, y, xs);
    else
        lora_update_kernel<R, true, false><<<dim3(nchunks(t, kUpdRows), 1), 256, 0, st>>>(part, nkc, scale, b, t, out,
                                                                                           y, xs);
    return hipGetLastError();
}

template <int R>
hipError_t lora_bwd_r(const float* x, const float* xs, const float* dy, const float* a, const float* b, float scale,
                      int t, int in, int out, float* dx, float* ga, float* gb, float* dxa, float* part,
                      hipStream_t st) {
    const int nkc = nchunks(out, kDotChunk);
    lora_rowdot_kernel<R, false><<<dim3(nchunks(t, kDotRows), nkc), 256, 0, st>>>(dy, b, t, out, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (dx)
        lora_update_kernel<R, false><<<dim3(nchunks(t, kUpdRows), nchunks(in, kUpdCols)), 256, 0, st>>>(
            part, nkc, scale, a, t, in, dx, dxa);
    else
        lora_update_kernel<R, false, false><<<dim3(nchunks(t, kUpdRows), 1), 256, 0, st>>>(part, nkc, scale, a, t, in,
                                                                                            dx, dxa);
    e = hipGetLastError();
    if (e != hipSuccess || (!ga && !gb)) return e;
    // The rowdot partials are consumed by now (same stream): reuse the buffer.
    const int nch = nchunks(t, kLoraChunk);
    const int nb_gb = gb ? nchunks(out, kGradCols) : 0, nb_ga = ga ? nchunks(in, kGradCols) : 0;
    float* pgb = part;
    float* pga = part + (size_t)nch * out * R;
    lora_grad_part_kernel<R><<<dim3(nb_gb + nb_ga, nch), 256, 0, st>>>(dy, xs, x, dxa, t, in, out, nb_gb, pgb, pga);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int n_gb = gb ? out * R : 0, n_ga = ga ? R * in : 0;
    lora_grad_reduce_kernel<<<nchunks(n_gb + n_ga, 256), 256, 0, st>>>(pgb, pga, nch, R, n_gb, n_ga, in, gb, ga);
    return hipGetLastError();
}

}  // namespace

bool lora_fused_applies(size_t rank, size_t t, size_t in, size_t out, const void* const* ptrs, int nptr) {
    if (!(rank == 4 || rank == 8 || rank == 16)) return false;
    if (in % 4 || out % 4 || t >= ((size_t)1 << 26) || in >= ((size_t)1 << 26) || out >= ((size_t)1 << 26))
        return false;
    for (int i = 0; i < nptr; i++)
        if (ptrs[i] && (uintptr_t)ptrs[i] % 16) return false;
    return true;
}

size_t lora_partial_floats(size_t rank, size_t t, size_t in, size_t out) {
    const size_t rowdot = (size_t)nchunks((int)(in > out ? in : out), kDotChunk) * t * rank;
    const size_t grad = (size_t)nchunks((int)t, kLoraChunk) * (in + out) * rank;
    return rowdot > grad ? rowdot : grad;
}

hipError_t launch_lora_fwd(size_t rank, const float* x, const float* a, const float* b, float scale, size_t t,
                           size_t in, size_t out, float* y, float* xs, float* part, hipStream_t st) {
    switch (rank) {
        case 4: return lora_fwd_r<4>(x, a, b, scale, (int)t, (int)in, (int)out, y, xs, part, st);
        case 8: return lora_fwd_r<8>(x, a, b, scale, (int)t, (int)in, (int)out, y, xs, part, st);
        default: return lora_fwd_r<16>(x, a, b, scale, (int)t, (int)in, (int)out, y, xs, part, st);
    }
}

hipError_t launch_lora_merge(size_t rank, const float* w, const float* a, const float* b, float scale, size_t out,
                             size_t in, float* weff, hipStream_t st) {
    const long blocks = (long)((out * in / 4 + 255) / 256);  // in % 4 == 0: whole float4 rows
    if (blocks > 0x7fffffffL) return hipErrorInvalidConfiguration;
    const dim3 grid((unsigned)blocks);
    switch (rank) {
        case 4: lora_merge_kernel<4><<<grid, 256, 0, st>>>(w, a, b, scale, (int)out, (int)in, weff); break;
        case 8: lora_merge_kernel<8><<<grid, 256, 0, st>>>(w, a, b, scale, (int)out, (int)in, weff); break;
        default: lora_merge_kernel<16><<<grid, 256, 0, st>>>(w, a, b, scale, (int)out, (int)in, weff); break;
    }
    return hipGetLastError();
}

hipError_t launch_lora_bwd(size_t rank, const float* x, const float* xs, const float* dy, const float* a,
                           const float* b, float scale, size_t t, size_t in, size_t out, float* dx, float* ga,
                           float* gb, float* dxa, float* part, hipStream_t st) {
    switch (rank) {
        case 4: return lora_bwd_r<4>(x, xs, dy, a, b, scale, (int)t, (int)in, (int)out, dx, ga, gb, dxa, part, st);
        case 8: return lora_bwd_r<8>(x, xs, dy, a, b, scale, (int)t, (int)in, (int)out, dx, ga, gb, dxa, part, st);
        default:
            return lora_bwd_r<16>(x, xs, dy, a, b, scale, (int)t, (int)in, (int)out, dx, ga, gb, dxa, part, st);
    }
}

}  // namespace cfattn
