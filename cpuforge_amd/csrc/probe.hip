// Throughput probes: the matrix-pipe ceiling the bf16 attention kernels are
// measured against on the board they run on, and loops of LDS reads and of
// VALU operations for the power each instruction class draws.
//
// The published MI355X figure (2516.6 TFLOP/s dense bf16) assumes the 2.4 GHz
// top clock.  Under a sustained MFMA load the board's power limit sets the
// clock, and the power a bf16 MFMA draws depends on how many operand bits
// change from one instruction to the next.  The probe therefore runs a loop
// of v_mfma_f32_32x32x16_bf16 with nothing else in it, on operands that are
// either pseudo-random bf16 values (bit activity like the attention
// kernels' inputs) or zeros (the least power the instruction can draw), two
// waves per SIMD on every CU, and reports FLOPs over the loop's event time.
#include "cfattn_common.hpp"
#include "cfattn_kernels.hpp"

namespace cfattn {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// A 32-bit integer hash (xorshift-multiply, the "lowbias32" constants of
// Chris Wellons' public hash survey): consecutive inputs give unrelated
// outputs, so every lane and operand gets independent bits.
__device__ __forceinline__ uint32_t probe_hash(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352du;
    x ^= x >> 15;
    x *= 0x846ca68bu;
    x ^= x >> 16;
    return x;
}

// Two bf16 values from 32 hash bits: random sign and mantissa, exponent
// 2^-2 .. 2^1 (magnitudes 0.25 .. 4, like N(0,1) data).
__device__ __forceinline__ uint32_t probe_pair(uint32_t h) {
    const uint32_t lo = (h & 0x807fu) | ((125u + ((h >> 7) & 3u)) << 7);
    const uint32_t hi = ((h >> 16) & 0x807fu) | ((125u + ((h >> 23) & 3u)) << 7);
    return lo | (hi << 16);
}

__global__ __launch_bounds__(256) void mfma_probe_kernel(int iters, int zeros, float* sink) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = blockIdx.x * 4u + (threadIdx.x >> 6);
    bf16x8 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t wa[4], wb[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t seed = ((wave * 64u + lane) * 4u + (uint32_t)i) * 8u + (uint32_t)j;
            wa[j] = zeros ? 0u : probe_pair(probe_hash(seed));
            wb[j] = zeros ? 0u : probe_pair(probe_hash(seed + 4u));
        }
        a[i] = __builtin_bit_cast(bf16x8, make_uint4(wa[0], wa[1], wa[2], wa[3]));
        b[i] = __builtin_bit_cast(bf16x8, make_uint4(wb[0], wb[1], wb[2], wb[3]));
    }
    f32x16 acc[4];
#pragma unroll
    for (int c = 0; c < 4; c++) acc[c] = zero16();
    // Four independent accumulator chains, a different operand pair for
    // every instruction of an iteration.
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int c = 0; c < 4; c++) acc[c] = mfma32(a[(j + c) & 3], b[(j + 2 * c + (c >> 1)) & 3], acc[c]);
    }
    // Keeps the loop live; callers pass no sink.
    if (sink) {
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) s += acc[c][r];
        sink[wave * 64u + lane] = s;
    }
}

// The same loop with v_mfma_f32_16x16x32_bf16 (half the FLOPs per
// instruction, a quarter of the accumulator per product): eight independent
// accumulator chains, 32 MFMAs (the 32x32x16 loop's FLOPs) per iteration, on
// pseudo-random operands.  Whether the other shape draws less energy per FLOP
// (and so runs faster under the power limit) is what it measures.
__global__ __launch_bounds__(256) void mfma16_probe_kernel(int iters, float* sink) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave = blockIdx.x * 4u + (threadIdx.x >> 6);
    bf16x8 a[4], b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        uint32_t wa[4], wb[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t seed = ((wave * 64u + lane) * 4u + (uint32_t)i) * 8u + (uint32_t)j;
            wa[j] = probe_pair(probe_hash(seed));
            wb[j] = probe_pair(probe_hash(seed + 4u));
        }
        a[i] = __builtin_bit_cast(bf16x8, make_uint4(wa[0], wa[1], wa[2], wa[3]));
        b[i] = __builtin_bit_cast(bf16x8, make_uint4(wb[0], wb[1], wb[2], wb[3]));
    }
    f32x4 acc[8];
#pragma unroll
    for (int c = 0; c < 8; c++) acc[c] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
            for (int c = 0; c < 8; c++)
                acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[(j + c) & 3], b[(j + 2 * c + (c >> 1)) & 3], acc[c],
                                                                  0, 0, 0);
    }
    // Keeps the loop live; callers pass no sink.
    if (sink) {
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < 8; c++) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
        sink[wave * 64u + lane] = s;
    }
}

// Loops of one other instruction class, one 1024-thread workgroup per CU
// (four waves per SIMD), for the board power each draws at its rate:
//   LDS: 16-byte reads of a 64 KiB LDS buffer, a wave's 64 lanes on 1 KiB of
//        consecutive bytes (no bank conflict), eight per loop iteration;
//   VALU: v_fma_f32 on eight independent registers, sixteen per iteration.
__global__ __launch_bounds__(1024) void lds_probe_kernel(int iters, float* sink) {
    __shared__ float4 buf[4096];
    const int tid = threadIdx.x;
    for (int i = tid; i < 4096; i += 1024)
        buf[i] = make_float4((float)i, (float)(i ^ 0x55), (float)(i * 3), (float)(i + 7));
    __syncthreads();
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    int idx = tid & 4095;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float4 v = buf[(idx + u * 64) & 4095];
            acc.x += v.x, acc.y += v.y, acc.z += v.z, acc.w += v.w;
        }
        idx = (idx + 512) & 4095;
    }
    // Keeps the loop live; callers pass no sink.
    if (sink) sink[blockIdx.x * 1024 + tid] = acc.x + acc.y + acc.z + acc.w;
}

__global__ __launch_bounds__(1024) void valu_probe_kernel(int iters, float* sink) {
    float a[8];
#pragma unroll
    for (int i = 0; i < 8; i++) a[i] = (float)threadIdx.x * 1e-3f + 0.1f * (float)i;
    const float m = 0.999f, c = 0.001f;
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int i = 0; i < 8; i++)
            asm volatile("v_fma_f32 %0, %0, %1, %2\n\tv_fma_f32 %0, %0, %1, %2" : "+v"(a[i]) : "v"(m), "v"(c));
    }
    if (sink) {
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) s += a[i];
        sink[blockIdx.x * 1024 + threadIdx.x] = s;
    }
}

}  // namespace

// MFMAs per wave per loop iteration and FLOPs per MFMA (32 x 32 x 16 x 2).
constexpr double kProbeMfmaPerIter = 16.0, kProbeFlopsPerMfma = 32.0 * 32.0 * 16.0 * 2.0;

hipError_t probe_mfma_bf16(hipStream_t st, int zeros, int iters, double* tflops) {
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    const int wgs = 2 * cus;  // eight waves per CU: two per SIMD
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if ((e = hipEventCreate(&e0)) != hipSuccess) return e;
    if ((e = hipEventCreate(&e1)) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return e;
    }
    float ms = 0.0f;
    e = hipEventRecord(e0, st);
    if (e == hipSuccess) {
        hipLaunchKernelGGL(mfma_probe_kernel, dim3(wgs), dim3(256), 0, st, iters, zeros, (float*)nullptr);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipEventRecord(e1, st);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (e != hipSuccess) return e;
    const double flops = (double)wgs * 4.0 * (double)iters * kProbeMfmaPerIter * kProbeFlopsPerMfma;
    *tflops = ms > 0.0f ? flops / ((double)ms * 1e-3) / 1e12 : 0.0;
    return hipSuccess;
}

hipError_t probe_loop(hipStream_t st, int kind, int iters, double* rate) {
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    if ((e = hipEventCreate(&e0)) != hipSuccess) return e;
    if ((e = hipEventCreate(&e1)) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return e;
    }
    float ms = 0.0f;
    e = hipEventRecord(e0, st);
    if (e == hipSuccess) {
        if (kind == kProbeLds)
            hipLaunchKernelGGL(lds_probe_kernel, dim3(cus), dim3(1024), 0, st, iters, (float*)nullptr);
        else if (kind == kProbeValu)
            hipLaunchKernelGGL(valu_probe_kernel, dim3(cus), dim3(1024), 0, st, iters, (float*)nullptr);
        else  // kProbeMfma16: two waves per SIMD, as the 32x32x16 probe
            hipLaunchKernelGGL(mfma16_probe_kernel, dim3(2 * cus), dim3(256), 0, st, iters, (float*)nullptr);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipEventRecord(e1, st);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (e != hipSuccess) return e;
    // Bytes read from LDS, lane operations (one per lane per v_fma_f32), or
    // FLOPs (32 MFMAs of 16 x 16 x 32 x 2 per wave and iteration, 8 waves
    // per CU).
    double units;
    if (kind == kProbeMfma16)
        units = (double)cus * 8.0 * (double)iters * 32.0 * (16.0 * 16.0 * 32.0 * 2.0);
    else
        units = (double)cus * 1024.0 * (double)iters * (kind == kProbeLds ? 8.0 * 16.0 : 16.0);
    *rate = ms > 0.0f ? units / ((double)ms * 1e-3) : 0.0;
    return hipSuccess;
}

}  // namespace cfattn
