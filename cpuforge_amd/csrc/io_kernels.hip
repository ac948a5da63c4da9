// Kernels of the on-disk formats: widening bf16 / f16 tensors to f32
// (crates/io/src/dtype.rs:3-33) and moving the runs of a staged file chunk
// to or from their device tensors.  All of it is HBM-bound streaming work:
// coalesced loads and stores, no LDS.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "cfio_kernels.hpp"

namespace cfio {
namespace {

__device__ __forceinline__ uint32_t bf16_bits(uint32_t h) { return h << 16; }

// dtype.rs:7-33: the f32 bit pattern of an IEEE half.  A subnormal half is
// renormalised (its leading one moved to bit 10, the exponent lowered by the
// same count, which is what the reference's shift loop computes), inf and
// NaN keep their payload bits.
__device__ __forceinline__ uint32_t f16_bits(uint32_t h) {
    const uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    if (exp == 0x1fu) return (sign << 31) | (0xffu << 23) | (man << 13);
    if (exp != 0u) return (sign << 31) | ((exp + 112u) << 23) | (man << 13);
    if (man == 0u) return sign << 31;
    const uint32_t s = __clz(man) - 21u;  // 1..10
    return (sign << 31) | ((113u - s) << 23) | (((man << s) & 0x3ffu) << 13);
}

template <bool F16>
__device__ __forceinline__ uint32_t widen(uint32_t h) {
    return F16 ? f16_bits(h) : bf16_bits(h);
}

// Eight halves (16 B) in, eight floats (32 B) out per lane and iteration;
// src and dst 16-byte aligned.
template <bool F16>
__global__ __launch_bounds__(256) void widen8_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                     size_t n8) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8; i += stride) {
        const uint4 r = src[i];
        uint4 a, b;
        a.x = widen<F16>(r.x & 0xffffu);
        a.y = widen<F16>(r.x >> 16);
        a.z = widen<F16>(r.y & 0xffffu);
        a.w = widen<F16>(r.y >> 16);
        b.x = widen<F16>(r.z & 0xffffu);
        b.y = widen<F16>(r.z >> 16);
        b.z = widen<F16>(r.w & 0xffffu);
        b.w = widen<F16>(r.w >> 16);
        dst[2 * i] = a;
        dst[2 * i + 1] = b;
    }
}

template <bool F16>
__global__ __launch_bounds__(256) void widen1_kernel(const uint16_t* __restrict__ src, uint32_t* __restrict__ dst,
                                                     size_t begin, size_t n) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = begin + (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = widen<F16>(src[i]);
}

// The run holding workgroup b: the last piece whose first workgroup is <= b.
__device__ __forceinline__ IoPiece find_piece(const IoPiece* pieces, int np, uint32_t b) {
    int lo = 0, hi = np - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pieces[mid].blk0 <= b) lo = mid;
        else hi = mid - 1;
    }
    return pieces[lo];
}

// Staged file bytes -> f32 device tensors: workgroup b converts its
// kPieceBlockBytes of source bytes of one run.  Runs start 16-byte aligned in
// the chunk; destinations are 4-byte aligned.
__global__ __launch_bounds__(256) void scatter_kernel(const uint8_t* __restrict__ chunk,
                                                     const IoPiece* __restrict__ pieces, int np) {
    const IoPiece pc = find_piece(pieces, np, blockIdx.x);
    const uint32_t begin = (blockIdx.x - pc.blk0) * kPieceBlockBytes;
    const uint32_t end = min(pc.bytes, begin + kPieceBlockBytes);
    uint32_t* dst = reinterpret_cast<uint32_t*>(pc.dev);
    if (pc.kind == kCopyF32) {
        const uint32_t* s = reinterpret_cast<const uint32_t*>(chunk + pc.off);
        for (uint32_t e = begin / 4 + threadIdx.x; e < end / 4; e += blockDim.x) dst[e] = s[e];
    } else {
        const uint16_t* s = reinterpret_cast<const uint16_t*>(chunk + pc.off);
        if (pc.kind == kWidenF16) {
            for (uint32_t e = begin / 2 + threadIdx.x; e < end / 2; e += blockDim.x) dst[e] = f16_bits(s[e]);
        } else {
            for (uint32_t e = begin / 2 + threadIdx.x; e < end / 2; e += blockDim.x) dst[e] = bf16_bits(s[e]);
        }
    }
}

// f32 device tensors -> a chunk laid out as the file's data section.
__global__ __launch_bounds__(256) void gather_kernel(uint8_t* __restrict__ chunk, const IoPiece* __restrict__ pieces,
                                                     int np) {
    const IoPiece pc = find_piece(pieces, np, blockIdx.x);
    const uint32_t begin = (blockIdx.x - pc.blk0) * kPieceBlockBytes;
    const uint32_t end = min(pc.bytes, begin + kPieceBlockBytes);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(pc.dev);
    uint32_t* d = reinterpret_cast<uint32_t*>(chunk + pc.off);
    for (uint32_t e = begin / 4 + threadIdx.x; e < end / 4; e += blockDim.x) d[e] = src[e];
}

}  // namespace

hipError_t launch_widen(bool f16, const uint16_t* src, float* dst, size_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const bool vec = ((uintptr_t)src % 16 == 0) && ((uintptr_t)dst % 16 == 0);
    const size_t n8 = vec ? n / 8 : 0;
    if (n8) {
        const size_t want = (n8 + 255) / 256;
        const unsigned grid = (unsigned)(want < 8192 ? want : 8192);
        if (f16) widen8_kernel<true><<<grid, 256, 0, st>>>((const uint4*)src, (uint4*)dst, n8);
        else widen8_kernel<false><<<grid, 256, 0, st>>>((const uint4*)src, (uint4*)dst, n8);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const size_t begin = n8 * 8;
    if (begin < n) {
        const size_t want = (n - begin + 255) / 256;
        const unsigned grid = (unsigned)(want < 8192 ? want : 8192);
        if (f16) widen1_kernel<true><<<grid, 256, 0, st>>>(src, (uint32_t*)dst, begin, n);
        else widen1_kernel<false><<<grid, 256, 0, st>>>(src, (uint32_t*)dst, begin, n);
        return hipGetLastError();
    }
    return hipSuccess;
}

hipError_t launch_scatter(const uint8_t* chunk, const IoPiece* pieces, int np, uint32_t blocks, hipStream_t st) {
    if (np <= 0 || blocks == 0) return hipSuccess;
    scatter_kernel<<<blocks, 256, 0, st>>>(chunk, pieces, np);
    return hipGetLastError();
}

hipError_t launch_gather(uint8_t* chunk, const IoPiece* pieces, int np, uint32_t blocks, hipStream_t st) {
    if (np <= 0 || blocks == 0) return hipSuccess;
    gather_kernel<<<blocks, 256, 0, st>>>(chunk, pieces, np);
    return hipGetLastError();
}

}  // namespace cfio
