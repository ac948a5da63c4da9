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

// dtype.rs:7-33: the f32 bit pattern of an IEEE half, without branches (a
// divergent branch splits the caller's stores into partial-wave writes).
// Normal halves rebias the exponent by 127 - 15 = 112; inf and NaN (exponent
// 31) rebias by 112 twice, which lands on 255 with the payload kept; a zero
// or subnormal half is man * 2^-24, which f32 holds exactly as a normal
// number, so the product's bits are the reference's renormalised pattern.
__device__ __forceinline__ uint32_t f16_bits(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16, em = h & 0x7fffu, exp = em >> 10;
    const uint32_t normal = (em << 13) + (112u << 23);
    const uint32_t special = normal + (112u << 23);
    const uint32_t sub = __float_as_uint((float)(em & 0x3ffu) * 0x1p-24f);
    return sign | (exp == 0x1fu ? special : (exp == 0u ? sub : normal));
}

template <bool F16>
__device__ __forceinline__ uint32_t widen(uint32_t h) {
    return F16 ? f16_bits(h) : bf16_bits(h);
}

// Four halves (8 B) in, four floats (16 B) out per lane, one lane per
// quad and no loop: an exact grid keeps every wave's loads and stores
// contiguous.  The stores are nontemporal (the output is not read back by
// this kernel; measured 6.6 TB/s against 6.2 with cached stores and 4.5-4.7
// with a grid-stride loop over 8 halves a lane).  src 8-byte and dst 16-byte
// aligned.
template <bool F16>
__global__ __launch_bounds__(256) void widen4_kernel(const uint2* __restrict__ src, uint32_t* __restrict__ dst,
                                                     size_t n4) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n4) return;
    const uint2 r = src[i];
    uint32_t* o = dst + 4 * i;
    __builtin_nontemporal_store(widen<F16>(r.x & 0xffffu), o);
    __builtin_nontemporal_store(widen<F16>(r.x >> 16), o + 1);
    __builtin_nontemporal_store(widen<F16>(r.y & 0xffffu), o + 2);
    __builtin_nontemporal_store(widen<F16>(r.y >> 16), o + 3);
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
    const bool vec = ((uintptr_t)src % 8 == 0) && ((uintptr_t)dst % 16 == 0);
    const size_t n4 = vec ? n / 4 : 0;
    if (n4) {
        const size_t grid = (n4 + 255) / 256;
        if (grid > 0x7fffffffu) return hipErrorInvalidValue;
        if (f16) widen4_kernel<true><<<(unsigned)grid, 256, 0, st>>>((const uint2*)src, (uint32_t*)dst, n4);
        else widen4_kernel<false><<<(unsigned)grid, 256, 0, st>>>((const uint2*)src, (uint32_t*)dst, n4);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const size_t begin = n4 * 4;
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
