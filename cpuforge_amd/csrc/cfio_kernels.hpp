// Launchers of the on-disk-format kernels (io_kernels.hip), used by
// cfio_capi.cpp.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace cfio {

// Element conversions of a staged tensor piece.
enum PieceKind : uint32_t { kCopyF32 = 0, kWidenBF16 = 1, kWidenF16 = 2 };

// One contiguous run of a tensor inside a staging chunk.  Reading a file,
// `dev` is where the run's first f32 output goes and `bytes` counts the staged
// source bytes; writing one, `dev` is the f32 source and `bytes` the bytes
// gathered into the chunk.  Each run is handled by consecutive workgroups of
// kPieceBlockBytes source bytes each, starting at workgroup `blk0`.
struct alignas(32) IoPiece {
    uint64_t dev;
    uint32_t off;    // byte offset of the run in the staging chunk
    uint32_t bytes;
    uint32_t kind;   // PieceKind
    uint32_t blk0;
    uint64_t pad;
};
constexpr uint32_t kPieceBlockBytes = 4096;
constexpr int kMaxPieces = 8192;  // runs per chunk

inline uint32_t piece_blocks(uint32_t bytes) { return (bytes + kPieceBlockBytes - 1) / kPieceBlockBytes; }

// dst[i] = f32 value of the 16-bit pattern src[i] (bf16 or f16).
hipError_t launch_widen(bool f16, const uint16_t* src, float* dst, size_t n, hipStream_t st);
// Staged chunk -> device tensors (read) and device tensors -> chunk (write);
// `pieces` lives in device memory, `blocks` is the sum of piece_blocks.
hipError_t launch_scatter(const uint8_t* chunk, const IoPiece* pieces, int np, uint32_t blocks, hipStream_t st);
hipError_t launch_gather(uint8_t* chunk, const IoPiece* pieces, int np, uint32_t blocks, hipStream_t st);

}  // namespace cfio
