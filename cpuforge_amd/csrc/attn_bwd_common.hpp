// Device helpers shared by the backward kernel files (attn_bwd.hip,
// attn_dkdv.hip): gradient row accumulation and the stored-dS block layout.
#pragma once
#include "cfattn_common.hpp"

namespace cfattn {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Accumulate one lane's 4 x (4 consecutive head dims) of a transposed
// accumulator block into a global row: dst[d0 + 8*rq + 4*hh + i] += acc[4*rq + i].
__device__ __forceinline__ void add_row_block(float* row, const f32x16& acc, int dbase, int hh, int hd, bool vec_ok) {
#pragma unroll
    for (int rq = 0; rq < 4; rq++) {
        const int d0 = dbase + rq * 8 + hh * 4;
        if (vec_ok && d0 + 4 <= hd) {
            float4 v = *reinterpret_cast<float4*>(row + d0);
            v.x += acc[rq * 4 + 0];
            v.y += acc[rq * 4 + 1];
            v.z += acc[rq * 4 + 2];
            v.w += acc[rq * 4 + 3];
            *reinterpret_cast<float4*>(row + d0) = v;
        } else {
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (d0 + i < hd) row[d0 + i] += acc[rq * 4 + i];
        }
    }
}

// Stored dS block: kDsBlock bf16 values (2 KiB) for query block qi and key
// block ki.  Element (MFMA row m, key k) of the 32x32 block -- query
// 32*qi + qperm(m), key 32*ki + k -- sits in 16-byte slot
//   c*64 + (l ^ (2*c + hh)),   l = k + 32*hh,  hh = (m/4) % 2,  c = m / 16,
// at position 4*((m/8) % 2) + m % 4 of the slot.  Slot l ^ .. thus holds the
// eight values lane l of a dK/dV dS wave has for its key, in accumulator
// order, so the writer stores two 16-byte pieces per lane.  The XOR spreads
// the 8-byte pieces one transposed read of the dQ kernel gathers (keys 4
// apart, four row quads) over all 64 LDS banks.
constexpr int kDsBlock = 1024;

}  // namespace cfattn
