// Device helpers shared by the backward kernel files (attn_bwd.hip,
// attn_dkdv.hip): gradient row accumulation and the stored-dS block layout.
#pragma once
#include "cfattn_common.hpp"
#include "attn_params.hpp"

namespace cfattn {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Direction in which a dK/dV workgroup (one per CU) walks its query tiles,
// heads innermost.  The XCDs dispatch workgroups in rounds of xcd_cus, one
// per CU; key tiles ascend within a round.  In even rounds every workgroup
// starts at the last query tile and walks down: they all start together
// and so read each Q/dO tile of a head within a step of each other.  The
// next round's workgroups start as the previous round's end, the one with
// the fewest query tiles (the highest key tile) first; walking up from
// their own first tile, each reaches tile q when the others do (a
// workgroup that starts d tiles later starts d tiles higher), so they too
// share each tile in the XCD's L2.  Walking every workgroup up from its
// diagonal instead leaves neighbours 2 tiles (8 steps, about 8 MB of an
// XCD's reads at C5) apart, more than a 4 MB L2 holds.
__device__ __forceinline__ bool dkdv_walks_down(unsigned hw_id, int xcd_cus) {
    return ((hw_id / 8u / (unsigned)xcd_cus) & 1u) == 0u;
}

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

// One lane's part of a gradient row held as NDB transposed accumulator blocks
// (block db: head dims db*32 + 8*rq + 4*hh + [0, 4) in acc[db][4*rq + i]),
// written per the epilogue mode (p.epi, EpilogueMode): added, or unrotated
// (inverse rotate-half RoPE with the cos/sin row of position
// p.rope_pos0 + t) and then added or stored.  Rotate-half pairs head dims j
// and j + DP/2, which sit in blocks db and db + NDB/2 of the same lane, so the
// rotation is lane-local.  The unrotation repeats the prologue backward's
// expressions (s = -sin; lo' = lo c - hi s, hi' = hi c + lo s), uncontracted,
// so both paths give the same bits.
// With PRE (the += modes), the row's current values come from `pre` instead
// of memory: grad_row_prefetch read them earlier, so that the read is not a
// dependent round trip at the end of the kernel.
template <int NDB, bool PRE = false>
__device__ __forceinline__ void write_grad_row(float* row, const f32x16 (&acc)[NDB], int hh, int t,
                                               const BwdParams& p, const float4 (*pre)[4] = nullptr) {
#pragma clang fp contract(off)
    constexpr int DP = NDB * 32, HALF = DP / 2;
    if (p.epi == kEpiAdd) {
        if constexpr (PRE) {
#pragma unroll
            for (int db = 0; db < NDB; db++)
#pragma unroll
                for (int rq = 0; rq < 4; rq++) {
                    float4 v = pre[db][rq];
                    v.x += acc[db][rq * 4 + 0];
                    v.y += acc[db][rq * 4 + 1];
                    v.z += acc[db][rq * 4 + 2];
                    v.w += acc[db][rq * 4 + 3];
                    *reinterpret_cast<float4*>(row + db * 32 + rq * 8 + hh * 4) = v;
                }
            return;
        }
#pragma unroll
        for (int db = 0; db < NDB; db++) add_row_block(row, acc[db], db * 32, hh, DP, true);
        return;
    }
    const float* cs = p.rope_cos + (long)(p.rope_pos0 + t) * HALF;
    const float* sn = p.rope_sin + (long)(p.rope_pos0 + t) * HALF;
#pragma unroll
    for (int db = 0; db < NDB / 2; db++) {
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            const int d0 = db * 32 + rq * 8 + hh * 4;
            const float4 c4 = *reinterpret_cast<const float4*>(cs + d0);
            const float4 s4 = *reinterpret_cast<const float4*>(sn + d0);
            const float c[4] = {c4.x, c4.y, c4.z, c4.w}, sv[4] = {s4.x, s4.y, s4.z, s4.w};
            float lo[4], hi[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float g1 = acc[db][rq * 4 + i], g2 = acc[db + NDB / 2][rq * 4 + i];
                const float s = -1.0f * sv[i];
                lo[i] = g1 * c[i] - g2 * s;
                hi[i] = g2 * c[i] + g1 * s;
            }
            float4* r1 = reinterpret_cast<float4*>(row + d0);
            float4* r2 = reinterpret_cast<float4*>(row + d0 + HALF);
            if (p.epi == kEpiUnrotAdd) {
                float4 a, b;
                if constexpr (PRE) {
                    a = pre[db][rq];
                    b = pre[db + NDB / 2][rq];
                } else {
                    a = *r1;
                    b = *r2;
                }
                a.x += lo[0], a.y += lo[1], a.z += lo[2], a.w += lo[3];
                b.x += hi[0], b.y += hi[1], b.z += hi[2], b.w += hi[3];
                *r1 = a;
                *r2 = b;
            } else {
                *r1 = make_float4(lo[0], lo[1], lo[2], lo[3]);
                *r2 = make_float4(hi[0], hi[1], hi[2], hi[3]);
            }
        }
    }
}

// The lane's part of a gradient row (the layout write_grad_row writes), read
// ahead for the += epilogue modes; false (nothing read) for the others.
template <int NDB>
__device__ __forceinline__ bool grad_row_prefetch(float4 (&pre)[NDB][4], const float* row, int hh,
                                                  const BwdParams& p) {
    if (p.epi != kEpiAdd && p.epi != kEpiUnrotAdd) return false;
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++) pre[db][rq] = *reinterpret_cast<const float4*>(row + db * 32 + rq * 8 + hh * 4);
    return true;
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
