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
// `mode` is p.epi unless given (>= 0).
template <int NDB, bool PRE = false>
__device__ __forceinline__ void write_grad_row(float* row, const f32x16 (&acc)[NDB], int hh, int t,
                                               const BwdParams& p, const float4 (*pre)[4] = nullptr,
                                               int mode = -1) {
#pragma clang fp contract(off)
    constexpr int DP = NDB * 32, HALF = DP / 2;
    if (mode < 0) mode = p.epi;
    if (mode == kEpiAdd) {
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
    // The row's cos/sin entries, read before the first store (a store may
    // alias them as far as the compiler knows, which would hold each later
    // read behind it).
    float4 cs4[NDB / 2][4], sn4[NDB / 2][4];
#pragma unroll
    for (int db = 0; db < NDB / 2; db++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            cs4[db][rq] = *reinterpret_cast<const float4*>(cs + db * 32 + rq * 8 + hh * 4);
            sn4[db][rq] = *reinterpret_cast<const float4*>(sn + db * 32 + rq * 8 + hh * 4);
        }
#pragma unroll
    for (int db = 0; db < NDB / 2; db++) {
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            const int d0 = db * 32 + rq * 8 + hh * 4;
            const float4 c4 = cs4[db][rq];
            const float4 s4 = sn4[db][rq];
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
            if (mode == kEpiUnrotAdd) {
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

// The kEpiUnrotNorm epilogue's pre-norm rows are staged in LDS first: each
// wave copies the head dims its lanes hold of their rows (lane hh of row l32:
// dims db*32 + 8*rq + 4*hh + [0, 4)) with direct-to-LDS loads into its own
// region, chunk-major -- the 16 bytes of chunk (db, rq) of lane `lane` at
// float (4*db + rq)*256 + 4*lane -- so the loads hold no registers, all are in
// flight at once, and every read of the epilogue is 64 consecutive 16-byte
// slots.  The caller passes a valid row for lanes whose row is past the end
// (read, unused), waits for the loads (vmcnt) and makes sure no wave still
// reads the region's earlier contents.
template <int NDB>
__device__ __forceinline__ void stage_norm_row(const float* xrow, float* xs, int hh) {
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++) lds_load16_asm(xrow + db * 32 + rq * 8 + hh * 4, xs + (db * 4 + rq) * 256);
}

// The kEpiUnrotNorm epilogue of one gradient row: the inverse RoPE of
// write_grad_row, then the Qwen3 per-head RMSNorm backward (rmsnorm.rs:31-67
// with one row of `dim` = DP): with x the pre-norm row (staged at xs by
// stage_norm_row), inv its rstd and w the gains,
//   dot = sum_i dy_i w_i x_i inv,   dx_i += inv (dy_i w_i - x_i inv dot / DP),
// added into `dst`; the gain gradient's terms dy_i x_i inv replace the row's
// accumulators in `acc` (acc holds dy in between).  The lane pair (hh = 0, 1)
// holds the row: lane hh has head dims db*32 + 8*rq + 4*hh + i.  The dot is
// summed exactly as prologue_bwd_norm_vec_kernel sums it, so the rows equal
// that kernel's bit for bit: each chunk of eight dims 8j .. 8j+7
// (j = 4*db + rq) in order from 0 -- the hh = 0 lane's four terms, then,
// after one lane-half swap, the hh = 1 lane's four -- and the DP/8 chunk sums
// over the xor tree of that kernel's G = DP/8 lanes (offsets G/2 .. 1; every
// lane of such a tree ends with the same bits, so one lane's order suffices).
// Every lane of the wave takes part (the swaps); a row with `ok` false writes
// nothing and its gain terms are zero.  The row's current values come from
// `pre` (the lane's part, read earlier: grad_row_prefetch or load_grad_row).
template <int NDB>
__device__ __forceinline__ void write_grad_row_norm(float* dst, const float* xs, float inv, const float* w,
                                                    f32x16 (&acc)[NDB], int lane, int t, bool ok, const BwdParams& p,
                                                    const float4 (&pre)[NDB][4]) {
#pragma clang fp contract(off)
    constexpr int DP = NDB * 32, HALF = DP / 2, NB2 = NDB / 2, G = DP / 8;
    const int hh = lane >> 5;
    const int tt = ok ? t : 0;  // a row past the end reads the first table row (unused)
    const float* cs = p.rope_cos + (long)(p.rope_pos0 + tt) * HALF;
    const float* sn = p.rope_sin + (long)(p.rope_pos0 + tt) * HALF;
    auto load4 = [&](const float* src, float (&v)[4]) {
        const float4 u = *reinterpret_cast<const float4*>(src);
        v[0] = u.x, v[1] = u.y, v[2] = u.z, v[3] = u.w;
    };
    auto x4 = [&](int db, int rq, float (&v)[4]) { load4(xs + (db * 4 + rq) * 256 + lane * 4, v); };
    // Pass 1: dy (write_grad_row's expressions) in place of acc, and the
    // dot's terms.
    f32x16 term[NDB];
#pragma unroll
    for (int db = 0; db < NB2; db++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            float c[4], sv[4];
            load4(cs + db * 32 + rq * 8 + hh * 4, c);
            load4(sn + db * 32 + rq * 8 + hh * 4, sv);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int e = rq * 4 + i;
                const float g1 = acc[db][e], g2 = acc[db + NB2][e];
                const float s = -1.0f * sv[i];
                acc[db][e] = g1 * c[i] - g2 * s;
                acc[db + NB2][e] = g2 * c[i] + g1 * s;
            }
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const int dbh = db + h * NB2;
                float x[4], wv[4];
                x4(dbh, rq, x);
                load4(w + dbh * 32 + rq * 8 + hh * 4, wv);
#pragma unroll
                for (int i = 0; i < 4; i++) term[dbh][rq * 4 + i] = acc[dbh][rq * 4 + i] * wv[i] * x[i] * inv;
            }
        }
    // The chunk sums (chunk j = 4*db + rq): each lane's four terms from 0,
    // the hh = 0 lane's sum swapped to the hh = 1 lane, which continues with
    // its own four; then the tree.
    float ch[G];
#pragma unroll
    for (int j = 0; j < G; j++) {
        float own = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) own += term[j / 4][(j % 4) * 4 + i];
        ch[j] = own;
    }
#pragma unroll
    for (int j = 0; j < G; j++) {
        float lo, hi;
        swap_halves(ch[j], lo, hi);  // lo: the hh = 0 lane's four-term sum
#pragma unroll
        for (int i = 0; i < 4; i++) lo += term[j / 4][(j % 4) * 4 + i];
        ch[j] = lo;  // the chunk's sum in the hh = 1 lane
    }
#pragma unroll
    for (int off = G / 2; off >= 1; off >>= 1)
#pragma unroll
        for (int j = 0; j < off; j++) ch[j] = ch[j] + ch[j + off];
    float dlo, dot;
    swap_halves(ch[0], dlo, dot);  // the hh = 1 lane's dot, in both lanes
    const float mean = dot / (float)DP;
    if (!ok) {
#pragma unroll
        for (int db = 0; db < NDB; db++) acc[db] = zero16();
        return;
    }
    // Pass 2: the row and the gain terms.
#pragma unroll
    for (int dbh = 0; dbh < NDB; dbh++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            const int d0 = dbh * 32 + rq * 8 + hh * 4;
            float x[4], wv[4];
            x4(dbh, rq, x);
            load4(w + d0, wv);
            const float4 o4 = pre[dbh][rq];
            float o[4] = {o4.x, o4.y, o4.z, o4.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float dy = acc[dbh][rq * 4 + i];
                const float xh = x[i] * inv;
                o[i] += inv * (dy * wv[i] - xh * mean);
                acc[dbh][rq * 4 + i] = dy * xh;
            }
            *reinterpret_cast<float4*>(dst + d0) = make_float4(o[0], o[1], o[2], o[3]);
        }
}

// The wave's gain-gradient partial: gp summed over the 32 lanes of each half
// (every lane of a half holds one row's terms for the same head dims),
// through the wave's LDS region xs (its pre-norm rows are no longer read):
// lane l writes chunk (db, rq) of its terms to the 16-byte slot
// (4*db + rq)*64 + l, then lane L = 4*k + i sums element i of chunk k over
// the 32 rows of each half, rows in the order k, k+1, .. (mod 32), so that the
// 16 lanes reading element i at once hit distinct banks.  The two sums are
// head dims (k/4)*32 + 8*(k%4) + 4*hh + i, written to part[0 .. DP) when
// `store`.
template <int NDB>
__device__ __forceinline__ void norm_partial_store(const f32x16 (&gp)[NDB], int lane, float* xs, float* part,
                                                   bool store) {
#pragma clang fp contract(off)
    constexpr int NK = NDB * 4;  // chunks of four dims per half row
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++)
            *reinterpret_cast<float4*>(xs + ((db * 4 + rq) * 64 + lane) * 4) =
                make_float4(gp[db][rq * 4 + 0], gp[db][rq * 4 + 1], gp[db][rq * 4 + 2], gp[db][rq * 4 + 3]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (lane >= NK * 4) return;
    const int k = lane >> 2, i = lane & 3;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        float sum = 0.0f;
        for (int r = 0; r < 32; r++) {
            const int row = (r + k) & 31;
            sum += xs[((k * 64) + h * 32 + row) * 4 + i];
        }
        if (store) part[(k >> 2) * 32 + (k & 3) * 8 + h * 4 + i] = sum;
    }
}

// The lane's part of a row (the layout write_grad_row writes), or zeros when
// `ok` is false.
template <int NDB>
__device__ __forceinline__ void load_grad_row(float4 (&v)[NDB][4], const float* row, int hh, bool ok) {
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++)
            v[db][rq] = ok ? *reinterpret_cast<const float4*>(row + db * 32 + rq * 8 + hh * 4)
                           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
}

// The lane's part of a gradient row, read ahead for the += epilogue modes
// (kEpiUnrotNorm too with NORM); false (nothing read) for the others.
template <int NDB, bool NORM = false>
__device__ __forceinline__ bool grad_row_prefetch(float4 (&pre)[NDB][4], const float* row, int hh,
                                                  const BwdParams& p) {
    if (p.epi != kEpiAdd && p.epi != kEpiUnrotAdd && !(NORM && p.epi == kEpiUnrotNorm)) return false;
    load_grad_row<NDB>(pre, row, hh, true);
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
