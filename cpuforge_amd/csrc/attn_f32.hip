// fp32 parity mode on gfx950: causal GQA attention forward, dQ and dK/dV with
// f32 inputs and v_mfma_f32_32x32x2_f32 (exact f32 products, f32
// accumulation), for head_dim 64 and 128 with 16-byte aligned rows.
//
// An f32 MFMA takes one value per lane and operand (lane l: A[l%32][l/32],
// B[l/32][l%32]), so every operand is read row-major:
//   - a "row" operand (K rows for S^T = K Q^T, Q/dO rows for S and dP in
//     dK/dV) is four consecutive head dims of one row per lane, one
//     ds_read_b128 feeding four MFMAs;
//   - a "column" operand (V^T for O^T += V^T P^T, K^T for dQ, dO^T and Q^T for
//     dK/dV) is one head dim per lane of one row per half-wave, a ds_read_b32.
// Tiles go straight from global memory into LDS (global_load_lds, 16 bytes a
// lane) through three-buffer rings, two tiles ahead of the compute; 16-byte
// chunk c of tile row r sits at chunk slot c ^ swz(r) of its row, so both
// read shapes are bank-conflict-free (see f32_swz).  The per-query softmax follows the bf16 kernels: the running
// max moves lazily, P is formed in the exp2 domain, and the MFMA k-index of
// every P/dS product is chosen so the accumulator registers of one product are
// the operands of the next.
//
// dK/dV parallelism: a workgroup owns 128 keys of one KV head for ONE query
// head of its group (and, on small grids, every QS-th query tile), so the
// serial chain of a workgroup is one head's query tiles, not the whole
// group's.  Each workgroup writes its dK/dV contribution to a scratch slot;
// attn_f32_reduce_kernel adds the slots of a KV head in a fixed order (query
// head, then query split), so results are reproducible bit for bit.  Where the
// scratch holds it, dK/dV also stores dS and dQ is one product per key tile
// over it (attn_bwd_dq_f32_ds_kernel), bit for bit the recompute's dQ.
//
// Grids: where the work units fill every workgroup slot, a persistent grid
// whose workgroups walk their XCD's units (persistent_item); else one
// workgroup per unit, with small grids' key (forward, dQ) or query (dK/dV)
// ranges split for balance.
#include <algorithm>
#include <vector>

#include "attn_params.hpp"
#include "cfattn_common.hpp"
#include "cfattn_kernels.hpp"

namespace cfattn {

namespace {

// Chunk slot swizzle of a tile row: a bijection on r % 16 (bits 2 and 3
// swapped), so (1) the 16 rows of a ds_read_b128 (same logical chunk) land on
// 16 distinct 16-byte bank groups, and (2) the two half-waves of a column read
// (rows r and r + 4 of the accumulator layout) use disjoint bank halves.
__device__ __forceinline__ int f32_swz(int r) { return (r & 3) | ((r >> 1) & 4) | ((r << 1) & 8); }
// Element (r, d) of a DP-wide f32 tile.
template <int DP>
__device__ __forceinline__ int f32_at(int r, int d) {
    return r * DP + ((((d >> 2) ^ f32_swz(r & 15))) << 2) + (d & 3);
}
// Accumulator row held by lane half hh at register index r of a 32x32 block.
__device__ __forceinline__ int acc_row(int r, int hh) { return ((r >> 2) << 3) + (hh << 2) + (r & 3); }

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, const f32x16& c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Issue this wave's share of the direct-to-LDS loads of a 32-row tile: rows
// row0 .. row0 + 31 (clamped to last_row, so padding rows repeat finite
// data) of a DP-wide f32 tensor with row stride `rs` floats.  A 1 KiB block
// is 64 chunk slots; slot p holds chunk (p % CPR) ^ swz(row) of row p / CPR.
// The loads are issued from inline assembly, so the compiler's wait-count
// tracking does not see them: the kernels wait for them with exact counts
// (f32_tile_wait), which lets a tile stay in flight across a barrier.
template <int DP, int NW>
__device__ __forceinline__ void f32_tile_dma(const float* __restrict__ g, long rs, int row0, int last_row,
                                             float* __restrict__ tile, int wv, int lane) {
    constexpr int CPR = DP / 4;
    constexpr int NBLK = 32 * DP / 256;
    constexpr int BPW = NBLK / NW;
    static_assert(NBLK % NW == 0, "tile blocks must split evenly over the waves");
#pragma unroll
    for (int i = 0; i < BPW; i++) {
        const int blk = wv * BPW + i;
        const int slot = blk * 64 + lane;
        const int r = slot / CPR;
        const int c = (slot % CPR) ^ f32_swz(r & 15);
        const long row = min(row0 + r, last_row);
        lds_load16_asm(g + row * rs + c * 4, tile + blk * 256);
    }
}

// End of a ring step: this wave's loads for the next step have landed (with
// `newer`, the EXTRA + two tiles' loads issued after them may still be in
// flight: loads complete in issue order) and its LDS reads of this step are
// done; then a barrier without __syncthreads' workgroup fence, whose
// vmcnt(0) would also wait for the newer loads.  Only the ring's
// direct-to-LDS loads are outstanding where it is called.
template <int DP, int NW, int EXTRA = 0>
__device__ __forceinline__ void f32_step_end(bool newer) {
    constexpr int kNewer = 2 * (32 * DP / 256) / NW + EXTRA;
    static_assert(kNewer >= 0 && kNewer < 64, "vmcnt range");
    if (newer)
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kNewer) : "memory");
    else
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Stored fp32 dS block (32 queries x 32 keys): the value of query row q and
// key column k sits where the dQ kernel's lane (q, (k >> 2) & 1) finds
// operand j = 4 * (k >> 3) + (k & 3) (its key acc_row(j, hh) = k), chunk-
// major so that each of the four 16-byte loads of a lane covers one
// contiguous KiB: slot (j / 4) * 256 + lane * 4 + j % 4.
__device__ __forceinline__ int f32_ds_slot(int q, int k) {
    return (k >> 3) * 256 + (q + 32 * ((k >> 2) & 1)) * 4 + (k & 3);
}

// Query tile, key split and split count of work unit u of one (sequence, KV
// head, head subset).  Without a key split (ks == 0) unit u is tile
// n_ttiles - 1 - u; with one, the units run over the tiles from the last
// (longest) down and over a tile's ks-key-tile runs in order.
struct F32Unit {
    int tile, split, ns;
};
__device__ __forceinline__ F32Unit f32_unit(int u, int n_ttiles, int tt, int seq, int ks) {
    if (ks == 0) return F32Unit{n_ttiles - 1 - u, 0, 1};
    for (int t = n_ttiles - 1;; t--) {
        const int n_kt = (min(seq, (t + 1) * tt) + 31) / 32;
        const int ns = (n_kt + ks - 1) / ks;
        if (u < ns || t == 0) return F32Unit{t, u, ns};
        u -= ns;
    }
}

}  // namespace

// ------------------------------------------------------------------ forward
// A wave owns 32 queries of one head; a workgroup of four waves covers hpw
// heads of one GQA group x tpw query blocks and shares 32-key K/V tiles.
// One work unit of the forward: query tile un.tile (key run un.split of
// un.ns) of group `rest` = (sequence * nkv + KV head) * n_sub + head subset.
// Every wave passes the same barriers; after the last one no wave reads the
// K/V buffers, so the next unit of a persistent workgroup may load into them.
template <int DP>
__device__ __forceinline__ void fwd_f32_unit(const FwdParams& p, const F32Unit un, int rest, float* sK0, float* sK1,
                                             float* sK2, float* sV0, float* sV1, float* sV2) {
    constexpr int NW = 4, BN = 32, HALF = DP / 2, NDB = DP / 32;
    constexpr float kLazy = 8.0f;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hh = lane >> 5;
    const int wv = wave_uniform(wave);

    const int TT = 32 * p.tpw;
    const int tile = un.tile;
    const int sub = rest % p.n_sub;
    rest /= p.n_sub;
    const int g = rest % p.nkv;
    const int b = rest / p.nkv;
    const int head = g * p.group + sub * p.hpw + wave % p.hpw;
    const int t_wave = tile * TT + (wave / p.hpw) * 32;
    const int tq = t_wave + l32;
    const int wg_end = min(p.seq, tile * TT + TT);
    const int kt_all = (wg_end + BN - 1) / BN;
    const int kt0 = un.ns > 1 ? un.split * p.ksplit : 0;
    const int n_kt = un.ns > 1 ? min(kt_all, kt0 + p.ksplit) : kt_all;
    const bool wave_active = t_wave < p.seq;
    const int wave_last = min(t_wave + 31, p.seq - 1);

    const long qrs = (long)p.nh * DP, kvrs = (long)p.nkv * DP;
    const float* kg = static_cast<const float*>(p.k) + (long)b * p.kv_bs + (long)g * DP;
    const float* vg = static_cast<const float*>(p.v) + (long)b * p.kv_bs + (long)g * DP;

    auto dma = [&](int kt, float* Kd, float* Vd) {
        f32_tile_dma<DP, NW>(kg, kvrs, kt * BN, p.seq - 1, Kd, wv, lane);
        f32_tile_dma<DP, NW>(vg, kvrs, kt * BN, p.seq - 1, Vd, wv, lane);
    };
    dma(kt0, sK0, sV0);

    // Q^T operand: query tq, head dims hh*HALF + kd.
    float qf[HALF];
    {
        const float* qrow = static_cast<const float*>(p.q) + (long)b * p.q_bs + (long)min(tq, p.seq - 1) * qrs +
                            (long)head * DP + hh * HALF;
#pragma unroll
        for (int i = 0; i < HALF / 4; i++) {
            const float4 v = *reinterpret_cast<const float4*>(qrow + 4 * i);
            qf[4 * i] = v.x;
            qf[4 * i + 1] = v.y;
            qf[4 * i + 2] = v.z;
            qf[4 * i + 3] = v.w;
        }
    }
    // The Q rows and tile kt0 have landed; a wait the compiler sees, so that
    // it puts none for the Q rows inside the loop (where the asm-issued tile
    // loads are in flight).
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);

    f32x16 oacc[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) oacc[i] = zero16();
    float m2 = -INFINITY, lsum = 0.0f;

    // Three K/V buffers: the tile two steps ahead is loaded during a step,
    // into the buffer the previous step read.
    auto step = [&](int kt, const float* Ks, const float* Vs, float* Kn, float* Vn) {
        const bool ahead = kt + 2 < n_kt;
        const int k0 = kt * BN;
        if (wave_active && k0 <= wave_last) {
            // S^T: rows = keys k0 + [0, 32), columns = this wave's queries.
            // The loads two tiles ahead issue behind the first MFMAs, whose
            // shadow covers their address arithmetic.
            // Each group's K row operands are read before the previous
            // group's MFMAs issue (pinned: the compiler otherwise reads them
            // after, and the products wait for the read).
            f32x16 sc = zero16();
            float4 an = *reinterpret_cast<const float4*>(Ks + f32_at<DP>(l32, hh * HALF));
#pragma unroll
            for (int c = 0; c < HALF / 4; c++) {
                const float4 a = an;
                if (c + 1 < HALF / 4) an = *reinterpret_cast<const float4*>(Ks + f32_at<DP>(l32, hh * HALF + 4 * c + 4));
                __builtin_amdgcn_sched_barrier(0);
                sc = mfma_f32(a.x, qf[4 * c], sc);
                sc = mfma_f32(a.y, qf[4 * c + 1], sc);
                sc = mfma_f32(a.z, qf[4 * c + 2], sc);
                sc = mfma_f32(a.w, qf[4 * c + 3], sc);
                __builtin_amdgcn_sched_barrier(0);
                if (c == 0 && ahead) dma(kt + 2, Kn, Vn);
            }
            float mx = -INFINITY;
            const bool masked = k0 + 31 > t_wave;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                if (masked && k0 + acc_row(r, hh) > tq) sc[r] = -INFINITY;
                mx = fmaxf(mx, sc[r]);
            }
            // Key k0 + 0 is unmasked for every query of the first tile the
            // wave visits (k0 <= t_wave there), so m2 is finite from then on.
            mx = max_halves(mx) * p.sl2;
            const float mnew = mx > m2 + kLazy ? mx : m2;
            if (__any(mnew != m2)) {
                const float alpha = __builtin_amdgcn_exp2f(m2 - mnew);
                lsum *= alpha;
#pragma unroll
                for (int i = 0; i < NDB; i++) oacc[i] *= alpha;
                m2 = mnew;
            }
            float pr[16];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                pr[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], p.sl2, -m2));
                lsum += pr[r];
            }
            // O^T += V^T P^T: product j pairs key acc_row(j, hh) of both operands.
#pragma unroll
            for (int db = 0; db < NDB; db++)
#pragma unroll
                for (int j = 0; j < 16; j++)
                    oacc[db] = mfma_f32(Vs[f32_at<DP>(acc_row(j, hh), db * 32 + l32)], pr[j], oacc[db]);
        } else if (ahead) {
            dma(kt + 2, Kn, Vn);
        }
        f32_step_end<DP, NW>(ahead);  // tile kt + 1 is in LDS
    };

    if (kt0 + 1 < n_kt) dma(kt0 + 1, sK1, sV1);
    f32_step_end<DP, NW>(kt0 + 1 < n_kt);
    for (int kt = kt0; kt < n_kt; kt += 3) {
        step(kt, sK0, sV0, sK2, sV2);
        if (kt + 1 < n_kt) step(kt + 1, sK1, sV1, sK0, sV0);
        if (kt + 2 < n_kt) step(kt + 2, sK2, sV2, sK1, sV1);
    }

    if (!wave_active) return;
    const float ltot = sum_halves(lsum);
    if (tq >= p.seq) return;
    if (un.ns > 1) {
        // A partial: only waves that saw a key of this split (every query of
        // such a wave did), unnormalised.
        if (t_wave < kt0 * BN) return;
        const long row = (long)un.split * p.part_rows + ((long)b * p.nh + head) * p.seq + tq;
        float* prow = p.part + row * DP;
#pragma unroll
        for (int db = 0; db < NDB; db++)
#pragma unroll
            for (int rq = 0; rq < 4; rq++)
                *reinterpret_cast<float4*>(prow + db * 32 + rq * 8 + hh * 4) =
                    make_float4(oacc[db][rq * 4], oacc[db][rq * 4 + 1], oacc[db][rq * 4 + 2], oacc[db][rq * 4 + 3]);
        if (hh == 0) p.part_ml[row] = make_float2(m2, ltot);
        return;
    }
    const float inv = 1.0f / ltot;
    float* orow = p.o + (long)b * p.q_bs + (long)tq * qrs + (long)head * DP;
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++)
            *reinterpret_cast<float4*>(orow + db * 32 + rq * 8 + hh * 4) =
                make_float4(oacc[db][rq * 4] * inv, oacc[db][rq * 4 + 1] * inv, oacc[db][rq * 4 + 2] * inv,
                            oacc[db][rq * 4 + 3] * inv);
    if (hh == 0) p.lse[((long)b * p.nh + head) * p.seq + tq] = (m2 + __log2f(ltot)) * kLn2;
}

template <int DP>
__global__ __launch_bounds__(256) void attn_fwd_f32_kernel(const FwdParams p) {
    constexpr int BN = 32;
    __shared__ __attribute__((aligned(16))) float sK0[BN * DP];
    __shared__ __attribute__((aligned(16))) float sK1[BN * DP];
    __shared__ __attribute__((aligned(16))) float sK2[BN * DP];
    __shared__ __attribute__((aligned(16))) float sV0[BN * DP];
    __shared__ __attribute__((aligned(16))) float sV1[BN * DP];
    __shared__ __attribute__((aligned(16))) float sV2[BN * DP];
    if (p.xcd_wgs > 0) {
        const int n_groups = p.n_items / p.n_ttiles;
        int tile, grp;
        for (int it = 0; persistent_item(it, n_groups, p.n_ttiles, p.xcd_wgs, p.walk_gm, tile, grp); it++)
            fwd_f32_unit<DP>(p, F32Unit{tile, 0, 1}, grp, sK0, sK1, sK2, sV0, sV1, sV2);
        return;
    }
    const int id = xcd_remap(blockIdx.x, p.n_wg, p.xcd);
    const F32Unit un = f32_unit(id % p.units, p.n_ttiles, 32 * p.tpw, p.seq, p.ksplit);  // longest tiles first
    fwd_f32_unit<DP>(p, un, id / p.units, sK0, sK1, sK2, sV0, sV1, sV2);
}

// -------------------------------------------------------------------- dQ
// The forward's decomposition; per 32-key tile: S^T = K Q^T, dP^T = V dO^T,
// dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T.  The softmax scale is applied
// once to dQ.
// One work unit of the dQ grid, as fwd_f32_unit.
template <int DP>
__device__ __forceinline__ void dq_f32_unit(const BwdParams& p, const F32Unit un, int rest, float* sK0, float* sK1,
                                            float* sK2, float* sV0, float* sV1, float* sV2) {
    constexpr int NW = 4, BN = 32, HALF = DP / 2, NDB = DP / 32;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hh = lane >> 5;
    const int wv = wave_uniform(wave);

    const int TT = 32 * p.tpw;
    const int tile = un.tile;
    const int sub = rest % p.n_sub;
    rest /= p.n_sub;
    const int g = rest % p.nkv;
    const int b = rest / p.nkv;
    const int head = g * p.group + sub * p.hpw + wave % p.hpw;
    const int t_wave = tile * TT + (wave / p.hpw) * 32;
    const int tq = t_wave + l32;
    const int wg_end = min(p.seq, tile * TT + TT);
    const int kt_all = (wg_end + BN - 1) / BN;
    const int kt0 = un.ns > 1 ? un.split * p.ksplit : 0;
    const int n_kt = un.ns > 1 ? min(kt_all, kt0 + p.ksplit) : kt_all;
    const bool wave_active = t_wave < p.seq;
    const int wave_last = min(t_wave + 31, p.seq - 1);

    const long qrs = (long)p.nh * DP, kvrs = (long)p.nkv * DP;
    const float* kg = static_cast<const float*>(p.k) + (long)b * p.kv_bs + (long)g * DP;
    const float* vg = static_cast<const float*>(p.v) + (long)b * p.kv_bs + (long)g * DP;
    const long qoff = (long)b * p.q_bs + (long)min(tq, p.seq - 1) * qrs + (long)head * DP + hh * HALF;

    auto dma = [&](int kt, float* Kd, float* Vd) {
        f32_tile_dma<DP, NW>(kg, kvrs, kt * BN, p.seq - 1, Kd, wv, lane);
        f32_tile_dma<DP, NW>(vg, kvrs, kt * BN, p.seq - 1, Vd, wv, lane);
    };
    dma(kt0, sK0, sV0);

    float qf[HALF], of[HALF];
#pragma unroll
    for (int i = 0; i < HALF / 4; i++) {
        const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p.q) + qoff + 4 * i);
        const float4 c = *reinterpret_cast<const float4*>(static_cast<const float*>(p.d_o) + qoff + 4 * i);
        qf[4 * i] = a.x, qf[4 * i + 1] = a.y, qf[4 * i + 2] = a.z, qf[4 * i + 3] = a.w;
        of[4 * i] = c.x, of[4 * i + 1] = c.y, of[4 * i + 2] = c.z, of[4 * i + 3] = c.w;
    }
    const long lrow = ((long)b * p.nh + head) * p.seq + min(tq, p.seq - 1);
    const float lq = p.lse[lrow] * kLog2e;
    const float dlq = p.delta[lrow];
    // The rows above and tile kt0 have landed; a wait the compiler sees (see
    // the forward).
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);

    f32x16 acc[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) acc[i] = zero16();

    auto step = [&](int kt, const float* Ks, const float* Vs, float* Kn, float* Vn) {
        const bool ahead = kt + 2 < n_kt;
        const int k0 = kt * BN;
        if (wave_active && k0 <= wave_last) {
            f32x16 sc = zero16(), dp = zero16();
#pragma unroll
            for (int c = 0; c < HALF / 4; c++) {
                const float4 a = *reinterpret_cast<const float4*>(Ks + f32_at<DP>(l32, hh * HALF + 4 * c));
                const float4 v = *reinterpret_cast<const float4*>(Vs + f32_at<DP>(l32, hh * HALF + 4 * c));
                sc = mfma_f32(a.x, qf[4 * c], sc);
                dp = mfma_f32(v.x, of[4 * c], dp);
                sc = mfma_f32(a.y, qf[4 * c + 1], sc);
                dp = mfma_f32(v.y, of[4 * c + 1], dp);
                sc = mfma_f32(a.z, qf[4 * c + 2], sc);
                dp = mfma_f32(v.z, of[4 * c + 2], dp);
                sc = mfma_f32(a.w, qf[4 * c + 3], sc);
                dp = mfma_f32(v.w, of[4 * c + 3], dp);
                if (c == 0 && ahead) dma(kt + 2, Kn, Vn);  // behind the first MFMAs, as the forward
            }
            const bool masked = k0 + 31 > t_wave;
            float ds[16];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], p.sl2, -lq));
                if (masked && k0 + acc_row(r, hh) > tq) pv = 0.0f;
                ds[r] = pv * (dp[r] - dlq);
            }
#pragma unroll
            for (int db = 0; db < NDB; db++)
#pragma unroll
                for (int j = 0; j < 16; j++)
                    acc[db] = mfma_f32(Ks[f32_at<DP>(acc_row(j, hh), db * 32 + l32)], ds[j], acc[db]);
        } else if (ahead) {
            dma(kt + 2, Kn, Vn);
        }
        f32_step_end<DP, NW>(ahead);
    };

    if (kt0 + 1 < n_kt) dma(kt0 + 1, sK1, sV1);
    f32_step_end<DP, NW>(kt0 + 1 < n_kt);
    for (int kt = kt0; kt < n_kt; kt += 3) {
        step(kt, sK0, sV0, sK2, sV2);
        if (kt + 1 < n_kt) step(kt + 1, sK1, sV1, sK0, sV0);
        if (kt + 2 < n_kt) step(kt + 2, sK2, sV2, sK1, sV1);
    }
    if (!wave_active || tq >= p.seq) return;
    if (un.ns > 1) {
        // A partial (scaled), written only by waves that saw a key of this
        // split; attn_f32_dq_merge_kernel adds the splits to dq in order.
        if (t_wave < kt0 * BN) return;
        float* prow =
            p.qpart + ((long)un.split * p.part_rows + ((long)b * p.nh + head) * p.seq + tq) * DP;
#pragma unroll
        for (int db = 0; db < NDB; db++)
#pragma unroll
            for (int rq = 0; rq < 4; rq++)
                *reinterpret_cast<float4*>(prow + db * 32 + rq * 8 + hh * 4) =
                    make_float4(acc[db][rq * 4] * p.scale, acc[db][rq * 4 + 1] * p.scale,
                                acc[db][rq * 4 + 2] * p.scale, acc[db][rq * 4 + 3] * p.scale);
        return;
    }
    float* row = p.dq + (long)b * p.q_bs + (long)tq * qrs + (long)head * DP;
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            float4* dst = reinterpret_cast<float4*>(row + db * 32 + rq * 8 + hh * 4);
            float4 v = *dst;
            v.x += acc[db][rq * 4] * p.scale;
            v.y += acc[db][rq * 4 + 1] * p.scale;
            v.z += acc[db][rq * 4 + 2] * p.scale;
            v.w += acc[db][rq * 4 + 3] * p.scale;
            *dst = v;
        }
}

// Two waves per SIMD at head_dim 64 (the registers fit; measured 7% faster
// at B8 S2048 9/3 heads), one at 128.
template <int DP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DP == 64 ? 2 : 1, DP == 64 ? 2 : 1))) void
attn_bwd_dq_f32_kernel(const BwdParams p) {
    constexpr int BN = 32;
    __shared__ __attribute__((aligned(16))) float sK0[BN * DP];
    __shared__ __attribute__((aligned(16))) float sK1[BN * DP];
    __shared__ __attribute__((aligned(16))) float sK2[BN * DP];
    __shared__ __attribute__((aligned(16))) float sV0[BN * DP];
    __shared__ __attribute__((aligned(16))) float sV1[BN * DP];
    __shared__ __attribute__((aligned(16))) float sV2[BN * DP];
    if (p.q_xcd_wgs > 0) {
        const int n_groups = p.q_items / p.n_ttiles;
        int tile, grp;
        for (int it = 0; persistent_item(it, n_groups, p.n_ttiles, p.q_xcd_wgs, p.q_walk_gm, tile, grp); it++)
            dq_f32_unit<DP>(p, F32Unit{tile, 0, 1}, grp, sK0, sK1, sK2, sV0, sV1, sV2);
        return;
    }
    const int id = xcd_remap(blockIdx.x, p.n_wg_q, p.xcd);
    const F32Unit un = f32_unit(id % p.units_q, p.n_ttiles, 32 * p.tpw, p.seq, p.ksplit);
    dq_f32_unit<DP>(p, un, id / p.units_q, sK0, sK1, sK2, sV0, sV1, sV2);
}

// ------------------------------------------------------ dQ from stored dS
// dQ^T += K^T dS^T with dS read from the blocks the dK/dV kernel stored
// (p.ds32), no S / dP recompute: the dQ kernel's decomposition and product
// order, so dQ is bitwise the recompute's.  Per 32-key tile the workgroup
// loads the K tile (shared) and each wave its own dS block, both straight
// into three-buffer LDS rings; every wave loads a block each step (past its
// diagonal, or past the end, a valid block it does not use), so the per-wave
// load count stays uniform for the exact waits.
template <int DP>
__device__ __forceinline__ void dq_f32_ds_unit(const BwdParams& p, const int tile, int rest, float* sK0, float* sK1,
                                               float* sK2, float* sD0, float* sD1, float* sD2) {
    constexpr int NW = 4, BN = 32, NDB = DP / 32;
    constexpr int BPW = (32 * DP / 256) / NW;  // K tile loads per wave
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hh = lane >> 5;
    const int wv = wave_uniform(wave);

    const int TT = 32 * p.tpw;
    const int sub = rest % p.n_sub;
    rest /= p.n_sub;
    const int g = rest % p.nkv;
    const int b = rest / p.nkv;
    const int head = g * p.group + sub * p.hpw + wave % p.hpw;
    const int t_wave = tile * TT + (wave / p.hpw) * 32;
    const int tq = t_wave + l32;
    const int wg_end = min(p.seq, tile * TT + TT);
    const int n_kt = (wg_end + BN - 1) / BN;
    const bool wave_active = t_wave < p.seq;
    const int wave_last = min(t_wave + 31, p.seq - 1);

    const long qrs = (long)p.nh * DP, kvrs = (long)p.nkv * DP;
    const float* kg = static_cast<const float*>(p.k) + (long)b * p.kv_bs + (long)g * DP;
    // The wave's dS row of blocks: query block qi (clamped to the last one,
    // whose blocks exist, for a wave past the end), key block kt at + kt.
    const int qi = min(t_wave, p.seq - 1) >> 5;
    const float* dsrow = p.ds32 + (((long)b * p.nh + head) * p.ds_ntri + (long)qi * (qi + 1) / 2) * 1024;

    auto dma = [&](int kt, float* Kd, float* Dd) {
        f32_tile_dma<DP, NW>(kg, kvrs, kt * BN, p.seq - 1, Kd, wv, lane);
        const float* src = dsrow + (long)min(kt, qi) * 1024 + lane * 4;
        float* dst = Dd + wv * 1024;
#pragma unroll
        for (int c = 0; c < 4; c++) lds_load16_asm(src + c * 256, dst + c * 256);
    };
    dma(0, sK0, sD0);

    f32x16 acc[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) acc[i] = zero16();

    auto step = [&](int kt, const float* Ks, const float* Ds, float* Kn, float* Dn) {
        const bool ahead = kt + 2 < n_kt;
        const int k0 = kt * BN;
        if (ahead) dma(kt + 2, Kn, Dn);
        if (wave_active && k0 <= wave_last) {
            float ds[16];
            const float* dsl = Ds + wv * 1024 + lane * 4;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const float4 v = *reinterpret_cast<const float4*>(dsl + c * 256);
                ds[4 * c] = v.x, ds[4 * c + 1] = v.y, ds[4 * c + 2] = v.z, ds[4 * c + 3] = v.w;
            }
#pragma unroll
            for (int db = 0; db < NDB; db++)
#pragma unroll
                for (int j = 0; j < 16; j++)
                    acc[db] = mfma_f32(Ks[f32_at<DP>(acc_row(j, hh), db * 32 + l32)], ds[j], acc[db]);
        }
        f32_step_end<DP, NW, 4 - BPW>(ahead);  // tile kt + 1 and its dS blocks are in LDS
    };

    if (n_kt > 1) dma(1, sK1, sD1);
    f32_step_end<DP, NW, 4 - BPW>(n_kt > 1);
    for (int kt = 0; kt < n_kt; kt += 3) {
        step(kt, sK0, sD0, sK2, sD2);
        if (kt + 1 < n_kt) step(kt + 1, sK1, sD1, sK0, sD0);
        if (kt + 2 < n_kt) step(kt + 2, sK2, sD2, sK1, sD1);
    }
    if (!wave_active || tq >= p.seq) return;
    const long qoff = (long)b * p.q_bs + (long)tq * qrs + (long)head * DP;
    float* row = p.dq + qoff;
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            float4* dst = reinterpret_cast<float4*>(row + db * 32 + rq * 8 + hh * 4);
            float4 v = *dst;
            v.x += acc[db][rq * 4] * p.scale;
            v.y += acc[db][rq * 4 + 1] * p.scale;
            v.z += acc[db][rq * 4 + 2] * p.scale;
            v.w += acc[db][rq * 4 + 3] * p.scale;
            *dst = v;
        }
}

template <int DP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DP == 64 ? 2 : 1, DP == 64 ? 2 : 1))) void
attn_bwd_dq_f32_ds_kernel(const BwdParams p) {
    constexpr int BN = 32;
    __shared__ __attribute__((aligned(16))) float sK0[BN * DP];
    __shared__ __attribute__((aligned(16))) float sK1[BN * DP];
    __shared__ __attribute__((aligned(16))) float sK2[BN * DP];
    __shared__ __attribute__((aligned(16))) float sD0[4 * 1024];
    __shared__ __attribute__((aligned(16))) float sD1[4 * 1024];
    __shared__ __attribute__((aligned(16))) float sD2[4 * 1024];
    if (p.q_xcd_wgs > 0) {
        int tile, grp;
        for (int it = 0;
             persistent_item(it, p.q_items / p.n_ttiles, p.n_ttiles, p.q_xcd_wgs, p.q_walk_gm, tile, grp); it++)
            dq_f32_ds_unit<DP>(p, tile, grp, sK0, sK1, sK2, sD0, sD1, sD2);
        return;
    }
    const int id = xcd_remap(blockIdx.x, p.n_wg_q, p.xcd);
    dq_f32_ds_unit<DP>(p, p.n_ttiles - 1 - id % p.n_ttiles, id / p.n_ttiles, sK0, sK1, sK2, sD0, sD1, sD2);
}

// ------------------------------------------------------------------ dK/dV
// Workgroup = (128-key tile, query head h, sequence, query split qs): four
// waves of 32 keys share 32-query Q/dO tiles of head h; the workgroup visits
// the query tiles qt_begin + qs, + QS, ... that can see its keys.  Per step:
// S = Q K^T, dP = dO V^T, P = exp2(S*scale*log2e - lse*log2e), dS = P (dP -
// delta), dV^T += dO^T P, dK^T += Q^T dS.  The result goes to scratch slot
// (h % group) * qs_n + qs of the KV head, dK already scaled.  QS depends on
// the key tile: low key tiles see more query tiles and get more splits, so
// every workgroup has at most qt_run steps (f32_kv_splits).
struct F32DkdvArgs {
    float* part;     // dK slots [slots][batch][seq][nkv][DP], then the dV slots
    long part_half;  // floats per slot
    int qs_n;        // slot stride: the largest QS (key tile 0)
    int slots;       // group * qs_n
    int qt_run;      // query tiles per split at most
    int units;       // workgroups per (sequence, query head)
    int xcd_wgs;     // persistent grid: workgroups per XCD (0: one unit per workgroup)
    int walk_gm;     // its walk order (persistent_item)
};

// Query splits of 128-key tile kvt: its n_qt - 4 kvt query tiles in runs of
// at most qt_run.
__device__ __forceinline__ int f32_kv_splits(int kvt, int n_qt, int qt_run) {
    return (n_qt - 4 * kvt + qt_run - 1) / qt_run;
}

// One work unit of the dK/dV grid: unit u of group rest = sequence * nh +
// query head (units in key-tile order, a key tile's query splits
// consecutive).  As fwd_f32_unit, every wave passes the same barriers and no
// LDS read follows the last one.
template <int DP>
__device__ __forceinline__ void dkdv_f32_unit(const BwdParams& p, const F32DkdvArgs& a, int u, int rest, float* sQ0,
                                              float* sQ1, float* sQ2, float* sO0, float* sO1, float* sO2,
                                              float (*sLD)[64]) {
    constexpr int NW = 4, BM = 32, HALF = DP / 2, NDB = DP / 32;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hh = lane >> 5;
    const int wv = wave_uniform(wave);

    const int n_qt = (p.seq + BM - 1) / BM;
    int kvt = 0, qs_n = 1;  // low key tiles see the most queries: first
    for (;; kvt++) {
        qs_n = f32_kv_splits(kvt, n_qt, a.qt_run);
        if (u < qs_n || kvt == p.n_kvtiles - 1) break;
        u -= qs_n;
    }
    const int qs = u;
    const int h = rest % p.nh;
    const int b = rest / p.nh;
    const int g = h / p.group;
    const int wg_key0 = kvt * 128;
    const int key0 = wg_key0 + wave * 32;
    const int kw = key0 + l32;
    const bool wave_active = key0 < p.seq;

    const long qrs = (long)p.nh * DP, kvrs = (long)p.nkv * DP;
    const float* qg = static_cast<const float*>(p.q) + (long)b * p.q_bs + (long)h * DP;
    const float* og = static_cast<const float*>(p.d_o) + (long)b * p.q_bs + (long)h * DP;
    const float* lse_h = p.lse + ((long)b * p.nh + h) * p.seq;
    const float* dlt_h = p.delta + ((long)b * p.nh + h) * p.seq;

    const int qt_first = wg_key0 / BM + qs;
    const int n_steps = qt_first < n_qt ? (n_qt - qt_first + qs_n - 1) / qs_n : 0;
    auto step_q0 = [&](int s) { return (qt_first + s * qs_n) * BM; };

    // Step s's Q and dO tiles, and its lse / delta entries (every wave
    // loads all 64, so each wave's load count per step is the same; rows
    // past the end repeat the last row and are masked in the step).
    auto dma = [&](int s, float* Qd, float* Od, float* LDd) {
        const int q0 = step_q0(s);
        f32_tile_dma<DP, NW>(qg, qrs, q0, p.seq - 1, Qd, wv, lane);
        f32_tile_dma<DP, NW>(og, qrs, q0, p.seq - 1, Od, wv, lane);
        const int t = min(q0 + (lane & (BM - 1)), p.seq - 1);
        lds_load4_asm((lane < BM ? lse_h : dlt_h) + t, LDd);
    };
    if (n_steps > 0) dma(0, sQ0, sO0, sLD[0]);

    // K^T / V^T operands: key kw, head dims hh*HALF + kd.
    float kf[HALF], vf[HALF];
    {
        const long off = (long)b * p.kv_bs + (long)min(kw, p.seq - 1) * kvrs + (long)g * DP + hh * HALF;
#pragma unroll
        for (int i = 0; i < HALF / 4; i++) {
            const float4 x = *reinterpret_cast<const float4*>(static_cast<const float*>(p.k) + off + 4 * i);
            const float4 y = *reinterpret_cast<const float4*>(static_cast<const float*>(p.v) + off + 4 * i);
            kf[4 * i] = x.x, kf[4 * i + 1] = x.y, kf[4 * i + 2] = x.z, kf[4 * i + 3] = x.w;
            vf[4 * i] = y.x, vf[4 * i + 1] = y.y, vf[4 * i + 2] = y.z, vf[4 * i + 3] = y.w;
        }
    }
    // The K/V rows and step 0's loads have landed; a wait the compiler sees
    // (see the forward).
    __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    f32x16 dkt[NDB], dvt[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) dkt[i] = zero16(), dvt[i] = zero16();

    // Three Q/dO buffers: the tiles two steps ahead are loaded during a
    // step, into the buffers the previous step read.
    auto step = [&](int s, const float* Qs, const float* Os, const float* LDs, float* Qn, float* On, float* LDn) {
        const bool ahead = s + 2 < n_steps;
        const int q0 = step_q0(s);
        if (wave_active && q0 + BM - 1 >= key0 && q0 < p.seq) {
            // S and dP: rows = queries q0 + [0, 32), columns = this wave's keys.
            // Q / dO row operands read a group ahead, as the forward's K rows.
            f32x16 sc = zero16(), dp = zero16();
            float4 xn = *reinterpret_cast<const float4*>(Qs + f32_at<DP>(l32, hh * HALF));
            float4 yn = *reinterpret_cast<const float4*>(Os + f32_at<DP>(l32, hh * HALF));
#pragma unroll
            for (int c = 0; c < HALF / 4; c++) {
                const float4 x = xn, y = yn;
                if (c + 1 < HALF / 4) {
                    xn = *reinterpret_cast<const float4*>(Qs + f32_at<DP>(l32, hh * HALF + 4 * c + 4));
                    yn = *reinterpret_cast<const float4*>(Os + f32_at<DP>(l32, hh * HALF + 4 * c + 4));
                }
                __builtin_amdgcn_sched_barrier(0);
                sc = mfma_f32(x.x, kf[4 * c], sc);
                dp = mfma_f32(y.x, vf[4 * c], dp);
                sc = mfma_f32(x.y, kf[4 * c + 1], sc);
                dp = mfma_f32(y.y, vf[4 * c + 1], dp);
                sc = mfma_f32(x.z, kf[4 * c + 2], sc);
                dp = mfma_f32(y.z, vf[4 * c + 2], dp);
                sc = mfma_f32(x.w, kf[4 * c + 3], sc);
                dp = mfma_f32(y.w, vf[4 * c + 3], dp);
                __builtin_amdgcn_sched_barrier(0);
                if (c == 0 && ahead) dma(s + 2, Qn, On, LDn);  // behind the first MFMAs, as the forward
            }
            // Masked: the diagonal steps and the one past the sequence end
            // (P = 0 for keys after the query and for queries >= seq).
            const bool masked = q0 < key0 + 31 || q0 + BM > p.seq;
            float pr[16], ds[16];
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const float4 l4 = *reinterpret_cast<const float4*>(LDs + g4 * 8 + hh * 4);
                const float4 d4 = *reinterpret_cast<const float4*>(LDs + BM + g4 * 8 + hh * 4);
                const float lv[4] = {l4.x * kLog2e, l4.y * kLog2e, l4.z * kLog2e, l4.w * kLog2e};
                const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = g4 * 4 + i;
                    const int qr = q0 + acc_row(r, hh);
                    float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], p.sl2, -lv[i]));
                    if (masked && (kw > qr || qr >= p.seq)) pv = 0.0f;
                    pr[r] = pv;
                    ds[r] = pv * (dp[r] - dv[i]);
                }
            }
            if (p.ds32) {
                // dS block (query block q0 / 32, key block key0 / 32) for the
                // stored-dS dQ kernel: the values it would recompute, bit for
                // bit (the same S, dP, lse and delta arithmetic).  Non-
                // temporal: read once, by the dQ kernel.  (Issued after the
                // step's barrier instead, the values held across it spill.)
                const int qi = q0 >> 5, ki = key0 >> 5;
                float* blk = p.ds32 + (((long)b * p.nh + h) * p.ds_ntri + (long)qi * (qi + 1) / 2 + ki) * 1024;
#pragma unroll
                for (int r = 0; r < 16; r++) __builtin_nontemporal_store(ds[r], blk + f32_ds_slot(acc_row(r, hh), l32));
            }
            // dV^T += dO^T P and dK^T += Q^T dS; product j pairs query
            // acc_row(j, hh) of both operands.
#pragma unroll
            for (int db = 0; db < NDB; db++)
#pragma unroll
                for (int j = 0; j < 16; j++) {
                    const int at = f32_at<DP>(acc_row(j, hh), db * 32 + l32);
                    dvt[db] = mfma_f32(Os[at], pr[j], dvt[db]);
                    dkt[db] = mfma_f32(Qs[at], ds[j], dkt[db]);
                }
        } else if (ahead) {
            dma(s + 2, Qn, On, LDn);
        }
        f32_step_end<DP, NW, 1>(ahead);  // step s + 1's tiles and entries are in LDS
    };

    if (n_steps > 1) dma(1, sQ1, sO1, sLD[1]);
    f32_step_end<DP, NW, 1>(n_steps > 1);
    for (int s = 0; s < n_steps; s += 3) {
        step(s, sQ0, sO0, sLD[0], sQ2, sO2, sLD[2]);
        if (s + 1 < n_steps) step(s + 1, sQ1, sO1, sLD[1], sQ0, sO0, sLD[0]);
        if (s + 2 < n_steps) step(s + 2, sQ2, sO2, sLD[2], sQ1, sO1, sLD[1]);
    }

    if (!wave_active || kw >= p.seq) return;
    const int slot = (h % p.group) * a.qs_n + qs;
    const long roff = (long)b * p.kv_bs + (long)kw * kvrs + (long)g * DP;
    float* pk = a.part + (long)slot * a.part_half + roff;
    float* pv = pk + (long)a.slots * a.part_half;
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            const int d = db * 32 + rq * 8 + hh * 4;
            *reinterpret_cast<float4*>(pk + d) =
                make_float4(dkt[db][rq * 4] * p.scale, dkt[db][rq * 4 + 1] * p.scale, dkt[db][rq * 4 + 2] * p.scale,
                            dkt[db][rq * 4 + 3] * p.scale);
            *reinterpret_cast<float4*>(pv + d) =
                make_float4(dvt[db][rq * 4], dvt[db][rq * 4 + 1], dvt[db][rq * 4 + 2], dvt[db][rq * 4 + 3]);
        }
}

// Two waves per SIMD at head_dim 64 (two workgroups per CU: the registers
// fit with a few spills outside the step loop; measured 13% faster at B8
// S2048 9/3 heads than one), one at 128.
template <int DP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DP == 64 ? 2 : 1, DP == 64 ? 2 : 1))) void
attn_bwd_dkdv_f32_kernel(const BwdParams p, const F32DkdvArgs a) {
    constexpr int BM = 32;
    __shared__ __attribute__((aligned(16))) float sQ0[BM * DP];
    __shared__ __attribute__((aligned(16))) float sQ1[BM * DP];
    __shared__ __attribute__((aligned(16))) float sQ2[BM * DP];
    __shared__ __attribute__((aligned(16))) float sO0[BM * DP];
    __shared__ __attribute__((aligned(16))) float sO1[BM * DP];
    __shared__ __attribute__((aligned(16))) float sO2[BM * DP];
    // lse (entries 0..31) and delta (32..63) of a step's queries, one ring
    // slot per tile buffer.
    __shared__ __attribute__((aligned(16))) float sLD[3][2 * BM];
    if (a.xcd_wgs > 0) {
        // Persistent: units longest (lowest key tile) first, as the forward.
        int t, grp;
        for (int it = 0; persistent_item(it, p.batch * p.nh, a.units, a.xcd_wgs, a.walk_gm, t, grp); it++)
            dkdv_f32_unit<DP>(p, a, a.units - 1 - t, grp, sQ0, sQ1, sQ2, sO0, sO1, sO2, sLD);
        return;
    }
    const int id = xcd_remap(blockIdx.x, p.n_wg_kv, p.xcd);
    dkdv_f32_unit<DP>(p, a, id % a.units, id / a.units, sQ0, sQ1, sQ2, sO0, sO1, sO2, sLD);
}

// dk += sum over slots (query head of the group, then query split) of the
// dK slots, dv likewise; four floats per thread.  The workgroups of a key
// tile's splits write their slots for all of its keys (zeros where they saw
// no query), so the slots read here are defined; the splits beyond the key
// tile's count are neither written nor read.
__global__ __launch_bounds__(256) void attn_f32_reduce_kernel(const float* __restrict__ part, const F32DkdvArgs a,
                                                              int seq, int row_floats, int group,
                                                              float* __restrict__ dk, float* __restrict__ dv) {
    const long i4 = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long half = a.part_half;
    if (i4 * 4 >= half) return;
    const int key = (int)((i4 * 4 / row_floats) % seq);
    const int qs_n = f32_kv_splits(key / 128, (seq + 31) / 32, a.qt_run);
    const float4* pk = reinterpret_cast<const float4*>(part) + i4;
    const float4* pv = reinterpret_cast<const float4*>(part + (long)a.slots * half) + i4;
    const long stride = half / 4;
    float4 sk = pk[0], sv = pv[0];
    for (int hg = 0; hg < group; hg++)
        for (int q = hg == 0 ? 1 : 0; q < qs_n; q++) {
            const long s = (long)hg * a.qs_n + q;
            const float4 x = pk[s * stride], c = pv[s * stride];
            sk.x += x.x, sk.y += x.y, sk.z += x.z, sk.w += x.w;
            sv.x += c.x, sv.y += c.y, sv.z += c.z, sv.w += c.w;
        }
    float4* dk4 = reinterpret_cast<float4*>(dk) + i4;
    float4* dv4 = reinterpret_cast<float4*>(dv) + i4;
    float4 x = *dk4, y = *dv4;
    x.x += sk.x, x.y += sk.y, x.z += sk.z, x.w += sk.w;
    y.x += sv.x, y.y += sv.y, y.z += sv.z, y.w += sv.w;
    *dk4 = x;
    *dv4 = y;
}

// ------------------------------------------------------------ key splits
// Shared by the two merges: the number of splits holding row `tq` (0 when its
// query tile has a single split and its workgroup wrote the final result).
// Split s holds the row iff the row's 32-query block qb reaches it
// (s * ks <= qb), the condition under which the kernels wrote it.
__device__ __forceinline__ int f32_row_splits(int tq, int seq, int tt, int ks) {
    const int t = tq / tt;
    const int n_kt = (min(seq, (t + 1) * tt) + 31) / 32;
    if (n_kt <= ks) return 0;
    return (tq >> 5) / ks + 1;
}

// O and lse of the rows of split query tiles: m = max_s m_s, w_s =
// 2^(m_s - m), l = sum_s w_s l_s, O = sum_s w_s O_s / l, lse = (m + log2 l) ln 2,
// splits in order.  DP/4 threads per row, four head dims each.
template <int DP>
__global__ __launch_bounds__(256) void attn_f32_fwd_merge_kernel(const FwdParams p) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long row = i / (DP / 4);
    if (row >= p.part_rows) return;
    const int c = (int)(i % (DP / 4));
    const int tq = (int)(row % p.seq);
    const int ns = f32_row_splits(tq, p.seq, 32 * p.tpw, p.ksplit);
    if (ns == 0) return;
    float m = -INFINITY;
    for (int s = 0; s < ns; s++) m = fmaxf(m, p.part_ml[s * p.part_rows + row].x);
    float l = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s = 0; s < ns; s++) {
        const float2 ml = p.part_ml[s * p.part_rows + row];
        const float w = __builtin_amdgcn_exp2f(ml.x - m);
        const float4 o = reinterpret_cast<const float4*>(p.part + (s * p.part_rows + row) * DP)[c];
        l += w * ml.y;
        acc.x += w * o.x, acc.y += w * o.y, acc.z += w * o.z, acc.w += w * o.w;
    }
    const float inv = 1.0f / l;
    const long bh = row / p.seq;  // sequence * nh + head
    const long b = bh / p.nh, head = bh % p.nh;
    float* orow = p.o + b * p.q_bs + (long)tq * p.nh * DP + head * DP;
    reinterpret_cast<float4*>(orow)[c] = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    if (c == 0) p.lse[row] = (m + __log2f(l)) * kLn2;
}

// dq += sum over the splits of a row, in split order.
template <int DP>
__global__ __launch_bounds__(256) void attn_f32_dq_merge_kernel(const BwdParams p) {
    const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long row = i / (DP / 4);
    if (row >= p.part_rows) return;
    const int c = (int)(i % (DP / 4));
    const int tq = (int)(row % p.seq);
    const int ns = f32_row_splits(tq, p.seq, 32 * p.tpw, p.ksplit);
    if (ns == 0) return;
    float4 sum = reinterpret_cast<const float4*>(p.qpart + row * DP)[c];
    for (int s = 1; s < ns; s++) {
        const float4 v = reinterpret_cast<const float4*>(p.qpart + (s * p.part_rows + row) * DP)[c];
        sum.x += v.x, sum.y += v.y, sum.z += v.z, sum.w += v.w;
    }
    const long bh = row / p.seq;
    const long b = bh / p.nh, head = bh % p.nh;
    float4* dst = reinterpret_cast<float4*>(p.dq + b * p.q_bs + (long)tq * p.nh * DP + head * DP) + c;
    float4 v = *dst;
    v.x += sum.x, v.y += sum.y, v.z += sum.z, v.w += sum.w;
    *dst = v;
}

// ------------------------------------------------------------- launchers
static bool f32_fast_ok(int hd) { return hd == 64 || hd == 128; }

static int f32_hpw(int group) { return group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1; }

// Waves below which the fp32 grids are split (the kernels run best at two or
// more waves per SIMD).
constexpr long kSplitWaves = 2048;

// Query splits of the dK/dV grid: the query tiles a key tile sees are cut
// into runs of at most qt_run, halved from the longest (key tile 0) until the
// grid gives two waves per SIMD, with at most 8 splits.
struct F32KvPlan {
    int qt_run, qs_max, units;
};
static F32KvPlan f32_kv_plan(const Dims& d) {
    const int n_qt = (d.seq + 31) / 32, n_kvt = (d.seq + 127) / 128;
    const long per = (long)d.nh * d.batch;
    F32KvPlan pl{n_qt, 1, n_kvt};
    for (int run = n_qt; run >= 1; run = (run + 1) / 2) {
        const int qs_max = (n_qt + run - 1) / run;
        if (qs_max > 8) break;
        int units = 0;
        for (int t = 0; t < n_kvt; t++) units += (n_qt - 4 * t + run - 1) / run;
        pl = F32KvPlan{run, qs_max, units};
        if (4L * units * per >= kSplitWaves || run == 1) break;
    }
    return pl;
}

static hipError_t f32_cus(int* cus) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return hipErrorInvalidDevice;
    return hipSuccess;
}

// Workgroups per XCD of the persistent dK/dV grid (two workgroups per CU at
// head_dim 64, one at 128), or 0 for one workgroup per unit: persistent
// when XCD-aware with a (sequence, head) group per XCD and units for every
// workgroup slot.
static hipError_t f32_kv_persistent(const Dims& d, int xcd, long units, int* wgs) {
    *wgs = 0;
    if (!xcd) return hipSuccess;
    int cus = 0;
    const hipError_t e = f32_cus(&cus);
    if (e != hipSuccess) return e;
    const int per_cu = d.hd == 64 ? 2 : 1;
    if (cus >= 8 && cus % 8 == 0 && (long)d.batch * d.nh >= 8 && units >= (long)cus * per_cu)
        *wgs = cus / 8 * per_cu;
    return hipSuccess;
}

// Grid of the forward and dQ kernels: hpw heads x tpw 32-query blocks per
// workgroup, and the key split.  A causal grid is as slow as its longest query
// tile, and at one wave per SIMD the kernels also wait on every load; when
// the grid gives fewer than two waves per SIMD (kSplitWaves on 256 CUs), the
// key tiles of a query tile are cut into runs of ks (halved from below the
// longest tile's count until the grid reaches that, not below 2), and a merge
// combines the runs.
struct F32Plan {
    int hpw, tpw, n_sub, n_ttiles;
    int ks, units, max_ns;  // ks == 0: no split, units == n_ttiles
};

static int f32_units(const Dims& d, int tt, int n_ttiles, int ks) {
    int u = 0;
    for (int t = 0; t < n_ttiles; t++) {
        const int n_kt = (std::min(d.seq, (t + 1) * tt) + 31) / 32;
        u += (n_kt + ks - 1) / ks;
    }
    return u;
}

static F32Plan f32_plan(const Dims& d, int group) {
    F32Plan pl{};
    pl.hpw = f32_hpw(group);
    pl.tpw = 4 / pl.hpw;
    pl.n_sub = group / pl.hpw;
    pl.n_ttiles = (d.seq + 32 * pl.tpw - 1) / (32 * pl.tpw);
    pl.ks = 0;
    pl.units = pl.n_ttiles;
    pl.max_ns = 1;
    const long per_unit = (long)d.nkv * pl.n_sub * d.batch;
    const int kt_max = (d.seq + 31) / 32;
    if (4L * pl.n_ttiles * per_unit >= kSplitWaves || kt_max <= 2) return pl;
    int ks = 1;
    while (2 * ks < kt_max) ks *= 2;
    for (; ks >= 2; ks /= 2) {
        pl.ks = ks;
        pl.units = f32_units(d, 32 * pl.tpw, pl.n_ttiles, ks);
        if (4L * pl.units * per_unit >= kSplitWaves) break;
    }
    pl.max_ns = (kt_max + pl.ks - 1) / pl.ks;
    return pl;
}

static size_t f32_rows(const Dims& d) { return (size_t)d.batch * d.nh * d.seq; }

// Walk order of the persistent forward / dQ grid: a query tile's work is its
// 32-key tiles.
static int f32_walk_order(const Dims& d, const F32Plan& pl, long items, int wgs) {
    const int tt = 32 * pl.tpw, seq = d.seq;
    return persistent_group_major((int)(items / pl.n_ttiles), pl.n_ttiles, wgs,
                                  [&](int t) { return (long)(std::min(seq, (t + 1) * tt) + 31) / 32; });
}

// Workgroups per XCD of the persistent forward / dQ grid, or 0 for one
// workgroup per unit: persistent when the grid is unsplit, XCD-aware, has a
// group per XCD and fills every workgroup slot (two per CU at head_dim 64,
// where two waves per SIMD fit, one at 128).
static int f32_persistent_wgs(const Dims& d, const F32Plan& pl, int xcd, long units, hipError_t* err) {
    *err = hipSuccess;
    if (pl.ks || !xcd) return 0;
    int cus = 0;
    if ((*err = f32_cus(&cus)) != hipSuccess) return 0;
    const int per_cu = d.hd == 64 ? 2 : 1;
    const long groups = (long)d.nkv * pl.n_sub * d.batch;
    if (cus < 8 || cus % 8 != 0 || groups < 8 || units < (long)cus * per_cu) return 0;
    return cus / 8 * per_cu;
}

size_t attn_f32_scratch_bytes(const Dims& d) {
    if (!f32_fast_ok(d.hd) || d.batch <= 0 || d.seq <= 0 || d.nkv <= 0) return 0;
    const size_t half = (size_t)d.batch * d.seq * d.nkv * d.hd;
    const size_t slots = (size_t)(d.nh / d.nkv) * f32_kv_plan(d).qs_max;
    const size_t dkdv = 2 * slots * half * sizeof(float);
    // The dQ split reuses the region once the dK/dV sum has read it.
    const F32Plan pl = f32_plan(d, d.nh / d.nkv);
    const size_t dq = pl.ks ? (size_t)pl.max_ns * f32_rows(d) * d.hd * sizeof(float) : 0;
    return std::max(dkdv, dq);
}

size_t attn_f32_fwd_scratch_bytes(const Dims& d) {
    if (!f32_fast_ok(d.hd) || d.batch <= 0 || d.seq <= 0 || d.nkv <= 0) return 0;
    const F32Plan pl = f32_plan(d, d.nh / d.nkv);
    if (!pl.ks) return 0;
    return (size_t)pl.max_ns * f32_rows(d) * (d.hd + 2) * sizeof(float);
}

bool attn_f32_fast_applies(const Dims& d, int vec_ok, int o_vec_ok) {
    return f32_fast_ok(d.hd) && vec_ok && o_vec_ok;
}

// `scratch` (attn_f32_fwd_scratch_bytes(d) bytes) holds the key splits'
// partial results; without it the grid runs unsplit.
hipError_t launch_attn_fwd_f32(const Dims& d, FwdParams p, void* scratch, size_t scratch_bytes, bool persistent,
                               hipStream_t st, KernelTimer* tm) {
    F32Plan pl = f32_plan(d, p.group);
    const size_t need = attn_f32_fwd_scratch_bytes(d);
    if (pl.ks && (scratch == nullptr || scratch_bytes < need)) pl.ks = 0, pl.units = pl.n_ttiles;
    p.hpw = pl.hpw;
    p.tpw = pl.tpw;
    p.n_sub = pl.n_sub;
    p.n_ttiles = pl.n_ttiles;
    p.ksplit = pl.ks;
    p.units = pl.units;
    p.part_rows = (long)f32_rows(d);
    p.part = pl.ks ? static_cast<float*>(scratch) : nullptr;
    p.part_ml = pl.ks ? reinterpret_cast<float2*>(p.part + (size_t)pl.max_ns * p.part_rows * d.hd) : nullptr;
    const long n_wg = (long)pl.units * d.nkv * p.n_sub * d.batch;
    if (n_wg > 0x7fffffffL) return hipErrorInvalidConfiguration;
    p.n_wg = (int)n_wg;
    hipError_t pe = hipSuccess;
    p.xcd_wgs = persistent ? f32_persistent_wgs(d, pl, p.xcd, n_wg, &pe) : 0;
    if (pe != hipSuccess) return pe;
    p.n_items = p.n_wg;
    if (p.xcd_wgs > 0) {
        p.n_wg = 8 * p.xcd_wgs;
        p.walk_gm = f32_walk_order(d, pl, p.n_items, p.xcd_wgs);
    }
    TimedLaunch tl(tm, kKernFwd, st);
    if (d.hd == 128)
        hipLaunchKernelGGL(attn_fwd_f32_kernel<128>, dim3(p.n_wg), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(attn_fwd_f32_kernel<64>, dim3(p.n_wg), dim3(256), 0, st, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !pl.ks) return e;
    const long threads = p.part_rows * (d.hd / 4);
    const unsigned grid = (unsigned)((threads + 255) / 256);
    if (d.hd == 128)
        hipLaunchKernelGGL(attn_f32_fwd_merge_kernel<128>, dim3(grid), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(attn_f32_fwd_merge_kernel<64>, dim3(grid), dim3(256), 0, st, p);
    return hipGetLastError();
}

// dK/dV then dQ (delta is already computed); `scratch` holds
// attn_f32_scratch_bytes(d) bytes.
size_t attn_f32_ds_bytes(const Dims& d) {
    if (!f32_fast_ok(d.hd) || d.batch <= 0 || d.seq <= 0 || d.nkv <= 0) return 0;
    const size_t nqb = ((size_t)d.seq + 31) / 32;
    return (size_t)d.batch * d.nh * (nqb * (nqb + 1) / 2) * 1024 * sizeof(float);
}

hipError_t launch_attn_bwd_f32(const Dims& d, BwdParams p, void* scratch, size_t scratch_bytes, bool persistent,
                               bool stored_ds, hipStream_t st, KernelTimer* tm) {
    F32DkdvArgs a;
    const F32KvPlan kp = f32_kv_plan(d);
    a.qs_n = kp.qs_max;
    a.qt_run = kp.qt_run;
    a.units = kp.units;
    a.part = static_cast<float*>(scratch);
    a.part_half = (long)d.batch * d.seq * d.nkv * d.hd;
    const int slots = p.group * a.qs_n;
    a.slots = slots;
    p.n_kvtiles = (d.seq + 127) / 128;
    // Stored dS when the scratch holds it past the slots.  Its dQ grid runs
    // unsplit: one product per key tile makes even the longest query tile of
    // a small grid short (the split, with its partials and merge, is for the
    // recompute's three).
    F32Plan pl = f32_plan(d, p.group);
    const size_t ds_off = (attn_f32_scratch_bytes(d) + 255) / 256 * 256, ds_need = attn_f32_ds_bytes(d);
    p.ds32 = nullptr;
    if (stored_ds && ds_need > 0 && scratch_bytes >= ds_off + ds_need) {
        p.ds32 = reinterpret_cast<float*>(static_cast<char*>(scratch) + ds_off);
        const long nqb = (d.seq + 31) / 32;
        p.ds_ntri = nqb * (nqb + 1) / 2;
        pl.ks = 0;
        pl.units = pl.n_ttiles;
    }
    const long nkv_wg = (long)kp.units * d.nh * d.batch;
    if (nkv_wg > 0x7fffffffL) return hipErrorInvalidConfiguration;
    p.n_wg_kv = (int)nkv_wg;
    hipError_t e = f32_kv_persistent(d, p.xcd && persistent, nkv_wg, &a.xcd_wgs);
    if (e != hipSuccess) return e;
    a.walk_gm = 0;
    if (a.xcd_wgs > 0) {
        p.n_wg_kv = 8 * a.xcd_wgs;
        // A unit's work is its steps (query tiles); units in key-tile
        // order, a key tile's splits consecutive (as dkdv_f32_unit decodes).
        const int n_qt = (d.seq + 31) / 32;
        std::vector<long> steps;
        for (int kvt = 0; kvt < p.n_kvtiles; kvt++) {
            const int qs_n = (n_qt - 4 * kvt + a.qt_run - 1) / a.qt_run;
            for (int qs = 0; qs < qs_n; qs++) {
                const int first = 4 * kvt + qs;
                steps.push_back(first < n_qt ? (n_qt - first + qs_n - 1) / qs_n : 0);
            }
        }
        if ((int)steps.size() == a.units)
            a.walk_gm = persistent_group_major(d.batch * d.nh, a.units, a.xcd_wgs,
                                               [&](int t) { return steps[a.units - 1 - t]; });
    }
    {
        TimedLaunch tl(tm, kKernBwdDkdv, st);
        if (d.hd == 128)
            hipLaunchKernelGGL(attn_bwd_dkdv_f32_kernel<128>, dim3(p.n_wg_kv), dim3(256), 0, st, p, a);
        else
            hipLaunchKernelGGL(attn_bwd_dkdv_f32_kernel<64>, dim3(p.n_wg_kv), dim3(256), 0, st, p, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        const long n4 = a.part_half / 4;
        hipLaunchKernelGGL(attn_f32_reduce_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, st, a.part, a,
                           d.seq, d.nkv * d.hd, p.group, p.dk, p.dv);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return e;
    p.hpw = pl.hpw;
    p.tpw = pl.tpw;
    p.n_sub = pl.n_sub;
    p.n_ttiles = pl.n_ttiles;
    p.ksplit = pl.ks;
    p.units_q = pl.units;
    p.part_rows = (long)f32_rows(d);
    p.qpart = pl.ks ? static_cast<float*>(scratch) : nullptr;  // read by the sum above, free now
    const long nq_wg = (long)pl.units * d.nkv * p.n_sub * d.batch;
    if (nq_wg > 0x7fffffffL) return hipErrorInvalidConfiguration;
    p.n_wg_q = (int)nq_wg;
    hipError_t pe = hipSuccess;
    p.q_xcd_wgs = persistent ? f32_persistent_wgs(d, pl, p.xcd, nq_wg, &pe) : 0;
    if (pe != hipSuccess) return pe;
    p.q_items = p.n_wg_q;
    if (p.q_xcd_wgs > 0) {
        p.n_wg_q = 8 * p.q_xcd_wgs;
        p.q_walk_gm = f32_walk_order(d, pl, p.q_items, p.q_xcd_wgs);
    }
    TimedLaunch tl(tm, kKernBwdDq, st);
    if (p.ds32 && d.hd == 128)
        hipLaunchKernelGGL(attn_bwd_dq_f32_ds_kernel<128>, dim3(p.n_wg_q), dim3(256), 0, st, p);
    else if (p.ds32)
        hipLaunchKernelGGL(attn_bwd_dq_f32_ds_kernel<64>, dim3(p.n_wg_q), dim3(256), 0, st, p);
    else if (d.hd == 128)
        hipLaunchKernelGGL(attn_bwd_dq_f32_kernel<128>, dim3(p.n_wg_q), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(attn_bwd_dq_f32_kernel<64>, dim3(p.n_wg_q), dim3(256), 0, st, p);
    e = hipGetLastError();
    if (e != hipSuccess || !pl.ks) return e;
    const long threads = p.part_rows * (d.hd / 4);
    const unsigned grid = (unsigned)((threads + 255) / 256);
    if (d.hd == 128)
        hipLaunchKernelGGL(attn_f32_dq_merge_kernel<128>, dim3(grid), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL(attn_f32_dq_merge_kernel<64>, dim3(grid), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace cfattn
