// Causal grouped-query attention forward on gfx950 MFMA.
//
// Computes, per query head h and token t (reference semantics:
// crates/core/src/ops/attention.rs:46-122):
//   O[t,h]   = sum_{j<=t} softmax_j(q_t . k_j / sqrt(D)) v_j   (overwritten)
//   lse[h,t] = max_j s_tj + ln sum_j exp(s_tj - max)            (overwritten)
// with KV head g = h / group serving `group` consecutive query heads.
//
// Work decomposition.  A workgroup owns one tile of TT = 32*tpw tokens and
// `hpw` query heads of one GQA group (hpw divides group).  Each wave owns 32
// tokens of one head.  K/V tiles of BN keys are staged once into LDS and
// shared by every head and token block of the workgroup.  Per wave and key
// tile:
//   S^T = K Q^T  (MFMA, K from LDS rows, Q held in registers)
//        -> each lane owns one query (column) and 16 keys of every 32-key
//           block, so the row max needs one exchange between lane halves;
//   online softmax in the exp2 domain (running max m, per-lane partial sum);
//   O^T += V^T P^T (MFMA, V^T read from a transposed LDS tile, P^T fed
//        straight from the S^T accumulators, rounded to bf16 in bf16 mode).
// Workgroups are ordered longest-first (most key tiles) and remapped so each
// XCD works through contiguous (sequence, KV head) ranges.
#include <algorithm>

#include "cfattn_common.hpp"
#include "attn_params.hpp"
#include "cfattn_kernels.hpp"

namespace cfattn {

template <typename T, int DP, int BN>
__global__ __launch_bounds__(256) void attn_fwd_kernel(const FwdParams p) {
    using M = Mode<T>;
    constexpr int EPL = M::EPL;
    constexpr int HALF = DP / 2;     // head-dim range of each lane half
    constexpr int NKD = HALF / EPL;  // MFMAs over the head dim per 32x32 block
    constexpr int NDB = DP / 32;     // 32-row head-dim blocks of O^T
    constexpr int NKB = BN / 32;     // 32-key blocks per key tile
    constexpr int LDK = RowLD<T, DP>::value;
    constexpr int LDV = TLD<T, BN>::value;
    __shared__ __attribute__((aligned(16))) T sK[BN * LDK];
    __shared__ __attribute__((aligned(16))) T sVt[DP * LDV];

    const int nthreads = blockDim.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int l32 = lane & 31, hh = lane >> 5;

    const int id = xcd_remap(blockIdx.x, p.n_wg, p.xcd);
    const int tile = p.n_ttiles - 1 - id % p.n_ttiles;  // longest tiles first
    int rest = id / p.n_ttiles;
    const int sub = rest % p.n_sub;
    rest /= p.n_sub;
    const int g = rest % p.nkv;
    const int b = rest / p.nkv;

    const int head = g * p.group + sub * p.hpw + wave % p.hpw;
    const int TT = 32 * p.tpw;
    const int t_wave = tile * TT + (wave / p.hpw) * 32;
    const int tq = t_wave + l32;
    const int wg_end = min(p.seq, tile * TT + TT);
    const int n_kt = (wg_end + BN - 1) / BN;
    const bool wave_active = t_wave < p.seq;
    const int wave_last = min(t_wave + 31, p.seq - 1);

    const long qrs = (long)p.nh * p.hd, kvrs = (long)p.nkv * p.hd;
    const T* qg = static_cast<const T*>(p.q) + (long)b * p.q_bs;
    const T* kg = static_cast<const T*>(p.k) + (long)b * p.kv_bs + (long)g * p.hd;
    const T* vg = static_cast<const T*>(p.v) + (long)b * p.kv_bs + (long)g * p.hd;

    // Q^T operand for this lane: query tq, head dims [hh*HALF, hh*HALF+HALF).
    T qraw[HALF];
    load_row_frag<T, HALF>(qraw, qg + (long)tq * qrs + (long)head * p.hd, hh * HALF, p.hd, tq < p.seq, p.vec_ok);
    typename M::frag qf[NKD];
#pragma unroll
    for (int kd = 0; kd < NKD; kd++) {
        if constexpr (EPL == 8) {
            Chunk<T> c;
#pragma unroll
            for (int i = 0; i < 8; i++) c.e[i] = qraw[kd * 8 + i];
            qf[kd] = __builtin_bit_cast(bf16x8, c.u);
        } else {
            qf[kd] = qraw[kd];
        }
    }

    f32x16 oacc[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) oacc[i] = zero16();
    float m2 = -INFINITY, lsum = 0.0f;

    for (int kt = 0; kt < n_kt; kt++) {
        const int k0 = kt * BN;
        const int nrows = min(BN, p.seq - k0);
        __syncthreads();
        stage_rows<T, BN, DP, LDK>(sK, kg + (long)k0 * kvrs, kvrs, nrows, p.hd, p.vec_ok, nthreads);
        stage_rows_t<T, BN, DP, LDV>(sVt, vg + (long)k0 * kvrs, kvrs, nrows, p.hd, p.vec_ok, nthreads);
        __syncthreads();
        if (!wave_active || k0 > wave_last) continue;

        // S^T blocks: rows = keys k0 + kb*32 + [0,32), columns = this wave's queries.
        f32x16 s[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            s[kb] = zero16();
            if (k0 + kb * 32 > wave_last) continue;
            const T* krow = sK + (kb * 32 + l32) * LDK + hh * HALF;
            if constexpr (EPL == 8) {
#pragma unroll
                for (int kd = 0; kd < NKD; kd++) s[kb] = mfma32(load_bf16x8(krow + kd * 8), qf[kd], s[kb]);
            } else {
#pragma unroll
                for (int kd = 0; kd < NKD; kd += 4) {
                    const float4 a = *reinterpret_cast<const float4*>(krow + kd);
                    s[kb] = mfma32(a.x, qf[kd + 0], s[kb]);
                    s[kb] = mfma32(a.y, qf[kd + 1], s[kb]);
                    s[kb] = mfma32(a.z, qf[kd + 2], s[kb]);
                    s[kb] = mfma32(a.w, qf[kd + 3], s[kb]);
                }
            }
        }

        // Scale into the exp2 domain, apply the causal mask, row max.
        const bool need_mask = k0 + BN - 1 > t_wave;
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float x = s[kb][r] * p.sl2;
                if (need_mask) {
                    const int key = k0 + kb * 32 + (r >> 2) * 8 + hh * 4 + (r & 3);
                    if (key > tq) x = -INFINITY;
                }
                s[kb][r] = x;
                mx = fmaxf(mx, x);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // Key 0 is in the first tile every wave processes, so m2 is finite
        // from the first tile on and alpha never sees inf - inf.
        const float mnew = fmaxf(m2, mx);
        const float alpha = exp2f(m2 - mnew);
        m2 = mnew;
        lsum *= alpha;
#pragma unroll
        for (int i = 0; i < NDB; i++) oacc[i] *= alpha;

#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const float e = exp2f(s[kb][r] - mnew);
                s[kb][r] = e;
                lsum += e;
            }
        }

        // O^T += V^T P^T.
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            if (k0 + kb * 32 > wave_last) continue;
            float pv[16];
#pragma unroll
            for (int r = 0; r < 16; r++) pv[r] = s[kb][r];
            if constexpr (EPL == 8) {
                const bf16x8 p0 = pack_bf16x8(&pv[0]);
                const bf16x8 p1 = pack_bf16x8(&pv[8]);
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    const T* vt = sVt + (db * 32 + l32) * LDV + kb * 32 + hh * 4;
                    oacc[db] = mfma32(load_bf16x4x2(vt, vt + 8), p0, oacc[db]);
                    oacc[db] = mfma32(load_bf16x4x2(vt + 16, vt + 24), p1, oacc[db]);
                }
            } else {
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    const T* vt = sVt + (db * 32 + l32) * LDV + kb * 32 + hh * 4;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float4 a = *reinterpret_cast<const float4*>(vt + j * 8);
                        oacc[db] = mfma32(a.x, pv[j * 4 + 0], oacc[db]);
                        oacc[db] = mfma32(a.y, pv[j * 4 + 1], oacc[db]);
                        oacc[db] = mfma32(a.z, pv[j * 4 + 2], oacc[db]);
                        oacc[db] = mfma32(a.w, pv[j * 4 + 3], oacc[db]);
                    }
                }
            }
        }
    }

    if (!wave_active) return;
    const float ltot = lsum + __shfl_xor(lsum, 32);
    if (tq >= p.seq) return;
    const float inv = 1.0f / ltot;
    float* orow = p.o + (long)b * p.q_bs + (long)tq * qrs + (long)head * p.hd;
#pragma unroll
    for (int db = 0; db < NDB; db++) {
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            const int d0 = db * 32 + rq * 8 + hh * 4;
            const float4 v = make_float4(oacc[db][rq * 4 + 0] * inv, oacc[db][rq * 4 + 1] * inv,
                                         oacc[db][rq * 4 + 2] * inv, oacc[db][rq * 4 + 3] * inv);
            if (p.o_vec_ok && d0 + 4 <= p.hd) {
                *reinterpret_cast<float4*>(orow + d0) = v;
            } else {
                if (d0 + 0 < p.hd) orow[d0 + 0] = v.x;
                if (d0 + 1 < p.hd) orow[d0 + 1] = v.y;
                if (d0 + 2 < p.hd) orow[d0 + 2] = v.z;
                if (d0 + 3 < p.hd) orow[d0 + 3] = v.w;
            }
        }
    }
    if (hh == 0) p.lse[((long)b * p.nh + head) * p.seq + tq] = (m2 + log2f(ltot)) * kLn2;
}

// ---------------------------------------------------------------------------
// Fast path: bf16 inputs, head_dim == DP (64 or 128), 16-byte aligned rows.
// NW waves per workgroup, the same (tile, heads) decomposition as above.
// K/V tiles of BN keys go straight from global memory into double-buffered
// blocked LDS tiles (global_load_lds, issued one tile ahead by all the
// waves), so each tile costs one barrier.  S^T = K Q^T reads K rows with
// ds_read_b128; O^T += V^T P^T reads V^T straight from the V tile with
// transposed reads (ds_read_b64_tr_b16).  MFMA row i of a 32-key block is key
// qperm(i) of the block (see BlkTile).  The running max is only moved when a
// tile's max exceeds it by more than kLazyRescale (log2 units): exp2 of the
// shifted scores then stays below 2^kLazyRescale, and O and the row sum are
// rescaled only on those tiles.  O = acc / sum and lse = m + log2(sum) do not
// depend on which shift was used.
constexpr float kLazyRescale = 8.0f;
// Waves per workgroup of the fast forward.  All of them share each K/V tile;
// four (two workgroups per CU) measured faster than eight (one).
constexpr int kFastWaves = 4;

// One query tile of hpw heads x tpw 32-query blocks: tile `tile` of group
// rest = (sequence * nkv + KV head) * n_sub + head subset.  Every wave passes
// the same barriers and no LDS read follows the last one, so the next tile of
// a persistent workgroup may load into the buffers.
template <int DP, int BN, int NW>
__device__ __forceinline__ void fwd_bf16_unit(const FwdParams& p, const int tile, int rest, bf16_bits* sK0,
                                              bf16_bits* sK1, bf16_bits* sV0, bf16_bits* sV1) {
    constexpr int CPR = DP / 8;  // 16-byte chunks per row
    using L = BlkTile<DP, BN>;
    constexpr int CPW = L::NB / NW;  // 1 KiB loads per wave per tile
    // Local copies: hipcc's host pass drops the kernel (an undefined launch
    // stub) when a lambda in it names these static members directly.
    constexpr int BSTRIDE = L::STRIDE, ROW16 = L::ROW16;
    static_assert(L::NB % NW == 0, "tile must split evenly over the waves");
    constexpr int HALF = DP / 2, NKD = HALF / 8, NDB = DP / 32, NKB = BN / 32;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hh = lane >> 5;

    const int sub = rest % p.n_sub;
    rest /= p.n_sub;
    const int g = rest % p.nkv;
    const int b = rest / p.nkv;

    const int head = g * p.group + sub * p.hpw + wave % p.hpw;
    const int TT = 32 * p.tpw;
    const int t_wave = tile * TT + (wave / p.hpw) * 32;
    const int tq = t_wave + l32;
    const int wg_end = min(p.seq, tile * TT + TT);
    const int n_kt = (wg_end + BN - 1) / BN;
    const bool wave_active = t_wave < p.seq;
    const int wave_last = min(t_wave + 31, p.seq - 1);

    const long qrs = (long)p.nh * DP, kvrs = (long)p.nkv * DP;
    const bf16_bits* kg = static_cast<const bf16_bits*>(p.k) + (long)b * p.kv_bs + (long)g * DP;
    const bf16_bits* vg = static_cast<const bf16_bits*>(p.v) + (long)b * p.kv_bs + (long)g * DP;

    // Q^T operand: query tq, head dims hh*HALF + kd*8 + [0, 8).
    bf16x8 qf[NKD];
    {
        const bf16_bits* qrow = static_cast<const bf16_bits*>(p.q) + (long)b * p.q_bs + (long)tq * qrs +
                                (long)head * DP + hh * HALF;
        const bool ok = tq < p.seq;
#pragma unroll
        for (int kd = 0; kd < NKD; kd++) {
            uint4 u = ok ? *reinterpret_cast<const uint4*>(qrow + kd * 8) : make_uint4(0, 0, 0, 0);
            qf[kd] = __builtin_bit_cast(bf16x8, u);
        }
    }

    // Row reads: lane (l32, hh) reads MFMA row l32 (key qperm(l32)), chunks
    // hh*NKD + kd.  Transposed reads: in each 16-lane group G, lane 4k + m
    // supplies head dims 16*(G%2) + 4m + [0, 4) of MFMA row 4*hh + k (+8,
    // +16, +24), that is tile row 4k + hh (+2, +16, +18).
    const int rrow = L::row(qperm(l32)) + hh * HALF;
    const int G = lane >> 4, jj = lane & 15;
    const int trow = L::row(4 * (jj >> 2) + hh) + 16 * (G & 1) + 4 * (jj & 3);

    // Tile kt's K and V rows: wave w fills load blocks w*CPW.., lane l of
    // block b loading chunk l % CPR of tile row b + NB*(l / CPR).  Keys past
    // the end load the last key (finite values); the causal mask removes them.
    // The per-lane part of each offset does not change from tile to tile (the
    // compiler keeps it out of the loop); a whole tile adds a scalar base.
    const int wv = wave_uniform(wave);
    constexpr int NBL = L::NB;
    const int lane_off = NBL * (lane / CPR) * (int)kvrs + (lane % CPR) * 8;
    // Full tiles: a scalar tile base plus the lane's byte offset within the
    // tile (the saddr form: no 64-bit address arithmetic per lane and load).
    const uint32_t lane_boff = (uint32_t)lane_off * 2u;
    auto dma = [&](int kt, bf16_bits* Kd, bf16_bits* Vd) {
        if ((kt + 1) * BN <= p.seq) {
            const long base = (long)kt * BN * kvrs;
#pragma unroll
            for (int i = 0; i < CPW; i++) {
                const int blk = wv * CPW + i;
                const uint32_t off = lane_boff + (uint32_t)(blk * kvrs) * 2u;
                lds_load16_sv(kg + base, off, Kd + blk * BSTRIDE);
                lds_load16_sv(vg + base, off, Vd + blk * BSTRIDE);
            }
        } else {
#pragma unroll
            for (int i = 0; i < CPW; i++) {
                const int blk = wv * CPW + i;
                const int r = blk + L::NB * (lane / CPR);
                const long off = (long)min(kt * BN + r, p.seq - 1) * kvrs + (lane % CPR) * 8;
                __builtin_amdgcn_global_load_lds(kg + off, Kd + blk * BSTRIDE, 16, 0, 0);
                __builtin_amdgcn_global_load_lds(vg + off, Vd + blk * BSTRIDE, 16, 0, 0);
            }
        }
    };

    f32x16 oacc[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) oacc[i] = zero16();
    float m2 = -INFINITY, lsum = 0.0f;

    auto step = [&](int kt, const bf16_bits* Ks, const bf16_bits* Vs, bf16_bits* Kn, bf16_bits* Vn) {
        // The next tile's loads are issued after this tile's score products:
        // issuing stalls the wave until the load queue takes them, and the
        // products then run meanwhile.
        const bool more = kt + 1 < n_kt;
        const int k0 = kt * BN;
        if (wave_active && k0 <= wave_last) {
            // S^T block kb: keys k0 + kb*32 + qperm([0,32)) x this wave's 32 queries.
            auto scores = [&](int kb) {
                f32x16 sc = zero16();
#pragma unroll
                for (int kd = 0; kd < NKD; kd++)
                    sc = mfma32(__builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(
                                                             Ks + rrow + kb * 2 * ROW16 + kd * 8)),
                                qf[kd], sc);
                return sc;
            };
            // Move the running max to m (log2 units) when the block max exceeds
            // it by more than kLazyRescale; rescale O and the row sum then.
            auto update_max = [&](float mx) {
                mx = max_halves(mx) * p.sl2;
                const float mnew = mx > m2 + kLazyRescale ? mx : m2;
                if (__any(mnew != m2)) {
                    const float alpha = __builtin_amdgcn_exp2f(m2 - mnew);
                    lsum *= alpha;
#pragma unroll
                    for (int i = 0; i < NDB; i++) oacc[i] *= alpha;
                    m2 = mnew;
                }
            };
            // P^T = exp2(S^T * scale*log2e - m), then O^T += V^T P^T over the
            // block's two 16-key halves (V^T read transposed from the V tile).
            auto accumulate = [&](int kb, const f32x16& sc) {
                float pr[16];
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    pr[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], p.sl2, -m2));
                    lsum += pr[r];
                }
                const bf16x8 p0 = cvt_bf16x8(&pr[0]), p1 = cvt_bf16x8(&pr[8]);
                const bf16_bits* t0 = Vs + trow + kb * 2 * ROW16;
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    const bf16_bits* tp = t0 + db * 32;
                    const bf16x8 a0 = join_bf16x4(ds_read_tr16(tp), ds_read_tr16(tp + 2 * BSTRIDE));
                    const bf16x8 a1 =
                        join_bf16x4(ds_read_tr16(tp + ROW16), ds_read_tr16(tp + ROW16 + 2 * BSTRIDE));
                    oacc[db] = mfma32(a0, p0, oacc[db]);
                    oacc[db] = mfma32(a1, p1, oacc[db]);
                }
            };
            if (k0 + BN - 1 <= t_wave) {
                // Interior tile: every key precedes every query of the wave.
                // All score blocks are issued first; each block's max is taken
                // on its own, so block kb's softmax runs while the products of
                // block kb+1 (scores) and of block kb-1 (O^T) are in flight.
                // The K row operands are read kLA MFMAs ahead of their product
                // (the order pinned: left to itself the compiler reads each
                // right before its MFMA and waits for it).
                f32x16 sc[NKB];
                {
                    constexpr int N = NKB * NKD, kLA = 4;
                    auto rd = [&](int j) {
                        return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(
                                                              Ks + rrow + (j % NKB) * 2 * ROW16 + (j / NKB) * 8));
                    };
                    bf16x8 kr[N];
#pragma unroll
                    for (int j = 0; j < kLA; j++) kr[j] = rd(j);
#pragma unroll
                    for (int j = 0; j < N; j++) {
                        if (j + kLA < N) kr[j + kLA] = rd(j + kLA);
                        const int kb = j % NKB, kd = j / NKB;
                        sc[kb] = mfma32(kr[j], qf[kd], kd == 0 ? zero16() : sc[kb]);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
                if (more) dma(kt + 1, Kn, Vn);
#pragma unroll
                for (int kb = 0; kb < NKB; kb++) {
                    float mx = -INFINITY;
#pragma unroll
                    for (int r = 0; r < 16; r++) mx = fmaxf(mx, sc[kb][r]);
                    update_max(mx);
                    accumulate(kb, sc[kb]);
                }
            } else {
                // Diagonal tile: causal mask, blocks past the wave's last query skipped.
                if (more) dma(kt + 1, Kn, Vn);
#pragma unroll
                for (int kb = 0; kb < NKB; kb++) {
                    const int kb0 = k0 + kb * 32;
                    if (kb0 > wave_last) break;
                    f32x16 sc = scores(kb);
                    if (kb0 + 31 > t_wave) {
#pragma unroll
                        for (int r = 0; r < 16; r++) {
                            const int key = kb0 + qperm((r >> 2) * 8 + hh * 4 + (r & 3));
                            if (key > tq) sc[r] = -INFINITY;
                        }
                    }
                    float mx = -INFINITY;
#pragma unroll
                    for (int r = 0; r < 16; r++) mx = fmaxf(mx, sc[r]);
                    // Keys 0..31 are unmasked for every row, so mx is finite on
                    // the first block and m2 from then on.
                    update_max(mx);
                    accumulate(kb, sc);
                }
            }
        } else if (more) {
            dma(kt + 1, Kn, Vn);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads for tile kt + 1 have landed
        __syncthreads();
    };

    dma(0, sK0, sV0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int kt = 0; kt < n_kt; kt += 2) {
        step(kt, sK0, sV0, sK1, sV1);
        if (kt + 1 < n_kt) step(kt + 1, sK1, sV1, sK0, sV0);
    }

    if (!wave_active) return;
    const float ltot = sum_halves(lsum);
    if (tq >= p.seq) return;
    const float inv = 1.0f / ltot;
    float* orow = p.o + (long)b * p.q_bs + (long)tq * qrs + (long)head * DP;
#pragma unroll
    for (int db = 0; db < NDB; db++) {
#pragma unroll
        for (int rq = 0; rq < 4; rq++) {
            const int d0 = db * 32 + rq * 8 + hh * 4;
            *reinterpret_cast<float4*>(orow + d0) =
                make_float4(oacc[db][rq * 4 + 0] * inv, oacc[db][rq * 4 + 1] * inv, oacc[db][rq * 4 + 2] * inv,
                            oacc[db][rq * 4 + 3] * inv);
        }
    }
    if (hh == 0) p.lse[((long)b * p.nh + head) * p.seq + tq] = (m2 + __log2f(ltot)) * kLn2;
}

template <int DP, int BN, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_fwd_bf16_kernel(
    const FwdParams p) {
    using L = BlkTile<DP, BN>;
    __shared__ __attribute__((aligned(16))) bf16_bits sK0[L::SIZE];
    __shared__ __attribute__((aligned(16))) bf16_bits sK1[L::SIZE];
    __shared__ __attribute__((aligned(16))) bf16_bits sV0[L::SIZE];
    __shared__ __attribute__((aligned(16))) bf16_bits sV1[L::SIZE];
    if (p.xcd_wgs > 0) {
        int tile, grp;
        for (int it = 0; persistent_item(it, p.n_items / p.n_ttiles, p.n_ttiles, p.xcd_wgs, p.walk_gm, tile, grp); it++)
            fwd_bf16_unit<DP, BN, NW>(p, tile, grp, sK0, sK1, sV0, sV1);
        return;
    }
    const int id = xcd_remap(blockIdx.x, p.n_wg, p.xcd);
    fwd_bf16_unit<DP, BN, NW>(p, p.n_ttiles - 1 - id % p.n_ttiles, id / p.n_ttiles, sK0, sK1, sV0, sV1);  // longest first
}

// Heads per workgroup: the largest divisor of `group` not above `cap`.
static int pick_hpw(int group, int cap) {
    for (int h = cap < group ? cap : group; h >= 1; h--)
        if (group % h == 0) return h;
    return 1;
}

template <typename T, int DP, int BN>
static hipError_t fwd_dispatch(const Dims& d, FwdParams p, hipStream_t st, int nwaves, KernelTimer* tm) {
    TimedLaunch tl(tm, kKernFwd, st);
    hipLaunchKernelGGL((attn_fwd_kernel<T, DP, BN>), dim3(p.n_wg), dim3(64 * nwaves), 0, st, p);
    return hipGetLastError();
}

template <typename T, int DP>
static hipError_t fwd_dp(const Dims& d, FwdParams p, hipStream_t st, int nwaves, KernelTimer* tm) {
    // fp32 tiles are twice the bytes: keep them to 32 keys.
    if constexpr (sizeof(T) == 2)
        return fwd_dispatch<T, DP, 64>(d, p, st, nwaves, tm);
    else
        return fwd_dispatch<T, DP, 32>(d, p, st, nwaves, tm);
}

size_t attn_fwd_scratch_bytes(Dtype dt, const Dims& d) { return dt == kF32 ? attn_f32_fwd_scratch_bytes(d) : 0; }

hipError_t launch_attn_fwd(Dtype dt, const Dims& d, const void* q, const void* k, const void* v, float* o,
                           float* lse, hipStream_t st, const Tuning& tu, void* scratch, size_t scratch_bytes) {
    if (d.batch == 0 || d.seq == 0 || d.nh == 0) return hipSuccess;
    FwdParams p{};
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    p.lse = lse;
    p.seq = d.seq;
    p.nh = d.nh;
    p.nkv = d.nkv;
    p.hd = d.hd;
    p.group = d.nh / d.nkv;
    p.hpw = tu.fwd_heads_per_wg > 0 ? pick_hpw(p.group, tu.fwd_heads_per_wg) : pick_hpw(p.group, 4);
    p.tpw = tu.fwd_tblocks_per_wg > 0 ? tu.fwd_tblocks_per_wg : (4 / p.hpw > 0 ? 4 / p.hpw : 1);
    if (p.hpw * p.tpw > 4) p.tpw = 4 / p.hpw > 0 ? 4 / p.hpw : 1;
    p.n_sub = p.group / p.hpw;
    p.n_ttiles = (d.seq + 32 * p.tpw - 1) / (32 * p.tpw);
    long n_wg = (long)p.n_ttiles * d.nkv * p.n_sub * d.batch;
    if (n_wg > 0x7fffffffL) return hipErrorInvalidConfiguration;
    p.n_wg = (int)n_wg;
    const float scale = 1.0f / sqrtf((float)d.hd);  // attention.rs:62
    p.sl2 = scale * kLog2e;
    p.q_bs = (long)d.seq * d.nh * d.hd;
    p.kv_bs = (long)d.seq * d.nkv * d.hd;
    const int ch = dt == kBF16 ? 8 : 4;
    const size_t al = 16;
    p.vec_ok = (d.hd % ch == 0) && ((uintptr_t)q % al == 0) && ((uintptr_t)k % al == 0) && ((uintptr_t)v % al == 0);
    p.o_vec_ok = (d.hd % 4 == 0) && ((uintptr_t)o % al == 0);
    p.xcd = tu.xcd_remap;
    if (dt == kBF16 && tu.fwd_variant == kFwdAuto && attn_fwd_q64_applies(d, p.vec_ok, p.o_vec_ok) &&
        tu.fwd_heads_per_wg == 0 && tu.fwd_tblocks_per_wg == 0) {
        p.settles = tu.fwd_settles;
        return launch_attn_fwd_q64(d, p, st, tu.timer);
    }
    if (dt == kBF16 && p.vec_ok && p.o_vec_ok && (d.hd == 64 || d.hd == 128) && tu.fwd_heads_per_wg == 0 &&
        tu.fwd_tblocks_per_wg == 0) {
        // Fast path: kFastWaves waves per workgroup, heads per workgroup in
        // {4, 2, 1}, the rest of the waves on further 32-query blocks.
        p.hpw = p.group % 4 == 0 ? 4 : p.group % 2 == 0 ? 2 : 1;
        p.tpw = kFastWaves / p.hpw;
        p.n_sub = p.group / p.hpw;
        p.n_ttiles = (d.seq + 32 * p.tpw - 1) / (32 * p.tpw);
        n_wg = (long)p.n_ttiles * d.nkv * p.n_sub * d.batch;
        if (n_wg > 0x7fffffffL) return hipErrorInvalidConfiguration;
        p.n_wg = (int)n_wg;
        // Persistent grid (two workgroups per CU) when the tiles fill every
        // workgroup slot with a group per XCD, up to four tiles per slot;
        // else one workgroup per tile.  (With few tiles per slot the in-
        // order dispatch leaves CUs idle: C2's grid, 2.25 tiles per slot, runs
        // 16% faster persistent; with many the idle share is small and the
        // persistent grid measured slower: C3's, 8 per slot, 7%.)
        p.n_items = p.n_wg;
        p.xcd_wgs = 0;
        if (tu.bf16_persistent && p.xcd) {
            int dev = 0, cus = 0;
            if (hipGetDevice(&dev) != hipSuccess ||
                hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
                return hipErrorInvalidDevice;
            if (cus >= 8 && cus % 8 == 0 && (long)d.nkv * p.n_sub * d.batch >= 8 && n_wg >= 2L * cus &&
                n_wg <= 8L * cus) {
                p.xcd_wgs = cus / 8 * 2;
                p.n_wg = 8 * p.xcd_wgs;
                const int bn = d.hd == 128 ? 64 : 128, tt = 32 * p.tpw, seq = d.seq;
                p.walk_gm = persistent_group_major(p.n_items / p.n_ttiles, p.n_ttiles, p.xcd_wgs,
                                                   [&](int t) { return (long)(std::min(seq, (t + 1) * tt) + bn - 1) / bn; });
            }
        }
        TimedLaunch tl(tu.timer, kKernFwd, st);
        if (d.hd == 128)
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<128, 64, kFastWaves>), dim3(p.n_wg), dim3(64 * kFastWaves), 0, st,
                               p);
        else
            hipLaunchKernelGGL((attn_fwd_bf16_kernel<64, 128, kFastWaves>), dim3(p.n_wg), dim3(64 * kFastWaves), 0, st,
                               p);
        return hipGetLastError();
    }
    if (dt == kF32 && attn_f32_fast_applies(d, p.vec_ok, p.o_vec_ok) && tu.fwd_heads_per_wg == 0 &&
        tu.fwd_tblocks_per_wg == 0)
        return launch_attn_fwd_f32(d, p, scratch, scratch_bytes, tu.f32_persistent != 0, st, tu.timer);
    const int nwaves = p.hpw * p.tpw;
    const int dp = d.hd <= 32 ? 32 : d.hd <= 64 ? 64 : d.hd <= 128 ? 128 : 256;
    if (dt == kBF16) {
        switch (dp) {
            case 32: return fwd_dp<bf16_bits, 32>(d, p, st, nwaves, tu.timer);
            case 64: return fwd_dp<bf16_bits, 64>(d, p, st, nwaves, tu.timer);
            case 128: return fwd_dp<bf16_bits, 128>(d, p, st, nwaves, tu.timer);
            default: return fwd_dp<bf16_bits, 256>(d, p, st, nwaves, tu.timer);
        }
    }
    switch (dp) {
        case 32: return fwd_dp<float, 32>(d, p, st, nwaves, tu.timer);
        case 64: return fwd_dp<float, 64>(d, p, st, nwaves, tu.timer);
        case 128: return fwd_dp<float, 128>(d, p, st, nwaves, tu.timer);
        default: return fwd_dp<float, 256>(d, p, st, nwaves, tu.timer);
    }
}

}  // namespace cfattn
