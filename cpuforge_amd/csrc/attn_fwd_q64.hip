// Causal GQA attention forward on gfx950: bf16 inputs at head_dim 128, fp32
// accumulation, one wave per SIMD.
//
// Reference semantics (crates/core/src/ops/attention.rs:46-122): per query
// head h and token t,
//   O[t,h]   = sum_{j<=t} softmax_j(q_t . k_j / sqrt(D)) v_j   (overwritten)
//   lse[h,t] = max_j s_tj + ln sum_j exp(s_tj - max)            (overwritten)
// with KV head g = h / group serving `group` consecutive query heads.
//
// A workgroup is four waves, one per SIMD; each wave owns 64 queries (two
// 32-query blocks, A and B) of one head, and the workgroup hpw heads x
// 4 / hpw such query tiles of one GQA group.  K and V tiles of 64 keys are
// loaded once into LDS for the four waves.  Holding 64 queries, a wave
// uses every K or V operand it reads from LDS for two MFMAs (one per query
// block) -- half the LDS bytes per product of the two-waves-per-SIMD kernel
// (attn_fwd_bf16_kernel), whose register budget holds 32 queries per wave.
// Per key tile, per wave:
//   S^T = K Q^T   (32 MFMAs, Q^T of both blocks held in registers),
//   online softmax in the exp2 domain (running max m per query, moved
//   lazily: only when a tile's max exceeds it by more than kLazyRescaleQ,
//   which keeps every P below 2^64; P is formed against m first and the
//   tile's row sums tell whether its max could have moved), P^T rounded to
//   bf16,
//   O^T += V^T P^T (32 MFMAs, O^T in AGPRs, V^T read transposed).
//
// Interval t (between barriers t - 1 and t) runs two regions of 32 MFMAs:
//   X  S of tile t (both blocks)        | P of tile t - 1, block B; then
//                                         tile t - 1's row-sum guard
//   Y  O += V^T P^T of tile t - 1       | P of tile t, block A
// so that the softmax of one tile issues in the shadow of the products of
// the next (one wave hides only about five other instructions per
// 32x32x16 MFMA).  Tile t's K is read in X(t) (its first operands at the
// end of Y(t - 1)), its V in Y(t + 1): X(t) issues the loads of K(t + 2)
// (three K buffers) and Y(t), in its first slots, those of V(t) (two V
// buffers), into buffers whose last readers passed barrier t - 1.  The key tile on the wave's diagonal is the last one
// it computes (its scores masked where the key follows the query); tiles
// past it are only loaded, for the workgroup's other waves.
#include "cfattn_common.hpp"
#include "attn_params.hpp"
#include "cfattn_kernels.hpp"
#include "mfma_asm.hpp"

namespace cfattn {

// The running max moves only when a tile's max exceeds it by more than this
// (log2 units), so P <= 2^64.  The softmax is scale-invariant and bf16 P,
// the fp32 row sums and the fp32 O^T accumulators (in AGPRs) have the fp32
// exponent range: with |V| up to 2^13 and 2^13 keys the largest term is
// 2^90, far below 2^128.  With this bound the first tile of a row sets m
// and later tiles move it only when their scores grow by more than 64
// log2 units; a smaller bound makes rows whose scores keep growing along
// the sequence (late keys larger than early ones) move m, and trip the
// row-sum guard below, on most of their tiles.
constexpr float kLazyRescaleQ = 64.0f;

__device__ __forceinline__ void q64_item(const FwdParams& p, const int id, bf16_bits* sK, bf16_bits* sV);

__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void attn_fwd_q64_kernel(
    const FwdParams p) {
    constexpr int TSZ = BlkTile<128, 64>::SIZE;
    __shared__ __attribute__((aligned(16))) bf16_bits sK[3 * TSZ];
    __shared__ __attribute__((aligned(16))) bf16_bits sV[2 * TSZ];

    // Items (query tiles) of this workgroup.  Persistent grid: the XCD of
    // workgroup w (w % 8; the dispatcher deals workgroups round robin)
    // takes a contiguous run of the items, so that its L2 holds few KV
    // heads, and its xcd_wgs workgroups walk the run zig-zag (positions l,
    // 2W - 1 - l, 2W + l, ...): with the items of a run longest first this
    // gives every workgroup nearly the same number of key tiles.
    const int xq = blockIdx.x % 8, xl = blockIdx.x / 8;
    int run0 = 0, run_n = 1;
    if (p.xcd_wgs > 0) {
        const int q = p.n_items / 8, r = p.n_items % 8;
        run0 = xq < r ? xq * (q + 1) : r * (q + 1) + (xq - r) * q;
        run_n = q + (xq < r ? 1 : 0);
    }
    for (int it = 0;; it++) {
        int id;
        if (p.xcd_wgs > 0) {
            const int W = p.xcd_wgs;
            const int pos = (it >> 1) * 2 * W + ((it & 1) ? 2 * W - 1 - xl : xl);
            if (pos >= run_n) break;
            id = run0 + pos;
        } else {
            if (it > 0) break;
            id = xcd_remap(blockIdx.x, p.n_wg, p.xcd);
        }
        q64_item(p, id, sK, sV);
    }
}

// One item: a query tile of hpw heads x 4 / hpw 64-query blocks of one GQA
// group.  Every wave of the workgroup passes the same number of barriers;
// after the last one no wave reads the K/V tiles, so the next item may
// load into them.
__device__ __forceinline__ void q64_item(const FwdParams& p, const int id, bf16_bits* sK, bf16_bits* sV) {
    constexpr int DP = 128, BN = 64, BQ = 64;
    constexpr int CPR = DP / 8;  // 16-byte chunks per row
    using L = BlkTile<DP, BN>;
    constexpr int NBL = L::NB;  // 1 KiB load blocks per tile
    constexpr int BSTRIDE = L::STRIDE, ROW16 = L::ROW16, TSZ = L::SIZE;
    constexpr int BPW = NBL / 4;  // blocks of each tile one wave loads
    constexpr int HALF = DP / 2, NKD = HALF / 8, NDB = DP / 32;
    // K row / V^T operands are read this many operands ahead of their MFMAs.
    constexpr int LA = 3;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = wave_uniform(tid >> 6);
    const int l32 = lane & 31, hh = lane >> 5;

    const int tile = p.n_ttiles - 1 - id % p.n_ttiles;  // longest tiles first
    int rest = id / p.n_ttiles;
    const int sub = rest % p.n_sub;
    rest /= p.n_sub;
    const int g = rest % p.nkv;
    const int b = rest / p.nkv;
    const int head = g * p.group + sub * p.hpw + wv % p.hpw;
    const int TT = BQ * p.tpw;
    const int t0 = tile * TT + (wv / p.hpw) * BQ;  // the wave's first query
    const int wg_end = min(p.seq, tile * TT + TT);
    const int n_kt = (wg_end + BN - 1) / BN;  // key tiles the workgroup loads
    const bool active = t0 < p.seq;
    const int dt = t0 / BN;  // the wave's diagonal tile; tiles before it are full

    const long qrs = (long)p.nh * DP, kvrs = (long)p.nkv * DP;
    const char* kgb = reinterpret_cast<const char*>(static_cast<const bf16_bits*>(p.k) + (long)b * p.kv_bs + (long)g * DP);
    const char* vgb = reinterpret_cast<const char*>(static_cast<const bf16_bits*>(p.v) + (long)b * p.kv_bs + (long)g * DP);

    // Q^T operands: query t0 + 32*qb + l32, head dims hh*HALF + kd*8 + [0, 8);
    // queries past the end are zero (their results are not stored).
    bf16x8 qf[2][NKD];
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        const int tq = t0 + qb * 32 + l32;
        const bf16_bits* qrow =
            static_cast<const bf16_bits*>(p.q) + (long)b * p.q_bs + (long)tq * qrs + (long)head * DP + hh * HALF;
#pragma unroll
        for (int kd = 0; kd < NKD; kd++) {
            const uint4 u = tq < p.seq ? *reinterpret_cast<const uint4*>(qrow + kd * 8) : make_uint4(0, 0, 0, 0);
            qf[qb][kd] = __builtin_bit_cast(bf16x8, u);
        }
    }
    // (The first barrier waits for these loads and K(0), K(1)'s together.)

    // Tile loads: wave w fills blocks w*BPW.. of a K and a V tile, lane l of
    // block bk reading chunk l % CPR of tile row bk + NB*(l / CPR), through a
    // bounds-checked buffer that starts at the tile and ends with the
    // sequence (keys past the end read zeros; the mask removes them).
    uint32_t tile_off[BPW];
#pragma unroll
    for (int i = 0; i < BPW; i++)
        tile_off[i] = (uint32_t)(((NBL * (lane / CPR) + wv * BPW + i) * (int)kvrs + (lane % CPR) * 8) * 2);
    const uint32_t kv_row = (uint32_t)kvrs * 2u;  // bytes per key row
    const uint32_t sk0 = lds_offset(sK) + (uint32_t)(wv * BPW * BSTRIDE * 2);
    const uint32_t sv0 = lds_offset(sV) + (uint32_t)(wv * BPW * BSTRIDE * 2);
    auto tile_rsrc = [&](const char* base, int kt) {
        return buf_rsrc(base + (uint32_t)(kt * BN) * kv_row, (uint32_t)(p.seq - kt * BN) * kv_row);
    };
    // K tile kt lives in buffer kt % 3 (loaded two intervals ahead, so that
    // Y(t) can read X(t + 1)'s first operands), V tile kt in buffer kt % 2.
    auto k_dst = [&](int kt) { return sk0 + (uint32_t)((kt % 3) * TSZ * 2); };
    auto v_dst = [&](int kt) { return sv0 + (uint32_t)((kt & 1) * TSZ * 2); };
    // Load i (< 2 * BPW) of interval t: K(t + 2) blocks to kdst, then V(t)
    // blocks to vdst.
    auto issue_load = [&](int i, const BufRsrc& rk, const BufRsrc& rv, uint32_t kdst, uint32_t vdst) {
        if (i < BPW)
            lds_buf_load16(rk, tile_off[i], kdst + (uint32_t)(i * BSTRIDE * 2));
        else
            lds_buf_load16(rv, tile_off[i - BPW], vdst + (uint32_t)((i - BPW) * BSTRIDE * 2));
    };
    // Interval t's loads, all at once (intervals outside the pipelined run).
    auto issue_all = [&](int t) {
        if (t + 2 < n_kt) {
            const BufRsrc rk = tile_rsrc(kgb, t + 2);
#pragma unroll
            for (int i = 0; i < BPW; i++) issue_load(i, rk, rk, k_dst(t + 2), 0);
        }
        if (t < n_kt) {
            const BufRsrc rv = tile_rsrc(vgb, t);
#pragma unroll
            for (int i = BPW; i < 2 * BPW; i++) issue_load(i, rv, rv, 0, v_dst(t));
        }
    };
    auto barrier = [&]() {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    // Row reads (K): lane (l32, hh) reads MFMA row l32 (key qperm(l32)),
    // chunks hh*NKD + kd.  Transposed reads (V^T): in each 16-lane group G,
    // lane 4k + m supplies head dims 16*(G%2) + 4m + [0, 4) of MFMA row
    // 4*hh + k (+8, +16, +24), that is tile row 4k + hh (+2, +16, +18).
    const int rrow = L::row(qperm(l32)) + hh * HALF;
    const int G = lane >> 4, jj = lane & 15;
    const int trow = L::row(4 * (jj >> 2) + hh) + 16 * (G & 1) + 4 * (jj & 3);
    // K operand o (kd = o / 2, key block kb = o % 2) of the K tile at Ks.
    auto rd_k = [&](const bf16_bits* Ks, int o) {
        return __builtin_bit_cast(bf16x8,
                                  *reinterpret_cast<const uint4*>(Ks + rrow + (o & 1) * 2 * ROW16 + (o >> 1) * 8));
    };
    // V^T operand o (key block kb = o / 8, 16-key half h = (o / 4) % 2,
    // head-dim block db = o % 4) of the V tile at Vs: each P^T operand
    // (kb, h) is used by four consecutive operands, so it is free as soon
    // as the next tile's replaces it.
    auto rd_v = [&](const bf16_bits* Vs, int o) {
        const bf16_bits* t = Vs + trow + (o >> 3) * 2 * ROW16 + (o & 3) * 32 + ((o >> 2) & 1) * ROW16;
        return join_bf16x4(ds_read_tr16(t), ds_read_tr16(t + 2 * BSTRIDE));
    };

    f32x16 oacc[2][NDB];  // O^T of blocks A and B, in AGPRs
#pragma unroll
    for (int qb = 0; qb < 2; qb++)
#pragma unroll
        for (int db = 0; db < NDB; db++) {
            oacc[qb][db] = zero16();
            agpr_pin(oacc[qb][db]);
        }
    auto acc_ready = [&]() {
        acc_ready8(oacc[0][0], oacc[0][1], oacc[0][2], oacc[0][3], oacc[1][0], oacc[1][1], oacc[1][2], oacc[1][3]);
    };
    auto acc_wait = [&]() {
        acc_wait8(oacc[0][0], oacc[0][1], oacc[0][2], oacc[0][3], oacc[1][0], oacc[1][1], oacc[1][2], oacc[1][3]);
    };
    float m2[2] = {-INFINITY, -INFINITY}, lsum[2] = {0.0f, 0.0f};
    float lpre[2];  // the row sums before the current tile's P was added

    // Scores of a tile kt, [qb][kb]: keys kt*BN + kb*32 + qperm(MFMA row) x
    // the block's 32 queries (lanes); two sets, for even and odd tiles (X
    // forms one while block B of the other is still turned into P).  The
    // diagonal tile masks keys after the query (element r: MFMA row
    // (r/4)*8 + hh*4 + r%4).
    f32x16 s0[2][2], s1[2][2];
    bf16x8 pA[2][2], pB[2][2];  // P^T operands [kb][half] of the previous tile
    auto mask_diag = [&](f32x16 (&sc)[2][2]) {
#pragma unroll
        for (int qb = 0; qb < 2; qb++)
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int key = kb * 32 + qperm((r >> 2) * 8 + hh * 4 + (r & 3));
                    if (key > qb * 32 + l32) sc[qb][kb][r] = -INFINITY;
                }
    };
    // P of a tile is formed against the running max m as it stands, with no
    // row max first: the lazy rule moves m only when the tile's max exceeds
    // it by more than kLazyRescaleQ, and while it does not, every P is at
    // most 2^kLazyRescaleQ.  An element above that bound makes its lane's
    // share of the tile's row sum (32 elements) exceed kGuard =
    // 2^kLazyRescaleQ, so once the tile's P is summed, a lane whose share
    // exceeds kGuard (or is not a number: the first tile, against m = -inf)
    // sends the wave to `settle`, which takes the exact row max, applies the
    // lazy rule and forms the tile's P again; a share above kGuard with no
    // element above the bound settles to no change of m.  m moves exactly
    // when the lazy rule says, so O, lse and every P are the same as with
    // the max taken first.
    constexpr float kGuard = 18446744073709551616.0f;  // 2^64 = 2^kLazyRescaleQ
    static_assert(kLazyRescaleQ == 64.0f, "kGuard is 2^kLazyRescaleQ");
    // P of element e of block qb's 32 (key block e / 16, element e % 16 of
    // the score block) into the block's staging; the bf16 operands of the
    // eight elements of group g and their sum into the row sum (two per
    // v_dot2 with (1, 1), in element order: O is normalised by the sum of
    // exactly the weights in its numerator) follow in `p_group`, a slot or
    // more after the last of them.
    float prA[16], prB[16];
    const bf16x2 ones2 = {(__bf16)1.0f, (__bf16)1.0f};
    auto p_elem = [&](const f32x16 (&sc)[2][2], int qb, int e) {
        float* pr = qb == 0 ? prA : prB;
        pr[e & 15] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[qb][e >> 4][e & 15], p.sl2, -m2[qb]));
    };
    auto p_group = [&](int qb, int g, bf16x8 (&pq)[2][2]) {
        const float* pr = qb == 0 ? prA : prB;
        const bf16x8 v = cvt_bf16x8(&pr[(g & 1) * 8]);
        pq[g >> 1][g & 1] = v;
        float l = lsum[qb];
#pragma unroll
        for (int i = 0; i < 4; i++) l = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{v[2 * i], v[2 * i + 1]}, ones2, l, false);
        lsum[qb] = l;
    };
    // The slow path of the guard for tile scores sp (unscheduled; the first
    // tile of every row takes it): per block, the exact row max, the lazy
    // rule, the row sum restarted from lpre and, if m moved anywhere in the
    // wave, O^T rescaled and the block's P formed again.
    auto settle = [&](const f32x16 (&sp)[2][2]) {
        if (p.settles != nullptr && lane == 0) atomicAdd(p.settles, 1u);
        acc_wait();
#pragma unroll
        for (int qb = 0; qb < 2; qb++) {
            float mx = -INFINITY;
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int r = 0; r < 16; r++) mx = fmaxf(mx, sp[qb][kb][r]);
            mx = max_halves(mx) * p.sl2;
            const float mnew = mx > m2[qb] + kLazyRescaleQ ? mx : m2[qb];
            const float a = __builtin_amdgcn_exp2f(m2[qb] - mnew);
            if (__any(mnew != m2[qb])) {
                m2[qb] = mnew;
                lsum[qb] = lpre[qb] * a;
#pragma unroll
                for (int g = 0; g < 4; g++) {
#pragma unroll
                    for (int e = 0; e < 8; e++) p_elem(sp, qb, g * 8 + e);
                    if (qb == 0)
                        p_group(0, g, pA);
                    else
                        p_group(1, g, pB);
                }
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    oacc[qb][db] *= a;
                    agpr_pin(oacc[qb][db]);
                }
            }
        }
    };
    // The guard, once the tile's P of both blocks is summed: whether this
    // lane's share of either block's tile sum exceeds kGuard (or is not a
    // number).
    auto guard_test = [&]() {
        const float da = lsum[0] - lpre[0], db = lsum[1] - lpre[1];
        return !(da <= kGuard) || !(db <= kGuard);
    };
    auto guard = [&](const f32x16 (&sp)[2][2]) {
        if (__any(guard_test())) settle(sp);
    };
    bool trip = false;

    // X(t): S of tile t into sc in 32 slots (K operand o = j / 2 for blocks
    // A, B); P of block B of tile t - 1 (scores sp), one element per slot,
    // each group's operand a slot after its last element; interval t's K
    // loads (K(t + 2) to kdst) in the odd slots of the first quarter.
    bf16x8 kr[NKD * 2];  // K operands of the current X
    auto region_x = [&](auto prev_tag, const bf16_bits* Ks, uint32_t kdst, const BufRsrc& rk, f32x16 (&sc)[2][2],
                        const f32x16 (&sp)[2][2]) {
        constexpr bool PREV = decltype(prev_tag)::value;
        // After interval 0 the previous Y read the first operands.
        if (!PREV) {
#pragma unroll
            for (int o = 0; o < LA; o++) kr[o] = rd_k(Ks, o);
        }
        if (PREV) lpre[1] = lsum[1];
        CF_FENCE();
#pragma unroll
        for (int j = 0; j < 4 * NKD; j++) {
            const int o = j >> 1, qb = j & 1, kd = o >> 1, kb = o & 1;
            // The MFMA first, then the slot's other work in its shadow.
            sc[qb][kb] = mfma32(kr[o], qf[qb][kd], kd == 0 ? zero16() : sc[qb][kb]);
            CF_FENCE();
            if (qb == 0 && o + LA < 2 * NKD) kr[o + LA] = rd_k(Ks, o + LA);
            if (PREV) {
                // Elements 0-23 one per slot, 24-31 two per slot in 24-27;
                // the last group's operand in slot 28 and the guard's test
                // in slot 30, so that its branch waits for nothing.
                if (j > 0 && (j & 7) == 0 && j <= 24) p_group(1, (j >> 3) - 1, pB);
                if (j < 24) {
                    p_elem(sp, 1, j);
                } else if (j < 28) {
                    p_elem(sp, 1, 24 + 2 * (j - 24));
                    p_elem(sp, 1, 25 + 2 * (j - 24));
                }
                if (j == 28) p_group(1, 3, pB);
                if (j == 30) trip = guard_test();
            }
            if ((j & 1) && j < 2 * BPW) issue_load(j >> 1, rk, rk, kdst, 0);
            CF_FENCE();
        }
        if (PREV && __any(trip)) settle(sp);
    };
    // Y(t): O^T += V^T P^T of tile t - 1 (V operand o = j / 2 for blocks
    // A, B); P of block A of tile t (scores sc), one element per slot, each
    // group's operand once the products have read the previous tile's.
    // With tile t's P (NEXT) the last slots also read the first K operands
    // of X(t + 1) from Kn (K(t + 1) is complete since barrier t - 1).
    auto region_y = [&](auto prev_tag, auto next_tag, const bf16_bits* Vs, const bf16_bits* Kn, int tv,
                        const f32x16 (&sc)[2][2]) {
        constexpr bool PREV = decltype(prev_tag)::value, NEXT = decltype(next_tag)::value;
        // The interval's V loads (V(tv)), early in Y: they land before the
        // barrier like X's K loads.
        const BufRsrc rvy = tile_rsrc(vgb, tv);
        bf16x8 vt[4 * NDB];
        if (PREV) {
#pragma unroll
            for (int o = 0; o < LA; o++) vt[o] = rd_v(Vs, o);
            acc_ready();
        }
        if (NEXT) lpre[0] = lsum[0];
        CF_HAZARD_FENCE();
#pragma unroll
        for (int j = 0; j < 8 * NDB; j++) {
            const int o = j >> 1, qb = j & 1, kb = o >> 3, h = (o >> 2) & 1, db = o & 3;
            if (PREV) {
                mfma_acc(oacc[qb][db], vt[o], qb == 0 ? pA[kb][h] : pB[kb][h]);
                CF_FENCE();
                if (qb == 0 && o + LA < 4 * NDB) vt[o + LA] = rd_v(Vs, o + LA);
            }
            if (NEXT) {
                // Group g of block A replaces operand pA[g / 2][g % 2], last
                // read by the product in slot 8g + 6.
                if (j > 0 && (j & 7) == 0) p_group(0, (j >> 3) - 1, pA);
                p_elem(sc, 0, j);
                if (j >= 32 - 2 * LA && (j & 1) == 0) kr[(j - (32 - 2 * LA)) >> 1] = rd_k(Kn, (j - (32 - 2 * LA)) >> 1);
                if ((j & 1) && j < 2 * BPW) issue_load(BPW + (j >> 1), rvy, rvy, 0, v_dst(tv));
            }
            CF_FENCE();
        }
        if (NEXT) p_group(0, 3, pA);
    };
    // Interval t (1 <= t <= dt): S(t) into sc with P of block B of tile
    // t - 1 (scores sp) and the guard of tile t - 1, then the products of
    // tile t - 1 with block A's P of tile t.
    auto interval = [&](int t, f32x16 (&sc)[2][2], const f32x16 (&sp)[2][2]) {
        const bf16_bits* Ks = sK + (t % 3) * TSZ;
        const bf16_bits* Vs = sV + ((t - 1) & 1) * TSZ;
        // Past the last tile the K loads reload tile n_kt - 1 into the free
        // buffer (no X reads it).
        const BufRsrc rk = tile_rsrc(kgb, t + 2 < n_kt ? t + 2 : n_kt - 1);
        region_x(std::true_type{}, Ks, k_dst(t + 2), rk, sc, sp);
        if (t == dt) mask_diag(sc);
        region_y(std::true_type{}, std::true_type{}, Vs, sK + ((t + 1) % 3) * TSZ, t, sc);
        barrier();
    };

    // ---------------------------------------------------------------- walk
    // Intervals 0 and 1 need K(0) and K(1).
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
        const BufRsrc rk = tile_rsrc(kgb, kt < n_kt ? kt : 0);
#pragma unroll
        for (int i = 0; i < BPW; i++) lds_buf_load16(rk, tile_off[i], k_dst(kt) + (uint32_t)(i * BSTRIDE * 2));
    }
    barrier();
    // The wave computes tiles 0..dt in intervals 0..dt + 1; the workgroup
    // runs n_kt + 1 intervals (its last wave's).
    const int n_int = n_kt + 1;
    int t = 0;
    if (active) {
        // Interval 0: S(0) (into s0) and block A's P.
        {
            const BufRsrc rk = tile_rsrc(kgb, 2 < n_kt ? 2 : n_kt - 1);
            region_x(std::false_type{}, sK, k_dst(2), rk, s0, s1);
            if (dt == 0) mask_diag(s0);
            region_y(std::false_type{}, std::true_type{}, sV, sK + TSZ, 0, s0);
            barrier();
            t = 1;
        }
        // Intervals 1..dt, two per iteration (odd t forms s1, even t s0).
        for (; t + 1 <= dt; t += 2) {
            interval(t, s1, s0);
            interval(t + 1, s0, s1);
            acc_wait();
        }
        if (t <= dt) {
            // One interval left (t odd): tile dt's scores to s1, then moved
            // to s0 for the last interval.
            interval(t, s1, s0);
            acc_wait();
#pragma unroll
            for (int qb = 0; qb < 2; qb++)
#pragma unroll
                for (int kb = 0; kb < 2; kb++) s0[qb][kb] = s1[qb][kb];
            t++;
        }
        // Interval dt + 1: P of block B and the products of the diagonal tile
        // (its scores in sl).
        auto last = [&](const f32x16 (&sl)[2][2]) {
            const bf16_bits* Vs = sV + ((t - 1) & 1) * TSZ;
            lpre[1] = lsum[1];
#pragma unroll
            for (int j = 0; j < 32; j++) {
                if (j > 0 && (j & 7) == 0) p_group(1, (j >> 3) - 1, pB);
                p_elem(sl, 1, j);
            }
            p_group(1, 3, pB);
            guard(sl);
            issue_all(t);
            region_y(std::true_type{}, std::false_type{}, Vs, sK, 0, sl);
            acc_wait();
            barrier();
        };
        last(s0);
        t++;
    }
    for (; t < n_int; t++) {
        issue_all(t);
        barrier();
    }
    if (!active) return;

    // O = O^T / l per query, lse = (m + log2 l) ln 2.
    acc_wait();
#pragma unroll
    for (int qb = 0; qb < 2; qb++) {
        const int tq = t0 + qb * 32 + l32;
        const float ltot = sum_halves(lsum[qb]);
        if (tq >= p.seq) continue;
        const float inv = 1.0f / ltot;
        float* orow = p.o + (long)b * p.q_bs + (long)tq * qrs + (long)head * DP;
#pragma unroll
        for (int db = 0; db < NDB; db++) {
#pragma unroll
            for (int rq = 0; rq < 4; rq++) {
                const int d0 = db * 32 + rq * 8 + hh * 4;
                *reinterpret_cast<float4*>(orow + d0) =
                    make_float4(oacc[qb][db][rq * 4 + 0] * inv, oacc[qb][db][rq * 4 + 1] * inv,
                                oacc[qb][db][rq * 4 + 2] * inv, oacc[qb][db][rq * 4 + 3] * inv);
            }
        }
        if (hh == 0) p.lse[((long)b * p.nh + head) * p.seq + tq] = (m2[qb] + __log2f(ltot)) * kLn2;
    }
}

// The kernel's grid for dims d: hpw heads x 4 / hpw 64-query tiles per
// workgroup.
bool attn_fwd_q64_applies(const Dims& d, bool vec_ok, bool o_vec_ok) {
    return d.hd == 128 && vec_ok && o_vec_ok;
}

hipError_t launch_attn_fwd_q64(const Dims& d, FwdParams p, hipStream_t st, KernelTimer* tm) {
    p.hpw = p.group % 4 == 0 ? 4 : p.group % 2 == 0 ? 2 : 1;
    p.tpw = 4 / p.hpw;
    p.n_sub = p.group / p.hpw;
    p.n_ttiles = (d.seq + 64 * p.tpw - 1) / (64 * p.tpw);
    const long n_items = (long)p.n_ttiles * d.nkv * p.n_sub * d.batch;
    if (n_items > 0x7fffffffL) return hipErrorInvalidConfiguration;
    p.n_items = (int)n_items;
    // One workgroup per CU (the kernel's registers allow no second) when
    // the items fill every CU at least once, in whole XCDs; else one
    // workgroup per item.
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return hipErrorInvalidDevice;
    if (p.xcd && cus >= 8 && cus % 8 == 0 && n_items >= cus) {
        p.xcd_wgs = cus / 8;
        p.n_wg = cus;
    } else {
        p.xcd_wgs = 0;
        p.n_wg = p.n_items;
    }
    TimedLaunch tl(tm, kKernFwd, st);
    hipLaunchKernelGGL(attn_fwd_q64_kernel, dim3(p.n_wg), dim3(256), 0, st, p);
    return hipGetLastError();
}

}  // namespace cfattn
