// Causal GQA attention backward on gfx950: dK/dV at head_dim 128 (bf16
// inputs, fp32 accumulation) with one wave per SIMD.
//
// Reference semantics (crates/core/src/ops/attention.rs:197-258): with P
// recomputed from the saved log-sum-exp,
//   dV_g += P^T dO,   dP = dO V^T,   dS = P * (dP - delta) * scale,
//   dK_g += dS^T Q,
// accumulated (+=) into the caller's dk, dv (ops/mod.rs:1-6).
//
// A workgroup is four waves, one per SIMD, owning 128 keys of one KV head;
// each wave holds 64 keys (two 32-key MFMA blocks), so every Q / dO operand
// it reads from LDS feeds two MFMAs -- half the LDS bytes per product of
// the two-waves-per-SIMD kernel (attn_bwd_dkdv_ws_kernel), whose register
// budget leaves room for only 32 keys per wave.
//   waves 0, 1 (P waves; keys 0-63 / 64-127 of the tile) hold K^T and the
//     dV^T accumulators: S = Q K^T, P = exp2(S*scale*log2e - lse*log2e)
//     (lse*log2e per row from the delta kernel)
//     (causally masked), P to LDS as bf16 MFMA operands, dV^T += dO^T P;
//   waves 2, 3 (dS waves; the same keys) hold -V^T and the dK^T
//     accumulators: the dO (-V^T) products accumulate onto delta, giving
//     m = delta - dP with no subtraction per element (negating bf16 is
//     exact), then with P from LDS dS = P (dP - delta) = -P m and
//     dK^T += Q^T dS.
// Steps (query head, 64-query tile = query blocks 0 and 1) run in
// attn_bwd_dkdv_ws_kernel's order and every element's products are summed
// in its order, so dK, dV and the stored dS are bitwise equal to that
// kernel's.
//
// One barrier per step; "interval t" is the time between barriers t - 1 and
// t.  Each role issues 64 MFMAs per interval in four regions of 16, and the
// VALU work (softmax, dS) is spread over all four so that it issues in the
// MFMAs' shadow: one wave hides only about three VALU instructions per
// 32x32x16 MFMA.  In interval t (a "quarter" is one 32x32 block's 16
// elements per lane, key block 0 = keys 0-31 of the wave):
//   P wave:  R1  S of (t, block 1)      | softmax of (t, block 0, key block 1)
//            R2  dV of (t, block 0)     | softmax of (t, block 1, key block 0)
//            R3  S of (t+1, block 0)    | softmax of (t, block 1, key block 1)
//            R4  dV of (t, block 1)     | softmax of (t+1, block 0, key block 0)
//   dS wave: R1  m of (t, block 0)      | dS of (t-1, block 0)
//            R2  dK of (t-1, block 0)   | dS of (t-1, block 1, key block 0), stored dS of (t-1, block 0)
//            R3  m of (t, block 1)      | dS of (t-1, block 1, key block 1), stored dS of (t-1, 1, 0)
//            R4  dK of (t-1, block 1)   | the last stored dS piece of t-1
// (stores early in the interval: the barrier's wait covers them).
// P of step t is in LDS at barrier t; the dS wave uses it in interval t + 1.
// Diagonal and ragged steps (a few per head) take a plain, unpipelined path.
// The full steps of a wave's walk are one run; each role loops over the
// masked steps before it, the run (branch-free, two steps per iteration)
// and the masked steps after it.  The per-step bookkeeping (cursors,
// buffers, the next step's buffer resources) is scalar and runs in the MFMA
// shadow of the last region.
//
// Buffers: Q (and lse) of step t are read in intervals t - 1, t and t + 1
// and loaded in interval t - 2: four buffers.  dO (and delta) of step t are
// read in interval t and loaded in interval t - 1: two buffers (three for
// delta).  P of step t is written in interval t and read in t + 1: two
// buffers.  A load issued in interval t has landed before barrier t (each
// wave waits for its own loads before the barrier) and overwrites a buffer
// whose last reader passed barrier t - 1.
#include "cfattn_common.hpp"
#include "attn_params.hpp"
#include "attn_bwd_common.hpp"
#include "mfma_asm.hpp"

#include <type_traits>

namespace cfattn {

template <bool WDS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void attn_bwd_dkdv_k64_kernel(
    const BwdParams p) {
    constexpr int DP = 128, BM = 64;
    constexpr int CPR = DP / 8;
    using L = BlkTile<DP, BM>;
    constexpr int NBL = L::NB;  // 1 KiB load blocks per tile
    constexpr int BSTRIDE = L::STRIDE, ROW16 = L::ROW16, TSZ = L::SIZE;
    constexpr int HALF = DP / 2, NKD = HALF / 8, NDB = DP / 32, NKB = 2;
    constexpr int BPW = NBL / 4;                 // blocks of each tile one wave loads
    // LDS operands are read this many operands (2*LA MFMA slots) ahead of
    // their MFMA, so that their latency hides behind the MFMAs in between.
    constexpr int LA = 3;
    constexpr int NQBUF = 4, NOBUF = 2, NDBUF = 3;  // Q, dO and delta buffers
    static_assert(NBL % 4 == 0 && BM == 64, "tile must split evenly over the four waves");
    __shared__ __attribute__((aligned(16))) bf16_bits sQ[NQBUF * TSZ];
    __shared__ __attribute__((aligned(16))) bf16_bits sO[NOBUF * TSZ];  // dO rows
    __shared__ __attribute__((aligned(16))) float sL[NQBUF][BM];        // lse*log2e, by MFMA row
    __shared__ __attribute__((aligned(16))) float sD[NDBUF][BM];        // delta, by MFMA row
    // P as the P waves' bf16 MFMA operands: [buffer][pair][qb][kb][half][lane].
    __shared__ uint4 sP[2][2][2][NKB][2][64];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // Wave index and everything derived from it, uniform (scalar registers).
    const int wv = wave_uniform(tid >> 6);
    const int pair = (tid >> 6) & 1;
    const bool pwave = wv < 2;
    const int l32 = lane & 31, hh = lane >> 5;

    const int id = xcd_remap(blockIdx.x, p.n_wg_kv, p.xcd);
    const int kvt = id % p.n_kvtiles;  // low key tiles see the most queries: first
    const int rest = id / p.n_kvtiles;
    const int g = rest % p.nkv;
    const int b = rest / p.nkv;
    const int wg_key0 = kvt * p.kv_tile;
    const int key0 = wg_key0 + pair * 64;
    // key0 as a scalar, for addresses (the branch conditions keep the
    // per-lane form, with which the compiler allocates registers better).
    const int key0s = wg_key0 + (wv & 1) * 64;
    const bool pair_live = key0 < p.seq;

    const long qrs = (long)p.nh * DP, kvrs = (long)p.nkv * DP;
    const bf16_bits* qg = static_cast<const bf16_bits*>(p.q) + (long)b * p.q_bs;
    const bf16_bits* og = static_cast<const bf16_bits*>(p.d_o) + (long)b * p.q_bs;
    const long lrow_base = (long)b * p.nh * p.seq;

    // Row reads: lane (l32, hh) reads MFMA row l32 (tile row qperm(l32)),
    // chunks hh*NKD + kd.  Transposed reads: in each 16-lane group G, lane
    // 4k + m supplies head dims 16*(G%2) + 4m + [0, 4) of MFMA row 4*hh + k
    // (+8, +16, +24), that is tile row 4k + hh (+2, +16, +18).
    const int rrow = L::row(qperm(l32)) + hh * HALF;
    const int G = lane >> 4, jj = lane & 15;
    const int trow = L::row(4 * (jj >> 2) + hh) + 16 * (G & 1) + 4 * (jj & 3);
    // Stored dS (kDsBlock layout): lane l writes its first eight values to
    // 16-byte slot l ^ hh and the other eight to slot 64 + (l ^ (2 + hh)).
    // Byte offsets of the lane's two 16-byte pieces in a stored-dS block.
    const uint32_t ds_off0 = (uint32_t)(lane ^ hh) * 16, ds_off1 = (uint32_t)(64 + (lane ^ (2 + hh))) * 16;

    const int n_qt = (p.seq + BM - 1) / BM;
    const int qt_begin = wg_key0 / BM;
    const int n_steps = p.group * (n_qt - qt_begin);
    // A step: query tile [q0, q0 + BM) of query head h.  Steps run over the
    // heads of the group for one query tile, then the next tile, walking the
    // tiles qt_begin..n_qt-1 down or up (dkdv_walks_down).  Each wave walks
    // them with cursors that also carry the step's byte offsets: qo of its
    // Q / dO rows (row q0, head h) and lo of its lse / delta rows, both
    // within the sequence (32-bit: a sequence's Q has fewer than 2^31
    // elements, checked by the launcher's shape limits).  Past the last step
    // a cursor starts over at the first, so the loads a wave issues for
    // steps beyond its last stay inside the sequence (they fill buffers that
    // are never read).
    struct Pos {
        int q0, h;
        uint32_t qo, lo;
    };
    const bool down = dkdv_walks_down(blockIdx.x, p.xcd_cus);
    const int h0 = g * p.group, h_end = h0 + p.group, q_step = down ? -BM : BM;
    const int q_first = (down ? n_qt - 1 : qt_begin) * BM, q_past = (down ? qt_begin - 1 : n_qt) * BM;
    const uint32_t qo_row = (uint32_t)qrs * 2u;  // bytes per query row
    const uint32_t qo_head = DP * 2, lo_head = (uint32_t)p.seq * 4u;
    const uint32_t qo_wrap = (uint32_t)q_step * qo_row - (uint32_t)(p.group - 1) * qo_head;
    const uint32_t lo_wrap = (uint32_t)q_step * 4u - (uint32_t)(p.group - 1) * lo_head;
    const uint32_t qo_again = (uint32_t)(q_first - q_past) * qo_row, lo_again = (uint32_t)(q_first - q_past) * 4u;
    const Pos first{q_first, h0, (uint32_t)q_first * qo_row + (uint32_t)h0 * qo_head,
                    (uint32_t)h0 * lo_head + (uint32_t)q_first * 4u};
    // (Selects, not branches: it runs in MFMA shadows.)
    auto next_pos = [&](Pos x) {
        const bool wrap = x.h + 1 == h_end;
        x.h = wrap ? h0 : x.h + 1;
        x.q0 += wrap ? q_step : 0;
        x.qo += wrap ? qo_wrap : qo_head;
        x.lo += wrap ? lo_wrap : lo_head;
        const bool again = x.q0 == q_past;
        x.q0 = again ? q_first : x.q0;
        x.qo += again ? qo_again : 0u;
        x.lo += again ? lo_again : 0u;
        return x;
    };
    // The wave's keys meet at least one query of the step.
    auto pos_act = [&](Pos x) { return pair_live && x.q0 + BM - 1 >= key0; };
    // Every query of the step is past every key of the wave and inside the
    // sequence: no mask, and every block is on or below the diagonal.
    auto pos_full = [&](Pos x) { return x.q0 >= key0 + 63 && x.q0 + BM <= p.seq; };
    // The full steps of the wave's walk are one run, steps [s_full0,
    // s_full1): query tiles t with 64 t >= key0 + 63 (past the diagonal) and
    // 64 (t + 1) <= seq (not cut by the end), met in walk order.  The loops
    // below run the steps before and after the run through the masked path
    // and the run itself through the pipelined one, with no per-step branch.
    int s_full0 = 0, s_full1 = 0;
    {
        const int t_lo = max((key0s + 63 + BM - 1) / BM, qt_begin), t_hi = p.seq / BM - 1;
        if (key0s < p.seq && t_lo <= t_hi) {
            s_full0 = (down ? n_qt - 1 - t_hi : t_lo - qt_begin) * p.group;
            s_full1 = (down ? n_qt - t_lo : t_hi + 1 - qt_begin) * p.group;
        }
    }

    // Tile loads: wave w loads blocks w*BPW.. of a Q and a dO tile, lane l of
    // block bk reading chunk l % CPR of tile row bk + NB*(l / CPR).  Wave 0
    // also loads lse*log2e (lse2) and wave 1 delta, one value per MFMA row (MFMA row
    // `lane`: tile row (lane & 32) + qperm(lane & 31)).  The loads are
    // bounds-checked buffer loads whose buffer starts at the step's rows and
    // ends with the sequence: rows past the end read zeros (masked below),
    // and the per-lane byte offsets are the same for every step.
    const int lane_row = NBL * (lane / CPR), lane_col = (lane % CPR) * 8;
    const int lrow = (lane & 32) + qperm(lane & 31);
    constexpr int kLoadsP = 2 * BPW + 1, kLoadsDs = 2 * BPW;
    uint32_t tile_off[BPW];
#pragma unroll
    for (int i = 0; i < BPW; i++) tile_off[i] = (uint32_t)(((lane_row + wv * BPW + i) * (int)qrs + lane_col) * 2);
    const uint32_t row_off = (uint32_t)lrow * 4u;
    struct Loads {
        BufRsrc q, o, l;            // the Q tile, the dO tile, the lse (wave 0) or delta (wave 1) rows
        uint32_t qlds, olds, llds;  // LDS byte addresses of this wave's first block / of the row values
    };
    const char* qgb = reinterpret_cast<const char*>(qg);
    const char* ogb = reinterpret_cast<const char*>(og);
    const char* lgb = reinterpret_cast<const char*>((wv == 0 ? p.lse2 : p.delta) + lrow_base);
    const uint32_t sq0 = lds_offset(sQ) + (uint32_t)(wv * BPW * BSTRIDE * 2);
    const uint32_t so0 = lds_offset(sO) + (uint32_t)(wv * BPW * BSTRIDE * 2);
    const uint32_t sl0 = lds_offset(wv == 0 ? &sL[0][0] : &sD[0][0]);
    auto set_loads = [&](Pos xq, int qbuf, Pos xo, int obuf, int dbuf) {
        Loads l;
        l.q = buf_rsrc(qgb + xq.qo, (uint32_t)(p.seq - xq.q0) * qo_row);
        l.o = buf_rsrc(ogb + xo.qo, (uint32_t)(p.seq - xo.q0) * qo_row);
        const Pos xl = wv == 0 ? xq : xo;
        l.l = buf_rsrc(lgb + xl.lo, (uint32_t)(p.seq - xl.q0) * 4u);
        l.qlds = sq0 + (uint32_t)(qbuf * TSZ * 2);
        l.olds = so0 + (uint32_t)(obuf * TSZ * 2);
        l.llds = sl0 + (uint32_t)((wv == 0 ? qbuf : dbuf) * BM * 4);
        return l;
    };
    // Load i of this wave's share: Q blocks, dO blocks, then lse / delta.
    auto issue_load = [&](int i, const Loads& l) {
        if (i < BPW) {
            lds_buf_load16(l.q, tile_off[i], l.qlds + (uint32_t)(i * BSTRIDE * 2));
        } else if (i < 2 * BPW) {
            lds_buf_load16(l.o, tile_off[i - BPW], l.olds + (uint32_t)((i - BPW) * BSTRIDE * 2));
        } else {
            lds_buf_load4(l.l, row_off, l.llds);
        }
    };
    auto issue_all = [&](const Loads& l, auto n) {
#pragma unroll
        for (int i = 0; i < decltype(n)::value; i++) issue_load(i, l);
    };
    // This wave's loads have landed and its LDS accesses are done; then the
    // workgroup barrier (no fence: the waits above are exactly the ones the
    // barrier must cover).
    auto step_barrier = [&]() {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    // Operands, read ahead of their use.  Row operand (kd) of query block qb
    // of tile A.
    auto rd_row = [&](const bf16_bits* A, int qb, int kd) {
        return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(A + rrow + qb * 2 * ROW16 + kd * 8));
    };
    // Transposed operand o = 2*db + sub (sub 0: MFMA rows 4hh..+3 and
    // 8+4hh..+3; 1: 16 more) of query block qb of tile A.
    auto rd_tr = [&](const bf16_bits* A, int qb, int o) {
        const bf16_bits* t = A + trow + qb * 2 * ROW16 + (o >> 1) * 32 + (o & 1) * ROW16;
        return join_bf16x4(ds_read_tr16(t), ds_read_tr16(t + 2 * BSTRIDE));
    };
    // x[kb] = rows of query block qb of tile A times the wave's K^T / V^T
    // operands (S or dP of the block), unscheduled (masked steps).
    auto score = [&](const bf16_bits* A, int qb, const bf16x8 (&xf)[NKB][NKD], f32x16 (&x)[NKB],
                     const f32x16& init) {
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) x[kb] = init;
#pragma unroll
        for (int kd = 0; kd < NKD; kd++) {
            const bf16x8 a = rd_row(A, qb, kd);
#pragma unroll
            for (int kb = 0; kb < NKB; kb++) x[kb] = mfma32(a, xf[kb][kd], x[kb]);
        }
    };
    // acc[db][kb] += (tile A, query block qb)^T op[kb], unscheduled.
    auto products = [&](const bf16_bits* A, int qb, const bf16x8 (&op)[NKB][2], f32x16 (&acc)[NDB][NKB]) {
#pragma unroll
        for (int o = 0; o < 2 * NDB; o++) {
            const bf16x8 t = rd_tr(A, qb, o);
#pragma unroll
            for (int kb = 0; kb < NKB; kb++) mfma_acc(acc[o >> 1][kb], t, op[kb][o & 1]);
        }
    };

    // K^T (P waves) or V^T (dS waves) operands: key key0 + 32*kb + l32,
    // head dims hh*HALF + kd*8 + [0, 8).
    auto load_keys = [&](const void* src_, bf16x8 (&xf)[NKB][NKD], bool negate) {
        const uint32_t sgn = negate ? 0x80008000u : 0u;
        const bf16_bits* src = static_cast<const bf16_bits*>(src_) + (long)b * p.kv_bs + (long)g * DP + hh * HALF;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const int kw = key0 + kb * 32 + l32;
            const bool ok = kw < p.seq;
            const bf16_bits* xr = src + (long)(ok ? kw : 0) * kvrs;
#pragma unroll
            for (int kd = 0; kd < NKD; kd++) {
                uint4 u = ok ? *reinterpret_cast<const uint4*>(xr + kd * 8) : make_uint4(0, 0, 0, 0);
                u.x ^= sgn, u.y ^= sgn, u.z ^= sgn, u.w ^= sgn;
                xf[kb][kd] = __builtin_bit_cast(bf16x8, u);
            }
        }
        // Wait for the operands here, with a wait the compiler sees: the
        // loop's own waits are inline assembly, invisible to its wait-count
        // tracking, which would otherwise put a full vmcnt(0) wait (on the
        // tile loads just issued) before the first use in every step.
        __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
    };
    auto zero_acc = [&](f32x16 (&acc)[NDB][NKB]) {
#pragma unroll
        for (int db = 0; db < NDB; db++)
#pragma unroll
            for (int kb = 0; kb < NKB; kb++) {
                acc[db][kb] = zero16();
                agpr_pin(acc[db][kb]);
            }
    };
    // After a wave's last step: its last loads (a step past the end, into an
    // unused buffer) have landed before it can leave the workgroup's LDS,
    // and the last MFMA writing an accumulator completes before anything
    // reads it: 34 wait states (a 32x32x16 MFMA takes 8 passes of 4
    // cycles), tied to every accumulator so that no read is scheduled above
    // them.
    auto acc_drain = [&](f32x16 (&acc)[NDB][NKB]) {
        asm volatile("s_waitcnt vmcnt(0)\n\ts_nop 15\n\ts_nop 15\n\ts_nop 3"
                     : "+a"(acc[0][0]), "+a"(acc[0][1]), "+a"(acc[1][0]), "+a"(acc[1][1]), "+a"(acc[2][0]),
                       "+a"(acc[2][1]), "+a"(acc[3][0]), "+a"(acc[3][1]));
    };
    // The same 34 wait states without the load wait, at the end of every
    // iteration of the loops over a wave's steps (masked steps, the full
    // run, masked steps): the compiler may keep the accumulators in other
    // registers in each loop and copy them across on leaving it, and it
    // cannot see that the MFMAs right before such a copy (inline assembly)
    // are still writing them.  Copies for a loop's exit come after the
    // iteration's last instruction.
    auto acc_settle = [&](f32x16 (&acc)[NDB][NKB]) {
        acc_wait8(acc[0][0], acc[0][1], acc[1][0], acc[1][1], acc[2][0], acc[2][1], acc[3][0], acc[3][1]);
    };
    // dV rows are added; dK rows (scaled: dS was accumulated without the
    // softmax scale) go through the epilogue mode.  The current values of
    // the lane's rows (both key blocks) are read before any is written, so
    // that the wave waits for one round of reads rather than one per block.
    auto store_rows = [&](float* dst, f32x16 (&acc)[NDB][NKB], bool dk_rows) {
        if (!pair_live) return;
        const int mode = dk_rows ? p.epi : kEpiAdd;
        float* row[NKB];
        bool ok[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const int kw = key0 + kb * 32 + l32;
            ok[kb] = kw < p.seq;
            row[kb] = dst + (long)b * p.kv_bs + (long)kw * kvrs + (long)g * DP;
        }
        float4 cur[NKB][NDB][4];
        if (mode == kEpiAdd || mode == kEpiUnrotAdd) {
#pragma unroll
            for (int kb = 0; kb < NKB; kb++) load_grad_row<NDB>(cur[kb], row[kb], hh, ok[kb]);
        }
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            if (!ok[kb]) continue;
            const int kw = key0 + kb * 32 + l32;
            f32x16 r[NDB];
#pragma unroll
            for (int db = 0; db < NDB; db++) r[db] = dk_rows ? acc[db][kb] * p.scale : acc[db][kb];
            if (mode == kEpiAdd || mode == kEpiUnrotAdd)
                write_grad_row<NDB, true>(row[kb], r, hh, kw, p, cur[kb], mode);
            else
                write_grad_row<NDB>(row[kb], r, hh, kw, p, nullptr, mode);
        }
    };
    // Per-row values (lse or delta) of MFMA rows 8*g4 + 4*hh + [0, 4) of
    // query block qb: elements 4*g4 .. 4*g4 + 3 of a lane's 16.
    auto row_vals4 = [&](const float* src, int qb, int g4) {
        return *reinterpret_cast<const float4*>(&src[qb * 32 + g4 * 8 + hh * 4]);
    };

    // ------------------------------------------------------------ P waves
    auto run_p = [&]() {
        bf16x8 xf[NKB][NKD];
        load_keys(p.k, xf, false);
        f32x16 acc[NDB][NKB];  // dV^T, in AGPRs
        zero_acc(acc);

        // P of an element: exp2(S*scale*log2e - lse*log2e), lv = lse*log2e
        // (the delta kernel's lse2 rows: the same f32 product, formed once
        // per row instead of once per row and key tile).
        auto p_elem = [&](float s, float lv) { return __builtin_amdgcn_exp2f(__builtin_fmaf(s, p.sl2, -lv)); };
        // lse*log2e of the lane's 16 rows of query block qb.
        auto lse_raw = [&](const float* Ls, int qb, float (&lv)[16]) {
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const float4 l = row_vals4(Ls, qb, g4);
                lv[g4 * 4 + 0] = l.x, lv[g4 * 4 + 1] = l.y, lv[g4 * 4 + 2] = l.z, lv[g4 * 4 + 3] = l.w;
            }
        };
        auto lse_part = [&](const float* Ls, int qb, int g4, float (&lv)[16]) {
            const float4 l = row_vals4(Ls, qb, g4);
            lv[g4 * 4 + 0] = l.x;
            lv[g4 * 4 + 1] = l.y;
            lv[g4 * 4 + 2] = l.z;
            lv[g4 * 4 + 3] = l.w;
        };
        auto publish = [&](int pbuf, int qb, int kb, const bf16x8 (&pb)[2]) {
            sP[pbuf][pair][qb][kb][0][lane] = __builtin_bit_cast(uint4, pb[0]);
            sP[pbuf][pair][qb][kb][1][lane] = __builtin_bit_cast(uint4, pb[1]);
        };

        // Masked step (diagonal or ragged): everything in program order.
        // Element r of block (qb, kb) is MFMA row g4*8 + hh*4 + i (r = 4*g4 + i)
        // and key key0 + 32*kb + l32; masked are keys past the query and rows
        // past the sequence.
        auto masked_step = [&](Pos x, int qbuf, int obuf, int pbuf) {
            const bf16_bits* Qs = sQ + qbuf * TSZ;
            const bf16_bits* Os = sO + obuf * TSZ;
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                f32x16 sc[NKB];
                bf16x8 pq[NKB][2];
                float lv[16];
                score(Qs, qb, xf, sc, zero16());
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) lse_part(sL[qbuf], qb, g4, lv);
#pragma unroll
                for (int kb = 0; kb < NKB; kb++) {
                    const int kw = key0 + kb * 32 + l32;
                    float pr[16];
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        float pv = p_elem(sc[kb][r], lv[r]);
                        const int q = x.q0 + qb * 32 + qperm((r >> 2) * 8 + hh * 4 + (r & 3));
                        if (kw > q || q >= p.seq) pv = 0.0f;
                        pr[r] = pv;
                    }
                    pq[kb][0] = cvt_bf16x8(&pr[0]);
                    pq[kb][1] = cvt_bf16x8(&pr[8]);
                    publish(pbuf, qb, kb, pq[kb]);
                }
                CF_HAZARD_FENCE();
                products(Os, qb, pq, acc);
            }
        };

        // Pipeline state entering a full step t: S of (t, block 0, key block
        // 1), lse*log2e of block 0's rows, and P of (t, block 0, key block 0)
        // as operands (published in R1 of interval t, where its LDS buffer is
        // free).  Two copies, for even and odd steps: each step reads one and
        // forms the other in place.
        struct PState {
            f32x16 s01;
            float lv0[16];
            bf16x8 p00[2];
            bf16x8 q1[LA];  // the first row operands of (t, block 1), read before barrier t - 1
        };
        PState st0, st1;
        // Forms the state of full step x (unscheduled: after a masked step).
        auto prime = [&](int qbuf, PState& o) {
            f32x16 sc[NKB];
            score(sQ + qbuf * TSZ, 0, xf, sc, zero16());
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) lse_part(sL[qbuf], 0, g4, o.lv0);
            float pr[16];
#pragma unroll
            for (int r = 0; r < 16; r++) pr[r] = p_elem(sc[0][r], o.lv0[r]);
            o.p00[0] = cvt_bf16x8(&pr[0]);
            o.p00[1] = cvt_bf16x8(&pr[8]);
            o.s01 = sc[1];
#pragma unroll
            for (int i = 0; i < LA; i++) o.q1[i] = rd_row(sQ + qbuf * TSZ, 1, i);
        };

        // Full step t in regions R1-R4, fenced in slots of one MFMA and the
        // work that issues in its shadow (a second MFMA right behind would
        // block issue until the pipe frees).  EARLY: step t + 1 is full too,
        // and its S of block 0 and first softmax quarter are formed here.
        auto full_step = [&](auto early_tag, int qbuf, int obuf, int pbuf, int nqbuf, const Loads& ld,
                             const PState& in, PState& out, auto&& adv) {
            constexpr bool EARLY = decltype(early_tag)::value;
            const bf16_bits* Qs = sQ + qbuf * TSZ;
            const bf16_bits* Qn = sQ + nqbuf * TSZ;  // Q of step t + 1
            const bf16_bits* Os = sO + obuf * TSZ;
            bf16x8 qr[NKD], tr[2 * NDB];
            float lv1[16], pr[16];
            f32x16 s1[NKB], sn0;
            bf16x8 p01[2], p10[2], p11[2];
            // Element e of a softmax quarter per slot; the quarter's halves
            // are rounded to bf16 operands after elements 7 and 15 (and
            // published unless the quarter belongs to the next step).
            auto sm = [&](int e, const f32x16& sc, const float (&lv)[16], bf16x8 (&pb)[2], int qb, int kb, bool pub) {
                pr[e] = p_elem(sc[e], lv[e]);
                if ((e & 7) == 7) {
                    pb[e >> 3] = cvt_bf16x8(&pr[e & 8]);
                    if (pub) sP[pbuf][pair][qb][kb][e >> 3][lane] = __builtin_bit_cast(uint4, pb[e >> 3]);
                }
            };
            // R1: S of (t, 1) | softmax (t, 0, 1); P (t, 0, 0) published;
            // lse*log2e of block 1 (read here, used from R2 on); this
            // interval's loads.  The first row operands came with the state
            // (read in the previous step's last region), so that the first
            // MFMAs wait for no LDS read.
#pragma unroll
            for (int i = 0; i < LA; i++) qr[i] = in.q1[i];
            lse_raw(sL[qbuf], 1, lv1);
            publish(pbuf, 0, 0, in.p00);
            CF_FENCE();
#pragma unroll
            for (int k = 0; k < 2 * NKD; k++) {
                const int kd = k >> 1, kb = k & 1;
                if (kb == 0 && kd + LA < NKD) qr[kd + LA] = rd_row(Qs, 1, kd + LA);
                if (k >= 2 * NKD - LA) tr[k - (2 * NKD - LA)] = rd_tr(Os, 0, k - (2 * NKD - LA));
                s1[kb] = mfma32(qr[kd], xf[kb][kd], kd == 0 ? zero16() : s1[kb]);
                sm(k, in.s01, in.lv0, p01, 0, 1, true);
                if (kb == 0) issue_load(kd, ld);
                CF_FENCE();
            }
            // lse*log2e of (t+1, 0), for R4.
            if (EARLY) lse_raw(sL[nqbuf], 0, out.lv0);
            CF_HAZARD_FENCE();
            // R2: dV of (t, 0) | softmax (t, 1, 0); the first Q rows of
            // (t+1, 0) for R3.
#pragma unroll
            for (int k = 0; k < 2 * NKD; k++) {
                const int o = k >> 1, kb = k & 1;
                if (kb == 0 && o + LA < 2 * NDB) tr[o + LA] = rd_tr(Os, 0, o + LA);
                if (EARLY && (k & 3) == 1 && (k >> 2) < LA) qr[k >> 2] = rd_row(Qn, 0, k >> 2);
                // The step's first MFMA into each accumulator waits for a
                // copy the compiler may place right before it.
                if ((o & 1) == 0)
                    mfma_acc_lead(acc[o >> 1][kb], tr[o], kb == 0 ? in.p00[o & 1] : p01[o & 1]);
                else
                    mfma_acc(acc[o >> 1][kb], tr[o], kb == 0 ? in.p00[o & 1] : p01[o & 1]);
                sm(k, s1[0], lv1, p10, 1, 0, true);
                if (k == 0) issue_load(NKD, ld);
                CF_FENCE();
            }
            // R3: S of (t+1, 0) | softmax (t, 1, 1).
#pragma unroll
            for (int k = 0; k < 2 * NKD; k++) {
                const int kd = k >> 1, kb = k & 1;
                if (EARLY && kb == 0 && kd + LA < NKD) qr[kd + LA] = rd_row(Qn, 0, kd + LA);
                if (k >= 2 * NKD - LA) tr[k - (2 * NKD - LA)] = rd_tr(Os, 1, k - (2 * NKD - LA));
                if (EARLY) {
                    if (kb == 0)
                        sn0 = mfma32(qr[kd], xf[0][kd], kd == 0 ? zero16() : sn0);
                    else
                        out.s01 = mfma32(qr[kd], xf[1][kd], kd == 0 ? zero16() : out.s01);
                }
                sm(k, s1[1], lv1, p11, 1, 1, true);
                CF_FENCE();
            }
            CF_HAZARD_FENCE();
            // R4: dV of (t, 1) | softmax (t+1, 0, 0), kept for the next
            // interval.
#pragma unroll
            for (int k = 0; k < 2 * NKD; k++) {
                const int o = k >> 1, kb = k & 1;
                if (kb == 0 && o + LA < 2 * NDB) tr[o + LA] = rd_tr(Os, 1, o + LA);
                mfma_acc(acc[o >> 1][kb], tr[o], kb == 0 ? p10[o & 1] : p11[o & 1]);
                if (EARLY) sm(k, sn0, out.lv0, out.p00, 0, 0, false);
                // The next step's first row operands: Q(t + 1) is complete
                // since barrier t - 1.
                if (EARLY && k >= 2 * NKD - 2 * LA && (k & 1)) out.q1[(k - (2 * NKD - 2 * LA)) >> 1] = rd_row(Qn, 1, (k - (2 * NKD - 2 * LA)) >> 1);
                adv(k);
                CF_FENCE();
            }
        };

        Pos cur = first, n1 = next_pos(first), n2 = next_pos(n1);
        int qbuf = 0, obuf = 0, dbuf = 0;  // buffers of the current step
        // The current step's loads: Q of the step two ahead, dO of the next
        // one (past the last step, the cursors' restarted walk: loaded,
        // unused).
        Loads ld = set_loads(n2, 2, n1, 1, 1);
        // Part k of moving the bookkeeping above on to the next step; a full
        // step spreads the parts over the slots of its last region (whose
        // MFMAs leave issue slots free), after its own loads are issued.
        auto adv = [&](int k) {
            if (k == 1) {
                cur = n1;
                n1 = n2;
            }
            if (k == 3) n2 = next_pos(n2);
            if (k == 5) {
                qbuf = (qbuf + 1) & 3;
                obuf ^= 1;
                dbuf = dbuf == 2 ? 0 : dbuf + 1;
            }
            if (k == 7) ld = set_loads(n2, (qbuf + 2) & 3, n1, obuf ^ 1, dbuf == 2 ? 0 : dbuf + 1);
        };
        // Step s outside the full run; the one right before it forms the
        // run's first state (in st0).
        auto masked = [&](int s) {
            issue_all(ld, std::integral_constant<int, kLoadsP>{});
            if (pos_act(cur)) masked_step(cur, qbuf, obuf, s & 1);
            if (s + 1 == s_full0) prime((qbuf + 1) & 3, st0);
#pragma unroll
            for (int k = 0; k < 2 * NKD; k++) adv(k);
            step_barrier();
        };
        // Step s of the full run with state `in`, forming `out` if the next
        // step is in the run too (EARLY).
        auto full = [&](auto early, int s, const PState& in, PState& out) {
            full_step(early, qbuf, obuf, s & 1, (qbuf + 1) & 3, ld, in, out, adv);
            step_barrier();
        };
        if (s_full0 == 0 && s_full1 > 0) prime(qbuf, st0);
        int s = 0;
        for (; s < s_full0; s++) {
            masked(s);
            acc_settle(acc);
        }
        for (; s + 2 < s_full1; s += 2) {
            full(std::true_type{}, s, st0, st1);
            full(std::true_type{}, s + 1, st1, st0);
            acc_settle(acc);
        }
        if (s + 1 < s_full1) {
            full(std::true_type{}, s, st0, st1);
            full(std::false_type{}, s + 1, st1, st0);
            acc_settle(acc);
            s += 2;
        } else if (s < s_full1) {
            full(std::false_type{}, s, st0, st1);
            acc_settle(acc);
            s++;
        }
        for (; s < n_steps; s++) {
            masked(s);
            acc_settle(acc);
        }
        acc_drain(acc);
        store_rows(p.dv, acc, false);
    };

    // ----------------------------------------------------------- dS waves
    auto run_ds = [&]() {
        bf16x8 xf[NKB][NKD];
        load_keys(p.v, xf, true);
        f32x16 acc[NDB][NKB];  // dK^T, in AGPRs
        zero_acc(acc);

        // dS of element r of a block: P (the bf16 value the P wave's dV
        // product used; widening is exact) times dP - delta.  w: the block's
        // two published halves as eight words.
        // dS element r from the P words and m = delta - dP (the negated
        // product's accumulator): P (dP - delta) = P * -m.
        auto ds_elem = [&](const uint32_t (&w)[8], int r, float m) {
            const uint32_t word = w[r >> 1];
            return __uint_as_float((r & 1) ? (word & 0xffff0000u) : (word << 16)) * -m;
        };
        auto p_words = [&](int pbuf, int qb, int kb, uint32_t (&w)[8]) {
            const uint4 a = sP[pbuf][pair][qb][kb][0][lane], c = sP[pbuf][pair][qb][kb][1][lane];
            w[0] = a.x, w[1] = a.y, w[2] = a.z, w[3] = a.w, w[4] = c.x, w[5] = c.y, w[6] = c.z, w[7] = c.w;
        };
        // delta of the lane's 16 rows of query block qb, as an accumulator.
        auto delta16 = [&](int dbuf_, int qb) {
            f32x16 dl;
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const float4 d = row_vals4(sD[dbuf_], qb, g4);
                dl[g4 * 4 + 0] = d.x, dl[g4 * 4 + 1] = d.y, dl[g4 * 4 + 2] = d.z, dl[g4 * 4 + 3] = d.w;
            }
            return dl;
        };
        // One 16-byte piece (qb, kb, half h) of a step's dS (rounded to bf16)
        // to the stored-dS scratch: blocks on or below the causal diagonal
        // only (the layout has no others), non-temporal (the dQ kernel reads
        // each once).
        // The block index is below 2^32 (the scratch would be 8 TiB), so it
        // is formed in 32-bit scalar arithmetic and the store addressed as
        // a scalar base plus the lane's byte offset.
        auto ds_store = [&](Pos x, int qb, int kb, int h, const bf16x8& v, bool check) {
            const int qi = (x.q0 >> 5) + qb, ki = (key0 >> 5) + kb;
            if (check && !(ki <= qi && x.q0 + qb * 32 < p.seq)) return;
            const uint32_t blk = __builtin_amdgcn_readfirstlane(
                ((uint32_t)b * (uint32_t)p.nh + (uint32_t)x.h) * (uint32_t)p.ds_ntri +
                (uint32_t)(qi * (qi + 1) / 2 + ki));
            const char* base = reinterpret_cast<const char*>(p.ds) + (size_t)blk * (kDsBlock * sizeof(bf16_bits));
            __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v),
                                        reinterpret_cast<u32x4*>(const_cast<char*>(base) + (h ? ds_off1 : ds_off0)));
        };
        // The same for a full step, from the step's block (query block 0,
        // key block 0) address: key block kb is the next block, query block
        // 1 starts qi + 1 blocks on (its row of the triangle is one longer).
        constexpr uint32_t kDsBytes = kDsBlock * sizeof(bf16_bits);
        auto ds_row_base = [&](Pos x) {
            const uint32_t qi = (uint32_t)x.q0 >> 5, ki = (uint32_t)key0s >> 5;
            const uint32_t blk = ((uint32_t)b * (uint32_t)p.nh + (uint32_t)x.h) * (uint32_t)p.ds_ntri +
                                 qi * (qi + 1) / 2 + ki;
            return reinterpret_cast<const char*>(p.ds) + (size_t)blk * kDsBytes;
        };
        auto ds_store_at = [&](const char* base, int kb, int h, const bf16x8& v) {
            __builtin_nontemporal_store(
                __builtin_bit_cast(u32x4, v),
                reinterpret_cast<u32x4*>(const_cast<char*>(base) + kb * kDsBytes + (h ? ds_off1 : ds_off0)));
        };

        // delta - dP of the step whose dS comes next, by query block and key
        // block: the products with the negated V^T operands accumulated onto
        // delta.  Two copies, for even and odd steps: each iteration reads
        // one and forms the other in place.
        struct DState {
            f32x16 d[2][NKB];
        };
        DState st0, st1;
        // Forms it for the step with dO in buffer obuf (unscheduled).
        auto dp_of = [&](int obuf, int dbuf_, DState& o) {
            score(sO + obuf * TSZ, 0, xf, o.d[0], delta16(dbuf_, 0));
            score(sO + obuf * TSZ, 1, xf, o.d[1], delta16(dbuf_, 1));
        };
        // dS and dK of step x (unscheduled; its P in buffer pbuf).
        auto ds_dk = [&](Pos x, int qbuf, int pbuf, bool check, const DState& in) {
            const bf16_bits* Qs = sQ + qbuf * TSZ;
#pragma unroll
            for (int qb = 0; qb < 2; qb++) {
                bf16x8 dq[NKB][2];
#pragma unroll
                for (int kb = 0; kb < NKB; kb++) {
                    uint32_t w[8];
                    p_words(pbuf, qb, kb, w);
                    float ds[16];
#pragma unroll
                    for (int r = 0; r < 16; r++) ds[r] = ds_elem(w, r, in.d[qb][kb][r]);
                    dq[kb][0] = cvt_bf16x8(&ds[0]);
                    dq[kb][1] = cvt_bf16x8(&ds[8]);
                    if constexpr (WDS) {
                        ds_store(x, qb, kb, 0, dq[kb][0], check);
                        ds_store(x, qb, kb, 1, dq[kb][1], check);
                    }
                }
                CF_HAZARD_FENCE();
                products(Qs, qb, dq, acc);
            }
        };

        // Iteration t (interval t + 1): dS and dK of step t, dP - delta of
        // step t + 1, in regions R1-R4 (see the file header).  Step t is
        // unmasked and step t + 1 active.
        auto full_iter = [&](Pos x, const char* dsb, int qbuf, int pbuf, int nobuf, int ndbuf, const Loads& ld,
                             const DState& in, DState& out, auto&& adv) {
            const bf16_bits* Qs = sQ + qbuf * TSZ;
            const bf16_bits* On = sO + nobuf * TSZ;  // dO of step t + 1
            bf16x8 orow[NKD], tr[2 * NDB];
            uint32_t w[NKB][8];
            float ds[NKB][16];
            bf16x8 d0[NKB][2], d1[NKB][2];
            // dS element e of (t, qb, kb) per slot, rounded after 7 and 15.
            auto dse = [&](int qb, int kb, int e, bf16x8 (&dd)[NKB][2]) {
                ds[kb][e] = ds_elem(w[kb], e, in.d[qb][kb][e]);
                if ((e & 7) == 7) dd[kb][e >> 3] = cvt_bf16x8(&ds[kb][e & 8]);
            };
            // Piece i of the step's stored dS: (qb, kb, half) = (i / 4, (i / 2) % 2, i % 2).
            const char* dsq1 = dsb + ((uint32_t)(x.q0 >> 5) + 1u) * kDsBytes;  // query block 1
            auto store_piece = [&](int i) {
                const int sq = i >> 2, skb = (i >> 1) & 1, sh = i & 1;
                ds_store_at(sq ? dsq1 : dsb, skb, sh, sq ? d1[skb][sh] : d0[skb][sh]);
            };
            f32x16 dl = delta16(ndbuf, 0);
#pragma unroll
            for (int i = 0; i < LA; i++) orow[i] = rd_row(On, 0, i);
            p_words(pbuf, 0, 0, w[0]);
            p_words(pbuf, 0, 1, w[1]);
            CF_FENCE();
            // R1: dP of (t+1, 0) | dS of (t, 0); this interval's loads.
#pragma unroll
            for (int k = 0; k < 2 * NKD; k++) {
                const int kd = k >> 1, kb = k & 1;
                if (kb == 0 && kd + LA < NKD) orow[kd + LA] = rd_row(On, 0, kd + LA);
                if (k >= 2 * NKD - LA) tr[k - (2 * NKD - LA)] = rd_tr(Qs, 0, k - (2 * NKD - LA));
                out.d[0][kb] = mfma32(orow[kd], xf[kb][kd], kd == 0 ? dl : out.d[0][kb]);
                dse(0, 0, k, d0);
                dse(0, 1, k, d0);
                if (kb == 0) issue_load(kd, ld);
                CF_FENCE();
            }
            // Block 1's P words for R2/R3, and delta of (t+1, 1).
            p_words(pbuf, 1, 0, w[0]);
            p_words(pbuf, 1, 1, w[1]);
            dl = delta16(ndbuf, 1);
            CF_HAZARD_FENCE();
            // R2: dK of (t, 0) | dS of (t, 1, 0).
#pragma unroll
            for (int k = 0; k < 2 * NKD; k++) {
                const int o = k >> 1, kb = k & 1;
                if (kb == 0 && o + LA < 2 * NDB) tr[o + LA] = rd_tr(Qs, 0, o + LA);
                if ((k & 3) == 1 && (k >> 2) < LA) orow[k >> 2] = rd_row(On, 1, k >> 2);
                mfma_acc(acc[o >> 1][kb], tr[o], d0[kb][o & 1]);
                dse(1, 0, k, d1);
                // Stores of (t, 0), early in the interval so that they have
                // completed by the barrier's wait.
                if constexpr (WDS) {
                    if ((k & 3) == 2) store_piece(k >> 2);
                }
                CF_FENCE();
            }
            // R3: dP of (t+1, 1) | dS of (t, 1, 1); stores of (t, 1, 0) and
            // the first half of (t, 1, 1).
#pragma unroll
            for (int k = 0; k < 2 * NKD; k++) {
                const int kd = k >> 1, kb = k & 1;
                if (kb == 0 && kd + LA < NKD) orow[kd + LA] = rd_row(On, 1, kd + LA);
                if (k >= 2 * NKD - LA) tr[k - (2 * NKD - LA)] = rd_tr(Qs, 1, k - (2 * NKD - LA));
                out.d[1][kb] = mfma32(orow[kd], xf[kb][kd], kd == 0 ? dl : out.d[1][kb]);
                dse(1, 1, k, d1);
                if constexpr (WDS) {
                    if (k == 2 || k == 6 || k == 10) store_piece(4 + (k >> 2));
                }
                CF_FENCE();
            }
            CF_HAZARD_FENCE();
            // R4: dK of (t, 1); the last store of (t, 1, 1).
#pragma unroll
            for (int k = 0; k < 2 * NKD; k++) {
                const int o = k >> 1, kb = k & 1;
                if (kb == 0 && o + LA < 2 * NDB) tr[o + LA] = rd_tr(Qs, 1, o + LA);
                mfma_acc(acc[o >> 1][kb], tr[o], d1[kb][o & 1]);
                if constexpr (WDS) {
                    if (k == 0) store_piece(7);
                }
                adv(k);
                CF_FENCE();
            }
        };

        // Interval 0: dP - delta of step 0 and this wave's loads of interval
        // 0 (Q of step 2, dO of step 1).
        Pos cur = first, n1 = next_pos(first), n2 = next_pos(n1), n3 = next_pos(n2);
        issue_all(set_loads(n2, 2, n1, 1, 1),
                  std::integral_constant<int, kLoadsDs>{});
        if (pos_act(cur)) dp_of(0, 0, st0);
        // Iteration s runs in interval s + 1, whose loads are Q of step s + 3
        // and dO of step s + 2 (past the last step, the cursors' restarted
        // walk: loaded, unused).
        int qbuf = 0, dbuf = 0;  // buffers of step s
        Loads ld = set_loads(n3, 3, n2, 0, 2);
        const char* dsb = WDS ? ds_row_base(cur) : nullptr;  // stored-dS address of step s (full steps)
        // Part k of moving the bookkeeping above on to the next iteration
        // (spread over the last region's slots in a full iteration).
        auto adv = [&](int s, int k) {
            if (k == 1) {
                cur = n1;
                n1 = n2;
                n2 = n3;
            }
            if (k == 3) n3 = next_pos(n3);
            if (k == 5) {
                qbuf = (qbuf + 1) & 3;
                dbuf = dbuf == 2 ? 0 : dbuf + 1;
            }
            if (k == 7) ld = set_loads(n3, (qbuf + 3) & 3, n2, (s + 1) & 1, dbuf == 2 ? 1 : dbuf == 1 ? 0 : 2);
            if (WDS && k == 9) dsb = ds_row_base(cur);
        };
        // Iterations of the pipelined path: step s is full and step s + 1
        // active, that is s in [s_full0, s_ds1).  Past the run the next step
        // is masked (active: it is the diagonal tile or the cut last tile)
        // unless the run ends the walk.
        const int s_ds1 = s_full1 < n_steps ? s_full1 : s_full1 - 1;
        // Iteration s outside that range: dS of step s from the state in
        // st0, the state of step s + 1 formed in st1 and moved to st0.
        auto masked = [&](int s) {
            step_barrier();
            const int ndbuf = dbuf == 2 ? 0 : dbuf + 1;
            issue_all(ld, std::integral_constant<int, kLoadsDs>{});
            if (pos_act(cur)) ds_dk(cur, qbuf, s & 1, !pos_full(cur), st0);
            if (s + 1 < n_steps && pos_act(n1)) {
                dp_of((s + 1) & 1, ndbuf, st1);
                st0 = st1;
            }
#pragma unroll
            for (int k = 0; k < 2 * NKD; k++) adv(s, k);
        };
        auto full = [&](int s, const DState& in, DState& out) {
            step_barrier();
            const int ndbuf = dbuf == 2 ? 0 : dbuf + 1;
            full_iter(cur, dsb, qbuf, s & 1, (s + 1) & 1, ndbuf, ld, in, out, [&](int k) { adv(s, k); });
        };
        int s = 0;
        for (; s < s_full0; s++) {
            masked(s);
            acc_settle(acc);
        }
        for (; s + 1 < s_ds1; s += 2) {
            full(s, st0, st1);
            full(s + 1, st1, st0);
            acc_settle(acc);
        }
        if (s < s_ds1) {
            full(s, st0, st1);
            acc_settle(acc);
            st0 = st1;
            s++;
        }
        for (; s < n_steps; s++) {
            masked(s);
            acc_settle(acc);
        }
        acc_drain(acc);
        store_rows(p.dk, acc, true);
    };

    // Interval 0 needs Q (and lse) of steps 0 and 1, dO (and delta) of step 0.
    {
        const Loads l0 = set_loads(first, 0, first, 0, 0);
        if (pwave)
            issue_all(l0, std::integral_constant<int, kLoadsP>{});
        else
            issue_all(l0, std::integral_constant<int, kLoadsDs>{});
        const Loads l1 = set_loads(next_pos(first), 1, first, 0, 0);
#pragma unroll
        for (int i = 0; i < BPW; i++) issue_load(i, l1);
        if (wv == 0) issue_load(2 * BPW, l1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (pwave)
        run_p();
    else
        run_ds();
}

void launch_attn_bwd_dkdv_k64(const BwdParams& p, bool wds, hipStream_t st) {
    if (wds)
        hipLaunchKernelGGL((attn_bwd_dkdv_k64_kernel<true>), dim3(p.n_wg_kv), dim3(256), 0, st, p);
    else
        hipLaunchKernelGGL((attn_bwd_dkdv_k64_kernel<false>), dim3(p.n_wg_kv), dim3(256), 0, st, p);
}

}  // namespace cfattn
