// Causal grouped-query attention backward on gfx950 MFMA.
//
// Reference semantics (crates/core/src/ops/attention.rs:142-262): with
// P = exp(s*scale - lse) recomputed from the saved log-sum-exp,
//   dV_g += P^T dO,   dP = dO V^T,   dS = P * (dP - delta) * scale,
//   dQ   += dS K,     dK_g += dS^T Q,   delta_t = sum_d dO[t,d] * O[t,d],
// all accumulated (+=) into the caller's gradients (ops/mod.rs:1-6).
//
// Three kernels, no atomics, so every result is bitwise reproducible:
//   delta: one row reduction per (token, head).
//   dK/dV: a workgroup owns 32*waves keys of one KV head and loops over
//          every query head of its GQA group and every query tile that can
//          see those keys; K and V stay in registers, Q/dO tiles are staged
//          in LDS (row-major for S = Q K^T and dP = dO V^T, transposed for
//          dV^T += dO^T P and dK^T += Q^T dS).  Each dK/dV element is owned
//          by one lane, and its sum over heads and query tiles runs in a
//          fixed order.
//   dQ:    the forward's decomposition (a wave owns 32 queries of one head);
//          K/V tiles in LDS are shared across the heads of the group;
//          S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T.
#include "cfattn_common.hpp"
#include "attn_params.hpp"
#include "cfattn_kernels.hpp"
#include "attn_bwd_common.hpp"

#include <algorithm>

namespace cfattn {

// Eight consecutive values as f32 (16-byte aligned source).
__device__ __forceinline__ void load8(const bf16_bits* g, float* v) {
    const uint4 u = *reinterpret_cast<const uint4*>(g);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}
__device__ __forceinline__ void load8(const float* g, float* v) {
    const float4 a = reinterpret_cast<const float4*>(g)[0], b = reinterpret_cast<const float4*>(g)[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}

// delta[b][h][t] = sum_d dO[b,t,h,d] * O[b,t,h,d]; 16 lanes per row.  With
// head_dim a multiple of 8 and 16-byte aligned rows, lane l sums its runs of
// eight consecutive head dims (8l .. 8l + 7, then + 128) with 16-byte loads;
// otherwise every 16th head dim.  The lanes' sums meet in a fixed shuffle
// tree.
template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(const BwdParams p) {
    const long rows = (long)p.batch * p.seq * p.nh;
    const long row = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
    const int sl = threadIdx.x & 15;
    float acc = 0.0f;
    if (row < rows) {
        const T* g = static_cast<const T*>(p.d_o) + row * p.hd;
        const float* o = p.o + row * p.hd;
        const bool vec = p.hd % 8 == 0 && (((uintptr_t)p.d_o | (uintptr_t)p.o) & 15) == 0;
        if (vec) {
            for (int d = sl * 8; d < p.hd; d += 128) {
                float gv[8], ov[8];
                load8(g + d, gv);
                load8(o + d, ov);
#pragma unroll
                for (int i = 0; i < 8; i++) acc += gv[i] * ov[i];
            }
        } else {
            for (int d = sl; d < p.hd; d += 16) acc += to_f32<T>(g[d]) * o[d];
        }
    }
#pragma unroll
    for (int off = 8; off >= 1; off >>= 1) acc += __shfl_xor(acc, off, 16);
    if (row < rows && sl == 0) {
        const long b = row / ((long)p.seq * p.nh);
        const long t = (row / p.nh) % p.seq;
        const long h = row % p.nh;
        p.delta[(b * p.nh + h) * p.seq + t] = acc;
        if (p.lse2) p.lse2[(b * p.nh + h) * p.seq + t] = p.lse[(b * p.nh + h) * p.seq + t] * kLog2e;
    }
}

template <typename T, int DP, int BM>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_kernel(const BwdParams p) {
    using M = Mode<T>;
    constexpr int EPL = M::EPL;
    constexpr int HALF = DP / 2;
    constexpr int NKD = HALF / EPL;
    constexpr int NDB = DP / 32;
    constexpr int LDQ = RowLD<T, DP>::value;
    constexpr int LDT = TLD<T, BM>::value;
    __shared__ __attribute__((aligned(16))) T sQ[BM * LDQ];
    __shared__ __attribute__((aligned(16))) T sO[BM * LDQ];  // dO rows
    __shared__ __attribute__((aligned(16))) T sQt[DP * LDT];
    __shared__ __attribute__((aligned(16))) T sOt[DP * LDT];  // dO transposed
    __shared__ float sL[BM], sD[BM];

    const int nthreads = blockDim.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int l32 = lane & 31, hh = lane >> 5;

    const int id = xcd_remap(blockIdx.x, p.n_wg_kv, p.xcd);
    const int kvt = id % p.n_kvtiles;  // low key tiles see the most queries: first
    const int rest = id / p.n_kvtiles;
    const int g = rest % p.nkv;
    const int b = rest / p.nkv;
    const int wg_key0 = kvt * p.kv_tile;
    const int key0 = wg_key0 + wave * 32;
    const int kw = key0 + l32;
    const bool wave_active = key0 < p.seq;

    const long qrs = (long)p.nh * p.hd, kvrs = (long)p.nkv * p.hd;
    const T* qg = static_cast<const T*>(p.q) + (long)b * p.q_bs;
    const T* og = static_cast<const T*>(p.d_o) + (long)b * p.q_bs;
    const T* kg = static_cast<const T*>(p.k) + (long)b * p.kv_bs + (long)g * p.hd;
    const T* vg = static_cast<const T*>(p.v) + (long)b * p.kv_bs + (long)g * p.hd;

    // K and V operand rows for key kw, head dims [hh*HALF, hh*HALF+HALF).
    typename M::frag kf[NKD], vf[NKD];
    {
        T raw[HALF];
        load_row_frag<T, HALF>(raw, kg + (long)kw * kvrs, hh * HALF, p.hd, kw < p.seq, p.vec_ok);
#pragma unroll
        for (int kd = 0; kd < NKD; kd++) {
            if constexpr (EPL == 8) {
                Chunk<T> c;
#pragma unroll
                for (int i = 0; i < 8; i++) c.e[i] = raw[kd * 8 + i];
                kf[kd] = __builtin_bit_cast(bf16x8, c.u);
            } else {
                kf[kd] = raw[kd];
            }
        }
        load_row_frag<T, HALF>(raw, vg + (long)kw * kvrs, hh * HALF, p.hd, kw < p.seq, p.vec_ok);
#pragma unroll
        for (int kd = 0; kd < NKD; kd++) {
            if constexpr (EPL == 8) {
                Chunk<T> c;
#pragma unroll
                for (int i = 0; i < 8; i++) c.e[i] = raw[kd * 8 + i];
                vf[kd] = __builtin_bit_cast(bf16x8, c.u);
            } else {
                vf[kd] = raw[kd];
            }
        }
    }

    f32x16 dkt[NDB], dvt[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) {
        dkt[i] = zero16();
        dvt[i] = zero16();
    }

    const int qt_begin = wg_key0 / BM;
    const int n_qt = (p.seq + BM - 1) / BM;
    for (int hi = 0; hi < p.group; hi++) {
        const int h = g * p.group + hi;
        const float* lse_h = p.lse + ((long)b * p.nh + h) * p.seq;
        const float* dlt_h = p.delta + ((long)b * p.nh + h) * p.seq;
        for (int qt = qt_begin; qt < n_qt; qt++) {
            const int q0 = qt * BM;
            const int nrows = min(BM, p.seq - q0);
            __syncthreads();
            const long goff = (long)q0 * qrs + (long)h * p.hd;
            stage_rows<T, BM, DP, LDQ>(sQ, qg + goff, qrs, nrows, p.hd, p.vec_ok, nthreads);
            stage_rows<T, BM, DP, LDQ>(sO, og + goff, qrs, nrows, p.hd, p.vec_ok, nthreads);
            stage_rows_t<T, BM, DP, LDT>(sQt, qg + goff, qrs, nrows, p.hd, p.vec_ok, nthreads);
            stage_rows_t<T, BM, DP, LDT>(sOt, og + goff, qrs, nrows, p.hd, p.vec_ok, nthreads);
            for (int i = threadIdx.x; i < BM; i += nthreads) {
                const bool ok = q0 + i < p.seq;
                // Rows past the sequence get lse = +inf, so P = 0 there.
                sL[i] = ok ? lse_h[q0 + i] * kLog2e : INFINITY;
                sD[i] = ok ? dlt_h[q0 + i] : 0.0f;
            }
            __syncthreads();
            if (!wave_active || q0 + BM - 1 < key0) continue;

#pragma unroll
            for (int qb = 0; qb < BM / 32; qb++) {
                const int tq0 = q0 + qb * 32;
                if (tq0 + 31 < key0 || tq0 >= p.seq) continue;
                // S and dP: rows = queries tq0 + [0,32), columns = this wave's keys.
                f32x16 s = zero16(), dp = zero16();
                const T* qrow = sQ + (qb * 32 + l32) * LDQ + hh * HALF;
                const T* orow = sO + (qb * 32 + l32) * LDQ + hh * HALF;
                if constexpr (EPL == 8) {
#pragma unroll
                    for (int kd = 0; kd < NKD; kd++) {
                        s = mfma32(load_bf16x8(qrow + kd * 8), kf[kd], s);
                        dp = mfma32(load_bf16x8(orow + kd * 8), vf[kd], dp);
                    }
                } else {
#pragma unroll
                    for (int kd = 0; kd < NKD; kd += 4) {
                        const float4 a = *reinterpret_cast<const float4*>(qrow + kd);
                        const float4 c = *reinterpret_cast<const float4*>(orow + kd);
                        s = mfma32(a.x, kf[kd + 0], s);
                        s = mfma32(a.y, kf[kd + 1], s);
                        s = mfma32(a.z, kf[kd + 2], s);
                        s = mfma32(a.w, kf[kd + 3], s);
                        dp = mfma32(c.x, vf[kd + 0], dp);
                        dp = mfma32(c.y, vf[kd + 1], dp);
                        dp = mfma32(c.z, vf[kd + 2], dp);
                        dp = mfma32(c.w, vf[kd + 3], dp);
                    }
                }
                const bool need_mask = tq0 < key0 + 31;
                float pr[16], ds[16];
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int qi = qb * 32 + (r >> 2) * 8 + hh * 4 + (r & 3);
                    float pv = exp2f(s[r] * p.sl2 - sL[qi]);
                    if (need_mask && kw > q0 + qi) pv = 0.0f;
                    pr[r] = pv;
                    ds[r] = pv * (dp[r] - sD[qi]) * p.scale;
                }
                if constexpr (EPL == 8) {
                    const bf16x8 p0 = pack_bf16x8(&pr[0]), p1 = pack_bf16x8(&pr[8]);
                    const bf16x8 d0 = pack_bf16x8(&ds[0]), d1 = pack_bf16x8(&ds[8]);
#pragma unroll
                    for (int db = 0; db < NDB; db++) {
                        const T* ot = sOt + (db * 32 + l32) * LDT + qb * 32 + hh * 4;
                        const T* qt_ = sQt + (db * 32 + l32) * LDT + qb * 32 + hh * 4;
                        dvt[db] = mfma32(load_bf16x4x2(ot, ot + 8), p0, dvt[db]);
                        dvt[db] = mfma32(load_bf16x4x2(ot + 16, ot + 24), p1, dvt[db]);
                        dkt[db] = mfma32(load_bf16x4x2(qt_, qt_ + 8), d0, dkt[db]);
                        dkt[db] = mfma32(load_bf16x4x2(qt_ + 16, qt_ + 24), d1, dkt[db]);
                    }
                } else {
#pragma unroll
                    for (int db = 0; db < NDB; db++) {
                        const T* ot = sOt + (db * 32 + l32) * LDT + qb * 32 + hh * 4;
                        const T* qt_ = sQt + (db * 32 + l32) * LDT + qb * 32 + hh * 4;
#pragma unroll
                        for (int j = 0; j < 4; j++) {
                            const float4 a = *reinterpret_cast<const float4*>(ot + j * 8);
                            const float4 c = *reinterpret_cast<const float4*>(qt_ + j * 8);
                            dvt[db] = mfma32(a.x, pr[j * 4 + 0], dvt[db]);
                            dvt[db] = mfma32(a.y, pr[j * 4 + 1], dvt[db]);
                            dvt[db] = mfma32(a.z, pr[j * 4 + 2], dvt[db]);
                            dvt[db] = mfma32(a.w, pr[j * 4 + 3], dvt[db]);
                            dkt[db] = mfma32(c.x, ds[j * 4 + 0], dkt[db]);
                            dkt[db] = mfma32(c.y, ds[j * 4 + 1], dkt[db]);
                            dkt[db] = mfma32(c.z, ds[j * 4 + 2], dkt[db]);
                            dkt[db] = mfma32(c.w, ds[j * 4 + 3], dkt[db]);
                        }
                    }
                }
            }
        }
    }

    if (!wave_active || kw >= p.seq) return;
    float* dkrow = p.dk + (long)b * p.kv_bs + (long)kw * kvrs + (long)g * p.hd;
    float* dvrow = p.dv + (long)b * p.kv_bs + (long)kw * kvrs + (long)g * p.hd;
#pragma unroll
    for (int db = 0; db < NDB; db++) {
        add_row_block(dkrow, dkt[db], db * 32, hh, p.hd, p.g_vec_ok);
        add_row_block(dvrow, dvt[db], db * 32, hh, p.hd, p.g_vec_ok);
    }
}

template <typename T, int DP, int BN>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(const BwdParams p) {
    using M = Mode<T>;
    constexpr int EPL = M::EPL;
    constexpr int HALF = DP / 2;
    constexpr int NKD = HALF / EPL;
    constexpr int NDB = DP / 32;
    constexpr int NKB = BN / 32;
    constexpr int LDK = RowLD<T, DP>::value;
    constexpr int LDT = TLD<T, BN>::value;
    __shared__ __attribute__((aligned(16))) T sK[BN * LDK];
    __shared__ __attribute__((aligned(16))) T sV[BN * LDK];
    __shared__ __attribute__((aligned(16))) T sKt[DP * LDT];

    const int nthreads = blockDim.x;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int l32 = lane & 31, hh = lane >> 5;

    const int id = xcd_remap(blockIdx.x, p.n_wg_q, p.xcd);
    const int tile = p.n_ttiles - 1 - id % p.n_ttiles;
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
    const bool row_ok = tq < p.seq;

    const long qrs = (long)p.nh * p.hd, kvrs = (long)p.nkv * p.hd;
    const long qoff = (long)b * p.q_bs + (long)tq * qrs + (long)head * p.hd;
    const T* kg = static_cast<const T*>(p.k) + (long)b * p.kv_bs + (long)g * p.hd;
    const T* vg = static_cast<const T*>(p.v) + (long)b * p.kv_bs + (long)g * p.hd;

    typename M::frag qf[NKD], of[NKD];
    {
        T raw[HALF];
        load_row_frag<T, HALF>(raw, static_cast<const T*>(p.q) + qoff, hh * HALF, p.hd, row_ok, p.vec_ok);
#pragma unroll
        for (int kd = 0; kd < NKD; kd++) {
            if constexpr (EPL == 8) {
                Chunk<T> c;
#pragma unroll
                for (int i = 0; i < 8; i++) c.e[i] = raw[kd * 8 + i];
                qf[kd] = __builtin_bit_cast(bf16x8, c.u);
            } else {
                qf[kd] = raw[kd];
            }
        }
        load_row_frag<T, HALF>(raw, static_cast<const T*>(p.d_o) + qoff, hh * HALF, p.hd, row_ok, p.vec_ok);
#pragma unroll
        for (int kd = 0; kd < NKD; kd++) {
            if constexpr (EPL == 8) {
                Chunk<T> c;
#pragma unroll
                for (int i = 0; i < 8; i++) c.e[i] = raw[kd * 8 + i];
                of[kd] = __builtin_bit_cast(bf16x8, c.u);
            } else {
                of[kd] = raw[kd];
            }
        }
    }
    const long lrow = ((long)b * p.nh + head) * p.seq + tq;
    const float lse2 = row_ok ? p.lse[lrow] * kLog2e : INFINITY;
    const float dlt = row_ok ? p.delta[lrow] : 0.0f;

    f32x16 dqt[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) dqt[i] = zero16();

    for (int kt = 0; kt < n_kt; kt++) {
        const int k0 = kt * BN;
        const int nrows = min(BN, p.seq - k0);
        __syncthreads();
        stage_rows<T, BN, DP, LDK>(sK, kg + (long)k0 * kvrs, kvrs, nrows, p.hd, p.vec_ok, nthreads);
        stage_rows<T, BN, DP, LDK>(sV, vg + (long)k0 * kvrs, kvrs, nrows, p.hd, p.vec_ok, nthreads);
        stage_rows_t<T, BN, DP, LDT>(sKt, kg + (long)k0 * kvrs, kvrs, nrows, p.hd, p.vec_ok, nthreads);
        __syncthreads();
        if (!wave_active || k0 > wave_last) continue;
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const int kb0 = k0 + kb * 32;
            if (kb0 > wave_last) continue;
            f32x16 s = zero16(), dp = zero16();
            const T* krow = sK + (kb * 32 + l32) * LDK + hh * HALF;
            const T* vrow = sV + (kb * 32 + l32) * LDK + hh * HALF;
            if constexpr (EPL == 8) {
#pragma unroll
                for (int kd = 0; kd < NKD; kd++) {
                    s = mfma32(load_bf16x8(krow + kd * 8), qf[kd], s);
                    dp = mfma32(load_bf16x8(vrow + kd * 8), of[kd], dp);
                }
            } else {
#pragma unroll
                for (int kd = 0; kd < NKD; kd += 4) {
                    const float4 a = *reinterpret_cast<const float4*>(krow + kd);
                    const float4 c = *reinterpret_cast<const float4*>(vrow + kd);
                    s = mfma32(a.x, qf[kd + 0], s);
                    s = mfma32(a.y, qf[kd + 1], s);
                    s = mfma32(a.z, qf[kd + 2], s);
                    s = mfma32(a.w, qf[kd + 3], s);
                    dp = mfma32(c.x, of[kd + 0], dp);
                    dp = mfma32(c.y, of[kd + 1], dp);
                    dp = mfma32(c.z, of[kd + 2], dp);
                    dp = mfma32(c.w, of[kd + 3], dp);
                }
            }
            const bool need_mask = kb0 + 31 > t_wave;
            float ds[16];
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int key = kb0 + (r >> 2) * 8 + hh * 4 + (r & 3);
                float pv = exp2f(s[r] * p.sl2 - lse2);
                if (need_mask && key > tq) pv = 0.0f;
                ds[r] = pv * (dp[r] - dlt) * p.scale;
            }
            if constexpr (EPL == 8) {
                const bf16x8 d0 = pack_bf16x8(&ds[0]), d1 = pack_bf16x8(&ds[8]);
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    const T* kt_ = sKt + (db * 32 + l32) * LDT + kb * 32 + hh * 4;
                    dqt[db] = mfma32(load_bf16x4x2(kt_, kt_ + 8), d0, dqt[db]);
                    dqt[db] = mfma32(load_bf16x4x2(kt_ + 16, kt_ + 24), d1, dqt[db]);
                }
            } else {
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    const T* kt_ = sKt + (db * 32 + l32) * LDT + kb * 32 + hh * 4;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        const float4 a = *reinterpret_cast<const float4*>(kt_ + j * 8);
                        dqt[db] = mfma32(a.x, ds[j * 4 + 0], dqt[db]);
                        dqt[db] = mfma32(a.y, ds[j * 4 + 1], dqt[db]);
                        dqt[db] = mfma32(a.z, ds[j * 4 + 2], dqt[db]);
                        dqt[db] = mfma32(a.w, ds[j * 4 + 3], dqt[db]);
                    }
                }
            }
        }
    }

    if (!wave_active || !row_ok) return;
    float* dqrow = p.dq + qoff;
#pragma unroll
    for (int db = 0; db < NDB; db++) add_row_block(dqrow, dqt[db], db * 32, hh, p.hd, p.g_vec_ok);
}

// ---------------------------------------------------------------------------
// Fast paths: bf16 inputs, head_dim == DP (64 or 128), 16-byte aligned rows.
// Tiles are staged row-major in double-buffered LDS; every transposed operand
// (dO^T, Q^T, K^T) is read from the row-major tile with ds_read_b64_tr_b16.
// The contraction order over heads and tiles is fixed, so results stay
// bitwise reproducible.

// Waves per workgroup of the fast dQ kernel.  All of them share each K/V
// tile; four (two workgroups per CU) measured faster than eight (one).
constexpr int kDqWaves = 4;
// Waves per workgroup of the stored-dS dQ kernel: more query blocks share
// each K tile, which that kernel streams as many bytes of as it does dS.
constexpr int kDqDsWaves = 8;

// Cache-policy operand of global_load_lds: nt (non-temporal, streamed past
// the caches), for data read exactly once.
constexpr int kCacheNT = 2;
// s_waitcnt vmcnt(N): at most N vector memory operations of this wave still
// outstanding (counts up to 63).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    // gfx9 encoding: vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14;
    // expcnt (bits 6:4) and lgkmcnt (bits 11:8) left at their maximum.
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// dQ: the forward's decomposition (a wave owns 32 queries of one head, NW
// waves per workgroup); K/V tiles of BN keys are shared by the workgroup and
// go straight from global memory into double-buffered blocked LDS tiles
// (global_load_lds, issued one tile ahead by all the waves).  MFMA row i of
// a 32-key block is key qperm(i) of the block (see BlkTile).
// The NORM instance runs the kEpiUnrotNorm epilogue, the other one every
// other mode.
// One query tile (tile `tile` of group rest = (sequence * nkv + KV head) *
// n_sub + head subset); without NORM no LDS read follows its last barrier,
// so the next tile of a persistent workgroup may load into the buffers.
template <int DP, int BN, int NW, bool NORM>
__device__ __forceinline__ void dq_bf16_unit(const BwdParams& p, const int tile, int rest, bf16_bits* sK0,
                                             bf16_bits* sK1, bf16_bits* sV0, bf16_bits* sV1) {
    constexpr int CPR = DP / 8;
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
    const bool row_ok = tq < p.seq;

    const long qrs = (long)p.nh * DP, kvrs = (long)p.nkv * DP;
    const long qoff = (long)b * p.q_bs + (long)tq * qrs + (long)head * DP;
    const bf16_bits* kg = static_cast<const bf16_bits*>(p.k) + (long)b * p.kv_bs + (long)g * DP;
    const bf16_bits* vg = static_cast<const bf16_bits*>(p.v) + (long)b * p.kv_bs + (long)g * DP;

    // Q and -dO operands of the lane's query: the dP^T product accumulates
    // the negated products onto delta, giving delta - dP (as the dK/dV
    // kernels form it, so both dQ paths see the same dS).
    bf16x8 qf[NKD], of[NKD];
    {
        const bf16_bits* qr = static_cast<const bf16_bits*>(p.q) + qoff + hh * HALF;
        const bf16_bits* orr = static_cast<const bf16_bits*>(p.d_o) + qoff + hh * HALF;
#pragma unroll
        for (int kd = 0; kd < NKD; kd++) {
            qf[kd] = __builtin_bit_cast(bf16x8,
                                        row_ok ? *reinterpret_cast<const uint4*>(qr + kd * 8) : make_uint4(0, 0, 0, 0));
            uint4 u = row_ok ? *reinterpret_cast<const uint4*>(orr + kd * 8) : make_uint4(0, 0, 0, 0);
            u.x ^= 0x80008000u, u.y ^= 0x80008000u, u.z ^= 0x80008000u, u.w ^= 0x80008000u;
            of[kd] = __builtin_bit_cast(bf16x8, u);
        }
    }
    const long lrow = ((long)b * p.nh + head) * p.seq + tq;
    const float lse2 = row_ok ? p.lse[lrow] * kLog2e : INFINITY;
    const float dlt = row_ok ? p.delta[lrow] : 0.0f;

    // Row reads (K and V rows, MFMA row l32 = key qperm(l32)) and transposed
    // reads (K^T: tile rows 4k + hh (+2, +16, +18)), as in the forward.
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
    auto dma = [&](int kt, bf16_bits* Kd, bf16_bits* Vd) {
        if ((kt + 1) * BN <= p.seq) {
            const long base = (long)kt * BN * kvrs;
#pragma unroll
            for (int i = 0; i < CPW; i++) {
                const int blk = wv * CPW + i;
                const long off = base + (long)blk * kvrs + lane_off;
                __builtin_amdgcn_global_load_lds(kg + off, Kd + blk * BSTRIDE, 16, 0, 0);
                __builtin_amdgcn_global_load_lds(vg + off, Vd + blk * BSTRIDE, 16, 0, 0);
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

    f32x16 dqt[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) dqt[i] = zero16();

    auto step = [&](int kt, const bf16_bits* Ks, const bf16_bits* Vs, bf16_bits* Kn, bf16_bits* Vn) {
        if (kt + 1 < n_kt) dma(kt + 1, Kn, Vn);
        const int k0 = kt * BN;
        if (wave_active && k0 <= wave_last) {
            // Block kb: S^T = K Q^T and dP^T = V dO^T, then
            // dS^T = P^T (dP^T - delta) * scale and dQ^T += K^T dS^T.
            auto block = [&](int kb, bool masked) {
                // S^T first, then dP^T: P = exp2(...) needs only S^T and runs
                // while the dP^T products are in flight.
                f32x16 sc = zero16(), dp;
#pragma unroll
                for (int r = 0; r < 16; r++) dp[r] = dlt;
#pragma unroll
                for (int kd = 0; kd < NKD; kd++)
                    sc = mfma32(__builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(
                                                             Ks + rrow + kb * 2 * ROW16 + kd * 8)),
                                qf[kd], sc);
#pragma unroll
                for (int kd = 0; kd < NKD; kd++)
                    dp = mfma32(__builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(
                                                             Vs + rrow + kb * 2 * ROW16 + kd * 8)),
                                of[kd], dp);
                const int kb0 = k0 + kb * 32;
                float pr[16];
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    pr[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[r], p.sl2, -lse2));
                    if (masked && kb0 + qperm((r >> 2) * 8 + hh * 4 + (r & 3)) > tq) pr[r] = 0.0f;
                }
                // dS^T = P^T * -(delta - dP^T) without the softmax scale
                // (applied once to dQ), from P rounded to bf16 as the dK/dV
                // kernel forms it, so both dQ paths see the same dS.
                float ds[16];
#pragma unroll
                for (int r = 0; r < 16; r++) ds[r] = (float)(__bf16)pr[r] * -dp[r];
                const bf16x8 d0 = cvt_bf16x8(&ds[0]), d1 = cvt_bf16x8(&ds[8]);
                const bf16_bits* t0 = Ks + trow + kb * 2 * ROW16;
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    const bf16_bits* tp = t0 + db * 32;
                    const bf16x8 a0 = join_bf16x4(ds_read_tr16(tp), ds_read_tr16(tp + 2 * BSTRIDE));
                    const bf16x8 a1 =
                        join_bf16x4(ds_read_tr16(tp + ROW16), ds_read_tr16(tp + ROW16 + 2 * BSTRIDE));
                    dqt[db] = mfma32(a0, d0, dqt[db]);
                    dqt[db] = mfma32(a1, d1, dqt[db]);
                }
            };
            if (k0 + BN - 1 <= t_wave) {
                // Interior tile: every key precedes every query of the wave.
#pragma unroll
                for (int kb = 0; kb < NKB; kb++) block(kb, false);
            } else {
#pragma unroll
                for (int kb = 0; kb < NKB; kb++) {
                    const int kb0 = k0 + kb * 32;
                    if (kb0 > wave_last) break;
                    block(kb, kb0 + 31 > t_wave);
                }
            }
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

    if constexpr (NORM) {
        // Every lane takes part (the row's lane pair, the wave's gain sums).
        // LDS is free (the loop ends with a barrier): wave w stages its q_pre
        // rows in the K or V buffer w.
        const bool ok = wave_active && row_ok;
        const int wu = wave_uniform(wave);
        float* xs = reinterpret_cast<float*>(wu == 0 ? sK0 : wu == 1 ? sK1 : wu == 2 ? sV0 : sV1);
        const long r = ((long)b * p.seq + tq) * p.nh + head;
        stage_norm_row<NDB>(p.norm_qx + (ok ? r : 0) * DP, xs, hh);
#pragma unroll
        for (int db = 0; db < NDB; db++) dqt[db] *= p.scale;
        const float inv = ok ? p.norm_qr[r] : 0.0f;
        float4 cur[NDB][4];
        load_grad_row<NDB>(cur, p.dq + qoff, hh, ok);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        write_grad_row_norm<NDB>(p.dq + qoff, xs, inv, p.norm_qw, dqt, lane, tq, ok, p, cur);
        const int slot = blockIdx.x * NW + wave;
        norm_partial_store<NDB>(dqt, lane, xs, p.norm_part + (long)slot * DP, slot < p.norm_nq);
        return;
    }
    if (!wave_active || !row_ok) return;
#pragma unroll
    for (int db = 0; db < NDB; db++) dqt[db] *= p.scale;  // dS was accumulated without the softmax scale
    write_grad_row<NDB>(p.dq + qoff, dqt, hh, tq, p);
}

template <int DP, int BN, int NW, bool NORM>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_bwd_dq_bf16_kernel(
    const BwdParams p) {
    using L = BlkTile<DP, BN>;
    __shared__ __attribute__((aligned(16))) bf16_bits sK0[L::SIZE];
    __shared__ __attribute__((aligned(16))) bf16_bits sK1[L::SIZE];
    __shared__ __attribute__((aligned(16))) bf16_bits sV0[L::SIZE];
    __shared__ __attribute__((aligned(16))) bf16_bits sV1[L::SIZE];
    if constexpr (!NORM && DP == 64) {
        // Persistent grid at head_dim 64 (the NORM epilogue's gain partials
        // are per workgroup, so that instance keeps one workgroup per tile;
        // at 128 the loop's registers would spill).
        if (p.q_xcd_wgs > 0) {
            int tile, grp;
            for (int it = 0; persistent_item(it, p.q_items / p.n_ttiles, p.n_ttiles, p.q_xcd_wgs, p.q_walk_gm, tile, grp); it++)
                dq_bf16_unit<DP, BN, NW, NORM>(p, tile, grp, sK0, sK1, sV0, sV1);
            return;
        }
    }
    const int id = xcd_remap(blockIdx.x, p.n_wg_q, p.xcd);
    dq_bf16_unit<DP, BN, NW, NORM>(p, p.n_ttiles - 1 - id % p.n_ttiles, id / p.n_ttiles, sK0, sK1, sV0, sV1);
}

// dQ from the stored dS: dQ^T += K^T dS^T over the key blocks at or before
// each wave's 32 queries, with no softmax recompute (one product per key
// block instead of three).  NW waves per workgroup (query heads of one GQA
// group x query blocks, as in attn_bwd_dq_bf16_kernel) share each K tile.
// Both the K tile and each wave's dS blocks (2 KiB each, non-temporal: read
// once) go straight to LDS two tiles ahead, in a three-stage ring.  Two tiles
// in flight (96 KiB per CU) keep the HBM stream busy; one (48 KiB) left it at
// two thirds of the bandwidth.  The loads are issued from inline assembly
// (lds_load16_asm): with the builtin, the compiler's wait-count tracking lost
// the ring's buffers at the loop head and waited for every load before the
// first read.  Each step ends with an exact vmcnt wait and a bare barrier.
// The dS blocks are read transposed: in 16-lane
// group G, lane 4*kk + a supplies the 8-byte piece of key
// 16*(u/2) + 4*kk + 2*(u%2) + hh and rows 16*(G%2) + 4*a.. for read u, so
// lane l ends up with MFMA column l32 (query 32*qi + qperm(l32)) and, for
// each k-index, the key the K^T operand read uses.
// Workgroup barrier without the memory fence of __syncthreads: the caller
// has already waited for exactly the loads and LDS reads the barrier must
// cover.  The empty asm statements keep the compiler from moving memory
// accesses across it.
__device__ __forceinline__ void ring_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// The NORM instance runs the kEpiUnrotNorm epilogue (the Qwen3 norm
// backward, write_grad_row_norm), the other one every other mode.
template <int DP, int BN, int NW, bool NORM>
__global__ __launch_bounds__(64 * NW) void attn_bwd_dq_ds_kernel(const BwdParams p) {
    constexpr int CPR = DP / 8;
    using L = BlkTile<DP, BN>;
    constexpr int CPW = L::NB / NW;  // 1 KiB K loads per wave per tile
    constexpr int BSTRIDE = L::STRIDE, ROW16 = L::ROW16;
    static_assert(L::NB % NW == 0, "tile must split evenly over the waves");
    constexpr int NDB = DP / 32, NKB = BN / 32;
    constexpr int SB = kDsBlock;
    __shared__ __attribute__((aligned(16))) bf16_bits sK0[L::SIZE];
    __shared__ __attribute__((aligned(16))) bf16_bits sK1[L::SIZE];
    __shared__ __attribute__((aligned(16))) bf16_bits sK2[L::SIZE];
    __shared__ __attribute__((aligned(16))) bf16_bits sS0[NW * NKB * SB];
    __shared__ __attribute__((aligned(16))) bf16_bits sS1[NW * NKB * SB];
    __shared__ __attribute__((aligned(16))) bf16_bits sS2[NW * NKB * SB];
    // Direct-to-LDS loads one wave issues per tile (its K blocks and the two
    // halves of each of its dS blocks).
    constexpr int kLoadsPerTile = CPW + 2 * NKB;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int l32 = lane & 31, hh = lane >> 5;

    const int id = xcd_remap(blockIdx.x, p.n_wg_q, p.xcd);
    const int tile = p.n_ttiles - 1 - id % p.n_ttiles;
    int rest = id / p.n_ttiles;
    const int sub = rest % p.n_sub;
    rest /= p.n_sub;
    const int g = rest % p.nkv;
    const int b = rest / p.nkv;

    const int head = g * p.group + sub * p.hpw + wave % p.hpw;
    const int TT = 32 * p.tpw;
    const int t_wave = tile * TT + (wave / p.hpw) * 32;
    const int wg_end = min(p.seq, tile * TT + TT);
    const int n_kt = (wg_end + BN - 1) / BN;
    const bool wave_active = t_wave < p.seq;
    // Query block of the wave; a wave past the end reads block 0 (unused).
    const int qi = wave_active ? t_wave >> 5 : 0;
    const int tq = t_wave + qperm(l32);
    const bool row_ok = wave_active && tq < p.seq;

    const long qrs = (long)p.nh * DP, kvrs = (long)p.nkv * DP;
    const bf16_bits* kg = static_cast<const bf16_bits*>(p.k) + (long)b * p.kv_bs + (long)g * DP;
    // This wave's first stored block (query block qi, key block 0), lane part.
    const bf16_bits* dsg = p.ds + (((long)b * p.nh + head) * p.ds_ntri + (long)qi * (qi + 1) / 2) * SB + lane * 8;

    // K^T reads as in attn_bwd_dq_bf16_kernel: tile rows 4k + hh (+2, +16, +18).
    const int G = lane >> 4, jj = lane & 15;
    const int trow = L::row(4 * (jj >> 2) + hh) + 16 * (G & 1) + 4 * (jj & 3);
    // dS reads (elements): reads u = 0, 2 use srd0 (+128 for u = 2), reads
    // u = 1, 3 use srd1; the XOR of the layout flips the key's bit 1 with G%2.
    const int sc_ = G & 1, kk_ = jj >> 2, a_ = jj & 3;
    const int sbase = sc_ * 64 + 32 * (a_ & 1) + 4 * kk_ + (hh ^ (a_ & 1));
    const int srd0 = (sbase + 2 * sc_) * 8 + (a_ >> 1) * 4;
    const int srd1 = (sbase + 2 * (sc_ ^ 1)) * 8 + (a_ >> 1) * 4;

    // Tile kt: wave w loads K blocks w*CPW.. (lane l of block bk: chunk
    // l % CPR of tile row bk + NB*(l / CPR), keys past the end reading the
    // last key), and its own dS blocks of the tile (blocks past the
    // diagonal reload the diagonal block, unused).
    const int wv = wave_uniform(wave);
    constexpr int NBL = L::NB;
    const int lane_off = NBL * (lane / CPR) * (int)kvrs + (lane % CPR) * 8;
    auto dma = [&](int kt, bf16_bits* Kd, bf16_bits* Sd) {
        if ((kt + 1) * BN <= p.seq) {
            const long base = (long)kt * BN * kvrs;
#pragma unroll
            for (int i = 0; i < CPW; i++) {
                const int blk = wv * CPW + i;
                lds_load16_asm(kg + base + (long)blk * kvrs + lane_off, Kd + blk * BSTRIDE);
            }
        } else {
#pragma unroll
            for (int i = 0; i < CPW; i++) {
                const int blk = wv * CPW + i;
                const int r = blk + L::NB * (lane / CPR);
                const long off = (long)min(kt * BN + r, p.seq - 1) * kvrs + (lane % CPR) * 8;
                lds_load16_asm(kg + off, Kd + blk * BSTRIDE);
            }
        }
#pragma unroll
        for (int kb = 0; kb < NKB; kb++) {
            const bf16_bits* src = dsg + (long)min(kt * NKB + kb, qi) * SB;
            bf16_bits* dst = Sd + (wv * NKB + kb) * SB;
            lds_load16_nt_asm(src, dst);
            lds_load16_nt_asm(src + SB / 2, dst + SB / 2);
        }
    };

    f32x16 dqt[NDB];
#pragma unroll
    for (int i = 0; i < NDB; i++) dqt[i] = zero16();
    // With a += epilogue the lane's dq row part is read here, while the first
    // tiles stream in, instead of as a dependent read at the end.
    float* const dq_row = p.dq + (long)b * p.q_bs + (long)tq * qrs + (long)head * DP;
    float4 dq_pre[NDB][4];
    const bool pre = row_ok && grad_row_prefetch<NDB, NORM>(dq_pre, dq_row, hh, p);

    // Step kt reads buffer kt % 3 and fills buffer (kt + 2) % 3, which the
    // barrier closing step kt - 1 has freed.
    auto step = [&](int kt, const bf16_bits* Ks, const bf16_bits* Ss, bf16_bits* Kn, bf16_bits* Sn) {
        if (kt + 2 < n_kt) dma(kt + 2, Kn, Sn);
        // Key blocks of the tile at or before the wave's query block.
        const int nkb = wave_active ? min(NKB, qi - kt * NKB + 1) : 0;
        if (nkb > 0) {
            const bf16_bits* sw = Ss + wv * NKB * SB;
            auto block = [&](int kb) {
                const bf16_bits* sp = sw + kb * SB;
                const bf16x8 d0 = join_bf16x4(ds_read_tr16(sp + srd0), ds_read_tr16(sp + srd1));
                const bf16x8 d1 = join_bf16x4(ds_read_tr16(sp + srd0 + 128), ds_read_tr16(sp + srd1 + 128));
                const bf16_bits* t0 = Ks + trow + kb * 2 * ROW16;
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    const bf16_bits* tp = t0 + db * 32;
                    const bf16x8 a0 = join_bf16x4(ds_read_tr16(tp), ds_read_tr16(tp + 2 * BSTRIDE));
                    const bf16x8 a1 =
                        join_bf16x4(ds_read_tr16(tp + ROW16), ds_read_tr16(tp + ROW16 + 2 * BSTRIDE));
                    dqt[db] = mfma32(a0, d0, dqt[db]);
                    dqt[db] = mfma32(a1, d1, dqt[db]);
                }
            };
            if (nkb == NKB) {
#pragma unroll
                for (int kb = 0; kb < NKB; kb++) block(kb);
            } else {
#pragma unroll
                for (int kb = 0; kb < NKB; kb++)
                    if (kb < nkb) block(kb);
            }
        }
        // This wave's loads for tile kt + 1 have landed (loads complete in
        // issue order; tile kt + 2's may still be in flight) and its LDS
        // reads of this step are done; then the bare barrier.  (__syncthreads
        // would add a workgroup fence, whose vmcnt(0) also waits for tile
        // kt + 2.)
        if (kt + 2 < n_kt) asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kLoadsPerTile) : "memory");
        else asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        ring_barrier();
    };

    dma(0, sK0, sS0);
    if (n_kt > 1) {
        dma(1, sK1, sS1);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLoadsPerTile) : "memory");
    } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    ring_barrier();
    for (int kt = 0; kt < n_kt; kt += 3) {
        step(kt, sK0, sS0, sK2, sS2);
        if (kt + 1 < n_kt) step(kt + 1, sK1, sS1, sK0, sS0);
        if (kt + 2 < n_kt) step(kt + 2, sK2, sS2, sK1, sS1);
    }

    if constexpr (NORM) {
        // Every lane takes part (the row's lane pair, the wave's gain sums).
        // The ring is free: every wave has passed the loop's last barrier.
        // Wave w stages its q_pre rows in 16 KiB of it: waves 0-5 in the dS
        // buffers, 6 and 7 in the first two K buffers.
        bf16_bits* region = wv == 7 ? sK1 : wv == 6 ? sK0 : wv >= 4 ? sS2 : wv >= 2 ? sS1 : sS0;
        if (wv < 6) region += (wv & 1) * (NW * NKB * SB / 2);
        float* xs = reinterpret_cast<float*>(region);
        const long r = ((long)b * p.seq + tq) * p.nh + head;
        stage_norm_row<NDB>(p.norm_qx + (row_ok ? r : 0) * DP, xs, hh);
#pragma unroll
        for (int db = 0; db < NDB; db++) dqt[db] *= p.scale;
        const float inv = row_ok ? p.norm_qr[r] : 0.0f;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // A row past the end (pre false) writes nothing: dq_pre is unused.
        write_grad_row_norm<NDB>(dq_row, xs, inv, p.norm_qw, dqt, lane, tq, row_ok, p, dq_pre);
        const int slot = blockIdx.x * NW + wave;
        norm_partial_store<NDB>(dqt, lane, xs, p.norm_part + (long)slot * DP, slot < p.norm_nq);
        return;
    }
    if (!row_ok) return;
#pragma unroll
    for (int db = 0; db < NDB; db++) dqt[db] *= p.scale;  // dS was stored without the softmax scale
    if (pre)
        write_grad_row<NDB, true>(dq_row, dqt, hh, tq, p, dq_pre);
    else
        write_grad_row<NDB>(dq_row, dqt, hh, tq, p);
}

// dK/dV with two specialised waves per 32-key slice: eight waves, 128 keys per
// workgroup of one KV head; steps run over (query head of the group, query
// tile of BM rows) in a fixed order, low key tiles (the most queries) first.
//   P waves (0-3) hold K^T and the dV^T accumulators: S = Q K^T,
//     P = exp2(S*scale*log2e - lse*log2e) (causally masked), P to LDS as the
//     bf16 operands of its own dV product (half the bytes of f32),
//     then dV^T += dO^T P.
//   dS waves (4-7) hold V^T and the dK^T accumulators: dP = dO V^T, then with
//     P from LDS dS = P (dP - delta) and dK^T += Q^T dS.
// Wave w and wave w + 4 work on the same keys and share a SIMD, so the
// softmax of one runs while the other issues matrix work, and each needs half
// the registers of a wave doing both.  Two barriers per step: P is written
// before the first and read after it.
// With WDS the dS waves also store each 32x32 block of dS (bf16, the values
// their dK product uses) for attn_bwd_dq_ds_kernel; the layout is given at
// kDsBlock.
// The NORM instance runs the kEpiUnrotNorm epilogue for the dK rows, the
// other one every other mode.
// One key tile (kvt) of group rest = sequence * nkv + KV head, walking its
// query tiles down or up.  Without NORM no LDS read follows the last step's
// barrier, so the next tile of a persistent workgroup may load into the
// buffers.
template <int DP, int BM, bool WDS, bool NORM>
__device__ __forceinline__ void dkdv_ws_unit(const BwdParams& p, const int kvt, const int rest, const bool down,
                                             bf16_bits* sQ0, bf16_bits* sQ1, bf16_bits* sO0, bf16_bits* sO1,
                                             float (*sL)[BM], float (*sD)[BM], uint4 (*sPb)[BM / 32][2][64]) {
    constexpr int NT = 512;
    constexpr int CPR = DP / 8;
    using L = BlkTile<DP, BM>;
    constexpr int CPW = L::NB / 4;  // 1 KiB loads per dS wave per tile
    // Local copies: hipcc's host pass drops the kernel (an undefined launch
    // stub) when a lambda in it names these static members directly.
    constexpr int BSTRIDE = L::STRIDE, ROW16 = L::ROW16;
    static_assert(L::NB % 4 == 0 && 2 * BM <= NT / 2, "tile must split evenly over the four dS waves");
    static_assert(BM % 32 == 0, "query tile must be whole 32-row blocks");
    constexpr int HALF = DP / 2, NKD = HALF / 8, NDB = DP / 32, NQB = BM / 32;

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int slice = wave & 3;
    const bool pwave = wave < 4;
    const int l32 = lane & 31, hh = lane >> 5;

    const int g = rest % p.nkv;
    const int b = rest / p.nkv;
    const int wg_key0 = kvt * p.kv_tile;
    const int key0 = wg_key0 + slice * 32;
    const int kw = key0 + l32;
    const bool wave_active = key0 < p.seq;

    const long qrs = (long)p.nh * DP, kvrs = (long)p.nkv * DP;
    const bf16_bits* qg = static_cast<const bf16_bits*>(p.q) + (long)b * p.q_bs;
    const bf16_bits* og = static_cast<const bf16_bits*>(p.d_o) + (long)b * p.q_bs;

    // Row reads: lane (l32, hh) reads MFMA row l32, chunks hh*NKD + kd.
    const int rrow = L::row(qperm(l32)) + hh * HALF;
    // Transposed reads: in each 16-lane group G, lane 4k + m supplies head
    // dims 16*(G%2) + 4m + [0, 4) of MFMA row 4*hh + k (+8, +16, +24), that
    // is tile row 4k + hh (+2, +16, +18).
    const int G = lane >> 4, jj = lane & 15;
    const int trow = L::row(4 * (jj >> 2) + hh) + 16 * (G & 1) + 4 * (jj & 3);

    // Stored dS: lane l (key l32 of the slice, MFMA rows 4*hh + ...) writes
    // its first eight values to 16-byte slot l ^ hh of the block and the
    // other eight to slot 64 + (l ^ (2 + hh)) (see kDsBlock).
    const int ds_off0 = (lane ^ hh) * 8, ds_off1 = (64 + (lane ^ (2 + hh))) * 8;
    const int ki = key0 >> 5;

    const int n_qt = (p.seq + BM - 1) / BM;
    const int qt_begin = wg_key0 / BM;
    const int nq = n_qt - qt_begin;
    const int n_steps = p.group * nq;
    // Step s covers query head g * group + s % group of query tile
    // n_qt - 1 - s / group (walking down) or qt_begin + s / group (walking
    // up): the order of attn_bwd_dkdv_k64_kernel, whose sums this kernel
    // reproduces bit for bit.
    auto step_q0 = [&](int s) { return (down ? n_qt - 1 - s / p.group : qt_begin + s / p.group) * BM; };
    auto step_h = [&](int s) { return g * p.group + s % p.group; };

    float pl = 0.0f;
    // The dS waves (threads 256..511) load the tiles, lse and delta: they
    // would otherwise wait for the P waves' softmax at the mid-step barrier.
    const int dt = tid - NT / 2;
    // Query of MFMA row i (0 <= i < BM) of a tile.
    const int lrow = (dt % BM & ~31) + qperm(dt & 31);
    // A step's Q and dO rows go straight into the blocked LDS tile: dS wave w fills load
    // blocks w*CPW.., lane l of block b loading chunk l % CPR of tile row
    // b + NB*(l / CPR).  Rows past the end load the last row (finite values);
    // their lse is +inf and delta 0 below, so P = dS = 0 there.
    // The per-lane part of each offset does not change from step to step;
    // a step adds a scalar base (query tile and head).
    const int wd = wave_uniform(wave) - 4;
    constexpr int NBL = L::NB;
    const int lane_off = NBL * (lane / CPR) * (int)qrs + (lane % CPR) * 8;
    auto dma = [&](int s, bf16_bits* Qd, bf16_bits* Od) {
        const int h = step_h(s);
        const int q0 = step_q0(s);
        if (dt < 0) return;
        if (q0 + BM <= p.seq) {
            const long base = (long)q0 * qrs + (long)h * DP;
#pragma unroll
            for (int i = 0; i < CPW; i++) {
                const int blk = wd * CPW + i;
                const long off = base + (long)blk * qrs + lane_off;
                __builtin_amdgcn_global_load_lds(qg + off, Qd + blk * BSTRIDE, 16, 0, 0);
                __builtin_amdgcn_global_load_lds(og + off, Od + blk * BSTRIDE, 16, 0, 0);
            }
        } else {
#pragma unroll
            for (int i = 0; i < CPW; i++) {
                const int blk = wd * CPW + i;
                const int r = blk + L::NB * (lane / CPR);
                const long off = (long)min(q0 + r, p.seq - 1) * qrs + (long)h * DP + (lane % CPR) * 8;
                __builtin_amdgcn_global_load_lds(qg + off, Qd + blk * BSTRIDE, 16, 0, 0);
                __builtin_amdgcn_global_load_lds(og + off, Od + blk * BSTRIDE, 16, 0, 0);
            }
        }
        if (dt >= 0 && dt < 2 * BM) {
            const int t = min(q0 + lrow, p.seq - 1);
            const long li = ((long)b * p.nh + h) * p.seq + t;
            pl = dt < BM ? p.lse[li] : p.delta[li];
        }
    };
    auto store_ld = [&](int s, int st) {
        const int t = step_q0(s) + lrow;
        if (dt < 0) return;
        if (dt < BM)
            sL[st][dt] = t < p.seq ? pl * kLog2e : INFINITY;  // rows past the end: P = 0
        else if (dt < 2 * BM)
            sD[st][dt - BM] = t < p.seq ? pl : 0.0f;
    };

    // Each role runs its own copy of the step loop: the registers one role
    // needs are then not held live across the other role's code.  Both
    // copies pass the same barriers in the same order.
    auto run = [&](auto role) {
        constexpr bool PW = decltype(role)::value;
        // K^T (P waves) or -V^T (dS waves) operand: key kw, head dims
        // hh*HALF + kd*8 + [0, 8).  The dS waves accumulate the negated
        // products onto delta, so their dP product yields delta - dP (the
        // negation is exact, and so it is in the dS rounding below).
        bf16x8 xf[NKD];
        {
            const long off = (long)b * p.kv_bs + (long)kw * kvrs + (long)g * DP + hh * HALF;
            const bf16_bits* xr = static_cast<const bf16_bits*>(PW ? p.k : p.v) + off;
            const bool ok = kw < p.seq;
            const uint32_t sgn = PW ? 0u : 0x80008000u;
#pragma unroll
            for (int kd = 0; kd < NKD; kd++) {
                uint4 u = ok ? *reinterpret_cast<const uint4*>(xr + kd * 8) : make_uint4(0, 0, 0, 0);
                u.x ^= sgn, u.y ^= sgn, u.z ^= sgn, u.w ^= sgn;
                xf[kd] = __builtin_bit_cast(bf16x8, u);
            }
        }
        f32x16 acc[NDB];  // dV^T (P waves) or dK^T (dS waves)
#pragma unroll
        for (int i = 0; i < NDB; i++) acc[i] = zero16();

        auto step = [&](int s, const bf16_bits* Qs, const bf16_bits* Os, bf16_bits* Qn, bf16_bits* On) {
            const int st = s & 1;
            const bool more = s + 1 < n_steps;
            const int q0 = step_q0(s);
            const bool act = wave_active && q0 + BM - 1 >= key0;
            // Every query of the step is past every key of the slice: no mask
            // and no per-block tests.
            const bool full = wave_active && q0 >= key0 + 31 && q0 + BM <= p.seq;
            const float* Ls = sL[st];
            const float* Ds = sD[st];
            // Phase-1 rows (Q for P waves, dO for dS waves) and the phase-2
            // transposed tile (dO^T, Q^T); the role is a compile-time constant,
            // so each names its LDS array directly.
            const bf16_bits* A1 = PW ? Qs : Os;
            const bf16_bits* A2 = PW ? Os : Qs;
            const long ds_head = ((long)b * p.nh + step_h(s)) * p.ds_ntri;
            bf16x8 pbf[NQB][2];  // P waves: P of each block as MFMA operands
            f32x16 dpv[NQB];     // dS waves: delta - dP of each block
            bf16x8 dsv[NQB][2];  // dS waves with WDS: dS of each block, stored after the step
            auto row_read = [&](int qb, int kd) {
                return __builtin_bit_cast(bf16x8,
                                          *reinterpret_cast<const uint4*>(A1 + rrow + qb * 2 * ROW16 + kd * 8));
            };
            // P waves: P = exp2(S*scale*log2e - lse*log2e), causally masked,
            // to LDS in f32 for the dS waves and to registers as bf16 operands.
            // lse of MFMA rows g4*8 + hh*4 + [0, 4) of block qb.
            auto lse4 = [&](int qb, int g4) { return *reinterpret_cast<const float4*>(&Ls[qb * 32 + g4 * 8 + hh * 4]); };
            // Initial accumulator of block qb's product: 0 for S, delta of
            // the lane's MFMA rows g4*8 + hh*4 + [0, 4) for the dS waves.
            auto init16 = [&](int qb) {
                f32x16 c = zero16();
                if constexpr (!PW) {
#pragma unroll
                    for (int g4 = 0; g4 < 4; g4++) {
                        const float4 d4 = *reinterpret_cast<const float4*>(&Ds[qb * 32 + g4 * 8 + hh * 4]);
                        c[g4 * 4 + 0] = d4.x, c[g4 * 4 + 1] = d4.y, c[g4 * 4 + 2] = d4.z, c[g4 * 4 + 3] = d4.w;
                    }
                }
                return c;
            };
            auto p_block = [&](int qb, const f32x16& sc, bool masked, const float4 (&l4s)[4]) {
                float pr[16];
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    const float4 l4 = l4s[g4];
                    const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[g4 * 4 + i], p.sl2, -lv[i]));
                        if (masked && kw > q0 + qb * 32 + qperm(g4 * 8 + hh * 4 + i)) pv = 0.0f;
                        pr[g4 * 4 + i] = pv;
                    }
                }
                pbf[qb][0] = cvt_bf16x8(&pr[0]);
                pbf[qb][1] = cvt_bf16x8(&pr[8]);
                sPb[slice][qb][0][lane] = __builtin_bit_cast(uint4, pbf[qb][0]);
                sPb[slice][qb][1][lane] = __builtin_bit_cast(uint4, pbf[qb][1]);
            };
            // Phase 1: S -> P (P waves) and dP (dS waves).
            if (full) {
                // The softmax's lse values are read before the products, so
                // their latency is not paid once per group of four.
                // (With more than two query blocks the registers are not there:
                // each block's values are read just before its softmax.)
                float4 l4s[NQB][4];
                if constexpr (PW && NQB <= 2) {
#pragma unroll
                    for (int qb = 0; qb < NQB; qb++)
#pragma unroll
                        for (int g4 = 0; g4 < 4; g4++) l4s[qb][g4] = lse4(qb, g4);
                    __builtin_amdgcn_sched_barrier(0);
                }
                f32x16 sc[NQB];
#pragma unroll
                for (int qb = 0; qb < NQB; qb++) sc[qb] = init16(qb);
#pragma unroll
                for (int kd = 0; kd < NKD; kd++)
#pragma unroll
                    for (int qb = 0; qb < NQB; qb++) sc[qb] = mfma32(row_read(qb, kd), xf[kd], sc[qb]);
#pragma unroll
                for (int qb = 0; qb < NQB; qb++) {
                    if constexpr (PW) {
                        if constexpr (NQB > 2)
#pragma unroll
                            for (int g4 = 0; g4 < 4; g4++) l4s[qb][g4] = lse4(qb, g4);
                        p_block(qb, sc[qb], false, l4s[qb]);
                    } else {
                        dpv[qb] = sc[qb];
                    }
                }
            } else if (act) {
#pragma unroll
                for (int qb = 0; qb < NQB; qb++) {
                    const int tq0 = q0 + qb * 32;
                    if (tq0 >= p.seq || tq0 + 31 < key0) continue;
                    f32x16 sc = init16(qb);
#pragma unroll
                    for (int kd = 0; kd < NKD; kd++) sc = mfma32(row_read(qb, kd), xf[kd], sc);
                    if constexpr (PW) {
                        float4 l4s[4];
#pragma unroll
                        for (int g4 = 0; g4 < 4; g4++) l4s[g4] = lse4(qb, g4);
                        p_block(qb, sc, tq0 < key0 + 31, l4s);
                    } else {
                        dpv[qb] = sc;
                    }
                }
            }
            // The dS waves start the next step's loads here, while the P waves
            // finish the softmax; the loads overlap phase 2.  P is published
            // with this wave's LDS writes done and a plain barrier:
            // __syncthreads() would also wait for the loads.
            if constexpr (!PW)
                if (more) dma(s + 1, Qn, On);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            // Phase 2: dV^T += dO^T P (P waves), dS -> dK^T += Q^T dS (dS waves).
            // dS waves: P of MFMA rows g4*8 + hh*4 + [0, 4) of block qb.
            // P is the bf16 value the P wave's dV product used (widening is
            // exact); dS = P (dP - delta) = P * -(delta - dP) then rounds once
            // more, to bf16.
            auto pd4 = [&](int qb, int g4) {
                const uint2 h = reinterpret_cast<const uint2*>(&sPb[slice][qb][g4 >> 1][lane])[g4 & 1];
                return make_float4(__uint_as_float(h.x << 16), __uint_as_float(h.x & 0xffff0000u),
                                   __uint_as_float(h.y << 16), __uint_as_float(h.y & 0xffff0000u));
            };
            auto phase2 = [&](int qb, const float4 (&p4s)[4]) {
                bf16x8 b0, b1;
                if constexpr (PW) {
                    b0 = pbf[qb][0];
                    b1 = pbf[qb][1];
                } else {
                    float ds[16];
#pragma unroll
                    for (int g4 = 0; g4 < 4; g4++) {
                        const float4 p4 = p4s[g4];
                        ds[g4 * 4 + 0] = p4.x * -dpv[qb][g4 * 4 + 0];
                        ds[g4 * 4 + 1] = p4.y * -dpv[qb][g4 * 4 + 1];
                        ds[g4 * 4 + 2] = p4.z * -dpv[qb][g4 * 4 + 2];
                        ds[g4 * 4 + 3] = p4.w * -dpv[qb][g4 * 4 + 3];
                    }
                    b0 = cvt_bf16x8(&ds[0]);
                    b1 = cvt_bf16x8(&ds[8]);
                    if constexpr (WDS) {
                        dsv[qb][0] = b0;
                        dsv[qb][1] = b1;
                    }
                }
                // dO^T (P waves) or Q^T (dS waves), read transposed from the
                // tile: MFMA rows 4hh..+3 and 8+4hh..+3 of the block for b0,
                // 16 more for b1.
                const bf16_bits* t0 = A2 + trow + qb * 2 * ROW16;
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    const bf16_bits* t = t0 + db * 32;
                    const bf16x8 a0 = join_bf16x4(ds_read_tr16(t), ds_read_tr16(t + 2 * BSTRIDE));
                    const bf16x8 a1 =
                        join_bf16x4(ds_read_tr16(t + ROW16), ds_read_tr16(t + ROW16 + 2 * BSTRIDE));
                    acc[db] = mfma32(a0, b0, acc[db]);
                    acc[db] = mfma32(a1, b1, acc[db]);
                }
            };
            if (full) {
                // dS waves read every P value of the step first.
                float4 p4s[NQB][4];
                if constexpr (!PW && NQB <= 2) {
#pragma unroll
                    for (int qb = 0; qb < NQB; qb++)
#pragma unroll
                        for (int g4 = 0; g4 < 4; g4++) p4s[qb][g4] = pd4(qb, g4);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int qb = 0; qb < NQB; qb++) {
                    if constexpr (!PW && NQB > 2)
#pragma unroll
                        for (int g4 = 0; g4 < 4; g4++) p4s[qb][g4] = pd4(qb, g4);
                    phase2(qb, p4s[qb]);
                }
            } else if (act) {
#pragma unroll
                for (int qb = 0; qb < NQB; qb++) {
                    const int tq0 = q0 + qb * 32;
                    if (tq0 >= p.seq || tq0 + 31 < key0) continue;
                    float4 p4s[4];
                    if constexpr (!PW)
#pragma unroll
                        for (int g4 = 0; g4 < 4; g4++) p4s[g4] = pd4(qb, g4);
                    phase2(qb, p4s);
                }
            }
            if constexpr (!PW)
                if (more) store_ld(s + 1, st ^ 1);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's loads for step s + 1 have landed
            __syncthreads();
            // The step's dS goes out only now: stores still in flight at the
            // wait above would hold it up (the wait counts them too); issued
            // here they complete during the next step.  Non-temporal: the
            // 2 KiB blocks are read once, by the dQ kernel, and should not
            // displace the Q/dO tiles in the caches.
            if constexpr (!PW && WDS) {
#pragma unroll
                for (int qb = 0; qb < NQB; qb++) {
                    const int tq0 = q0 + qb * 32;
                    if (full || (act && tq0 < p.seq && tq0 + 31 >= key0)) {
                        const long qi = tq0 >> 5;
                        bf16_bits* blk = p.ds + (ds_head + qi * (qi + 1) / 2 + ki) * kDsBlock;
                        __builtin_nontemporal_store(__builtin_bit_cast(u32x4, dsv[qb][0]),
                                                    reinterpret_cast<u32x4*>(blk + ds_off0));
                        __builtin_nontemporal_store(__builtin_bit_cast(u32x4, dsv[qb][1]),
                                                    reinterpret_cast<u32x4*>(blk + ds_off1));
                    }
                }
            }
        };

        for (int s = 0; s < n_steps; s += 2) {
            step(s, sQ0, sO0, sQ1, sO1);
            if (s + 1 < n_steps) step(s + 1, sQ1, sO1, sQ0, sO0);
        }

        if constexpr (NORM) {
            // Both roles: after this barrier no wave reads the Q/dO tiles,
            // whose buffers the dS waves' epilogue then reuses.
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
        }
        if constexpr (!PW && NORM) {
            {
                // Every lane of the dS wave takes part (the row's lane pair,
                // the wave's gain sums); slice s stages its k_pre rows in
                // buffer s of the Q and dO tiles.
                const bool ok = wave_active && kw < p.seq;
                float* xs = reinterpret_cast<float*>(slice == 0 ? sQ0 : slice == 1 ? sQ1 : slice == 2 ? sO0 : sO1);
                const long r = ((long)b * p.seq + kw) * p.nkv + g;
                stage_norm_row<NDB>(p.norm_kx + (ok ? r : 0) * DP, xs, hh);
#pragma unroll
                for (int db = 0; db < NDB; db++) acc[db] *= p.scale;
                const float inv = ok ? p.norm_kr[r] : 0.0f;
                float4 cur[NDB][4];
                load_grad_row<NDB>(cur, p.dk + r * DP, hh, ok);
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                write_grad_row_norm<NDB>(p.dk + r * DP, xs, inv, p.norm_kw, acc, lane, kw, ok, p, cur);
                const int slot = blockIdx.x * 4 + slice;
                norm_partial_store<NDB>(acc, lane, xs, p.norm_part + (long)(p.norm_nq + slot) * DP, slot < p.norm_nk);
                return;
            }
        }
        if (!wave_active || kw >= p.seq) return;
        float* row = (PW ? p.dv : p.dk) + (long)b * p.kv_bs + (long)kw * kvrs + (long)g * DP;
        if constexpr (PW) {
#pragma unroll
            for (int db = 0; db < NDB; db++) add_row_block(row, acc[db], db * 32, hh, DP, true);
        } else {
#pragma unroll
            for (int db = 0; db < NDB; db++) acc[db] *= p.scale;  // dS was accumulated without the softmax scale
            write_grad_row<NDB>(row, acc, hh, kw, p);
        }
    };

    if (!pwave) {
        dma(0, sQ0, sO0);
        store_ld(0, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (pwave)
        run(RoleTag<true>{});
    else
        run(RoleTag<false>{});
}

template <int DP, int BM, bool WDS, bool NORM>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_bwd_dkdv_ws_kernel(
    const BwdParams p) {
    using L = BlkTile<DP, BM>;
    constexpr int NQB = BM / 32;
    // Query tiles: MFMA row i of block qb is query q0 + 32*qb + qperm(i).
    __shared__ __attribute__((aligned(16))) bf16_bits sQ0[L::SIZE];
    __shared__ __attribute__((aligned(16))) bf16_bits sQ1[L::SIZE];
    __shared__ __attribute__((aligned(16))) bf16_bits sO0[L::SIZE];  // dO rows
    __shared__ __attribute__((aligned(16))) bf16_bits sO1[L::SIZE];
    __shared__ __attribute__((aligned(16))) float sL[2][BM];  // lse * log2(e), by MFMA row
    __shared__ __attribute__((aligned(16))) float sD[2][BM];  // delta, by MFMA row
    // P of each (key slice, query block) as the P waves' bf16 MFMA operands:
    // lane l's eight values of row groups 2h and 2h + 1 (h = 0, 1).
    __shared__ uint4 sPb[4][NQB][2][64];
    if constexpr (!NORM && !WDS && DP == 64) {
        // Persistent grid (head_dim 64): key tile kvt of group grp is unit id
        // grp * n_kvtiles + kvt of the one-workgroup-per-tile grid, and walks
        // the way that grid's workgroup for it does (the same sums).
        if (p.kv_xcd_wgs > 0) {
            int unit, grp;
            for (int it = 0;
                 persistent_item(it, p.kv_items / p.n_kvtiles, p.n_kvtiles, p.kv_xcd_wgs, p.kv_walk_gm, unit, grp);
                 it++) {
                const int kvt = p.n_kvtiles - 1 - unit;
                const int id = grp * p.n_kvtiles + kvt;
                const bool down = ((xcd_local(id, p.kv_items) / p.xcd_cus) & 1) == 0;
                dkdv_ws_unit<DP, BM, WDS, NORM>(p, kvt, grp, down, sQ0, sQ1, sO0, sO1, sL, sD, sPb);
            }
            return;
        }
    }
    const int id = xcd_remap(blockIdx.x, p.n_wg_kv, p.xcd);
    dkdv_ws_unit<DP, BM, WDS, NORM>(p, id % p.n_kvtiles, id / p.n_kvtiles, dkdv_walks_down(blockIdx.x, p.xcd_cus),
                                    sQ0, sQ1, sO0, sO1, sL, sD, sPb);  // low key tiles (the most queries) first
}

static int pick_hpw_b(int group, int cap) {
    for (int h = cap < group ? cap : group; h >= 1; h--)
        if (group % h == 0) return h;
    return 1;
}

template <typename T, int DP>
static hipError_t bwd_dp(const BwdParams& p, hipStream_t st, int kv_waves, int q_waves, KernelTimer* tm) {
    const long rows = (long)p.batch * p.seq * p.nh;
    hipError_t e;
    {
        TimedLaunch tl(tm, kKernBwdDelta, st);
        hipLaunchKernelGGL((attn_bwd_delta_kernel<T>), dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, st, p);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return e;
    constexpr int BM = sizeof(T) == 2 ? 64 : 32;
    {
        TimedLaunch tl(tm, kKernBwdDkdv, st);
        hipLaunchKernelGGL((attn_bwd_dkdv_kernel<T, DP, BM>), dim3(p.n_wg_kv), dim3(64 * kv_waves), 0, st, p);
        e = hipGetLastError();
    }
    if (e != hipSuccess) return e;
    constexpr int BN = sizeof(T) == 2 ? 64 : 32;
    TimedLaunch tl(tm, kKernBwdDq, st);
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, DP, BN>), dim3(p.n_wg_q), dim3(64 * q_waves), 0, st, p);
    return hipGetLastError();
}

size_t attn_bwd_ds_bytes(Dtype dt, const Dims& d) {
    if (dt == kF32) {
        // The slots, then (256-aligned) room for the stored dS; a caller
        // whose limit does not hold that passes the slots alone
        // (attn_f32_scratch_bytes) and dQ recomputes S and dP.
        const size_t slots = attn_f32_scratch_bytes(d), ds = attn_f32_ds_bytes(d);
        return slots && ds ? (slots + 255) / 256 * 256 + ds : slots;
    }
    // head_dim 128 only: at 64 the recompute costs half the matrix work per
    // stored byte and measured faster than the dS round trip through HBM.
    if (dt != kBF16 || d.hd != 128 || d.batch <= 0 || d.seq <= 0) return 0;
    const size_t nqb = ((size_t)d.seq + 31) / 32;
    return (size_t)d.batch * d.nh * (nqb * (nqb + 1) / 2) * kDsBlock * sizeof(bf16_bits);
}

// The fast bf16 kernels' condition (launch_attn_bwd below).
static bool fast_bf16_applies(Dtype dt, const Dims& d, const void* d_o, const void* q, const void* k, const void* v,
                              const float* dq, const float* dk, const float* dv, const Tuning& tu) {
    const uintptr_t al = 16;
    const bool vec_ok = d.hd % 8 == 0 && (uintptr_t)q % al == 0 && (uintptr_t)k % al == 0 &&
                        (uintptr_t)v % al == 0 && (uintptr_t)d_o % al == 0;
    const bool g_vec_ok = d.hd % 4 == 0 && (uintptr_t)dq % al == 0 && (uintptr_t)dk % al == 0 &&
                          (uintptr_t)dv % al == 0;
    return dt == kBF16 && vec_ok && g_vec_ok && (d.hd == 64 || d.hd == 128) && tu.bwd_kv_waves == 0;
}

bool attn_bwd_norm_dk_epilogue(const Dims& d, const Tuning& tu) {
    return !(d.hd == 128 && tu.dkdv_variant != kDkdvWaveSpecialised);
}

size_t attn_bwd_norm_part_floats(const Dims& d, const Tuning& tu) {
    if (d.batch <= 0 || d.seq <= 0 || d.nh <= 0 || d.nkv <= 0 || d.nh % d.nkv != 0) return 0;
    // The fast path's grids (launch_attn_bwd): the larger of the two dQ
    // kernels' wave counts, and the dK waves of either dK/dV kernel.
    const int group = d.nh / d.nkv;
    const int hpw = group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
    const long n_sub = group / hpw;
    long nq = 0;
    for (int waves : {kDqWaves, kDqDsWaves}) {
        const int tpw = waves / hpw;
        const long n_tt = (d.seq + 32L * tpw - 1) / (32L * tpw);
        nq = std::max(nq, n_tt * d.nkv * n_sub * d.batch * waves);
    }
    const long n_wg_kv = (d.seq + 127L) / 128L * d.nkv * d.batch;
    return (size_t)(nq + (attn_bwd_norm_dk_epilogue(d, tu) ? n_wg_kv * 4 : 0)) * d.hd;
}

bool attn_bwd_epilogue_applies(Dtype dt, const Dims& d, const void* d_o, const void* q, const void* k,
                               const void* v, const float* dq, const float* dk, const float* dv, const Tuning& tu) {
    return fast_bf16_applies(dt, d, d_o, q, k, v, dq, dk, dv, tu);
}

hipError_t launch_attn_bwd(Dtype dt, const Dims& d, const void* d_o, const void* q, const void* k, const void* v,
                           const float* o, const float* lse, float* delta, float* dq, float* dk, float* dv,
                           hipStream_t st, const Tuning& tu, void* ds, size_t ds_bytes, const BwdEpilogue* epi) {
    if (d.batch == 0 || d.seq == 0 || d.nh == 0) return hipSuccess;
    const bool fast = fast_bf16_applies(dt, d, d_o, q, k, v, dq, dk, dv, tu);
    // The epilogue reads the cos/sin rows (and with the norm the pre-norm
    // rows and the gains) 16 bytes at a time.
    if (epi && epi->mode != kEpiAdd &&
        (!fast || !epi->cos || !epi->sin ||
         (reinterpret_cast<uintptr_t>(epi->cos) | reinterpret_cast<uintptr_t>(epi->sin)) % 16 != 0))
        return hipErrorInvalidValue;
    const int mode_k = !epi ? kEpiAdd : epi->mode_k < 0 ? epi->mode : epi->mode_k;
    if (epi && mode_k != epi->mode && !(epi->mode == kEpiUnrotNorm && mode_k == kEpiUnrotStore))
        return hipErrorInvalidValue;
    if (mode_k == kEpiUnrotNorm && !attn_bwd_norm_dk_epilogue(d, tu)) return hipErrorInvalidValue;
    if (epi && epi->mode == kEpiUnrotNorm) {
        const BwdNorm& n = epi->norm;
        if (!n.q_x || !n.k_x || !n.q_rstd || !n.k_rstd || !n.qw || !n.kw || !n.dqw || !n.dkw || !n.part ||
            (reinterpret_cast<uintptr_t>(n.q_x) | reinterpret_cast<uintptr_t>(n.k_x) |
             reinterpret_cast<uintptr_t>(n.qw) | reinterpret_cast<uintptr_t>(n.kw) |
             reinterpret_cast<uintptr_t>(n.part)) % 16 != 0)
            return hipErrorInvalidValue;
    }
    BwdParams p{};
    p.d_o = d_o;
    p.q = q;
    p.k = k;
    p.v = v;
    p.o = o;
    p.lse = lse;
    p.delta = delta;
    p.dq = dq;
    p.dk = dk;
    p.dv = dv;
    p.batch = d.batch;
    p.seq = d.seq;
    p.nh = d.nh;
    p.nkv = d.nkv;
    p.hd = d.hd;
    p.group = d.nh / d.nkv;
    const int kv_waves = tu.bwd_kv_waves > 0 ? tu.bwd_kv_waves : 4;
    p.kv_tile = 32 * kv_waves;
    p.n_kvtiles = (d.seq + p.kv_tile - 1) / p.kv_tile;
    long nkv_wg = (long)p.n_kvtiles * d.nkv * d.batch;
    p.hpw = pick_hpw_b(p.group, 4);
    p.tpw = 4 / p.hpw > 0 ? 4 / p.hpw : 1;
    p.n_sub = p.group / p.hpw;
    p.n_ttiles = (d.seq + 32 * p.tpw - 1) / (32 * p.tpw);
    long nq_wg = (long)p.n_ttiles * d.nkv * p.n_sub * d.batch;
    if (nkv_wg > 0x7fffffffL || nq_wg > 0x7fffffffL) return hipErrorInvalidConfiguration;
    p.n_wg_kv = (int)nkv_wg;
    p.n_wg_q = (int)nq_wg;
    p.scale = 1.0f / sqrtf((float)d.hd);  // attention.rs:163
    p.sl2 = p.scale * kLog2e;
    p.q_bs = (long)d.seq * d.nh * d.hd;
    p.kv_bs = (long)d.seq * d.nkv * d.hd;
    const int ch = dt == kBF16 ? 8 : 4;
    const size_t al = 16;
    p.vec_ok = (d.hd % ch == 0) && ((uintptr_t)q % al == 0) && ((uintptr_t)k % al == 0) &&
               ((uintptr_t)v % al == 0) && ((uintptr_t)d_o % al == 0);
    p.g_vec_ok = (d.hd % 4 == 0) && ((uintptr_t)dq % al == 0) && ((uintptr_t)dk % al == 0) && ((uintptr_t)dv % al == 0);
    p.xcd = tu.xcd_remap;
    {
        int dev = 0, cus = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            return hipErrorInvalidDevice;
        p.xcd_cus = cus >= 8 ? cus / 8 : 1;
    }
    if (epi) {
        p.epi = epi->mode;
        p.rope_cos = epi->cos;
        p.rope_sin = epi->sin;
        p.rope_pos0 = epi->pos0;
        if (epi->mode == kEpiUnrotNorm) {
            p.norm_qx = epi->norm.q_x;
            p.norm_kx = epi->norm.k_x;
            p.norm_qr = epi->norm.q_rstd;
            p.norm_kr = epi->norm.k_rstd;
            p.norm_qw = epi->norm.qw;
            p.norm_kw = epi->norm.kw;
            p.norm_part = epi->norm.part;
        }
    }
    if (fast) {
        // Fast paths: the dQ kernel runs kDqWaves waves per workgroup, dK/dV eight.
        p.hpw = p.group % 4 == 0 ? 4 : p.group % 2 == 0 ? 2 : 1;
        p.tpw = kDqWaves / p.hpw;
        p.n_sub = p.group / p.hpw;
        p.n_ttiles = (d.seq + 32 * p.tpw - 1) / (32 * p.tpw);
        nq_wg = (long)p.n_ttiles * d.nkv * p.n_sub * d.batch;
        if (nq_wg > 0x7fffffffL) return hipErrorInvalidConfiguration;
        p.n_wg_q = (int)nq_wg;
        const long rows = (long)p.batch * p.seq * p.nh;
        const bool k64 = d.hd == 128 && tu.dkdv_variant != kDkdvWaveSpecialised;
        // The one-wave-per-SIMD dK/dV kernel reads lse * log2(e) rows, which
        // the delta kernel writes after the delta rows.
        if (k64) p.lse2 = delta + rows;
        const size_t need = attn_bwd_ds_bytes(dt, d);
        const bool use_ds = ds != nullptr && need > 0 && ds_bytes >= need;
        // The stored-dS dQ kernel's grid: kDqDsWaves waves per workgroup, the
        // group's heads x query blocks.
        const int tpw_ds = kDqDsWaves / p.hpw;
        const int n_ttiles_ds = (d.seq + 32 * tpw_ds - 1) / (32 * tpw_ds);
        const long n_wg_ds = (long)n_ttiles_ds * d.nkv * p.n_sub * d.batch;
        if (use_ds && n_wg_ds > 0x7fffffffL) return hipErrorInvalidConfiguration;
        if (p.epi == kEpiUnrotNorm) {
            // One gain partial per wave that writes dQ rows, then per dS wave
            // of the two-waves-per-SIMD dK/dV kernel (four per workgroup)
            // when dK has the norm epilogue too.
            const long nq = use_ds ? n_wg_ds * kDqDsWaves : (long)p.n_wg_q * kDqWaves;
            const long nk = mode_k == kEpiUnrotNorm ? (long)p.n_wg_kv * 4 : 0;
            if (nq + nk > 0x7fffffffL || (size_t)(nq + nk) * d.hd > epi->norm.part_floats) return hipErrorInvalidValue;
            p.norm_nq = (int)nq;
            p.norm_nk = (int)nk;
        }
        hipError_t e;
        {
            TimedLaunch tl(tu.timer, kKernBwdDelta, st);
            hipLaunchKernelGGL((attn_bwd_delta_kernel<bf16_bits>), dim3((unsigned)((rows + 15) / 16)), dim3(256), 0,
                               st, p);
            e = hipGetLastError();
        }
        if (e != hipSuccess) return e;
        if (use_ds) {
            p.ds = static_cast<bf16_bits*>(ds);
            const long nqb = (d.seq + 31) / 32;
            p.ds_ntri = nqb * (nqb + 1) / 2;
        }
        // The dK/dV kernel writes dK rows per mode_k; dQ rows follow `mode`.
        const int epi_q = p.epi;
        p.epi = mode_k;
        {
            TimedLaunch tl(tu.timer, kKernBwdDkdv, st);
            if (k64) {
                launch_attn_bwd_dkdv_k64(p, use_ds, st);
            } else if (d.hd == 128) {
                const dim3 g(p.n_wg_kv), blk(512);
                if (use_ds && mode_k == kEpiUnrotNorm)
                    hipLaunchKernelGGL((attn_bwd_dkdv_ws_kernel<128, 64, true, true>), g, blk, 0, st, p);
                else if (use_ds)
                    hipLaunchKernelGGL((attn_bwd_dkdv_ws_kernel<128, 64, true, false>), g, blk, 0, st, p);
                else if (mode_k == kEpiUnrotNorm)
                    hipLaunchKernelGGL((attn_bwd_dkdv_ws_kernel<128, 64, false, true>), g, blk, 0, st, p);
                else
                    hipLaunchKernelGGL((attn_bwd_dkdv_ws_kernel<128, 64, false, false>), g, blk, 0, st, p);
            } else {
                // Persistent grid (one workgroup per CU) at head_dim 64 when
                // the key tiles fill every CU, up to two per CU, with a group
                // per XCD; not with the norm epilogue (its gain partials are
                // per workgroup).  (C2, 1.5 tiles per CU: 0.170 -> 0.150 ms;
                // C3, 4 per CU: 0.752 -> 0.765 ms, so it keeps the per-tile
                // grid.)
                p.kv_items = p.n_wg_kv;
                p.kv_xcd_wgs = 0;
                const int cus = 8 * p.xcd_cus;
                if (mode_k != kEpiUnrotNorm && tu.bf16_persistent && p.xcd && cus % 8 == 0 &&
                    (long)d.nkv * d.batch >= 8 && p.n_wg_kv >= cus && p.n_wg_kv <= 2L * cus) {
                    p.kv_xcd_wgs = p.xcd_cus;
                    p.n_wg_kv = cus;
                    const int n_qt = (d.seq + 127) / 128, nkvt = p.n_kvtiles;
                    p.kv_walk_gm = persistent_group_major(p.kv_items / nkvt, nkvt, p.kv_xcd_wgs,
                                                          [&](int u) { return (long)(n_qt - (nkvt - 1 - u)); });
                }
                const dim3 g(p.n_wg_kv), blk(512);
                if (mode_k == kEpiUnrotNorm)
                    hipLaunchKernelGGL((attn_bwd_dkdv_ws_kernel<64, 128, false, true>), g, blk, 0, st, p);
                else
                    hipLaunchKernelGGL((attn_bwd_dkdv_ws_kernel<64, 128, false, false>), g, blk, 0, st, p);
            }
            e = hipGetLastError();
        }
        if (e != hipSuccess) return e;
        p.epi = epi_q;
        {
            TimedLaunch tl(tu.timer, kKernBwdDq, st);
            if (use_ds) {
                p.tpw = tpw_ds;
                p.n_ttiles = n_ttiles_ds;
                p.n_wg_q = (int)n_wg_ds;
                if (p.epi == kEpiUnrotNorm)
                    hipLaunchKernelGGL((attn_bwd_dq_ds_kernel<128, 64, kDqDsWaves, true>), dim3(p.n_wg_q),
                                       dim3(64 * kDqDsWaves), 0, st, p);
                else
                    hipLaunchKernelGGL((attn_bwd_dq_ds_kernel<128, 64, kDqDsWaves, false>), dim3(p.n_wg_q),
                                       dim3(64 * kDqDsWaves), 0, st, p);
            } else {
                const bool norm = p.epi == kEpiUnrotNorm;
                // Persistent grid (two workgroups per CU) at head_dim 64 when
                // the tiles fill every workgroup slot with a group per XCD,
                // up to four tiles per slot (as the forward); not with the
                // norm epilogue (its gain partials are per workgroup).
                p.q_items = p.n_wg_q;
                p.q_xcd_wgs = 0;
                if (!norm && d.hd == 64 && tu.bf16_persistent && p.xcd) {
                    int dev = 0, cus = 0;
                    if (hipGetDevice(&dev) != hipSuccess ||
                        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
                        return hipErrorInvalidDevice;
                    if (cus >= 8 && cus % 8 == 0 && (long)d.nkv * p.n_sub * d.batch >= 8 && nq_wg >= 2L * cus &&
                        nq_wg <= 8L * cus) {
                        p.q_xcd_wgs = cus / 8 * 2;
                        p.n_wg_q = 8 * p.q_xcd_wgs;
                        const int tt = 32 * p.tpw, seq = d.seq;
                        p.q_walk_gm = persistent_group_major(
                            p.q_items / p.n_ttiles, p.n_ttiles, p.q_xcd_wgs,
                            [&](int t) { return (long)(std::min(seq, (t + 1) * tt) + 127) / 128; });
                    }
                }
                const dim3 g(p.n_wg_q), blk(64 * kDqWaves);
                if (d.hd == 128 && norm)
                    hipLaunchKernelGGL((attn_bwd_dq_bf16_kernel<128, 64, kDqWaves, true>), g, blk, 0, st, p);
                else if (d.hd == 128)
                    hipLaunchKernelGGL((attn_bwd_dq_bf16_kernel<128, 64, kDqWaves, false>), g, blk, 0, st, p);
                else if (norm)
                    hipLaunchKernelGGL((attn_bwd_dq_bf16_kernel<64, 128, kDqWaves, true>), g, blk, 0, st, p);
                else
                    hipLaunchKernelGGL((attn_bwd_dq_bf16_kernel<64, 128, kDqWaves, false>), g, blk, 0, st, p);
            }
            e = hipGetLastError();
        }
        if (e != hipSuccess || p.epi != kEpiUnrotNorm) return e;
        return launch_norm_gain_reduce(p.norm_part, p.norm_nq, p.norm_nk, d.hd, epi->norm.dqw, epi->norm.dkw, st);
    }
    if (dt == kF32 && attn_f32_fast_applies(d, p.vec_ok, p.g_vec_ok) && tu.bwd_kv_waves == 0 && ds != nullptr &&
        ds_bytes >= attn_f32_scratch_bytes(d)) {
        const long rows = (long)p.batch * p.seq * p.nh;
        {
            TimedLaunch tl(tu.timer, kKernBwdDelta, st);
            hipLaunchKernelGGL((attn_bwd_delta_kernel<float>), dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, st, p);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_attn_bwd_f32(d, p, ds, ds_bytes, tu.f32_persistent != 0, tu.f32_stored_ds != 0, st,
                                   tu.timer);
    }
    const int q_waves = p.hpw * p.tpw;
    const int dp = d.hd <= 32 ? 32 : d.hd <= 64 ? 64 : d.hd <= 128 ? 128 : 256;
    if (dt == kBF16) {
        switch (dp) {
            case 32: return bwd_dp<bf16_bits, 32>(p, st, kv_waves, q_waves, tu.timer);
            case 64: return bwd_dp<bf16_bits, 64>(p, st, kv_waves, q_waves, tu.timer);
            case 128: return bwd_dp<bf16_bits, 128>(p, st, kv_waves, q_waves, tu.timer);
            default: return bwd_dp<bf16_bits, 256>(p, st, kv_waves, q_waves, tu.timer);
        }
    }
    switch (dp) {
        case 32: return bwd_dp<float, 32>(p, st, kv_waves, q_waves, tu.timer);
        case 64: return bwd_dp<float, 64>(p, st, kv_waves, q_waves, tu.timer);
        case 128: return bwd_dp<float, 128>(p, st, kv_waves, q_waves, tu.timer);
        default: return bwd_dp<float, 256>(p, st, kv_waves, q_waves, tu.timer);
    }
}

}  // namespace cfattn
