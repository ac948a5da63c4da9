// Kernel parameter blocks of the attention kernels, shared by the files that
// launch them (attn_fwd.hip, attn_bwd.hip, attn_f32.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "cfattn_kernels.hpp"

namespace cfattn {

struct FwdParams {
    const void* q;
    const void* k;
    const void* v;
    float* o;
    float* lse;
    int seq, nh, nkv, hd;
    int group, hpw, tpw, n_sub, n_ttiles, n_wg;
    float sl2;  // softmax scale * log2(e)
    long q_bs, kv_bs;
    int vec_ok, o_vec_ok, xcd;
    // Persistent grid of the bf16 kernels and of the fp32 kernel: n_items
    // query tiles, xcd_wgs workgroups per XCD (0: one item per workgroup),
    // walk_gm the walk order (persistent_item).
    int n_items, xcd_wgs, walk_gm;
    // Key split of the fp32 kernel (0: none): a query tile's key tiles are
    // cut into runs of `ksplit`, one workgroup each; `units` workgroups per
    // (sequence, KV head, head subset).  Split s of a row writes its
    // unnormalised O to part[s][row][hd] and (max, sum) to
    // part_ml[s][row], row = (sequence * nh + head) * seq + query.
    int ksplit, units;
    long part_rows;  // batch * nh * seq
    float* part;
    float2* part_ml;
    // Counter of settled wave-tiles (attn_fwd_q64_kernel), null when off.
    unsigned* settles;
};

struct BwdParams {
    const void* d_o;
    const void* q;
    const void* k;
    const void* v;
    const float* o;
    const float* lse;
    float* delta;
    // lse * log2(e) per row (the P recompute's exponent offset, in base 2),
    // written by the delta kernel when set; same layout as delta.
    float* lse2;
    float* dq;
    float* dk;
    float* dv;
    int batch, seq, nh, nkv, hd, group;
    // dK/dV grid; xcd_cus: compute units per XCD, that is the workgroups of
    // one XCD's dispatch round for the one-workgroup-per-CU dK/dV kernels
    int kv_tile, n_kvtiles, n_wg_kv, xcd_cus;
    // dQ grid
    int hpw, tpw, n_sub, n_ttiles, n_wg_q;
    float scale, sl2;
    long q_bs, kv_bs;
    int vec_ok, g_vec_ok, xcd;
    // Stored dS (fast bf16 path only, null otherwise): per (sequence, query
    // head), the 32x32 blocks (query block qi, key block ki <= qi) of the
    // causal triangle, block qi*(qi+1)/2 + ki, 2 KiB each (kDsBlock).
    uint16_t* ds;
    long ds_ntri;  // blocks per (sequence, head)
    // Key split of the fp32 dQ kernel, as FwdParams: split s of a row writes
    // its scaled dQ to qpart[s][row][hd] unless the query tile has one split.
    int ksplit, units_q;
    long part_rows;
    float* qpart;
    // Persistent dQ grid (fp32, and bf16 recompute at head_dim 64): q_items
    // query tiles, q_xcd_wgs workgroups per XCD (0: one unit per workgroup),
    // q_walk_gm the walk order (persistent_item).
    int q_items, q_xcd_wgs, q_walk_gm;
    // Persistent wave-specialised dK/dV grid (head_dim 64): kv_items key
    // tiles, kv_xcd_wgs workgroups per XCD (0: one unit per workgroup),
    // kv_walk_gm the walk order (persistent_item).
    int kv_items, kv_xcd_wgs, kv_walk_gm;
    // Stored fp32 dS (fp32 fast path, null otherwise): per (sequence, query
    // head), the 32x32 blocks (query block qi, key block ki <= qi) of the
    // causal triangle, block qi*(qi+1)/2 + ki, ds_ntri blocks each, 1024
    // floats per block in the dQ kernel's operand order (f32_ds_slot).
    float* ds32;
    // Epilogue of the fast bf16 kernels' dQ and dK rows (BwdEpilogue).
    int epi;
    const float* rope_cos;
    const float* rope_sin;
    int rope_pos0;
    // kEpiUnrotNorm (BwdNorm): pre-norm rows, rstd and gains of q and k;
    // the wave writing dQ rows w of its kernel's grid puts its gain partial
    // in row w of norm_part (w < norm_nq), the wave writing dK rows w in row
    // norm_nq + w (w < norm_nk).
    const float* norm_qx;
    const float* norm_kx;
    const float* norm_qr;
    const float* norm_kr;
    const float* norm_qw;
    const float* norm_kw;
    float* norm_part;
    int norm_nq, norm_nk;
};

// fp32 fast path (attn_f32.hip): head_dim 64 or 128, 16-byte aligned rows.
bool attn_f32_fast_applies(const Dims& d, int vec_ok, int o_vec_ok);
// Scratch of the fp32 dK/dV path: the per-head (and per query split)
// contributions before their fixed-order sum.
size_t attn_f32_scratch_bytes(const Dims& d);
// Scratch of the fp32 forward's key split (0 when the grid needs none).
size_t attn_f32_fwd_scratch_bytes(const Dims& d);
hipError_t launch_attn_fwd_f32(const Dims& d, FwdParams p, void* scratch, size_t scratch_bytes, bool persistent,
                               hipStream_t st, KernelTimer* tm);
// fp32 backward; `scratch` holds scratch_bytes >= attn_f32_scratch_bytes(d):
// with attn_f32_ds_bytes(d) more (after the first attn_f32_scratch_bytes(d)
// rounded up to 256) and `stored_ds`, dK/dV stores dS for the dQ kernel.
hipError_t launch_attn_bwd_f32(const Dims& d, BwdParams p, void* scratch, size_t scratch_bytes, bool persistent,
                               bool stored_ds, hipStream_t st, KernelTimer* tm);
// Bytes of the stored fp32 dS (0 where the fp32 fast path does not apply).
size_t attn_f32_ds_bytes(const Dims& d);
// bf16 dK/dV at head_dim 128, one wave per SIMD (attn_dkdv.hip); with
// `wds` it also stores dS for the stored-dS dQ kernel.  p.kv_tile is 128.
void launch_attn_bwd_dkdv_k64(const BwdParams& p, bool wds, hipStream_t st);
// bf16 forward at head_dim 128, one wave per SIMD (attn_fwd_q64.hip): 16-byte
// aligned rows.  Sets the grid fields of p (heads and query tiles per
// workgroup) itself.
bool attn_fwd_q64_applies(const Dims& d, bool vec_ok, bool o_vec_ok);
hipError_t launch_attn_fwd_q64(const Dims& d, FwdParams p, hipStream_t st, KernelTimer* tm);

}  // namespace cfattn
