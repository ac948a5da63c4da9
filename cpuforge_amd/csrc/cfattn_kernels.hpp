// Internal launch interface between the C ABI (cfattn_capi.cpp) and the
// gfx950 kernel files.  Plain structs of device pointers and sizes; all
// tensors are row-major and contiguous:
//   q, o, d_o, dq : [batch][seq][n_heads][head_dim]
//   k, v, dk, dv  : [batch][seq][n_kv][head_dim]
//   lse, delta    : [batch][n_heads][seq]
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace cfattn {

enum Dtype { kF32 = 0, kBF16 = 1 };

struct Dims {
    int batch, seq, nh, nkv, hd;
};

// Kernels a launcher may time (ids are part of the C ABI: cfattn_kernel_name).
enum KernelId {
    kKernFwd = 0,
    kKernBwdDelta = 1,
    kKernBwdDkdv = 2,
    kKernBwdDq = 3,
    kKernProFwd = 4,
    kKernProBwd = 5,
    kNumKernels = 6
};

// Optional per-kernel timing: a launcher brackets each kernel it queues with
// begin/end on the kernel's own stream (the C ABI records hipEvents there).
struct KernelTimer {
    virtual void begin(int kernel, hipStream_t st) = 0;
    virtual void end(int kernel, hipStream_t st) = 0;
    virtual ~KernelTimer() = default;
};

// dK/dV kernel of the bf16 fast path at head_dim 128.
enum DkdvVariant {
    kDkdvAuto = 0,              // one wave per SIMD, 64 keys per wave
    kDkdvWaveSpecialised = 1    // two waves per SIMD, 32 keys per wave (same results, bit for bit)
};

// Forward kernel of the bf16 fast path at head_dim 128.
enum FwdVariant {
    kFwdAuto = 0,        // one wave per SIMD, 64 queries per wave
    kFwdTwoPerSimd = 1   // two waves per SIMD, 32 queries per wave
};

// Walk order of a persistent grid (persistent_item): 1 (group-major) when it
// gives the busiest workgroup at most 2% more work than the unit-major walk,
// else 0.  len(u) is the work of unit u (unit n_units - 1 the longest).
template <class Len>
inline int persistent_group_major(int n_groups, int n_units, int W, Len len) {
    long worst[2] = {0, 0};
    const int q = n_groups / 8, r = n_groups % 8;
    for (int gn : {q, q + 1}) {
        if (gn == 0 || (gn == q + 1 && r == 0)) continue;
        for (int order = 0; order < 2; order++)
            for (int l = 0; l < W; l++) {
                long sum = 0;
                for (int it = 0;; it++) {
                    const long pos = (long)(it >> 1) * 2 * W + ((it & 1) ? 2 * W - 1 - l : l);
                    if (pos >= (long)gn * n_units) break;
                    sum += len(n_units - 1 - (int)(order ? pos % n_units : pos / gn));
                }
                if (sum > worst[order]) worst[order] = sum;
            }
    }
    return worst[1] * 100 <= worst[0] * 102 ? 1 : 0;
}

// Tuning knobs of one launch; defaults are chosen by the launchers.
struct Tuning {
    int xcd_remap = 1;  // XCD-aware workgroup ordering
    int fwd_heads_per_wg = 0;  // 0 = automatic
    int fwd_tblocks_per_wg = 0;
    int bwd_kv_waves = 0;
    int dkdv_variant = kDkdvAuto;
    int fwd_variant = kFwdAuto;
    // The fused backward's Qwen3 norm in the dQ/dK epilogues (kEpiUnrotNorm);
    // 0: the epilogues store the unrotated rows and a separate norm pass runs.
    int norm_epilogue = 1;
    // fp32 kernels: persistent grids (0: one workgroup per work unit; the
    // same bits either way).
    int f32_persistent = 1;
    // fp32 backward: dK/dV stores dS and dQ reads it when the scratch holds
    // it (0: dQ recomputes S and dP; the same bits either way).
    int f32_stored_ds = 1;
    // bf16 two-waves-per-SIMD kernels (forward, recompute dQ, wave-
    // specialised dK/dV): persistent grids (0: one workgroup per unit).
    int bf16_persistent = 1;
    KernelTimer* timer = nullptr;
    // Device counter of the bf16 head_dim-128 forward's settled wave-tiles
    // (the slow path of its row-sum guard), incremented when non-null.
    unsigned* fwd_settles = nullptr;
};

// RAII bracket used by the launchers.
struct TimedLaunch {
    KernelTimer* t;
    int k;
    hipStream_t st;
    TimedLaunch(KernelTimer* t_, int k_, hipStream_t st_) : t(t_), k(k_), st(st_) {
        if (t) t->begin(k, st);
    }
    ~TimedLaunch() {
        if (t) t->end(k, st);
    }
};

// `scratch` is optional: with f32 inputs on small grids the forward splits
// long query tiles over key ranges and merges the parts, which needs
// attn_fwd_scratch_bytes(dt, d) bytes (0: no split for this shape).  Without
// the scratch the grid runs unsplit; both give the same result up to f32
// rounding.
size_t attn_fwd_scratch_bytes(Dtype dt, const Dims& d);
hipError_t launch_attn_fwd(Dtype dt, const Dims& d, const void* q, const void* k, const void* v, float* o,
                           float* lse, hipStream_t st, const Tuning& tu, void* scratch = nullptr,
                           size_t scratch_bytes = 0);

// Backward.  `delta` is caller-provided scratch of batch*n_heads*seq floats.
// dq, dk, dv are accumulated (+=).
//
// `ds` is optional scratch for the stored-dS dQ path: when it is non-null
// and `ds_bytes` >= attn_bwd_ds_bytes(dt, d), and the fast bf16 kernels run,
// the dK/dV kernel writes dS (bf16, causal blocks only) and dQ is one
// product over it instead of a second softmax recompute.  Otherwise dQ
// recomputes S and dP.  Both paths give the same result up to bf16
// rounding of dS, which both apply.  In fp32 the same scratch first holds
// the dK/dV slots (attn_f32_scratch_bytes, the least the fast fp32 path
// takes), then the stored fp32 dS, with which dQ reads dS instead of
// recomputing it (the same bits).
size_t attn_bwd_ds_bytes(Dtype dt, const Dims& d);
size_t attn_f32_scratch_bytes(const Dims& d);
// How the fast bf16 kernels write the dQ and dK rows (dV rows are always
// added).  The inverse-RoPE modes fold the prologue backward's rotation
// (RopeCache::apply with inverse = true, rope.rs:71-89) into the kernels:
// row t of a sequence is unrotated with cos/sin row pos0 + t of the
// [max_pos][head_dim/2] tables, elementwise as the prologue backward does.
enum EpilogueMode {
    kEpiAdd = 0,          // dq/dk += rows
    kEpiUnrotAdd = 1,     // dq/dk += inverse-RoPE(rows)
    kEpiUnrotStore = 2,   // dq/dk  = inverse-RoPE(rows), every row written once
    kEpiUnrotNorm = 3     // dq/dk += RMSNorm-backward(inverse-RoPE(rows)), gain gradients += their row sums
};
// kEpiUnrotNorm's operands (the Qwen3 per-head q/k norm, layer.rs:195-206):
// the pre-norm rows (the gradient rows' layout), their rstd, the gains
// ([head_dim] each, accumulated into dqw/dkw), and scratch for the per-wave
// gain-gradient partial sums of attn_bwd_norm_part_floats floats.
struct BwdNorm {
    const float* q_x = nullptr;
    const float* k_x = nullptr;
    const float* q_rstd = nullptr;
    const float* k_rstd = nullptr;
    const float* qw = nullptr;
    const float* kw = nullptr;
    float* dqw = nullptr;
    float* dkw = nullptr;
    float* part = nullptr;
    size_t part_floats = 0;
};
struct BwdEpilogue {
    int mode = kEpiAdd;
    // The dK rows' mode: -1 for `mode`; with kEpiUnrotNorm also
    // kEpiUnrotStore (the dK/dV kernel stores the unrotated rows into dk, and
    // their norm backward is left to the caller) -- the only choice where the
    // dK/dV kernel has no norm epilogue (attn_bwd_norm_dk_epilogue).
    int mode_k = -1;
    const float* cos = nullptr;
    const float* sin = nullptr;
    int pos0 = 0;
    BwdNorm norm;
};
// True when launch_attn_bwd takes the fast bf16 kernels for these operands,
// the only ones that honour a BwdEpilogue other than kEpiAdd.
bool attn_bwd_epilogue_applies(Dtype dt, const Dims& d, const void* d_o, const void* q, const void* k,
                               const void* v, const float* dq, const float* dk, const float* dv, const Tuning& tu);
// Whether the fast dK/dV kernel for d has the norm epilogue: the
// two-waves-per-SIMD kernel does; the one-wave-per-SIMD kernel (head_dim
// 128), whose registers are all taken by its step loop, does not.
bool attn_bwd_norm_dk_epilogue(const Dims& d, const Tuning& tu);
// Scratch floats a kEpiUnrotNorm backward needs for its gain-gradient
// partials (one head_dim row per wave that writes dQ rows, or dK rows with
// the norm epilogue), for either dQ kernel.
size_t attn_bwd_norm_part_floats(const Dims& d, const Tuning& tu);
// The fixed-order reduction of the partials (prologue.hip): dqw[i] += the sum
// over rows [0, nq) of part[.][i], dkw[i] over rows [nq, nq + nk).
hipError_t launch_norm_gain_reduce(float* part, int nq, int nk, int hd, float* dqw, float* dkw, hipStream_t st);
// With f32 inputs the same scratch (when large enough) holds the per-head
// dK/dV contributions of the fp32 fast path (attn_f32.hip), which
// attn_bwd_ds_bytes reports for kF32.
// A non-default `epi` needs attn_bwd_epilogue_applies and 16-byte aligned
// cos/sin tables; kEpiUnrotNorm also 16-byte aligned pre-norm rows and gains
// and part_floats >= attn_bwd_norm_part_floats (hipErrorInvalidValue
// otherwise).  `delta` is scratch of 2 * batch * n_heads * seq floats: the
// delta rows, then (head_dim 128, bf16) the lse * log2(e) rows.
hipError_t launch_attn_bwd(Dtype dt, const Dims& d, const void* d_o, const void* q, const void* k, const void* v,
                           const float* o, const float* lse, float* delta, float* dq, float* dk, float* dv,
                           hipStream_t st, const Tuning& tu, void* ds = nullptr, size_t ds_bytes = 0,
                           const BwdEpilogue* epi = nullptr);

// Attention prologue: optional per-head RMSNorm of q_pre/k_pre (when qw/kw
// are non-null) followed by rotate-half RoPE at positions pos0+t, written in
// the compute dtype.  rstd outputs are written only with the norm.
struct Prologue {
    const float* cos;  // [max_pos][head_dim/2]
    const float* sin;
    int max_pos;
    int pos0;
    const float* qw;  // [head_dim] or null
    const float* kw;
    float eps;
};
hipError_t launch_prologue_fwd(Dtype dt, const Dims& d, const Prologue& pr, const float* q_pre, const float* k_pre,
                               void* q_out, void* k_out, float* q_rstd, float* k_rstd, hipStream_t st,
                               KernelTimer* timer = nullptr);

// Prologue backward: inverse RoPE of dq/dk, then (with the norm) RMSNorm
// backward.  dq_pre/dk_pre and dqw/dkw are accumulated.  `partial` is
// scratch of prologue_bwd_scratch_floats(d) floats (unused without norm).
size_t prologue_bwd_scratch_floats(const Dims& d);
// With `unrotated`, dq/dk already hold the inverse-RoPE'd gradients (a
// kEpiUnrotStore backward) and only the norm backward runs (pr.qw/kw set).
// With `k_only`, only the k rows (the q arguments are not used).
hipError_t launch_prologue_bwd(const Dims& d, const Prologue& pr, const float* dq, const float* dk,
                               const float* q_pre, const float* k_pre, const float* q_rstd, const float* k_rstd,
                               float* dq_pre, float* dk_pre, float* dqw, float* dkw, float* partial, hipStream_t st,
                               KernelTimer* timer = nullptr, bool unrotated = false, bool k_only = false);

// Elementwise helpers.
hipError_t launch_f32_to_bf16(const float* src, uint16_t* dst, size_t n, hipStream_t st);
hipError_t launch_fill_zero(float* dst, size_t n, hipStream_t st);

// Largest head_dim the kernels take.
constexpr int kMaxHeadDim = 256;

// Fixed per-device scratch of the entry points that allocate nothing
// (noalloc.hip).  16 MiB: the backward's delta rows and lse * log2(e) rows,
// 2*batch*n_heads*seq floats, up to 2^21 rows of each.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
// Looks up the scratch array's address on `device`, which must be current;
// idempotent per device.
hipError_t noalloc_init_device(int device);
// The address noalloc_init_device found for `device`, or null before it.
void* noalloc_scratch(int device);

// Matrix-pipe throughput probe (probe.hip): `iters` loop iterations of 16
// bf16 32x32x16 MFMAs per wave, two waves per SIMD on every CU, on
// pseudo-random operands (zeros = 0) or zero operands; waits for the run and
// returns its TFLOP/s.
hipError_t probe_mfma_bf16(hipStream_t st, int zeros, int iters, double* tflops);
// LDS-read (kProbeLds: bytes/s) or v_fma_f32 (kProbeValu: lane operations/s)
// loop of `iters` iterations, four waves per SIMD on every CU, or a bf16
// 16x16x32 MFMA loop (kProbeMfma16: FLOP/s, two waves per SIMD); waits for
// the run and returns its rate.
enum ProbeKind { kProbeLds = 0, kProbeValu = 1, kProbeMfma16 = 2 };
hipError_t probe_loop(hipStream_t st, int kind, int iters, double* rate);

}  // namespace cfattn
