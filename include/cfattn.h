/*
 * cfattn -- MI355X (gfx950) causal grouped-query attention for cpuforge.
 *
 * C ABI of libcfattn.so: plain pointers, sizes and integer status codes.
 * Every entry point names the reference interface it replaces
 * (paths under the reference repository's crates/).
 *
 * Layouts are the reference's (crates/core/src/ops/attention.rs:1-6), row-major:
 *   q, o, d_o, dq : [seq, n_heads, head_dim]
 *   k, v, dk, dv  : [seq, n_kv, head_dim]
 *   lse           : [n_heads, seq]
 * Device entry points take `batch` independent sequences stacked in front
 * ([batch, seq, ...], lse [batch, n_heads, seq]); the reference's trainer
 * runs the same sequences one call at a time (train/src/trainer.rs:147-169).
 *
 * Conventions kept from the reference:
 *   - forward OVERWRITES o and lse; backward ACCUMULATES (+=) into dq, dk,
 *     dv (core/src/ops/mod.rs:1-6);
 *   - query head h reads KV head h / (n_heads / n_kv) (attention.rs:61,66);
 *   - every shape check the reference asserts is an error return here,
 *     with a message from cfattn_last_error() (attention.rs:35-38, 55-58,
 *     155-158);
 *   - results do not depend on q_block (attention.rs:336-354); the
 *     *_blocked entry points accept it and validate it only.
 * Limits of this implementation: 1 <= head_dim <= 256; seq * n_heads *
 * head_dim and batch * seq * n_heads below 2^31.
 */
#ifndef CFATTN_H
#define CFATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Mirrors `AttnShape` (core/src/ops/attention.rs:20-26). */
typedef struct cfattn_shape {
    size_t seq;
    size_t n_heads;
    size_t n_kv;
    size_t head_dim;
} cfattn_shape;

/* Mirrors `Llama3Scaling` (core/src/ops/rope.rs:16-22). */
typedef struct cfattn_llama3_scaling {
    double factor;
    double low_freq_factor;
    double high_freq_factor;
    double original_max_position;
} cfattn_llama3_scaling;

/* The attention prologue of Layer::forward (model/src/layer.rs:104-116): an
 * optional per-head RMSNorm of q/k (Qwen3, model/src/config.rs:83-85) and
 * RoPE with a cos/sin table as built by cfattn_rope_table.  All pointers are
 * device pointers. */
typedef struct cfattn_prologue {
    const float* cos;     /* [max_pos, head_dim/2] */
    const float* sin;     /* [max_pos, head_dim/2] */
    size_t max_pos;
    size_t pos0;          /* position of token 0; Layer::forward uses 0 */
    const float* q_norm;  /* [head_dim] gains, or NULL for no q/k norm */
    const float* k_norm;  /* [head_dim] gains, or NULL */
    float eps;            /* rms_norm_eps */
} cfattn_prologue;

typedef struct cfattn_ctx cfattn_ctx;

enum {
    CFATTN_F32 = 0,  /* fp32 inputs, fp32 MFMA (parity mode) */
    CFATTN_BF16 = 1  /* bf16 inputs (raw 16-bit patterns), fp32 accumulation */
};

enum {
    CFATTN_OK = 0,
    CFATTN_ERR_SHAPE = 1,        /* a reference assert would have fired */
    CFATTN_ERR_ARG = 2,          /* NULL pointer, bad dtype, bad context */
    CFATTN_ERR_UNSUPPORTED = 3,  /* outside the documented limits */
    CFATTN_ERR_HIP = 4,          /* HIP runtime error (message has details) */
    CFATTN_ERR_NOMEM = 5,        /* device allocation failed */
    CFATTN_ERR_IO = 6            /* file I/O failed or the file is malformed (cfio.h) */
};

/* ---- context ------------------------------------------------------------ */
/* Creates a context on HIP device `device`: its own stream (used by the
 * host-slice entry points), a grow-only pool of device buffers for them, and
 * scratch.  Calls on one context are serialised by a lock. */
int cfattn_create(int device, cfattn_ctx** out);
int cfattn_destroy(cfattn_ctx* ctx);
/* Message of the last failed call on this context (empty if none). */
const char* cfattn_last_error(const cfattn_ctx* ctx);
/* Arithmetic of the host-slice entry points below: CFATTN_F32 (default) or
 * CFATTN_BF16 (inputs rounded to bf16 on the device, fp32 accumulation). */
int cfattn_set_mode(cfattn_ctx* ctx, int dtype);
int cfattn_get_mode(const cfattn_ctx* ctx);
/* Blocks until all work queued on the context's stream has finished. */
int cfattn_synchronize(cfattn_ctx* ctx);
/* The context's stream (a hipStream_t). */
void* cfattn_stream(cfattn_ctx* ctx);

/* ---- host slices: drop-in for the reference's functions ----------------- */
/* Replaces attention_forward (core/src/ops/attention.rs:42-44).  Host f32
 * buffers; lengths are element counts checked like the reference's asserts.
 * Blocks until o and lse are written. */
int cfattn_attention_forward(cfattn_ctx* ctx, const float* q, size_t q_len, const float* k, size_t k_len,
                             const float* v, size_t v_len, float* o, size_t o_len, float* lse, size_t lse_len,
                             cfattn_shape s);
/* Replaces attention_forward_blocked (attention.rs:46-54). q_block > 0. */
int cfattn_attention_forward_blocked(cfattn_ctx* ctx, const float* q, size_t q_len, const float* k, size_t k_len,
                                     const float* v, size_t v_len, float* o, size_t o_len, float* lse,
                                     size_t lse_len, cfattn_shape s, size_t q_block);
/* Replaces attention_backward (attention.rs:126-139): accumulates into
 * dq, dk, dv. */
int cfattn_attention_backward(cfattn_ctx* ctx, const float* d_o, size_t d_o_len, const float* q, size_t q_len,
                              const float* k, size_t k_len, const float* v, size_t v_len, const float* o,
                              size_t o_len, const float* lse, size_t lse_len, float* dq, size_t dq_len, float* dk,
                              size_t dk_len, float* dv, size_t dv_len, cfattn_shape s);
/* Replaces attention_backward_blocked (attention.rs:142-154). */
int cfattn_attention_backward_blocked(cfattn_ctx* ctx, const float* d_o, size_t d_o_len, const float* q,
                                      size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len,
                                      const float* o, size_t o_len, const float* lse, size_t lse_len, float* dq,
                                      size_t dq_len, float* dk, size_t dk_len, float* dv, size_t dv_len,
                                      cfattn_shape s, size_t q_block);

/* ---- device pointers, batched, caller's stream -------------------------- */
/* Forward on device buffers.  q, k, v are f32 or bf16 (`dtype`); o and lse
 * are f32.  `stream` is a hipStream_t; NULL is the device's null (default)
 * stream, as in every HIP API (pass cfattn_stream(ctx) for the context's own
 * stream).  Asynchronous: returns after queuing the kernels. */
int cfattn_fwd(cfattn_ctx* ctx, cfattn_shape s, size_t batch, int dtype, const void* q, const void* k,
               const void* v, float* o, float* lse, void* stream);
/* Backward on device buffers; accumulates into the f32 dq, dk, dv.  Uses
 * batch*n_heads*seq floats of context scratch: calls on one context must not
 * overlap on different streams. */
int cfattn_bwd(cfattn_ctx* ctx, cfattn_shape s, size_t batch, int dtype, const void* d_o, const void* q,
               const void* k, const void* v, const float* o, const float* lse, float* dq, float* dk, float* dv,
               void* stream);

/* No reference counterpart.  cfattn_bwd that allocates nothing, for callers
 * that cannot call hipMalloc (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation).  The same arguments, results and
 * accumulation as cfattn_bwd; its only scratch (the delta and lse*log2(e)
 * rows, 2*batch*n_heads*seq floats) is a fixed 16 MiB device array of the
 * library, one per device, so batch*n_heads*seq must not exceed 2^21
 * (CFATTN_ERR_UNSUPPORTED otherwise).
 * It never stores dS: in bf16, dQ recomputes the softmax (equal to
 * cfattn_bwd with cfattn_set_ds_limit(ctx, 0)); in f32 it runs the generic
 * kernels.  Calls that overlap on one device race on the shared array. */
int cfattn_bwd_noalloc(cfattn_ctx* ctx, cfattn_shape s, size_t batch, int dtype, const void* d_o, const void* q,
                       const void* k, const void* v, const float* o, const float* lse, float* dq, float* dk,
                       float* dv, void* stream);

/* ---- fused prologue ------------------------------------------------------ */
/* Layer::forward's prologue (model/src/layer.rs:104-116): from f32 q_pre
 * [batch, seq, n_heads, D] and k_pre [batch, seq, n_kv, D] writes q_out and
 * k_out in `dtype`, plus q_rstd [batch*seq*n_heads] and k_rstd
 * [batch*seq*n_kv] when the norm is on (may be NULL otherwise).  In f32 the
 * outputs equal rmsnorm_forward + RopeCache::apply bit for bit. */
int cfattn_prologue_fwd(cfattn_ctx* ctx, cfattn_shape s, size_t batch, int dtype, const cfattn_prologue* pr,
                        const float* q_pre, const float* k_pre, void* q_out, void* k_out, float* q_rstd,
                        float* k_rstd, void* stream);
/* Layer::backward's chain after attention (model/src/layer.rs:191-206): from
 * dq, dk (gradients of the post-prologue q, k) accumulates dq_pre, dk_pre
 * and, with the norm, the gain gradients dq_norm, dk_norm ([head_dim]). */
int cfattn_prologue_bwd(cfattn_ctx* ctx, cfattn_shape s, size_t batch, const cfattn_prologue* pr, const float* dq,
                        const float* dk, const float* q_pre, const float* k_pre, const float* q_rstd,
                        const float* k_rstd, float* dq_pre, float* dk_pre, float* dq_norm, float* dk_norm,
                        void* stream);
/* Prologue + attention forward in one call (Layer::forward's
 * q_pre/k_pre -> attn_o, lse).  q_out/k_out keep the post-prologue q/k the
 * backward needs (LayerCache.q/k, model/src/layer.rs:65-86). */
int cfattn_fused_fwd(cfattn_ctx* ctx, cfattn_shape s, size_t batch, int dtype, const cfattn_prologue* pr,
                     const float* q_pre, const float* k_pre, const void* v, void* q_out, void* k_out, float* q_rstd,
                     float* k_rstd, float* o, float* lse, void* stream);
/* Attention backward + prologue backward in one call (Layer::backward from
 * d_attn_o to dq_pre/dk_pre, dv and the norm gains' gradients).  All
 * gradients are accumulated. */
int cfattn_fused_bwd(cfattn_ctx* ctx, cfattn_shape s, size_t batch, int dtype, const cfattn_prologue* pr,
                     const void* d_o, const float* q_pre, const float* k_pre, const void* q, const void* k,
                     const void* v, const float* o, const float* lse, const float* q_rstd, const float* k_rstd,
                     float* dq_pre, float* dk_pre, float* dv, float* dq_norm, float* dk_norm, void* stream);

/* ---- host helpers ---------------------------------------------------------- */
/* RopeCache::with_scaling (core/src/ops/rope.rs:46-63): cos/sin tables
 * [max_pos, head_dim/2] computed in double and rounded to float, into host
 * buffers.  scaling may be NULL (plain RoPE).  head_dim must be even. */
int cfattn_rope_table(size_t head_dim, size_t max_pos, double theta, const cfattn_llama3_scaling* scaling,
                      float* cos_out, float* sin_out);
/* Llama3Scaling::apply (core/src/ops/rope.rs:26-38). */
double cfattn_llama3_scale(const cfattn_llama3_scaling* scaling, double inv_freq);
/* Device f32 -> bf16 (round to nearest even) conversion on `stream`. */
int cfattn_f32_to_bf16(cfattn_ctx* ctx, const float* src, uint16_t* dst, size_t n, void* stream);
/* ---- backward scratch ---------------------------------------------------- */
/* No reference counterpart (the reference's backward recomputes everything
 * per query block, attention.rs:142-262).  Limit, in bytes, of the device
 * scratch the bf16 backward (head_dim 64 or 128) may keep in the context's
 * pool to store dS: bf16 values of the causal 32x32 blocks,
 * batch * n_heads * nb*(nb+1)/2 * 2 KiB with nb = ceil(seq/32) (2.2 GB at
 * seq 8192, 32 heads).  With it, dQ is one product over the stored dS instead
 * of a second softmax recompute; results agree to bf16 rounding of dS, which
 * both paths apply.  Larger shapes, or limit 0, use the recompute.  The same
 * limit bounds the f32 path's scratch: the backward's per-head dK/dV and
 * key-split dQ parts (without it the f32 backward takes the generic kernels)
 * and the forward's key-split parts on small grids (without it the forward
 * runs unsplit; results agree to f32 rounding).  Lowering the limit below
 * the kept scratch frees it.  Default: 8 GiB. */
int cfattn_set_ds_limit(cfattn_ctx* ctx, size_t bytes);
size_t cfattn_get_ds_limit(const cfattn_ctx* ctx);

/* ---- measurement ----------------------------------------------------------- */
/* No reference counterpart: the reference times whole steps with a wall clock
 * (cli/src/cmd_bench.rs:13-22).  While enabled, every kernel this context
 * queues is bracketed by two hipEvents on the kernel's stream; enabling
 * again resets the totals.  Disable with on = 0. */
int cfattn_profile_enable(cfattn_ctx* ctx, int on);
/* Which kernels profiling brackets: bit k of kernel_mask for kernel id k
 * (default: all).  Applies at once and to later profiling sessions; a
 * kernel left out costs no events (each bracket adds a few microseconds of
 * queue time to a step). */
int cfattn_profile_select(cfattn_ctx* ctx, unsigned kernel_mask);
/* Waits for the recorded launches and returns, for kernel id `kernel`
 * (0 .. cfattn_kernel_count()-1), the summed event time in milliseconds and
 * the number of launches since profiling was enabled. */
int cfattn_profile_read(cfattn_ctx* ctx, int kernel, double* total_ms, long long* launches);
/* No reference counterpart: counts the wave-tiles on which the bf16
 * head_dim-128 forward takes the slow path of its row-sum guard (exact row
 * max, lazy rescale, P formed again; the first key tile of every wave always
 * takes it).  Enabling allocates and zeroes a device counter; forward calls
 * of this context then add to it, whatever stream they run on.  Off (on = 0)
 * frees it.  For measurement: the count costs one atomic per settled
 * wave-tile. */
int cfattn_fwd_stats_enable(cfattn_ctx* ctx, int on);
/* Waits for the device and returns the count since enabling. */
int cfattn_fwd_stats_read(cfattn_ctx* ctx, long long* settles);
/* No reference counterpart: the on-board ceiling of the bf16 roofline.  Runs
 * `iters` iterations of 16 v_mfma_f32_32x32x16_bf16 per wave (two waves per
 * SIMD on every CU, nothing but the MFMA loop) on the context's stream, on
 * pseudo-random bf16 operands (zeros = 0: the bit activity of real data) or
 * on zero operands (zeros != 0: the least power the instruction draws),
 * waits for it and returns its TFLOP/s.  The board's power limit, not the
 * 2.4 GHz top clock, sets the sustained rate: run it long enough (tens of
 * milliseconds) for the clock to settle. */
int cfattn_probe_mfma_peak(cfattn_ctx* ctx, int zeros, int iters, double* tflops);
/* No reference counterpart: loops of one instruction class for the board
 * power each draws (read beside it with amd-smi).  kind 0: 16-byte LDS reads
 * (rate in bytes/s); kind 1: v_fma_f32 (rate in lane operations/s), both four
 * waves per SIMD on every CU; kind 2: v_mfma_f32_16x16x32_bf16 on
 * pseudo-random operands (rate in FLOP/s, two waves per SIMD: the other MFMA
 * shape against cfattn_probe_mfma_peak's).  `iters` loop iterations, on the
 * context's stream; waits for the run. */
int cfattn_probe_loop(cfattn_ctx* ctx, int kind, int iters, double* rate);
/* Name of kernel id `kernel` ("attn_fwd", "attn_bwd_dkdv", ...), or NULL. */
const char* cfattn_kernel_name(int kernel);
int cfattn_kernel_count(void);
/* Algorithmic FLOPs of one fwd+bwd over the causal triangle:
 * 7 * batch * n_heads * head_dim * seq * (seq + 1). */
double cfattn_flops_fwd_bwd(cfattn_shape s, size_t batch);
/* Library version string. */
const char* cfattn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CFATTN_H */
