/* libcfattn.so -- the layer ops around the attention in a cpuforge training
 * step, on HBM-resident buffers (AMD MI355X, gfx950).
 *
 * Each entry point replaces one reference function of the CPU trainer with
 * the same argument meaning, the same overwrite / accumulate (+=) contract
 * and the same checks, on device pointers and a HIP stream instead of host
 * slices, so a layer's activations stay in HBM between the projections, the
 * norms and the attention (include/cfattn.h).  `stream` NULL is the device's
 * null stream.  A context (cfattn_create) provides the device, the scratch
 * pool and the hipBLASLt handle of the GEMMs; calls on one context are
 * serialised.  Status codes and cfattn_last_error() are those of cfattn.h.
 *
 * Reference sources (Sm0r3s-source/cpuforge, crates/...):
 *   core/src/matmul.rs:127-147   matmul_nn / matmul_nt / matmul_tn
 *   core/src/ops/rmsnorm.rs      rmsnorm_forward / rmsnorm_backward
 *   core/src/ops/swiglu.rs       silu_mul_forward / silu_mul_backward
 *   core/src/ops/loss.rs         cross_entropy_fwd_bwd, IGNORE_INDEX
 *   model/src/linear.rs:56-91    Linear::forward / Linear::backward (LoRA)
 *   model/src/model.rs:436-457   LM head + loss in Model::forward_backward
 *   train/src/optim.rs:9-30      adamw_update
 */
#ifndef CFOPS_H
#define CFOPS_H

#include <stddef.h>
#include <stdint.h>

#include "cfattn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* crates/core/src/ops/loss.rs:4: targets equal to this are not scored. */
#define CFOPS_IGNORE_INDEX (-100)

/* matmul kinds (core/src/matmul.rs:127-147), row-major, C[m,n] (+)= ...:
 *   CFOPS_NN  A[m,k]  . B[k,n]
 *   CFOPS_NT  A[m,k]  . B[n,k]^T
 *   CFOPS_TN  A[k,m]^T . B[k,n]
 * acc != 0 accumulates into C, acc == 0 overwrites it (k == 0 then zeroes C). */
enum { CFOPS_NN = 0, CFOPS_NT = 1, CFOPS_TN = 2 };
int cfops_matmul(cfattn_ctx* ctx, int kind, const float* a, const float* b, float* c, size_t m, size_t k, size_t n,
                 int acc, void* stream);

/* rmsnorm_forward (rmsnorm.rs:4-28): y = x * rsqrt(mean(x^2) + eps) * w per
 * row of `dim`; y and rstd (1/rms per row) are overwritten.  The sum of
 * squares runs in element order, so y and rstd equal the reference's f32
 * results bit for bit. */
int cfops_rmsnorm_forward(cfattn_ctx* ctx, const float* x, const float* w, float* y, float* rstd, size_t rows,
                          size_t dim, float eps, void* stream);
/* rmsnorm_backward (rmsnorm.rs:33-67): accumulates into dx and, when dw is
 * non-null, into dw (NULL: a frozen gain, no gradient work). */
int cfops_rmsnorm_backward(cfattn_ctx* ctx, const float* dy, const float* x, const float* w, const float* rstd,
                           float* dx, float* dw, size_t rows, size_t dim, void* stream);

/* silu_mul_forward / _backward (swiglu.rs:10-30): h = silu(g) * u
 * (overwritten); the backward accumulates into dg and du. */
int cfops_silu_mul_forward(cfattn_ctx* ctx, const float* g, const float* u, float* h, size_t n, void* stream);
int cfops_silu_mul_backward(cfattn_ctx* ctx, const float* dh, const float* g, const float* u, float* dg, float* du,
                            size_t n, void* stream);

/* cross_entropy_fwd_bwd (loss.rs:9-55): mean cross-entropy over the rows
 * whose target is not CFOPS_IGNORE_INDEX; dlogits [rows, vocab] is
 * overwritten (ignored rows get zeros; dlogits may equal logits).  Like the
 * reference it returns the loss, so it waits for the stream and writes the
 * loss to host *loss.  A target outside [0, vocab) is CFATTN_ERR_ARG (the
 * reference panics). */
int cfops_cross_entropy_fwd_bwd(cfattn_ctx* ctx, const float* logits, const int64_t* targets, float* dlogits,
                                size_t rows, size_t vocab, float* loss, void* stream);

/* The LM head and its loss, as Model::forward_backward and backward_from run
 * them (model.rs:436-457): logits = hn . head^T, the loss and dlogits of
 * cross_entropy_fwd_bwd, dhn = dlogits . head (overwritten) and, when dhead
 * is non-null, dhead += dlogits^T . hn.  hn [t, d], head [vocab, d].  Rows
 * go through in chunks whose logits fit the context's head chunk limit
 * (cfops_set_head_chunk_limit, default 512 MiB), so the [t, vocab] logits
 * are never held whole.  Waits for the stream; the loss goes to host *loss. */
int cfops_lm_head_ce(cfattn_ctx* ctx, const float* hn, const float* head, const int64_t* targets, size_t t, size_t d,
                     size_t vocab, float* dhn, float* dhead, float* loss, void* stream);
int cfops_set_head_chunk_limit(cfattn_ctx* ctx, size_t bytes);

/* The loss block cfops_lm_head_ce_dev writes, in device memory. */
typedef struct cfops_ce_result {
    int32_t n_valid; /* rows scored (target != CFOPS_IGNORE_INDEX) */
    int32_t bad_row; /* first row whose target is outside [0, vocab), or INT32_MAX */
    float loss;      /* the mean cross-entropy over the scored rows */
} cfops_ce_result;

/* No reference counterpart: cfops_lm_head_ce for callers that capture the
 * training step in a HIP graph or keep host waits out of it.  The same
 * launches on `stream`, with the loss block written to `result` (device
 * memory) and no wait for the stream: once the stream has drained,
 * result->loss is the loss, and result->bad_row != INT32_MAX names a row
 * whose target is out of range, which the caller reports (cfops_lm_head_ce
 * fails with "target T out of range for vocab V" there).  t must be
 * positive; dhn and dhead as in cfops_lm_head_ce. */
int cfops_lm_head_ce_dev(cfattn_ctx* ctx, const float* hn, const float* head, const int64_t* targets, size_t t,
                         size_t d, size_t vocab, float* dhn, float* dhead, cfops_ce_result* result, void* stream);

/* Linear::forward (linear.rs:56-71): y [t,out] = x [t,in] . W^T (overwritten),
 * W [out,in].  With an adapter (lora_a non-null; A [rank,in], B [out,rank]):
 * xs [t,rank] = scale * x . A^T (overwritten) and y += xs . B^T.  For ranks
 * 4, 8 and 16 with in and out multiples of 4 and 16-byte aligned operands,
 * y is formed as x . (W + scale * B . A)^T in one GEMM: the same sum,
 * rounded differently (within f32 rounding of the reference's). */
int cfops_linear_forward(cfattn_ctx* ctx, const float* x, const float* w, const float* lora_a, const float* lora_b,
                         float lora_scale, size_t t, size_t in, size_t out, size_t rank, float* y, float* xs,
                         void* stream);
/* Linear::backward (linear.rs:73-91): dx += dy . W; gw += dy^T . x when gw is
 * non-null; with an adapter gb += dy^T . xs (gb non-null), and with
 * dxa = scale * dy . B: ga += dxa^T . x (ga non-null) and dx += dxa . A
 * (on the forward's fast shapes: dx += dy . (W + scale * B . A) in one GEMM).
 * NULL gradients are frozen tensors (the reference's empty LinGrad vectors). */
int cfops_linear_backward(cfattn_ctx* ctx, const float* x, const float* xs, const float* dy, const float* w,
                          const float* lora_a, const float* lora_b, float lora_scale, size_t t, size_t in, size_t out,
                          size_t rank, float* dx, float* gw, float* ga, float* gb, void* stream);

/* adamw_update (optim.rs:9-30): one AdamW step of one tensor of n values,
 * t the 1-based step count; p, m, v updated in place.  Every product and sum
 * is rounded in the reference's order, so results equal its f32 arithmetic
 * bit for bit. */
int cfops_adamw_update(cfattn_ctx* ctx, float* p, const float* g, float* m, float* v, size_t n, uint64_t t, float lr,
                       float beta1, float beta2, float eps, float weight_decay, void* stream);

#ifdef __cplusplus
}
#endif
#endif
