// Internal launch interface of the layer-op kernels (layer_ops.hip) used by
// the C ABI in cfops_capi.cpp.  All pointers are device memory, f32 unless
// stated, row-major and contiguous.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace cfattn {

// RMSNorm (crates/core/src/ops/rmsnorm.rs:4-67).  Forward overwrites y and
// rstd.  Backward accumulates into dx and, when dw is non-null, into dw; it
// needs `partial` scratch of rmsnorm_bwd_partial_floats(rows, dim) floats.
hipError_t launch_rmsnorm_fwd(const float* x, const float* w, float* y, float* rstd, size_t rows, size_t dim, float eps,
                              hipStream_t st);
size_t rmsnorm_bwd_partial_floats(size_t rows, size_t dim);
hipError_t launch_rmsnorm_bwd(const float* dy, const float* x, const float* w, const float* rstd, float* dx, float* dw,
                              float* partial, size_t rows, size_t dim, hipStream_t st);

// SwiGLU gate (crates/core/src/ops/swiglu.rs:10-30): forward overwrites h,
// backward accumulates into dg and du.
hipError_t launch_silu_mul_fwd(const float* g, const float* u, float* h, size_t n, hipStream_t st);
hipError_t launch_silu_mul_bwd(const float* dh, const float* g, const float* u, float* dg, float* du, size_t n,
                               hipStream_t st);

// Cross-entropy with its gradient (crates/core/src/ops/loss.rs:9-55), in three
// launches over a `misc` block of kCeMiscBytes (valid-row count, first bad
// row, loss) and `row_loss` scratch of `rows` floats:
//   ce_begin:  count the rows to score, reset the bad-row marker;
//   ce_rows:   rows [row0, row0 + nrows): `logits` and `dlogits` point at
//              row row0 (dlogits may alias logits: each row is read before it
//              is written), targets and row_loss are indexed from row 0; a
//              target outside [0, vocab) marks its row as bad;
//   ce_finish: the mean loss, summed in f64 in row order.
constexpr size_t kCeMiscBytes = 256;
struct CeMisc {
    int n_valid;
    int bad_row;  // first row with a target out of range, or INT_MAX
    float loss;
};
hipError_t launch_ce_begin(const int64_t* targets, size_t rows, void* misc, hipStream_t st);
hipError_t launch_ce_rows(const float* logits, const int64_t* targets, float* dlogits, float* row_loss, size_t row0,
                          size_t nrows, size_t vocab, void* misc, hipStream_t st);
hipError_t launch_ce_finish(const int64_t* targets, const float* row_loss, size_t rows, void* misc, hipStream_t st);

// One AdamW update (crates/train/src/optim.rs:9-30); bc1, bc2 are the bias
// corrections 1 - beta^t, computed by the caller.
hipError_t launch_adamw(float* p, const float* g, float* m, float* v, size_t n, float lr, float beta1, float beta2,
                        float eps, float weight_decay, float bc1, float bc2, hipStream_t st);

// LoRA adapter products of Linear::forward / backward (linear.rs:56-91) as
// streaming kernels (lora.hip), for ranks 4, 8 and 16 with 16-byte aligned
// rows; `part` is scratch of lora_partial_floats floats for the per-chunk
// partial sums, which are added in chunk order:
//   forward:  xs = scale * x A^T (overwritten), y += xs B^T (y non-null);
//   backward: dxa = scale * dy B (into `dxa`, t x rank), dx += dxa A (dx
//             non-null), and when non-null gb += dy^T xs, ga += dxa^T x;
//   merge:    weff = w + scale * B A ([out x in], w's layout), the base
//             weight with the adapter folded in.
constexpr int kLoraChunk = 64;  // tokens per partial sum of the gradients
bool lora_fused_applies(size_t rank, size_t t, size_t in, size_t out, const void* const* ptrs, int nptr);
size_t lora_partial_floats(size_t rank, size_t t, size_t in, size_t out);
hipError_t launch_lora_fwd(size_t rank, const float* x, const float* a, const float* b, float scale, size_t t,
                           size_t in, size_t out, float* y, float* xs, float* part, hipStream_t st);
hipError_t launch_lora_merge(size_t rank, const float* w, const float* a, const float* b, float scale, size_t out,
                             size_t in, float* weff, hipStream_t st);
hipError_t launch_lora_bwd(size_t rank, const float* x, const float* xs, const float* dy, const float* a,
                           const float* b, float scale, size_t t, size_t in, size_t out, float* dx, float* ga,
                           float* gb, float* dxa, float* part, hipStream_t st);

}  // namespace cfattn
