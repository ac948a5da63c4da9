/* cpuforge layer-op oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * Plain-C restatements of the reference's CPU ops that surround the
 * attention in a training step, used by tests/ and bench.py as the checker
 * of the GPU entry points in include/cfops.h.  Nothing in the product links
 * or calls this file.  Compiled with -ffp-contract=off: Rust never fuses a
 * multiply and an add, so every product and sum below is rounded on its own,
 * in the order the reference writes it.
 *
 * Pinned in tests/test_oracle_layer.py against the reference's own tests
 * (closed forms, f64 references, finite differences, hand-computed AdamW
 * steps) -- see the comment on each function for its source.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#include "oracle.h"

/* crates/core/src/ops/swiglu.rs:6-8 */
static float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }

/* h = silu(g) * u, silu(g) = g * sigmoid(g): crates/core/src/ops/swiglu.rs:10-16.
 * The reference evaluates gv * sigmoid(gv) * uv left to right. */
void orc_silu_mul_forward(const float* g, const float* u, float* h, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const float s = sigmoid_f(g[i]);
        const float gs = g[i] * s;
        h[i] = gs * u[i];
    }
}

/* Accumulates into dg and du: crates/core/src/ops/swiglu.rs:18-30. */
void orc_silu_mul_backward(const float* dh, const float* g, const float* u, float* dg, float* du, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const float s = sigmoid_f(g[i]);
        const float silu = g[i] * s;
        const float one_minus = 1.0f - s;
        const float inner = g[i] * one_minus;
        const float dsilu = s * (1.0f + inner);
        const float a = dh[i] * u[i];
        dg[i] += a * dsilu;
        du[i] += dh[i] * silu;
    }
}

/* Mean cross-entropy over rows whose target is not IGNORE_INDEX (-100), with
 * its gradient written to dlogits (overwritten; ignored rows get zeros):
 * crates/core/src/ops/loss.rs:9-55.  Returns the loss; *bad_row receives the
 * first row whose target is out of range (the reference panics there), or
 * -1.  The per-row loss is formed in f32 and summed in f64, in row order. */
float orc_cross_entropy_fwd_bwd(const float* logits, const int64_t* targets, float* dlogits, size_t rows,
                                size_t vocab, long* bad_row) {
    *bad_row = -1;
    size_t n_valid = 0;
    for (size_t r = 0; r < rows; r++) n_valid += targets[r] != -100;
    if (n_valid == 0) {
        memset(dlogits, 0, rows * vocab * sizeof(float));
        return 0.0f;
    }
    const float inv_n = 1.0f / (float)n_valid;
    double total = 0.0;
    for (size_t r = 0; r < rows; r++) {
        const float* lr = logits + r * vocab;
        float* dr = dlogits + r * vocab;
        const int64_t t = targets[r];
        if (t == -100) {
            memset(dr, 0, vocab * sizeof(float));
            continue;
        }
        if (t < 0 || (uint64_t)t >= vocab) {
            *bad_row = (long)r;
            return NAN;
        }
        float mx = -INFINITY;
        for (size_t i = 0; i < vocab; i++) mx = fmaxf(mx, lr[i]);
        float sum = 0.0f;
        for (size_t i = 0; i < vocab; i++) {
            const float e = expf(lr[i] - mx);
            dr[i] = e;
            sum += e;
        }
        const float row_loss = logf(sum) + mx - lr[t];
        total += (double)row_loss;
        const float inv_sum = 1.0f / sum;
        const float sc = inv_sum * inv_n;
        for (size_t i = 0; i < vocab; i++) dr[i] *= sc;
        dr[t] -= inv_n;
    }
    return (float)(total / (double)n_valid);
}

/* x^n for integer n as Rust's f32::powi evaluates it at run time (LLVM's
 * llvm.powi.f32, lowered to compiler-rt's __powisf2: square-and-multiply
 * from the low bit, reciprocal for a negative exponent). */
float orc_powi_f32(float a, int b) {
    const int recip = b < 0;
    float r = 1.0f;
    unsigned int e = recip ? (unsigned int)(-(long)b) : (unsigned int)b;
    for (;;) {
        if (e & 1u) r *= a;
        e >>= 1;
        if (e == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

/* One AdamW update of one tensor, t the 1-based step:
 * crates/train/src/optim.rs:9-30. */
void orc_adamw_update(float* p, const float* g, float* m, float* v, size_t n, uint64_t t, float lr, float beta1,
                      float beta2, float eps, float weight_decay) {
    const float bc1 = 1.0f - orc_powi_f32(beta1, (int)t);
    const float bc2 = 1.0f - orc_powi_f32(beta2, (int)t);
    const float ob1 = 1.0f - beta1, ob2 = 1.0f - beta2;
    for (size_t i = 0; i < n; i++) {
        m[i] = beta1 * m[i] + ob1 * g[i];
        v[i] = beta2 * v[i] + ob2 * g[i] * g[i];
        const float mhat = m[i] / bc1;
        const float vhat = v[i] / bc2;
        p[i] -= lr * (mhat / (sqrtf(vhat) + eps) + weight_decay * p[i]);
    }
}

/* matmul_nt / matmul_nn / matmul_tn (crates/core/src/matmul.rs:127-147) over
 * the oracle's strided GEMM. */
static void mm_nt(const float* a, const float* b, float* c, size_t m, size_t k, size_t n, int acc) {
    orc_gemm_strided(a, (long)k, 1, b, 1, (long)k, c, (long)n, 1, m, k, n, acc);
}
static void mm_nn(const float* a, const float* b, float* c, size_t m, size_t k, size_t n, int acc) {
    orc_gemm_strided(a, (long)k, 1, b, (long)n, 1, c, (long)n, 1, m, k, n, acc);
}
static void mm_tn(const float* a, const float* b, float* c, size_t m, size_t k, size_t n, int acc) {
    orc_gemm_strided(a, 1, (long)m, b, (long)n, 1, c, (long)n, 1, m, k, n, acc);
}

/* Linear::forward (crates/model/src/linear.rs:56-71): y = x W^T, and with an
 * adapter (a non-null) xs = scale * x A^T, y += xs B^T.  W [out,in],
 * A [r,in], B [out,r]; x [t,in], y [t,out] (overwritten), xs [t,r]. */
void orc_linear_forward(const float* x, const float* w, const float* a, const float* b, float scale, size_t t,
                        size_t in, size_t out, size_t r, float* y, float* xs) {
    mm_nt(x, w, y, t, in, out, 0);
    if (!a) return;
    mm_nt(x, a, xs, t, in, r, 0);
    for (size_t i = 0; i < t * r; i++) xs[i] *= scale;
    mm_nt(xs, b, y, t, r, out, 1);
}

/* Linear::backward (crates/model/src/linear.rs:73-91): accumulates into dx
 * and into each non-null gradient (gw [out,in], ga [r,in], gb [out,r]);
 * dxa [t,r] is scratch. */
void orc_linear_backward(const float* x, const float* xs, const float* dy, const float* w, const float* a,
                         const float* b, float scale, size_t t, size_t in, size_t out, size_t r, float* dx, float* gw,
                         float* ga, float* gb, float* dxa) {
    mm_nn(dy, w, dx, t, out, in, 1);
    if (gw) mm_tn(dy, x, gw, out, t, in, 1);
    if (!a) return;
    if (gb) mm_tn(dy, xs, gb, out, t, r, 1);
    mm_nn(dy, b, dxa, t, out, r, 0);
    for (size_t i = 0; i < t * r; i++) dxa[i] *= scale;
    if (ga) mm_tn(dxa, x, ga, r, t, in, 1);
    mm_nn(dxa, a, dx, t, r, in, 1);
}
