/*
 * cpuforge attention oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the CPU algorithms on cpuforge's attention hot path,
 * used as the checker for the HIP kernels in cpuforge_amd/.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this
 * library; the product path (libcfattn.so) never links or calls it.
 *
 * What is restated, and where it comes from in the reference
 * (/root/reference, paths relative to crates/):
 *   - Rng (xorshift64*, uniform, Box-Muller normal)  core/src/rng.rs:10-43
 *   - gemm_strided semantics (acc / k==0 / strides)   core/src/matmul.rs:37-98
 *   - attention_forward_blocked                       core/src/ops/attention.rs:46-122
 *   - attention_backward_blocked                      core/src/ops/attention.rs:142-262
 *   - naive f64 attention (attn_ref)                  core/src/ops/attention.rs:271-296
 *   - RopeCache::with_scaling / apply                 core/src/ops/rope.rs:46-89
 *   - Llama3Scaling::apply                            core/src/ops/rope.rs:26-38
 *   - rmsnorm_forward / rmsnorm_backward              core/src/ops/rmsnorm.rs:4-67
 *   - assert_grad_close metric                        core/src/gradcheck.rs:31-48
 *
 * The reference is Rust and its contraction arithmetic lives in the
 * un-vendored `gemm 0.19.0` crate (Cargo.lock:488-491), so it cannot be built
 * here; the restatement matches its semantics (and the reference's own f32
 * softmax order), not its SIMD summation order.  Each function is pinned by a
 * test in tests/test_oracle.py (f64 brute force, torch float64 autograd,
 * finite differences, closed forms and the reference's own invariants).
 *
 * Compiled with -ffp-contract=off so that every f32 expression rounds exactly
 * as the Rust source does (Rust never fuses a*b+c).  The GEMM used by the
 * attention restatement lives in oracle_gemm.c.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* ------------------------------------------------------------------ Rng */
/* core/src/rng.rs:10-13: state = seed ^ golden | 1 (Rust: ^ binds tighter). */
uint64_t orc_rng_seed(uint64_t seed) { return (seed ^ 0x9E3779B97F4A7C15ull) | 1ull; }

/* core/src/rng.rs:16-23 */
uint64_t orc_rng_next_u64(uint64_t* state) {
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return x * 0x2545F4914F6CDD1Dull;
}

/* core/src/rng.rs:27-29: top 24 bits / 2^24. */
float orc_rng_uniform(uint64_t* state) {
    return (float)(orc_rng_next_u64(state) >> 40) / (float)(1ull << 24);
}

/* core/src/rng.rs:32-36: f32 Box-Muller, one uniform pair per sample. */
float orc_rng_normal(uint64_t* state) {
    float u1 = fmaxf(orc_rng_uniform(state), 1e-12f);
    float u2 = orc_rng_uniform(state);
    const float two_pi = 2.0f * 3.14159265358979323846f; /* 2.0 * f32::consts::PI */
    return sqrtf(-2.0f * logf(u1)) * cosf(two_pi * u2);
}

/* core/src/rng.rs:38-42 (fill_normal) from a fresh Rng::new(seed). */
void orc_fill_normal(uint64_t seed, float* out, size_t n, float std) {
    uint64_t st = orc_rng_seed(seed);
    for (size_t i = 0; i < n; i++) out[i] = orc_rng_normal(&st) * std;
}

/* --------------------------------------------------------- attention f32 */
/* Restates attention_forward_blocked, core/src/ops/attention.rs:46-122:
 * per query head, per block of q_block queries, S = Q_blk K[0..t1]^T by GEMM,
 * then a row-wise f32 scale / max / exp / sum / normalise with the masked
 * tail zeroed, then O_blk = P V[0..t1].  Heads are strided views.
 * Restricted to query heads [h_begin, h_end) (the reference's per-head loop,
 * attention.rs:65, over a sub-range) so one GQA group of a large
 * configuration can be checked in seconds. */
int orc_attention_forward_heads(const float* q, const float* k, const float* v, float* o, float* lse,
                                size_t seq, size_t nh, size_t nkv, size_t hd, size_t q_block,
                                size_t h_begin, size_t h_end) {
    if (nkv == 0 || nh % nkv != 0 || q_block == 0) return -1;
    const size_t t_len = seq;
    const long qs = (long)(nh * hd), kvs = (long)(nkv * hd);
    const size_t group = nh / nkv;
    const float scale = 1.0f / sqrtf((float)hd);
    size_t cap = (q_block < (t_len > 0 ? t_len : 1) ? q_block : (t_len > 0 ? t_len : 1)) * t_len;
    float* p = (float*)calloc(cap ? cap : 1, sizeof(float));
    if (!p) return -2;
    for (size_t h = h_begin; h < h_end; h++) {
        size_t g = h / group;
        for (size_t t0 = 0; t0 < t_len;) {
            size_t t1 = t0 + q_block < t_len ? t0 + q_block : t_len;
            size_t bq = t1 - t0, l = t1;
            /* S = Q_blk . K[0..l]^T  (attention.rs:72-83) */
            orc_gemm_strided(q + t0 * qs + h * hd, qs, 1, k + g * hd, 1, kvs, p, (long)l, 1, bq, hd, l, 0);
            for (size_t r = 0; r < bq; r++) { /* attention.rs:86-105 */
                size_t valid = t0 + r + 1;
                float* row = p + r * l;
                float mx = -INFINITY;
                for (size_t j = 0; j < valid; j++) {
                    row[j] *= scale;
                    mx = fmaxf(mx, row[j]);
                }
                float sum = 0.0f;
                for (size_t j = 0; j < valid; j++) {
                    row[j] = expf(row[j] - mx);
                    sum += row[j];
                }
                lse[h * t_len + t0 + r] = mx + logf(sum);
                float inv = 1.0f / sum;
                for (size_t j = 0; j < valid; j++) row[j] *= inv;
                for (size_t j = valid; j < l; j++) row[j] = 0.0f;
            }
            /* O_blk = P . V[0..l]  (attention.rs:107-118) */
            orc_gemm_strided(p, (long)l, 1, v + g * hd, kvs, 1, o + t0 * qs + h * hd, qs, 1, bq, l, hd, 0);
            t0 = t1;
        }
    }
    free(p);
    return 0;
}

int orc_attention_forward_blocked(const float* q, const float* k, const float* v, float* o, float* lse,
                                  size_t seq, size_t nh, size_t nkv, size_t hd, size_t q_block) {
    return orc_attention_forward_heads(q, k, v, o, lse, seq, nh, nkv, hd, q_block, 0, nh);
}

/* Restates attention_backward_blocked, core/src/ops/attention.rs:142-262.
 * Accumulates (+=) into dq, dk, dv (core/src/ops/mod.rs:1-6). */
int orc_attention_backward_blocked(const float* d_o, const float* q, const float* k, const float* v,
                                   const float* o, const float* lse, float* dq, float* dk, float* dv,
                                   size_t seq, size_t nh, size_t nkv, size_t hd, size_t q_block) {
    return orc_attention_backward_heads(d_o, q, k, v, o, lse, dq, dk, dv, seq, nh, nkv, hd, q_block, 0, nh);
}

/* The same loop restricted to query heads [h_begin, h_end): the reference's
 * per-head loop (attention.rs:167) over a sub-range.  Used to check one GQA
 * group of a large configuration in seconds; dk/dv then hold only the
 * contributions of those heads. */
int orc_attention_backward_heads(const float* d_o, const float* q, const float* k, const float* v,
                                 const float* o, const float* lse, float* dq, float* dk, float* dv,
                                 size_t seq, size_t nh, size_t nkv, size_t hd, size_t q_block,
                                 size_t h_begin, size_t h_end) {
    if (nkv == 0 || nh % nkv != 0 || q_block == 0) return -1;
    const size_t t_len = seq;
    const long qs = (long)(nh * hd), kvs = (long)(nkv * hd);
    const size_t group = nh / nkv;
    const float scale = 1.0f / sqrtf((float)hd);
    size_t cap = (q_block < (t_len > 0 ? t_len : 1) ? q_block : (t_len > 0 ? t_len : 1)) * t_len;
    float* p = (float*)calloc(cap ? cap : 1, sizeof(float));
    float* ds = (float*)calloc(cap ? cap : 1, sizeof(float));
    if (!p || !ds) {
        free(p);
        free(ds);
        return -2;
    }
    for (size_t h = h_begin; h < h_end; h++) {
        size_t g = h / group;
        for (size_t t0 = 0; t0 < t_len;) {
            size_t t1 = t0 + q_block < t_len ? t0 + q_block : t_len;
            size_t bq = t1 - t0, l = t1;
            size_t q_off = t0 * qs + h * hd;
            /* Recompute P from the saved log-sum-exp (attention.rs:176-195). */
            orc_gemm_strided(q + q_off, qs, 1, k + g * hd, 1, kvs, p, (long)l, 1, bq, hd, l, 0);
            for (size_t r = 0; r < bq; r++) {
                size_t valid = t0 + r + 1;
                float* row = p + r * l;
                float lse_r = lse[h * t_len + t0 + r];
                for (size_t j = 0; j < valid; j++) row[j] = expf(row[j] * scale - lse_r);
                for (size_t j = valid; j < l; j++) row[j] = 0.0f;
            }
            /* dV[0..l] += P^T . dO_blk (attention.rs:197-208) */
            orc_gemm_strided(p, 1, (long)l, d_o + q_off, qs, 1, dv + g * hd, kvs, 1, l, bq, hd, 1);
            /* dP = dO_blk . V[0..l]^T (attention.rs:210-221) */
            orc_gemm_strided(d_o + q_off, qs, 1, v + g * hd, 1, kvs, ds, (long)l, 1, bq, hd, l, 0);
            /* dS = P * (dP - D) * scale, D = rowsum(dO * O) (attention.rs:223-232) */
            for (size_t r = 0; r < bq; r++) {
                size_t off = q_off + r * qs;
                float dsum = 0.0f;
                for (size_t d = 0; d < hd; d++) dsum += d_o[off + d] * o[off + d];
                const float* prow = p + r * l;
                float* drow = ds + r * l;
                for (size_t j = 0; j < l; j++) drow[j] = prow[j] * (drow[j] - dsum) * scale;
            }
            /* dQ_blk += dS . K[0..l] (attention.rs:234-245) */
            orc_gemm_strided(ds, (long)l, 1, k + g * hd, kvs, 1, dq + q_off, qs, 1, bq, l, hd, 1);
            /* dK[0..l] += dS^T . Q_blk (attention.rs:247-258) */
            orc_gemm_strided(ds, 1, (long)l, q + q_off, qs, 1, dk + g * hd, kvs, 1, l, bq, hd, 1);
            t0 = t1;
        }
    }
    free(p);
    free(ds);
    return 0;
}

/* ---------------------------------------------------- attention in f64 */
/* attn_ref, core/src/ops/attention.rs:271-296, extended to also return the
 * log-sum-exp of the scaled causal scores.  Rows (t, h) with
 * row_mask[t*nh+h]==0 are skipped (o, lse left untouched) so that a sample of
 * rows of a large configuration can be checked; row_mask may be NULL. */
void orc_attn_ref_f64(const double* q, const double* k, const double* v, double* o, double* lse,
                      size_t seq, size_t nh, size_t nkv, size_t hd, const uint8_t* row_mask) {
    const size_t group = nh / nkv;
    const double sc = 1.0 / sqrt((double)hd);
    double* sco = (double*)malloc((seq ? seq : 1) * sizeof(double));
    for (size_t h = 0; h < nh; h++) {
        size_t g = h / group;
        for (size_t t = 0; t < seq; t++) {
            if (row_mask && !row_mask[t * nh + h]) continue;
            const double* qv = q + (t * nh + h) * hd;
            double mx = -INFINITY;
            for (size_t j = 0; j <= t; j++) {
                const double* kv = k + (j * nkv + g) * hd;
                double s = 0.0;
                for (size_t d = 0; d < hd; d++) s += qv[d] * kv[d];
                sco[j] = s * sc;
                if (sco[j] > mx) mx = sco[j];
            }
            double sum = 0.0;
            for (size_t j = 0; j <= t; j++) {
                sco[j] = exp(sco[j] - mx);
                sum += sco[j];
            }
            double* ov = o + (t * nh + h) * hd;
            for (size_t d = 0; d < hd; d++) ov[d] = 0.0;
            for (size_t j = 0; j <= t; j++) {
                const double* vv = v + (j * nkv + g) * hd;
                double w = sco[j] / sum;
                for (size_t d = 0; d < hd; d++) ov[d] += w * vv[d];
            }
            lse[h * seq + t] = mx + log(sum);
        }
    }
    free(sco);
}

/* Closed-form gradients of sum(dO * attn(q,k,v)) in f64, written (not
 * accumulated) into dq, dk, dv.  Same math as attention.rs:142-262 with no
 * blocking: P from the exact softmax, dV = P^T dO, dP = dO V^T,
 * dS = P (dP - rowsum(P dP)) / sqrt(D), dQ = dS K, dK = dS^T Q.  Only query
 * heads [h_begin, h_end) contribute (pass 0, nh for the whole op). */
void orc_attn_bwd_ref_f64(const double* d_o, const double* q, const double* k, const double* v,
                          double* dq, double* dk, double* dv, size_t seq, size_t nh, size_t nkv, size_t hd,
                          size_t h_begin, size_t h_end) {
    const size_t group = nh / nkv;
    const double sc = 1.0 / sqrt((double)hd);
    memset(dq, 0, seq * nh * hd * sizeof(double));
    memset(dk, 0, seq * nkv * hd * sizeof(double));
    memset(dv, 0, seq * nkv * hd * sizeof(double));
    double* pr = (double*)malloc((seq ? seq : 1) * sizeof(double));
    double* dp = (double*)malloc((seq ? seq : 1) * sizeof(double));
    for (size_t h = h_begin; h < h_end; h++) {
        size_t g = h / group;
        for (size_t t = 0; t < seq; t++) {
            const double* qv = q + (t * nh + h) * hd;
            const double* gv = d_o + (t * nh + h) * hd;
            double mx = -INFINITY;
            for (size_t j = 0; j <= t; j++) {
                const double* kv = k + (j * nkv + g) * hd;
                double s = 0.0;
                for (size_t d = 0; d < hd; d++) s += qv[d] * kv[d];
                pr[j] = s * sc;
                if (pr[j] > mx) mx = pr[j];
            }
            double sum = 0.0;
            for (size_t j = 0; j <= t; j++) {
                pr[j] = exp(pr[j] - mx);
                sum += pr[j];
            }
            double delta = 0.0;
            for (size_t j = 0; j <= t; j++) {
                pr[j] /= sum;
                const double* vv = v + (j * nkv + g) * hd;
                double s = 0.0;
                for (size_t d = 0; d < hd; d++) s += gv[d] * vv[d];
                dp[j] = s;
                delta += pr[j] * s;
            }
            double* dqv = dq + (t * nh + h) * hd;
            for (size_t j = 0; j <= t; j++) {
                double dsj = pr[j] * (dp[j] - delta) * sc;
                const double* kv = k + (j * nkv + g) * hd;
                double* dkv = dk + (j * nkv + g) * hd;
                double* dvv = dv + (j * nkv + g) * hd;
                for (size_t d = 0; d < hd; d++) {
                    dqv[d] += dsj * kv[d];
                    dkv[d] += dsj * qv[d];
                    dvv[d] += pr[j] * gv[d];
                }
            }
        }
    }
    free(pr);
    free(dp);
}

/* ----------------------------------------------------------------- RoPE */
/* Llama3Scaling::apply, core/src/ops/rope.rs:26-38 (f64). */
double orc_llama3_scale(double inv_freq, double factor, double low_freq_factor, double high_freq_factor,
                        double original_max_position) {
    const double pi = 3.14159265358979323846;
    double wavelen = 2.0 * pi / inv_freq;
    double low_wavelen = original_max_position / low_freq_factor;
    double high_wavelen = original_max_position / high_freq_factor;
    if (wavelen < high_wavelen) return inv_freq;
    if (wavelen > low_wavelen) return inv_freq / factor;
    double smooth = (original_max_position / wavelen - low_freq_factor) / (high_freq_factor - low_freq_factor);
    return (1.0 - smooth) * inv_freq / factor + smooth * inv_freq;
}

/* RopeCache::with_scaling, core/src/ops/rope.rs:46-63: cos/sin [max_pos, D/2]
 * computed in f64 and rounded to f32.  scaling==NULL means plain RoPE;
 * otherwise scaling = {factor, low, high, original_max_position}. */
int orc_rope_table(size_t head_dim, size_t max_pos, double theta, const double* scaling, float* cos_out,
                   float* sin_out) {
    if (head_dim % 2 != 0) return -1;
    size_t half = head_dim / 2;
    for (size_t pos = 0; pos < max_pos; pos++) {
        for (size_t i = 0; i < half; i++) {
            double inv_freq = pow(theta, -(2.0 * (double)i) / (double)head_dim);
            if (scaling) inv_freq = orc_llama3_scale(inv_freq, scaling[0], scaling[1], scaling[2], scaling[3]);
            double angle = (double)pos * inv_freq;
            cos_out[pos * half + i] = (float)cos(angle);
            sin_out[pos * half + i] = (float)sin(angle);
        }
    }
    return 0;
}

/* RopeCache::apply, core/src/ops/rope.rs:71-89: rotate-half in place, token t
 * at position pos0+t; inverse flips the sine (the transpose). */
int orc_rope_apply(const float* cos_t, const float* sin_t, size_t max_pos, size_t head_dim, float* x, size_t seq,
                   size_t heads, size_t pos0, int inverse) {
    if (pos0 + seq > max_pos) return -1;
    size_t half = head_dim / 2;
    float sign = inverse ? -1.0f : 1.0f;
    for (size_t t = 0; t < seq; t++) {
        const float* cs = cos_t + (pos0 + t) * half;
        const float* sn = sin_t + (pos0 + t) * half;
        for (size_t h = 0; h < heads; h++) {
            float* lo = x + (t * heads + h) * head_dim;
            float* hi = lo + half;
            for (size_t i = 0; i < half; i++) {
                float c = cs[i], s = sign * sn[i];
                float x1 = lo[i], x2 = hi[i];
                lo[i] = x1 * c - x2 * s;
                hi[i] = x2 * c + x1 * s;
            }
        }
    }
    return 0;
}

/* -------------------------------------------------------------- RMSNorm */
/* rmsnorm_forward, core/src/ops/rmsnorm.rs:4-26. */
void orc_rmsnorm_forward(const float* x, const float* w, float* y, float* rstd, size_t rows, size_t dim, float eps) {
    for (size_t r = 0; r < rows; r++) {
        const float* xr = x + r * dim;
        float ss = 0.0f;
        for (size_t i = 0; i < dim; i++) ss += xr[i] * xr[i];
        float ms = ss / (float)dim;
        float inv = 1.0f / sqrtf(ms + eps);
        rstd[r] = inv;
        for (size_t i = 0; i < dim; i++) y[r * dim + i] = xr[i] * inv * w[i];
    }
}

/* rmsnorm_backward, core/src/ops/rmsnorm.rs:32-67: accumulates into dx, dw. */
void orc_rmsnorm_backward(const float* dy, const float* x, const float* w, const float* rstd, float* dx, float* dw,
                          size_t rows, size_t dim) {
    for (size_t r = 0; r < rows; r++) {
        const float* xr = x + r * dim;
        const float* dyr = dy + r * dim;
        float inv = rstd[r];
        float dot = 0.0f;
        for (size_t i = 0; i < dim; i++) dot += dyr[i] * w[i] * xr[i] * inv;
        float mean = dot / (float)dim;
        float* dxr = dx + r * dim;
        for (size_t i = 0; i < dim; i++) {
            float xhat = xr[i] * inv;
            dw[i] += dyr[i] * xhat;
            dxr[i] += inv * (dyr[i] * w[i] - xhat * mean);
        }
    }
}

/* ---------------------------------------------------------------- bf16 */
/* Round-to-nearest-even f32 -> bf16 bits (NaN kept quiet), and the exact
 * widening back (crates/io/src/dtype.rs:3-5 is the widening direction). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void orc_round_bf16(const float* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; i++) {
        uint32_t u = (uint32_t)orc_f32_to_bf16(src[i]) << 16;
        memcpy(&dst[i], &u, 4);
    }
}

/* --------------------------------------------------------- grad metric */
/* assert_grad_close's metric, core/src/gradcheck.rs:31-48: worst
 * |a - n| / (1 + |n|); *worst_i receives its index. */
double orc_grad_close_metric(const float* a, const double* n, size_t len, size_t* worst_i) {
    double worst = 0.0;
    size_t wi = 0;
    for (size_t i = 0; i < len; i++) {
        double err = fabs((double)a[i] - n[i]) / (1.0 + fabs(n[i]));
        if (err > worst) {
            worst = err;
            wi = i;
        }
    }
    if (worst_i) *worst_i = wi;
    return worst;
}
