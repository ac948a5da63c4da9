/* cpuforge attention oracle -- TEST INFRASTRUCTURE ONLY (see cforge_oracle.c). */
#ifndef CFORGE_ORACLE_H
#define CFORGE_ORACLE_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif
uint64_t orc_rng_seed(uint64_t seed);
uint64_t orc_rng_next_u64(uint64_t* state);
float orc_rng_uniform(uint64_t* state);
float orc_rng_normal(uint64_t* state);
void orc_fill_normal(uint64_t seed, float* out, size_t n, float std);

void orc_gemm_strided(const float* a, long a_rs, long a_cs, const float* b, long b_rs, long b_cs, float* c,
                      long c_rs, long c_cs, size_t m, size_t k, size_t n, int acc);
int orc_gemm_threads(void);
void orc_set_gemm_threads(int n);

int orc_attention_forward_blocked(const float* q, const float* k, const float* v, float* o, float* lse,
                                  size_t seq, size_t nh, size_t nkv, size_t hd, size_t q_block);
int orc_attention_forward_heads(const float* q, const float* k, const float* v, float* o, float* lse,
                                size_t seq, size_t nh, size_t nkv, size_t hd, size_t q_block,
                                size_t h_begin, size_t h_end);
int orc_attention_backward_blocked(const float* d_o, const float* q, const float* k, const float* v,
                                   const float* o, const float* lse, float* dq, float* dk, float* dv,
                                   size_t seq, size_t nh, size_t nkv, size_t hd, size_t q_block);
int orc_attention_backward_heads(const float* d_o, const float* q, const float* k, const float* v,
                                 const float* o, const float* lse, float* dq, float* dk, float* dv,
                                 size_t seq, size_t nh, size_t nkv, size_t hd, size_t q_block,
                                 size_t h_begin, size_t h_end);
void orc_attn_ref_f64(const double* q, const double* k, const double* v, double* o, double* lse,
                      size_t seq, size_t nh, size_t nkv, size_t hd, const uint8_t* row_mask);
void orc_attn_bwd_ref_f64(const double* d_o, const double* q, const double* k, const double* v,
                          double* dq, double* dk, double* dv, size_t seq, size_t nh, size_t nkv, size_t hd,
                          size_t h_begin, size_t h_end);

double orc_llama3_scale(double inv_freq, double factor, double low_freq_factor, double high_freq_factor,
                        double original_max_position);
int orc_rope_table(size_t head_dim, size_t max_pos, double theta, const double* scaling, float* cos_out,
                   float* sin_out);
int orc_rope_apply(const float* cos_t, const float* sin_t, size_t max_pos, size_t head_dim, float* x, size_t seq,
                   size_t heads, size_t pos0, int inverse);
void orc_rmsnorm_forward(const float* x, const float* w, float* y, float* rstd, size_t rows, size_t dim, float eps);
void orc_rmsnorm_backward(const float* dy, const float* x, const float* w, const float* rstd, float* dx, float* dw,
                          size_t rows, size_t dim);
void orc_silu_mul_forward(const float* g, const float* u, float* h, size_t n);
void orc_silu_mul_backward(const float* dh, const float* g, const float* u, float* dg, float* du, size_t n);
float orc_cross_entropy_fwd_bwd(const float* logits, const int64_t* targets, float* dlogits, size_t rows,
                                size_t vocab, long* bad_row);
float orc_powi_f32(float a, int b);
void orc_adamw_update(float* p, const float* g, float* m, float* v, size_t n, uint64_t t, float lr, float beta1,
                      float beta2, float eps, float weight_decay);
void orc_linear_forward(const float* x, const float* w, const float* a, const float* b, float scale, size_t t,
                        size_t in, size_t out, size_t r, float* y, float* xs);
void orc_linear_backward(const float* x, const float* xs, const float* dy, const float* w, const float* a,
                         const float* b, float scale, size_t t, size_t in, size_t out, size_t r, float* dx, float* gw,
                         float* ga, float* gb, float* dxa);
uint16_t orc_f32_to_bf16(float f);
void orc_round_bf16(const float* src, float* dst, size_t n);
double orc_grad_close_metric(const float* a, const double* n, size_t len, size_t* worst_i);
void orc_bf16_to_f32(const uint16_t* src, float* dst, size_t n);
void orc_f16_to_f32(const uint16_t* src, float* dst, size_t n);
#ifdef __cplusplus
}
#endif
#endif
