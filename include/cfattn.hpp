// C++ host interface mirroring cpuforge's attention op (the reference is Rust;
// crates/core/src/ops/attention.rs, crates/core/src/ops/rope.rs), implemented
// over the C ABI of libcfattn.so (cfattn.h).  Same item names, argument order
// and meaning; slices are std::span; where the reference panics through
// assert!/assert_eq! this throws cf_core::Panic with the same message.
//
//   cf_core::ops::AttnShape                    attention.rs:20-26
//   cf_core::ops::DEFAULT_Q_BLOCK              attention.rs:18
//   cf_core::ops::attention_forward(_blocked)  attention.rs:42-54
//   cf_core::ops::attention_backward(_blocked) attention.rs:126-154
//   cf_core::ops::Llama3Scaling, RopeCache     rope.rs:6-63 (tables; the
//       rotation itself runs on the GPU in the fused prologue, cfattn_fused_*)
//
// Calls are synchronous and go through one process-wide library context on
// HIP device 0, created on first use.  set_attention_mode(CFATTN_BF16)
// switches it to bf16 inputs with fp32 accumulation.
#pragma once

#include <cstddef>
#include <mutex>
#include <optional>
#include <span>
#include <stdexcept>
#include <string>
#include <vector>

#include "cfattn.h"

namespace cf_core {

// A reference assert that fired (the Rust op panics).
struct Panic : std::runtime_error {
    using std::runtime_error::runtime_error;
};

namespace detail {
inline cfattn_ctx* context() {
    static std::once_flag once;
    static cfattn_ctx* ctx = nullptr;
    static int rc = CFATTN_OK;
    std::call_once(once, [] { rc = cfattn_create(0, &ctx); });
    if (rc != CFATTN_OK || !ctx) throw Panic("cfattn_create failed: no usable HIP device");
    return ctx;
}
inline void check(cfattn_ctx* ctx, int rc) {
    if (rc != CFATTN_OK) throw Panic(std::string(cfattn_last_error(ctx)));
}
}  // namespace detail

namespace ops {

inline constexpr std::size_t DEFAULT_Q_BLOCK = 128;

struct AttnShape {
    std::size_t seq;
    std::size_t n_heads;
    std::size_t n_kv;
    std::size_t head_dim;
    cfattn_shape c() const { return cfattn_shape{seq, n_heads, n_kv, head_dim}; }
};

inline void set_attention_mode(int dtype) {
    cfattn_ctx* c = detail::context();
    detail::check(c, cfattn_set_mode(c, dtype));
}

inline void attention_forward_blocked(std::span<const float> q, std::span<const float> k, std::span<const float> v,
                                      std::span<float> o, std::span<float> lse, AttnShape s, std::size_t q_block) {
    cfattn_ctx* c = detail::context();
    detail::check(c, cfattn_attention_forward_blocked(c, q.data(), q.size(), k.data(), k.size(), v.data(), v.size(),
                                                      o.data(), o.size(), lse.data(), lse.size(), s.c(), q_block));
}

inline void attention_forward(std::span<const float> q, std::span<const float> k, std::span<const float> v,
                              std::span<float> o, std::span<float> lse, AttnShape s) {
    attention_forward_blocked(q, k, v, o, lse, s, DEFAULT_Q_BLOCK);
}

inline void attention_backward_blocked(std::span<const float> d_o, std::span<const float> q,
                                       std::span<const float> k, std::span<const float> v,
                                       std::span<const float> o, std::span<const float> lse, std::span<float> dq,
                                       std::span<float> dk, std::span<float> dv, AttnShape s, std::size_t q_block) {
    cfattn_ctx* c = detail::context();
    detail::check(c, cfattn_attention_backward_blocked(c, d_o.data(), d_o.size(), q.data(), q.size(), k.data(),
                                                       k.size(), v.data(), v.size(), o.data(), o.size(), lse.data(),
                                                       lse.size(), dq.data(), dq.size(), dk.data(), dk.size(),
                                                       dv.data(), dv.size(), s.c(), q_block));
}

inline void attention_backward(std::span<const float> d_o, std::span<const float> q, std::span<const float> k,
                               std::span<const float> v, std::span<const float> o, std::span<const float> lse,
                               std::span<float> dq, std::span<float> dk, std::span<float> dv, AttnShape s) {
    attention_backward_blocked(d_o, q, k, v, o, lse, dq, dk, dv, s, DEFAULT_Q_BLOCK);
}

// rope.rs:16-38
struct Llama3Scaling {
    double factor;
    double low_freq_factor;
    double high_freq_factor;
    double original_max_position;
    cfattn_llama3_scaling c() const {
        return cfattn_llama3_scaling{factor, low_freq_factor, high_freq_factor, original_max_position};
    }
    double apply(double inv_freq) const {
        const cfattn_llama3_scaling sc = c();
        return cfattn_llama3_scale(&sc, inv_freq);
    }
};

// rope.rs:6-12, 41-63: cos/sin tables [max_pos, head_dim/2], computed in f64
// and rounded to f32.
struct RopeCache {
    std::size_t head_dim = 0;
    std::size_t max_pos = 0;
    std::vector<float> cos;
    std::vector<float> sin;

    static RopeCache with_scaling(std::size_t head_dim, std::size_t max_pos, double theta,
                                  std::optional<Llama3Scaling> scaling) {
        if (head_dim % 2 != 0) throw Panic("head_dim must be even");
        RopeCache r;
        r.head_dim = head_dim;
        r.max_pos = max_pos;
        r.cos.resize(max_pos * head_dim / 2);
        r.sin.resize(max_pos * head_dim / 2);
        cfattn_llama3_scaling sc{};
        if (scaling) sc = scaling->c();
        const int rc = cfattn_rope_table(head_dim, max_pos, theta, scaling ? &sc : nullptr, r.cos.data(),
                                         r.sin.data());
        if (rc != CFATTN_OK) throw Panic("cfattn_rope_table failed");
        return r;
    }
    static RopeCache new_(std::size_t head_dim, std::size_t max_pos, double theta) {
        return with_scaling(head_dim, max_pos, theta, std::nullopt);
    }
};

}  // namespace ops
}  // namespace cf_core
