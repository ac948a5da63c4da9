// The reference's attention tests (crates/core/src/ops/attention.rs:264-394)
// restated in C++ against the C++ mirror of its interface (include/cfattn.hpp),
// so the GPU op runs under the reference's own checks: the same CASES, seeds,
// tolerances, f64 naive reference and central finite differences
// (crates/core/src/gradcheck.rs).  Inputs come from the reference's Rng, via
// the oracle library (test infrastructure).  Exit status 0 when every test
// passes; a failed check prints the reference's message and exits 1.
#include <cmath>
#include <cstdio>
#include <functional>
#include <string>
#include <vector>

#include "cfattn.hpp"

extern "C" {
void orc_fill_normal(uint64_t seed, float* out, size_t n, float std);
}

using cf_core::ops::AttnShape;
using cf_core::ops::attention_backward_blocked;
using cf_core::ops::attention_forward;
using cf_core::ops::attention_forward_blocked;
using Vec64 = std::vector<double>;
using Vec32 = std::vector<float>;

namespace {

int failures = 0;

void fail(const std::string& msg) {
    std::printf("FAILED: %s\n", msg.c_str());
    failures++;
}

// gradcheck.rs:6-23
Vec64 numeric_grad(const std::function<double(const Vec64&)>& f, const Vec64& x, double eps) {
    Vec64 xp = x, g(x.size());
    for (size_t i = 0; i < x.size(); i++) {
        const double orig = xp[i];
        xp[i] = orig + eps;
        const double hi = f(xp);
        xp[i] = orig - eps;
        const double lo = f(xp);
        xp[i] = orig;
        g[i] = (hi - lo) / (2.0 * eps);
    }
    return g;
}

Vec64 to_f64(const Vec32& x) { return Vec64(x.begin(), x.end()); }

// gradcheck.rs:31-52
void assert_grad_close(const std::string& name, const Vec32& a, const Vec64& n, double tol) {
    if (a.size() != n.size()) return fail(name + ": length mismatch");
    double worst = 0.0;
    size_t wi = 0;
    for (size_t i = 0; i < a.size(); i++) {
        const double err = std::fabs((double)a[i] - n[i]) / (1.0 + std::fabs(n[i]));
        if (err > worst) {
            worst = err;
            wi = i;
        }
    }
    if (worst > tol) {
        char buf[256];
        std::snprintf(buf, sizeof buf, "%s: worst relative error %.3e at index %zu (analytic %g, numeric %g), tol %.1e",
                      name.c_str(), worst, wi, (double)a[wi], n[wi], tol);
        fail(buf);
    }
}

// attention.rs:271-296
Vec64 attn_ref(const Vec64& q, const Vec64& k, const Vec64& v, AttnShape s) {
    const size_t hd = s.head_dim, group = s.n_heads / s.n_kv;
    Vec64 o(s.seq * s.n_heads * hd, 0.0);
    for (size_t h = 0; h < s.n_heads; h++) {
        const size_t g = h / group;
        for (size_t t = 0; t < s.seq; t++) {
            const double* qv = &q[(t * s.n_heads + h) * hd];
            Vec64 scores;
            for (size_t j = 0; j <= t; j++) {
                const double* kv = &k[(j * s.n_kv + g) * hd];
                double dot = 0.0;
                for (size_t d = 0; d < hd; d++) dot += qv[d] * kv[d];
                scores.push_back(dot / std::sqrt((double)hd));
            }
            double mx = -INFINITY;
            for (double x : scores) mx = std::fmax(mx, x);
            Vec64 e(scores.size());
            double sum = 0.0;
            for (size_t j = 0; j < scores.size(); j++) sum += (e[j] = std::exp(scores[j] - mx));
            for (size_t j = 0; j < e.size(); j++) {
                const double* vv = &v[(j * s.n_kv + g) * hd];
                for (size_t d = 0; d < hd; d++) o[(t * s.n_heads + h) * hd + d] += e[j] / sum * vv[d];
            }
        }
    }
    return o;
}

// attention.rs:298-301
Vec32 rand_vec(size_t n, uint64_t seed, float std) {
    Vec32 out(n);
    orc_fill_normal(seed, out.data(), n, std);
    return out;
}

struct Case {
    Vec32 q, k, v;
    AttnShape s;
};

// attention.rs:310-318
Case make_case(size_t seq, size_t n_heads, size_t n_kv, size_t hd, uint64_t seed) {
    AttnShape s{seq, n_heads, n_kv, hd};
    return Case{rand_vec(seq * n_heads * hd, seed, 1.0f), rand_vec(seq * n_kv * hd, seed + 1, 1.0f),
                rand_vec(seq * n_kv * hd, seed + 2, 1.0f), s};
}

// attention.rs:320-322
struct CaseDims {
    size_t seq, h, kv, hd, qb;
};
const CaseDims CASES[] = {{8, 4, 2, 6, 3}, {10, 3, 1, 4, 4}, {7, 2, 2, 8, 100}, {13, 6, 2, 4, 5}, {1, 2, 1, 4, 4}};

// attention.rs:324-334
void forward_matches_f64_reference() {
    for (size_t i = 0; i < sizeof CASES / sizeof CASES[0]; i++) {
        const auto [seq, h, kv, hd, qb] = CASES[i];
        Case c = make_case(seq, h, kv, hd, 10 + i);
        Vec32 o(seq * h * hd, 0.0f), lse(h * seq, 0.0f);
        attention_forward_blocked(c.q, c.k, c.v, o, lse, c.s, qb);
        const Vec64 want = attn_ref(to_f64(c.q), to_f64(c.k), to_f64(c.v), c.s);
        assert_grad_close("attn fwd case " + std::to_string(i), o, want, 1e-4);
    }
}

// attention.rs:336-354
void block_size_does_not_change_result() {
    Case c = make_case(37, 4, 2, 8, 30);
    auto run = [&](size_t qb) {
        Vec32 o(37 * 4 * 8, 0.0f), lse(4 * 37, 0.0f);
        attention_forward_blocked(c.q, c.k, c.v, o, lse, c.s, qb);
        return std::make_pair(o, lse);
    };
    auto [o1, l1] = run(1);
    auto [o2, l2] = run(16);
    auto [o3, l3] = run(1000);
    for (size_t i = 0; i < o1.size(); i++)
        if (!(std::fabs(o1[i] - o2[i]) < 1e-5f && std::fabs(o1[i] - o3[i]) < 1e-5f))
            return fail("block_size_does_not_change_result: o[" + std::to_string(i) + "]");
    for (size_t i = 0; i < l1.size(); i++)
        if (!(std::fabs(l1[i] - l2[i]) < 1e-5f && std::fabs(l1[i] - l3[i]) < 1e-5f))
            return fail("block_size_does_not_change_result: lse[" + std::to_string(i) + "]");
}

// attention.rs:356-368
void first_token_attends_only_to_itself() {
    Case c = make_case(5, 2, 1, 4, 40);
    Vec32 o(5 * 2 * 4, 0.0f), lse(2 * 5, 0.0f);
    attention_forward(c.q, c.k, c.v, o, lse, c.s);
    for (size_t h = 0; h < 2; h++)
        for (size_t d = 0; d < 4; d++)
            if (!(std::fabs(o[h * 4 + d] - c.v[d]) < 1e-6f))
                return fail("first_token_attends_only_to_itself: h " + std::to_string(h) + " d " + std::to_string(d));
}

// attention.rs:370-393
void backward_matches_finite_differences() {
    for (size_t i = 0; i < sizeof CASES / sizeof CASES[0]; i++) {
        const auto [seq, h, kv, hd, qb] = CASES[i];
        Case c = make_case(seq, h, kv, hd, 50 + i);
        const Vec32 g = rand_vec(seq * h * hd, 70 + i, 1.0f);
        Vec32 o(seq * h * hd, 0.0f), lse(h * seq, 0.0f);
        attention_forward_blocked(c.q, c.k, c.v, o, lse, c.s, qb);
        Vec32 dq(c.q.size(), 0.0f), dk(c.k.size(), 0.0f), dv(c.v.size(), 0.0f);
        attention_backward_blocked(g, c.q, c.k, c.v, o, lse, dq, dk, dv, c.s, qb);
        const Vec64 q64 = to_f64(c.q), k64 = to_f64(c.k), v64 = to_f64(c.v), g64 = to_f64(g);
        auto loss = [&](const Vec64& out) {
            double acc = 0.0;
            for (size_t j = 0; j < out.size(); j++) acc += out[j] * g64[j];
            return acc;
        };
        const Vec64 nq = numeric_grad([&](const Vec64& x) { return loss(attn_ref(x, k64, v64, c.s)); }, q64, 1e-6);
        const Vec64 nk = numeric_grad([&](const Vec64& x) { return loss(attn_ref(q64, x, v64, c.s)); }, k64, 1e-6);
        const Vec64 nv = numeric_grad([&](const Vec64& x) { return loss(attn_ref(q64, k64, x, c.s)); }, v64, 1e-6);
        assert_grad_close("attn dq case " + std::to_string(i), dq, nq, 1e-3);
        assert_grad_close("attn dk case " + std::to_string(i), dk, nk, 1e-3);
        assert_grad_close("attn dv case " + std::to_string(i), dv, nv, 1e-3);
    }
}

// The reference panics on a shape mismatch (attention.rs:35-38, 55-58).
void shape_mismatch_panics() {
    Case c = make_case(4, 4, 2, 8, 1);
    Vec32 o(4 * 4 * 8 - 1, 0.0f), lse(4 * 4, 0.0f);  // o one element short
    try {
        attention_forward(c.q, c.k, c.v, o, lse, c.s);
        fail("shape_mismatch_panics: no panic for a short o");
    } catch (const cf_core::Panic& e) {
        if (std::string(e.what()).find("o.len()") == std::string::npos)
            fail(std::string("shape_mismatch_panics: unexpected message: ") + e.what());
    }
    try {
        AttnShape bad{4, 3, 2, 8};  // n_heads not a multiple of n_kv
        Vec32 q(4 * 3 * 8), k(4 * 2 * 8), v(4 * 2 * 8), oo(4 * 3 * 8), ll(3 * 4);
        attention_forward(q, k, v, oo, ll, bad);
        fail("shape_mismatch_panics: no panic for n_heads % n_kv != 0");
    } catch (const cf_core::Panic&) {
    }
}

}  // namespace

int main() {
    const std::pair<const char*, void (*)()> tests[] = {
        {"forward_matches_f64_reference", forward_matches_f64_reference},
        {"block_size_does_not_change_result", block_size_does_not_change_result},
        {"first_token_attends_only_to_itself", first_token_attends_only_to_itself},
        {"backward_matches_finite_differences", backward_matches_finite_differences},
        {"shape_mismatch_panics", shape_mismatch_panics},
    };
    for (const auto& [name, fn] : tests) {
        const int before = failures;
        std::printf("test %s ... ", name);
        std::fflush(stdout);
        fn();
        std::printf("%s\n", failures == before ? "ok" : "FAILED");
    }
    std::printf("%d failure(s)\n", failures);
    return failures ? 1 : 0;
}
