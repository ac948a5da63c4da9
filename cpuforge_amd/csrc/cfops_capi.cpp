// C ABI of the layer ops (declared in include/cfops.h).
//
// Host-side plumbing only: argument checks, scratch from the context's pool,
// hipBLASLt for the plain f32 GEMMs of matmul_* and Linear, and dispatch to
// the gfx950 kernels of layer_ops.hip.  There is no CPU compute path.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <climits>
#include <cstddef>
#include <cstring>
#include <map>
#include <tuple>

#include "cfattn_ctx.hpp"
#include "cfops.h"
#include "cfops_kernels.hpp"

namespace {

using namespace cfcapi;

hipStream_t to_stream(void* st) { return static_cast<hipStream_t>(st); }

// hipBLASLt state of a context: the handle and, per GEMM shape, the
// descriptors and the algorithm its heuristic picked (queried once).
struct GemmPlan {
    hipblasLtMatmulDesc_t op = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t ws = 0;
};
struct BlasState {
    hipblasLtHandle_t h = nullptr;
    std::map<std::tuple<int, size_t, size_t, size_t>, GemmPlan> plans;
    ~BlasState() {
        for (auto& kv : plans) {
            GemmPlan& p = kv.second;
            if (p.a) (void)hipblasLtMatrixLayoutDestroy(p.a);
            if (p.b) (void)hipblasLtMatrixLayoutDestroy(p.b);
            if (p.c) (void)hipblasLtMatrixLayoutDestroy(p.c);
            if (p.op) (void)hipblasLtMatmulDescDestroy(p.op);
        }
        if (h) (void)hipblasLtDestroy(h);
    }
};
constexpr size_t kGemmWorkspace = (size_t)32 << 20;

void release_blas(void* p) { delete static_cast<BlasState*>(p); }

BlasState* blas(cfattn_ctx* c, int* rc) {
    if (!c->blas) {
        BlasState* bs = new BlasState();
        if (hipblasLtCreate(&bs->h) != HIPBLAS_STATUS_SUCCESS) {
            delete bs;
            *rc = fail(c, CFATTN_ERR_HIP, "hipblasLtCreate failed");
            return nullptr;
        }
        c->blas = bs;
        c->blas_release = release_blas;
    }
    return static_cast<BlasState*>(c->blas);
}

bool fits_int(size_t x) { return x <= (size_t)INT_MAX; }

// Row-major C[m,n] = alpha * op(A) op(B) (+ C when acc), as matmul.rs's
// matmul_nn / matmul_nt / matmul_tn (core/src/matmul.rs:127-147).  hipBLASLt
// is column-major, so it computes C^T = op(B)^T op(A)^T on the same memory:
// an n x m column-major product whose first operand is B.  f32 inputs,
// f32 compute (HIPBLAS_COMPUTE_32F, no reduced-precision shortcut).
int gemm(cfattn_ctx* c, int kind, const float* a, const float* b, float* out, size_t m, size_t k, size_t n,
         float alpha, bool acc, hipStream_t st) {
    if (m == 0 || n == 0) return CFATTN_OK;
    if (!fits_int(m) || !fits_int(n) || !fits_int(k))
        return fail(c, CFATTN_ERR_UNSUPPORTED, "GEMM dimension above 2^31 (m=%zu, k=%zu, n=%zu)", m, k, n);
    if (k == 0) {  // matmul.rs:58-67: zero C unless accumulating
        if (!acc) CF_HIP(c, cfattn::launch_fill_zero(out, m * n, st), "zero-fill launch");
        return CFATTN_OK;
    }
    if (kind != CFOPS_NN && kind != CFOPS_NT && kind != CFOPS_TN)
        return fail(c, CFATTN_ERR_ARG, "unknown matmul kind %d", kind);
    int rc = CFATTN_OK;
    BlasState* bs = blas(c, &rc);
    if (!bs) return rc;
    void* ws = slot(c, cfattn_ctx::OPS_WS, kGemmWorkspace, &rc);
    if (!ws) return rc;
    auto key = std::make_tuple(kind, m, k, n);
    auto it = bs->plans.find(key);
    if (it == bs->plans.end()) {
        GemmPlan p;
        // First operand (B) and second (A) of the column-major product, as
        // stored: NN  B n x k (ld n), A k x m (ld k);  NT  B k x n (ld k)
        // transposed, A k x m;  TN  B n x k, A m x k (ld m) transposed.
        const hipblasOperation_t ta = kind == CFOPS_NT ? HIPBLAS_OP_T : HIPBLAS_OP_N;
        const hipblasOperation_t tb = kind == CFOPS_TN ? HIPBLAS_OP_T : HIPBLAS_OP_N;
        const uint64_t ar = ta == HIPBLAS_OP_N ? n : k, ac = ta == HIPBLAS_OP_N ? k : n;
        const uint64_t br = tb == HIPBLAS_OP_N ? k : m, bc = tb == HIPBLAS_OP_N ? m : k;
        bool ok = hipblasLtMatmulDescCreate(&p.op, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS;
        ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta) ==
                       HIPBLAS_STATUS_SUCCESS;
        ok = ok && hipblasLtMatmulDescSetAttribute(p.op, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb) ==
                       HIPBLAS_STATUS_SUCCESS;
        ok = ok && hipblasLtMatrixLayoutCreate(&p.a, HIP_R_32F, ar, ac, (int64_t)ar) == HIPBLAS_STATUS_SUCCESS;
        ok = ok && hipblasLtMatrixLayoutCreate(&p.b, HIP_R_32F, br, bc, (int64_t)br) == HIPBLAS_STATUS_SUCCESS;
        ok = ok && hipblasLtMatrixLayoutCreate(&p.c, HIP_R_32F, n, m, (int64_t)n) == HIPBLAS_STATUS_SUCCESS;
        hipblasLtMatmulPreference_t pref = nullptr;
        ok = ok && hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS;
        const uint64_t wsb = kGemmWorkspace;
        ok = ok && hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsb,
                                                         sizeof wsb) == HIPBLAS_STATUS_SUCCESS;
        hipblasLtMatmulHeuristicResult_t res[1];
        int nres = 0;
        ok = ok && hipblasLtMatmulAlgoGetHeuristic(bs->h, p.op, p.a, p.b, p.c, p.c, pref, 1, res, &nres) ==
                       HIPBLAS_STATUS_SUCCESS && nres > 0;
        if (pref) (void)hipblasLtMatmulPreferenceDestroy(pref);
        if (ok) {
            p.algo = res[0].algo;
            p.ws = res[0].workspaceSize;
        }
        it = bs->plans.emplace(key, p).first;
        if (!ok) {
            bs->plans.erase(it);
            if (p.a) (void)hipblasLtMatrixLayoutDestroy(p.a);
            if (p.b) (void)hipblasLtMatrixLayoutDestroy(p.b);
            if (p.c) (void)hipblasLtMatrixLayoutDestroy(p.c);
            if (p.op) (void)hipblasLtMatmulDescDestroy(p.op);
            return fail(c, CFATTN_ERR_HIP, "hipBLASLt has no f32 GEMM for kind %d m=%zu k=%zu n=%zu", kind, m, k, n);
        }
    }
    const GemmPlan& p = it->second;
    const float beta = acc ? 1.0f : 0.0f;
    const hipblasStatus_t s = hipblasLtMatmul(bs->h, p.op, &alpha, b, p.a, a, p.b, &beta, out, p.c, out, p.c, &p.algo,
                                              ws, p.ws, st);
    if (s != HIPBLAS_STATUS_SUCCESS) return fail(c, CFATTN_ERR_HIP, "hipblasLtMatmul failed (status %d)", (int)s);
    return CFATTN_OK;
}

// Rust's f32::powi at run time (compiler-rt __powisf2): square-and-multiply
// from the low bit of the exponent, reciprocal for a negative one.
float powi_f32(float a, int b) {
    const bool recip = b < 0;
    unsigned int e = recip ? (unsigned int)(-(long)b) : (unsigned int)b;
    float r = 1.0f;
    for (;;) {
        if (e & 1u) r *= a;
        e >>= 1;
        if (e == 0) break;
        a *= a;
    }
    return recip ? 1.0f / r : r;
}

// Reads the loss block after the stream has drained; reports a target out
// of range as the reference's panic message.
int ce_result(cfattn_ctx* c, const void* misc, const int64_t* targets, size_t vocab, float* loss, hipStream_t st) {
    cfattn::CeMisc m{};
    CF_HIP(c, hipMemcpyAsync(&m, misc, sizeof m, hipMemcpyDeviceToHost, st), "hipMemcpyAsync D2H loss");
    CF_HIP(c, hipStreamSynchronize(st), "cross-entropy");
    if (m.bad_row != INT_MAX) {
        int64_t t = 0;
        CF_HIP(c, hipMemcpy(&t, targets + m.bad_row, sizeof t, hipMemcpyDeviceToHost), "hipMemcpy D2H target");
        return fail(c, CFATTN_ERR_ARG, "target %lld out of range for vocab %zu", (long long)t, vocab);
    }
    *loss = m.loss;
    return CFATTN_OK;
}

#define CF_LOCK(c)                                                                        \
    if (!(c)) return CFATTN_ERR_ARG;                                                      \
    std::lock_guard<std::mutex> lk((c)->mu);                                              \
    (c)->err.clear();                                                                     \
    DeviceGuard dev_guard_((c)->device);                                                  \
    if (!dev_guard_.ok) return fail((c), CFATTN_ERR_HIP, "hipSetDevice(%d) failed", (c)->device);

}  // namespace

extern "C" {

int cfops_matmul(cfattn_ctx* c, int kind, const float* a, const float* b, float* out, size_t m, size_t k, size_t n,
                 int acc, void* stream) {
    CF_LOCK(c);
    if ((m && n && !out) || (m && n && k && (!a || !b))) return fail(c, CFATTN_ERR_ARG, "null buffer");
    return gemm(c, kind, a, b, out, m, k, n, 1.0f, acc != 0, to_stream(stream));
}

int cfops_rmsnorm_forward(cfattn_ctx* c, const float* x, const float* w, float* y, float* rstd, size_t rows,
                          size_t dim, float eps, void* stream) {
    CF_LOCK(c);
    if (rows == 0 || dim == 0) return CFATTN_OK;
    if (!x || !w || !y || !rstd) return fail(c, CFATTN_ERR_ARG, "null buffer");
    if (!fits_int(dim)) return fail(c, CFATTN_ERR_UNSUPPORTED, "dim=%zu above 2^31", dim);
    CF_HIP(c, cfattn::launch_rmsnorm_fwd(x, w, y, rstd, rows, dim, eps, to_stream(stream)), "rmsnorm forward launch");
    return CFATTN_OK;
}

int cfops_rmsnorm_backward(cfattn_ctx* c, const float* dy, const float* x, const float* w, const float* rstd,
                           float* dx, float* dw, size_t rows, size_t dim, void* stream) {
    CF_LOCK(c);
    if (rows == 0 || dim == 0) return CFATTN_OK;
    if (!dy || !x || !w || !rstd || !dx) return fail(c, CFATTN_ERR_ARG, "null buffer");
    if (!fits_int(dim)) return fail(c, CFATTN_ERR_UNSUPPORTED, "dim=%zu above 2^31", dim);
    float* partial = nullptr;
    if (dw) {
        int rc = CFATTN_OK;
        partial = static_cast<float*>(
            slot(c, cfattn_ctx::OPS_PARTIAL, cfattn::rmsnorm_bwd_partial_floats(rows, dim) * sizeof(float), &rc));
        if (!partial) return rc;
    }
    CF_HIP(c, cfattn::launch_rmsnorm_bwd(dy, x, w, rstd, dx, dw, partial, rows, dim, to_stream(stream)),
           "rmsnorm backward launch");
    return CFATTN_OK;
}

int cfops_silu_mul_forward(cfattn_ctx* c, const float* g, const float* u, float* h, size_t n, void* stream) {
    CF_LOCK(c);
    if (n == 0) return CFATTN_OK;
    if (!g || !u || !h) return fail(c, CFATTN_ERR_ARG, "null buffer");
    CF_HIP(c, cfattn::launch_silu_mul_fwd(g, u, h, n, to_stream(stream)), "silu_mul forward launch");
    return CFATTN_OK;
}

int cfops_silu_mul_backward(cfattn_ctx* c, const float* dh, const float* g, const float* u, float* dg, float* du,
                            size_t n, void* stream) {
    CF_LOCK(c);
    if (n == 0) return CFATTN_OK;
    if (!dh || !g || !u || !dg || !du) return fail(c, CFATTN_ERR_ARG, "null buffer");
    CF_HIP(c, cfattn::launch_silu_mul_bwd(dh, g, u, dg, du, n, to_stream(stream)), "silu_mul backward launch");
    return CFATTN_OK;
}

int cfops_cross_entropy_fwd_bwd(cfattn_ctx* c, const float* logits, const int64_t* targets, float* dlogits,
                                size_t rows, size_t vocab, float* loss, void* stream) {
    CF_LOCK(c);
    if (!loss) return fail(c, CFATTN_ERR_ARG, "null loss");
    *loss = 0.0f;
    if (rows == 0) return CFATTN_OK;
    if (!logits || !targets || !dlogits) return fail(c, CFATTN_ERR_ARG, "null buffer");
    if (rows > (size_t)INT_MAX) return fail(c, CFATTN_ERR_UNSUPPORTED, "rows=%zu above 2^31", rows);
    const hipStream_t st = to_stream(stream);
    int rc = CFATTN_OK;
    void* misc = slot(c, cfattn_ctx::OPS_MISC, cfattn::kCeMiscBytes, &rc);
    if (!misc) return rc;
    float* row_loss = static_cast<float*>(slot(c, cfattn_ctx::OPS_ROWLOSS, rows * sizeof(float), &rc));
    if (!row_loss) return rc;
    CF_HIP(c, cfattn::launch_ce_begin(targets, rows, misc, st), "cross-entropy launch");
    CF_HIP(c, cfattn::launch_ce_rows(logits, targets, dlogits, row_loss, 0, rows, vocab, misc, st),
           "cross-entropy launch");
    CF_HIP(c, cfattn::launch_ce_finish(targets, row_loss, rows, misc, st), "cross-entropy launch");
    return ce_result(c, misc, targets, vocab, loss, st);
}

int cfops_set_head_chunk_limit(cfattn_ctx* c, size_t bytes) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->head_chunk_bytes = bytes;
    return CFATTN_OK;
}

// The LM head and loss queued on `st` with the loss block at `misc` (device
// memory: n_valid, bad_row, loss); the caller holds the context lock and
// has checked the arguments.
static int lm_head_ce_queue(cfattn_ctx* c, const float* hn, const float* head, const int64_t* targets, size_t t, size_t d,
                     size_t vocab, float* dhn, float* dhead, void* misc, hipStream_t st) {
    size_t chunk = c->head_chunk_bytes / (vocab * sizeof(float));
    if (chunk < 1) chunk = 1;
    if (chunk > t) chunk = t;
    int rc = CFATTN_OK;
    float* row_loss = static_cast<float*>(slot(c, cfattn_ctx::OPS_ROWLOSS, t * sizeof(float), &rc));
    if (!row_loss) return rc;
    float* logits = static_cast<float*>(slot(c, cfattn_ctx::OPS_LOGITS, chunk * vocab * sizeof(float), &rc));
    if (!logits) return rc;
    CF_HIP(c, cfattn::launch_ce_begin(targets, t, misc, st), "cross-entropy launch");
    for (size_t r0 = 0; r0 < t; r0 += chunk) {
        const size_t nr = t - r0 < chunk ? t - r0 : chunk;
        // logits = hn . head^T (model.rs:438), then dlogits in place.
        CF_TRY(gemm(c, CFOPS_NT, hn + r0 * d, head, logits, nr, d, vocab, 1.0f, false, st));
        CF_HIP(c, cfattn::launch_ce_rows(logits, targets, logits, row_loss, r0, nr, vocab, misc, st),
               "cross-entropy launch");
        // dhn = dlogits . head (model.rs:454, overwritten); dhead += dlogits^T . hn (:457).
        CF_TRY(gemm(c, CFOPS_NN, logits, head, dhn + r0 * d, nr, vocab, d, 1.0f, false, st));
        if (dhead) CF_TRY(gemm(c, CFOPS_TN, logits, hn + r0 * d, dhead, vocab, nr, d, 1.0f, true, st));
    }
    CF_HIP(c, cfattn::launch_ce_finish(targets, row_loss, t, misc, st), "cross-entropy launch");
    return CFATTN_OK;
}

int cfops_lm_head_ce(cfattn_ctx* c, const float* hn, const float* head, const int64_t* targets, size_t t, size_t d,
                     size_t vocab, float* dhn, float* dhead, float* loss, void* stream) {
    CF_LOCK(c);
    if (!loss) return fail(c, CFATTN_ERR_ARG, "null loss");
    *loss = 0.0f;
    if (t == 0) return CFATTN_OK;
    if (!hn || !head || !targets || !dhn) return fail(c, CFATTN_ERR_ARG, "null buffer");
    if (vocab == 0) return fail(c, CFATTN_ERR_ARG, "vocab must be positive");
    if (t > (size_t)INT_MAX) return fail(c, CFATTN_ERR_UNSUPPORTED, "t=%zu above 2^31", t);
    const hipStream_t st = to_stream(stream);
    int rc = CFATTN_OK;
    void* misc = slot(c, cfattn_ctx::OPS_MISC, cfattn::kCeMiscBytes, &rc);
    if (!misc) return rc;
    CF_TRY(lm_head_ce_queue(c, hn, head, targets, t, d, vocab, dhn, dhead, misc, st));
    return ce_result(c, misc, targets, vocab, loss, st);
}

static_assert(sizeof(cfops_ce_result) == sizeof(cfattn::CeMisc) &&
                  offsetof(cfops_ce_result, bad_row) == offsetof(cfattn::CeMisc, bad_row) &&
                  offsetof(cfops_ce_result, loss) == offsetof(cfattn::CeMisc, loss),
              "cfops_ce_result is the kernels' loss block");

int cfops_lm_head_ce_dev(cfattn_ctx* c, const float* hn, const float* head, const int64_t* targets, size_t t,
                         size_t d, size_t vocab, float* dhn, float* dhead, cfops_ce_result* result, void* stream) {
    CF_LOCK(c);
    if (!result) return fail(c, CFATTN_ERR_ARG, "null result");
    if (t == 0) return fail(c, CFATTN_ERR_ARG, "t must be positive");
    if (!hn || !head || !targets || !dhn) return fail(c, CFATTN_ERR_ARG, "null buffer");
    if (vocab == 0) return fail(c, CFATTN_ERR_ARG, "vocab must be positive");
    if (t > (size_t)INT_MAX) return fail(c, CFATTN_ERR_UNSUPPORTED, "t=%zu above 2^31", t);
    return lm_head_ce_queue(c, hn, head, targets, t, d, vocab, dhn, dhead, result, to_stream(stream));
}

int cfops_linear_forward(cfattn_ctx* c, const float* x, const float* w, const float* lora_a, const float* lora_b,
                         float lora_scale, size_t t, size_t in, size_t out, size_t rank, float* y, float* xs,
                         void* stream) {
    CF_LOCK(c);
    if (t == 0 || out == 0) return CFATTN_OK;
    if (!x || !w || !y) return fail(c, CFATTN_ERR_ARG, "null buffer");
    if (lora_a && (!lora_b || !xs || rank == 0)) return fail(c, CFATTN_ERR_ARG, "adapter needs A, B, xs and rank > 0");
    const hipStream_t st = to_stream(stream);
    // linear.rs:58-69.  With an adapter on the streaming kernels' shapes the
    // adapter is folded into the weight, y = x (W + scale B A)^T in one GEMM
    // (the same sum, rounded once per element instead of twice), and xs is
    // formed beside it for the backward.
    const void* ptrs[] = {x, lora_a, lora_b, xs, w};
    if (lora_a && cfattn::lora_fused_applies(rank, t, in, out, ptrs, 5)) {
        int rc = CFATTN_OK;
        float* part = static_cast<float*>(
            slot(c, cfattn_ctx::OPS_LORA, cfattn::lora_partial_floats(rank, t, in, out) * sizeof(float), &rc));
        if (!part) return rc;
        float* weff = static_cast<float*>(slot(c, cfattn_ctx::OPS_WEFF, out * in * sizeof(float), &rc));
        if (!weff) return rc;
        CF_HIP(c, cfattn::launch_lora_merge(rank, w, lora_a, lora_b, lora_scale, out, in, weff, st),
               "lora merge launch");
        CF_TRY(gemm(c, CFOPS_NT, x, weff, y, t, in, out, 1.0f, false, st));
        CF_HIP(c, cfattn::launch_lora_fwd(rank, x, lora_a, lora_b, lora_scale, t, in, out, nullptr, xs, part, st),
               "lora forward launch");
        return CFATTN_OK;
    }
    CF_TRY(gemm(c, CFOPS_NT, x, w, y, t, in, out, 1.0f, false, st));
    if (!lora_a) return CFATTN_OK;
    CF_TRY(gemm(c, CFOPS_NT, x, lora_a, xs, t, in, rank, lora_scale, false, st));
    return gemm(c, CFOPS_NT, xs, lora_b, y, t, rank, out, 1.0f, true, st);
}

int cfops_linear_backward(cfattn_ctx* c, const float* x, const float* xs, const float* dy, const float* w,
                          const float* lora_a, const float* lora_b, float lora_scale, size_t t, size_t in, size_t out,
                          size_t rank, float* dx, float* gw, float* ga, float* gb, void* stream) {
    CF_LOCK(c);
    if (t == 0) return CFATTN_OK;
    if (!x || !dy || !w || !dx) return fail(c, CFATTN_ERR_ARG, "null buffer");
    if (lora_a && (!lora_b || !xs || rank == 0)) return fail(c, CFATTN_ERR_ARG, "adapter needs A, B, xs and rank > 0");
    const hipStream_t st = to_stream(stream);
    // linear.rs:75-90.  With an adapter on the streaming kernels' shapes,
    // dx += dy (W + scale B A) in one GEMM (the forward's folded weight),
    // and the adapter kernels form dxa = scale dy B and the adapter's
    // gradients only.
    int rc = CFATTN_OK;
    const void* ptrs[] = {x, xs, dy, lora_a, lora_b, w};
    if (lora_a && cfattn::lora_fused_applies(rank, t, in, out, ptrs, 6)) {
        float* weff = static_cast<float*>(slot(c, cfattn_ctx::OPS_WEFF, out * in * sizeof(float), &rc));
        if (!weff) return rc;
        CF_HIP(c, cfattn::launch_lora_merge(rank, w, lora_a, lora_b, lora_scale, out, in, weff, st),
               "lora merge launch");
        CF_TRY(gemm(c, CFOPS_NN, dy, weff, dx, t, out, in, 1.0f, true, st));
        if (gw) CF_TRY(gemm(c, CFOPS_TN, dy, x, gw, out, t, in, 1.0f, true, st));
        float* dxa = static_cast<float*>(slot(c, cfattn_ctx::OPS_DXA, t * rank * sizeof(float), &rc));
        if (!dxa) return rc;
        float* part = static_cast<float*>(
            slot(c, cfattn_ctx::OPS_LORA, cfattn::lora_partial_floats(rank, t, in, out) * sizeof(float), &rc));
        if (!part) return rc;
        CF_HIP(c, cfattn::launch_lora_bwd(rank, x, xs, dy, lora_a, lora_b, lora_scale, t, in, out, nullptr, ga, gb,
                                          dxa, part, st),
               "lora backward launch");
        return CFATTN_OK;
    }
    CF_TRY(gemm(c, CFOPS_NN, dy, w, dx, t, out, in, 1.0f, true, st));
    if (gw) CF_TRY(gemm(c, CFOPS_TN, dy, x, gw, out, t, in, 1.0f, true, st));
    if (!lora_a) return CFATTN_OK;
    if (gb) CF_TRY(gemm(c, CFOPS_TN, dy, xs, gb, out, t, rank, 1.0f, true, st));
    float* dxa = static_cast<float*>(slot(c, cfattn_ctx::OPS_DXA, t * rank * sizeof(float), &rc));
    if (!dxa) return rc;
    CF_TRY(gemm(c, CFOPS_NN, dy, lora_b, dxa, t, out, rank, lora_scale, false, st));
    if (ga) CF_TRY(gemm(c, CFOPS_TN, dxa, x, ga, rank, t, in, 1.0f, true, st));
    return gemm(c, CFOPS_NN, dxa, lora_a, dx, t, rank, in, 1.0f, true, st);
}

int cfops_adamw_update(cfattn_ctx* c, float* p, const float* g, float* m, float* v, size_t n, uint64_t t, float lr,
                       float beta1, float beta2, float eps, float weight_decay, void* stream) {
    CF_LOCK(c);
    if (n == 0) return CFATTN_OK;
    if (!p || !g || !m || !v) return fail(c, CFATTN_ERR_ARG, "null buffer");
    // optim.rs:21-22: the bias corrections, `t as i32` as in the reference.
    const float bc1 = 1.0f - powi_f32(beta1, (int)(int32_t)t);
    const float bc2 = 1.0f - powi_f32(beta2, (int)(int32_t)t);
    CF_HIP(c, cfattn::launch_adamw(p, g, m, v, n, lr, beta1, beta2, eps, weight_decay, bc1, bc2, to_stream(stream)),
           "adamw launch");
    return CFATTN_OK;
}

}  // extern "C"
