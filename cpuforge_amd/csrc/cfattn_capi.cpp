// C ABI of libcfattn.so (declared in include/cfattn.h).
//
// Host-side plumbing only: argument checks that mirror the reference's
// asserts, a per-context stream and grow-only device buffer pool, host<->device
// copies for the host-slice entry points, and dispatch to the gfx950 kernels.
// There is no CPU compute path: every result comes from the HIP kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "cfattn.h"
#include "cfattn_ctx.hpp"
#include "cfattn_kernels.hpp"

namespace {

using namespace cfcapi;
using cfattn::Dims;
using cfattn::Dtype;

// Scratch for the stored-dS dQ path, or null (dQ recomputes the softmax)
// when the path does not apply, needs more than the context's limit, or the
// allocation fails.  Never an error: the recompute path needs no scratch.
void* ds_scratch(cfattn_ctx* c, Dtype dt, const Dims& d, size_t* bytes) {
    *bytes = cfattn::attn_bwd_ds_bytes(dt, d);
    // fp32: the slots alone when the stored dS does not fit under the limit.
    if (dt == cfattn::kF32 && *bytes > c->ds_limit) *bytes = cfattn::attn_f32_scratch_bytes(d);
    if (*bytes == 0 || *bytes > c->ds_limit) {
        *bytes = 0;
        return nullptr;
    }
    int rc = CFATTN_OK;
    void* p = slot(c, cfattn_ctx::DS, *bytes, &rc);
    if (!p) {
        c->err.clear();
        *bytes = 0;
    }
    return p;
}

// AttnShape::check plus the head-dim / size limits of the kernels
// (core/src/ops/attention.rs:35-38).
// Scratch for the forward's key split, or null (the grid runs unsplit) when
// the shape needs none, it is over the context's limit, or allocation fails.
void* fwd_scratch(cfattn_ctx* c, Dtype dt, const Dims& d, size_t* bytes) {
    *bytes = cfattn::attn_fwd_scratch_bytes(dt, d);
    if (*bytes == 0 || *bytes > c->ds_limit) {
        *bytes = 0;
        return nullptr;
    }
    int rc = CFATTN_OK;
    void* p = slot(c, cfattn_ctx::FWD_SPLIT, *bytes, &rc);
    if (!p) {
        c->err.clear();
        *bytes = 0;
    }
    return p;
}

int check_shape(cfattn_ctx* c, const cfattn_shape& s) {
    if (!(s.n_kv > 0 && s.n_heads % s.n_kv == 0))
        return fail(c, CFATTN_ERR_SHAPE, "n_heads must be a multiple of n_kv (n_heads=%zu, n_kv=%zu)", s.n_heads,
                    s.n_kv);
    if (s.head_dim == 0 || s.head_dim > (size_t)cfattn::kMaxHeadDim)
        return fail(c, CFATTN_ERR_UNSUPPORTED, "head_dim=%zu outside 1..=%d", s.head_dim, cfattn::kMaxHeadDim);
    const size_t lim = (size_t)1 << 31;
    if (s.seq >= lim || s.n_heads >= lim || s.seq * s.n_heads >= lim || s.seq * s.n_heads * s.head_dim >= lim)
        return fail(c, CFATTN_ERR_UNSUPPORTED, "shape too large (seq=%zu, n_heads=%zu, head_dim=%zu)", s.seq,
                    s.n_heads, s.head_dim);
    return CFATTN_OK;
}

int check_len(cfattn_ctx* c, const char* name, size_t got, size_t want) {
    if (got != want)
        return fail(c, CFATTN_ERR_SHAPE, "assertion `left == right` failed: %s.len() = %zu, expected %zu", name, got,
                    want);
    return CFATTN_OK;
}

int check_dtype(cfattn_ctx* c, int dt) {
    if (dt != CFATTN_F32 && dt != CFATTN_BF16) return fail(c, CFATTN_ERR_ARG, "unknown dtype %d", dt);
    return CFATTN_OK;
}

Dims dims_of(const cfattn_shape& s, size_t batch) {
    return Dims{(int)batch, (int)s.seq, (int)s.n_heads, (int)s.n_kv, (int)s.head_dim};
}

// Device entry points run on the caller's stream.  NULL is the device's null
// (default) stream, as everywhere in HIP, so work queued by other libraries
// on that stream (PyTorch's default stream, for one) stays ordered with ours.
hipStream_t pick_stream(cfattn_ctx*, void* st) { return static_cast<hipStream_t>(st); }



// Uploads an f32 host slice into a pool slot; with bf16 compute also rounds
// it into the matching bf16 slot.  Returns the device pointer the kernels read.
const void* upload(cfattn_ctx* c, int s32, int s16, const float* host, size_t n, bool bf16, int* rc) {
    float* d = static_cast<float*>(slot(c, s32, n * 4, rc));
    if (!d) return nullptr;
    if ((*rc = stage_upload(c, d, host, n * 4)) != CFATTN_OK) return nullptr;
    if (!bf16) return d;
    uint16_t* b = static_cast<uint16_t*>(slot(c, s16, n * 2, rc));
    if (!b) return nullptr;
    const hipError_t e = cfattn::launch_f32_to_bf16(d, b, n, c->stream);
    if (e != hipSuccess) {
        *rc = hip_fail(c, e, "f32_to_bf16 launch");
        return nullptr;
    }
    return b;
}

int forward_host(cfattn_ctx* c, const float* q, size_t q_len, const float* k, size_t k_len, const float* v,
                 size_t v_len, float* o, size_t o_len, float* lse, size_t lse_len, cfattn_shape s, size_t q_block) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    // attention.rs:55-58 order: shape check, then v, o and lse lengths.
    if (!(s.n_kv > 0 && s.n_heads % s.n_kv == 0)) CF_TRY(check_shape(c, s));
    CF_TRY(check_len(c, "q", q_len, s.seq * s.n_heads * s.head_dim));
    CF_TRY(check_len(c, "k", k_len, s.seq * s.n_kv * s.head_dim));
    CF_TRY(check_len(c, "v", v_len, k_len));
    CF_TRY(check_len(c, "o", o_len, q_len));
    CF_TRY(check_len(c, "lse", lse_len, s.n_heads * s.seq));
    if (q_block == 0) return fail(c, CFATTN_ERR_ARG, "q_block must be positive");
    if (s.seq == 0 || s.n_heads == 0) return CFATTN_OK;
    CF_TRY(check_shape(c, s));
    if (!q || !k || !v || !o || !lse) return fail(c, CFATTN_ERR_ARG, "null buffer");
    DeviceGuard dg(c->device);
    if (!dg.ok) return fail(c, CFATTN_ERR_HIP, "hipSetDevice(%d) failed", c->device);
    CF_TRY(order_after_device_calls(c));
    const bool bf = c->mode == CFATTN_BF16;
    int rc = CFATTN_OK;
    const void* dq = upload(c, cfattn_ctx::Q, cfattn_ctx::QB, q, q_len, bf, &rc);
    if (!dq) return rc;
    const void* dk = upload(c, cfattn_ctx::K, cfattn_ctx::KB, k, k_len, bf, &rc);
    if (!dk) return rc;
    const void* dv = upload(c, cfattn_ctx::V, cfattn_ctx::VB, v, v_len, bf, &rc);
    if (!dv) return rc;
    float* dout = static_cast<float*>(slot(c, cfattn_ctx::O, o_len * 4, &rc));
    if (!dout) return rc;
    float* dlse = static_cast<float*>(slot(c, cfattn_ctx::LSE, lse_len * 4, &rc));
    if (!dlse) return rc;
    size_t fs_bytes = 0;
    void* fs = fwd_scratch(c, bf ? cfattn::kBF16 : cfattn::kF32, dims_of(s, 1), &fs_bytes);
    CF_HIP(c, cfattn::launch_attn_fwd(bf ? cfattn::kBF16 : cfattn::kF32, dims_of(s, 1), dq, dk, dv, dout, dlse,
                                      c->stream, c->tuning(), fs, fs_bytes),
           "attention forward launch");
    CF_TRY(stage_download(c, o, dout, o_len * 4));
    CF_TRY(stage_download(c, lse, dlse, lse_len * 4));
    CF_HIP(c, hipStreamSynchronize(c->stream), "attention forward");
    return CFATTN_OK;
}

int backward_host(cfattn_ctx* c, const float* d_o, size_t d_o_len, const float* q, size_t q_len, const float* k,
                  size_t k_len, const float* v, size_t v_len, const float* o, size_t o_len, const float* lse,
                  size_t lse_len, float* dq, size_t dq_len, float* dk, size_t dk_len, float* dv, size_t dv_len,
                  cfattn_shape s, size_t q_block) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    // attention.rs:155-158 order.
    if (!(s.n_kv > 0 && s.n_heads % s.n_kv == 0)) CF_TRY(check_shape(c, s));
    CF_TRY(check_len(c, "q", q_len, s.seq * s.n_heads * s.head_dim));
    CF_TRY(check_len(c, "k", k_len, s.seq * s.n_kv * s.head_dim));
    CF_TRY(check_len(c, "v", v_len, k_len));
    CF_TRY(check_len(c, "dk", dk_len, k_len));
    CF_TRY(check_len(c, "dv", dv_len, k_len));
    CF_TRY(check_len(c, "d_o", d_o_len, q_len));
    CF_TRY(check_len(c, "o", o_len, q_len));
    CF_TRY(check_len(c, "dq", dq_len, q_len));
    CF_TRY(check_len(c, "lse", lse_len, s.n_heads * s.seq));
    if (q_block == 0) return fail(c, CFATTN_ERR_ARG, "q_block must be positive");
    if (s.seq == 0 || s.n_heads == 0) return CFATTN_OK;
    CF_TRY(check_shape(c, s));
    if (!d_o || !q || !k || !v || !o || !lse || !dq || !dk || !dv) return fail(c, CFATTN_ERR_ARG, "null buffer");
    DeviceGuard dg(c->device);
    if (!dg.ok) return fail(c, CFATTN_ERR_HIP, "hipSetDevice(%d) failed", c->device);
    CF_TRY(order_after_device_calls(c));
    const bool bf = c->mode == CFATTN_BF16;
    int rc = CFATTN_OK;
    const void* ddo = upload(c, cfattn_ctx::DO_, cfattn_ctx::DOB, d_o, d_o_len, bf, &rc);
    if (!ddo) return rc;
    const void* dq_in = upload(c, cfattn_ctx::Q, cfattn_ctx::QB, q, q_len, bf, &rc);
    if (!dq_in) return rc;
    const void* dk_in = upload(c, cfattn_ctx::K, cfattn_ctx::KB, k, k_len, bf, &rc);
    if (!dk_in) return rc;
    const void* dv_in = upload(c, cfattn_ctx::V, cfattn_ctx::VB, v, v_len, bf, &rc);
    if (!dv_in) return rc;
    const float* d_out = static_cast<const float*>(upload(c, cfattn_ctx::O, -1, o, o_len, false, &rc));
    if (!d_out) return rc;
    const float* d_lse = static_cast<const float*>(upload(c, cfattn_ctx::LSE, -1, lse, lse_len, false, &rc));
    if (!d_lse) return rc;
    float* g_q = static_cast<float*>(slot(c, cfattn_ctx::DQ, dq_len * 4, &rc));
    float* g_k = g_q ? static_cast<float*>(slot(c, cfattn_ctx::DK, dk_len * 4, &rc)) : nullptr;
    float* g_v = g_k ? static_cast<float*>(slot(c, cfattn_ctx::DV, dv_len * 4, &rc)) : nullptr;
    float* delta = g_v ? static_cast<float*>(slot(c, cfattn_ctx::DELTA, s.n_heads * s.seq * 8, &rc)) : nullptr;
    if (!delta) return rc;
    // The gradients accumulate (+=, attention.rs:145-154): their current
    // values go up with the inputs.
    CF_TRY(stage_upload(c, g_q, dq, dq_len * 4));
    CF_TRY(stage_upload(c, g_k, dk, dk_len * 4));
    CF_TRY(stage_upload(c, g_v, dv, dv_len * 4));
    size_t ds_bytes = 0;
    void* ds = ds_scratch(c, bf ? cfattn::kBF16 : cfattn::kF32, dims_of(s, 1), &ds_bytes);
    CF_HIP(c, cfattn::launch_attn_bwd(bf ? cfattn::kBF16 : cfattn::kF32, dims_of(s, 1), ddo, dq_in, dk_in, dv_in,
                                      d_out, d_lse, delta, g_q, g_k, g_v, c->stream, c->tuning(), ds, ds_bytes),
           "attention backward launch");
    CF_TRY(stage_download(c, dq, g_q, dq_len * 4));
    CF_TRY(stage_download(c, dk, g_k, dk_len * 4));
    CF_TRY(stage_download(c, dv, g_v, dv_len * 4));
    CF_HIP(c, hipStreamSynchronize(c->stream), "attention backward");
    return CFATTN_OK;
}

int check_prologue(cfattn_ctx* c, const cfattn_shape& s, const cfattn_prologue* pr) {
    if (!pr || !pr->cos || !pr->sin) return fail(c, CFATTN_ERR_ARG, "prologue needs a cos/sin table");
    if (s.head_dim % 2 != 0) return fail(c, CFATTN_ERR_SHAPE, "head_dim must be even");  // rope.rs:47
    if (pr->pos0 + s.seq > pr->max_pos)
        return fail(c, CFATTN_ERR_SHAPE, "position %zu exceeds cache size %zu", pr->pos0 + s.seq,
                    pr->max_pos);  // rope.rs:73
    if ((pr->q_norm == nullptr) != (pr->k_norm == nullptr))
        return fail(c, CFATTN_ERR_ARG, "q_norm and k_norm must both be given or both be NULL");
    if (pr->max_pos >= ((size_t)1 << 31)) return fail(c, CFATTN_ERR_UNSUPPORTED, "max_pos too large");
    return CFATTN_OK;
}

cfattn::Prologue to_prologue(const cfattn_prologue* pr) {
    cfattn::Prologue p;
    p.cos = pr->cos;
    p.sin = pr->sin;
    p.max_pos = (int)pr->max_pos;
    p.pos0 = (int)pr->pos0;
    p.qw = pr->q_norm;
    p.kw = pr->k_norm;
    p.eps = pr->eps;
    return p;
}

}  // namespace

extern "C" {

int cfattn_create(int device, cfattn_ctx** out) {
    if (!out) return CFATTN_ERR_ARG;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device < 0 || device >= n) return CFATTN_ERR_HIP;
    cfattn_ctx* c = new cfattn_ctx();
    c->device = device;
    DeviceGuard dg(device);
    if (!dg.ok || hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return CFATTN_ERR_HIP;
    }
    if (hipEventCreateWithFlags(&c->dev_done, hipEventDisableTiming) != hipSuccess) {
        (void)hipStreamDestroy(c->stream);
        delete c;
        return CFATTN_ERR_HIP;
    }
    // The fixed scratch of cfattn_bwd_noalloc on this device (looked up once
    // per device; a failure here is reported by that entry point, which
    // retries the lookup).
    (void)cfattn::noalloc_init_device(device);
    *out = c;
    return CFATTN_OK;
}

int cfattn_destroy(cfattn_ctx* c) {
    if (!c) return CFATTN_ERR_ARG;
    {
        DeviceGuard dg(c->device);
        if (c->stream) {
            (void)hipStreamSynchronize(c->stream);
            (void)hipStreamDestroy(c->stream);
        }
        delete c->timer;
        c->timer = nullptr;
        if (c->io && c->io_release) c->io_release(c->io);  // waits for its staging copies
        if (c->hs && c->hs_release) c->hs_release(c->hs);  // the same for the host-slice staging
        if (c->dev_done) (void)hipEventDestroy(c->dev_done);
        if (c->fwd_settles) (void)hipFree(c->fwd_settles);
        for (int i = 0; i < cfattn_ctx::NSLOT; i++)
            if (c->buf[i]) (void)hipFree(c->buf[i]);
        if (c->blas && c->blas_release) c->blas_release(c->blas);
    }
    delete c;
    return CFATTN_OK;
}

const char* cfattn_last_error(const cfattn_ctx* c) { return c ? c->err.c_str() : "null context"; }

int cfattn_set_mode(cfattn_ctx* c, int dtype) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    CF_TRY(check_dtype(c, dtype));
    c->mode = dtype;
    return CFATTN_OK;
}

int cfattn_get_mode(const cfattn_ctx* c) { return c ? c->mode : -1; }

int cfattn_synchronize(cfattn_ctx* c) {
    if (!c) return CFATTN_ERR_ARG;
    DeviceGuard dg(c->device);
    CF_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return CFATTN_OK;
}

void* cfattn_stream(cfattn_ctx* c) { return c ? static_cast<void*>(c->stream) : nullptr; }

int cfattn_attention_forward(cfattn_ctx* c, const float* q, size_t q_len, const float* k, size_t k_len,
                             const float* v, size_t v_len, float* o, size_t o_len, float* lse, size_t lse_len,
                             cfattn_shape s) {
    return forward_host(c, q, q_len, k, k_len, v, v_len, o, o_len, lse, lse_len, s, 128);
}

int cfattn_attention_forward_blocked(cfattn_ctx* c, const float* q, size_t q_len, const float* k, size_t k_len,
                                     const float* v, size_t v_len, float* o, size_t o_len, float* lse,
                                     size_t lse_len, cfattn_shape s, size_t q_block) {
    return forward_host(c, q, q_len, k, k_len, v, v_len, o, o_len, lse, lse_len, s, q_block);
}

int cfattn_attention_backward(cfattn_ctx* c, const float* d_o, size_t d_o_len, const float* q, size_t q_len,
                              const float* k, size_t k_len, const float* v, size_t v_len, const float* o,
                              size_t o_len, const float* lse, size_t lse_len, float* dq, size_t dq_len, float* dk,
                              size_t dk_len, float* dv, size_t dv_len, cfattn_shape s) {
    return backward_host(c, d_o, d_o_len, q, q_len, k, k_len, v, v_len, o, o_len, lse, lse_len, dq, dq_len, dk,
                         dk_len, dv, dv_len, s, 128);
}

int cfattn_attention_backward_blocked(cfattn_ctx* c, const float* d_o, size_t d_o_len, const float* q,
                                      size_t q_len, const float* k, size_t k_len, const float* v, size_t v_len,
                                      const float* o, size_t o_len, const float* lse, size_t lse_len, float* dq,
                                      size_t dq_len, float* dk, size_t dk_len, float* dv, size_t dv_len,
                                      cfattn_shape s, size_t q_block) {
    return backward_host(c, d_o, d_o_len, q, q_len, k, k_len, v, v_len, o, o_len, lse, lse_len, dq, dq_len, dk,
                         dk_len, dv, dv_len, s, q_block);
}

static int cfattn_fwd_locked(cfattn_ctx* c, cfattn_shape s, size_t batch, int dtype, const void* q, const void* k, const void* v,
               float* o, float* lse, void* stream) {
    CF_TRY(check_dtype(c, dtype));
    if (batch == 0 || s.seq == 0) return CFATTN_OK;
    CF_TRY(check_shape(c, s));
    if (batch * s.seq * s.n_heads >= ((size_t)1 << 31))
        return fail(c, CFATTN_ERR_UNSUPPORTED, "batch*seq*n_heads too large");
    if (!q || !k || !v || !o || !lse) return fail(c, CFATTN_ERR_ARG, "null buffer");
    DeviceGuard dg(c->device);
    size_t fs_bytes = 0;
    void* fs = fwd_scratch(c, (Dtype)dtype, dims_of(s, batch), &fs_bytes);
    CF_HIP(c, cfattn::launch_attn_fwd((Dtype)dtype, dims_of(s, batch), q, k, v, o, lse, pick_stream(c, stream),
                                      c->tuning(), fs, fs_bytes),
           "attention forward launch");
    return CFATTN_OK;
}

int cfattn_fwd(cfattn_ctx* c, cfattn_shape s, size_t batch, int dtype, const void* q, const void* k, const void* v,
               float* o, float* lse, void* stream) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    DeviceCallMark mark(c, pick_stream(c, stream));
    return cfattn_fwd_locked(c, s, batch, dtype, q, k, v, o, lse, stream);
}

static int cfattn_bwd_locked(cfattn_ctx* c, cfattn_shape s, size_t batch, int dtype, const void* d_o, const void* q, const void* k,
               const void* v, const float* o, const float* lse, float* dq, float* dk, float* dv, void* stream,
               const cfattn::BwdEpilogue* epi = nullptr) {
    CF_TRY(check_dtype(c, dtype));
    if (batch == 0 || s.seq == 0) return CFATTN_OK;
    CF_TRY(check_shape(c, s));
    if (batch * s.seq * s.n_heads >= ((size_t)1 << 31))
        return fail(c, CFATTN_ERR_UNSUPPORTED, "batch*seq*n_heads too large");
    if (!d_o || !q || !k || !v || !o || !lse || !dq || !dk || !dv) return fail(c, CFATTN_ERR_ARG, "null buffer");
    DeviceGuard dg(c->device);
    int rc = CFATTN_OK;
    float* delta = static_cast<float*>(slot(c, cfattn_ctx::DELTA, batch * s.n_heads * s.seq * 8, &rc));
    if (!delta) return rc;
    size_t ds_bytes = 0;
    void* ds = ds_scratch(c, (Dtype)dtype, dims_of(s, batch), &ds_bytes);
    CF_HIP(c, cfattn::launch_attn_bwd((Dtype)dtype, dims_of(s, batch), d_o, q, k, v, o, lse, delta, dq, dk, dv,
                                      pick_stream(c, stream), c->tuning(), ds, ds_bytes, epi),
           "attention backward launch");
    return CFATTN_OK;
}

int cfattn_bwd(cfattn_ctx* c, cfattn_shape s, size_t batch, int dtype, const void* d_o, const void* q, const void* k,
               const void* v, const float* o, const float* lse, float* dq, float* dk, float* dv, void* stream) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    DeviceCallMark mark(c, pick_stream(c, stream));
    return cfattn_bwd_locked(c, s, batch, dtype, d_o, q, k, v, o, lse, dq, dk, dv, stream);
}

int cfattn_bwd_noalloc(cfattn_ctx* c, cfattn_shape s, size_t batch, int dtype, const void* d_o, const void* q,
                       const void* k, const void* v, const float* o, const float* lse, float* dq, float* dk, float* dv,
                       void* stream) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    CF_TRY(check_dtype(c, dtype));
    if (batch == 0 || s.seq == 0) return CFATTN_OK;
    CF_TRY(check_shape(c, s));
    if (batch * s.seq * s.n_heads >= ((size_t)1 << 31))
        return fail(c, CFATTN_ERR_UNSUPPORTED, "batch*seq*n_heads too large");
    if (!d_o || !q || !k || !v || !o || !lse || !dq || !dk || !dv) return fail(c, CFATTN_ERR_ARG, "null buffer");
    // The only scratch of this path: two floats per (sequence, query head,
    // token), the delta row and the lse * log2(e) row.
    const size_t need = 2 * batch * s.n_heads * s.seq * sizeof(float);
    if (need > cfattn::kNoAllocScratchBytes)
        return fail(c, CFATTN_ERR_UNSUPPORTED,
                    "cfattn_bwd_noalloc: batch*n_heads*seq = %zu needs %zu bytes of scratch, above its fixed %zu",
                    batch * s.n_heads * s.seq, need, cfattn::kNoAllocScratchBytes);
    DeviceGuard dg(c->device);
    if (!dg.ok) return fail(c, CFATTN_ERR_HIP, "hipSetDevice(%d) failed", c->device);
    CF_HIP(c, cfattn::noalloc_init_device(c->device), "scratch symbol lookup");
    float* delta = static_cast<float*>(cfattn::noalloc_scratch(c->device));
    if (!delta) return fail(c, CFATTN_ERR_HIP, "no scratch address for device %d", c->device);
    // No timer (its events are created on demand) and no dS / slot scratch:
    // the bf16 backward recomputes the softmax for dQ, the fp32 backward
    // runs the generic kernels.
    cfattn::Tuning tu;
    CF_HIP(c, cfattn::launch_attn_bwd((Dtype)dtype, dims_of(s, batch), d_o, q, k, v, o, lse, delta, dq, dk, dv,
                                      pick_stream(c, stream), tu, nullptr, 0),
           "attention backward launch");
    return CFATTN_OK;
}

static int cfattn_prologue_fwd_locked(cfattn_ctx* c, cfattn_shape s, size_t batch, int dtype, const cfattn_prologue* pr,
                        const float* q_pre, const float* k_pre, void* q_out, void* k_out, float* q_rstd,
                        float* k_rstd, void* stream) {
    CF_TRY(check_dtype(c, dtype));
    if (batch == 0 || s.seq == 0) return CFATTN_OK;
    CF_TRY(check_shape(c, s));
    CF_TRY(check_prologue(c, s, pr));
    if (!q_pre || !k_pre || !q_out || !k_out) return fail(c, CFATTN_ERR_ARG, "null buffer");
    if (pr->q_norm && (!q_rstd || !k_rstd)) return fail(c, CFATTN_ERR_ARG, "q/k norm needs rstd outputs");
    DeviceGuard dg(c->device);
    CF_HIP(c, cfattn::launch_prologue_fwd((Dtype)dtype, dims_of(s, batch), to_prologue(pr), q_pre, k_pre, q_out,
                                          k_out, q_rstd, k_rstd, pick_stream(c, stream), c->timer),
           "prologue forward launch");
    return CFATTN_OK;
}

int cfattn_prologue_fwd(cfattn_ctx* c, cfattn_shape s, size_t batch, int dtype, const cfattn_prologue* pr,
                        const float* q_pre, const float* k_pre, void* q_out, void* k_out, float* q_rstd,
                        float* k_rstd, void* stream) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    return cfattn_prologue_fwd_locked(c, s, batch, dtype, pr, q_pre, k_pre, q_out, k_out, q_rstd, k_rstd, stream);
}

static int cfattn_prologue_bwd_locked(cfattn_ctx* c, cfattn_shape s, size_t batch, const cfattn_prologue* pr, const float* dq,
                        const float* dk, const float* q_pre, const float* k_pre, const float* q_rstd,
                        const float* k_rstd, float* dq_pre, float* dk_pre, float* dq_norm, float* dk_norm,
                        void* stream, bool unrotated = false) {
    if (batch == 0 || s.seq == 0) return CFATTN_OK;
    CF_TRY(check_shape(c, s));
    CF_TRY(check_prologue(c, s, pr));
    if (!dq || !dk || !dq_pre || !dk_pre) return fail(c, CFATTN_ERR_ARG, "null buffer");
    if (pr->q_norm && (!q_pre || !k_pre || !q_rstd || !k_rstd || !dq_norm || !dk_norm))
        return fail(c, CFATTN_ERR_ARG, "q/k norm backward needs q_pre, k_pre, rstd and gain-gradient buffers");
    DeviceGuard dg(c->device);
    const Dims d = dims_of(s, batch);
    int rc = CFATTN_OK;
    float* partial = nullptr;
    if (pr->q_norm) {
        partial = static_cast<float*>(slot(c, cfattn_ctx::PARTIAL, cfattn::prologue_bwd_scratch_floats(d) * 4, &rc));
        if (!partial) return rc;
    }
    CF_HIP(c, cfattn::launch_prologue_bwd(d, to_prologue(pr), dq, dk, q_pre, k_pre, q_rstd, k_rstd, dq_pre, dk_pre,
                                          dq_norm, dk_norm, partial, pick_stream(c, stream), c->timer, unrotated),
           "prologue backward launch");
    return CFATTN_OK;
}

int cfattn_prologue_bwd(cfattn_ctx* c, cfattn_shape s, size_t batch, const cfattn_prologue* pr, const float* dq,
                        const float* dk, const float* q_pre, const float* k_pre, const float* q_rstd,
                        const float* k_rstd, float* dq_pre, float* dk_pre, float* dq_norm, float* dk_norm,
                        void* stream) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    return cfattn_prologue_bwd_locked(c, s, batch, pr, dq, dk, q_pre, k_pre, q_rstd, k_rstd, dq_pre, dk_pre, dq_norm, dk_norm, stream);
}

int cfattn_fused_fwd(cfattn_ctx* c, cfattn_shape s, size_t batch, int dtype, const cfattn_prologue* pr,
                     const float* q_pre, const float* k_pre, const void* v, void* q_out, void* k_out, float* q_rstd,
                     float* k_rstd, float* o, float* lse, void* stream) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    DeviceCallMark mark(c, pick_stream(c, stream));
    CF_TRY(cfattn_prologue_fwd_locked(c, s, batch, dtype, pr, q_pre, k_pre, q_out, k_out, q_rstd, k_rstd, stream));
    return cfattn_fwd_locked(c, s, batch, dtype, q_out, k_out, v, o, lse, stream);
}

int cfattn_fused_bwd(cfattn_ctx* c, cfattn_shape s, size_t batch, int dtype, const cfattn_prologue* pr,
                     const void* d_o, const float* q_pre, const float* k_pre, const void* q, const void* k,
                     const void* v, const float* o, const float* lse, const float* q_rstd, const float* k_rstd,
                     float* dq_pre, float* dk_pre, float* dv, float* dq_norm, float* dk_norm, void* stream) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    DeviceCallMark mark(c, pick_stream(c, stream));
    CF_TRY(check_dtype(c, dtype));
    if (batch == 0 || s.seq == 0) return CFATTN_OK;
    CF_TRY(check_shape(c, s));
    CF_TRY(check_prologue(c, s, pr));
    DeviceGuard dg(c->device);
    int rc = CFATTN_OK;
    const size_t nq = batch * s.seq * s.n_heads * s.head_dim, nk = batch * s.seq * s.n_kv * s.head_dim;
    if (!d_o || !q || !k || !v || !dq_pre || !dk_pre || !dv) return fail(c, CFATTN_ERR_ARG, "null buffer");
    // The epilogue reads the cos/sin rows 16 bytes at a time: tables not
    // 16-byte aligned take the separate prologue backward instead.
    const bool tables16 = (reinterpret_cast<uintptr_t>(pr->cos) | reinterpret_cast<uintptr_t>(pr->sin)) % 16 == 0;
    if (tables16 && cfattn::attn_bwd_epilogue_applies((Dtype)dtype, dims_of(s, batch), d_o, q, k, v, dq_pre, dk_pre,
                                                      dv, c->tuning())) {
        // The fast kernels unrotate their dQ and dK rows themselves
        // (layer.rs:191-192): without the norm they add them into
        // dq_pre/dk_pre directly; with it they store the unrotated
        // gradients once, and the norm backward alone follows.
        const cfattn::Prologue P = to_prologue(pr);
        cfattn::BwdEpilogue epi;
        epi.cos = P.cos;
        epi.sin = P.sin;
        epi.pos0 = P.pos0;
        if (!pr->q_norm) {
            epi.mode = cfattn::kEpiUnrotAdd;
            return cfattn_bwd_locked(c, s, batch, dtype, d_o, q, k, v, o, lse, dq_pre, dk_pre, dv, stream, &epi);
        }
        if (!q_pre || !k_pre || !q_rstd || !k_rstd || !dq_norm || !dk_norm)
            return fail(c, CFATTN_ERR_ARG, "q/k norm backward needs q_pre, k_pre, rstd and gain-gradient buffers");
        // With the norm the epilogues also run its backward (layer.rs:195-206)
        // when its rows and gains can be read 16 bytes at a time: dq_pre/dk_pre
        // get the same bits as from the separate pass below, the gain
        // gradients the same sums in another fixed order.  Where the dK/dV
        // kernel has no norm epilogue (head_dim 128) it stores the unrotated
        // dK rows and K's norm backward runs as its own pass.
        const uintptr_t al = reinterpret_cast<uintptr_t>(q_pre) | reinterpret_cast<uintptr_t>(k_pre) |
                             reinterpret_cast<uintptr_t>(P.qw) | reinterpret_cast<uintptr_t>(P.kw);
        const cfattn::Tuning tu = c->tuning();
        if (tu.norm_epilogue && al % 16 == 0) {
            const cfattn::Dims dd = dims_of(s, batch);
            const bool kfused = cfattn::attn_bwd_norm_dk_epilogue(dd, tu);
            const size_t nf = cfattn::attn_bwd_norm_part_floats(dd, tu);
            const size_t pf = kfused ? nf : std::max(nf, cfattn::prologue_bwd_scratch_floats(dd));
            float* part = static_cast<float*>(slot(c, cfattn_ctx::PARTIAL, pf * 4, &rc));
            if (!part) return rc;
            float* dk_dst = dk_pre;
            if (!kfused) {
                dk_dst = static_cast<float*>(slot(c, cfattn_ctx::DKROT, nk * 4, &rc));
                if (!dk_dst) return rc;
            }
            epi.mode = cfattn::kEpiUnrotNorm;
            epi.mode_k = kfused ? cfattn::kEpiUnrotNorm : cfattn::kEpiUnrotStore;
            epi.norm.q_x = q_pre;
            epi.norm.k_x = k_pre;
            epi.norm.q_rstd = q_rstd;
            epi.norm.k_rstd = k_rstd;
            epi.norm.qw = P.qw;
            epi.norm.kw = P.kw;
            epi.norm.dqw = dq_norm;
            epi.norm.dkw = dk_norm;
            epi.norm.part = part;
            epi.norm.part_floats = nf;
            CF_TRY(cfattn_bwd_locked(c, s, batch, dtype, d_o, q, k, v, o, lse, dq_pre, dk_dst, dv, stream, &epi));
            if (kfused) return CFATTN_OK;
            CF_HIP(c,
                   cfattn::launch_prologue_bwd(dd, P, nullptr, dk_dst, nullptr, k_pre, nullptr, k_rstd, nullptr, dk_pre,
                                               nullptr, dk_norm, part, pick_stream(c, stream), c->timer,
                                               /*unrotated=*/true, /*k_only=*/true),
                   "prologue backward launch");
            return CFATTN_OK;
        }
        epi.mode = cfattn::kEpiUnrotStore;
        float* dy_q = static_cast<float*>(slot(c, cfattn_ctx::DQROT, nq * 4, &rc));
        if (!dy_q) return rc;
        float* dy_k = static_cast<float*>(slot(c, cfattn_ctx::DKROT, nk * 4, &rc));
        if (!dy_k) return rc;
        CF_TRY(cfattn_bwd_locked(c, s, batch, dtype, d_o, q, k, v, o, lse, dy_q, dy_k, dv, stream, &epi));
        return cfattn_prologue_bwd_locked(c, s, batch, pr, dy_q, dy_k, q_pre, k_pre, q_rstd, k_rstd, dq_pre, dk_pre,
                                          dq_norm, dk_norm, stream, /*unrotated=*/true);
    }
    float* dq_rot = static_cast<float*>(slot(c, cfattn_ctx::DQROT, nq * 4, &rc));
    if (!dq_rot) return rc;
    float* dk_rot = static_cast<float*>(slot(c, cfattn_ctx::DKROT, nk * 4, &rc));
    if (!dk_rot) return rc;
    hipStream_t st = pick_stream(c, stream);
    // Layer::backward starts from zeroed dq/dk (layer.rs:183-185).
    CF_HIP(c, cfattn::launch_fill_zero(dq_rot, nq, st), "zero dq");
    CF_HIP(c, cfattn::launch_fill_zero(dk_rot, nk, st), "zero dk");
    CF_TRY(cfattn_bwd_locked(c, s, batch, dtype, d_o, q, k, v, o, lse, dq_rot, dk_rot, dv, stream));
    return cfattn_prologue_bwd_locked(c, s, batch, pr, dq_rot, dk_rot, q_pre, k_pre, q_rstd, k_rstd, dq_pre, dk_pre,
                                      dq_norm, dk_norm, stream);
}

double cfattn_llama3_scale(const cfattn_llama3_scaling* sc, double inv_freq) {
    if (!sc) return inv_freq;
    const double pi = 3.14159265358979323846;
    const double wavelen = 2.0 * pi / inv_freq;
    const double low_wavelen = sc->original_max_position / sc->low_freq_factor;
    const double high_wavelen = sc->original_max_position / sc->high_freq_factor;
    if (wavelen < high_wavelen) return inv_freq;
    if (wavelen > low_wavelen) return inv_freq / sc->factor;
    const double smooth =
        (sc->original_max_position / wavelen - sc->low_freq_factor) / (sc->high_freq_factor - sc->low_freq_factor);
    return (1.0 - smooth) * inv_freq / sc->factor + smooth * inv_freq;
}

int cfattn_rope_table(size_t head_dim, size_t max_pos, double theta, const cfattn_llama3_scaling* scaling,
                      float* cos_out, float* sin_out) {
    if (head_dim % 2 != 0) return CFATTN_ERR_SHAPE;  // "head_dim must be even" (rope.rs:47)
    if ((!cos_out || !sin_out) && max_pos * head_dim > 0) return CFATTN_ERR_ARG;
    const size_t half = head_dim / 2;
    for (size_t pos = 0; pos < max_pos; pos++) {
        for (size_t i = 0; i < half; i++) {
            double inv_freq = std::pow(theta, -(2.0 * (double)i) / (double)head_dim);
            if (scaling) inv_freq = cfattn_llama3_scale(scaling, inv_freq);
            const double angle = (double)pos * inv_freq;
            cos_out[pos * half + i] = (float)std::cos(angle);
            sin_out[pos * half + i] = (float)std::sin(angle);
        }
    }
    return CFATTN_OK;
}

int cfattn_f32_to_bf16(cfattn_ctx* c, const float* src, uint16_t* dst, size_t n, void* stream) {
    if (!c) return CFATTN_ERR_ARG;
    if (n == 0) return CFATTN_OK;
    if (!src || !dst) return fail(c, CFATTN_ERR_ARG, "null buffer");
    DeviceGuard dg(c->device);
    CF_HIP(c, cfattn::launch_f32_to_bf16(src, dst, n, pick_stream(c, stream)), "f32_to_bf16 launch");
    return CFATTN_OK;
}

int cfattn_set_ds_limit(cfattn_ctx* c, size_t bytes) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    c->ds_limit = bytes;
    for (int sl : {(int)cfattn_ctx::DS, (int)cfattn_ctx::FWD_SPLIT}) {
        if (c->buf[sl] && c->cap[sl] > bytes) {
            DeviceGuard dg(c->device);
            (void)hipFree(c->buf[sl]);
            c->buf[sl] = nullptr;
            c->cap[sl] = 0;
        }
    }
    return CFATTN_OK;
}

size_t cfattn_get_ds_limit(const cfattn_ctx* c) { return c ? c->ds_limit : 0; }

int cfattn_fwd_stats_enable(cfattn_ctx* c, int on) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    DeviceGuard dg(c->device);
    if (on) {
        if (!c->fwd_settles) CF_HIP(c, hipMalloc(reinterpret_cast<void**>(&c->fwd_settles), sizeof(unsigned)), "hipMalloc");
        CF_HIP(c, hipMemsetAsync(c->fwd_settles, 0, sizeof(unsigned), c->stream), "hipMemsetAsync");
        CF_HIP(c, hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    } else if (c->fwd_settles) {
        CF_HIP(c, hipDeviceSynchronize(), "hipDeviceSynchronize");
        (void)hipFree(c->fwd_settles);
        c->fwd_settles = nullptr;
    }
    return CFATTN_OK;
}

int cfattn_fwd_stats_read(cfattn_ctx* c, long long* settles) {
    if (!c || !settles) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    if (!c->fwd_settles) return fail(c, CFATTN_ERR_ARG, "forward statistics are not enabled");
    DeviceGuard dg(c->device);
    unsigned v = 0;
    CF_HIP(c, hipDeviceSynchronize(), "hipDeviceSynchronize");
    CF_HIP(c, hipMemcpy(&v, c->fwd_settles, sizeof(unsigned), hipMemcpyDeviceToHost), "hipMemcpy");
    *settles = (long long)v;
    return CFATTN_OK;
}

int cfattn_probe_mfma_peak(cfattn_ctx* c, int zeros, int iters, double* tflops) {
    if (!c || !tflops) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    if (iters <= 0) return fail(c, CFATTN_ERR_ARG, "iters must be positive (got %d)", iters);
    DeviceGuard dg(c->device);
    CF_HIP(c, cfattn::probe_mfma_bf16(c->stream, zeros, iters, tflops), "MFMA probe");
    return CFATTN_OK;
}

int cfattn_probe_loop(cfattn_ctx* c, int kind, int iters, double* rate) {
    if (!c || !rate) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    if (iters <= 0) return fail(c, CFATTN_ERR_ARG, "iters must be positive (got %d)", iters);
    if (kind != cfattn::kProbeLds && kind != cfattn::kProbeValu && kind != cfattn::kProbeMfma16)
        return fail(c, CFATTN_ERR_ARG, "unknown probe %d", kind);
    DeviceGuard dg(c->device);
    CF_HIP(c, cfattn::probe_loop(c->stream, kind, iters, rate), "loop probe");
    return CFATTN_OK;
}

int cfattn_profile_enable(cfattn_ctx* c, int on) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    DeviceGuard dg(c->device);
    if (on) {
        if (!c->timer) c->timer = new EventTimer();
        (void)c->timer->collect();
        c->timer->reset();
        c->timer->mask = c->prof_mask;
    } else if (c->timer) {
        delete c->timer;
        c->timer = nullptr;
    }
    return CFATTN_OK;
}

int cfattn_profile_select(cfattn_ctx* c, unsigned kernel_mask) {
    if (!c) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    c->prof_mask = kernel_mask;
    if (c->timer) c->timer->mask = kernel_mask;
    return CFATTN_OK;
}

int cfattn_profile_read(cfattn_ctx* c, int kernel, double* total_ms, long long* launches) {
    if (!c || !total_ms || !launches) return CFATTN_ERR_ARG;
    std::lock_guard<std::mutex> lk(c->mu);
    c->err.clear();
    if (kernel < 0 || kernel >= cfattn::kNumKernels) return fail(c, CFATTN_ERR_ARG, "unknown kernel id %d", kernel);
    if (!c->timer) return fail(c, CFATTN_ERR_ARG, "profiling is not enabled");
    DeviceGuard dg(c->device);
    CF_HIP(c, c->timer->collect(), "profile event");
    *total_ms = c->timer->total_ms[kernel];
    *launches = c->timer->launches[kernel];
    return CFATTN_OK;
}

const char* cfattn_kernel_name(int kernel) {
    static const char* names[cfattn::kNumKernels] = {"attn_fwd", "attn_bwd_delta", "attn_bwd_dkdv", "attn_bwd_dq",
                                                      "prologue_fwd", "prologue_bwd"};
    return kernel >= 0 && kernel < cfattn::kNumKernels ? names[kernel] : nullptr;
}

int cfattn_kernel_count(void) { return cfattn::kNumKernels; }

double cfattn_flops_fwd_bwd(cfattn_shape s, size_t batch) {
    return 7.0 * (double)batch * (double)s.n_heads * (double)s.head_dim * (double)s.seq * ((double)s.seq + 1.0);
}

const char* cfattn_version(void) { return "cfattn 0.1.0 (gfx950)"; }

}  // extern "C"
