// Internal to libcfattn.so: the context behind the opaque cfattn_ctx handle
// of include/cfattn.h and the host helpers its C ABI files share
// (cfattn_capi.cpp for the attention, cfops_capi.cpp for the layer ops,
// cfio_capi.cpp for the on-disk formats).
#pragma once
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "cfattn.h"
#include "cfattn_kernels.hpp"

// Per-kernel timing for cfattn_profile_*: every launch a timed call queues is
// bracketed by two hipEvents recorded on the launch's stream; the elapsed
// times are summed when the caller reads them.
struct EventTimer final : cfattn::KernelTimer {
    struct Rec {
        int kernel;
        hipEvent_t a, b;
    };
    std::vector<hipEvent_t> pool;
    std::vector<Rec> pending;
    hipEvent_t open_ev = nullptr;
    int open_kernel = -1;
    double total_ms[cfattn::kNumKernels] = {};
    long long launches[cfattn::kNumKernels] = {};
    hipError_t err = hipSuccess;
    unsigned mask = ~0u;  // kernel ids bracketed (bit k: kernel k)

    hipEvent_t take() {
        if (!pool.empty()) {
            hipEvent_t e = pool.back();
            pool.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        hipError_t r = hipEventCreate(&e);
        if (r != hipSuccess && err == hipSuccess) err = r;
        return r == hipSuccess ? e : nullptr;
    }
    void begin(int kernel, hipStream_t st) override {
        if (!((mask >> kernel) & 1u)) {
            open_ev = nullptr;
            open_kernel = -1;
            return;
        }
        open_ev = take();
        open_kernel = kernel;
        if (open_ev) {
            hipError_t r = hipEventRecord(open_ev, st);
            if (r != hipSuccess && err == hipSuccess) err = r;
        }
    }
    void end(int kernel, hipStream_t st) override {
        hipEvent_t b = take();
        if (!open_ev || !b || kernel != open_kernel) {
            if (b) pool.push_back(b);
            return;
        }
        hipError_t r = hipEventRecord(b, st);
        if (r != hipSuccess && err == hipSuccess) err = r;
        pending.push_back(Rec{kernel, open_ev, b});
        open_ev = nullptr;
    }
    // Waits for every pending pair and folds it into the totals.
    hipError_t collect() {
        for (const Rec& r : pending) {
            hipError_t e = hipEventSynchronize(r.b);
            float ms = 0.0f;
            if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.a, r.b);
            if (e != hipSuccess && err == hipSuccess) err = e;
            total_ms[r.kernel] += ms;
            launches[r.kernel] += 1;
            pool.push_back(r.a);
            pool.push_back(r.b);
        }
        pending.clear();
        hipError_t e = err;
        err = hipSuccess;
        return e;
    }
    void reset() {
        for (int i = 0; i < cfattn::kNumKernels; i++) {
            total_ms[i] = 0.0;
            launches[i] = 0;
        }
    }
    ~EventTimer() override {
        for (const Rec& r : pending) {
            (void)hipEventSynchronize(r.b);
            pool.push_back(r.a);
            pool.push_back(r.b);
        }
        for (hipEvent_t e : pool) (void)hipEventDestroy(e);
    }
};

struct cfattn_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    int mode = CFATTN_F32;
    std::string err;
    std::mutex mu;
    enum Slot {
        Q, K, V, O, LSE, DO_, DQ, DK, DV, QB, KB, VB, DOB, DELTA, PARTIAL, DQROT, DKROT, DS, FWD_SPLIT,
        // layer ops (cfops_capi.cpp)
        OPS_PARTIAL, OPS_ROWLOSS, OPS_MISC, OPS_LOGITS, OPS_DXA, OPS_WS, OPS_LORA, OPS_WEFF,
        // on-disk formats (cfio_capi.cpp): the two device staging chunks
        IO_STAGE,
        NSLOT
    };
    void* buf[NSLOT] = {};
    size_t cap[NSLOT] = {};
    EventTimer* timer = nullptr;  // non-null while profiling is on
    unsigned prof_mask = ~0u;     // kernels profiling brackets (cfattn_profile_select)
    size_t ds_limit = (size_t)8 << 30;  // stored-dS scratch limit (cfattn_set_ds_limit)
    // GEMM library state of the layer ops (hipBLASLt handle and per-shape
    // plans), created on first use; released by cfattn_destroy through
    // blas_release.
    void* blas = nullptr;
    void (*blas_release)(void*) = nullptr;
    size_t head_chunk_bytes = (size_t)512 << 20;  // logits buffer limit of cfops_lm_head_ce
    // Pinned staging of the on-disk formats (two host chunks and their
    // events), created on first use; released by cfattn_destroy.
    void* io = nullptr;
    void (*io_release)(void*) = nullptr;
    size_t io_chunk = (size_t)8 << 20;
    // Pinned staging of the host-slice entry points (host_stage.cpp),
    // created on first use; released by cfattn_destroy.
    void* hs = nullptr;
    void (*hs_release)(void*) = nullptr;
    // Recorded on the caller's stream at the end of every device entry
    // point that uses the pool's attention slots; host-slice calls order
    // the context's stream after it before they reuse those slots.
    hipEvent_t dev_done = nullptr;
    bool dev_pending = false;
    // Device counter of the bf16 head_dim-128 forward's settled wave-tiles
    // while forward statistics are on (cfattn_fwd_stats_enable), else null.
    unsigned* fwd_settles = nullptr;

    cfattn::Tuning tuning() const {
        cfattn::Tuning t;
        t.timer = timer;
        t.fwd_settles = fwd_settles;
        // CFATTN_DKDV_KERNEL=ws selects the two-waves-per-SIMD dK/dV kernel
        // (bitwise equal results; kept for comparison and measurement).
        const char* v = std::getenv("CFATTN_DKDV_KERNEL");
        if (v && std::strcmp(v, "ws") == 0) t.dkdv_variant = cfattn::kDkdvWaveSpecialised;
        // CFATTN_FWD_KERNEL=two selects the two-waves-per-SIMD bf16 forward
        // at head_dim 128 (kept for comparison and measurement).
        const char* f = std::getenv("CFATTN_FWD_KERNEL");
        if (f && std::strcmp(f, "two") == 0) t.fwd_variant = cfattn::kFwdTwoPerSimd;
        // CFATTN_NORM_EPILOGUE=0 runs the fused backward's Qwen3 norm as its
        // own pass after the attention kernels (same dq_pre/dk_pre bits; kept
        // for comparison and measurement).
        const char* n = std::getenv("CFATTN_NORM_EPILOGUE");
        if (n && std::strcmp(n, "0") == 0) t.norm_epilogue = 0;
        // CFATTN_F32_GRID=unit launches the fp32 kernels with one workgroup
        // per work unit instead of persistent grids (same bits; kept for
        // comparison and measurement).
        const char* g = std::getenv("CFATTN_F32_GRID");
        if (g && std::strcmp(g, "unit") == 0) t.f32_persistent = 0;
        // CFATTN_F32_DS=0: the fp32 dQ recomputes S and dP instead of reading
        // the dS that dK/dV stored (same bits; kept for comparison).
        const char* fd = std::getenv("CFATTN_F32_DS");
        if (fd && std::strcmp(fd, "0") == 0) t.f32_stored_ds = 0;
        // CFATTN_BF16_GRID=unit: the same for the bf16 two-waves-per-SIMD
        // kernels.
        const char* h = std::getenv("CFATTN_BF16_GRID");
        if (h && std::strcmp(h, "unit") == 0) t.bf16_persistent = 0;
        return t;
    }
};

namespace cfcapi {

inline int fail(cfattn_ctx* c, int code, const char* fmt, ...) {
    char msg[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
    if (c) c->err = msg;
    return code;
}

inline int hip_fail(cfattn_ctx* c, hipError_t e, const char* what) {
    return fail(c, CFATTN_ERR_HIP, "%s: %s (%s)", what, hipGetErrorName(e), hipGetErrorString(e));
}

// Makes the context's device current for the duration of a call and restores
// the caller's device afterwards.
struct DeviceGuard {
    int prev = -1;
    bool ok = true;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) ok = hipSetDevice(dev) == hipSuccess;
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

// Grow-only device buffer of a pool slot.
inline void* slot(cfattn_ctx* c, int s, size_t bytes, int* rc) {
    if (bytes == 0) bytes = 256;
    if (c->cap[s] >= bytes) return c->buf[s];
    if (c->buf[s]) {
        (void)hipFree(c->buf[s]);
        c->buf[s] = nullptr;
        c->cap[s] = 0;
    }
    size_t want = (bytes + 4095) & ~(size_t)4095;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        *rc = fail(c, CFATTN_ERR_NOMEM, "hipMalloc of %zu bytes failed: %s", want, hipGetErrorString(e));
        return nullptr;
    }
    c->buf[s] = p;
    c->cap[s] = want;
    return p;
}

// Host-slice staging (host_stage.cpp): copies through two pinned chunks on
// the context's stream.  stage_upload returns once every chunk is queued
// (the caller's slice may then change); stage_download returns with the
// data in the caller's slice.
int stage_upload(cfattn_ctx* c, void* dev, const void* host, size_t bytes);
int stage_download(cfattn_ctx* c, void* host, const void* dev, size_t bytes);

// Marks the end of a device entry point's work on `st` (see dev_done).
struct DeviceCallMark {
    cfattn_ctx* c;
    hipStream_t st;
    DeviceCallMark(cfattn_ctx* c_, hipStream_t st_) : c(c_), st(st_) {}
    ~DeviceCallMark() {
        if (c->dev_done && hipEventRecord(c->dev_done, st) == hipSuccess) c->dev_pending = true;
    }
};

// Orders the context's stream after the last device entry point's work.
inline int order_after_device_calls(cfattn_ctx* c) {
    if (!c->dev_pending) return CFATTN_OK;
    const hipError_t e = hipStreamWaitEvent(c->stream, c->dev_done, 0);
    if (e != hipSuccess) return hip_fail(c, e, "hipStreamWaitEvent");
    c->dev_pending = false;
    return CFATTN_OK;
}

}  // namespace cfcapi

#define CF_TRY(expr)                 \
    do {                             \
        int _rc = (expr);            \
        if (_rc != CFATTN_OK) return _rc; \
    } while (0)

#define CF_HIP(c, expr, what)                                    \
    do {                                                         \
        hipError_t _e = (expr);                                  \
        if (_e != hipSuccess) return hip_fail((c), _e, (what));  \
    } while (0)
