// Pinned, chunked, double-buffered host staging for the host-slice entry
// points (cfattn_attention_forward/backward and their _blocked forms), whose
// calling convention (crates/core/src/ops/attention.rs:42-154) hands over
// plain host slices on every call.
//
// A pageable hipMemcpyAsync runs well below the PCIe rate.  Here every
// transfer goes through two pinned host chunks: while the DMA engine moves
// one chunk, a pool of threads copies the next one between the caller's
// slice and the other chunk (one thread's memcpy also runs below the PCIe
// rate).  Uploads return once their last chunk is queued (the chunks'
// events guard their reuse); downloads return with the data in the caller's
// slice.  All transfers are queued on the context's stream, in order with
// its kernels.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <condition_variable>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>
#include "cfattn_ctx.hpp"

namespace cfcapi {

namespace {

constexpr size_t kStageChunk = (size_t)32 << 20;  // bytes per pinned chunk
constexpr size_t kCopyTask = (size_t)2 << 20;     // bytes per parallel memcpy task
constexpr int kCopyThreads = 8;                   // pool workers besides the calling thread

// Runs memcpy(dst + off, src + off, len) over [0, n) in kCopyTask pieces on
// the pool's threads and the caller's.
class CopyPool {
   public:
    CopyPool() {
        for (int i = 0; i < kCopyThreads; i++) th_.emplace_back([this] { loop(); });
    }
    ~CopyPool() {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_.notify_all();
        for (auto& t : th_) t.join();
    }
    void copy(void* dst, const void* src, size_t n) {
        if (n <= kCopyTask) {
            std::memcpy(dst, src, n);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(mu_);
            dst_ = static_cast<uint8_t*>(dst);
            src_ = static_cast<const uint8_t*>(src);
            n_ = n;
            tasks_ = (n + kCopyTask - 1) / kCopyTask;
            next_ = 0;
            done_ = 0;
            ++gen_;
        }
        cv_.notify_all();
        work();
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] { return done_ == tasks_; });
        dst_ = nullptr;
    }

   private:
    std::vector<std::thread> th_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    uint8_t* dst_ = nullptr;
    const uint8_t* src_ = nullptr;
    size_t n_ = 0, tasks_ = 0, next_ = 0, done_ = 0;
    unsigned long gen_ = 0;
    bool stop_ = false;

    void work() {
        while (true) {
            size_t t;
            uint8_t* d;
            const uint8_t* s;
            size_t n;
            {
                std::lock_guard<std::mutex> lk(mu_);
                if (!dst_ || next_ >= tasks_) return;
                t = next_++;
                d = dst_;
                s = src_;
                n = n_;
            }
            const size_t off = t * kCopyTask, len = std::min(kCopyTask, n - off);
            std::memcpy(d + off, s + off, len);
            std::lock_guard<std::mutex> lk(mu_);
            if (++done_ == tasks_) done_cv_.notify_all();
        }
    }
    void loop() {
        unsigned long seen = 0;
        while (true) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
                if (stop_) return;
                seen = gen_;
            }
            work();
        }
    }
};

struct HostStage {
    uint8_t* host[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool busy[2] = {false, false};
    int next = 0;  // chunk the next upload fills
    CopyPool pool;
};

void stage_release(void* p) {
    HostStage* s = static_cast<HostStage*>(p);
    for (int k = 0; k < 2; k++) {
        if (s->ev[k]) {
            (void)hipEventSynchronize(s->ev[k]);
            (void)hipEventDestroy(s->ev[k]);
        }
        if (s->host[k]) (void)hipHostFree(s->host[k]);
    }
    delete s;
}

HostStage* get_stage(cfattn_ctx* c, int* rc) {
    if (c->hs) return static_cast<HostStage*>(c->hs);
    HostStage* s = new HostStage;
    for (int k = 0; k < 2; k++) {
        void* h = nullptr;
        hipError_t e = hipHostMalloc(&h, kStageChunk, hipHostMallocDefault);
        if (e == hipSuccess) {
            s->host[k] = static_cast<uint8_t*>(h);
            e = hipEventCreateWithFlags(&s->ev[k], hipEventDisableTiming);
        }
        if (e != hipSuccess) {
            stage_release(s);
            *rc = fail(c, CFATTN_ERR_NOMEM, "pinned host staging of %zu bytes: %s", kStageChunk,
                       hipGetErrorString(e));
            return nullptr;
        }
    }
    c->hs = s;
    c->hs_release = stage_release;
    return s;
}

int wait_chunk(cfattn_ctx* c, HostStage* s, int k) {
    if (!s->busy[k]) return CFATTN_OK;
    const hipError_t e = hipEventSynchronize(s->ev[k]);
    if (e != hipSuccess) return hip_fail(c, e, "host staging wait");
    s->busy[k] = false;
    return CFATTN_OK;
}

}  // namespace

int stage_upload(cfattn_ctx* c, void* dev, const void* host, size_t bytes) {
    int rc = CFATTN_OK;
    HostStage* s = get_stage(c, &rc);
    if (!s) return rc;
    for (size_t off = 0; off < bytes; off += kStageChunk) {
        const size_t len = std::min(kStageChunk, bytes - off);
        const int k = s->next;
        s->next ^= 1;
        if ((rc = wait_chunk(c, s, k)) != CFATTN_OK) return rc;
        s->pool.copy(s->host[k], static_cast<const uint8_t*>(host) + off, len);
        hipError_t e = hipMemcpyAsync(static_cast<uint8_t*>(dev) + off, s->host[k], len, hipMemcpyHostToDevice,
                                      c->stream);
        if (e == hipSuccess) e = hipEventRecord(s->ev[k], c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "hipMemcpyAsync H2D (staged)");
        s->busy[k] = true;
    }
    return CFATTN_OK;
}

int stage_download(cfattn_ctx* c, void* host, const void* dev, size_t bytes) {
    int rc = CFATTN_OK;
    HostStage* s = get_stage(c, &rc);
    if (!s) return rc;
    const size_t n = (bytes + kStageChunk - 1) / kStageChunk;
    // Chunk i goes through pinned chunk i % 2; chunk i + 1's DMA is queued
    // before chunk i is copied out.
    auto issue = [&](size_t i) -> int {
        const int k = (int)(i & 1);
        int r = wait_chunk(c, s, k);
        if (r != CFATTN_OK) return r;
        const size_t off = i * kStageChunk, len = std::min(kStageChunk, bytes - off);
        hipError_t e = hipMemcpyAsync(s->host[k], static_cast<const uint8_t*>(dev) + off, len,
                                      hipMemcpyDeviceToHost, c->stream);
        if (e == hipSuccess) e = hipEventRecord(s->ev[k], c->stream);
        if (e != hipSuccess) return hip_fail(c, e, "hipMemcpyAsync D2H (staged)");
        s->busy[k] = true;
        return CFATTN_OK;
    };
    if (n == 0) return CFATTN_OK;
    if ((rc = issue(0)) != CFATTN_OK) return rc;
    for (size_t i = 0; i < n; i++) {
        if (i + 1 < n && (rc = issue(i + 1)) != CFATTN_OK) return rc;
        const int k = (int)(i & 1);
        if ((rc = wait_chunk(c, s, k)) != CFATTN_OK) return rc;
        const size_t off = i * kStageChunk, len = std::min(kStageChunk, bytes - off);
        s->pool.copy(static_cast<uint8_t*>(host) + off, s->host[k], len);
    }
    s->next = 0;
    return CFATTN_OK;
}

}  // namespace cfcapi
