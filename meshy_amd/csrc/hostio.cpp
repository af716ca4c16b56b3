// Host-side staging of jagged sample columns.
//
// The reference builds its step inputs from per-sample tensors with Python
// loops and torch.cat (trainer.py:644-667 for the critic path, batch.py:126-178
// for the micro-batches, metrics.py:197-212 for the rollout statistics).  Here
// every column is staged into one pinned buffer for a single host-to-device
// copy; meshy_host_gather does that concatenation on a small persistent pool of
// threads, split by bytes, instead of torch.cat's one thread.
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <thread>
#include <vector>

#include "host_common.h"

namespace meshy {
namespace {

// Below this many bytes per worker a gather runs on fewer threads.
constexpr int64_t kBytesPerWorker = 128 * 1024;
constexpr int kMaxWorkers = 16;

// One gather: pieces [0, n) of sizes nbytes[i] land at dst + start[i]; worker w
// copies output bytes [w * total / k, (w + 1) * total / k).  With to_u8 the
// pieces are fp32 masks of nbytes[i] floats, each written as one byte.
struct Job {
    const void* const* srcs = nullptr;
    const int64_t* nbytes = nullptr;
    const int64_t* start = nullptr;  // exclusive prefix of nbytes, n + 1 entries
    int64_t n = 0;
    char* dst = nullptr;
    int64_t total = 0;
    int workers = 0;
    bool to_u8 = false;   // fp32 pieces -> one byte each (nbytes[i] counts floats)
    bool to_i32 = false;  // int64 pieces -> int32 each (nbytes[i] counts int64s)
    mutable std::atomic<bool> nonbinary{false};  // a float other than +0.0 and 1.0 was seen
    mutable std::atomic<bool> overflow{false};   // an int64 outside int32 was seen
};

// int64 to int32; false when some value does not fit.
bool narrow_to_i32(const int64_t* src, int64_t count, int32_t* dst) {
    uint64_t bad = 0;
    for (int64_t k = 0; k < count; ++k) {
        const int64_t v = src[k];
        bad |= static_cast<uint64_t>(v != static_cast<int64_t>(static_cast<int32_t>(v)));
        dst[k] = static_cast<int32_t>(v);
    }
    return bad == 0;
}

// Floats to bytes; false when some float is not exactly +0.0 or 1.0.
bool mask_to_u8(const float* src, int64_t count, uint8_t* dst) {
    uint32_t bad = 0;
    for (int64_t k = 0; k < count; ++k) {
        uint32_t bits;
        std::memcpy(&bits, src + k, 4);
        const bool one = bits == 0x3f800000u;
        bad |= static_cast<uint32_t>(!one && bits != 0u);
        dst[k] = static_cast<uint8_t>(one);
    }
    return bad == 0;
}

void copy_share(const Job& j, int w) {
    const int64_t lo = j.total * w / j.workers;
    const int64_t hi = j.total * (w + 1) / j.workers;
    if (lo >= hi) return;
    // First piece overlapping [lo, hi).
    int64_t i = std::upper_bound(j.start, j.start + j.n + 1, lo) - j.start - 1;
    bool binary = true, fits = true;
    for (; i < j.n && j.start[i] < hi; ++i) {
        const int64_t a = std::max(lo, j.start[i]);
        const int64_t b = std::min(hi, j.start[i] + j.nbytes[i]);
        if (b <= a) continue;
        if (j.to_u8)
            binary &= mask_to_u8(static_cast<const float*>(j.srcs[i]) + (a - j.start[i]), b - a,
                                 reinterpret_cast<uint8_t*>(j.dst) + a);
        else if (j.to_i32)
            fits &= narrow_to_i32(static_cast<const int64_t*>(j.srcs[i]) + (a - j.start[i]), b - a,
                                  reinterpret_cast<int32_t*>(j.dst) + a);
        else
            std::memcpy(j.dst + a, static_cast<const char*>(j.srcs[i]) + (a - j.start[i]), b - a);
    }
    if (!binary) j.nonbinary.store(true, std::memory_order_relaxed);
    if (!fits) j.overflow.store(true, std::memory_order_relaxed);
}

// Workers sleep on a condition variable between jobs; the calling thread takes
// share 0 of each job.  One job at a time (callers serialise on run_mu).
class Pool {
  public:
    static Pool& get() {
        // A child process after fork() has none of the parent's threads: it
        // builds its own pool (the parent's object is left alone).
        static std::mutex mu;
        static Pool* pool = nullptr;
        std::lock_guard<std::mutex> lk(mu);
        if (!pool || pool->pid_ != getpid()) pool = new Pool();
        return *pool;
    }

    void run(const Job& job) {
        std::lock_guard<std::mutex> serial(run_mu_);
        const int helpers = job.workers - 1;
        {
            std::lock_guard<std::mutex> lk(mu_);
            job_ = &job;
            pending_ = helpers;
            next_ = 1;
            ++generation_;
        }
        cv_.notify_all();
        copy_share(job, 0);
        std::unique_lock<std::mutex> lk(mu_);
        done_cv_.wait(lk, [&] { return pending_ == 0; });
        job_ = nullptr;
    }

    int size() const { return static_cast<int>(threads_.size()) + 1; }

  private:
    Pool() : pid_(getpid()) {
        const unsigned hw = std::thread::hardware_concurrency();
        const int n = std::max(0, std::min<int>(kMaxWorkers, hw ? static_cast<int>(hw) : 1) - 1);
        for (int t = 0; t < n; ++t) threads_.emplace_back([this] { loop(); });
        for (auto& th : threads_) th.detach();
    }

    void loop() {
        uint64_t seen = 0;
        std::unique_lock<std::mutex> lk(mu_);
        for (;;) {
            cv_.wait(lk, [&] { return generation_ != seen; });
            seen = generation_;
            // Take shares while the job has any left.
            while (job_ && next_ < job_->workers) {
                const int w = next_++;
                const Job* j = job_;
                lk.unlock();
                copy_share(*j, w);
                lk.lock();
                if (--pending_ == 0) done_cv_.notify_one();
            }
        }
    }

    pid_t pid_;
    std::vector<std::thread> threads_;
    std::mutex run_mu_;
    std::mutex mu_;
    std::condition_variable cv_, done_cv_;
    const Job* job_ = nullptr;
    int pending_ = 0;
    int next_ = 0;
    uint64_t generation_ = 0;
};

}  // namespace
}  // namespace meshy

namespace meshy {
namespace {

// Every gather: sizes checked, then the job split over the pool.  mode 0
// copies bytes, 1 converts fp32 masks to bytes, 2 narrows int64 to int32
// (sizes then count elements); the bytes read per unit of size (1, 4, 8) set
// how many workers the job is worth.  `ok` reports the conversion's check.
int run_gather(const char* who, const void* const* srcs, const int64_t* sizes, int64_t n, void* dst,
               int max_threads, int mode, bool& ok) {
    const bool to_u8 = mode == 1;
    ok = true;
    if (n < 0) return set_error(MESHY_EINVAL, "%s: negative count", who);
    if (n == 0) return MESHY_OK;
    if (!srcs || !sizes || !dst) return set_error(MESHY_ENULL, "%s: NULL pointer", who);
    std::vector<int64_t> start(static_cast<size_t>(n) + 1);
    start[0] = 0;
    for (int64_t i = 0; i < n; ++i) {
        if (sizes[i] < 0)
            return set_error(MESHY_EINVAL, "%s: piece %lld has a negative size", who, static_cast<long long>(i));
        if (sizes[i] > 0 && !srcs[i])
            return set_error(MESHY_ENULL, "%s: piece %lld is NULL", who, static_cast<long long>(i));
        start[i + 1] = start[i] + sizes[i];
    }
    Job job;
    job.srcs = srcs;
    job.nbytes = sizes;
    job.start = start.data();
    job.n = n;
    job.dst = static_cast<char*>(dst);
    job.total = start[n];
    job.to_u8 = to_u8;
    job.to_i32 = mode == 2;
    Pool& pool = Pool::get();
    const int64_t want = std::max<int64_t>(1, job.total * (mode == 0 ? 1 : mode == 1 ? 4 : 8) / kBytesPerWorker);
    const int cap = max_threads > 0 ? std::min(max_threads, pool.size()) : pool.size();
    job.workers = static_cast<int>(std::min<int64_t>(want, cap));
    if (job.workers <= 1) {
        job.workers = 1;
        copy_share(job, 0);
    } else {
        pool.run(job);
    }
    ok = !job.nonbinary.load(std::memory_order_relaxed) && !job.overflow.load(std::memory_order_relaxed);
    return MESHY_OK;
}

}  // namespace
}  // namespace meshy

extern "C" int meshy_host_gather(const void* const* srcs, const int64_t* nbytes, int64_t n, void* dst,
                                 int max_threads) {
    meshy::clear_error();
    bool ok;
    return meshy::run_gather("meshy_host_gather", srcs, nbytes, n, dst, max_threads, 0, ok);
}

extern "C" int meshy_host_gather_mask_u8(const float* const* srcs, const int64_t* counts, int64_t n, uint8_t* dst,
                                         int max_threads, int32_t* binary) {
    meshy::clear_error();
    if (!binary) return meshy::set_error(MESHY_ENULL, "meshy_host_gather_mask_u8: binary is NULL");
    bool ok;
    const int rc = meshy::run_gather("meshy_host_gather_mask_u8", reinterpret_cast<const void* const*>(srcs), counts,
                                     n, dst, max_threads, 1, ok);
    *binary = rc == MESHY_OK && ok ? 1 : 0;
    return rc;
}

extern "C" int meshy_host_gather_i32(const int64_t* const* srcs, const int64_t* counts, int64_t n, int32_t* dst,
                                     int max_threads, int32_t* fits) {
    meshy::clear_error();
    if (!fits) return meshy::set_error(MESHY_ENULL, "meshy_host_gather_i32: fits is NULL");
    bool ok;
    const int rc = meshy::run_gather("meshy_host_gather_i32", reinterpret_cast<const void* const*>(srcs), counts, n,
                                     dst, max_threads, 2, ok);
    *fits = rc == MESHY_OK && ok ? 1 : 0;
    return rc;
}
