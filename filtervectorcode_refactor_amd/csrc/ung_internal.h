// ung_internal.h -- helpers shared by the host (ung_host.cpp) and device
// (ung_kernels.hip) halves of libung_hip.so.  Not part of the public ABI.
#pragma once

#include <atomic>
#include <condition_variable>
#include <cstdarg>
#include <cstdint>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>
#include <type_traits>
#include <utility>
#include <vector>

namespace ung {

// Records the calling thread's last error message (read by ung_hip_last_error).
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

inline int resolve_threads(int nthreads)
{
    if (nthreads > 0)
        return nthreads;
    unsigned hc = std::thread::hardware_concurrency();
    if (hc == 0)
        hc = 1;
    return (int)(hc > 64 ? 64 : hc);
}

// Dynamic parallel loop over [0, n) in chunks of `chunk`, body(begin, end).
template <class F>
void parallel_for(int64_t n, int nthreads, int64_t chunk, F body)
{
    if (n <= 0)
        return;
    nthreads = resolve_threads(nthreads);
    if (chunk < 1)
        chunk = 1;
    const int64_t nchunks = (n + chunk - 1) / chunk;
    if (nthreads <= 1 || nchunks <= 1) {
        body((int64_t)0, n);
        return;
    }
    if ((int64_t)nthreads > nchunks)
        nthreads = (int)nchunks;
    std::atomic<int64_t> next{0};
    auto worker = [&]() {
        for (;;) {
            const int64_t c = next.fetch_add(1, std::memory_order_relaxed);
            if (c >= nchunks)
                break;
            const int64_t b = c * chunk;
            const int64_t e = b + chunk < n ? b + chunk : n;
            body(b, e);
        }
    };
    std::vector<std::thread> pool;
    pool.reserve(nthreads - 1);
    for (int t = 1; t < nthreads; ++t)
        pool.emplace_back(worker);
    worker();
    for (auto &t : pool)
        t.join();
}

// Allocator whose resize() leaves new elements of trivial types uninitialised: vectors
// that are refilled completely after every resize skip a zero-filling pass.
template <class T>
struct DefaultInitAllocator : std::allocator<T> {
    template <class U>
    struct rebind {
        using other = DefaultInitAllocator<U>;
    };
    DefaultInitAllocator() = default;
    template <class U>
    DefaultInitAllocator(const DefaultInitAllocator<U> &) noexcept
    {
    }
    template <class U>
    void construct(U *p) noexcept(std::is_nothrow_default_constructible<U>::value)
    {
        ::new (static_cast<void *>(p)) U;
    }
    template <class U, class... A>
    void construct(U *p, A &&...a)
    {
        ::new (static_cast<void *>(p)) U(std::forward<A>(a)...);
    }
};
template <class T>
using RawVector = std::vector<T, DefaultInitAllocator<T>>;

// A persistent pool of worker threads (created once, reused by every call): run(n, fn)
// calls fn(i) for every i in [0, n) on the workers and on the calling thread, and returns
// when all calls are done.  One run at a time.
class WorkerPool {
  public:
    explicit WorkerPool(int nthreads)
    {
        for (int t = 1; t < nthreads; ++t)
            threads_.emplace_back([this] { work(); });
    }
    ~WorkerPool()
    {
        {
            std::lock_guard<std::mutex> lk(mu_);
            stop_ = true;
        }
        cv_start_.notify_all();
        for (auto &t : threads_)
            t.join();
    }
    WorkerPool(const WorkerPool &) = delete;
    WorkerPool &operator=(const WorkerPool &) = delete;
    int size() const { return (int)threads_.size() + 1; }

    void run(int64_t n, const std::function<void(int64_t)> &fn)
    {
        if (n <= 0)
            return;
        if (threads_.empty() || n == 1) {
            for (int64_t i = 0; i < n; ++i)
                fn(i);
            return;
        }
        {
            std::lock_guard<std::mutex> lk(mu_);
            fn_ = &fn;
            n_ = n;
            next_.store(0, std::memory_order_relaxed);
            busy_ = (int)threads_.size();
            ++generation_;
        }
        cv_start_.notify_all();
        drain();
        std::unique_lock<std::mutex> lk(mu_);
        cv_done_.wait(lk, [this] { return busy_ == 0; });
        fn_ = nullptr;
    }

  private:
    void drain()
    {
        for (;;) {
            const int64_t i = next_.fetch_add(1, std::memory_order_relaxed);
            if (i >= n_)
                break;
            (*fn_)(i);
        }
    }
    void work()
    {
        uint64_t seen = 0;
        for (;;) {
            {
                std::unique_lock<std::mutex> lk(mu_);
                cv_start_.wait(lk, [&] { return stop_ || generation_ != seen; });
                if (stop_)
                    return;
                seen = generation_;
            }
            drain();
            std::lock_guard<std::mutex> lk(mu_);
            if (--busy_ == 0)
                cv_done_.notify_one();
        }
    }

    std::vector<std::thread> threads_;
    std::mutex mu_;
    std::condition_variable cv_start_, cv_done_;
    const std::function<void(int64_t)> *fn_ = nullptr;
    int64_t n_ = 0;
    std::atomic<int64_t> next_{0};
    int busy_ = 0;
    uint64_t generation_ = 0;
    bool stop_ = false;
};

} // namespace ung
