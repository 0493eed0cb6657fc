// ung_internal.h -- helpers shared by the host (ung_host.cpp) and device
// (ung_kernels.hip) halves of libung_hip.so.  Not part of the public ABI.
#pragma once

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <thread>
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

} // namespace ung
