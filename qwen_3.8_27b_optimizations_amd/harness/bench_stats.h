// bench_stats.h -- per-launch timing statistics of the reference's kernel
// bench harness (kernels/common/bench.h:12-98): warm-up launches, then one
// hipEvent pair around each timed launch; median (mean of the two middle
// values for an even count), p95 at index ceil(0.95 n) - 1, mean, population
// standard deviation, and GB/s = bytes / median.  Also the reference GEMM
// bench's aggregation of several such runs (bench_gemm_wmma.cpp:168-184).
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <functional>
#include <numeric>
#include <vector>

struct BenchStats {
    double median_us = 0.0, p95_us = 0.0, min_us = 0.0, max_us = 0.0, mean_us = 0.0, stdev_us = 0.0;
    int count = 0, warmup = 0;
    size_t bytes_transferred = 0;
    double gb_s = 0.0;
};

// Statistics of `times_us` (any order).
inline BenchStats bench_stats_from(std::vector<double> times_us, int warmup, size_t bytes) {
    BenchStats s;
    const size_t n = times_us.size();
    s.count = (int)n;
    s.warmup = warmup;
    s.bytes_transferred = bytes;
    if (n == 0) return s;
    std::sort(times_us.begin(), times_us.end());
    s.min_us = times_us.front();
    s.max_us = times_us.back();
    s.median_us = n % 2 == 0 ? 0.5 * (times_us[n / 2 - 1] + times_us[n / 2]) : times_us[n / 2];
    size_t p95 = (size_t)std::ceil(0.95 * (double)n);
    p95 = p95 == 0 ? 0 : p95 - 1;
    s.p95_us = times_us[std::min(p95, n - 1)];
    s.mean_us = std::accumulate(times_us.begin(), times_us.end(), 0.0) / (double)n;
    double sq = 0.0;
    for (double t : times_us) sq += (t - s.mean_us) * (t - s.mean_us);
    s.stdev_us = std::sqrt(sq / (double)n);
    if (bytes > 0 && s.median_us > 0.0) s.gb_s = (double)bytes / (s.median_us * 1000.0);
    return s;
}

// `warmup` untimed launches, then `iters` launches each between its own event
// pair on `stream`.  Returns false (and leaves `out` untouched) on a HIP error.
inline bool bench_event(const std::function<hipError_t(hipStream_t)>& launch, hipStream_t stream, int warmup,
                        int iters, size_t bytes, BenchStats& out) {
    for (int i = 0; i < warmup; ++i)
        if (launch(stream) != hipSuccess) return false;
    if (hipStreamSynchronize(stream) != hipSuccess) return false;
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess) return false;
    if (hipEventCreate(&b) != hipSuccess) {
        (void)hipEventDestroy(a);
        return false;
    }
    std::vector<double> t;
    t.reserve((size_t)iters);
    bool ok = true;
    for (int i = 0; i < iters && ok; ++i) {
        float ms = 0.0f;
        ok = hipEventRecord(a, stream) == hipSuccess && launch(stream) == hipSuccess &&
             hipEventRecord(b, stream) == hipSuccess && hipEventSynchronize(b) == hipSuccess &&
             hipEventElapsedTime(&ms, a, b) == hipSuccess;
        t.push_back((double)ms * 1000.0);
    }
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    if (ok) out = bench_stats_from(t, warmup, bytes);
    return ok;
}

// Several runs of bench_event folded into one record: median of the medians,
// mean of the means, stdev combining the mean within-run stdev with the spread
// of the run means, p95 of the run p95s.
inline BenchStats bench_aggregate(const std::vector<BenchStats>& runs) {
    BenchStats a;
    if (runs.empty()) return a;
    std::vector<double> med, mean, p95;
    double within = 0.0;
    for (const BenchStats& r : runs) {
        med.push_back(r.median_us);
        mean.push_back(r.mean_us);
        p95.push_back(r.p95_us);
        within += r.stdev_us;
    }
    const size_t n = runs.size();
    std::sort(med.begin(), med.end());
    std::sort(p95.begin(), p95.end());
    a.count = (int)n;
    a.median_us = n % 2 == 0 ? 0.5 * (med[n / 2 - 1] + med[n / 2]) : med[n / 2];
    a.mean_us = std::accumulate(mean.begin(), mean.end(), 0.0) / (double)n;
    double sq = 0.0;
    for (double m : mean) sq += (m - a.mean_us) * (m - a.mean_us);
    within /= (double)n;
    a.stdev_us = std::sqrt(within * within + sq / (double)n);
    size_t i95 = (size_t)std::ceil(0.95 * (double)n);
    i95 = i95 == 0 ? 0 : i95 - 1;
    a.p95_us = p95[std::min(i95, n - 1)];
    a.min_us = med.front();
    a.max_us = med.back();
    a.bytes_transferred = runs[0].bytes_transferred;
    a.gb_s = runs[0].gb_s;
    return a;
}
