// Threaded host loops of the host-pointer entry point (cwlb_spmm_mean_f32_host):
// the input checks that keep every device access in bounds and the copies
// through the pinned staging buffers.  Plain C++ (no HIP), so that the same
// code also builds under ThreadSanitizer on a machine without a GPU.
#pragma once

#include <algorithm>
#include <atomic>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>

namespace cwlb {

// fn(begin, end) over [0, n) split into contiguous parts, on up to 8 host
// threads (about one per `grain` items), the caller's thread included.  The
// parts are disjoint and every thread is joined before the call returns.
template <class Fn>
void parallel_ranges(size_t n, size_t grain, Fn fn)
{
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const size_t T = std::max<size_t>(1, std::min<size_t>({size_t{8}, hw, n / grain}));
    if (T == 1) {
        fn(size_t{0}, n);
        return;
    }
    std::vector<std::thread> pool;
    pool.reserve(T - 1);
    for (size_t t = 1; t < T; ++t)
        pool.emplace_back([&, t] { fn(n * t / T, n * (t + 1) / T); });
    fn(size_t{0}, n / T);
    for (auto& th : pool) th.join();
}

// memcpy of `bytes` bytes in parts of about 8 MiB on up to 8 threads.
inline void parallel_copy(void* dst, const void* src, size_t bytes)
{
    parallel_ranges(bytes, size_t{8} << 20, [&](size_t b, size_t e) {
        std::memcpy(static_cast<char*>(dst) + b, static_cast<const char*>(src) + b, e - b);
    });
}

// Whether row_ptr[0..n_rows] never decreases.
inline bool offsets_nondecreasing(const int32_t* row_ptr, int32_t n_rows)
{
    std::atomic<bool> bad{false};
    parallel_ranges(static_cast<size_t>(n_rows), size_t{1} << 20, [&](size_t b, size_t e) {
        bool mine = false;
        for (size_t r = b; r < e; ++r) mine |= row_ptr[r + 1] < row_ptr[r];
        if (mine) bad = true;
    });
    return !bad;
}

// Whether every column index lies in [0, h_rows).
inline bool columns_in_range(const int32_t* col_idx, int64_t nnz, int64_t h_rows)
{
    std::atomic<bool> bad{false};
    parallel_ranges(static_cast<size_t>(nnz), size_t{1} << 21, [&](size_t b, size_t e) {
        bool mine = false;
        for (size_t j = b; j < e; ++j) mine |= col_idx[j] < 0 || col_idx[j] >= h_rows;
        if (mine) bad = true;
    });
    return !bad;
}

}  // namespace cwlb
