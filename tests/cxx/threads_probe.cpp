// The host-pointer entry's threaded loops (csrc/host_threads.h) on their
// own, for a ThreadSanitizer build: the staged copies in ~8 MiB parts and
// the row-offset and column-index checks, on buffers large enough for
// every thread the host offers.  Prints "OK" when every result is right.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <numeric>
#include <vector>

#include "host_threads.h"

int main()
{
    using namespace cwlb;
    int failures = 0;
    // Copies: 96 MiB + 3 bytes (12 parts and a ragged end), twice into the
    // same destination, as the staging buffers are refilled.
    const size_t bytes = (size_t{96} << 20) + 3;
    std::vector<unsigned char> src(bytes), dst(bytes, 0);
    for (size_t i = 0; i < bytes; ++i) src[i] = static_cast<unsigned char>(i * 2654435761u >> 13);
    for (int pass = 0; pass < 2; ++pass) {
        parallel_copy(dst.data(), src.data(), bytes);
        if (std::memcmp(dst.data(), src.data(), bytes) != 0) ++failures;
        src[bytes / 3] ^= 0x5a;
    }
    // Offsets: 8M rows non-decreasing, then one decrease near the end and
    // one at the very start.
    const int32_t n = 8 << 20;
    std::vector<int32_t> rp(static_cast<size_t>(n) + 1);
    for (int32_t r = 0; r <= n; ++r) rp[r] = r / 3;
    if (!offsets_nondecreasing(rp.data(), n)) ++failures;
    rp[n - 7] = rp[n - 8] - 1;
    if (offsets_nondecreasing(rp.data(), n)) ++failures;
    rp[n - 7] = rp[n - 8];
    rp[1] = -1;
    if (offsets_nondecreasing(rp.data(), n)) ++failures;
    // Columns: 16M indices in [0, 1000), then one out of range at either end.
    const int64_t nnz = int64_t{16} << 20;
    std::vector<int32_t> ci(static_cast<size_t>(nnz));
    for (int64_t j = 0; j < nnz; ++j) ci[j] = static_cast<int32_t>(j % 1000);
    if (!columns_in_range(ci.data(), nnz, 1000)) ++failures;
    ci[nnz - 1] = 1000;
    if (columns_in_range(ci.data(), nnz, 1000)) ++failures;
    ci[nnz - 1] = 0;
    ci[0] = -3;
    if (columns_in_range(ci.data(), nnz, 1000)) ++failures;
    // Bad indices in every thread's part: the threads set the flag at once.
    for (int64_t j = 0; j < nnz; j += int64_t{1} << 19) ci[j] = 5000;
    if (columns_in_range(ci.data(), nnz, 1000)) ++failures;
    for (int32_t r = 1; r < n; r += 1 << 18) rp[r] = rp[r - 1] - 1;
    if (offsets_nondecreasing(rp.data(), n)) ++failures;
    std::printf(failures ? "FAILED %d\n" : "OK\n", failures);
    return failures ? 1 : 0;
}
