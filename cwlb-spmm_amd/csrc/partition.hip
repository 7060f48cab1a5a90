// Cost-weighted task partitioning on the GPU, task-for-task identical to the
// host partition (reference src/utils.cpp:832-1021).
//
// The host form is a sequential greedy state machine over the reordered
// rows: pack whole rows while the load stays within the capacity, cut a
// long row into segments of at most S nonzeros, let its deg % S prefix ride
// at the end of the open task or the end of the previous long row.  Every
// time the open task is closed its state collapses to one of two "fresh"
// nodes:
//   A(r)  at row r, the open task starts at row r, offset 0, load 0;
//   B(r)  at long row r, the open task starts at row r, offset deg % S
//         (the prefix went to the previous task), load 0.
// From a fresh node the machine is deterministic up to the next fresh node.
// So the partition is computed as
//   1. part_transitions: every node simulates to its next node and counts
//      the tasks it emits on the way (the host's double operations, in the
//      host's order; this file is compiled without fp contraction);
//   2. pointer doubling J_k = J_{k-1} o J_{k-1} until 2^k steps from A(0)
//      reach the end;
//   3. the chain from A(0) expanded by position in k rounds;
//   4. an exclusive scan of the chain nodes' task counts;
//   5. part_emit: each chain node simulates again and writes its tasks.
// Node ids: A(r) = r for r in [0, n] (A(n) is the end), B(r) = n + 1 + c
// where c is r's index among the long rows.
//
// A short-row scan adds at least C_store per row, so it is bounded by
// capacity / C_store; costs without that bound (C_store <= 0, a negative
// edge weight, a non-finite capacity, or a bound beyond kMaxScan rows) are
// CWLB_UNSUPPORTED here and stay with the host partition.
#pragma clang fp contract(off)

#include <rocprim/device/device_scan.hpp>

#include <algorithm>
#include <climits>
#include <cmath>
#include <vector>

#include "internal.h"
#include "partition_sim.h"

namespace cwlb {
namespace {

constexpr int kBlock = 256;
constexpr long long kMaxScan = 1 << 16;

using part::PartParams;
using part::Emitter;
using part::simulate;
using part::full_w;

__global__ void __launch_bounds__(kBlock)
part_flags(PartParams p, int* __restrict__ is_long)
{
    const int r = blockIdx.x * kBlock + threadIdx.x;
    if (r < p.n) is_long[r] = !(full_w(p, r) <= p.cap) ? 1 : 0;
}

__global__ void __launch_bounds__(kBlock)
part_compact(int n, const int* __restrict__ is_long, const int* __restrict__ scan,
             int* __restrict__ long_row, int* __restrict__ long_idx)
{
    const int r = blockIdx.x * kBlock + threadIdx.x;
    if (r >= n) return;
    if (is_long[r]) {
        long_row[scan[r]] = r;
        long_idx[r] = scan[r];
    } else {
        long_idx[r] = -1;
    }
}

__global__ void __launch_bounds__(kBlock)
part_transitions(PartParams p, long long V, int* __restrict__ next, int* __restrict__ cnt,
                 int* __restrict__ status)
{
    const long long x = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x;
    if (x >= V) return;
    Emitter em{nullptr, 0};
    int overrun = 0;
    next[x] = simulate(p, static_cast<int>(x), em, &overrun);
    cnt[x] = static_cast<int>(em.count);
    if (overrun) atomicOr(status, 1);
}

// levels[0] = 1 + the first k with J_k(A(0)) == n (J_k = 2^k steps; the
// J arrays are consecutive, V entries each), or 0 if none of the L reaches
// the end.
__global__ void part_levels(const int* __restrict__ J, long long V, int L, int n,
                            int* __restrict__ levels)
{
    int found = 0;
    for (int k = 0; k < L; ++k) {
        if (J[static_cast<long long>(k) * V] == n) {
            found = k + 1;
            break;
        }
    }
    *levels = found;
}

__global__ void __launch_bounds__(kBlock)
part_double(long long V, const int* __restrict__ src, int* __restrict__ dst)
{
    const long long x = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x;
    if (x < V) dst[x] = src[src[x]];
}

// Round of the chain expansion: positions pos = i * 2 * half get their
// successor at pos + half from jump table J (2^j steps, half = 2^j).
__global__ void __launch_bounds__(kBlock)
part_expand(long long count, long long half, const int* __restrict__ J, int* __restrict__ chain)
{
    const long long i = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= count) return;
    const long long pos = i * 2 * half;
    chain[pos + half] = J[chain[pos]];
}

__global__ void __launch_bounds__(kBlock)
part_chain_counts(long long len, int end, const int* __restrict__ chain,
                  const int* __restrict__ cnt, long long* __restrict__ c)
{
    const long long i = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x;
    if (i < len) c[i] = chain[i] == end ? 0 : cnt[chain[i]];
}

__global__ void __launch_bounds__(kBlock)
part_emit(PartParams p, long long len, const int* __restrict__ chain,
          const long long* __restrict__ offsets, cwlb_task* __restrict__ out)
{
    const long long i = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= len || chain[i] == p.n) return;
    Emitter em{out + offsets[i], 0};
    int overrun = 0;
    (void)simulate(p, chain[i], em, &overrun);
}

// Owning device allocation; movable, not copyable (the jump tables live in
// a growing vector).
struct Mem {
    void* p = nullptr;
    Mem() = default;
    Mem(const Mem&) = delete;
    Mem& operator=(const Mem&) = delete;
    Mem(Mem&& o) noexcept : p(o.p) { o.p = nullptr; }
    Mem& operator=(Mem&& o) noexcept
    {
        if (this != &o) {
            if (p) (void)hipFree(p);
            p = o.p;
            o.p = nullptr;
        }
        return *this;
    }
    ~Mem()
    {
        if (p) (void)hipFree(p);
    }
    hipError_t alloc(size_t bytes) { return hipMalloc(&p, bytes ? bytes : 1); }
    template <class T>
    T* as() const
    {
        return static_cast<T*>(p);
    }
};

template <class In, class Out>
cwlb_status exclusive_scan(hipStream_t st, In in, Out out, size_t n)
{
    using T = typename std::iterator_traits<Out>::value_type;
    size_t bytes = 0;
    CWLB_HIP_TRY(rocprim::exclusive_scan(nullptr, bytes, in, out, T(0), n, rocprim::plus<T>(), st));
    Mem temp;
    CWLB_HIP_TRY(temp.alloc(bytes));
    CWLB_HIP_TRY(rocprim::exclusive_scan(temp.p, bytes, in, out, T(0), n, rocprim::plus<T>(), st));
    CWLB_HIP_TRY(hipStreamSynchronize(st));
    return CWLB_OK;
}

unsigned grid_for(long long n) { return static_cast<unsigned>((n + kBlock - 1) / kBlock); }

// Clears one or two words with a kernel rather than hipMemsetAsync (memset
// nodes are kept out of anything a caller may record into a graph).
template <class T>
__global__ void part_clear(T* __restrict__ a, T* __restrict__ b)
{
    *a = T(0);
    if (b) *b = T(0);
}

}  // namespace

cwlb_status launch_partition(cwlb_ctx* ctx, const int32_t* rp, int32_t n,
                             const cwlb_cost_params* costs, double cap, cwlb_task* out,
                             int64_t capacity_tasks, int64_t* n_tasks)
{
    hipStream_t st = ctx->stream;
    *n_tasks = 0;
    if (n <= 0) return CWLB_OK;
    PartParams p{};
    p.n = n;
    p.rp = rp;
    p.wcl = costs->C_compute_ns + costs->C_load_ns;
    p.cs = costs->C_store_ns;
    p.ca = costs->C_atomic_ns;
    p.cap = cap;
    // S as the host recovers it from the capacity (utils.cpp:859-864).
    {
        const double denom = (1e-30 < p.wcl) ? p.wcl : 1e-30;
        const double x = std::floor((cap - p.ca) / denom);
        int s = INT_MIN;
        if (x == x && x < 2147483648.0 && x > -2147483649.0) s = static_cast<int>(x);
        p.S = std::max(1, s);
    }
    if (!(p.cs > 0.0) || !(p.wcl >= 0.0) || !std::isfinite(cap) || !std::isfinite(p.ca) ||
        !std::isfinite(p.wcl) || !std::isfinite(p.cs) || cap / p.cs > static_cast<double>(kMaxScan))
        return fail(CWLB_UNSUPPORTED,
                    "cwlb_partition_device: these costs do not bound a task's row count "
                    "(needs C_store > 0, C_compute + C_load >= 0, finite values and "
                    "capacity / C_store <= 65536); use cwlb_partition");
    // Accepted rows each add at least C_store; the margin covers rounding.
    p.max_scan = static_cast<long long>(cap / p.cs * (1.0 + 1e-6)) + 4;

    (void)hipGetLastError();  // a stale error of an earlier call must not be reported here
    // Long rows and their compact indices.
    Mem is_long, scan, long_row, long_idx, status;
    CWLB_HIP_TRY(is_long.alloc(sizeof(int) * (n + 1)));
    CWLB_HIP_TRY(scan.alloc(sizeof(int) * (n + 1)));
    CWLB_HIP_TRY(long_idx.alloc(sizeof(int) * n));
    CWLB_HIP_TRY(status.alloc(sizeof(int)));
    hipLaunchKernelGGL(part_clear<int>, dim3(1), dim3(1), 0, st, status.as<int>(),
                       is_long.as<int>() + n);
    CWLB_LAUNCH_CHECK("part_clear");
    hipLaunchKernelGGL(part_flags, dim3(grid_for(n)), dim3(kBlock), 0, st, p, is_long.as<int>());
    CWLB_LAUNCH_CHECK("part_flags");
    cwlb_status s = exclusive_scan(st, is_long.as<int>(), scan.as<int>(), static_cast<size_t>(n) + 1);
    if (s != CWLB_OK) return s;
    int n_long = 0;
    CWLB_HIP_TRY(hipMemcpyAsync(&n_long, scan.as<int>() + n, sizeof(int), hipMemcpyDeviceToHost, st));
    CWLB_HIP_TRY(hipStreamSynchronize(st));
    CWLB_HIP_TRY(long_row.alloc(sizeof(int) * std::max(n_long, 1)));
    hipLaunchKernelGGL(part_compact, dim3(grid_for(n)), dim3(kBlock), 0, st, n, is_long.as<int>(),
                       scan.as<int>(), long_row.as<int>(), long_idx.as<int>());
    CWLB_LAUNCH_CHECK("part_compact");
    p.long_row = long_row.as<int>();
    p.long_idx = long_idx.as<int>();

    // 1. transitions of every node.
    const long long V = static_cast<long long>(n) + 1 + n_long;
    if (V > INT_MAX) return fail(CWLB_UNSUPPORTED, "cwlb_partition_device: too many rows");
    // The chain from A(0) has at most V fresh nodes, so L doubling levels
    // (2^(L-1) >= V) always reach the end; all are computed back to back
    // in one allocation, then one read-back finds how many were needed.
    int L = 1;
    while ((1LL << (L - 1)) < V) ++L;
    Mem cnt, Jall;
    CWLB_HIP_TRY(cnt.alloc(sizeof(int) * V));
    CWLB_HIP_TRY(Jall.alloc(sizeof(int) * static_cast<size_t>(V) * L + sizeof(int)));
    int* const J0 = Jall.as<int>();
    auto J = [&](int k) { return J0 + static_cast<long long>(k) * V; };
    int* const d_levels = J0 + static_cast<long long>(L) * V;
    hipLaunchKernelGGL(part_transitions, dim3(grid_for(V)), dim3(kBlock), 0, st, p, V,
                       J(0), cnt.as<int>(), status.as<int>());
    CWLB_LAUNCH_CHECK("part_transitions");
    // 2. doubling: J_{k+1} = J_k o J_k.
    for (int k = 1; k < L; ++k) {
        hipLaunchKernelGGL(part_double, dim3(grid_for(V)), dim3(kBlock), 0, st, V, J(k - 1), J(k));
        CWLB_LAUNCH_CHECK("part_double");
    }
    hipLaunchKernelGGL(part_levels, dim3(1), dim3(1), 0, st, J0, V, L, n, d_levels);
    CWLB_LAUNCH_CHECK("part_levels");
    int host_status[2] = {0, 0};
    CWLB_HIP_TRY(hipMemcpyAsync(&host_status[0], status.p, sizeof(int), hipMemcpyDeviceToHost, st));
    CWLB_HIP_TRY(hipMemcpyAsync(&host_status[1], d_levels, sizeof(int), hipMemcpyDeviceToHost, st));
    CWLB_HIP_TRY(hipStreamSynchronize(st));
    if (host_status[0]) return fail(CWLB_RUNTIME_ERROR, "cwlb_partition_device: a row scan exceeded its bound");
    const int levels = host_status[1];
    if (levels <= 0) return fail(CWLB_RUNTIME_ERROR, "cwlb_partition_device: chain too long");
    // J[levels-1] maps A(0) to the end: the chain has at most 2^(levels-1)
    // fresh nodes before the end.
    const long long len = 1LL << (levels - 1);
    Mem chain, counts, offsets;
    CWLB_HIP_TRY(chain.alloc(sizeof(int) * len));
    hipLaunchKernelGGL(part_clear<int>, dim3(1), dim3(1), 0, st, chain.as<int>(),
                       static_cast<int*>(nullptr));
    CWLB_LAUNCH_CHECK("part_clear");
    // 3. expansion: positions that are multiples of 2 * half get their
    // successor half steps on.
    for (int j = levels - 2; j >= 0; --j) {
        const long long half = 1LL << j;
        const long long count = len / (2 * half);
        hipLaunchKernelGGL(part_expand, dim3(grid_for(count)), dim3(kBlock), 0, st, count, half,
                           J(j), chain.as<int>());
        CWLB_LAUNCH_CHECK("part_expand");
    }
    // 4. task offsets of the chain nodes.
    CWLB_HIP_TRY(counts.alloc(sizeof(long long) * (len + 1)));
    CWLB_HIP_TRY(offsets.alloc(sizeof(long long) * (len + 1)));
    hipLaunchKernelGGL(part_clear<long long>, dim3(1), dim3(1), 0, st,
                       counts.as<long long>() + len, static_cast<long long*>(nullptr));
    CWLB_LAUNCH_CHECK("part_clear");
    hipLaunchKernelGGL(part_chain_counts, dim3(grid_for(len)), dim3(kBlock), 0, st, len, n,
                       chain.as<int>(), cnt.as<int>(), counts.as<long long>());
    CWLB_LAUNCH_CHECK("part_chain_counts");
    s = exclusive_scan(st, counts.as<long long>(), offsets.as<long long>(),
                       static_cast<size_t>(len) + 1);
    if (s != CWLB_OK) return s;
    long long total = 0;
    CWLB_HIP_TRY(hipMemcpyAsync(&total, offsets.as<long long>() + len, sizeof(long long),
                                hipMemcpyDeviceToHost, st));
    CWLB_HIP_TRY(hipStreamSynchronize(st));
    *n_tasks = total;
    if (total > capacity_tasks || (!out && total > 0))
        return fail(CWLB_INSUFFICIENT, "cwlb_partition_device: output buffer too small");
    // 5. the tasks.
    if (total > 0) {
        hipLaunchKernelGGL(part_emit, dim3(grid_for(len)), dim3(kBlock), 0, st, p, len,
                           chain.as<int>(), offsets.as<long long>(), out);
        CWLB_LAUNCH_CHECK("part_emit");
    }
    CWLB_HIP_TRY(hipStreamSynchronize(st));
    return CWLB_OK;
}

}  // namespace cwlb
