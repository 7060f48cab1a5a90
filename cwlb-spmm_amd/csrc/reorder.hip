// Degree reordering on the GPU: the permutation, offsets and row copies of
// the reference's host reordering (main.cpp:197-278), computed from device
// arrays.
//
//   1. degree_keys: deg[i] = row_ptr[i+1] - row_ptr[i] as the sort key,
//      with the CSR checks of the host form (offsets inside [0, nnz],
//      non-decreasing) and the maximum degree;
//   2. a stable LSD radix sort of (deg, i) pairs over the bits the maximum
//      degree needs (rocPRIM): equal degrees keep ascending original ids, so
//      the order is the reference comparator's (degree, id) order;
//   3. row_ptr_out = 0 followed by the inclusive scan of the sorted degrees;
//   4. gather_rows / gather_long: each reordered row copies its entries from
//      the original row: a lane per row of at most 16 entries; the longer
//      rows (a suffix of the sorted order) as one contiguous output range
//      cut into equal chunks, so no wave copies a hub row alone.
// The call synchronises on the context's stream.
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>
#include <rocprim/iterator/counting_iterator.hpp>

#include "internal.h"

namespace cwlb {
namespace {

constexpr int kBlock = 256;
constexpr int kLaneRowMax = 16;
constexpr int kLongChunk = kBlock * 16;  // entries per gather_long block

// status bit 0: an offset outside [0, nnz] or a decreasing pair.  Each
// block writes its maximum degree to block_max[blockIdx.x] (one contended
// atomic per wave costs milliseconds at 16M rows).
__global__ void __launch_bounds__(kBlock)
degree_keys(const int* __restrict__ rp, int n, long long nnz, unsigned* __restrict__ deg,
            int* __restrict__ status, unsigned* __restrict__ block_max)
{
    __shared__ unsigned wave_max[kBlock / 64];
    const int i = blockIdx.x * kBlock + threadIdx.x;
    unsigned d = 0;
    if (i < n) {
        const int a = rp[i];
        const int b = rp[i + 1];
        if (a < 0 || b < a || static_cast<long long>(b) > nnz) {
            atomicOr(status, 1);
        } else {
            d = static_cast<unsigned>(b - a);
        }
        deg[i] = d;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        d = max(d, static_cast<unsigned>(__shfl_xor(static_cast<int>(d), off)));
    if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = d;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned m = 0;
#pragma unroll
        for (int w = 0; w < kBlock / 64; ++w) m = max(m, wave_max[w]);
        block_max[blockIdx.x] = m;
    }
}

// One block: the maximum of the per-block maxima into *out.
__global__ void __launch_bounds__(1024)
reduce_max(const unsigned* __restrict__ v, long long n, unsigned* __restrict__ out)
{
    __shared__ unsigned part[1024 / 64];
    unsigned m = 0;
    for (long long i = threadIdx.x; i < n; i += 1024) m = max(m, v[i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1)
        m = max(m, static_cast<unsigned>(__shfl_xor(static_cast<int>(m), off)));
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned r = 0;
        for (int w = 0; w < 1024 / 64; ++w) r = max(r, part[w]);
        *out = r;
    }
}

// Rows of at most kLaneRowMax entries: a lane per row.  Longer rows are
// gathered by gather_long.
__global__ void __launch_bounds__(kBlock)
gather_rows(const int* __restrict__ rp, const int* __restrict__ ci, const float* __restrict__ val,
            const int* __restrict__ origin, const int* __restrict__ rp_out, int n,
            int* __restrict__ ci_out, float* __restrict__ val_out)
{
    const int r = blockIdx.x * kBlock + threadIdx.x;
    if (r >= n) return;
    const int dst = rp_out[r];
    const int len = rp_out[r + 1] - dst;
    if (len > kLaneRowMax) return;
    const int src = rp[origin[r]];
    for (int j = 0; j < len; ++j) {
        ci_out[dst + j] = ci[src + j];
        val_out[dst + j] = val[src + j];
    }
}

// long_row[0] = the first reordered row with more than kLaneRowMax entries
// (n if none): the degrees are sorted ascending, so those rows are a suffix.
__global__ void find_long_rows(const unsigned* __restrict__ sorted_deg, int n,
                               int* __restrict__ long_row)
{
    int lo = 0, hi = n;
    while (lo < hi) {
        const int mid = lo + (hi - lo) / 2;
        if (sorted_deg[mid] > static_cast<unsigned>(kLaneRowMax)) hi = mid;
        else lo = mid + 1;
    }
    *long_row = lo;
}

// The entries of the long rows [long_row, n), which fill the output range
// [rp_out[long_row], nnz): block b copies the kLongChunk entries from
// rp_out[long_row] + b * kLongChunk on, a thread every kBlock-th entry, so a
// hub row is spread over many blocks and every access is coalesced.  The
// first row of the block's range is found by binary search; each thread then
// walks forward row by row.
__global__ void __launch_bounds__(kBlock)
gather_long(const int* __restrict__ rp, const int* __restrict__ ci, const float* __restrict__ val,
            const int* __restrict__ origin, const int* __restrict__ rp_out, int n,
            const int* __restrict__ long_row, int* __restrict__ ci_out, float* __restrict__ val_out)
{
    __shared__ int first_row;
    const int r0 = *long_row;
    if (r0 >= n) return;
    const long long begin = static_cast<long long>(rp_out[r0]) +
                            static_cast<long long>(blockIdx.x) * kLongChunk;
    const long long end = rp_out[n];
    if (begin >= end) return;
    if (threadIdx.x == 0) {
        int lo = r0, hi = n - 1;  // last row whose start is <= begin
        while (lo < hi) {
            const int mid = hi - (hi - lo) / 2;
            if (rp_out[mid] <= begin) lo = mid;
            else hi = mid - 1;
        }
        first_row = lo;
    }
    __syncthreads();
    int row = first_row;
    int row_begin = rp_out[row];
    int row_end = rp_out[row + 1];
    int src = rp[origin[row]];
    const long long stop = min(end, begin + kLongChunk);
    for (long long p = begin + threadIdx.x; p < stop; p += kBlock) {
        while (p >= row_end) {
            ++row;
            row_begin = row_end;
            row_end = rp_out[row + 1];
            src = rp[origin[row]];
        }
        const long long s = src + (p - row_begin);
        ci_out[p] = ci[s];
        val_out[p] = val[s];
    }
}

__global__ void set_first_zero(int* __restrict__ p) { p[0] = 0; }

// The two status words of the reorder, cleared by a kernel rather than
// hipMemsetAsync (memset nodes are kept out of anything a caller may record
// into a graph).
__global__ void clear_two(int* __restrict__ p)
{
    p[0] = 0;
    p[1] = 0;
}

struct DevMem {
    void* p = nullptr;
    DevMem() = default;
    DevMem(const DevMem&) = delete;
    DevMem& operator=(const DevMem&) = delete;
    ~DevMem()
    {
        if (p) (void)hipFree(p);
    }
    hipError_t alloc(size_t bytes) { return hipMalloc(&p, bytes ? bytes : 1); }
};

unsigned bits_for(unsigned v)
{
    unsigned b = 0;
    while (b < 32 && (v >> b) != 0) ++b;
    return b;
}

// key[r] = original id of the first row of run r (runs of M tasks).
__global__ void __launch_bounds__(kBlock)
run_keys(const cwlb_task* __restrict__ tasks, long long n_tasks, int M, long long n_runs,
         const int* __restrict__ origin, int n_rows, unsigned* __restrict__ keys)
{
    const long long r = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x;
    if (r >= n_runs) return;
    const long long t = r * M < n_tasks ? r * M : n_tasks - 1;
    const int rs = min(max(tasks[t].row_start, 0), n_rows - 1);
    keys[r] = static_cast<unsigned>(origin[rs]);
}

template <class T>
cwlb_status grow(T** p, long long have, long long want)
{
    if (want <= have && *p) return CWLB_OK;
    if (*p) CWLB_HIP_TRY(hipFree(*p));
    *p = nullptr;
    CWLB_HIP_TRY(hipMalloc(reinterpret_cast<void**>(p), sizeof(T) * static_cast<size_t>(want)));
    return CWLB_OK;
}

}  // namespace

cwlb_status build_run_order(cwlb_ctx* ctx, const SpmmArgs& a, int M, long long n_runs,
                            bool may_build, const int** order)
{
    hipStream_t st = ctx->stream;
    if (n_runs <= 0 || a.n_rows <= 0) {
        *order = nullptr;
        return CWLB_OK;
    }
    if (ctx->order_tasks == a.tasks && ctx->order_origin == a.origin &&
        ctx->order_n_tasks == a.n_tasks && ctx->order_runs == n_runs && ctx->order_M == M) {
        *order = ctx->d_run_order;
        if (!may_build) ctx->order_captured = true;
        return CWLB_OK;
    }
    if (!may_build) {
        *order = nullptr;
        return CWLB_OK;
    }
    ctx->order_runs = -1;
    if (ctx->order_captured) {
        // A captured graph reads this order: keep it until cwlb_ctx_destroy.
        if (ctx->d_run_order) ctx->retired.push_back(ctx->d_run_order);
        ctx->d_run_order = nullptr;
        ctx->run_cap = 0;
        ctx->order_captured = false;
    }
    if (n_runs > ctx->run_cap) {
        cwlb_status s = grow(&ctx->d_run_keys, 0, n_runs);
        if (s == CWLB_OK) s = grow(&ctx->d_run_keys_sorted, 0, n_runs);
        if (s == CWLB_OK) s = grow(&ctx->d_run_order, 0, n_runs);
        if (s != CWLB_OK) {
            ctx->run_cap = 0;
            return s;
        }
        ctx->run_cap = n_runs;
    }
    const unsigned end_bit = std::max(1u, bits_for(static_cast<unsigned>(a.n_rows)));
    rocprim::counting_iterator<int> ids(0);
    size_t bytes = 0;
    CWLB_HIP_TRY(rocprim::radix_sort_pairs(nullptr, bytes, ctx->d_run_keys, ctx->d_run_keys_sorted,
                                           ids, ctx->d_run_order, n_runs, 0u, end_bit, st));
    if (bytes > ctx->sort_temp_bytes || !ctx->d_sort_temp) {
        if (ctx->d_sort_temp) CWLB_HIP_TRY(hipFree(ctx->d_sort_temp));
        ctx->d_sort_temp = nullptr;
        ctx->sort_temp_bytes = 0;
        CWLB_HIP_TRY(hipMalloc(&ctx->d_sort_temp, bytes ? bytes : 1));
        ctx->sort_temp_bytes = bytes;
    }
    const unsigned grid = static_cast<unsigned>((n_runs + kBlock - 1) / kBlock);
    hipLaunchKernelGGL(run_keys, dim3(grid), dim3(kBlock), 0, st, a.tasks,
                       static_cast<long long>(a.n_tasks), M, n_runs, a.origin, a.n_rows,
                       ctx->d_run_keys);
    CWLB_HIP_TRY(hipGetLastError());
    bytes = ctx->sort_temp_bytes;
    CWLB_HIP_TRY(rocprim::radix_sort_pairs(ctx->d_sort_temp, bytes, ctx->d_run_keys,
                                           ctx->d_run_keys_sorted, ids, ctx->d_run_order, n_runs,
                                           0u, end_bit, st));
    // The order is complete before any stream can use it (the context's
    // stream may be switched before the next call).
    CWLB_HIP_TRY(hipStreamSynchronize(st));
    ctx->order_tasks = a.tasks;
    ctx->order_origin = a.origin;
    ctx->order_n_tasks = a.n_tasks;
    ctx->order_runs = n_runs;
    ctx->order_M = M;
    *order = ctx->d_run_order;
    return CWLB_OK;
}

cwlb_status launch_reorder(cwlb_ctx* ctx, int32_t n, int64_t nnz, const int32_t* rp,
                           const int32_t* ci, const float* val, int32_t* origin, int32_t* rp_out,
                           int32_t* ci_out, float* val_out)
{
    hipStream_t st = ctx->stream;
    (void)hipGetLastError();  // report only the launches below
    if (n == 0) {
        if (!rp_out) return fail(CWLB_INVALID_ARG, "reorder: null row_ptr_out");
        hipLaunchKernelGGL(set_first_zero, dim3(1), dim3(1), 0, st, rp_out);
        CWLB_HIP_TRY(hipGetLastError());
        CWLB_HIP_TRY(hipStreamSynchronize(st));
        return CWLB_OK;
    }
    if (!rp || !origin || !rp_out || (nnz > 0 && (!ci || !val || !ci_out || !val_out)))
        return fail(CWLB_INVALID_ARG, "reorder: null device pointer");

    const size_t un = static_cast<size_t>(n);
    const unsigned grid = static_cast<unsigned>((un + kBlock - 1) / kBlock);
    DevMem keys, keys_sorted, flags, bmax;
    CWLB_HIP_TRY(keys.alloc(sizeof(unsigned) * un));
    CWLB_HIP_TRY(keys_sorted.alloc(sizeof(unsigned) * un));
    CWLB_HIP_TRY(flags.alloc(2 * sizeof(int)));
    CWLB_HIP_TRY(bmax.alloc(sizeof(unsigned) * grid));
    auto* d_keys = static_cast<unsigned*>(keys.p);
    auto* d_sorted = static_cast<unsigned*>(keys_sorted.p);
    auto* d_status = static_cast<int*>(flags.p);
    auto* d_max = reinterpret_cast<unsigned*>(d_status + 1);
    hipLaunchKernelGGL(clear_two, dim3(1), dim3(1), 0, st, d_status);
    CWLB_LAUNCH_CHECK("clear_two");
    hipLaunchKernelGGL(degree_keys, dim3(grid), dim3(kBlock), 0, st, rp, n,
                       static_cast<long long>(nnz), d_keys, d_status,
                       static_cast<unsigned*>(bmax.p));
    CWLB_LAUNCH_CHECK("degree_keys");
    hipLaunchKernelGGL(reduce_max, dim3(1), dim3(1024), 0, st, static_cast<unsigned*>(bmax.p),
                       static_cast<long long>(grid), d_max);
    CWLB_LAUNCH_CHECK("reduce_max");
    int host_flags[2] = {0, 0};
    int ends[2] = {0, 0};
    CWLB_HIP_TRY(hipMemcpyAsync(host_flags, d_status, sizeof host_flags, hipMemcpyDeviceToHost, st));
    CWLB_HIP_TRY(hipMemcpyAsync(&ends[0], rp, sizeof(int), hipMemcpyDeviceToHost, st));
    CWLB_HIP_TRY(hipMemcpyAsync(&ends[1], rp + n, sizeof(int), hipMemcpyDeviceToHost, st));
    CWLB_HIP_TRY(hipStreamSynchronize(st));
    if (host_flags[0] & 1)
        return fail(CWLB_INVALID_ARG, "cwlb_reorder_by_degree_device: row_ptr not a CSR offset array");
    if (static_cast<int64_t>(ends[1]) - ends[0] != nnz)
        return fail(CWLB_RUNTIME_ERROR,
                    "DPL CPU degree reordering produced an inconsistent NNZ count.");
    const unsigned end_bit = std::max(1u, bits_for(static_cast<unsigned>(host_flags[1])));

    rocprim::counting_iterator<int> ids(0);
    size_t sort_bytes = 0, scan_bytes = 0;
    CWLB_HIP_TRY(rocprim::radix_sort_pairs(nullptr, sort_bytes, d_keys, d_sorted, ids, origin, un,
                                           0u, end_bit, st));
    CWLB_HIP_TRY(rocprim::inclusive_scan(nullptr, scan_bytes, d_sorted, rp_out + 1, un,
                                         rocprim::plus<unsigned>(), st));
    DevMem temp;
    CWLB_HIP_TRY(temp.alloc(std::max(sort_bytes, scan_bytes)));
    size_t bytes = sort_bytes;
    CWLB_HIP_TRY(rocprim::radix_sort_pairs(temp.p, bytes, d_keys, d_sorted, ids, origin, un, 0u,
                                           end_bit, st));
    bytes = scan_bytes;
    CWLB_HIP_TRY(rocprim::inclusive_scan(temp.p, bytes, d_sorted, rp_out + 1, un,
                                         rocprim::plus<unsigned>(), st));
    hipLaunchKernelGGL(set_first_zero, dim3(1), dim3(1), 0, st, rp_out);
    CWLB_HIP_TRY(hipGetLastError());
    if (nnz > 0) {
        hipLaunchKernelGGL(gather_rows, dim3(grid), dim3(kBlock), 0, st, rp, ci, val, origin,
                           rp_out, n, ci_out, val_out);
        CWLB_LAUNCH_CHECK("gather_rows");
        // d_status[0] is free again (checked above): it receives the first
        // long row.  The long rows hold at most nnz entries.
        hipLaunchKernelGGL(find_long_rows, dim3(1), dim3(1), 0, st, d_sorted, n, d_status);
        CWLB_LAUNCH_CHECK("find_long_rows");
        const unsigned long_grid =
            static_cast<unsigned>((static_cast<uint64_t>(nnz) + kLongChunk - 1) / kLongChunk);
        hipLaunchKernelGGL(gather_long, dim3(long_grid), dim3(kBlock), 0, st, rp, ci, val,
                           origin, rp_out, n, d_status, ci_out, val_out);
        CWLB_LAUNCH_CHECK("gather_long");
    }
    CWLB_HIP_TRY(hipStreamSynchronize(st));
    return CWLB_OK;
}

}  // namespace cwlb
