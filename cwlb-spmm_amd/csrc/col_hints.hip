// Cache-policy hints for the feature-row gathers.
//
// On graphs whose column in-degrees are skewed (R-MAT, power laws) a small
// set of feature rows takes most of the gathers.  The aggregation kernel can
// load the rows of the other, "cold" columns with the non-temporal policy,
// so that they do not push the hot rows out of L2 and the Infinity Cache.
// The hint is one bit per nonzero (1 = cold column), built on the device:
//   1. column_counts: the in-degree of every column, counted on every
//      stride-th nonzero (stride = 1 up to kSampleTarget nonzeros, then
//      the smallest stride that keeps about kSampleTarget of them: a
//      sample keeps the order of the large in-degrees that decide the hot
//      set, at a fraction of the contended atomics);
//   2. count_buckets: a histogram of the in-degrees over kBuckets
//      log-spaced buckets (exact below 64, then 8 buckets per octave);
//   3. on the host, the in-degree threshold theta: the lowest bucket floor
//      such that the columns with in-degree >= theta number at most
//      hot_rows (the requested hot set, in feature rows);
//   4. cold_bits: bit j of the hint array = in-degree(col_idx[j]) < theta,
//      one 64-bit word per 64 nonzeros (a wave ballot).
// Hints change only the cache policy of loads, never a value, so hints
// built for other contents of col_idx can only cost speed.  The hint array
// is kept on the context and rebuilt when the column array, its length, the
// feature row count or the hot-set size changes.
#include <algorithm>
#include <climits>
#include <vector>

#include "internal.h"

namespace cwlb {
namespace {

constexpr int kBlock = 256;
constexpr long long kSampleTarget = 8ll << 20;  // in-degree samples at most (about)
constexpr int kBuckets = 64 + 26 * 8;  // exact 0..63, then 8 per octave up to 2^32

__device__ __forceinline__ int bucket_of(unsigned v)
{
    if (v < 64) return static_cast<int>(v);
    const int e = 31 - __clz(static_cast<int>(v));  // 6..31
    const int sub = static_cast<int>((v >> (e - 3)) & 7u);
    return 64 + (e - 6) * 8 + sub;
}

// Smallest in-degree that falls into bucket b.
unsigned bucket_floor(int b)
{
    if (b < 64) return static_cast<unsigned>(b);
    const int e = (b - 64) / 8 + 6;
    const unsigned sub = static_cast<unsigned>((b - 64) % 8);
    return (8u + sub) << (e - 3);
}

__global__ void __launch_bounds__(kBlock) zero_u32(unsigned* __restrict__ p, long long n)
{
    const long long stride = static_cast<long long>(gridDim.x) * kBlock;
    for (long long i = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += stride)
        p[i] = 0u;
}

__global__ void __launch_bounds__(kBlock)
column_counts(const int* __restrict__ ci, long long nnz, long long h_rows, long long sample,
              unsigned* __restrict__ counts)
{
    const long long n = (nnz + sample - 1) / sample;
    const long long stride = static_cast<long long>(gridDim.x) * kBlock;
    for (long long i = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x; i < n;
         i += stride) {
        const int c = ci[i * sample];
        if (c >= 0 && c < h_rows) atomicAdd(counts + c, 1u);
    }
}

__global__ void __launch_bounds__(kBlock)
count_buckets(const unsigned* __restrict__ counts, long long h_rows, unsigned* __restrict__ hist)
{
    __shared__ unsigned local[kBuckets];
    for (int b = threadIdx.x; b < kBuckets; b += kBlock) local[b] = 0u;
    __syncthreads();
    const long long stride = static_cast<long long>(gridDim.x) * kBlock;
    for (long long i = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x; i < h_rows;
         i += stride)
        atomicAdd(local + bucket_of(counts[i]), 1u);
    __syncthreads();
    for (int b = threadIdx.x; b < kBuckets; b += kBlock)
        if (local[b]) atomicAdd(hist + b, local[b]);
}

__global__ void __launch_bounds__(kBlock)
cold_bits(const int* __restrict__ ci, long long nnz, long long h_rows,
          const unsigned* __restrict__ counts, unsigned theta, long long words,
          unsigned long long* __restrict__ bits)
{
    const long long j = static_cast<long long>(blockIdx.x) * kBlock + threadIdx.x;
    bool cold = false;
    if (j < nnz) {
        const int c = ci[j];
        cold = c >= 0 && c < h_rows && counts[c] < theta;
    }
    const unsigned long long m = __ballot(cold);
    if ((threadIdx.x & 63) == 0 && (j >> 6) < words) bits[j >> 6] = m;
}

template <class T>
cwlb_status grow_buffer(T** p, long long* cap, long long want)
{
    if (*p && want <= *cap) return CWLB_OK;
    if (*p) CWLB_HIP_TRY(hipFree(*p));
    *p = nullptr;
    *cap = 0;
    CWLB_HIP_TRY(hipMalloc(reinterpret_cast<void**>(p), sizeof(T) * static_cast<size_t>(want)));
    *cap = want;
    return CWLB_OK;
}

unsigned grid_for(long long n)
{
    return static_cast<unsigned>(std::max<long long>(1, std::min<long long>((n + kBlock - 1) / kBlock, 65536)));
}

}  // namespace

cwlb_status build_cache_hints(cwlb_ctx* ctx, const SpmmArgs& a, long long hot_rows,
                              bool may_build, const unsigned long long** hints)
{
    *hints = nullptr;
    if (a.nnz <= 0 || a.h_rows <= 0 || hot_rows <= 0) return CWLB_OK;
    if (ctx->hint_col == a.col_idx && ctx->hint_nnz == a.nnz && ctx->hint_h_rows == a.h_rows &&
        ctx->hint_hot_rows == hot_rows) {
        *hints = ctx->hint_any_cold ? ctx->d_hints : nullptr;
        if (!may_build && *hints) ctx->hints_captured = true;
        return CWLB_OK;
    }
    if (!may_build) return CWLB_OK;
    ctx->hint_col = nullptr;  // invalid until rebuilt
    if (ctx->hints_captured) {
        // A captured graph reads these bits: keep them until cwlb_ctx_destroy.
        if (ctx->d_hints) ctx->retired.push_back(ctx->d_hints);
        ctx->d_hints = nullptr;
        ctx->hint_cap = 0;
        ctx->hints_captured = false;
    }
    hipStream_t st = ctx->stream;
    const long long words = (static_cast<long long>(a.nnz) + 63) / 64;
    long long hist_cap = ctx->d_count_hist ? kBuckets : 0;
    cwlb_status s = grow_buffer(&ctx->d_col_counts, &ctx->col_count_cap, a.h_rows);
    if (s == CWLB_OK) s = grow_buffer(&ctx->d_count_hist, &hist_cap, kBuckets);
    if (s == CWLB_OK) s = grow_buffer(&ctx->d_hints, &ctx->hint_cap, words);
    if (s != CWLB_OK) return s;
    hipLaunchKernelGGL(zero_u32, dim3(grid_for(a.h_rows)), dim3(kBlock), 0, st,
                       ctx->d_col_counts, static_cast<long long>(a.h_rows));
    CWLB_LAUNCH_CHECK("zero_u32");
    hipLaunchKernelGGL(zero_u32, dim3(1), dim3(kBlock), 0, st, ctx->d_count_hist,
                       static_cast<long long>(kBuckets));
    CWLB_LAUNCH_CHECK("zero_u32");
    const long long sample = std::max(1ll, static_cast<long long>(a.nnz) / kSampleTarget);
    hipLaunchKernelGGL(column_counts, dim3(grid_for(a.nnz / sample)), dim3(kBlock), 0, st,
                       a.col_idx, static_cast<long long>(a.nnz), static_cast<long long>(a.h_rows),
                       sample, ctx->d_col_counts);
    CWLB_LAUNCH_CHECK("column_counts");
    hipLaunchKernelGGL(count_buckets, dim3(std::min(grid_for(a.h_rows), 1024u)), dim3(kBlock), 0,
                       st, ctx->d_col_counts, static_cast<long long>(a.h_rows), ctx->d_count_hist);
    CWLB_LAUNCH_CHECK("count_buckets");
    std::vector<unsigned> hist(kBuckets);
    CWLB_HIP_TRY(hipMemcpyAsync(hist.data(), ctx->d_count_hist, sizeof(unsigned) * kBuckets,
                                hipMemcpyDeviceToHost, st));
    CWLB_HIP_TRY(hipStreamSynchronize(st));
    // Columns from the top bucket down while at most hot_rows of them; the
    // top non-empty bucket is always hot.
    unsigned theta = UINT_MAX;
    unsigned long long taken = 0;
    for (int b = kBuckets - 1; b >= 1; --b) {
        if (!hist[b]) continue;
        if (theta != UINT_MAX && taken + hist[b] > static_cast<unsigned long long>(hot_rows)) break;
        taken += hist[b];
        theta = bucket_floor(b);
    }
    // Nothing cold (every gathered column is hot): no hints.  With a
    // sample, columns missing from it (count 0) are gathered and cold.
    ctx->hint_any_cold = theta != UINT_MAX && (theta > 1 || sample > 1);
    if (ctx->hint_any_cold) {
        hipLaunchKernelGGL(cold_bits, dim3(static_cast<unsigned>((a.nnz + kBlock - 1) / kBlock)),
                           dim3(kBlock), 0, st, a.col_idx, static_cast<long long>(a.nnz),
                           static_cast<long long>(a.h_rows), ctx->d_col_counts, theta, words,
                           ctx->d_hints);
        CWLB_LAUNCH_CHECK("cold_bits");
    }
    ctx->hint_col = a.col_idx;
    ctx->hint_nnz = a.nnz;
    ctx->hint_h_rows = a.h_rows;
    ctx->hint_hot_rows = hot_rows;
    ctx->hint_theta = theta;
    *hints = ctx->hint_any_cold ? ctx->d_hints : nullptr;
    return CWLB_OK;
}

}  // namespace cwlb
