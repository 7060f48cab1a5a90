// Operation-cost calibration for gfx950 (the reference's measure_spmm_costs,
// src/utils.cpp:342-829), re-measured here rather than reusing coefficients
// from other GPUs.
//
// Four micro-benchmarks, each with 20 warm-up launches and `repeat` timed
// launches (HIP events around each launch, then a wait):
//   compute  a chain of K dependent fmas per work-item      (utils.cpp:370-427)
//   load     every wave reads K floats of one random row of a
//            load_MB array, lane l reading column (t*64 + l) mod K
//                                                              (utils.cpp:430-531)
//   store    K coalesced stores per work-item                 (utils.cpp:534-591)
//   atomic   `writers` logical 128-lane groups add 1.0f into the
//            same K_block-wide output row, relaxed agent scope (utils.cpp:597-825)
// Each coefficient is (ns per op per work-item) x 10, as in the reference
// (utils.cpp:419-421, 522-524, 583-585, 791-806).  The load benchmark groups
// lanes by the 64-lane wavefront (the reference groups by 32 lanes) and
// issues non-temporal loads where the reference's are plain
// (utils.cpp:470-481).  Each wave reads its one row K times over, and plain
// loads serve those repeats from the L1 (measured: 0.01100 against 0.01584
// with non-temporal loads, K = 128, WI = 131072, 512 MB); the aggregation's
// gathers read a feature row once per nonzero, so they see no such reuse.
// Partitions from either figure run the aggregation equally fast (R-MAT,
// Chung-Lu and mesh within 0.2%).
#include <algorithm>
#include <cstdio>
#include <random>
#include <vector>

#include "internal.h"

namespace cwlb {
namespace {

constexpr int kCalWarmup = 20;

__global__ void bench_compute(float* __restrict__ sink, int WI, int K)
{
    const int id = blockIdx.x * blockDim.x + threadIdx.x;
    if (id >= WI) return;
    float acc = 0.0f;
    const float a = 1.001f, b = 0.999f;
    for (int i = 0; i < K; ++i) acc = __builtin_fmaf(acc, a, b);
    sink[id] = acc;
}

__global__ void bench_load(const float* __restrict__ data, const unsigned* __restrict__ idx,
                           int WI, int K, float* __restrict__ sink)
{
    const int gid = blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= WI) return;
    const int lane = gid & 63;
    const unsigned row = idx[gid - lane];
    const float* base = data + static_cast<size_t>(row) * K;
    float s = 0.0f;
    for (int t = 0; t < K; ++t) {
        int k = t * 64 + lane;
        if (k >= K) k %= K;
        s += __builtin_nontemporal_load(base + k);
    }
    // Keeps the loads live without writing in the common case.
    if (s == -1.0f) sink[gid] = s;
}

__global__ void bench_store(float* __restrict__ out, int WI, int K)
{
    const int tid = blockIdx.x * blockDim.x + threadIdx.x;
    if (tid >= WI) return;
    for (int i = 0; i < K; ++i) out[static_cast<size_t>(i) * WI + tid] = static_cast<float>(i);
}

__global__ void bench_atomic(float* __restrict__ counters, int G, int groups_per_row,
                             int K_block, long long counter_len, long long total_threads)
{
    const long long t = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total_threads) return;
    const unsigned lane = static_cast<unsigned>(t % 128);
    const unsigned group_id = static_cast<unsigned>(t / 128);
    const unsigned row_gid = group_id / static_cast<unsigned>(groups_per_row);
    if (row_gid >= static_cast<unsigned>(G)) return;
    for (unsigned kk = lane; kk < static_cast<unsigned>(K_block); kk += 128) {
        const long long i = static_cast<long long>(row_gid) * K_block + kk;
        if (i >= counter_len) return;
        unsafeAtomicAdd(counters + i, 1.0f);
    }
}

__global__ void fill_value(float* __restrict__ p, long long n, float v)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
         i += stride)
        p[i] = v;
}

// Times `launch` with events: warm-ups, then `repeat` timed runs, each
// preceded by `before` (not timed).  Returns the mean in milliseconds.
template <class Launch, class Before>
cwlb_status time_launches(cwlb_ctx* ctx, int repeat, Launch launch, Before before, double* mean_ms)
{
    hipStream_t st = ctx->stream;
    for (int w = 0; w < kCalWarmup; ++w) {
        before();
        launch();
        CWLB_HIP_TRY(hipGetLastError());
        CWLB_HIP_TRY(hipStreamSynchronize(st));
    }
    double total = 0.0;
    for (int r = 0; r < repeat; ++r) {
        before();
        CWLB_HIP_TRY(hipEventRecord(ctx->ev[0], st));
        launch();
        CWLB_HIP_TRY(hipGetLastError());
        CWLB_HIP_TRY(hipEventRecord(ctx->ev[1], st));
        CWLB_HIP_TRY(hipEventSynchronize(ctx->ev[1]));
        float ms = 0.0f;
        CWLB_HIP_TRY(hipEventElapsedTime(&ms, ctx->ev[0], ctx->ev[1]));
        total += ms;
    }
    *mean_ms = total / static_cast<double>(repeat);
    return CWLB_OK;
}

template <class T>
struct Buf {
    T* p = nullptr;
    Buf() = default;
    Buf(const Buf&) = delete;
    Buf& operator=(const Buf&) = delete;
    ~Buf()
    {
        if (p) (void)hipFree(p);
    }
};

}  // namespace

cwlb_status run_calibration(cwlb_ctx* ctx, int32_t K, int32_t repeat, int32_t WI, int32_t load_MB,
                            int32_t atomic_writers, cwlb_cost_params* out,
                            cwlb_calibration_report* report)
{
    hipStream_t st = ctx->stream;
    cwlb_calibration_report rep{};
    *out = cwlb_cost_params{};
    out->K = K;
    out->WI = WI;
    out->repeat = repeat;
    const int block = 256;
    const unsigned grid = static_cast<unsigned>((static_cast<long long>(WI) + block - 1) / block);
    auto nothing = [] {};

    {  // compute
        Buf<float> sink;
        CWLB_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&sink.p), sizeof(float) * WI));
        double ms = 0.0;
        cwlb_status s = time_launches(
            ctx, repeat,
            [&] { hipLaunchKernelGGL(bench_compute, dim3(grid), dim3(block), 0, st, sink.p, WI, K); },
            nothing, &ms);
        if (s != CWLB_OK) return s;
        out->C_compute_ns = (ms * 1e6) / static_cast<double>(WI) / static_cast<double>(K) * 10;
        rep.compute_ms = ms;
        rep.compute_ops = static_cast<int64_t>(WI) * K;
    }
    {  // load
        const size_t total_floats = static_cast<size_t>(load_MB) * 1024ull * 1024ull / sizeof(float);
        if (total_floats < static_cast<size_t>(K))
            return fail(CWLB_RUNTIME_ERROR, "data_MB_for_load too small for K.");
        const size_t rows = total_floats / static_cast<size_t>(K);
        Buf<float> data, sink;
        Buf<unsigned> idx;
        CWLB_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&data.p), sizeof(float) * total_floats));
        CWLB_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&idx.p), sizeof(unsigned) * WI));
        CWLB_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&sink.p), sizeof(float) * WI));
        hipLaunchKernelGGL(fill_value, dim3(4096), dim3(256), 0, st, data.p,
                           static_cast<long long>(total_floats), 1.2345f);
        std::vector<unsigned> h(static_cast<size_t>(WI));
        std::mt19937_64 rng(123456789ULL);
        std::uniform_int_distribution<unsigned> dist(0u, static_cast<unsigned>(rows - 1));
        for (int g0 = 0; g0 < WI; g0 += 64) {
            const unsigned row = dist(rng);
            for (int t = 0; t < 64 && g0 + t < WI; ++t) h[g0 + t] = row;
        }
        CWLB_HIP_TRY(hipMemcpy(idx.p, h.data(), sizeof(unsigned) * WI, hipMemcpyHostToDevice));
        double ms = 0.0;
        cwlb_status s = time_launches(
            ctx, repeat,
            [&] {
                hipLaunchKernelGGL(bench_load, dim3(grid), dim3(block), 0, st, data.p, idx.p, WI, K,
                                   sink.p);
            },
            nothing, &ms);
        if (s != CWLB_OK) return s;
        out->C_load_ns = (ms * 1e6) / static_cast<double>(WI) / static_cast<double>(K) * 10;
        rep.load_ms = ms;
        rep.load_ops = static_cast<int64_t>(WI) * K;
        rep.load_bytes = static_cast<int64_t>(WI) * K * 4;
    }
    {  // store
        Buf<float> obuf;
        CWLB_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&obuf.p),
                               sizeof(float) * static_cast<size_t>(WI) * static_cast<size_t>(K)));
        double ms = 0.0;
        cwlb_status s = time_launches(
            ctx, repeat,
            [&] { hipLaunchKernelGGL(bench_store, dim3(grid), dim3(block), 0, st, obuf.p, WI, K); },
            nothing, &ms);
        if (s != CWLB_OK) return s;
        out->C_store_ns = (ms * 1e6) / static_cast<double>(WI) / static_cast<double>(K) * 10;
        rep.store_ms = ms;
        rep.store_ops = static_cast<int64_t>(WI) * K;
        rep.store_bytes = static_cast<int64_t>(WI) * K * 4;
    }
    {  // atomic
        const int gpr = std::max(1, atomic_writers);
        const int pseudo = 128;
        int K_block = std::min(K, 128);
        K_block = (K_block / 32) * 32;
        if (K_block <= 0) K_block = 32;
        const int target = std::max(1, (WI + pseudo - 1) / pseudo);
        int G = std::max(1, target / gpr);
        long long total_groups = static_cast<long long>(G) * gpr;
        while (total_groups < target) {
            ++G;
            total_groups = static_cast<long long>(G) * gpr;
        }
        const long long threads = total_groups * pseudo;
        const long long counter_len = static_cast<long long>(G) * K_block;
        Buf<float> counters;
        CWLB_HIP_TRY(hipMalloc(reinterpret_cast<void**>(&counters.p), sizeof(float) * counter_len));
        const unsigned agrid = static_cast<unsigned>((threads + block - 1) / block);
        double ms = 0.0;
        cwlb_status s = time_launches(
            ctx, repeat,
            [&] {
                hipLaunchKernelGGL(bench_atomic, dim3(agrid), dim3(block), 0, st, counters.p, G, gpr,
                                   K_block, counter_len, threads);
            },
            [&] {
                hipLaunchKernelGGL(fill_value, dim3(256), dim3(256), 0, st, counters.p, counter_len,
                                   0.0f);
            },
            &ms);
        if (s != CWLB_OK) return s;
        const double ops = static_cast<double>(total_groups) * static_cast<double>(K_block);
        out->C_atomic_ns = (ms * 1e6) / ops * 10.0;
        out->atomic_writers_per_addr = gpr;
        rep.atomic_ms = ms;
        rep.atomic_ops = total_groups * K_block;
    }
    CWLB_HIP_TRY(hipStreamSynchronize(st));
    if (report) *report = rep;
    return CWLB_OK;
}

}  // namespace cwlb
