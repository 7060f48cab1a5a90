// Host pieces of the cwlb-spmm driver (reference main.cpp:86-429): degree
// reordering, segment-size selection, features and the timed single-S run.
#include <algorithm>
#include <cctype>
#include <cstdint>
#include <cstdlib>
#include <iomanip>
#include <iostream>
#include <limits>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "cwlb_driver.h"
#include "host_internal.h"

using cwlb::host::DeviceArray;

CSR_Order sortCSRByDegreeDPLCPU(const CSR& csr)
{
    CSR_Order out;
    if (csr.RowOffset.size() < 2) return out;
    if (csr.ColInd.size() != csr.Value.size())
        throw std::runtime_error("CSR ColInd and Value size mismatch.");
    const std::size_t rows = csr.RowOffset.size() - 1;
    const std::size_t nnz = csr.ColInd.size();
    if (rows > static_cast<std::size_t>(std::numeric_limits<int>::max()) ||
        nnz > static_cast<std::size_t>(std::numeric_limits<int>::max()))
        throw std::overflow_error(
            "DPL CPU degree reordering requires row and NNZ counts to fit in int.");
    // The C entry point checks the offsets against nnz; an inconsistent CSR
    // is the reference's "inconsistent NNZ count" runtime_error.
    for (std::size_t i = 0; i < rows; ++i)
        if (csr.RowOffset[i + 1] < csr.RowOffset[i] || csr.RowOffset[i] < 0 ||
            static_cast<std::size_t>(csr.RowOffset[i + 1]) > nnz)
            throw std::runtime_error("DPL CPU degree reordering produced an inconsistent NNZ count.");
    out.Origin_local.resize(rows);
    out.RowOffset.resize(rows + 1);
    out.ColInd.resize(nnz);
    out.Value.resize(nnz);
    cwlb::check(cwlb_reorder_by_degree(static_cast<int32_t>(rows), static_cast<int64_t>(nnz),
                                       csr.RowOffset.data(), csr.ColInd.data(), csr.Value.data(),
                                       out.Origin_local.data(), out.RowOffset.data(),
                                       out.ColInd.data(), out.Value.data()),
                "sortCSRByDegreeDPLCPU");
    return out;
}

double capacity_from_s(int s, const SpmmCostParams& costs)
{
    const cwlb_cost_params c = cwlb::host::to_c(costs);
    return cwlb_capacity_from_s(s, &c);
}

int wave_based_s(const CSR_Order& sorted_csr, int compute_units, int wave)
{
    const int64_t nnz = sorted_csr.RowOffset.empty() ? 0 : sorted_csr.RowOffset.back();
    int32_t s = 0;
    cwlb::check(cwlb_wave_based_s(nnz, static_cast<int64_t>(sorted_csr.RowOffset.size()),
                                  compute_units, wave, &s),
                "wave_based_s");
    return s;
}

std::array<int, 3> recommended_candidate_w(std::uint64_t nnz)
{
    int32_t w[3];
    cwlb_recommended_candidate_w(nnz, w);
    return {w[0], w[1], w[2]};
}

int positive_search_argument(const std::string& text)
{
    std::size_t used = 0;
    const int v = std::stoi(text, &used);
    if (used != text.size() || v <= 0)
        throw std::invalid_argument("Search count/step must be a positive integer.");
    return v;
}

std::pair<int, int> candidate_search_bounds(const std::array<int, 3>& values,
                                            std::size_t best_index)
{
    if (best_index >= values.size())
        throw std::invalid_argument("Invalid ordered candidate values or best index.");
    int32_t lo = 0, hi = 0;
    const int32_t v[3] = {values[0], values[1], values[2]};
    cwlb::check(cwlb_candidate_search_bounds(v, static_cast<int64_t>(best_index), &lo, &hi),
                "candidate_search_bounds");
    return {lo, hi};
}

namespace {

template <class Fn>
std::vector<int> search_grid(Fn fn, int lower, int upper, int third, const char* what)
{
    int64_t count = 0;
    cwlb_status st = fn(lower, upper, third, nullptr, 0, &count);
    if (st != CWLB_OK && st != CWLB_INSUFFICIENT) cwlb::throw_status(st, what);
    std::vector<int> out(static_cast<std::size_t>(count));
    cwlb::check(fn(lower, upper, third, out.data(), count, &count), what);
    return out;
}

}  // namespace

std::vector<int> candidate_search_by_count(int lower, int upper, int requested)
{
    return search_grid(cwlb_candidate_search_by_count, lower, upper, requested,
                       "candidate_search_by_count");
}

std::vector<int> candidate_search_by_step(int lower, int upper, int step)
{
    return search_grid(cwlb_candidate_search_by_step, lower, upper, step,
                       "candidate_search_by_step");
}

bool confirm_candidate_search()
{
    std::string answer;
    for (;;) {
        std::cout << "Continue CWLB-SpMM for these S values? (yes/no): " << std::flush;
        if (!std::getline(std::cin, answer)) return false;
        const auto b = answer.find_first_not_of(" \t\r\n");
        const auto e = answer.find_last_not_of(" \t\r\n");
        answer = b == std::string::npos ? std::string() : answer.substr(b, e - b + 1);
        for (char& ch : answer) ch = static_cast<char>(std::tolower(static_cast<unsigned char>(ch)));
        if (answer == "yes") return true;
        if (answer == "no") return false;
        std::cout << "Please enter yes or no.\n";
    }
}

Defined::RowMajorMatrixXf deterministic_features(int rows, int cols)
{
    Defined::RowMajorMatrixXf f(rows, cols);
    std::mt19937 gen(42);
    std::uniform_real_distribution<float> dist(0.0f, 1.0f);
    float* p = f.data();
    const long long total = static_cast<long long>(rows) * cols;
    for (long long i = 0; i < total; ++i) p[i] = dist(gen);
    return f;
}

SingleSResult run_single_s(cwlb::Device& queue, const CSR_Order& csr,
                           const Defined::RowMajorMatrixXf& features, int feature_dim,
                           const SpmmCostParams& costs, int s, bool retain_timed_samples)
{
    SingleSResult result;
    result.s = s;
    result.capacity = capacity_from_s(s, costs);
    // The GPU partition (identical tasks; the host one for costs it does not take).
    const std::vector<ParallelDataWeighted> tasks =
        costWeightedTaskPartitioning_HIP(csr, costs, result.capacity, queue);
    result.task_count = tasks.size();

    const bool large_k = feature_dim > queue.max_work_group_size();
    const long long K = features.cols();
    const std::size_t rows = csr.Origin_local.size();
    if (csr.RowOffset.size() != rows + 1 || csr.ColInd.size() != csr.Value.size())
        throw std::invalid_argument("run_single_s: inconsistent CSR_Order");
    if (K > std::numeric_limits<int32_t>::max())
        throw std::invalid_argument("run_single_s: K must fit int32");
    for (int c : csr.ColInd)
        if (c < 0 || c >= features.rows())
            throw std::invalid_argument("run_single_s: column index outside the feature rows");

    // Inputs stay on the device across the LOOPCOUNT launches.
    cwlb::host::CurrentDevice cur(queue);
    const std::size_t nnz = csr.ColInd.size();
    DeviceArray<int> d_rp(rows + 1), d_ci(nnz), d_o(rows);
    DeviceArray<float> d_v(nnz), d_h(static_cast<std::size_t>(features.size())),
        d_c(rows * static_cast<std::size_t>(K));
    DeviceArray<cwlb_task> d_t(tasks.size());
    d_rp.upload(csr.RowOffset);
    d_ci.upload(csr.ColInd);
    d_v.upload(csr.Value);
    d_o.upload(csr.Origin_local);
    d_h.upload(features.data(), static_cast<std::size_t>(features.size()));
    d_t.upload(cwlb::host::as_c_tasks(tasks), tasks.size());

    // The launch schedule for this graph and S, timed once before the timed
    // launches like the S search itself (cwlb_ctx_tune_schedule), unless
    // CWLB_TUNE_SCHEDULE=0 keeps the automatic schedule.  Both start from
    // the automatic schedule in task order with the standard kernel, no
    // cache hints and one pass, so every S is treated alike.
    cwlb::check(cwlb_ctx_set_schedule(queue.ctx(), 0, 0), "cwlb_ctx_set_schedule");
    cwlb::check(cwlb_ctx_set_locality(queue.ctx(), 0, 0), "cwlb_ctx_set_locality");
    cwlb::check(cwlb_ctx_set_cache_hints(queue.ctx(), 0), "cwlb_ctx_set_cache_hints");
    cwlb::check(cwlb_ctx_set_occupancy(queue.ctx(), 0), "cwlb_ctx_set_occupancy");
    cwlb::check(cwlb_ctx_set_column_phases(queue.ctx(), 0), "cwlb_ctx_set_column_phases");
    cwlb::check(cwlb_ctx_set_lane_tiling(queue.ctx(), 0), "cwlb_ctx_set_lane_tiling");
    const char* tune_env = std::getenv("CWLB_TUNE_SCHEDULE");
    const bool tune = !(tune_env && std::string(tune_env) == "0");
    if (tune && !tasks.empty() && K > 0) {
        int32_t m = 0, sl = 0, loc[2] = {0, 0};
        cwlb::check(cwlb_ctx_tune_schedule(queue.ctx(), d_rp.get(), d_ci.get(), d_v.get(),
                                           d_o.get(), static_cast<int32_t>(rows),
                                           static_cast<int64_t>(nnz), d_h.get(),
                                           static_cast<int64_t>(features.rows()),
                                           static_cast<int32_t>(K), d_t.get(),
                                           static_cast<int64_t>(tasks.size()), d_c.get(), 3, &m,
                                           &sl, loc),
                    "cwlb_ctx_tune_schedule");
        result.schedule = {m, sl, loc[0], loc[1]};
        cwlb::check(cwlb_ctx_get_cache_hints(queue.ctx(), &result.cache_hint_bytes),
                    "cwlb_ctx_get_cache_hints");
        cwlb::check(cwlb_ctx_get_occupancy(queue.ctx(), &result.waves_per_simd),
                    "cwlb_ctx_get_occupancy");
        cwlb::check(cwlb_ctx_get_column_phases(queue.ctx(), &result.column_phases),
                    "cwlb_ctx_get_column_phases");
        cwlb::check(cwlb_ctx_get_lane_tiling(queue.ctx(), &result.lane_tiling),
                    "cwlb_ctx_get_lane_tiling");
    }

    const std::string device_name = queue.name();
    double accumulated = 0.0;
    for (int it = 0; it < LOOPCOUNT; ++it) {
        cwlb_timing t{};
        // The first launch clears all of C (the reference's zeroed output);
        // later launches rewrite every row with nonzeros and, as the
        // reference's kernel, leave the rows without nonzeros at that 0.
        const uint32_t flags = it == 0 ? CWLB_SPMM_ZERO_OUTPUT : CWLB_SPMM_KEEP_EMPTY_ROWS;
        const auto fn = large_k ? cwlb_spmm_mean_f32_large_k : cwlb_spmm_mean_f32;
        cwlb::check(fn(queue.ctx(), d_rp.get(), d_ci.get(), d_v.get(), d_o.get(),
                       static_cast<int32_t>(rows), static_cast<int64_t>(nnz), d_h.get(),
                       static_cast<int64_t>(features.rows()), static_cast<int32_t>(K),
                       tasks.empty() ? nullptr : d_t.get(), static_cast<int64_t>(tasks.size()),
                       d_c.get(), flags, &t),
                    large_k ? "spmmKernelLargeKFallback" : "spmmKernel");
        // Clearing of split rows is part of the reported time; the full
        // clear of the first launch stands for the host-side Zero() and is not.
        const double elapsed_us = it == 0 ? t.main_us : t.total_us;
        const bool warmup = it < WARMUPCOUNT;
        std::cout << std::fixed << std::setprecision(6) << (warmup ? "[Warm-up " : "[Iteration ")
                  << (warmup ? it + 1 : it - WARMUPCOUNT + 1) << '/'
                  << (warmup ? WARMUPCOUNT : LOOPCOUNT - WARMUPCOUNT)
                  << "] device=" << device_name << " K=" << feature_dim
                  << " time=" << elapsed_us << " us\n";
        if (!warmup) {
            accumulated += elapsed_us;
            if (retain_timed_samples) result.timed_samples_us.push_back(elapsed_us);
        }
    }
    result.average_us = accumulated / static_cast<double>(LOOPCOUNT - WARMUPCOUNT);
    result.output = Defined::RowMajorMatrixXf(static_cast<long>(rows), K);
    d_c.download(result.output.data(), rows * static_cast<std::size_t>(K));
    return result;
}

void print_single_s_result(const std::string& dataset, int vertex_count, int edge_count,
                           const SpmmCostParams& costs, const SingleSResult& result)
{
    std::cout << std::fixed << std::setprecision(6) << "Dataset: " << dataset << '\n'
              << "V: " << vertex_count << ", E: " << edge_count << '\n'
              << "SpMM time: " << result.average_us << " us\n"
              << "costs: C_compute_ns=" << costs.C_compute_ns << " C_load_ns=" << costs.C_load_ns
              << " C_store_ns=" << costs.C_store_ns << " C_atomic_ns=" << costs.C_atomic_ns
              << '\n';
}
