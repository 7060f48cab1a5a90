/*
 * cwlb_driver.h -- the host pieces of the reference's cwlb-spmm driver,
 * exposed as a library so that other programs (and the tests) can use
 * them: degree reordering, segment-size selection, the deterministic
 * features and the timed single-S run (reference main.cpp:62-429).  The
 * reference defines these in main.cpp without a header; the cwlb-spmm
 * executable of this library is built from them.
 */
#pragma once

#include <array>
#include <cstddef>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "Matrix.h"
#include "config.h"
#include "cwlb_device.h"
#include "utils.h"

// Rows ordered by (degree, original id) ascending; RowOffset is the
// inclusive scan of the sorted degrees; each row keeps its entry order
// (reference main.cpp:197-278).  Fewer than 2 offsets give an empty result.
// Throws std::runtime_error when ColInd and Value differ in size or the
// offsets disagree with the entry count, std::overflow_error when a count
// does not fit int.
CSR_Order sortCSRByDegreeDPLCPU(const CSR& csr);

// Capacity of a task holding one full segment of s nonzeros:
// C_atomic + (C_compute + C_load) * max(1, s), clamped at 0 (main.cpp:281-292).
double capacity_from_s(int s, const SpmmCostParams& costs);

// S = clamp(ceil(NNZ / (compute_units * wave)), 1, INT_MAX); 1 for an empty
// RowOffset; std::invalid_argument for non-positive compute_units or wave
// (main.cpp:295-321).
int wave_based_s(const CSR_Order& sorted_csr, int compute_units, int wave);

// The three wave widths w of the --candidates mode, by NNZ (main.cpp:87-95).
std::array<int, 3> recommended_candidate_w(std::uint64_t nnz);

constexpr int MAX_CANDIDATE_SEARCH_POINTS = 10000;

// A positive integer spelled exactly (main.cpp:99-106).
int positive_search_argument(const std::string& text);
// Search interval around the best of three ordered S values (main.cpp:109-127).
std::pair<int, int> candidate_search_bounds(const std::array<int, 3>& values,
                                            std::size_t best_index);
// Near-uniform integer grid with both endpoints (main.cpp:130-148).
std::vector<int> candidate_search_by_count(int lower, int upper, int requested);
// lower, lower + step, ... plus upper (main.cpp:151-167).
std::vector<int> candidate_search_by_step(int lower, int upper, int step);

// Asks "Continue CWLB-SpMM for these S values? (yes/no): " on stdout until
// stdin gives yes or no (case-insensitive, trimmed); EOF means no
// (main.cpp:170-184).
bool confirm_candidate_search();

// rows x cols features, U[0, 1) from std::mt19937(42) in row-major order
// (main.cpp:324-336).
Defined::RowMajorMatrixXf deterministic_features(int rows, int cols);

struct SingleSResult {
    int s = 0;
    double capacity = 0.0;
    std::size_t task_count = 0;
    double average_us = 0.0;
    std::vector<double> timed_samples_us;
    Defined::RowMajorMatrixXf output;
    // Launch schedule the timed launches ran with: tasks per wave, feature
    // slices, run order, XCD placement (all 0 = the automatic schedule).
    std::array<int, 4> schedule{};
    // Cache-hint hot set in bytes the timed launches ran with (0 = none).
    std::int64_t cache_hint_bytes = 0;
    // 6 when the timed launches ran the occupancy variant, else 0.
    std::int32_t waves_per_simd = 0;
    // Column phases the timed launches ran with (0 = one pass).
    std::int32_t column_phases = 0;
    // Lane tiling the timed launches ran with (0 = automatic, 2 = packed
    // slots; see cwlb_ctx_set_lane_tiling).
    std::int32_t lane_tiling = 0;
};

// Builds the tasks for S (on the GPU, identical to the host partition), then
// runs LOOPCOUNT SpMM launches (the first
// WARMUPCOUNT untimed) and averages the kernel times of the rest, printing
// one line per launch (main.cpp:338-412).  The kernel is the large-K form
// when K exceeds the device's maximum work-group size.  The reordered CSR
// and H are uploaded once and stay on the device across the launches (the
// reference re-copies them every launch; its timing excludes the copies).
// Before the timed launches the launch schedule is tuned once for this S
// (cwlb_ctx_tune_schedule, untimed; the environment variable
// CWLB_TUNE_SCHEDULE=0 keeps the automatic schedule instead).  The schedule
// stays set on the device afterwards.
SingleSResult run_single_s(cwlb::Device& queue, const CSR_Order& sorted_csr,
                           const Defined::RowMajorMatrixXf& features, int feature_dim,
                           const SpmmCostParams& costs, int s, bool retain_timed_samples = false);

// "Dataset: ...", "V: .., E: ..", "SpMM time: .. us", "costs: ..." (main.cpp:414-429).
void print_single_s_result(const std::string& dataset, int vertex_count, int edge_count,
                           const SpmmCostParams& costs, const SingleSResult& result);

// The cwlb-spmm command line (main.cpp:431-741): returns the process exit
// status.  Exposed so the executable is a one-line main().
int cwlb_spmm_main(int argc, char* argv[]);

// The costWrite command line (weightCost.cpp:11-77).
int cost_write_main(int argc, char* argv[]);
