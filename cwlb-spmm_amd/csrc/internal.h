// Internal declarations shared by the libcwlb translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <vector>

#include "cwlb.h"

struct cwlb_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
    // Recorded on the old stream by cwlb_ctx_set_stream for the new one to
    // wait on.
    hipEvent_t switch_ev = nullptr;
    int compute_units = 0;
    int max_wg = 0;
    int wave = 64;
    size_t lds_per_block = 0;
    size_t total_mem = 0;
    char name[256] = {0};
    char arch[64] = {0};
    // Device status words written by the kernels.  [0]: bit 0 = a column
    // index was outside [0, h_rows), bit 1 = an origin entry was outside
    // [0, n_rows), bit 2 = a row's offsets left [0, nnz] or decreased.
    // [1]: cleared by each column-phased call's band sort, then set to the
    // call's sequence number when its task list is not a chain.
    int* d_status = nullptr;
    // Schedule overrides (0 = automatic): tasks per wave, feature slices,
    // run order (1 = task order, 2 = by output row id) and block placement
    // over the XCDs (1 = interleaved, 2 = contiguous per XCD).
    int sched_tasks_per_wave = 0;
    int sched_slices = 0;
    int sched_order = 0;
    int sched_xcd = 0;
    int sched_occupancy = 0;  // 0 standard kernel, 6 the 6-waves-per-SIMD variant
    int sched_tiling = 0;     // 0 automatic, 1 power-of-two slots, 2 packed slots
    // Grow-only device buffers for the run order: keys, sorted keys, the
    // order itself and the sort's temporary storage.
    unsigned* d_run_keys = nullptr;
    unsigned* d_run_keys_sorted = nullptr;
    int* d_run_order = nullptr;
    long long run_cap = 0;
    // What d_run_order was computed for.  Any permutation of the runs gives
    // the same result, so an order reused for rewritten task contents only
    // costs speed; cwlb_ctx_set_locality forgets it.
    const void* order_tasks = nullptr;
    const void* order_origin = nullptr;
    long long order_n_tasks = -1;
    long long order_runs = -1;
    int order_M = 0;
    void* d_sort_temp = nullptr;
    size_t sort_temp_bytes = 0;
    // Set when a launch under graph capture used d_run_order (resp.
    // d_hints): the graph keeps that address, so a later rebuild moves the
    // buffer to `retired` (freed by cwlb_ctx_destroy) and builds into a new
    // one instead of rewriting or freeing it.
    bool order_captured = false;
    bool hints_captured = false;
    bool phases_captured = false;
    std::vector<void*> retired;
    // Cache-policy hints of the feature-row gathers (0 = off): the hot set
    // in bytes of feature rows, the per-column in-degrees, their histogram
    // and the per-nonzero cold bits, with what they were built for.
    long long sched_hot_bytes = 0;
    unsigned* d_col_counts = nullptr;
    long long col_count_cap = 0;
    unsigned* d_count_hist = nullptr;
    unsigned long long* d_hints = nullptr;
    long long hint_cap = 0;
    const void* hint_col = nullptr;
    long long hint_nnz = -1;
    long long hint_h_rows = -1;
    long long hint_hot_rows = -1;
    unsigned hint_theta = 0;
    bool hint_any_cold = false;
    bool last_call_hinted = false;  // the last aggregation launch used hints
    bool last_call_packed = false;  // the last aggregation launch used packed slots
    // Column phases (0 or 1 = none): grow-only buffers that each phased call
    // rewrites -- the P - 1 interior row bounds (P - 1 arrays of n_rows
    // ints) and the band-sorted copy of the column and value arrays -- and
    // the sequence number of the last phased call.
    int sched_phases = 0;
    int* d_phase_bounds = nullptr;
    long long phase_cap = 0;
    int* d_band_col = nullptr;
    long long band_cap_col = 0;
    float* d_band_val = nullptr;
    long long band_cap_val = 0;
    int phase_seq = 0;
    cwlb_launch_info last_launch{};  // the last aggregation launch's schedule
    // Pinned host staging of the host-pointer entry point: two buffers used
    // alternately, each with the event of the last transfer through it.
    void* h_stage[2] = {nullptr, nullptr};
    hipEvent_t stage_ev[2] = {nullptr, nullptr};
};

namespace cwlb {

// Thread-local last-error message.
void set_error(const std::string& msg);
cwlb_status fail(cwlb_status st, const std::string& msg);
cwlb_status hip_fail(hipError_t e, const char* what);

#define CWLB_HIP_TRY(expr)                                   \
    do {                                                     \
        hipError_t e_ = (expr);                              \
        if (e_ != hipSuccess) return ::cwlb::hip_fail(e_, #expr); \
    } while (0)

// Checks the launch just enqueued, naming it in the error message.
#define CWLB_LAUNCH_CHECK(name)                                                    \
    do {                                                                           \
        hipError_t e_ = hipGetLastError();                                         \
        if (e_ != hipSuccess) return ::cwlb::hip_fail(e_, "launch of " name);      \
    } while (0)

// Scoped device switch.
struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev)
    {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard()
    {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

struct SpmmArgs {
    const int32_t* row_ptr;
    const int32_t* col_idx;
    const float* val;
    const int32_t* origin;
    int32_t n_rows;
    int64_t nnz;
    const float* H;
    int64_t h_rows;
    int32_t K;
    const cwlb_task* tasks;
    int64_t n_tasks;
    float* C;
};

// Every flag bit the aggregation entry points take; others are rejected.
constexpr uint32_t kSpmmFlags =
    CWLB_SPMM_ZERO_OUTPUT | CWLB_SPMM_PER_TASK | CWLB_SPMM_KEEP_EMPTY_ROWS;

// Enqueues the split-row clearing pass (or the full clear when zero_all)
// and the aggregation kernel on ctx->stream, bracketed by ctx->ev[0..2].
// per_task runs one task per wave (no task-run fusion, no feature slices).
// Rows without nonzeros are stored as zeros unless zero_all or keep_empty
// (the caller's C holds zeros there already).
cwlb_status launch_spmm_mean(cwlb_ctx* ctx, const SpmmArgs& a, bool zero_all, bool per_task,
                             bool keep_empty, bool record_events);

// Computes into ctx->d_run_order a permutation of the n_runs runs (runs of
// M tasks) sorted by the original id of each run's first row, on
// ctx->stream, unless the order of the same task array, origin array, task
// count and run length is already there; *order receives ctx->d_run_order.
// With may_build false (a stream under graph capture) nothing is computed:
// *order is the kept order when it matches, else null (task order).
cwlb_status build_run_order(cwlb_ctx* ctx, const SpmmArgs& a, int M, long long n_runs,
                            bool may_build, const int** order);

// The GPU partition (csrc/partition.hip): row_ptr and out are device
// arrays; synchronises.
cwlb_status launch_partition(cwlb_ctx* ctx, const int32_t* row_ptr, int32_t n_rows,
                             const cwlb_cost_params* costs, double capacity_weight,
                             cwlb_task* out, int64_t capacity_tasks, int64_t* n_tasks);

cwlb_status launch_fill_features(cwlb_ctx* ctx, float* H, int64_t rows, int32_t K, uint64_t seed);

// Builds (or reuses) the per-nonzero cold-column bits for a hot set of
// hot_rows feature rows (csrc/col_hints.hip); synchronises when it builds.
// *hints is null when no column is cold, and when the bits would have to be
// built but may_build is false (a stream under graph capture).
cwlb_status build_cache_hints(cwlb_ctx* ctx, const SpmmArgs& a, long long hot_rows,
                              bool may_build, const unsigned long long** hints);

// The context buffers of a column-phased call.
struct PhaseArrays {
    int32_t* bounds = nullptr;  // (P - 1) x n_rows
    int32_t* col = nullptr;     // nnz, each row's nonzeros sorted by band
    float* val = nullptr;       // nnz, likewise
};

// Sizes the context's phase buffers for `phases` column phases
// (csrc/col_phases.hip); all null when they cannot be used (a stream under
// graph capture, where nothing is allocated, and buffers too small).
cwlb_status prepare_column_phases(cwlb_ctx* ctx, const SpmmArgs& a, int phases, bool may_build,
                                  PhaseArrays* out);

// Enqueues the band sort: bounds[(p - 1) * n_rows + r] for p in [1, phases)
// (bounds may be null) and, when col_out is non-null, the band-sorted copy
// of col_idx and val.  A non-null chain_word (the aggregation's status[1])
// is cleared by the same launch.
cwlb_status launch_band_sort(hipStream_t st, const int32_t* row_ptr, const int32_t* col_idx,
                             const float* val, int32_t n_rows, int64_t nnz, int64_t h_rows,
                             int phases, int32_t* bounds, int32_t* col_out, float* val_out,
                             int32_t* chain_word = nullptr);

cwlb_status launch_reorder(cwlb_ctx* ctx, int32_t n_rows, int64_t nnz, const int32_t* row_ptr,
                           const int32_t* col_idx, const float* val, int32_t* origin,
                           int32_t* row_ptr_out, int32_t* col_idx_out, float* val_out);

cwlb_status run_calibration(cwlb_ctx* ctx, int32_t K, int32_t repeat, int32_t WI, int32_t load_MB,
                            int32_t atomic_writers, cwlb_cost_params* out,
                            cwlb_calibration_report* report);

}  // namespace cwlb
