// C ABI of libcwlb: contexts, errors and the SpMM entry points.
#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "host_threads.h"
#include "internal.h"

namespace cwlb {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }

cwlb_status fail(cwlb_status st, const std::string& msg)
{
    set_error(msg);
    return st;
}

cwlb_status hip_fail(hipError_t e, const char* what)
{
    set_error(std::string(what) + ": " + hipGetErrorString(e));
    return e == hipErrorOutOfMemory ? CWLB_OOM : CWLB_HIP_ERROR;
}

namespace {

cwlb_status check_spmm_args(cwlb_ctx* ctx, const SpmmArgs& a)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "spmm: null context");
    if (a.n_rows < 0 || a.nnz < 0 || a.K < 0 || a.n_tasks < 0 || a.h_rows < 0)
        return fail(CWLB_INVALID_ARG, "spmm: negative size");
    if (a.nnz > INT32_MAX) return fail(CWLB_INVALID_ARG, "spmm: nnz must fit int32");
    const bool work = a.K > 0 && a.n_tasks > 0;
    if (work) {
        if (!a.row_ptr || !a.origin || !a.tasks || !a.C)
            return fail(CWLB_INVALID_ARG, "spmm: null device pointer");
        if (a.nnz > 0 && (!a.col_idx || !a.val || !a.H))
            return fail(CWLB_INVALID_ARG, "spmm: null device pointer");
    }
    if (a.n_rows > 0 && a.K > 0 && !a.C) return fail(CWLB_INVALID_ARG, "spmm: null C");
    return CWLB_OK;
}

// Entry points that allocate, read results back or synchronise cannot be
// recorded into a graph: on a stream under capture they return
// CWLB_UNSUPPORTED before enqueueing anything, so the capture stays valid.
cwlb_status refuse_under_capture(hipStream_t st, const char* what)
{
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    CWLB_HIP_TRY(hipStreamIsCapturing(st, &capture));
    if (capture != hipStreamCaptureStatusNone)
        return fail(CWLB_UNSUPPORTED, std::string(what) +
                                          ": not available on a stream under graph capture "
                                          "(it allocates and synchronises)");
    return CWLB_OK;
}

// Reads the status word the last aggregation left (the stream must be idle).
cwlb_status read_status(cwlb_ctx* ctx)
{
    int st = 0;
    CWLB_HIP_TRY(hipMemcpyAsync(&st, ctx->d_status, sizeof(int), hipMemcpyDeviceToHost, ctx->stream));
    CWLB_HIP_TRY(hipStreamSynchronize(ctx->stream));
    if (st & 1) return fail(CWLB_INVALID_ARG, "spmm: a column index is outside [0, h_rows)");
    if (st & 2) return fail(CWLB_INVALID_ARG, "spmm: an origin entry is outside [0, n_rows)");
    if (st & 4)
        return fail(CWLB_INVALID_ARG, "spmm: a row's offsets leave [0, nnz] or decrease (row_ptr)");
    return CWLB_OK;
}

cwlb_status finish_timed(cwlb_ctx* ctx, cwlb_timing* timing)
{
    CWLB_HIP_TRY(hipEventSynchronize(ctx->ev[2]));
    float z = 0.0f, m = 0.0f;
    CWLB_HIP_TRY(hipEventElapsedTime(&z, ctx->ev[0], ctx->ev[1]));
    CWLB_HIP_TRY(hipEventElapsedTime(&m, ctx->ev[1], ctx->ev[2]));
    timing->zero_us = z * 1000.0f;
    timing->main_us = m * 1000.0f;
    timing->total_us = (z + m) * 1000.0f;
    return read_status(ctx);
}

cwlb_status run_spmm(cwlb_ctx* ctx, const SpmmArgs& a, uint32_t flags, cwlb_timing* timing)
{
    if (flags & ~kSpmmFlags) return fail(CWLB_INVALID_ARG, "spmm: unknown flag bits");
    cwlb_status st = check_spmm_args(ctx, a);
    if (st != CWLB_OK) return st;
    DeviceGuard g(ctx->device);
    const bool zero_all = (flags & CWLB_SPMM_ZERO_OUTPUT) != 0;
    const bool per_task = (flags & CWLB_SPMM_PER_TASK) != 0;
    const bool keep_empty = (flags & CWLB_SPMM_KEEP_EMPTY_ROWS) != 0;
    if (a.K == 0 || a.n_tasks == 0) {
        // The reference returns a zero matrix and time 0 (parallelMatrix.cpp:80-83, 101-104).
        if (zero_all && a.n_rows > 0 && a.K > 0) {
            st = launch_spmm_mean(ctx, a, true, per_task, keep_empty, false);
            if (st != CWLB_OK) return st;
        }
        if (timing) {
            CWLB_HIP_TRY(hipStreamSynchronize(ctx->stream));
            *timing = cwlb_timing{0.0f, 0.0f, 0.0f};
        }
        return CWLB_OK;
    }
    st = launch_spmm_mean(ctx, a, zero_all, per_task, keep_empty, timing != nullptr);
    if (st != CWLB_OK) return st;
    if (timing) return finish_timed(ctx, timing);
    return CWLB_OK;
}

// Host-pointer transfers through the context's two pinned staging buffers:
// while the DMA engine moves one buffer, the host threads fill (or drain)
// the other.
constexpr size_t kStageBytes = size_t{64} << 20;

// True when both staging buffers and their events exist (allocated at the
// first call).  Without them (pinned memory refused) the caller copies
// directly from its pageable arrays.
bool ensure_staging(cwlb_ctx* ctx)
{
    for (int b = 0; b < 2; ++b) {
        if (!ctx->h_stage[b] &&
            hipHostMalloc(&ctx->h_stage[b], kStageBytes, hipHostMallocDefault) != hipSuccess) {
            ctx->h_stage[b] = nullptr;
            (void)hipGetLastError();
            return false;
        }
        if (!ctx->stage_ev[b]) {
            if (hipEventCreateWithFlags(&ctx->stage_ev[b], hipEventDisableTiming) != hipSuccess ||
                hipEventRecord(ctx->stage_ev[b], ctx->stream) != hipSuccess) {
                if (ctx->stage_ev[b]) (void)hipEventDestroy(ctx->stage_ev[b]);
                ctx->stage_ev[b] = nullptr;
                (void)hipGetLastError();
                return false;
            }
        }
    }
    return true;
}

struct Stager {
    cwlb_ctx* ctx;
    bool direct;        // no pinned buffers: plain (pageable) copies
    unsigned next = 0;  // staging buffer of the next chunk

    cwlb_status to_device(void* d_dst, const void* h_src, size_t bytes)
    {
        if (direct) {
            if (bytes)
                CWLB_HIP_TRY(hipMemcpyAsync(d_dst, h_src, bytes, hipMemcpyHostToDevice,
                                            ctx->stream));
            return CWLB_OK;
        }
        for (size_t off = 0; off < bytes; off += kStageBytes) {
            const size_t n = std::min(kStageBytes, bytes - off);
            const unsigned b = next++ & 1u;
            CWLB_HIP_TRY(hipEventSynchronize(ctx->stage_ev[b]));  // its last DMA is done
            parallel_copy(ctx->h_stage[b], static_cast<const char*>(h_src) + off, n);
            CWLB_HIP_TRY(hipMemcpyAsync(static_cast<char*>(d_dst) + off, ctx->h_stage[b], n,
                                        hipMemcpyHostToDevice, ctx->stream));
            CWLB_HIP_TRY(hipEventRecord(ctx->stage_ev[b], ctx->stream));
        }
        return CWLB_OK;
    }

    cwlb_status to_host(void* h_dst, const void* d_src, size_t bytes)
    {
        if (direct) {
            if (bytes)
                CWLB_HIP_TRY(hipMemcpyAsync(h_dst, d_src, bytes, hipMemcpyDeviceToHost,
                                            ctx->stream));
            return CWLB_OK;
        }
        size_t prev_off = 0, prev_n = 0;
        unsigned prev_b = 0;
        bool pending = false;
        for (size_t off = 0; off < bytes; off += kStageBytes) {
            const size_t n = std::min(kStageBytes, bytes - off);
            const unsigned b = next++ & 1u;
            // Buffer b was drained (or only read by a finished upload).
            CWLB_HIP_TRY(hipEventSynchronize(ctx->stage_ev[b]));
            CWLB_HIP_TRY(hipMemcpyAsync(ctx->h_stage[b], static_cast<const char*>(d_src) + off,
                                        n, hipMemcpyDeviceToHost, ctx->stream));
            CWLB_HIP_TRY(hipEventRecord(ctx->stage_ev[b], ctx->stream));
            if (pending) {
                CWLB_HIP_TRY(hipEventSynchronize(ctx->stage_ev[prev_b]));
                parallel_copy(static_cast<char*>(h_dst) + prev_off, ctx->h_stage[prev_b], prev_n);
            }
            prev_off = off;
            prev_n = n;
            prev_b = b;
            pending = true;
        }
        if (pending) {
            CWLB_HIP_TRY(hipEventSynchronize(ctx->stage_ev[prev_b]));
            parallel_copy(static_cast<char*>(h_dst) + prev_off, ctx->h_stage[prev_b], prev_n);
        }
        return CWLB_OK;
    }
};

// Whether the tasks tile the nonzeros in order: every task well formed and
// each starting exactly where the previous one ended (the rule by which the
// aggregation kernel merges consecutive tasks).  Such a list covers each
// nonzero at most once.
bool tasks_tile(const cwlb_task* t, int64_t n, int32_t n_rows)
{
    auto well_formed = [n_rows](const cwlb_task& x) {
        return x.row_start >= 0 && x.row_start < x.row_end && x.row_end <= n_rows &&
               x.first_row_offset >= 0 && x.last_row_nnz >= 0 &&
               (x.row_end - x.row_start > 1 || x.last_row_nnz == 0 ||
                x.first_row_offset < x.last_row_nnz);
    };
    for (int64_t i = 0; i < n; ++i) {
        if (!well_formed(t[i])) return false;
        if (i == 0) continue;
        const cwlb_task& a = t[i - 1];
        const cwlb_task& b = t[i];
        const bool cont = a.last_row_nnz == 0
                              ? (b.row_start == a.row_end && b.first_row_offset == 0)
                              : (b.row_start == a.row_end - 1 &&
                                 b.first_row_offset == a.last_row_nnz);
        if (!cont) return false;
    }
    return true;
}

template <class T>
struct DevBuf {
    T* p = nullptr;
    DevBuf() = default;
    DevBuf(const DevBuf&) = delete;
    DevBuf& operator=(const DevBuf&) = delete;
    ~DevBuf()
    {
        if (p) (void)hipFree(p);
    }
    hipError_t alloc(size_t n) { return hipMalloc(reinterpret_cast<void**>(&p), sizeof(T) * (n ? n : 1)); }
};

}  // namespace
}  // namespace cwlb

using namespace cwlb;

extern "C" {

const char* cwlb_version(void) { return CWLB_VERSION_STRING " (gfx950)"; }

const char* cwlb_last_error(void) { return g_last_error.c_str(); }

cwlb_status cwlb_ctx_create(int device, void* stream, cwlb_ctx** out)
{
    if (!out) return fail(CWLB_INVALID_ARG, "cwlb_ctx_create: null out");
    *out = nullptr;
    int count = 0;
    CWLB_HIP_TRY(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) return fail(CWLB_INVALID_ARG, "cwlb_ctx_create: bad device id");
    DeviceGuard g(device);
    hipDeviceProp_t prop;
    CWLB_HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(CWLB_UNSUPPORTED, std::string("cwlb: built for gfx950 only, device is ") +
                                          prop.gcnArchName);
    auto* c = new (std::nothrow) cwlb_ctx();
    if (!c) return fail(CWLB_OOM, "cwlb_ctx_create: out of memory");
    c->device = device;
    c->stream = static_cast<hipStream_t>(stream);
    c->compute_units = prop.multiProcessorCount;
    c->max_wg = prop.maxThreadsPerBlock;
    c->wave = prop.warpSize;
    c->lds_per_block = prop.sharedMemPerBlock;
    c->total_mem = prop.totalGlobalMem;
    std::snprintf(c->name, sizeof c->name, "%s", prop.name[0] ? prop.name : prop.gcnArchName);
    std::snprintf(c->arch, sizeof c->arch, "%s", prop.gcnArchName);
    hipError_t e = hipSuccess;
    for (auto& ev : c->ev)
        if (e == hipSuccess) e = hipEventCreate(&ev);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&c->switch_ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&c->d_status), 2 * sizeof(int));
    if (e == hipSuccess) e = hipMemset(c->d_status, 0, 2 * sizeof(int));
    if (e != hipSuccess) {
        cwlb_ctx_destroy(c);
        return hip_fail(e, "cwlb_ctx_create");
    }
    *out = c;
    return CWLB_OK;
}

cwlb_status cwlb_ctx_destroy(cwlb_ctx* ctx)
{
    if (!ctx) return CWLB_OK;
    DeviceGuard g(ctx->device);
    for (auto& ev : ctx->ev)
        if (ev) (void)hipEventDestroy(ev);
    if (ctx->switch_ev) (void)hipEventDestroy(ctx->switch_ev);
    if (ctx->d_status) (void)hipFree(ctx->d_status);
    for (void* p : {static_cast<void*>(ctx->d_run_keys), static_cast<void*>(ctx->d_run_keys_sorted),
                    static_cast<void*>(ctx->d_run_order), ctx->d_sort_temp,
                    static_cast<void*>(ctx->d_col_counts), static_cast<void*>(ctx->d_count_hist),
                    static_cast<void*>(ctx->d_hints), static_cast<void*>(ctx->d_phase_bounds),
                    static_cast<void*>(ctx->d_band_col), static_cast<void*>(ctx->d_band_val)})
        if (p) (void)hipFree(p);
    for (void* p : ctx->retired) (void)hipFree(p);
    for (int b = 0; b < 2; ++b) {
        if (ctx->stage_ev[b]) (void)hipEventSynchronize(ctx->stage_ev[b]);
        if (ctx->stage_ev[b]) (void)hipEventDestroy(ctx->stage_ev[b]);
        if (ctx->h_stage[b]) (void)hipHostFree(ctx->h_stage[b]);
    }
    delete ctx;
    return CWLB_OK;
}

cwlb_status cwlb_ctx_set_stream(cwlb_ctx* ctx, void* stream)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    const auto next = static_cast<hipStream_t>(stream);
    if (next != ctx->stream) {
        // Calls on the old stream may still read or rewrite the context's
        // own buffers (status words, column-phase bounds, the band-sorted
        // copy); the new stream waits for everything enqueued on the old
        // one so far, so a call on it cannot overwrite them under a call
        // still running there.  Skipped when either stream is under graph
        // capture: a wait on a captured event would pull the other stream
        // into the capture (ordering against a graph is the caller's).
        DeviceGuard g(ctx->device);
        hipStreamCaptureStatus old_cap = hipStreamCaptureStatusNone;
        hipStreamCaptureStatus new_cap = hipStreamCaptureStatusNone;
        const bool known = hipStreamIsCapturing(ctx->stream, &old_cap) == hipSuccess &&
                           hipStreamIsCapturing(next, &new_cap) == hipSuccess;
        (void)hipGetLastError();  // a refused query (legacy stream during a capture) is not kept
        if (known && old_cap == hipStreamCaptureStatusNone &&
            new_cap == hipStreamCaptureStatusNone) {
            CWLB_HIP_TRY(hipEventRecord(ctx->switch_ev, ctx->stream));
            CWLB_HIP_TRY(hipStreamWaitEvent(next, ctx->switch_ev, 0));
        }
    }
    ctx->stream = next;
    return CWLB_OK;
}

cwlb_status cwlb_ctx_synchronize(cwlb_ctx* ctx)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    DeviceGuard g(ctx->device);
    CWLB_HIP_TRY(hipStreamSynchronize(ctx->stream));
    return read_status(ctx);
}

cwlb_status cwlb_ctx_device_info(cwlb_ctx* ctx, cwlb_device_info* out)
{
    if (!ctx || !out) return fail(CWLB_INVALID_ARG, "null argument");
    out->device = ctx->device;
    out->compute_units = ctx->compute_units;
    out->max_work_group_size = ctx->max_wg;
    out->wavefront_size = ctx->wave;
    out->lds_bytes_per_block = static_cast<int64_t>(ctx->lds_per_block);
    out->total_global_mem = static_cast<int64_t>(ctx->total_mem);
    std::snprintf(out->name, sizeof out->name, "%s", ctx->name);
    std::snprintf(out->arch, sizeof out->arch, "%s", ctx->arch);
    return CWLB_OK;
}

cwlb_status cwlb_ctx_set_schedule(cwlb_ctx* ctx, int32_t tasks_per_wave, int32_t feature_slices)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    if (tasks_per_wave < 0 || tasks_per_wave > (1 << 20))
        return fail(CWLB_INVALID_ARG,
                    "tasks_per_wave must be in [0, 1048576] (0 = automatic)");
    if (feature_slices != 0 && feature_slices != 1 && feature_slices != 2 && feature_slices != 4 &&
        feature_slices != 8)
        return fail(CWLB_INVALID_ARG, "feature_slices must be 0, 1, 2, 4 or 8");
    ctx->sched_tasks_per_wave = tasks_per_wave;
    ctx->sched_slices = feature_slices;
    return CWLB_OK;
}

cwlb_status cwlb_ctx_set_locality(cwlb_ctx* ctx, int32_t run_order, int32_t xcd_blocks)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    if (run_order < 0 || run_order > 2)
        return fail(CWLB_INVALID_ARG, "run_order must be 0 (automatic), 1 (task order) or 2 "
                                      "(by output row)");
    if (xcd_blocks < 0 || xcd_blocks > 2)
        return fail(CWLB_INVALID_ARG, "xcd_blocks must be 0 (automatic), 1 (interleaved) or 2 "
                                      "(contiguous)");
    ctx->sched_order = run_order;
    ctx->sched_xcd = xcd_blocks;
    ctx->order_runs = -1;  // recompute the run order at the next call
    return CWLB_OK;
}

cwlb_status cwlb_ctx_set_cache_hints(cwlb_ctx* ctx, int64_t hot_bytes)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    if (hot_bytes < 0) return fail(CWLB_INVALID_ARG, "hot_bytes must be >= 0 (0 = off)");
    ctx->sched_hot_bytes = hot_bytes;
    return CWLB_OK;
}

cwlb_status cwlb_ctx_get_cache_hints(cwlb_ctx* ctx, int64_t* hot_bytes)
{
    if (!ctx || !hot_bytes) return fail(CWLB_INVALID_ARG, "null argument");
    *hot_bytes = ctx->sched_hot_bytes;
    return CWLB_OK;
}

cwlb_status cwlb_ctx_set_occupancy(cwlb_ctx* ctx, int32_t waves_per_simd)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    if (waves_per_simd != 0 && waves_per_simd != 6)
        return fail(CWLB_INVALID_ARG, "waves_per_simd must be 0 (standard kernel) or 6");
    ctx->sched_occupancy = waves_per_simd;
    return CWLB_OK;
}

cwlb_status cwlb_ctx_get_occupancy(cwlb_ctx* ctx, int32_t* waves_per_simd)
{
    if (!ctx || !waves_per_simd) return fail(CWLB_INVALID_ARG, "null argument");
    *waves_per_simd = ctx->sched_occupancy;
    return CWLB_OK;
}

cwlb_status cwlb_ctx_set_lane_tiling(cwlb_ctx* ctx, int32_t tiling)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    if (tiling < 0 || tiling > 2)
        return fail(CWLB_INVALID_ARG, "tiling must be 0 (automatic), 1 (power-of-two slots) or 2 (packed)");
    ctx->sched_tiling = tiling;
    return CWLB_OK;
}

cwlb_status cwlb_ctx_get_lane_tiling(cwlb_ctx* ctx, int32_t* tiling)
{
    if (!ctx || !tiling) return fail(CWLB_INVALID_ARG, "null argument");
    *tiling = ctx->sched_tiling;
    return CWLB_OK;
}

cwlb_status cwlb_ctx_set_column_phases(cwlb_ctx* ctx, int32_t phases)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    if (phases < 0 || phases > 64)
        return fail(CWLB_INVALID_ARG, "phases must be in [0, 64] (0 or 1 = off)");
    ctx->sched_phases = phases;
    return CWLB_OK;
}

cwlb_status cwlb_ctx_get_column_phases(cwlb_ctx* ctx, int32_t* phases)
{
    if (!ctx || !phases) return fail(CWLB_INVALID_ARG, "null argument");
    *phases = ctx->sched_phases;
    return CWLB_OK;
}

cwlb_status cwlb_column_phase_sort(cwlb_ctx* ctx, const int32_t* row_ptr,
                                   const int32_t* col_idx, const float* val, int32_t n_rows,
                                   int64_t nnz, int64_t h_rows, int32_t phases,
                                   int32_t* bounds_out, int32_t* col_out, float* val_out)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    if (phases < 2 || phases > 64)
        return fail(CWLB_INVALID_ARG, "cwlb_column_phase_sort: phases must be in [2, 64]");
    if (n_rows < 0 || nnz < 0 || nnz > INT32_MAX || h_rows <= 0)
        return fail(CWLB_INVALID_ARG, "cwlb_column_phase_sort: n_rows >= 0, 0 <= nnz < 2^31 "
                                      "and h_rows > 0 required");
    if (!col_out != !val_out)
        return fail(CWLB_INVALID_ARG,
                    "cwlb_column_phase_sort: col_out and val_out go together");
    if (n_rows > 0 && (!row_ptr || (nnz > 0 && (!col_idx || (col_out && !val)))))
        return fail(CWLB_INVALID_ARG, "cwlb_column_phase_sort: null array");
    DeviceGuard g(ctx->device);
    (void)hipGetLastError();
    return launch_band_sort(ctx->stream, row_ptr, col_idx, val, n_rows, nnz, h_rows, phases,
                            bounds_out, col_out, val_out);
}

cwlb_status cwlb_ctx_last_launch(cwlb_ctx* ctx, cwlb_launch_info* out)
{
    if (!ctx || !out) return fail(CWLB_INVALID_ARG, "null argument");
    *out = ctx->last_launch;
    return CWLB_OK;
}

cwlb_status cwlb_spmm_mean_f32(cwlb_ctx* ctx, const int32_t* row_ptr, const int32_t* col_idx,
                               const float* val, const int32_t* origin, int32_t n_rows,
                               int64_t nnz, const float* H, int64_t h_rows, int32_t K,
                               const cwlb_task* tasks, int64_t n_tasks, float* C,
                               uint32_t flags, cwlb_timing* timing)
{
    if (ctx && K > ctx->max_wg)
        return fail(CWLB_INVALID_ARG,
                    "spmmKernel supports only K <= device max work-group size; "
                    "use spmmKernelLargeKFallback for larger K.");
    SpmmArgs a{row_ptr, col_idx, val, origin, n_rows, nnz, H, h_rows, K, tasks, n_tasks, C};
    return run_spmm(ctx, a, flags, timing);
}

cwlb_status cwlb_ctx_tune_schedule(cwlb_ctx* ctx, const int32_t* row_ptr, const int32_t* col_idx,
                                   const float* val, const int32_t* origin, int32_t n_rows,
                                   int64_t nnz, const float* H, int64_t h_rows, int32_t K,
                                   const cwlb_task* tasks, int64_t n_tasks, float* C,
                                   int32_t trials, int32_t* tasks_per_wave_out,
                                   int32_t* feature_slices_out, int32_t* locality_out)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    if (trials <= 0) return fail(CWLB_INVALID_ARG, "cwlb_ctx_tune_schedule: trials must be positive");
    SpmmArgs a{row_ptr, col_idx, val, origin, n_rows, nnz, H, h_rows, K, tasks, n_tasks, C};
    cwlb_status st = check_spmm_args(ctx, a);
    if (st != CWLB_OK) return st;
    {
        DeviceGuard g(ctx->device);
        st = refuse_under_capture(ctx->stream, "cwlb_ctx_tune_schedule");
        if (st != CWLB_OK) return st;
    }
    // Candidates: the automatic choice, then every run length and slice
    // count the kernel takes for this K.
    std::vector<std::pair<int, int>> cands{{0, 0}};
    for (int sl : {1, 2, 4, 8})
        if (sl == 1 || (K % 4 == 0 && K / sl >= 32))
            for (int m : {2, 4, 8, 16, 32, 64}) cands.emplace_back(m, sl);
    const int keep_m = ctx->sched_tasks_per_wave, keep_sl = ctx->sched_slices;
    // Tuning the hints and the occupancy variant too: the schedule and
    // placement are chosen without them.
    const long long keep_hot = ctx->sched_hot_bytes;
    const int keep_occ = ctx->sched_occupancy;
    const int keep_phases = ctx->sched_phases;
    const int keep_tiling = ctx->sched_tiling;
    if (locality_out) {
        ctx->sched_hot_bytes = 0;
        ctx->sched_occupancy = 0;
        ctx->sched_phases = 0;
        ctx->sched_tiling = 0;
    }
    float best_us = 0.0f;
    std::pair<int, int> best{0, 0};
    std::vector<float> times(static_cast<size_t>(trials));
    // One warm-up, then the median of `trials` event-timed calls under the
    // context's current settings.  The warm-up builds what the settings
    // need (run order, hints); `applies` (optional) reads the warm-up's
    // launch and skips the timing when it returns false.  A first timed
    // call above `cutoff` (> 0) ends the timing: that call's time is
    // returned, and a candidate 10% behind the best cannot win on noise.
    auto time_current = [&](float* med, bool (*applies)(const cwlb_ctx*),
                            float cutoff) -> cwlb_status {
        cwlb_status s = run_spmm(ctx, a, 0, nullptr);
        if (s != CWLB_OK) return s;
        if (applies && !applies(ctx)) {
            *med = 0.0f;
            return CWLB_OK;
        }
        for (int t = 0; t < trials; ++t) {
            cwlb_timing tm{};
            s = run_spmm(ctx, a, 0, &tm);
            if (s != CWLB_OK) return s;
            if (t == 0 && cutoff > 0.0f && tm.total_us > cutoff) {
                *med = tm.total_us;
                return CWLB_OK;
            }
            times[static_cast<size_t>(t)] = tm.total_us;
        }
        std::sort(times.begin(), times.end());
        *med = times[times.size() / 2];
        return CWLB_OK;
    };
    auto restore = [&](int order, int xcd) {
        ctx->sched_tasks_per_wave = keep_m;
        ctx->sched_slices = keep_sl;
        ctx->sched_order = order;
        ctx->sched_xcd = xcd;
        ctx->order_runs = -1;
        ctx->sched_hot_bytes = keep_hot;
        ctx->sched_occupancy = keep_occ;
        ctx->sched_phases = keep_phases;
        ctx->sched_tiling = keep_tiling;
    };
    const int keep_order = ctx->sched_order, keep_xcd = ctx->sched_xcd;
    for (const auto& c : cands) {
        ctx->sched_tasks_per_wave = c.first;
        ctx->sched_slices = c.second;
        float med = 0.0f;
        st = time_current(&med, nullptr, best_us * 1.1f);
        if (st != CWLB_OK) {
            restore(keep_order, keep_xcd);
            return st;
        }
        if (best_us == 0.0f || med < best_us) {
            best_us = med;
            best = c;
        }
    }
    ctx->sched_tasks_per_wave = best.first;
    ctx->sched_slices = best.second;
    if (locality_out) {
        // Locality placements for the best schedule: the context's own, and
        // runs sorted by output row with interleaved or contiguous XCD
        // stretches.  The three are timed afresh, in two interleaved rounds
        // (the best of each kept): two placements within a few percent of
        // each other (the mesh's) are otherwise decided by clock drift, and
        // the first stage's minimum over many candidates is biased low.
        int best_order = keep_order, best_xcd = keep_xcd;
        {
            const std::pair<int, int> locs[3] = {{keep_order, keep_xcd}, {2, 1}, {2, 2}};
            float loc_us[3] = {0.0f, 0.0f, 0.0f};
            for (int round = 0; round < 2 && st == CWLB_OK; ++round) {
                for (int i = 0; i < 3 && st == CWLB_OK; ++i) {
                    ctx->sched_order = locs[i].first;
                    ctx->sched_xcd = locs[i].second;
                    float med = 0.0f;
                    st = time_current(&med, nullptr, 0.0f);
                    if (st == CWLB_OK && (loc_us[i] == 0.0f || med < loc_us[i])) loc_us[i] = med;
                }
            }
            if (st != CWLB_OK) {
                restore(keep_order, keep_xcd);
                return st;
            }
            int k = 0;
            for (int i = 1; i < 3; ++i)
                if (loc_us[i] < loc_us[k]) k = i;
            best_order = locs[k].first;
            best_xcd = locs[k].second;
            best_us = loc_us[k];
        }
        ctx->sched_order = best_order;
        ctx->sched_xcd = best_xcd;
        ctx->order_runs = -1;
        locality_out[0] = best_order;
        locality_out[1] = best_xcd;
        // Then, one at a time, the occupancy variant and the cache hints
        // (hot sets of 24, 48 and 96 MB of feature rows; the hints are built
        // once per size and kept), each kept when faster than the current
        // settings.  The current settings are re-timed before each: the
        // minimum over many candidates above is biased low against a single
        // fresh timing.
        float base = 0.0f;
        const int m_standard = best.first;
        st = time_current(&base, nullptr, 0.0f);
        if (st == CWLB_OK) {
            ctx->sched_occupancy = 6;
            float med = 0.0f;
            st = time_current(&med, [](const cwlb_ctx* c) {
                return c->last_launch.waves_per_simd == 6;
            }, 0.0f);
            if (st == CWLB_OK && !(med > 0.0f && med < base)) ctx->sched_occupancy = 0;
            if (st == CWLB_OK && ctx->sched_occupancy == 6) {
                // More waves in flight can move the best run length: its
                // neighbours (half and double) under the variant.
                base = med;
                const int m0 = best.first;
                for (int m : {m0 / 2, m0 * 2}) {
                    if (st != CWLB_OK || m0 == 0 || m < 1 || m > 64) continue;
                    ctx->sched_tasks_per_wave = m;
                    st = time_current(&med, nullptr, 0.0f);
                    if (st == CWLB_OK && med < base) {
                        base = med;
                        best.first = m;
                    }
                }
                ctx->sched_tasks_per_wave = best.first;
            }
        }
        if (st == CWLB_OK) st = time_current(&base, nullptr, 0.0f);
        long long best_hot = 0;
        for (long long mb : {24ll, 48ll, 96ll}) {
            if (st != CWLB_OK) break;
            ctx->sched_hot_bytes = mb << 20;
            float med = 0.0f;
            // Hints that do not apply to this call (K, alignment, H size) or
            // mark no column cold leave nothing to time.
            st = time_current(&med, [](const cwlb_ctx* c) { return c->last_call_hinted; }, 0.0f);
            if (st != CWLB_OK || med == 0.0f) break;
            if (med < base) {
                base = med;
                best_hot = mb << 20;
            }
        }
        ctx->sched_hot_bytes = best_hot;
        if (st == CWLB_OK && ctx->sched_occupancy == 6) {
            // The variant was chosen without hints: with the chosen hints
            // the standard kernel (at its own run length) can be faster.
            // Both are timed afresh, one after the other.
            const int m6 = best.first;
            if (best_hot) st = time_current(&base, nullptr, 0.0f);
            ctx->sched_occupancy = 0;
            ctx->sched_tasks_per_wave = m_standard;
            float med = 0.0f;
            if (st == CWLB_OK) st = time_current(&med, nullptr, 0.0f);
            if (st == CWLB_OK && med < base) {
                best.first = m_standard;
            } else {
                ctx->sched_occupancy = 6;
                ctx->sched_tasks_per_wave = m6;
            }
        }
        // Packed slots (cwlb_ctx_set_lane_tiling) under the settings so far,
        // where they change the tiling; kept when faster, re-timed first.
        if (st == CWLB_OK) {
            st = time_current(&base, nullptr, 0.0f);
            ctx->sched_tiling = 2;
            float med = 0.0f;
            if (st == CWLB_OK)
                st = time_current(&med, [](const cwlb_ctx* c) { return c->last_call_packed; }, 0.0f);
            if (st == CWLB_OK && med > 0.0f && med < base) base = med;
            else ctx->sched_tiling = 0;
        }
        // Column phases, where they can pay: H beyond the Infinity Cache
        // (>= 512 MB) and rows of 64 nonzeros or more on average (each
        // phase reads and writes C once).  8, 12 and 16 phases, each with
        // every slice count whose widest slice fits one vector per lane,
        // at 16, 32 and 64 tasks per wave, under the placement chosen above;
        // kept when faster than the settings so far, re-timed first.
        const long long h_bytes = h_rows * static_cast<long long>(K) * 4;
        if (st == CWLB_OK && h_bytes >= (512ll << 20) && nnz >= 64ll * n_rows && K % 4 == 0) {
            st = time_current(&base, nullptr, 0.0f);
            const long long hot_kept = ctx->sched_hot_bytes;
            const int occ_kept = ctx->sched_occupancy;
            const int tiling_kept = ctx->sched_tiling;
            int best_p = 0, best_pm = best.first, best_psl = best.second, best_pt = 0;
            ctx->sched_hot_bytes = 0;
            ctx->sched_occupancy = 0;
            for (int P : {8, 12, 16}) {
                for (int sl : {1, 2, 4, 8}) {
                    if (K / 4 < sl || (K / 4 + sl - 1) / sl > 64) continue;
                    for (int m : {16, 32, 64}) {
                        // Each with power-of-two slots, then packed slots
                        // where those differ.
                        for (int til : {0, 2}) {
                            if (st != CWLB_OK) break;
                            ctx->sched_phases = P;
                            ctx->sched_slices = sl;
                            ctx->sched_tasks_per_wave = m;
                            ctx->sched_tiling = til;
                            float med = 0.0f;
                            st = time_current(&med, til == 0 ? +[](const cwlb_ctx* c) {
                                return c->last_launch.column_phases > 1;
                            } : +[](const cwlb_ctx* c) {
                                return c->last_launch.column_phases > 1 && c->last_call_packed;
                            }, base * 1.1f);
                            if (st == CWLB_OK && med > 0.0f && med < base) {
                                base = med;
                                best_p = P;
                                best_pm = m;
                                best_psl = sl;
                                best_pt = til;
                            }
                        }
                    }
                }
            }
            ctx->sched_phases = best_p;
            if (best_p) {
                // The phased kernel takes neither hints nor the variant.
                best.first = best_pm;
                best.second = best_psl;
                ctx->sched_tiling = best_pt;
            } else {
                ctx->sched_hot_bytes = hot_kept;
                ctx->sched_occupancy = occ_kept;
                ctx->sched_tiling = tiling_kept;
            }
            ctx->sched_tasks_per_wave = best.first;
            ctx->sched_slices = best.second;
        }
        if (st != CWLB_OK) {
            restore(keep_order, keep_xcd);
            return st;
        }
    }
    if (tasks_per_wave_out) *tasks_per_wave_out = best.first;
    if (feature_slices_out) *feature_slices_out = best.second;
    return CWLB_OK;
}

cwlb_status cwlb_spmm_mean_f32_large_k(cwlb_ctx* ctx, const int32_t* row_ptr,
                                       const int32_t* col_idx, const float* val,
                                       const int32_t* origin, int32_t n_rows, int64_t nnz,
                                       const float* H, int64_t h_rows, int32_t K,
                                       const cwlb_task* tasks, int64_t n_tasks, float* C,
                                       uint32_t flags, cwlb_timing* timing)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    if (ctx->max_wg <= 0)
        return fail(CWLB_RUNTIME_ERROR,
                    "Large-K fallback cannot use a device with max_work_group_size=0.");
    if (K <= ctx->max_wg)
        return fail(CWLB_INVALID_ARG,
                    "spmmKernelLargeKFallback requires K > device max work-group size.");
    SpmmArgs a{row_ptr, col_idx, val, origin, n_rows, nnz, H, h_rows, K, tasks, n_tasks, C};
    return run_spmm(ctx, a, flags, timing);
}

cwlb_status cwlb_spmm_mean_f32_host(cwlb_ctx* ctx, const int32_t* row_ptr,
                                    const int32_t* col_idx, const float* val,
                                    const int32_t* origin, int32_t n_rows, int64_t nnz,
                                    const float* H, int64_t h_rows, int32_t K,
                                    const cwlb_task* tasks, int64_t n_tasks, float* C,
                                    cwlb_timing* timing)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    if (n_rows < 0 || nnz < 0 || K < 0 || n_tasks < 0 || h_rows < 0)
        return fail(CWLB_INVALID_ARG, "spmm: negative size");
    if (nnz > INT32_MAX) return fail(CWLB_INVALID_ARG, "spmm: nnz must fit int32");
    DeviceGuard g(ctx->device);
    const cwlb_status cs = refuse_under_capture(ctx->stream, "cwlb_spmm_mean_f32_host");
    if (cs != CWLB_OK) return cs;
    const size_t out_elems = static_cast<size_t>(n_rows) * static_cast<size_t>(K);
    if (K == 0 || n_tasks == 0) {
        if (out_elems) std::memset(C, 0, out_elems * sizeof(float));
        if (timing) *timing = cwlb_timing{0.0f, 0.0f, 0.0f};
        return CWLB_OK;
    }
    if (!row_ptr || !origin || !tasks || !C || (nnz > 0 && (!col_idx || !val || !H)))
        return fail(CWLB_INVALID_ARG, "spmm: null host pointer");
    // Host-side validation keeps every device access in bounds.
    if (row_ptr[0] < 0 || row_ptr[n_rows] > nnz)
        return fail(CWLB_INVALID_ARG, "spmm: row_ptr outside [0, nnz]");
    if (!offsets_nondecreasing(row_ptr, n_rows))
        return fail(CWLB_INVALID_ARG, "spmm: row_ptr is not non-decreasing");
    if (!columns_in_range(col_idx, nnz, h_rows))
        return fail(CWLB_INVALID_ARG, "spmm: column index outside [0, h_rows)");
    const bool staged = ensure_staging(ctx);
    DevBuf<int32_t> d_rp, d_ci, d_or;
    DevBuf<float> d_val, d_H, d_C;
    DevBuf<cwlb_task> d_t;
    CWLB_HIP_TRY(d_rp.alloc(static_cast<size_t>(n_rows) + 1));
    CWLB_HIP_TRY(d_ci.alloc(static_cast<size_t>(nnz)));
    CWLB_HIP_TRY(d_val.alloc(static_cast<size_t>(nnz)));
    CWLB_HIP_TRY(d_or.alloc(static_cast<size_t>(n_rows)));
    CWLB_HIP_TRY(d_H.alloc(static_cast<size_t>(h_rows) * K));
    CWLB_HIP_TRY(d_C.alloc(out_elems));
    CWLB_HIP_TRY(d_t.alloc(static_cast<size_t>(n_tasks)));
    hipStream_t st = ctx->stream;
    Stager io{ctx, !staged};
    cwlb_status s = io.to_device(d_rp.p, row_ptr, sizeof(int32_t) * (n_rows + 1));
    if (s == CWLB_OK) s = io.to_device(d_ci.p, col_idx, sizeof(int32_t) * nnz);
    if (s == CWLB_OK) s = io.to_device(d_val.p, val, sizeof(float) * nnz);
    if (s == CWLB_OK) s = io.to_device(d_or.p, origin, sizeof(int32_t) * n_rows);
    if (s == CWLB_OK) s = io.to_device(d_H.p, H, sizeof(float) * h_rows * K);
    if (s == CWLB_OK) s = io.to_device(d_t.p, tasks, sizeof(cwlb_task) * n_tasks);
    if (s != CWLB_OK) {
        (void)hipStreamSynchronize(st);  // no DMA may outlive the device buffers
        return s;
    }
    SpmmArgs a{d_rp.p, d_ci.p, d_val.p, d_or.p, n_rows, nnz, d_H.p, h_rows, K, d_t.p, n_tasks, d_C.p};
    cwlb_timing local{};
    // A list that does not tile in order may cover a nonzero twice; one
    // task per wave then keeps the reference's task-at-a-time result.
    const uint32_t flags =
        CWLB_SPMM_ZERO_OUTPUT | (tasks_tile(tasks, n_tasks, n_rows) ? 0u : CWLB_SPMM_PER_TASK);
    s = run_spmm(ctx, a, flags, &local);
    if (s == CWLB_OK) s = io.to_host(C, d_C.p, sizeof(float) * out_elems);
    if (s != CWLB_OK) {
        (void)hipStreamSynchronize(st);
        return s;
    }
    CWLB_HIP_TRY(hipStreamSynchronize(st));
    // The reference times the aggregation kernel only; C's clearing is the
    // host-side Zero() there.
    if (timing) *timing = cwlb_timing{0.0f, local.main_us, local.main_us};
    return CWLB_OK;
}

cwlb_status cwlb_reorder_by_degree_device(cwlb_ctx* ctx, int32_t n_rows, int64_t nnz,
                                          const int32_t* row_ptr, const int32_t* col_idx,
                                          const float* val, int32_t* origin,
                                          int32_t* row_ptr_out, int32_t* col_idx_out,
                                          float* val_out)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    if (n_rows < 0 || nnz < 0 || nnz > INT32_MAX)
        return fail(CWLB_INVALID_ARG, "reorder: bad sizes");
    DeviceGuard g(ctx->device);
    const cwlb_status cs = refuse_under_capture(ctx->stream, "cwlb_reorder_by_degree_device");
    if (cs != CWLB_OK) return cs;
    return launch_reorder(ctx, n_rows, nnz, row_ptr, col_idx, val, origin, row_ptr_out,
                          col_idx_out, val_out);
}

cwlb_status cwlb_partition_device(cwlb_ctx* ctx, const int32_t* row_ptr, int32_t n_rows,
                                  const cwlb_cost_params* costs, double capacity_weight,
                                  cwlb_task* out, int64_t capacity_tasks, int64_t* n_tasks)
{
    if (!ctx || !costs || !n_tasks) return fail(CWLB_INVALID_ARG, "cwlb_partition_device: null argument");
    if (n_rows > 0 && !row_ptr) return fail(CWLB_INVALID_ARG, "cwlb_partition_device: null row_ptr");
    if (capacity_tasks < 0) return fail(CWLB_INVALID_ARG, "cwlb_partition_device: negative capacity");
    DeviceGuard g(ctx->device);
    const cwlb_status cs = refuse_under_capture(ctx->stream, "cwlb_partition_device");
    if (cs != CWLB_OK) return cs;
    return launch_partition(ctx, row_ptr, n_rows, costs, capacity_weight, out, capacity_tasks,
                            n_tasks);
}

cwlb_status cwlb_calibrate_report(cwlb_ctx* ctx, int32_t K, int32_t repeat, int32_t WI,
                                  int32_t load_MB, int32_t atomic_writers, cwlb_cost_params* out,
                                  cwlb_calibration_report* report)
{
    if (!ctx || !out) return fail(CWLB_INVALID_ARG, "null argument");
    if (K <= 0 || repeat <= 0 || WI <= 0 || load_MB <= 0 || atomic_writers <= 0)
        return fail(CWLB_INVALID_ARG, "All microbenchmark parameters must be positive.");
    DeviceGuard g(ctx->device);
    const cwlb_status cs = refuse_under_capture(ctx->stream, "cwlb_calibrate");
    if (cs != CWLB_OK) return cs;
    return run_calibration(ctx, K, repeat, WI, load_MB, atomic_writers, out, report);
}

cwlb_status cwlb_calibrate(cwlb_ctx* ctx, int32_t K, int32_t repeat, int32_t WI, int32_t load_MB,
                           int32_t atomic_writers, cwlb_cost_params* out)
{
    return cwlb_calibrate_report(ctx, K, repeat, WI, load_MB, atomic_writers, out, nullptr);
}

cwlb_status cwlb_fill_features_uniform(cwlb_ctx* ctx, float* H, int64_t rows, int32_t K,
                                       uint64_t seed)
{
    if (!ctx) return fail(CWLB_INVALID_ARG, "null context");
    if (rows < 0 || K < 0) return fail(CWLB_INVALID_ARG, "negative size");
    if (rows * K > 0 && !H) return fail(CWLB_INVALID_ARG, "null H");
    DeviceGuard g(ctx->device);
    return launch_fill_features(ctx, H, rows, K, seed);
}

}  // extern "C"
