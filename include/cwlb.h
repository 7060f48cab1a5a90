/*
 * cwlb.h -- C ABI of the MI355X (gfx950) CWLB-SpMM library, libcwlb.so.
 *
 * FP32 mean-aggregation SpMM over a degree-reordered CSR, executed as the
 * cost-weighted task list of CWLB-SpMM, plus the host preprocessing around
 * it (degree reordering, cost-weighted partitioning, segment-size
 * selection, cost calibration and the cost file).
 *
 * Conventions
 *   - Plain C types only; int32 CSR arrays, float32 values and features,
 *     row-major dense matrices (row r of H at H + r*K).
 *   - Every call returns cwlb_status; on failure cwlb_last_error() gives a
 *     thread-local message.
 *   - Device-pointer calls are enqueued on the context's HIP stream; they
 *     synchronise only when a timing struct is requested.
 *   - A context is used by one host thread at a time.
 * The C++17 drop-in headers (Matrix.h, utils.h, parallelMatrix.h, ...)
 * are thin wrappers over these entry points.
 */
#ifndef CWLB_H
#define CWLB_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CWLB_VERSION_STRING "0.1.0"

typedef enum cwlb_status {
    CWLB_OK = 0,
    CWLB_INVALID_ARG = 1,     /* std::invalid_argument in the reference */
    CWLB_UNSUPPORTED = 2,     /* configuration the device cannot run */
    CWLB_HIP_ERROR = 3,       /* a HIP runtime call failed */
    CWLB_OOM = 4,             /* host or device allocation failed */
    CWLB_IO_ERROR = 5,        /* file could not be opened / parsed / written */
    CWLB_INSUFFICIENT = 6,    /* output buffer too small; size reported */
    CWLB_RUNTIME_ERROR = 7    /* std::runtime_error in the reference */
} cwlb_status;

/* One task: half-open range of reordered rows; the first row starts at
 * first_row_offset nonzeros, the last row ends at last_row_nnz nonzeros
 * (0 = its full degree).  Same layout as ParallelDataWeighted
 * (reference include/utils.h:15-20). */
typedef struct cwlb_task {
    int32_t row_start;
    int32_t row_end;
    int32_t first_row_offset;
    int32_t last_row_nnz;
} cwlb_task;

/* Calibrated operation weights (ns per op per work-item, x10) and the
 * calibration metadata.  Same fields as SpmmCostParams (reference
 * include/utils.h:23-33). */
typedef struct cwlb_cost_params {
    double C_compute_ns;
    double C_load_ns;
    double C_store_ns;
    double C_atomic_ns;
    int32_t K;
    int32_t WI;
    int32_t repeat;
    int32_t atomic_writers_per_addr;
} cwlb_cost_params;

/* Kernel timings of one SpMM call, from HIP events on the context stream
 * (microseconds).  zero_us: clearing the rows that receive atomic partial
 * sums; main_us: the aggregation kernel; total_us: both. */
typedef struct cwlb_timing {
    float zero_us;
    float main_us;
    float total_us;
} cwlb_timing;

typedef struct cwlb_device_info {
    int32_t device;
    int32_t compute_units;        /* 256 on MI355X */
    int32_t max_work_group_size;  /* 1024 */
    int32_t wavefront_size;       /* 64 */
    int64_t lds_bytes_per_block;
    int64_t total_global_mem;
    char name[256];
    char arch[64];                /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
} cwlb_device_info;

typedef struct cwlb_ctx cwlb_ctx;

/* ---------------------------------------------------------------- basics */
const char* cwlb_version(void);
const char* cwlb_last_error(void);

/* Creates a context on HIP device `device` that launches on `stream`
 * (a hipStream_t; NULL selects the null stream).  Replaces the
 * sycl::queue the reference passes around (main.cpp:514-516). */
cwlb_status cwlb_ctx_create(int device, void* stream, cwlb_ctx** out);
cwlb_status cwlb_ctx_destroy(cwlb_ctx* ctx);
/* Later calls run on `stream`.  The new stream first waits for all work
 * enqueued on the old one so far (an event recorded there), because calls
 * still running on the old stream may read the context's own buffers that a
 * call on the new one rewrites; so the old stream must not have been
 * destroyed yet (switch away from a stream before destroying it).  Not done
 * when either stream is under graph capture: ordering against a captured
 * graph is then the caller's. */
cwlb_status cwlb_ctx_set_stream(cwlb_ctx* ctx, void* stream);
/* Waits for the context's stream; then reports, as CWLB_INVALID_ARG, a bad
 * column index, origin entry or row offset that the last aggregation met
 * (asynchronous calls cannot report it themselves). */
cwlb_status cwlb_ctx_synchronize(cwlb_ctx* ctx);
cwlb_status cwlb_ctx_device_info(cwlb_ctx* ctx, cwlb_device_info* out);
/* Schedule of later SpMM calls on this context: tasks executed per wave
 * (a run of consecutive tasks, at most 2^20) and feature slices spread
 * across the XCDs.  0 selects automatically (the default).  feature_slices must be 0, 1, 2, 4
 * or 8; the slices are whole 4-float vectors, as even as K allows (K = 600
 * in 4 slices: 38, 38, 37 and 37 vectors).  K not a multiple of 4, fewer
 * vectors than slices, or misaligned H / C fall back to 1 slice.
 * CWLB_SPMM_PER_TASK overrides both with 1.  No counterpart in the reference (its work-group per task is
 * fixed); tuning and tests use it. */
cwlb_status cwlb_ctx_set_schedule(cwlb_ctx* ctx, int32_t tasks_per_wave, int32_t feature_slices);

/* Locality of later SpMM calls on this context.  run_order: 0 automatic,
 * 1 runs in task order, 2 runs sorted by the original id of their first row
 * (a device sort, redone only when the task array, origin array, task count
 * or run length changes, by a call that then synchronises its stream; it
 * groups the rows of all degree classes that
 * neighbour each other in the original numbering.  Every order of the runs
 * gives the same result, so after rewriting a task array in place only the
 * speed can suffer; calling this function again forces a new sort).
 * xcd_blocks: 0 automatic, 1 consecutive run blocks interleaved over the 8
 * XCDs, 2 each XCD takes one contiguous stretch of run blocks.  Ignored with
 * CWLB_SPMM_PER_TASK.  No counterpart in the reference; tuning and tests use
 * it. */
cwlb_status cwlb_ctx_set_locality(cwlb_ctx* ctx, int32_t run_order, int32_t xcd_blocks);

/* Cache-policy hints of later SpMM calls on this context.  hot_bytes = 0
 * (the default): every feature row is loaded with the normal policy.
 * hot_bytes > 0: the columns are ranked by in-degree; the feature rows of
 * the most-gathered columns, about hot_bytes of them, keep the normal policy
 * and the rest are loaded non-temporally, so that on skewed graphs the hot
 * rows stay in L2 and the Infinity Cache.  The first call after a change of
 * the column array, nnz, h_rows or hot_bytes builds one bit per nonzero in a
 * context-owned device buffer (and synchronises the stream); later calls
 * reuse it.  A call on a stream under graph capture never builds: it reuses
 * matching hints or runs without them.  The hints steer
 * only the cache policy: results are the same with or without them, and
 * hints left over from earlier contents of col_idx only cost speed.
 * Applies with 16-byte aligned H and C, K a multiple of 4, at most 256
 * floats per feature slice and H below 4 GiB; otherwise ignored.  No
 * counterpart in the reference; cwlb_ctx_tune_schedule tries 24, 48 and
 * 96 MB. */
cwlb_status cwlb_ctx_set_cache_hints(cwlb_ctx* ctx, int64_t hot_bytes);
cwlb_status cwlb_ctx_get_cache_hints(cwlb_ctx* ctx, int64_t* hot_bytes);

/* Kernel occupancy of later SpMM calls on this context.  waves_per_simd = 0
 * (the default): the standard kernel, 5 waves per SIMD where its slots are
 * wider than 2 lanes.  6: a variant with at most 2 nonzeros per slot in
 * flight on long chunks, which fits 80 VGPRs and runs 6 waves per SIMD;
 * faster on graphs of short rows (latency-bound), slower on graphs with
 * hub rows.  It applies to 16-byte lanes with more than 8 and at most 64
 * floats per feature slice; otherwise the standard kernel runs.  Results
 * are the same within the documented tolerance (full short rows bit for
 * bit).  No counterpart in the reference; cwlb_ctx_tune_schedule tries it. */
cwlb_status cwlb_ctx_set_occupancy(cwlb_ctx* ctx, int32_t waves_per_simd);
cwlb_status cwlb_ctx_get_occupancy(cwlb_ctx* ctx, int32_t* waves_per_simd);

/* Lane tiling of later SpMM calls.  A feature slice of F vectors (4 floats
 * each) is covered by slots of G lanes, each lane holding R vectors per
 * pass; a wave has 64 / G slots, each working on its own row (short rows)
 * or nonzero (long rows).  1: power-of-two slots, G the smallest power of
 * two >= F and R = 1 (F <= 64; wider slices G = 64, R = ceil(F / 64) up to 8
 * without feature slices, else G = 64 in several passes).  2: packed slots,
 * G x R also in {4x3, 4x5, 8x3, 8x5, 16x3} (wider slices, without cache
 * hints or column phases: 16x5, 32x3, 32x5, 64x3, 64x5), whichever covers
 * the slice with the fewest vector loads per nonzero (the fewest idle
 * lanes), the smaller R on a tie: F = 24 (K = 96) runs in 8-lane slots of 3
 * vectors instead of 32-lane slots with 8 lanes idle.  Applies with 16-byte
 * aligned H and C and K a multiple of 4, not with the occupancy variant or
 * CWLB_SPMM_PER_TASK.  0 = automatic (currently 1).  Results agree within
 * the float tolerance (each lane still sums its vectors in CSR order, so
 * rows summed by one slot are unchanged bit for bit).  The reference pads
 * the row the same way (parallelMatrix.cpp:93-99: a work-group of K
 * rounded up).  No counterpart in the reference; cwlb_ctx_tune_schedule
 * tries it. */
cwlb_status cwlb_ctx_set_lane_tiling(cwlb_ctx* ctx, int32_t tiling);
cwlb_status cwlb_ctx_get_lane_tiling(cwlb_ctx* ctx, int32_t* tiling);

/* Column phases of later SpMM calls on this context.  phases = 0 or 1 (the
 * default): one pass.  phases = P in [2, 64]: the task list is executed P
 * times, pass p gathering only the nonzeros whose column c has
 * c mod P = p, so that the feature rows all waves read at a time are 1/P of
 * H and stay in the caches (the bands interleave the columns, so that
 * communities numbered as ranges of ids spread over all passes).  Each
 * phased call first writes, into context-owned buffers, a copy of col_idx
 * and val with every row's nonzeros stably sorted by band and the row
 * bounds of the bands (see cwlb_column_phase_sort; 8 bytes per nonzero
 * and 4 (P - 1) per row, kept and grown as needed; about 0.3 ms on a
 * 115M-nonzero graph, reported in the timing's zero_us), so rewritten
 * arrays are always read as they are.  A row that one stretch of
 * consecutive tasks covers whole (see CWLB_SPMM_PER_TASK) is stored in the
 * first pass and added to in the others without atomics, which reads and
 * writes C P times: phases pay when H is well beyond the 256 MB Infinity
 * Cache, the columns of a row are spread over H and rows hold many more
 * nonzeros than 2P (measured: a 240k-row block model with 480 nonzeros per
 * row and K = 600, 12 phases: 27.6 ms per call against 37.2 ms).  Under
 * graph capture the buffers are only used when an earlier call sized them
 * (otherwise the call runs in one pass); a buffer a capture used is never
 * freed before cwlb_ctx_destroy.  Applies to task lists that are chains -- every task
 * well formed and starting where its predecessor ended, as
 * cwlb_partition's lists are -- which the device checks on every call; any
 * other list runs in one pass over the caller's col_idx and val (its task
 * offsets index them), and the band sort it already paid for is unused.
 * Applies with
 * 16-byte aligned H and C, K a multiple of 4 and at most 256 floats per
 * feature slice, without CWLB_SPMM_PER_TASK; replaces the occupancy variant
 * and the cache hints while on.  Results agree with the one-pass ones
 * within the float tolerance (each row is summed band by band, each band's
 * partial sum divided and added separately).  No counterpart in the
 * reference; cwlb_ctx_tune_schedule tries it. */
cwlb_status cwlb_ctx_set_column_phases(cwlb_ctx* ctx, int32_t phases);
cwlb_status cwlb_ctx_get_column_phases(cwlb_ctx* ctx, int32_t* phases);

/* The band sort of P column phases (2 <= P <= 64), enqueued on the
 * context's stream from device arrays.  The band of a column c is c mod P
 * (a column below 0 or at or above h_rows is in band 0).  bounds_out
 * (optional, (P - 1) * n_rows ints): bounds_out[(p - 1) * n_rows + r] =
 * row_ptr[r] + the number of nonzeros of row r in bands below p, for p in
 * [1, P).  col_out and val_out (optional, together, nnz each): col_idx and
 * val with each row's nonzeros stably sorted by band, so that band p of
 * row r is [B_p(r), B_{p+1}(r)) with B_0(r) = row_ptr[r] and B_P(r) =
 * row_ptr[r + 1].  A row whose offsets leave [0, nnz] or decrease gets
 * bounds 0 and is not copied.  No counterpart in the reference; the
 * column-phased aggregation runs this itself, tests read it here. */
cwlb_status cwlb_column_phase_sort(cwlb_ctx* ctx, const int32_t* row_ptr,
                                   const int32_t* col_idx, const float* val, int32_t n_rows,
                                   int64_t nnz, int64_t h_rows, int32_t phases,
                                   int32_t* bounds_out, int32_t* col_out, float* val_out);

/* The schedule the last aggregation launch on this context used, as the
 * automatic choices and the context's settings resolved it (all zero before
 * the first launch).  No counterpart in the reference; tests and the bench
 * report it. */
typedef struct cwlb_launch_info {
    int32_t tasks_per_wave;  /* tasks per run (1 with CWLB_SPMM_PER_TASK) */
    int32_t feature_slices;  /* 1, 2, 4 or 8 */
    int32_t run_order;       /* 1 task order, 2 sorted by output row */
    int32_t xcd_blocks;      /* 1 interleaved over the XCDs, 2 contiguous */
    int32_t cache_hints;     /* 1 when the gathers carried cache hints */
    int32_t vector_width;    /* floats per load: 4, 2 or 1 */
    int32_t waves_per_simd;  /* 6 for the occupancy variant, else 0 */
    int32_t max_waves_per_cu; /* resident waves per CU the kernel's register
                                 and LDS use allow */
    int32_t column_phases;   /* column phases planned (1 = none; a task list
                                that is not a chain runs unphased all the
                                same, see cwlb_ctx_set_column_phases) */
    int32_t slot_lanes;      /* lanes per row slot (see cwlb_ctx_set_lane_tiling) */
    int64_t grid_blocks;     /* work-groups of the aggregation kernel (per
                                phase) */
    int32_t lane_vectors;    /* vectors each lane of a slot holds per pass */
} cwlb_launch_info;
cwlb_status cwlb_ctx_last_launch(cwlb_ctx* ctx, cwlb_launch_info* out);

/* ------------------------------------------------------------ aggregation
 * C[Origin_local[r]][k] = (sum over the task chunks of row r of
 *   val[j] * H[col_idx[j]][k]) / deg(r)
 * executed per task as in spmmKernel (reference parallelMatrix.cpp:63-254):
 * a chunk that is the full row is stored, a partial chunk is added
 * atomically (after its row was cleared), rows of degree 0 are written as
 * zeros.  All pointers are device pointers: row_ptr[n_rows+1],
 * col_idx[nnz], val[nnz], origin[n_rows], H[h_rows*K], tasks[n_tasks],
 * C[n_rows*K].
 *
 * Preconditions checked on the host: n_rows >= 0, nnz >= 0, K >= 0,
 * n_tasks >= 0, non-null pointers for non-empty arrays.  On the device:
 * task row ranges are clamped as in the reference (parallelMatrix.cpp:
 * 169-176); a column index outside [0, h_rows), an origin entry outside
 * [0, n_rows) or a row whose offsets leave [0, nnz] or decrease is skipped
 * and reported as CWLB_INVALID_ARG (by this call when it synchronises, else
 * by cwlb_ctx_synchronize).
 * With the flag CWLB_SPMM_ZERO_OUTPUT the whole of C is cleared first (the
 * reference's host-side Zero(), parallelMatrix.cpp:112).  Then every task
 * list in which no two tasks share a nonzero -- in any order, with gaps --
 * gives the reference's result; lists whose tasks overlap need
 * CWLB_SPMM_PER_TASK as well.  Without the flag, rows whose first nonzero
 * no task covers keep their previous contents.  A partition from
 * cwlb_partition covers every row with nonzeros; it leaves out the rows
 * without nonzeros when their slot cost Cs exceeds the capacity (as the
 * reference's does, utils.cpp:972-976), and the reference's result for
 * them is the 0 of its cleared C: clear C once (this flag on the first
 * call) before calls without it.
 * K == 0 or n_tasks == 0: C is cleared (when CWLB_SPMM_ZERO_OUTPUT is set)
 * and timings are 0, as the reference returns a zero matrix with time 0
 * (parallelMatrix.cpp:80-83, 101-104).
 * timing may be NULL (asynchronous: the bad entries above are then
 * reported by the next cwlb_ctx_synchronize); otherwise the call
 * synchronises.  With any of the flags a call launches kernels only (no
 * memset nodes, no allocation), so an asynchronous call can be
 * captured into a HIP graph.  Under capture the run order (run_order = 2)
 * and the cache hints are reused when an earlier call built them for the
 * same arrays, and otherwise left out (task order, normal cache policy);
 * the results are the same either way.  A captured graph stays valid until
 * cwlb_ctx_destroy: a run order or hint array that a capture used is never
 * rewritten or freed by later calls on the context (a rebuild goes into a
 * new buffer), so replays may be interleaved with eager calls on other
 * task or column arrays.
 *
 * cwlb_spmm_mean_f32 mirrors spmmKernel: K > max work-group size (1024)
 * returns CWLB_INVALID_ARG (parallelMatrix.cpp:84-88).
 * cwlb_spmm_mean_f32_large_k mirrors spmmKernelLargeKFallback: it requires
 * K > max work-group size (parallelMatrix.cpp:287-290). */
#define CWLB_SPMM_ZERO_OUTPUT 0x1u
/* Execute exactly one task per wave, each partial chunk added atomically
 * (the reference's structure).  Without this flag a wave executes a run of
 * consecutive tasks (run length chosen from the task count and the CU
 * count), and the feature columns may be split across the XCDs.  Inside a
 * run, each stretch of tasks in which every task starts where the previous
 * one ended (the partition's lists consist of such stretches) is executed
 * as one task: rows split only inside it are reduced in registers and
 * stored.  A task that does not continue its predecessor, or a malformed
 * one, starts a new stretch.  For task lists without overlapping tasks both
 * modes give the same result up to float rounding. */
#define CWLB_SPMM_PER_TASK 0x2u
/* Leave the rows without nonzeros unwritten: the caller's C holds zeros
 * there already (an earlier call with CWLB_SPMM_ZERO_OUTPUT on the same C
 * and row_ptr/origin, or a clear of its own).  This is what the reference's
 * kernel does: it never writes such rows, and its C starts cleared
 * (parallelMatrix.cpp:112, 166).  Without the flag they are stored as
 * zeros, so that C needs no clearing; with CWLB_SPMM_ZERO_OUTPUT they are
 * never stored either (the call has just cleared them).  No counterpart
 * flag in the reference; for repeated calls on one C, where it saves one
 * store per empty row (R-MAT 2^22: 52% of the rows). */
#define CWLB_SPMM_KEEP_EMPTY_ROWS 0x4u
/* The aggregation entry points return CWLB_INVALID_ARG for any other flag
 * bit. */

cwlb_status cwlb_spmm_mean_f32(cwlb_ctx* ctx, const int32_t* row_ptr, const int32_t* col_idx,
                               const float* val, const int32_t* origin, int32_t n_rows,
                               int64_t nnz, const float* H, int64_t h_rows, int32_t K,
                               const cwlb_task* tasks, int64_t n_tasks, float* C,
                               uint32_t flags, cwlb_timing* timing);

cwlb_status cwlb_spmm_mean_f32_large_k(cwlb_ctx* ctx, const int32_t* row_ptr,
                                       const int32_t* col_idx, const float* val,
                                       const int32_t* origin, int32_t n_rows, int64_t nnz,
                                       const float* H, int64_t h_rows, int32_t K,
                                       const cwlb_task* tasks, int64_t n_tasks, float* C,
                                       uint32_t flags, cwlb_timing* timing);

/* Times the aggregation of these (device) inputs under the automatic
 * schedule and under every tasks-per-wave value in {2, 4, ..., 64} with 1,
 * 2, 4 or 8 feature slices (slices of at least 32 floats), `trials`
 * event-timed calls each after one warm-up (median of split-row clearing +
 * aggregation; a run length or slice count, or later a phase setting,
 * whose first timed call is more than 10% behind the best so far is not
 * timed further), and sets
 * the fastest on the context (cwlb_ctx_set_schedule); the choice is also
 * returned through the optional out pointers (0, 0 = the automatic schedule
 * won).  With locality_out non-null (two int32), the fastest schedule is
 * timed afresh under the context's placement and with runs sorted by output
 * row (interleaved and contiguous XCD placement, cwlb_ctx_set_locality), in
 * two interleaved rounds; the winner is kept on the context and written
 * there (the context's previous setting when it wins);
 * then with the occupancy variant (cwlb_ctx_set_occupancy, kept when
 * faster, and then also timed at half and double the run length, so the
 * tasks per wave returned can be 1); then with cache hints of 24, 48 and
 * 96 MB (cwlb_ctx_set_cache_hints), the fastest kept on the context (0 =
 * none; read it with cwlb_ctx_get_cache_hints); then the standard kernel
 * again with those hints when the variant was kept; then with packed
 * slots (cwlb_ctx_set_lane_tiling(2), where they change the tiling), kept
 * when faster; then, when H holds at least 512 MB, K is a multiple of 4 and
 * rows average 64 nonzeros or more, with 8, 12 and 16 column phases
 * (cwlb_ctx_set_column_phases) at every slice count they take and 16, 32
 * or 64 tasks per wave, each with power-of-two and with packed slots: the
 * fastest is kept when it beats the settings so far (its tasks per wave and
 * slices are then the ones returned; read the phases with
 * cwlb_ctx_get_column_phases and the tiling with
 * cwlb_ctx_get_lane_tiling), otherwise phases stay off.  In that mode
 * every timing before the hint sizes runs without hints, every timing
 * before the occupancy variant with the standard kernel, every timing
 * before the packed slots with the automatic tiling, and every timing
 * before the phases in one pass, whatever the context held.  C receives
 * the result.  Synchronises.  No counterpart in the reference, whose one task
 * per work-group has nothing to tune; like its S search, it is meant to run
 * once per graph before timed runs. */
cwlb_status cwlb_ctx_tune_schedule(cwlb_ctx* ctx, const int32_t* row_ptr, const int32_t* col_idx,
                                   const float* val, const int32_t* origin, int32_t n_rows,
                                   int64_t nnz, const float* H, int64_t h_rows, int32_t K,
                                   const cwlb_task* tasks, int64_t n_tasks, float* C,
                                   int32_t trials, int32_t* tasks_per_wave_out,
                                   int32_t* feature_slices_out, int32_t* locality_out);

/* Host-pointer form: copies the inputs to the device, runs the call, copies
 * C back (the reference's per-call sycl::buffer behaviour,
 * parallelMatrix.cpp:115-121).  C is always cleared first.  Dispatches on K
 * like run_single_s (main.cpp:359-365).  A task list that does not tile the
 * nonzeros in order runs one task per wave, so every list, overlapping ones
 * included, gives the reference's result.  Timing covers the kernels only.
 * The host arrays may be pageable: transfers go through two 64 MiB pinned
 * staging buffers that the context allocates at its first host-pointer call
 * and keeps until cwlb_ctx_destroy, filled and drained by up to 8 host
 * threads while the DMA engine moves the other buffer (if pinned memory is
 * refused, the arrays are copied directly). */
cwlb_status cwlb_spmm_mean_f32_host(cwlb_ctx* ctx, const int32_t* row_ptr,
                                    const int32_t* col_idx, const float* val,
                                    const int32_t* origin, int32_t n_rows, int64_t nnz,
                                    const float* H, int64_t h_rows, int32_t K,
                                    const cwlb_task* tasks, int64_t n_tasks, float* C,
                                    cwlb_timing* timing);

/* Allocation-free form of cwlb_spmm_mean_f32, with no counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
 * needs no context: it runs on the current HIP device and the given stream
 * (NULL = the null stream), with the automatic schedule or the given tasks
 * per wave and feature slices (as cwlb_ctx_set_schedule; 0 = automatic), in
 * task order, in one pass (no column phases) and without cache hints.  Any K is accepted (both
 * cwlb_spmm_mean_f32's range and the large-K entry's); flags and results
 * are those of cwlb_spmm_mean_f32.  It calls no hipMalloc, hipFree or other
 * allocating routine: the kernels' status word lives in a 256-byte device
 * array of the library (one per GPU, kept until the process ends, located
 * on a device's first call); its size does not depend on the inputs, so no
 * input is too large for it.  synchronize != 0: the call waits for the
 * stream and reports a bad column index, origin entry or row offset as
 * CWLB_INVALID_ARG; 0: asynchronous, such entries are skipped unreported.
 * On a stream under graph capture synchronize must be 0: a call with
 * synchronize != 0 there returns CWLB_INVALID_ARG before enqueueing
 * anything, so the capture stays valid.
 * All calls on one GPU share that status word, which each call resets:
 * calls that overlap on one GPU (different streams) may report each
 * other's errors. */
cwlb_status cwlb_spmm_mean_f32_noalloc(void* stream, const int32_t* row_ptr,
                                       const int32_t* col_idx, const float* val,
                                       const int32_t* origin, int32_t n_rows, int64_t nnz,
                                       const float* H, int64_t h_rows, int32_t K,
                                       const cwlb_task* tasks, int64_t n_tasks, float* C,
                                       uint32_t flags, int32_t tasks_per_wave,
                                       int32_t feature_slices, int32_t synchronize);

/* ----------------------------------------------------------- preprocessing
 * Degree reordering, sortCSRByDegreeDPLCPU (reference main.cpp:197-278):
 * rows ordered by (degree, original id) ascending; origin[new] = old;
 * row_ptr_out is the inclusive scan of the sorted degrees; each row's
 * entries keep their order.  Host arrays.  Returns CWLB_RUNTIME_ERROR when
 * row_ptr[n_rows] != nnz (the reference's inconsistent-nnz error). */
cwlb_status cwlb_reorder_by_degree(int32_t n_rows, int64_t nnz, const int32_t* row_ptr,
                                   const int32_t* col_idx, const float* val, int32_t* origin,
                                   int32_t* row_ptr_out, int32_t* col_idx_out, float* val_out);

/* The same permutation and arrays computed on the GPU from device arrays
 * (stable counting sort by degree + row gather).  Bit-identical to
 * cwlb_reorder_by_degree.  Synchronises. */
cwlb_status cwlb_reorder_by_degree_device(cwlb_ctx* ctx, int32_t n_rows, int64_t nnz,
                                          const int32_t* row_ptr, const int32_t* col_idx,
                                          const float* val, int32_t* origin,
                                          int32_t* row_ptr_out, int32_t* col_idx_out,
                                          float* val_out);

/* Cost-weighted task partitioning, costWeightedTaskPartitioning (reference
 * utils.cpp:832-1021), bit-exact.  row_ptr is the reordered CSR's host
 * offsets (n_rows + 1 entries; n_rows <= 0 gives no tasks).  Writes at most
 * capacity_tasks tasks to out (may be NULL when capacity_tasks == 0) and
 * stores the full count in *n_tasks; returns CWLB_INSUFFICIENT when the
 * buffer was too small. */
cwlb_status cwlb_partition(const int32_t* row_ptr, int32_t n_rows, const cwlb_cost_params* costs,
                           double capacity_weight, cwlb_task* out, int64_t capacity_tasks,
                           int64_t* n_tasks);

/* The same partition computed on the GPU from the device offsets
 * row_ptr[n_rows + 1] into the device array out; identical task lists.
 * Each fresh state of the host's greedy state machine (a task opening at a
 * row, or at a long row whose deg % S prefix went to the previous task) is
 * simulated to the next one in parallel, and the chain from row 0 is found
 * by pointer doubling.  Returns CWLB_INSUFFICIENT (with *n_tasks set) when
 * capacity_tasks is too small, and CWLB_UNSUPPORTED for costs under which a
 * task's row count has no bound (C_store <= 0, C_compute + C_load < 0,
 * non-finite values, capacity / C_store > 65536): cwlb_partition handles
 * those.  row_ptr must be non-decreasing.  Synchronises. */
cwlb_status cwlb_partition_device(cwlb_ctx* ctx, const int32_t* row_ptr, int32_t n_rows,
                                  const cwlb_cost_params* costs, double capacity_weight,
                                  cwlb_task* out, int64_t capacity_tasks, int64_t* n_tasks);

/* --------------------------------------------------- segment-size selection
 * capacity_from_s (reference main.cpp:281-292). */
double cwlb_capacity_from_s(int32_t s, const cwlb_cost_params* costs);
/* wave_based_s (main.cpp:295-321): S = clamp(ceil(nnz/(cu*wave)), 1,
 * INT_MAX); row_ptr_len == 0 (empty RowOffset) gives 1.  Non-positive cu or
 * wave -> CWLB_INVALID_ARG. */
cwlb_status cwlb_wave_based_s(int64_t nnz, int64_t row_ptr_len, int32_t compute_units,
                              int32_t wave, int32_t* s_out);
/* recommended_candidate_w (main.cpp:87-95). */
void cwlb_recommended_candidate_w(uint64_t nnz, int32_t out3[3]);
/* candidate_search_bounds (main.cpp:109-127). */
cwlb_status cwlb_candidate_search_bounds(const int32_t values3[3], int64_t best_index,
                                         int32_t* lower, int32_t* upper);
/* candidate_search_by_count / _by_step (main.cpp:130-167); two-call sizing
 * as cwlb_partition. */
cwlb_status cwlb_candidate_search_by_count(int32_t lower, int32_t upper, int32_t requested,
                                           int32_t* out, int64_t capacity, int64_t* count);
cwlb_status cwlb_candidate_search_by_step(int32_t lower, int32_t upper, int32_t step,
                                          int32_t* out, int64_t capacity, int64_t* count);

/* ------------------------------------------------------------- calibration
 * measure_spmm_costs (reference utils.cpp:342-829) on gfx950: compute,
 * load, store and atomic micro-benchmarks, 20 warm-ups and `repeat` timed
 * launches each, coefficients in ns per op per work-item x10.  The load
 * benchmark groups lanes by 64 (one wave) instead of the reference's 32.
 * Fills out->K, WI, repeat and atomic_writers_per_addr too. */
cwlb_status cwlb_calibrate(cwlb_ctx* ctx, int32_t K, int32_t repeat, int32_t WI,
                           int32_t load_MB, int32_t atomic_writers, cwlb_cost_params* out);

/* What each coefficient of a calibration was computed from: the mean
 * event-timed launch duration of its micro-benchmark (ms) and the operation
 * count it is divided by.  coefficient = ms * 1e6 / ops * 10, with ops =
 * WI * K for compute, load and store (utils.cpp:419-421, 522-524, 583-585)
 * and ops = writer groups * feature block for the atomic (:791-806).
 * bytes_* are the bytes one launch of the load / store benchmark reads /
 * writes through its loads and stores (4 per op). */
typedef struct cwlb_calibration_report {
    double compute_ms;
    double load_ms;
    double store_ms;
    double atomic_ms;
    int64_t compute_ops;
    int64_t load_ops;
    int64_t store_ops;
    int64_t atomic_ops;
    int64_t load_bytes;
    int64_t store_bytes;
} cwlb_calibration_report;

/* cwlb_calibrate that also fills *report (may be NULL).  No counterpart in
 * the reference, which prints these figures (utils.cpp:806-825); tests use
 * it to check the normalisation. */
cwlb_status cwlb_calibrate_report(cwlb_ctx* ctx, int32_t K, int32_t repeat, int32_t WI,
                                  int32_t load_MB, int32_t atomic_writers, cwlb_cost_params* out,
                                  cwlb_calibration_report* report);

/* Cost file (utils.cpp:1024-1092): four lines compute/load/store/atomic,
 * fixed notation with `precision` decimals; the parent directory is
 * created; a parent that exists as a file fails.  Returns CWLB_IO_ERROR on
 * failure. */
cwlb_status cwlb_save_costs(const cwlb_cost_params* costs, const char* path, int append,
                            int precision);
cwlb_status cwlb_read_costs(cwlb_cost_params* out, const char* path);

/* -------------------------------------------------------------- utilities
 * Features in U[-1, 1) written on the device, bit-identical to the host
 * generator used by the tests: value(i) = (int(top 24 bits of
 * mix64(mix64(seed) + i)) - 2^23) * 2^-23 for i = row*K + k. */
cwlb_status cwlb_fill_features_uniform(cwlb_ctx* ctx, float* H, int64_t rows, int32_t K,
                                       uint64_t seed);

#ifdef __cplusplus
}
#endif

#endif /* CWLB_H */
