// cwlb_spmm_mean_f32_noalloc: the device-pointer aggregation without a
// context and without any allocation, for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops).
//
// The only device memory the aggregation needs beyond its inputs and output
// is the status word its kernels report malformed entries through (the
// context path keeps it in a hipMalloc'd int).  Here it lives in `scratch`,
// a file-scope device array: 256 bytes per GPU, held until the process ends.
// Its size does not depend on the inputs, so no input is too large for it.
// Every call on a GPU shares that GPU's copy; the kernels reset the status
// word at the start of each call, so calls that overlap on one GPU (on
// different streams) race on it and may report each other's errors.
#include <cstring>
#include <mutex>

#include "internal.h"

// 256 bytes per GPU: [0] = the status word of the last call.
static __device__ __align__(256) int scratch[64];

namespace cwlb {
namespace {

constexpr int kMaxDevices = 64;

struct DeviceSlot {
    std::once_flag once;
    cwlb_status st = CWLB_OK;
    std::string err;
    int* ptr = nullptr;  // this device's copy of `scratch`
    int compute_units = 0;
    int max_wg = 0;
};

DeviceSlot g_slots[kMaxDevices];

// Once per device, with that device current: the device address of its
// copy of `scratch` and the launch limits the schedule needs.  The host
// symbol `scratch` itself is never handed to a kernel or a copy.
void init_slot(DeviceSlot& s, int device)
{
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) {
        s.st = e == hipErrorOutOfMemory ? CWLB_OOM : CWLB_HIP_ERROR;
        s.err = std::string("cwlb_spmm_mean_f32_noalloc: hipGetDeviceProperties: ") +
                hipGetErrorString(e);
        return;
    }
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        s.st = CWLB_UNSUPPORTED;
        s.err = std::string("cwlb: built for gfx950 only, device is ") + prop.gcnArchName;
        return;
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        s.st = CWLB_HIP_ERROR;
        s.err = std::string("cwlb_spmm_mean_f32_noalloc: hipGetSymbolAddress(scratch): ") +
                hipGetErrorString(e);
        return;
    }
    s.ptr = static_cast<int*>(p);
    s.compute_units = prop.multiProcessorCount;
    s.max_wg = prop.maxThreadsPerBlock;
}

}  // namespace
}  // namespace cwlb

using namespace cwlb;

extern "C" cwlb_status cwlb_spmm_mean_f32_noalloc(
    void* stream, const int32_t* row_ptr, const int32_t* col_idx, const float* val,
    const int32_t* origin, int32_t n_rows, int64_t nnz, const float* H, int64_t h_rows, int32_t K,
    const cwlb_task* tasks, int64_t n_tasks, float* C, uint32_t flags, int32_t tasks_per_wave,
    int32_t feature_slices, int32_t synchronize)
{
    int device = -1;
    CWLB_HIP_TRY(hipGetDevice(&device));
    if (device < 0 || device >= kMaxDevices)
        return fail(CWLB_UNSUPPORTED, "cwlb_spmm_mean_f32_noalloc: device id out of range");
    DeviceSlot& slot = g_slots[device];
    std::call_once(slot.once, [&] { init_slot(slot, device); });
    if (slot.st != CWLB_OK) return fail(slot.st, slot.err);
    if (flags & ~kSpmmFlags) return fail(CWLB_INVALID_ARG, "spmm: unknown flag bits");
    if (tasks_per_wave < 0 || tasks_per_wave > (1 << 20))
        return fail(CWLB_INVALID_ARG,
                    "tasks_per_wave must be in [0, 1048576] (0 = automatic)");
    if (feature_slices != 0 && feature_slices != 1 && feature_slices != 2 &&
        feature_slices != 4 && feature_slices != 8)
        return fail(CWLB_INVALID_ARG, "feature_slices must be 0, 1, 2, 4 or 8");
    if (n_rows < 0 || nnz < 0 || K < 0 || n_tasks < 0 || h_rows < 0)
        return fail(CWLB_INVALID_ARG, "spmm: negative size");
    if (nnz > INT32_MAX) return fail(CWLB_INVALID_ARG, "spmm: nnz must fit int32");
    if (K > 0 && n_tasks > 0) {
        if (!row_ptr || !origin || !tasks || !C)
            return fail(CWLB_INVALID_ARG, "spmm: null device pointer");
        if (nnz > 0 && (!col_idx || !val || !H))
            return fail(CWLB_INVALID_ARG, "spmm: null device pointer");
    }
    if (n_rows > 0 && K > 0 && !C) return fail(CWLB_INVALID_ARG, "spmm: null C");
    if (synchronize) {
        // The status read-back and the wait cannot be recorded into a graph;
        // refused before anything is enqueued, so the capture stays valid.
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        CWLB_HIP_TRY(hipStreamIsCapturing(static_cast<hipStream_t>(stream), &capture));
        if (capture != hipStreamCaptureStatusNone)
            return fail(CWLB_INVALID_ARG,
                        "cwlb_spmm_mean_f32_noalloc: synchronize must be 0 on a stream under "
                        "graph capture");
    }

    // A context on the stack: default schedule or the given run length and
    // slices, task order, no cache hints.  Nothing in it is allocated (its
    // retired-buffer list stays empty) and nothing is built.
    cwlb_ctx c;
    c.device = device;
    c.stream = static_cast<hipStream_t>(stream);
    c.compute_units = slot.compute_units;
    c.max_wg = slot.max_wg;
    c.d_status = slot.ptr;
    c.sched_tasks_per_wave = tasks_per_wave;
    c.sched_slices = feature_slices;
    c.sched_order = 1;
    c.sched_xcd = 1;
    const bool zero_all = (flags & CWLB_SPMM_ZERO_OUTPUT) != 0;
    const bool per_task = (flags & CWLB_SPMM_PER_TASK) != 0;
    const bool keep_empty = (flags & CWLB_SPMM_KEEP_EMPTY_ROWS) != 0;
    SpmmArgs a{row_ptr, col_idx, val, origin, n_rows, nnz, H, h_rows, K, tasks, n_tasks, C};
    if (K > 0 && n_tasks > 0) {
        const cwlb_status s = launch_spmm_mean(&c, a, zero_all, per_task, keep_empty, false);
        if (s != CWLB_OK) return s;
    } else if (zero_all && n_rows > 0 && K > 0) {
        const cwlb_status s = launch_spmm_mean(&c, a, true, per_task, keep_empty, false);
        if (s != CWLB_OK) return s;
    }
    if (!synchronize) return CWLB_OK;
    int st = 0;
    CWLB_HIP_TRY(hipMemcpyAsync(&st, slot.ptr, sizeof(int), hipMemcpyDeviceToHost, c.stream));
    CWLB_HIP_TRY(hipStreamSynchronize(c.stream));
    if (K > 0 && n_tasks > 0) {
        if (st & 1) return fail(CWLB_INVALID_ARG, "spmm: a column index is outside [0, h_rows)");
        if (st & 2) return fail(CWLB_INVALID_ARG, "spmm: an origin entry is outside [0, n_rows)");
        if (st & 4)
            return fail(CWLB_INVALID_ARG,
                        "spmm: a row's offsets leave [0, nnz] or decrease (row_ptr)");
    }
    return CWLB_OK;
}
