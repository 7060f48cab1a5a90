"""ctypes binding of libcwlb.so (include/cwlb.h).

Host arrays are numpy; device arrays are passed as raw addresses (for
example ``torch.Tensor.data_ptr()``).  Every non-OK status raises
``CwlbError`` carrying the status and ``cwlb_last_error()``.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import paths

OK, INVALID_ARG, UNSUPPORTED, HIP_ERROR, OOM, IO_ERROR, INSUFFICIENT, RUNTIME_ERROR = range(8)
STATUS_NAMES = ["OK", "INVALID_ARG", "UNSUPPORTED", "HIP_ERROR", "OOM", "IO_ERROR",
                "INSUFFICIENT", "RUNTIME_ERROR"]
ZERO_OUTPUT = 0x1
PER_TASK = 0x2
KEEP_EMPTY_ROWS = 0x4

# Every function declared in include/cwlb.h (checked by the CPU tests).
EXPORTS = [
    "cwlb_version", "cwlb_last_error", "cwlb_ctx_create", "cwlb_ctx_destroy",
    "cwlb_ctx_set_stream", "cwlb_ctx_synchronize", "cwlb_ctx_device_info", "cwlb_ctx_set_schedule",
    "cwlb_ctx_set_locality", "cwlb_ctx_set_cache_hints", "cwlb_ctx_get_cache_hints",
    "cwlb_ctx_last_launch", "cwlb_ctx_set_occupancy", "cwlb_ctx_get_occupancy",
    "cwlb_ctx_set_column_phases", "cwlb_ctx_get_column_phases", "cwlb_column_phase_sort",
    "cwlb_ctx_set_lane_tiling", "cwlb_ctx_get_lane_tiling",
    "cwlb_ctx_tune_schedule",
    "cwlb_spmm_mean_f32", "cwlb_spmm_mean_f32_large_k", "cwlb_spmm_mean_f32_host",
    "cwlb_spmm_mean_f32_noalloc",
    "cwlb_reorder_by_degree", "cwlb_reorder_by_degree_device", "cwlb_partition",
    "cwlb_partition_device",
    "cwlb_capacity_from_s", "cwlb_wave_based_s", "cwlb_recommended_candidate_w",
    "cwlb_candidate_search_bounds", "cwlb_candidate_search_by_count",
    "cwlb_candidate_search_by_step", "cwlb_calibrate", "cwlb_calibrate_report", "cwlb_save_costs",
    "cwlb_read_costs",
    "cwlb_fill_features_uniform",
]


class CwlbError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"{STATUS_NAMES[status] if 0 <= status < 8 else status}: {msg}")
        self.status = status


class Task(C.Structure):
    _fields_ = [("row_start", C.c_int32), ("row_end", C.c_int32),
                ("first_row_offset", C.c_int32), ("last_row_nnz", C.c_int32)]


class CostParams(C.Structure):
    _fields_ = [("C_compute_ns", C.c_double), ("C_load_ns", C.c_double),
                ("C_store_ns", C.c_double), ("C_atomic_ns", C.c_double),
                ("K", C.c_int32), ("WI", C.c_int32), ("repeat", C.c_int32),
                ("atomic_writers_per_addr", C.c_int32)]

    def tuple4(self):
        return (self.C_compute_ns, self.C_load_ns, self.C_store_ns, self.C_atomic_ns)


def costs(c4) -> CostParams:
    p = CostParams()
    p.C_compute_ns, p.C_load_ns, p.C_store_ns, p.C_atomic_ns = (float(x) for x in c4)
    return p


class CalibrationReport(C.Structure):
    _fields_ = [("compute_ms", C.c_double), ("load_ms", C.c_double), ("store_ms", C.c_double),
                ("atomic_ms", C.c_double), ("compute_ops", C.c_int64), ("load_ops", C.c_int64),
                ("store_ops", C.c_int64), ("atomic_ops", C.c_int64), ("load_bytes", C.c_int64),
                ("store_bytes", C.c_int64)]


class Timing(C.Structure):
    _fields_ = [("zero_us", C.c_float), ("main_us", C.c_float), ("total_us", C.c_float)]


class LaunchInfo(C.Structure):
    _fields_ = [("tasks_per_wave", C.c_int32), ("feature_slices", C.c_int32),
                ("run_order", C.c_int32), ("xcd_blocks", C.c_int32),
                ("cache_hints", C.c_int32), ("vector_width", C.c_int32),
                ("waves_per_simd", C.c_int32), ("max_waves_per_cu", C.c_int32),
                ("column_phases", C.c_int32), ("slot_lanes", C.c_int32),
                ("grid_blocks", C.c_int64), ("lane_vectors", C.c_int32)]


class DeviceInfo(C.Structure):
    _fields_ = [("device", C.c_int32), ("compute_units", C.c_int32),
                ("max_work_group_size", C.c_int32), ("wavefront_size", C.c_int32),
                ("lds_bytes_per_block", C.c_int64), ("total_global_mem", C.c_int64),
                ("name", C.c_char * 256), ("arch", C.c_char * 64)]


_LIB = None
vp = C.c_void_p
i32, i64, u32, u64 = C.c_int32, C.c_int64, C.c_uint32, C.c_uint64
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")


def lib_path():
    return os.path.join(paths.LIB_DIR, "libcwlb.so")


def _share_torch_hip_runtime():
    """One HIP runtime per process.  torch ships its own libamdhip64 and
    libhsa-runtime64 under the same sonames as ROCm's (libamdhip64.so.7,
    libhsa-runtime64.so.1) and loads them by file name.  Loaded after this
    library, which links ROCm's, they would form a second runtime in the
    process, and whichever initialises the GPU second finds no device
    ("no ROCm-capable device is detected").  Importing torch first makes
    this library bind to the runtime torch has loaded, as it does whenever
    torch is imported before it.  Without torch the library uses ROCm's."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def lib():
    global _LIB
    if _LIB is None:
        path = lib_path()
        if not os.path.exists(path):
            raise RuntimeError(f"{path} missing: build with __graft_entry__.build()")
        _share_torch_hip_runtime()
        L = C.CDLL(path)
        L.cwlb_version.restype = C.c_char_p
        L.cwlb_last_error.restype = C.c_char_p
        L.cwlb_ctx_create.argtypes = [C.c_int, vp, C.POINTER(vp)]
        L.cwlb_ctx_destroy.argtypes = [vp]
        L.cwlb_ctx_set_stream.argtypes = [vp, vp]
        L.cwlb_ctx_synchronize.argtypes = [vp]
        L.cwlb_ctx_device_info.argtypes = [vp, C.POINTER(DeviceInfo)]
        L.cwlb_ctx_set_schedule.argtypes = [vp, i32, i32]
        L.cwlb_ctx_set_locality.argtypes = [vp, i32, i32]
        L.cwlb_ctx_set_cache_hints.argtypes = [vp, i64]
        L.cwlb_ctx_get_cache_hints.argtypes = [vp, C.POINTER(i64)]
        L.cwlb_ctx_last_launch.argtypes = [vp, C.POINTER(LaunchInfo)]
        L.cwlb_ctx_set_occupancy.argtypes = [vp, i32]
        L.cwlb_ctx_get_occupancy.argtypes = [vp, C.POINTER(i32)]
        L.cwlb_ctx_set_column_phases.argtypes = [vp, i32]
        L.cwlb_ctx_get_column_phases.argtypes = [vp, C.POINTER(i32)]
        L.cwlb_ctx_set_lane_tiling.argtypes = [vp, i32]
        L.cwlb_ctx_get_lane_tiling.argtypes = [vp, C.POINTER(i32)]
        L.cwlb_column_phase_sort.argtypes = [vp, vp, vp, vp, i32, i64, i64, i32, vp, vp, vp]
        L.cwlb_ctx_tune_schedule.argtypes = [vp, vp, vp, vp, vp, i32, i64, vp, i64, i32, vp, i64,
                                             vp, i32, C.POINTER(i32), C.POINTER(i32), vp]
        spmm = [vp, vp, vp, vp, vp, i32, i64, vp, i64, i32, vp, i64, vp, u32, C.POINTER(Timing)]
        L.cwlb_spmm_mean_f32.argtypes = spmm
        L.cwlb_spmm_mean_f32_large_k.argtypes = spmm
        L.cwlb_spmm_mean_f32_host.argtypes = [vp, vp, vp, vp, vp, i32, i64, vp, i64, i32, vp, i64,
                                              vp, C.POINTER(Timing)]
        L.cwlb_spmm_mean_f32_noalloc.argtypes = [vp, vp, vp, vp, vp, i32, i64, vp, i64, i32, vp,
                                                 i64, vp, u32, i32, i32, i32]
        L.cwlb_reorder_by_degree.argtypes = [i32, i64, vp, vp, vp, vp, vp, vp, vp]
        L.cwlb_reorder_by_degree_device.argtypes = [vp, i32, i64, vp, vp, vp, vp, vp, vp, vp]
        L.cwlb_partition.argtypes = [vp, i32, C.POINTER(CostParams), C.c_double, vp, i64,
                                     C.POINTER(i64)]
        L.cwlb_partition_device.argtypes = [vp, vp, i32, C.POINTER(CostParams), C.c_double, vp,
                                            i64, C.POINTER(i64)]
        L.cwlb_capacity_from_s.argtypes = [i32, C.POINTER(CostParams)]
        L.cwlb_capacity_from_s.restype = C.c_double
        L.cwlb_wave_based_s.argtypes = [i64, i64, i32, i32, C.POINTER(i32)]
        L.cwlb_recommended_candidate_w.argtypes = [u64, i32p]
        L.cwlb_recommended_candidate_w.restype = None
        L.cwlb_candidate_search_bounds.argtypes = [i32p, i64, C.POINTER(i32), C.POINTER(i32)]
        L.cwlb_candidate_search_by_count.argtypes = [i32, i32, i32, vp, i64, C.POINTER(i64)]
        L.cwlb_candidate_search_by_step.argtypes = [i32, i32, i32, vp, i64, C.POINTER(i64)]
        L.cwlb_calibrate.argtypes = [vp, i32, i32, i32, i32, i32, C.POINTER(CostParams)]
        L.cwlb_calibrate_report.argtypes = [vp, i32, i32, i32, i32, i32, C.POINTER(CostParams),
                                            C.POINTER(CalibrationReport)]
        L.cwlb_save_costs.argtypes = [C.POINTER(CostParams), C.c_char_p, C.c_int, C.c_int]
        L.cwlb_read_costs.argtypes = [C.POINTER(CostParams), C.c_char_p]
        L.cwlb_fill_features_uniform.argtypes = [vp, vp, i64, i32, u64]
        for name in EXPORTS:
            f = getattr(L, name)
            if name not in ("cwlb_version", "cwlb_last_error", "cwlb_capacity_from_s",
                            "cwlb_recommended_candidate_w"):
                f.restype = C.c_int
        _LIB = L
    return _LIB


def check(status):
    if status != OK:
        raise CwlbError(status, lib().cwlb_last_error().decode(errors="replace"))


def version() -> str:
    return lib().cwlb_version().decode()


def _ptr(a):
    """Address of a numpy array or anything with data_ptr() (torch), or an int."""
    if a is None:
        return None
    if isinstance(a, int):
        return a
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    return a.ctypes.data


# ------------------------------------------------------------------ host-side
def partition(row_ptr, costs4, capacity):
    """cwlb_partition -> int32 (T, 4) array."""
    rp = np.ascontiguousarray(row_ptr, np.int32)
    n = len(rp) - 1
    cp = costs(costs4)
    cnt = i64()
    st = lib().cwlb_partition(rp.ctypes.data, n, C.byref(cp), float(capacity), None, 0,
                              C.byref(cnt))
    if st not in (OK, INSUFFICIENT):
        check(st)
    out = np.zeros((max(cnt.value, 1), 4), np.int32)
    check(lib().cwlb_partition(rp.ctypes.data, n, C.byref(cp), float(capacity), out.ctypes.data,
                               cnt.value, C.byref(cnt)))
    return out[:cnt.value].copy()


def reorder_by_degree(row_ptr, col_idx, val):
    rp = np.ascontiguousarray(row_ptr, np.int32)
    ci = np.ascontiguousarray(col_idx, np.int32)
    v = np.ascontiguousarray(val, np.float32)
    n = len(rp) - 1
    origin = np.zeros(max(n, 1), np.int32)
    rp_out = np.zeros(n + 1, np.int32)
    ci_out = np.zeros(max(len(ci), 1), np.int32)
    v_out = np.zeros(max(len(v), 1), np.float32)
    check(lib().cwlb_reorder_by_degree(n, len(ci), rp.ctypes.data, ci.ctypes.data, v.ctypes.data,
                                       origin.ctypes.data, rp_out.ctypes.data, ci_out.ctypes.data,
                                       v_out.ctypes.data))
    return origin[:n], rp_out, ci_out[:len(ci)], v_out[:len(v)]


def capacity_from_s(s, costs4):
    cp = costs(costs4)
    return lib().cwlb_capacity_from_s(int(s), C.byref(cp))


def wave_based_s(nnz, row_ptr_len, cu, wave):
    s = i32()
    check(lib().cwlb_wave_based_s(int(nnz), int(row_ptr_len), int(cu), int(wave), C.byref(s)))
    return s.value


def recommended_candidate_w(nnz):
    out = np.zeros(3, np.int32)
    lib().cwlb_recommended_candidate_w(int(nnz), out)
    return [int(x) for x in out]


def candidate_search_bounds(values, best):
    lo, hi = i32(), i32()
    check(lib().cwlb_candidate_search_bounds(np.asarray(values, np.int32), int(best), C.byref(lo),
                                             C.byref(hi)))
    return lo.value, hi.value


def _search(fn, a, b, c):
    cnt = i64()
    st = fn(int(a), int(b), int(c), None, 0, C.byref(cnt))
    if st not in (OK, INSUFFICIENT):
        check(st)
    out = np.zeros(max(cnt.value, 1), np.int32)
    check(fn(int(a), int(b), int(c), out.ctypes.data, cnt.value, C.byref(cnt)))
    return [int(x) for x in out[:cnt.value]]


def candidate_search_by_count(lo, hi, count):
    return _search(lib().cwlb_candidate_search_by_count, lo, hi, count)


def candidate_search_by_step(lo, hi, step):
    return _search(lib().cwlb_candidate_search_by_step, lo, hi, step)


def save_costs(c4, path, append=False, precision=6):
    cp = costs(c4)
    check(lib().cwlb_save_costs(C.byref(cp), str(path).encode(), int(bool(append)), int(precision)))


def read_costs(path):
    cp = CostParams()
    check(lib().cwlb_read_costs(C.byref(cp), str(path).encode()))
    return cp.tuple4()


# ---------------------------------------------------------------- device-side
def spmm_noalloc(stream, row_ptr, col_idx, val, origin, n_rows, nnz, H, h_rows, K, tasks,
                 n_tasks, C_out, flags=0, tasks_per_wave=0, feature_slices=0, synchronize=True):
    """cwlb_spmm_mean_f32_noalloc on device arrays (no context, nothing
    allocated); stream is a hipStream_t handle (0 = the null stream)."""
    check(lib().cwlb_spmm_mean_f32_noalloc(
        C.c_void_p(stream or None), _ptr(row_ptr), _ptr(col_idx), _ptr(val), _ptr(origin),
        int(n_rows), int(nnz), _ptr(H), int(h_rows), int(K), _ptr(tasks), int(n_tasks),
        _ptr(C_out), int(flags), int(tasks_per_wave), int(feature_slices), int(bool(synchronize))))


class Context:
    """A libcwlb context on one device, launching on `stream` (hipStream_t handle)."""

    def __init__(self, device=0, stream=None):
        self.h = vp()
        check(lib().cwlb_ctx_create(int(device), stream, C.byref(self.h)))

    def close(self):
        if self.h:
            lib().cwlb_ctx_destroy(self.h)
            self.h = vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_stream(self, stream):
        check(lib().cwlb_ctx_set_stream(self.h, stream))

    def set_schedule(self, tasks_per_wave=0, feature_slices=0):
        check(lib().cwlb_ctx_set_schedule(self.h, int(tasks_per_wave), int(feature_slices)))

    def set_locality(self, run_order=0, xcd_blocks=0):
        check(lib().cwlb_ctx_set_locality(self.h, int(run_order), int(xcd_blocks)))

    def set_cache_hints(self, hot_bytes=0):
        check(lib().cwlb_ctx_set_cache_hints(self.h, int(hot_bytes)))

    def cache_hints(self):
        v = i64()
        check(lib().cwlb_ctx_get_cache_hints(self.h, C.byref(v)))
        return v.value

    def last_launch(self):
        """The schedule of the last aggregation launch, as a dict."""
        info = LaunchInfo()
        check(lib().cwlb_ctx_last_launch(self.h, C.byref(info)))
        return {name: getattr(info, name) for name, _ in LaunchInfo._fields_
                if name != "reserved"}

    def set_occupancy(self, waves_per_simd=0):
        check(lib().cwlb_ctx_set_occupancy(self.h, int(waves_per_simd)))

    def occupancy(self):
        v = i32()
        check(lib().cwlb_ctx_get_occupancy(self.h, C.byref(v)))
        return v.value

    def set_lane_tiling(self, tiling=0):
        check(lib().cwlb_ctx_set_lane_tiling(self.h, int(tiling)))

    def lane_tiling(self):
        v = i32()
        check(lib().cwlb_ctx_get_lane_tiling(self.h, C.byref(v)))
        return v.value

    def set_column_phases(self, phases=0):
        check(lib().cwlb_ctx_set_column_phases(self.h, int(phases)))

    def column_phases(self):
        v = i32()
        check(lib().cwlb_ctx_get_column_phases(self.h, C.byref(v)))
        return v.value

    def column_phase_sort(self, row_ptr, col_idx, val, n_rows, nnz, h_rows, phases,
                            bounds_out=None, col_out=None, val_out=None):
        """cwlb_column_phase_sort on device tensors (enqueued on the stream)."""
        check(lib().cwlb_column_phase_sort(self.h, _ptr(row_ptr), _ptr(col_idx), _ptr(val),
                                             int(n_rows), int(nnz), int(h_rows), int(phases),
                                             _ptr(bounds_out), _ptr(col_out), _ptr(val_out)))

    def tune_schedule(self, row_ptr, col_idx, val, origin, n_rows, nnz, H, h_rows, K, tasks,
                      n_tasks, C_out, trials=3, locality=False):
        """cwlb_ctx_tune_schedule: sets and returns the fastest (tasks_per_wave, slices), and
        with locality=True also (run_order, xcd_blocks) as a third element."""
        m, sl = i32(), i32()
        loc = np.zeros(2, np.int32)
        check(lib().cwlb_ctx_tune_schedule(self.h, _ptr(row_ptr), _ptr(col_idx), _ptr(val),
                                           _ptr(origin), int(n_rows), int(nnz), _ptr(H),
                                           int(h_rows), int(K), _ptr(tasks), int(n_tasks),
                                           _ptr(C_out), int(trials), C.byref(m), C.byref(sl),
                                           loc.ctypes.data if locality else None))
        if locality:
            return m.value, sl.value, (int(loc[0]), int(loc[1]))
        return m.value, sl.value

    def synchronize(self):
        check(lib().cwlb_ctx_synchronize(self.h))

    def info(self) -> DeviceInfo:
        d = DeviceInfo()
        check(lib().cwlb_ctx_device_info(self.h, C.byref(d)))
        return d

    def spmm(self, row_ptr, col_idx, val, origin, n_rows, nnz, H, h_rows, K, tasks, n_tasks, C_out,
             flags=0, timed=True, large_k=False):
        """Device-pointer SpMM; returns Timing (synchronous) or None (timed=False)."""
        t = Timing() if timed else None
        fn = lib().cwlb_spmm_mean_f32_large_k if large_k else lib().cwlb_spmm_mean_f32
        check(fn(self.h, _ptr(row_ptr), _ptr(col_idx), _ptr(val), _ptr(origin), int(n_rows),
                 int(nnz), _ptr(H), int(h_rows), int(K), _ptr(tasks), int(n_tasks), _ptr(C_out),
                 int(flags), C.byref(t) if timed else None))
        return t

    def spmm_host(self, row_ptr, col_idx, val, origin, H, tasks):
        """Host-array SpMM (copies in and out); returns (C, Timing)."""
        rp = np.ascontiguousarray(row_ptr, np.int32)
        ci = np.ascontiguousarray(col_idx, np.int32)
        v = np.ascontiguousarray(val, np.float32)
        o = np.ascontiguousarray(origin, np.int32)
        Hh = np.ascontiguousarray(H, np.float32)
        tk = np.ascontiguousarray(tasks, np.int32).reshape(-1, 4)
        n = len(rp) - 1
        K = Hh.shape[1]
        out = np.zeros((n, K), np.float32)
        t = Timing()
        check(lib().cwlb_spmm_mean_f32_host(self.h, rp.ctypes.data, ci.ctypes.data, v.ctypes.data,
                                            o.ctypes.data, n, len(ci), Hh.ctypes.data, Hh.shape[0],
                                            K, tk.ctypes.data, len(tk), out.ctypes.data,
                                            C.byref(t)))
        return out, t

    def reorder_device(self, n_rows, nnz, row_ptr, col_idx, val, origin, rp_out, ci_out, v_out):
        check(lib().cwlb_reorder_by_degree_device(self.h, int(n_rows), int(nnz), _ptr(row_ptr),
                                                  _ptr(col_idx), _ptr(val), _ptr(origin),
                                                  _ptr(rp_out), _ptr(ci_out), _ptr(v_out)))

    def partition_device(self, row_ptr, n_rows, costs4, capacity, out, capacity_tasks):
        """cwlb_partition_device on device arrays; returns the task count."""
        cp = costs(costs4)
        cnt = i64()
        check(lib().cwlb_partition_device(self.h, _ptr(row_ptr), int(n_rows), C.byref(cp),
                                          float(capacity), _ptr(out), int(capacity_tasks),
                                          C.byref(cnt)))
        return cnt.value

    def partition_device_count(self, row_ptr, n_rows, costs4, capacity):
        """Task count only (the INSUFFICIENT sizing call)."""
        cp = costs(costs4)
        cnt = i64()
        st = lib().cwlb_partition_device(self.h, _ptr(row_ptr), int(n_rows), C.byref(cp),
                                         float(capacity), None, 0, C.byref(cnt))
        if st not in (OK, INSUFFICIENT):
            check(st)
        return cnt.value

    def calibrate(self, K=128, repeat=500, WI=131072, load_MB=512, atomic_writers=8):
        cp = CostParams()
        check(lib().cwlb_calibrate(self.h, int(K), int(repeat), int(WI), int(load_MB),
                                   int(atomic_writers), C.byref(cp)))
        return cp

    def calibrate_report(self, K=128, repeat=500, WI=131072, load_MB=512, atomic_writers=8):
        """(CostParams, CalibrationReport): the coefficients and what each was
        computed from (mean launch ms, operation count)."""
        cp, rep = CostParams(), CalibrationReport()
        check(lib().cwlb_calibrate_report(self.h, int(K), int(repeat), int(WI), int(load_MB),
                                          int(atomic_writers), C.byref(cp), C.byref(rep)))
        return cp, rep

    def fill_features(self, H, rows, K, seed=42):
        check(lib().cwlb_fill_features_uniform(self.h, _ptr(H), int(rows), int(K), int(seed)))
