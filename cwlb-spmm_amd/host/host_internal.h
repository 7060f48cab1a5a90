// Internal helpers of the C++17 drop-in layer: device arrays (RAII over the
// HIP runtime) and the task-type bridge to the C ABI.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <new>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <vector>

#include "cwlb.h"
#include "cwlb_device.h"
#include "utils.h"

static_assert(sizeof(ParallelDataWeighted) == sizeof(cwlb_task) &&
                  alignof(ParallelDataWeighted) == alignof(cwlb_task) &&
                  std::is_standard_layout<ParallelDataWeighted>::value,
              "ParallelDataWeighted must match cwlb_task field for field");

namespace cwlb {
namespace host {

inline void hip_check(hipError_t e, const char* what)
{
    if (e == hipSuccess) return;
    if (e == hipErrorOutOfMemory) throw std::bad_alloc();
    throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// Makes q's device current for the lifetime of the guard.
class CurrentDevice {
public:
    explicit CurrentDevice(const Device& q)
    {
        hip_check(hipGetDevice(&prev_), "hipGetDevice");
        if (prev_ != q.ordinal()) hip_check(hipSetDevice(q.ordinal()), "hipSetDevice");
    }
    ~CurrentDevice() { (void)hipSetDevice(prev_); }
    CurrentDevice(const CurrentDevice&) = delete;
    CurrentDevice& operator=(const CurrentDevice&) = delete;

private:
    int prev_ = 0;
};

// A device array of n elements of T (at least one element is allocated so
// that the pointer is never null).
template <class T>
class DeviceArray {
public:
    DeviceArray() = default;
    explicit DeviceArray(std::size_t n) { allocate(n); }
    ~DeviceArray() { release(); }
    DeviceArray(const DeviceArray&) = delete;
    DeviceArray& operator=(const DeviceArray&) = delete;

    void allocate(std::size_t n)
    {
        release();
        hip_check(hipMalloc(reinterpret_cast<void**>(&p_), sizeof(T) * (n ? n : 1)), "hipMalloc");
        n_ = n;
    }
    void release()
    {
        if (p_) (void)hipFree(p_);
        p_ = nullptr;
        n_ = 0;
    }
    T* get() const { return p_; }
    std::size_t size() const { return n_; }

    void upload(const T* src, std::size_t n)
    {
        if (n > n_) throw std::logic_error("DeviceArray::upload beyond the allocation");
        if (n) hip_check(hipMemcpy(p_, src, sizeof(T) * n, hipMemcpyHostToDevice), "hipMemcpy H2D");
    }
    void download(T* dst, std::size_t n) const
    {
        if (n > n_) throw std::logic_error("DeviceArray::download beyond the allocation");
        if (n) hip_check(hipMemcpy(dst, p_, sizeof(T) * n, hipMemcpyDeviceToHost), "hipMemcpy D2H");
    }
    void upload(const std::vector<T>& v) { upload(v.data(), v.size()); }

private:
    T* p_ = nullptr;
    std::size_t n_ = 0;
};

inline const cwlb_task* as_c_tasks(const std::vector<ParallelDataWeighted>& t)
{
    return reinterpret_cast<const cwlb_task*>(t.data());
}

inline cwlb_cost_params to_c(const SpmmCostParams& c)
{
    cwlb_cost_params p{};
    p.C_compute_ns = c.C_compute_ns;
    p.C_load_ns = c.C_load_ns;
    p.C_store_ns = c.C_store_ns;
    p.C_atomic_ns = c.C_atomic_ns;
    p.K = c.K;
    p.WI = c.WI;
    p.repeat = c.repeat;
    p.atomic_writers_per_addr = c.atomic_writers_per_addr;
    return p;
}

inline SpmmCostParams from_c(const cwlb_cost_params& p)
{
    SpmmCostParams c;
    c.C_compute_ns = p.C_compute_ns;
    c.C_load_ns = p.C_load_ns;
    c.C_store_ns = p.C_store_ns;
    c.C_atomic_ns = p.C_atomic_ns;
    c.K = p.K;
    c.WI = p.WI;
    c.repeat = p.repeat;
    c.atomic_writers_per_addr = p.atomic_writers_per_addr;
    return c;
}

}  // namespace host
}  // namespace cwlb
