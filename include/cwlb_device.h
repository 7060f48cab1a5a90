/*
 * cwlb_device.h -- the device handle of the C++17 drop-in layer.
 *
 * The reference passes a sycl::queue created with the GPU selector and
 * event profiling (main.cpp:514-516, weightCost.cpp:44-46) and reads
 * max_compute_units, max_work_group_size, local_mem_size and the device name
 * from it (main.cpp:535-536, src/parallelMatrix.cpp:76-77,349-350).
 * cwlb::Device is that handle for one HIP device and stream: it owns a
 * cwlb_ctx (include/cwlb.h) and is what every drop-in entry point takes in
 * place of sycl::queue&.  Construction fails with std::runtime_error when
 * no gfx950 device is available.
 *
 * Errors of the C ABI become the reference's exception types:
 * CWLB_INVALID_ARG -> std::invalid_argument, CWLB_OOM -> std::bad_alloc,
 * anything else -> std::runtime_error (message from cwlb_last_error()).
 */
#pragma once

#include <string>

#include "cwlb.h"

namespace cwlb {

[[noreturn]] void throw_status(cwlb_status st, const std::string& context);

// Throws the mapped exception unless st == CWLB_OK.
inline void check(cwlb_status st, const char* context)
{
    if (st != CWLB_OK) throw_status(st, context);
}

class Device {
public:
    // Device `device` (HIP ordinal), launching on `hip_stream` (a
    // hipStream_t; nullptr = the null stream).
    explicit Device(int device = 0, void* hip_stream = nullptr);
    ~Device();
    Device(const Device&) = delete;
    Device& operator=(const Device&) = delete;
    Device(Device&& other) noexcept;
    Device& operator=(Device&& other) noexcept;

    cwlb_ctx* ctx() const { return ctx_; }
    int ordinal() const { return info_.device; }
    int max_compute_units() const { return info_.compute_units; }
    int max_work_group_size() const { return info_.max_work_group_size; }
    int wavefront_size() const { return info_.wavefront_size; }
    long long local_mem_size() const { return info_.lds_bytes_per_block; }
    long long global_mem_size() const { return info_.total_global_mem; }
    std::string name() const { return info_.name; }
    std::string arch() const { return info_.arch; }

    // Blocks until the device's stream is idle (sycl::queue::wait).
    void wait();

private:
    cwlb_ctx* ctx_ = nullptr;
    cwlb_device_info info_{};
};

}  // namespace cwlb
