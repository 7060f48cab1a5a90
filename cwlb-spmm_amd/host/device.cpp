// cwlb::Device: the sycl::queue replacement of the drop-in layer.
#include <new>
#include <stdexcept>
#include <string>
#include <utility>

#include "cwlb_device.h"

namespace cwlb {

void throw_status(cwlb_status st, const std::string& context)
{
    const std::string msg = cwlb_last_error();
    const std::string text = msg.empty() ? context : msg;
    switch (st) {
    case CWLB_INVALID_ARG:
        throw std::invalid_argument(text);
    case CWLB_OOM:
        throw std::bad_alloc();
    default:
        throw std::runtime_error(text);
    }
}

Device::Device(int device, void* hip_stream)
{
    check(cwlb_ctx_create(device, hip_stream, &ctx_), "cwlb_ctx_create");
    const cwlb_status st = cwlb_ctx_device_info(ctx_, &info_);
    if (st != CWLB_OK) {
        cwlb_ctx_destroy(ctx_);
        ctx_ = nullptr;
        throw_status(st, "cwlb_ctx_device_info");
    }
}

Device::~Device()
{
    if (ctx_) cwlb_ctx_destroy(ctx_);
}

Device::Device(Device&& other) noexcept : ctx_(other.ctx_), info_(other.info_)
{
    other.ctx_ = nullptr;
}

Device& Device::operator=(Device&& other) noexcept
{
    if (this != &other) {
        if (ctx_) cwlb_ctx_destroy(ctx_);
        ctx_ = other.ctx_;
        info_ = other.info_;
        other.ctx_ = nullptr;
    }
    return *this;
}

void Device::wait() { check(cwlb_ctx_synchronize(ctx_), "cwlb_ctx_synchronize"); }

}  // namespace cwlb
