// spmmKernel / spmmKernelLargeKFallback of the drop-in layer (reference
// src/parallelMatrix.cpp:63-683) over the host-pointer C entry point.
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "host_internal.h"
#include "parallelMatrix.h"

namespace {

void check_inputs(const CSR_Order& a, const Defined::RowMajorMatrixXf& H)
{
    if (a.RowOffset.size() != a.Origin_local.size() + 1)
        throw std::invalid_argument("spmm: RowOffset must have Origin_local.size() + 1 entries");
    if (a.ColInd.size() != a.Value.size())
        throw std::invalid_argument("spmm: ColInd and Value sizes differ");
    if (a.ColInd.size() > static_cast<std::size_t>(INT32_MAX) ||
        a.Origin_local.size() > static_cast<std::size_t>(INT32_MAX) || H.cols() > INT32_MAX)
        throw std::invalid_argument("spmm: sizes must fit int32");
}

Defined::RowMajorMatrixXf run(cwlb::Device& q, const CSR_Order& a,
                              const Defined::RowMajorMatrixXf& H,
                              const std::vector<ParallelDataWeighted>& tasks, double& time)
{
    check_inputs(a, H);
    const auto rows = static_cast<Defined::RowMajorMatrixXf::Index>(a.Origin_local.size());
    Defined::RowMajorMatrixXf C(rows, H.cols());
    cwlb_timing t{};
    cwlb::check(cwlb_spmm_mean_f32_host(
                    q.ctx(), a.RowOffset.data(), a.ColInd.data(), a.Value.data(),
                    a.Origin_local.data(), static_cast<int32_t>(rows),
                    static_cast<int64_t>(a.ColInd.size()), H.data(), static_cast<int64_t>(H.rows()),
                    static_cast<int32_t>(H.cols()), cwlb::host::as_c_tasks(tasks),
                    static_cast<int64_t>(tasks.size()), C.data(), &t),
                "spmmKernel");
    time = static_cast<double>(t.main_us);
    return C;
}

Defined::RowMajorMatrixXf zero_result(const CSR_Order& a, const Defined::RowMajorMatrixXf& H,
                                      double& time)
{
    time = 0.0;
    return Defined::RowMajorMatrixXf::Zero(
        static_cast<Defined::RowMajorMatrixXf::Index>(a.Origin_local.size()), H.cols());
}

}  // namespace

Defined::RowMajorMatrixXf spmmKernel(cwlb::Device& q, const CSR_Order& adjOrder,
                                     const Defined::RowMajorMatrixXf& H, int, int,
                                     std::vector<ParallelDataWeighted> tasks, double& time)
{
    const long long K = H.cols();
    if (K == 0) return zero_result(adjOrder, H, time);
    if (K > q.max_work_group_size())
        throw std::invalid_argument(
            "spmmKernel supports only K <= device max work-group size; "
            "use spmmKernelLargeKFallback for larger K.");
    if (tasks.empty()) return zero_result(adjOrder, H, time);
    return run(q, adjOrder, H, tasks, time);
}

Defined::RowMajorMatrixXf spmmKernelLargeKFallback(cwlb::Device& q, const CSR_Order& adjOrder,
                                                   const Defined::RowMajorMatrixXf& H, int, int,
                                                   std::vector<ParallelDataWeighted> tasks,
                                                   double& time)
{
    if (q.max_work_group_size() == 0)
        throw std::runtime_error("Large-K fallback cannot use a device with max_work_group_size=0.");
    if (H.cols() <= q.max_work_group_size())
        throw std::invalid_argument(
            "spmmKernelLargeKFallback requires K > device max work-group size.");
    if (tasks.empty()) return zero_result(adjOrder, H, time);
    return run(q, adjOrder, H, tasks, time);
}
