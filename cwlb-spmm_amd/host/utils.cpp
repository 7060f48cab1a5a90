// Task partitioning, calibration, cost file, GPU reordering and the result
// validator of the drop-in layer (reference src/utils.cpp).  The numeric
// work is in the C ABI (include/cwlb.h); this file adapts the types.
#include <algorithm>
#include <cmath>
#include <iomanip>
#include <iostream>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

#include "host_internal.h"
#include "utils.h"

using cwlb::host::DeviceArray;

CSR_Order sortCSRByDegree_HIP(const CSR& csr, cwlb::Device& q)
{
    CSR_Order out;
    if (csr.RowOffset.size() < 2) return out;
    if (csr.ColInd.size() != csr.Value.size())
        throw std::runtime_error("CSR ColInd and Value size mismatch.");
    const std::size_t rows = csr.RowOffset.size() - 1;
    const std::size_t nnz = csr.ColInd.size();
    if (rows > static_cast<std::size_t>(std::numeric_limits<int>::max()) ||
        nnz > static_cast<std::size_t>(std::numeric_limits<int>::max()))
        throw std::overflow_error("GPU degree reordering requires row and NNZ counts to fit in int.");
    cwlb::host::CurrentDevice cur(q);
    DeviceArray<int> rp(rows + 1), ci(nnz), o(rows), rp2(rows + 1), ci2(nnz);
    DeviceArray<float> v(nnz), v2(nnz);
    rp.upload(csr.RowOffset);
    ci.upload(csr.ColInd);
    v.upload(csr.Value);
    cwlb::check(cwlb_reorder_by_degree_device(q.ctx(), static_cast<int32_t>(rows),
                                              static_cast<int64_t>(nnz), rp.get(), ci.get(),
                                              v.get(), o.get(), rp2.get(), ci2.get(), v2.get()),
                "sortCSRByDegree_HIP");
    out.Origin_local.resize(rows);
    out.RowOffset.resize(rows + 1);
    out.ColInd.resize(nnz);
    out.Value.resize(nnz);
    o.download(out.Origin_local.data(), rows);
    rp2.download(out.RowOffset.data(), rows + 1);
    ci2.download(out.ColInd.data(), nnz);
    v2.download(out.Value.data(), nnz);
    return out;
}

SpmmCostParams measure_spmm_costs(cwlb::Device& q, int K, int repeat, int WI, int data_MB_for_load,
                                  int atomic_target_writers, const std::vector<int>&)
{
    cwlb_cost_params p{};
    cwlb::check(cwlb_calibrate(q.ctx(), K, repeat, WI, data_MB_for_load, atomic_target_writers, &p),
                "measure_spmm_costs");
    return cwlb::host::from_c(p);
}

std::vector<ParallelDataWeighted> costWeightedTaskPartitioning(const CSR_Order& csr,
                                                               const SpmmCostParams& costs,
                                                               double capacity_weight)
{
    std::vector<ParallelDataWeighted> tasks;
    const int n = static_cast<int>(csr.RowOffset.size()) - 1;
    if (n <= 0) return tasks;
    const cwlb_cost_params c = cwlb::host::to_c(costs);
    int64_t count = 0;
    cwlb_status st = cwlb_partition(csr.RowOffset.data(), n, &c, capacity_weight, nullptr, 0, &count);
    if (st != CWLB_OK && st != CWLB_INSUFFICIENT) cwlb::throw_status(st, "costWeightedTaskPartitioning");
    tasks.resize(static_cast<std::size_t>(count));
    if (count == 0) return tasks;
    st = cwlb_partition(csr.RowOffset.data(), n, &c, capacity_weight,
                        reinterpret_cast<cwlb_task*>(tasks.data()), count, &count);
    cwlb::check(st, "costWeightedTaskPartitioning");
    return tasks;
}

std::vector<ParallelDataWeighted> costWeightedTaskPartitioning_HIP(const CSR_Order& csr,
                                                                   const SpmmCostParams& costs,
                                                                   double capacity_weight,
                                                                   cwlb::Device& q)
{
    const int n = static_cast<int>(csr.RowOffset.size()) - 1;
    if (n <= 0) return {};
    cwlb::host::CurrentDevice cur(q);
    DeviceArray<int> rp(csr.RowOffset.size());
    rp.upload(csr.RowOffset);
    const cwlb_cost_params c = cwlb::host::to_c(costs);
    int64_t count = 0;
    cwlb_status st = cwlb_partition_device(q.ctx(), rp.get(), n, &c, capacity_weight, nullptr, 0,
                                           &count);
    if (st == CWLB_UNSUPPORTED) return costWeightedTaskPartitioning(csr, costs, capacity_weight);
    if (st != CWLB_OK && st != CWLB_INSUFFICIENT) cwlb::throw_status(st, "costWeightedTaskPartitioning_HIP");
    std::vector<ParallelDataWeighted> tasks(static_cast<std::size_t>(count));
    if (count == 0) return tasks;
    DeviceArray<cwlb_task> out(static_cast<std::size_t>(count));
    cwlb::check(cwlb_partition_device(q.ctx(), rp.get(), n, &c, capacity_weight, out.get(), count,
                                      &count),
                "costWeightedTaskPartitioning_HIP");
    out.download(reinterpret_cast<cwlb_task*>(tasks.data()), tasks.size());
    return tasks;
}

bool save_costs_one_per_line(SpmmCostParams costs, const std::string& filepath, bool append,
                             int precision)
{
    if (filepath.empty()) return false;
    const cwlb_cost_params c = cwlb::host::to_c(costs);
    return cwlb_save_costs(&c, filepath.c_str(), append ? 1 : 0, precision) == CWLB_OK;
}

bool read_costs_one_per_line(SpmmCostParams& out, const std::string& filepath)
{
    cwlb_cost_params c = cwlb::host::to_c(out);
    if (cwlb_read_costs(&c, filepath.c_str()) != CWLB_OK) return false;
    out.C_compute_ns = c.C_compute_ns;
    out.C_load_ns = c.C_load_ns;
    out.C_store_ns = c.C_store_ns;
    out.C_atomic_ns = c.C_atomic_ns;
    return true;
}

std::vector<std::pair<int, float>> get_csr_row_elements(const CSR& csr, int row)
{
    std::vector<std::pair<int, float>> out;
    const int rows = static_cast<int>(csr.RowOffset.size()) - 1;
    if (row < 0 || row >= rows) return out;
    const int b = csr.RowOffset[row];
    const int e = csr.RowOffset[row + 1];
    out.reserve(static_cast<std::size_t>(std::max(0, e - b)));
    for (int j = b; j < e; ++j) out.emplace_back(csr.ColInd[j], csr.Value[j]);
    return out;
}

namespace {

// Mismatch rule of the validator: NaN only matches NaN, an infinity only
// the same infinity, finite values within abs_tolerance.
bool mismatch(float got, float want, float tol, float& abs_err)
{
    if (std::isnan(got) || std::isnan(want)) {
        const bool bad = !(std::isnan(got) && std::isnan(want));
        abs_err = bad ? std::numeric_limits<float>::infinity() : 0.0f;
        return bad;
    }
    if (std::isinf(got) || std::isinf(want)) {
        const bool bad = got != want;
        abs_err = bad ? std::numeric_limits<float>::infinity() : 0.0f;
        return bad;
    }
    abs_err = std::abs(got - want);
    return abs_err > tol;
}

void print_error(const ErrorElement& e, std::size_t number, const CSR& csr)
{
    std::cout << "\nStored entries in CSR row " << e.result_row << ":\n"
              << "RowOffset[" << e.result_row << "]: " << csr.RowOffset[e.result_row] << '\n'
              << "RowOffset[" << e.result_row + 1 << "]: " << csr.RowOffset[e.result_row + 1]
              << '\n'
              << "Format: [ColInd] -> Value\n";
    for (const auto& el : e.csr_row_elements)
        std::cout << "  [" << el.first << "] -> " << el.second << '\n';
    std::cout << "\nDense matrix column " << e.result_col << " (up to the first 5 rows):\n";
    const std::size_t shown = std::min<std::size_t>(5, e.dense_col_elements.size());
    for (std::size_t r = 0; r < shown; ++r)
        std::cout << "  Row " << r << ": " << e.dense_col_elements[r] << '\n';
    std::cout << "\n\033[1;34mMismatch #" << number << ":\033[0m\n"
              << "Result matrix position: (" << e.result_row << ", " << e.result_col << ")\n"
              << std::fixed << std::setprecision(6) << "SYCL result:     " << e.sycl_value << '\n'
              << "Reference value: " << e.reference_value << '\n'
              << "Absolute error:  " << e.absolute_error << '\n';
}

}  // namespace

bool validate_custom_csr_result(const Defined::RowMajorMatrixXf& result,
                                const Defined::RowMajorMatrixXf& reference, const CSR& csr,
                                const Defined::RowMajorMatrixXf& dense, float tol)
{
    try {
        if (tol < 0.0f || !std::isfinite(tol))
            throw std::invalid_argument("Validation tolerance must be finite and non-negative.");
        if (result.rows() != reference.rows() || result.cols() != reference.cols()) {
            std::cerr << "Validation failed: result matrix shape is (" << result.rows() << ", "
                      << result.cols() << "), but reference matrix shape is (" << reference.rows()
                      << ", " << reference.cols() << ").\n";
            return false;
        }
        if (csr.RowOffset.size() != static_cast<std::size_t>(reference.rows()) + 1) {
            std::cerr << "Validation failed: CSR row count does not match the reference matrix.\n";
            return false;
        }
        if (dense.rows() <= 0 || dense.cols() != reference.cols()) {
            std::cerr << "Validation failed: input dense matrix shape is incompatible with the "
                         "reference result.\n";
            return false;
        }
        constexpr std::size_t kMaxReported = 10;
        std::vector<ErrorElement> errors;
        for (long r = 0; r < reference.rows() && errors.size() < kMaxReported; ++r) {
            for (long c = 0; c < reference.cols() && errors.size() < kMaxReported; ++c) {
                float err = 0.0f;
                if (!mismatch(result(r, c), reference(r, c), tol, err)) continue;
                ErrorElement e;
                e.result_row = static_cast<int>(r);
                e.result_col = static_cast<int>(c);
                e.sycl_value = result(r, c);
                e.reference_value = reference(r, c);
                e.absolute_error = err;
                e.csr_row_elements = get_csr_row_elements(csr, static_cast<int>(r));
                e.dense_col_elements.resize(static_cast<std::size_t>(dense.rows()));
                for (long d = 0; d < dense.rows(); ++d)
                    e.dense_col_elements[static_cast<std::size_t>(d)] = dense(d, c);
                errors.push_back(std::move(e));
            }
        }
        if (errors.empty()) {
            std::cout << "\033[1;32mValidation passed: all elements satisfy the comparison "
                         "criteria.\033[0m\n";
            return true;
        }
        std::cout << "\033[1;31mValidation failed: showing " << errors.size()
                  << " mismatched elements (up to the first 10).\033[0m\n";
        for (std::size_t i = 0; i < errors.size(); ++i) print_error(errors[i], i + 1, csr);
        return false;
    } catch (const std::exception& e) {
        std::cerr << "Validation error: " << e.what() << '\n';
        return false;
    }
}
