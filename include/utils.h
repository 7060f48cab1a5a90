/*
 * utils.h -- task and cost types, cost calibration, cost-weighted
 * partitioning, the cost file and the result validator of the C++17 drop-in
 * layer (reference include/utils.h:1-83).
 *
 * Same names, fields, defaults and return conventions as the reference; the
 * sycl::queue& parameters become cwlb::Device& (include/cwlb_device.h).
 */
#pragma once

#include <string>
#include <utility>
#include <vector>

#include "Matrix.h"
#include "config.h"
#include "cwlb_device.h"

// Degree reordering on the GPU: the permutation, offsets and row copies of
// sortCSRByDegreeDPLCPU (reference main.cpp:197-278), computed on the
// device with a stable sort by degree, so ties keep the original row order
// and the result is identical to the host reordering.  Takes the place of
// the reference's optional sortCSRByDegree_SYCL (include/utils.h:12-13),
// whose atomic scatter leaves equal-degree rows in no fixed order.
CSR_Order sortCSRByDegree_HIP(const CSR& csr, cwlb::Device& q);

// One task: the half-open reordered-row range [row_start, row_end); the
// first row starts at nonzero first_row_offset, the last row ends at
// nonzero last_row_nnz (0 = its full degree).  Layout-identical to
// cwlb_task (include/cwlb.h).
struct ParallelDataWeighted {
    int row_start;
    int row_end;
    int first_row_offset;
    int last_row_nnz;
};

// Calibrated relative operation weights and calibration metadata.
struct SpmmCostParams {
    double C_compute_ns = 0.0;
    double C_load_ns = 0.0;
    double C_store_ns = 0.0;
    double C_atomic_ns = 0.0;

    int K = 0;
    int WI = 0;
    int repeat = 0;
    int atomic_writers_per_addr = 0;
};

// One mismatch retained by validate_custom_csr_result.  The field names are
// the reference's (sycl_value is the device result).
struct ErrorElement {
    int result_row = 0;
    int result_col = 0;
    float sycl_value = 0.0f;
    float reference_value = 0.0f;
    float absolute_error = 0.0f;
    std::vector<std::pair<int, float>> csr_row_elements;
    std::vector<float> dense_col_elements;
};

// Calibrates the compute, load, direct-store and atomic-update weights on
// the device (reference src/utils.cpp:342-829), re-measured on gfx950.
// atomic_group_candidates is accepted and ignored, as in the reference
// (src/utils.cpp:360).  Throws std::invalid_argument for non-positive
// parameters.
SpmmCostParams measure_spmm_costs(cwlb::Device& q, int K = 128, int repeat = 500,
                                  int WI = 131072, int data_MB_for_load = 512,
                                  int atomic_target_writers = 8,
                                  const std::vector<int>& atomic_group_candidates = {});

// Packs complete rows and splits oversized rows under the weighted capacity
// (reference src/utils.cpp:832-1021); bit-identical task lists.
std::vector<ParallelDataWeighted> costWeightedTaskPartitioning(const CSR_Order& csr,
                                                               const SpmmCostParams& costs,
                                                               double capacity_weight);

// The same partition computed on the GPU (cwlb_partition_device): the
// RowOffset array is copied to the device, the task list back.  Costs under
// which a task's row count has no bound (see include/cwlb.h) are partitioned
// on the host instead; the result is identical either way.
std::vector<ParallelDataWeighted> costWeightedTaskPartitioning_HIP(const CSR_Order& csr,
                                                                   const SpmmCostParams& costs,
                                                                   double capacity_weight,
                                                                   cwlb::Device& q);

// Cost-file order: compute, load, store, atomic; one per line, fixed
// notation (reference src/utils.cpp:1024-1092).  Both return false on any
// failure instead of throwing.
bool save_costs_one_per_line(SpmmCostParams costs, const std::string& filepath = COSTFILEPATH,
                             bool append = false, int precision = 6);
bool read_costs_one_per_line(SpmmCostParams& out, const std::string& filepath = COSTFILEPATH);

// (column, value) pairs of CSR row `row`; empty for a row out of range
// (reference src/utils.cpp:1095-1115).
std::vector<std::pair<int, float>> get_csr_row_elements(const CSR& csr, int row);

// Compares a result with a caller-supplied reference under an absolute
// tolerance; NaN matches NaN and an infinity matches the same infinity;
// prints up to 10 mismatches with their CSR row and dense column (reference
// src/utils.cpp:1117-1265).
bool validate_custom_csr_result(const Defined::RowMajorMatrixXf& sycl_result,
                                const Defined::RowMajorMatrixXf& reference, const CSR& csr,
                                const Defined::RowMajorMatrixXf& dense_matrix,
                                float abs_tolerance = 1e-4f);
