/*
 * config.h -- timing protocol, runtime paths and the dense layout of the
 * C++17 drop-in layer (reference include/config.h:1-25).
 *
 * Same names and values as the reference: 20 warm-up launches out of 70,
 * the cost file and dataset directory relative to the process's working
 * directory (the reference runs from its build/ directory), and the
 * row-major float matrix used for the features H and the output C.
 */
#pragma once

#include <string>

#include "cwlb_dense.h"

// Timed samples = LOOPCOUNT - WARMUPCOUNT; LOOPCOUNT includes the warm-ups.
inline const int WARMUPCOUNT = 20;
inline const int LOOPCOUNT = 70;
inline const std::string COSTFILEPATH = "../resources/spmm_costs.txt";

constexpr const char* DATA_CSR_FILE_PATH = "../resources/datasets/";

namespace Defined {
// Adjacent feature columns are contiguous: row r of H at data() + r * cols().
using RowMajorMatrixXf = cwlb::RowMajorMatrix<float>;
}  // namespace Defined
