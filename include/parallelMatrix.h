/*
 * parallelMatrix.h -- the SpMM entry points of the C++17 drop-in layer
 * (reference include/parallelMatrix.h:11-32).
 *
 * Both compute the mean aggregation of a degree-reordered CSR over a
 * cost-weighted task list and return C in ORIGINAL row order:
 *     C[Origin_local[r]] = (sum_j Value[j] * H[ColInd[j]]) / deg(r),
 * a row of degree 0 giving zeros.  The host matrices are copied to the
 * device per call and C is copied back, as the reference's per-call
 * sycl::buffers do (src/parallelMatrix.cpp:115-121); `time` receives the
 * aggregation kernel's duration in microseconds (HIP events), transfers
 * excluded.  K = H.cols() == 0 or an empty task list gives a zero matrix
 * and time 0.
 *
 * dim_hint and local_dimension are accepted and ignored: the gfx950 kernel
 * sizes its own tiles (the reference uses local_dimension only as its
 * local-memory tile length, and its large-K form ignores both).
 *
 * spmmKernel throws std::invalid_argument for K > the device's maximum
 * work-group size (1024), spmmKernelLargeKFallback for K <= it, with the
 * reference's messages (src/parallelMatrix.cpp:84-88, 287-290).  Both
 * throw std::invalid_argument for inconsistent inputs (RowOffset size,
 * ColInd/Value sizes, a column index outside [0, H.rows())).
 */
#pragma once

#include <vector>

#include "Matrix.h"
#include "config.h"
#include "cwlb_device.h"
#include "utils.h"

Defined::RowMajorMatrixXf spmmKernel(cwlb::Device& q, const CSR_Order& adjOrder,
                                     const Defined::RowMajorMatrixXf& H, int dim_hint,
                                     int local_dimension, std::vector<ParallelDataWeighted> tasks,
                                     double& time);

Defined::RowMajorMatrixXf spmmKernelLargeKFallback(cwlb::Device& q, const CSR_Order& adjOrder,
                                                   const Defined::RowMajorMatrixXf& H,
                                                   int dim_hint, int local_dimension,
                                                   std::vector<ParallelDataWeighted> tasks,
                                                   double& time);
