/*
 * Matrix.h -- the sparse types of the C++17 drop-in layer (reference
 * include/Matrix.h:15-36).
 *
 * CSR: RowOffset[n + 1], ColInd[nnz], Value[nnz] (int32 / float32).
 * CSR_Order: the degree-reordered CSR plus Origin_local, where
 * Origin_local[r] is the original row id of reordered row r; the SpMM writes
 * row r's result to C[Origin_local[r]].
 */
#pragma once

#include <vector>

#include "config.h"

class CSR {
public:
    std::vector<int> RowOffset;
    std::vector<int> ColInd;
    std::vector<float> Value;

    // Dense square adjacency to CSR, nonzeros in row-major order
    // (reference src/Matrix.cpp:14-52).  Throws std::invalid_argument when
    // adj is not square.
    explicit CSR(const Defined::RowMajorMatrixXf& adj);
    CSR(std::vector<int> RowOffset, std::vector<int> ColInd, std::vector<float> Value);
    CSR() {}
    ~CSR() {}
};

class CSR_Order {
public:
    std::vector<int> Origin_local;  // reordered row -> original row id
    std::vector<int> RowOffset;
    std::vector<int> ColInd;
    std::vector<float> Value;
};
