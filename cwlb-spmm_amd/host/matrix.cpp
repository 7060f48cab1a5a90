// CSR constructors of the drop-in layer (reference src/Matrix.cpp:14-58).
#include <iostream>
#include <stdexcept>
#include <utility>

#include "Matrix.h"

CSR::CSR(const Defined::RowMajorMatrixXf& adj)
{
    std::cout << "Converting the dense adjacency matrix to CSR." << std::endl;
    if (adj.rows() != adj.cols()) throw std::invalid_argument("Adjacency matrix must be square");
    const auto n = adj.rows();
    RowOffset.reserve(static_cast<std::size_t>(n) + 1);
    RowOffset.push_back(0);
    for (decltype(adj.rows()) i = 0; i < n; ++i) {
        for (decltype(adj.rows()) j = 0; j < n; ++j) {
            const float a = adj(i, j);
            if (a != 0.0f) {
                ColInd.push_back(static_cast<int>(j));
                Value.push_back(a);
            }
        }
        RowOffset.push_back(static_cast<int>(ColInd.size()));
    }
}

CSR::CSR(std::vector<int> row_offset, std::vector<int> col_ind, std::vector<float> value)
    : RowOffset(std::move(row_offset)), ColInd(std::move(col_ind)), Value(std::move(value))
{
}
