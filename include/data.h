/*
 * data.h -- the text-CSR dataset loader of the C++17 drop-in layer
 * (reference include/data.h:8, src/data.cpp:10-130).
 *
 * File DATA_CSR_FILE_PATH + name (".csr" appended when missing): line 1 the
 * comma-separated row offsets, line 2 the comma-separated column indices;
 * empty cells are skipped.  Values are all 1.0f.  V = offsets - 1,
 * E = last offset.  Throws std::runtime_error (with the reference's
 * messages) for an empty name, a missing file or line, an empty offset
 * list, a negative NNZ, a column count != NNZ, RowOffset[0] != 0,
 * decreasing offsets, an offset > NNZ or a negative column; std::stoi's
 * std::invalid_argument / std::out_of_range for a cell that is not an int.
 */
#pragma once

#include <string>

#include "Matrix.h"

CSR loadDatasetToCSR(const std::string& datasetName, int& V, int& E);
