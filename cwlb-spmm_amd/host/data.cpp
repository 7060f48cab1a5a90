// Text-CSR dataset loader of the drop-in layer (reference src/data.cpp:10-130).
#include <fstream>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "config.h"
#include "data.h"

namespace {

// Appends every non-empty comma-separated cell of `line`, parsed as std::stoi
// does (leading blanks skipped, trailing characters ignored).
void parse_int_list(const std::string& line, std::vector<int>& out)
{
    std::stringstream cells(line);
    std::string cell;
    while (std::getline(cells, cell, ','))
        if (!cell.empty()) out.push_back(std::stoi(cell));
}

void check_csr(const CSR& csr, const std::string& path, int& V, int& E)
{
    if (csr.RowOffset.empty()) throw std::runtime_error(".csr file has an empty RowOffset: " + path);
    V = static_cast<int>(csr.RowOffset.size()) - 1;
    E = csr.RowOffset.back();
    if (V < 0) throw std::runtime_error("Invalid RowOffset size. It should be vertex_count + 1");
    if (E < 0) throw std::runtime_error("RowOffset.back(), namely NNZ, is negative");
    if (static_cast<int>(csr.ColInd.size()) != E)
        throw std::runtime_error("ColInd size does not match RowOffset.back()(NNZ): ColInd=" +
                                 std::to_string(csr.ColInd.size()) + ", NNZ=" + std::to_string(E));
    if (csr.RowOffset.front() != 0)
        throw std::runtime_error("RowOffset[0] must be 0, current value is " +
                                 std::to_string(csr.RowOffset.front()));
    for (std::size_t i = 1; i < csr.RowOffset.size(); ++i) {
        if (csr.RowOffset[i] < csr.RowOffset[i - 1])
            throw std::runtime_error("RowOffset is not monotonically non-decreasing at index " +
                                     std::to_string(i));
        if (csr.RowOffset[i] > E)
            throw std::runtime_error("RowOffset contains a value larger than NNZ at index " +
                                     std::to_string(i));
    }
    for (int c : csr.ColInd)
        if (c < 0) throw std::runtime_error("ColInd contains a negative column index");
}

}  // namespace

CSR loadDatasetToCSR(const std::string& datasetName, int& V, int& E)
{
    if (datasetName.empty()) throw std::runtime_error("Dataset name is empty");
    const std::string ext = ".csr";
    const bool has_ext = datasetName.size() >= ext.size() &&
                         datasetName.compare(datasetName.size() - ext.size(), ext.size(), ext) == 0;
    const std::string path = DATA_CSR_FILE_PATH + (has_ext ? datasetName : datasetName + ext);

    std::ifstream in(path);
    if (!in.is_open()) throw std::runtime_error("Failed to open .csr file: " + path);
    CSR csr;
    std::string line;
    if (!std::getline(in, line))
        throw std::runtime_error("Failed to read the first line of .csr file: " + path);
    parse_int_list(line, csr.RowOffset);
    if (!std::getline(in, line))
        throw std::runtime_error("Failed to read the second line of .csr file: " + path);
    parse_int_list(line, csr.ColInd);
    check_csr(csr, path, V, E);
    csr.Value.assign(csr.ColInd.size(), 1.0f);
    return csr;
}
