/*
 * cwlb_dense.h -- the dense row-major matrix of the C++17 drop-in layer.
 *
 * The reference stores H and C as Eigen::Matrix<float, Dynamic, Dynamic,
 * RowMajor> (reference include/config.h:17-25) and uses only its storage:
 * the (rows, cols) constructor, rows(), cols(), data(), operator()(r, c)
 * and Zero(rows, cols) (src/parallelMatrix.cpp:73-74,112,119-120;
 * main.cpp:324-336; src/utils.cpp:1130-1201; src/Matrix.cpp:19-33).  Eigen
 * is not a dependency of this library, so this class provides that subset
 * with the same layout: element (r, c) at data()[r * cols() + c].
 * Unlike Eigen, the (rows, cols) constructor zero-fills.
 */
#ifndef CWLB_DENSE_H
#define CWLB_DENSE_H

#include <algorithm>
#include <cstddef>
#include <limits>
#include <stdexcept>
#include <vector>

namespace cwlb {

template <class T>
class RowMajorMatrix {
public:
    using Scalar = T;
    using Index = std::ptrdiff_t;

    RowMajorMatrix() = default;
    RowMajorMatrix(Index rows, Index cols) { resize(rows, cols); }

    static RowMajorMatrix Zero(Index rows, Index cols) { return RowMajorMatrix(rows, cols); }
    static RowMajorMatrix Constant(Index rows, Index cols, const T& value)
    {
        RowMajorMatrix m(rows, cols);
        m.setConstant(value);
        return m;
    }

    Index rows() const { return rows_; }
    Index cols() const { return cols_; }
    Index size() const { return rows_ * cols_; }

    T* data() { return data_.data(); }
    const T* data() const { return data_.data(); }

    T& operator()(Index r, Index c) { return data_[static_cast<std::size_t>(r * cols_ + c)]; }
    const T& operator()(Index r, Index c) const
    {
        return data_[static_cast<std::size_t>(r * cols_ + c)];
    }

    // Resizes to rows x cols; the contents become zero.
    void resize(Index rows, Index cols)
    {
        if (rows < 0 || cols < 0)
            throw std::invalid_argument("RowMajorMatrix: negative dimension");
        if (cols != 0 && rows > std::numeric_limits<Index>::max() / cols)
            throw std::length_error("RowMajorMatrix: size overflows");
        data_.assign(static_cast<std::size_t>(rows * cols), T());
        rows_ = rows;
        cols_ = cols;
    }
    RowMajorMatrix& setZero()
    {
        std::fill(data_.begin(), data_.end(), T());
        return *this;
    }
    RowMajorMatrix& setConstant(const T& value)
    {
        std::fill(data_.begin(), data_.end(), value);
        return *this;
    }

private:
    Index rows_ = 0;
    Index cols_ = 0;
    std::vector<T> data_;
};

}  // namespace cwlb

#endif /* CWLB_DENSE_H */
