// Shape: a dimension vector (rank-0 = scalar, numel 1), as the reference's
// include/tensor/core/shape.hpp defines it.
#pragma once
#include <cstddef>
#include <vector>

namespace tensor::core {

class Shape : public std::vector<std::size_t> {
public:
    using std::vector<std::size_t>::vector;
    std::size_t rank() const noexcept { return size(); }
    std::size_t numel() const noexcept {
        std::size_t n = 1;
        for (std::size_t d : *this) n *= d;
        return n;
    }
};

}  // namespace tensor::core
