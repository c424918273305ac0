#pragma once
// Tensor shape (reference include/dl/core/Shape.hpp).  As in the reference,
// a shape with no dimensions has numel() == 0.

#include <cstdint>
#include <initializer_list>
#include <string>
#include <vector>

namespace dl {

class Shape {
public:
    std::vector<int64_t> dims;

    Shape() = default;
    Shape(std::initializer_list<int64_t> dims);
    explicit Shape(std::vector<int64_t> dims);

    int64_t rank() const;
    int64_t numel() const;
    int64_t operator[](int index) const;
    std::string str() const;
};

}  // namespace dl

using Shape = dl::Shape;
