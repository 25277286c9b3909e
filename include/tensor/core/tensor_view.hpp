// Non-owning host views (reference: include/tensor/core/tensor_view.hpp).
#pragma once
#include <cstddef>
#include <stdexcept>
#include <string>

#include <tensor/core/dtype.hpp>
#include <tensor/core/shape.hpp>

namespace tensor::core {

template <typename T>
struct Span {
    const T* ptr = nullptr;
    std::size_t len = 0;
    const T* begin() const noexcept { return ptr; }
    const T* end() const noexcept { return ptr + len; }
    const T& operator[](std::size_t i) const noexcept { return ptr[i]; }
    std::size_t size() const noexcept { return len; }
    std::size_t size_bytes() const noexcept { return len * sizeof(T); }
    bool empty() const noexcept { return len == 0; }
};

struct TensorView {
    const void* data = nullptr;  // never owned
    DType dtype = DType::F32;
    Shape shape = {};

    std::size_t rank() const noexcept { return shape.rank(); }
    std::size_t numel() const noexcept { return shape.numel(); }
    std::size_t nbytes() const noexcept { return numel() * dtype_size(dtype); }

    // Typed view of the bytes; sizeof(T) must equal the element size
    // (uint16_t serves both BF16 and F16).
    template <typename T>
    Span<T> as() const {
        if (sizeof(T) != dtype_size(dtype))
            throw std::invalid_argument("TensorView::as<T>(): sizeof(T) (" +
                                        std::to_string(sizeof(T)) + ") does not match " +
                                        to_string(dtype));
        return Span<T>{static_cast<const T*>(data), numel()};
    }
};

}  // namespace tensor::core
