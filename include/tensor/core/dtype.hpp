// Element types of the host API (same enumerators and sizes as the
// reference's include/tensor/core/dtype.hpp, so that code switching to this
// backend keeps its DType values).
#pragma once
#include <cstddef>
#include <stdexcept>
#include <string>

namespace tensor::core {

enum class DType { F64, F32, BF16, F16, F8_E5M2, F8_E4M3, I64, I32, I16, I8, U8, BOOL };

inline std::size_t dtype_size(DType d) {
    static constexpr std::size_t kSize[] = {8, 4, 2, 2, 1, 1, 8, 4, 2, 1, 1, 1};
    auto i = static_cast<std::size_t>(d);
    if (i >= sizeof kSize / sizeof kSize[0]) throw std::invalid_argument("dtype_size: unknown DType");
    return kSize[i];
}

inline std::string to_string(DType d) {
    static const char* kName[] = {"F64", "F32", "BF16", "F16", "F8_E5M2", "F8_E4M3",
                                  "I64", "I32", "I16",  "I8",  "U8",      "BOOL"};
    auto i = static_cast<std::size_t>(d);
    if (i >= sizeof kName / sizeof kName[0])
        throw std::invalid_argument("to_string(DType): unknown DType");
    return kName[i];
}

}  // namespace tensor::core
