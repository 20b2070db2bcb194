#pragma once

// Static tensor types. Same surface as the reference's
// include/minicompiler/tensor.hpp:13-91 (DType, Shape, kMaxElements,
// checked_num_elements, TensorType, to_string).

#include <cstddef>
#include <cstdint>
#include <optional>
#include <ostream>
#include <string>
#include <utility>
#include <vector>

namespace minicompiler {

enum class DType : std::uint8_t { Float32, Float64, Int32, Int64, Bool };

inline std::size_t dtype_size_bytes(DType dt) {
    switch (dt) {
        case DType::Float32:
        case DType::Int32: return 4;
        case DType::Float64:
        case DType::Int64: return 8;
        case DType::Bool: return 1;
    }
    return 0;
}

inline const char* dtype_name(DType dt) {
    static const char* const names[] = {"f32", "f64", "i32", "i64", "bool"};
    const auto i = static_cast<unsigned>(dt);
    return i < 5 ? names[i] : "?";
}

using Shape = std::vector<std::int64_t>;

// The generated kernels index with 32-bit unsigned integers and the GEMM
// launchers take int dimensions, so every tensor stays below 2^31 elements.
inline constexpr std::size_t kMaxElements = (std::size_t{1} << 31) - 1;

// Element count of `shape`, or nullopt when a dimension is < 1 or the count
// passes kMaxElements (checked before anything is allocated).
inline std::optional<std::size_t> checked_num_elements(const Shape& shape) {
    std::size_t count = 1;
    for (std::int64_t d : shape) {
        if (d < 1) return std::nullopt;
        const auto ud = static_cast<std::size_t>(d);
        if (count > kMaxElements / ud) return std::nullopt;
        count *= ud;
    }
    return count;
}

inline std::size_t num_elements(const Shape& shape) {
    std::size_t count = 1;
    for (std::int64_t d : shape) count *= static_cast<std::size_t>(d);
    return count;
}

struct TensorType {
    Shape shape;
    DType dtype = DType::Float32;

    TensorType() = default;
    explicit TensorType(Shape s, DType d = DType::Float32) : shape(std::move(s)), dtype(d) {}

    std::size_t rank() const { return shape.size(); }
    std::size_t num_elements() const { return minicompiler::num_elements(shape); }
    std::size_t size_bytes() const { return num_elements() * dtype_size_bytes(dtype); }

    bool operator==(const TensorType& o) const { return dtype == o.dtype && shape == o.shape; }
    bool operator!=(const TensorType& o) const { return !(*this == o); }
};

// "[4,8]"; rank 0 prints as "[]".
inline std::string to_string(const Shape& shape) {
    std::string text = "[";
    for (std::size_t i = 0; i < shape.size(); ++i) {
        if (i) text += ',';
        text += std::to_string(shape[i]);
    }
    text += ']';
    return text;
}

// "f32[4,8]"
inline std::string to_string(const TensorType& t) { return std::string(dtype_name(t.dtype)) + to_string(t.shape); }

inline std::ostream& operator<<(std::ostream& os, const TensorType& t) { return os << to_string(t); }

}  // namespace minicompiler
