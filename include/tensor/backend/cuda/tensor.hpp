// Tensor — owning device buffer with shape and dtype, and the two GEMM entry
// points.  Drop-in for include/tensor/backend/cuda/tensor.hpp:25-101
// (src/backend/cuda/tensor.cu).  Memory comes from the backend's caching
// allocator (ta_mem_alloc / ta_mem_free) instead of one hipMalloc/hipFree
// per tensor: a freed block returns to a per-device cache and is handed out
// again in stream order.  BF16 elements are uint16_t bit patterns.
#pragma once
#include <cstddef>
#include <cstdint>
#include <vector>

#include <tensor/backend/cuda/device.hpp>
#include <tensor/core/dtype.hpp>
#include <tensor/core/shape.hpp>
#include <tensor/core/tensor_view.hpp>

namespace tensor::backend::cuda {

using core::DType;
using core::Shape;
using core::TensorView;
using bf16_t = std::uint16_t;  // BF16 bit pattern

class Tensor {
public:
    Tensor() = default;

    static Tensor empty(const Shape& shape, DType dtype, const Device& dev);
    static Tensor zeros(const Shape& shape, DType dtype, const Device& dev);
    // Copies src to the device and waits for the copy (tensor.cu:40-49).
    static Tensor from_host(const TensorView& src, const Device& dev);
    static Tensor empty_bf16(const Shape& shape, const Device& dev);
    static Tensor empty_f32(const Shape& shape, const Device& dev);
    static Tensor zeros_f32(const Shape& shape, const Device& dev);

    const Shape& shape() const noexcept { return shape_; }
    DType dtype() const noexcept { return dtype_; }
    int device_id() const noexcept { return device_id_; }
    std::size_t rank() const noexcept { return shape_.rank(); }
    std::size_t numel() const noexcept { return shape_.numel(); }
    std::size_t nbytes() const noexcept { return numel() * core::dtype_size(dtype_); }
    bool empty() const noexcept { return ptr_ == nullptr; }

    void* data() noexcept { return ptr_; }
    const void* data() const noexcept { return ptr_; }
    bf16_t* bf16() noexcept { return static_cast<bf16_t*>(ptr_); }
    const bf16_t* bf16() const noexcept { return static_cast<const bf16_t*>(ptr_); }
    float* f32() noexcept { return static_cast<float*>(ptr_); }
    const float* f32() const noexcept { return static_cast<const float*>(ptr_); }
    int* i32() noexcept { return static_cast<int*>(ptr_); }
    const int* i32() const noexcept { return static_cast<const int*>(ptr_); }

    // Blocking device-to-host copies; each checks the dtype first and throws
    // std::runtime_error on a mismatch (tensor.cu:63-95: to_host_u32 reads
    // an I32 tensor).  They wait for all work on the device.
    std::vector<bf16_t> to_host_bf16() const;
    std::vector<float> to_host_f32() const;
    std::vector<uint32_t> to_host_u32() const;

    // Asynchronous zero fill on the device's stream.
    void zero_(const Device& dev);

    Tensor(Tensor&&) noexcept;
    Tensor& operator=(Tensor&&) noexcept;
    Tensor(const Tensor&) = delete;
    Tensor& operator=(const Tensor&) = delete;
    ~Tensor();

private:
    void* ptr_ = nullptr;
    Shape shape_;
    DType dtype_ = DType::F32;
    int device_id_ = 0;
};

// Column-major GEMM parameters (tensor.hpp:79-86).
struct GemmParams {
    bool transA = false;
    bool transB = false;
    int M = 0, N = 0, K = 0;
    float alpha = 1.0f;
    float beta = 0.0f;
};

// C = alpha * op(A) op(B) + beta * C with the BLAS column-major convention,
// on the device's stream.  Throws CudaError when M, N, K or a leading
// dimension is <= 0 (tensor.cu:134-142).  gemm_bf16: FP32 accumulation,
// one BF16 rounding of the output.  gemm_f32: F32 in/out at F32 accuracy:
// each F32 operand is split into three BF16 parts (24 significand bits in
// all) and the part products are accumulated in F32 on the BF16 MFMA.
void gemm_bf16(const Device& dev, const GemmParams& p, const bf16_t* A, int lda,
               const bf16_t* B, int ldb, bf16_t* C, int ldc);
void gemm_f32(const Device& dev, const GemmParams& p, const float* A, int lda, const float* B,
              int ldb, float* C, int ldc);

}  // namespace tensor::backend::cuda
