// Device — one GPU and the one stream all of its work is ordered on.
//
// Drop-in for the reference's tensor::backend::cuda::Device
// (include/tensor/backend/cuda/device.hpp:52-79, src/backend/cuda/device.cu),
// implemented on HIP for MI355X (gfx950): the header path, namespace and
// class name are kept so that callers compile unchanged; there is no BLAS
// handle (GEMMs are the backend's own kernels) and no CUDA symbol.
#pragma once
#include <hip/hip_runtime_api.h>

#include <stdexcept>
#include <string>

namespace tensor::backend::cuda {

// Error thrown by every host-API failure (the reference's exception type
// and message prefix, device.hpp:15-19).
struct CudaError : std::runtime_error {
    explicit CudaError(const std::string& msg) : std::runtime_error("CudaError: " + msg) {}
};

// Throws CudaError with the backend's last error message when a ta_* call
// returns a non-zero status.
void check_status(int status, const char* what);

class Device {
public:
    // "hip:N" or "cuda:N" (the reference's spec form, device.cu:9-23).
    static Device open(const std::string& spec);

    int id() const noexcept { return id_; }
    hipStream_t stream() const noexcept { return stream_; }
    // gfx major version (9 for gfx950) in place of the CUDA SM major.
    int sm_major() const noexcept { return sm_major_; }
    // BF16 MFMA is native on every supported target.
    bool supports_bf16_gemm() const noexcept { return true; }
    const std::string& arch() const noexcept { return arch_; }
    void sync() const;

    Device(Device&&) noexcept;
    Device& operator=(Device&&) noexcept;
    Device(const Device&) = delete;
    Device& operator=(const Device&) = delete;
    ~Device();

private:
    Device() = default;
    int id_ = 0;
    int sm_major_ = 0;
    std::string arch_;
    hipStream_t stream_ = nullptr;
};

}  // namespace tensor::backend::cuda
