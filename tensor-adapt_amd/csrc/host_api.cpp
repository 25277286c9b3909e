// host_api.cpp — the C++ host API over the C-ABI: Device, Tensor, the GEMM
// and ops:: wrappers, the Centroid Accumulator and Dataset, with the
// reference's names and error behaviour (exceptions), see
// include/tensor/**/*.hpp.  Host code only (compiled with the host
// compiler); every device operation goes through a ta_* entry point.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "ta_backend.h"
#include "ta_engine.h"
#include <tensor/backend/cuda/device.hpp>
#include <tensor/backend/cuda/ops.hpp>
#include <tensor/backend/cuda/tensor.hpp>
#include <tensor/centroid/centroid_accumulator.hpp>
#include <tensor/centroid/centroid_merge.hpp>
#include <tensor/data/dataset.hpp>

namespace fs = std::filesystem;

namespace tensor::backend::cuda {

void check_status(int status, const char* what) {
    if (status != 0) throw CudaError(std::string(what) + ": " + ta_last_error());
}

static void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw CudaError(std::string(what) + ": " + hipGetErrorString(e));
}

// ── Device ──────────────────────────────────────────────────────────────
static int parse_spec(const std::string& spec) {
    std::string rest;
    if (spec.rfind("hip:", 0) == 0)
        rest = spec.substr(4);
    else if (spec.rfind("cuda:", 0) == 0)
        rest = spec.substr(5);
    else
        throw CudaError("invalid device spec \"" + spec + "\"; expected \"hip:N\" or \"cuda:N\"");
    size_t used = 0;
    int id = -1;
    try {
        id = std::stoi(rest, &used);
    } catch (...) {
        used = 0;
    }
    if (used == 0 || used != rest.size() || id < 0)
        throw CudaError("invalid device index in \"" + spec + "\"");
    return id;
}

Device Device::open(const std::string& spec) {
    Device d;
    d.id_ = parse_spec(spec);
    int n = 0;
    hip_check(hipGetDeviceCount(&n), "Device::open");
    if (d.id_ >= n)
        throw CudaError("Device::open: no device " + std::to_string(d.id_) + " (" +
                        std::to_string(n) + " visible)");
    hip_check(hipSetDevice(d.id_), "Device::open");
    hipDeviceProp_t prop{};
    hip_check(hipGetDeviceProperties(&prop, d.id_), "Device::open");
    d.sm_major_ = prop.major;
    d.arch_ = prop.gcnArchName;
    hip_check(hipStreamCreate(&d.stream_), "Device::open");
    std::cerr << "[device] hip:" << d.id_ << " " << d.arch_ << " (" << prop.name << ")\n";
    return d;
}

void Device::sync() const { hip_check(hipStreamSynchronize(stream_), "Device::sync"); }

Device::Device(Device&& o) noexcept
    : id_(o.id_), sm_major_(o.sm_major_), arch_(std::move(o.arch_)), stream_(o.stream_) {
    o.stream_ = nullptr;
}

Device& Device::operator=(Device&& o) noexcept {
    if (this != &o) {
        if (stream_) (void)hipStreamDestroy(stream_);
        id_ = o.id_;
        sm_major_ = o.sm_major_;
        arch_ = std::move(o.arch_);
        stream_ = o.stream_;
        o.stream_ = nullptr;
    }
    return *this;
}

Device::~Device() {
    if (stream_) {
        (void)hipStreamSynchronize(stream_);
        (void)hipStreamDestroy(stream_);
        stream_ = nullptr;
    }
}

// ── Tensor ──────────────────────────────────────────────────────────────
Tensor Tensor::empty(const Shape& shape, DType dtype, const Device& dev) {
    Tensor t;
    t.shape_ = shape;
    t.dtype_ = dtype;
    t.device_id_ = dev.id();
    size_t bytes = shape.numel() * core::dtype_size(dtype);
    if (bytes > 0) check_status(ta_mem_alloc(&t.ptr_, (int64_t)bytes, dev.id()), "Tensor::empty");
    return t;
}

Tensor Tensor::zeros(const Shape& shape, DType dtype, const Device& dev) {
    Tensor t = empty(shape, dtype, dev);
    t.zero_(dev);
    return t;
}

Tensor Tensor::from_host(const TensorView& src, const Device& dev) {
    Tensor t = empty(src.shape, src.dtype, dev);
    if (src.data && t.ptr_) {
        hip_check(hipMemcpyAsync(t.ptr_, src.data, t.nbytes(), hipMemcpyHostToDevice,
                                 dev.stream()),
                  "Tensor::from_host");
        dev.sync();
    }
    return t;
}

Tensor Tensor::empty_bf16(const Shape& s, const Device& d) { return empty(s, DType::BF16, d); }
Tensor Tensor::empty_f32(const Shape& s, const Device& d) { return empty(s, DType::F32, d); }
Tensor Tensor::zeros_f32(const Shape& s, const Device& d) { return zeros(s, DType::F32, d); }

template <typename T>
static std::vector<T> read_back(const void* ptr, size_t n, size_t bytes, int dev) {
    std::vector<T> out(n);
    if (ptr) {
        hip_check(hipSetDevice(dev), "Tensor::to_host");
        hip_check(hipDeviceSynchronize(), "Tensor::to_host");
        hip_check(hipMemcpy(out.data(), ptr, bytes, hipMemcpyDeviceToHost), "Tensor::to_host");
    }
    return out;
}

std::vector<bf16_t> Tensor::to_host_bf16() const {
    if (dtype_ != DType::BF16) throw std::runtime_error("Tensor::to_host_bf16: dtype mismatch");
    return read_back<bf16_t>(ptr_, numel(), nbytes(), device_id_);
}

std::vector<float> Tensor::to_host_f32() const {
    if (dtype_ != DType::F32) throw std::runtime_error("Tensor::to_host_f32: dtype mismatch");
    return read_back<float>(ptr_, numel(), nbytes(), device_id_);
}

std::vector<uint32_t> Tensor::to_host_u32() const {
    if (dtype_ != DType::I32)
        throw std::runtime_error("Tensor::to_host_u32: dtype mismatch (expected I32)");
    return read_back<uint32_t>(ptr_, numel(), nbytes(), device_id_);
}

void Tensor::zero_(const Device& dev) {
    if (ptr_) hip_check(hipMemsetAsync(ptr_, 0, nbytes(), dev.stream()), "Tensor::zero_");
}

Tensor::Tensor(Tensor&& o) noexcept
    : ptr_(o.ptr_), shape_(std::move(o.shape_)), dtype_(o.dtype_), device_id_(o.device_id_) {
    o.ptr_ = nullptr;
}

Tensor& Tensor::operator=(Tensor&& o) noexcept {
    if (this != &o) {
        if (ptr_) (void)ta_mem_free(ptr_, device_id_);
        ptr_ = o.ptr_;
        shape_ = std::move(o.shape_);
        dtype_ = o.dtype_;
        device_id_ = o.device_id_;
        o.ptr_ = nullptr;
    }
    return *this;
}

Tensor::~Tensor() {
    if (ptr_) {
        (void)ta_mem_free(ptr_, device_id_);
        ptr_ = nullptr;
    }
}

// ── GEMM ────────────────────────────────────────────────────────────────
static void validate_gemm(const char* name, const GemmParams& p, int lda, int ldb, int ldc) {
    if (p.M <= 0 || p.N <= 0 || p.K <= 0)
        throw CudaError(std::string(name) + ": M/N/K must be > 0");
    if (lda <= 0 || ldb <= 0 || ldc <= 0)
        throw CudaError(std::string(name) + ": leading dims must be > 0");
}

void gemm_bf16(const Device& dev, const GemmParams& p, const bf16_t* A, int lda, const bf16_t* B,
               int ldb, bf16_t* C, int ldc) {
    validate_gemm("gemm_bf16", p, lda, ldb, ldc);
    check_status(ta_gemm_bf16(p.transA, p.transB, p.M, p.N, p.K, p.alpha, A, lda, B, ldb, p.beta,
                              C, ldc, dev.stream()),
                 "gemm_bf16");
}

void gemm_f32(const Device& dev, const GemmParams& p, const float* A, int lda, const float* B,
              int ldb, float* C, int ldc) {
    validate_gemm("gemm_f32", p, lda, ldb, ldc);
    check_status(ta_gemm_f32(p.transA, p.transB, p.M, p.N, p.K, p.alpha, A, lda, B, ldb, p.beta,
                             C, ldc, dev.stream()),
                 "gemm_f32");
}

// ── ops ─────────────────────────────────────────────────────────────────
namespace ops {

void rms_norm_fwd(const bf16_t* x, const bf16_t* w, bf16_t* out, float* rms_out, int B, int T,
                  int D, float eps, hipStream_t s) {
    check_status(ta_rms_norm_fwd(x, w, out, rms_out, B, T, D, eps, s), "rms_norm_fwd");
}
void rms_norm_bwd(const bf16_t* dy, const bf16_t* x, const bf16_t* w, const float* rms,
                  bf16_t* dx, float* dw, int B, int T, int D, float eps, hipStream_t s) {
    check_status(ta_rms_norm_bwd(dy, x, w, rms, dx, dw, B, T, D, eps, s), "rms_norm_bwd");
}
void rope_fwd(bf16_t* x, int B, int T, int H, int hd, float theta, hipStream_t s) {
    check_status(ta_rope_fwd(x, B, T, H, hd, theta, s), "rope_fwd");
}
void rope_bwd(bf16_t* dx, int B, int T, int H, int hd, float theta, hipStream_t s) {
    check_status(ta_rope_bwd(dx, B, T, H, hd, theta, s), "rope_bwd");
}
void sdpa_fwd(const bf16_t* Q, const bf16_t* K, const bf16_t* V, bf16_t* out, float* attn_w,
              int B, int T, int Hq, int Hkv, int hd, const Device& dev) {
    check_status(ta_sdpa_fwd(Q, K, V, out, attn_w, B, T, Hq, Hkv, hd, dev.stream()), "sdpa_fwd");
}
void sdpa_bwd(const bf16_t* dout, const bf16_t* Q, const bf16_t* K, const bf16_t* V,
              const float* attn_w, bf16_t* dQ, bf16_t* dK, bf16_t* dV, int B, int T, int Hq,
              int Hkv, int hd, const Device& dev) {
    check_status(ta_sdpa_bwd(dout, Q, K, V, attn_w, dQ, dK, dV, B, T, Hq, Hkv, hd, dev.stream()),
                 "sdpa_bwd");
}
void silu_mul_fwd(const bf16_t* gate, const bf16_t* up, bf16_t* out, int N, hipStream_t s) {
    check_status(ta_silu_mul_fwd(gate, up, out, N, s), "silu_mul_fwd");
}
void silu_mul_bwd(const bf16_t* dout, const bf16_t* gate, const bf16_t* up, bf16_t* dgate,
                  bf16_t* dup, int N, hipStream_t s) {
    check_status(ta_silu_mul_bwd(dout, gate, up, dgate, dup, N, s), "silu_mul_bwd");
}
void cross_entropy_fwd(const bf16_t* logits, const int* targets, float* loss_out,
                       bf16_t* dlogits, int N, int V, hipStream_t s) {
    check_status(ta_cross_entropy_fwd(logits, targets, loss_out, dlogits, N, V, s),
                 "cross_entropy_fwd");
}
void embed_fwd(const bf16_t* table, const int* tokens, bf16_t* out, int BT, int D,
               hipStream_t s) {
    check_status(ta_embed_fwd(table, tokens, out, BT, D, s), "embed_fwd");
}
void embed_bwd(const bf16_t* dout, const int* tokens, float* dtable, int BT, int D,
               hipStream_t s) {
    check_status(ta_embed_bwd(dout, tokens, dtable, BT, D, s), "embed_bwd");
}
void add_bias(bf16_t* out, const bf16_t* bias, int BT, int D, hipStream_t s) {
    check_status(ta_add_bias(out, bias, BT, D, s), "add_bias");
}
void add_inplace(bf16_t* out, const bf16_t* delta, int N, hipStream_t s) {
    check_status(ta_add_inplace(out, delta, N, s), "add_inplace");
}
void lora_add(bf16_t* out, const bf16_t* delta, float scale, int N, hipStream_t s) {
    check_status(ta_lora_add(out, delta, scale, N, s), "lora_add");
}
void cast_bf16_to_f32(const bf16_t* src, float* dst, int N, hipStream_t s) {
    check_status(ta_cast_bf16_to_f32(src, dst, N, s), "cast_bf16_to_f32");
}
void cast_f32_to_bf16(const float* src, bf16_t* dst, int N, hipStream_t s) {
    check_status(ta_cast_f32_to_bf16(src, dst, N, s), "cast_f32_to_bf16");
}
void adamw_step(float* master, bf16_t* working, float* m, float* v, const float* grad, int N,
                float lr, float b1, float b2, float eps, float wd, int step, hipStream_t s) {
    check_status(ta_adamw_step(master, working, m, v, grad, N, lr, b1, b2, eps, wd, step, s),
                 "adamw_step");
}
void sum_sq_into(const float* g, float* accum, int N, hipStream_t s) {
    check_status(ta_sum_sq_into(g, accum, N, s), "sum_sq_into");
}
void adamw_fused(float* master, bf16_t* working, float* m, float* v, float* grad,
                 int64_t N, float lr, float b1, float b2, float eps, float wd, int step,
                 float max_norm, float* norm_out, hipStream_t s) {
    check_status(ta_adamw_fused(master, working, m, v, grad, N, lr, b1, b2, eps, wd, step,
                                max_norm, norm_out, s),
                 "adamw_fused");
}
void centroid_accumulate(const bf16_t* h, const bf16_t* g, int64_t BT, int D, double* acc,
                         hipStream_t s) {
    check_status(ta_centroid_accumulate_bf16(h, g, BT, D, acc, s), "centroid_accumulate");
}

}  // namespace ops
}  // namespace tensor::backend::cuda

// ── Centroid Accumulator ────────────────────────────────────────────────
namespace tensor::centroid {

using backend::cuda::check_status;
using backend::cuda::CudaError;

CentroidAccumulator::CentroidAccumulator(int hidden_dim, const std::string& dir)
    : D_(hidden_dim), dir_(dir) {
    fs::create_directories(dir);
}

CentroidAccumulator::~CentroidAccumulator() {
    if (acc_) {
        (void)hipSetDevice(device_);
        (void)hipStreamSynchronize(stream_);
        (void)ta_mem_free(acc_, device_);
    }
}

void CentroidAccumulator::accumulate(const backend::cuda::Tensor& hidden,
                                     const backend::cuda::Tensor& grad,
                                     const backend::cuda::Device& dev) {
    if (hidden.rank() != 2 || grad.shape() != hidden.shape()) return;
    const int64_t BT = (int64_t)hidden.shape()[0];
    if ((int)hidden.shape()[1] != D_) return;
    device_sums(dev);
    using backend::cuda::DType;
    if (hidden.dtype() == DType::BF16 && grad.dtype() == DType::BF16)
        check_status(ta_centroid_accumulate_bf16(hidden.bf16(), grad.bf16(), BT, D_, acc_,
                                                 dev.stream()),
                     "CentroidAccumulator::accumulate");
    else if (hidden.dtype() == DType::F32 && grad.dtype() == DType::F32)
        check_status(ta_centroid_accumulate_f32(hidden.f32(), grad.f32(), BT, D_, acc_,
                                                dev.stream()),
                     "CentroidAccumulator::accumulate");
    else
        throw CudaError("CentroidAccumulator::accumulate: hidden and grad_signal must both be "
                        "BF16 or both F32");
}

double* CentroidAccumulator::device_sums(const backend::cuda::Device& dev) {
    if (acc_ && dev.id() != device_)
        throw CudaError("CentroidAccumulator: accumulate on device " + std::to_string(dev.id()) +
                        " after device " + std::to_string(device_));
    if (!acc_) {
        void* p = nullptr;
        check_status(ta_mem_alloc(&p, (int64_t)(D_ + 1) * sizeof(double), dev.id()),
                     "CentroidAccumulator");
        acc_ = (double*)p;
        device_ = dev.id();
        if (hipMemsetAsync(acc_, 0, (D_ + 1) * sizeof(double), dev.stream()) != hipSuccess)
            throw CudaError("CentroidAccumulator: clearing the accumulator failed");
    }
    stream_ = dev.stream();
    return acc_;
}

std::vector<double> CentroidAccumulator::sums() const {
    std::vector<double> s(D_ + 1, 0.0);
    if (!acc_) return s;
    if (hipSetDevice(device_) != hipSuccess || hipStreamSynchronize(stream_) != hipSuccess ||
        hipMemcpy(s.data(), acc_, s.size() * sizeof(double), hipMemcpyDeviceToHost) != hipSuccess)
        throw CudaError("CentroidAccumulator: reading the accumulator failed");
    return s;
}

void CentroidAccumulator::write_snapshot(std::size_t step) {
    std::vector<double> s = sums();
    float w = (float)s[D_];
    if (w == 0.f) return;
    std::vector<float> c(D_);
    for (int d = 0; d < D_; d++) c[d] = (float)(s[d] / s[D_]);
    std::string path = dir_ + "/step-" + std::to_string(step) + ".centroid";
    std::ofstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("CentroidAccumulator: cannot write " + path);
    int32_t D = D_;
    f.write(reinterpret_cast<const char*>(&D), sizeof D);
    f.write(reinterpret_cast<const char*>(c.data()), (std::streamsize)(c.size() * sizeof(float)));
    f.write(reinterpret_cast<const char*>(&w), sizeof w);
    if (!snapshot_steps_.empty() && snapshot_steps_.back() == step) {
        snapshots_.back() = std::move(c);
    } else {
        snapshots_.push_back(std::move(c));
        snapshot_steps_.push_back(step);
    }
    std::cerr << "[centroid] snapshot -> " << path << " (weight=" << w << ")\n";
}

// step number of "step-<N>.centroid" (files named otherwise sort after, by name)
static bool snapshot_order(const fs::path& a, const fs::path& b) {
    auto num = [](const fs::path& p, long long* v) {
        std::string s = p.stem().string();
        if (s.rfind("step-", 0) != 0) return false;
        char* end = nullptr;
        *v = std::strtoll(s.c_str() + 5, &end, 10);
        return end && *end == 0 && s.size() > 5;
    };
    long long va = 0, vb = 0;
    bool ha = num(a, &va), hb = num(b, &vb);
    if (ha != hb) return ha;
    if (ha && va != vb) return va < vb;
    return a.filename().string() < b.filename().string();
}

static std::vector<fs::path> snapshot_files(const std::string& dir) {
    std::vector<fs::path> files;
    for (const auto& e : fs::directory_iterator(dir))
        if (e.path().extension() == ".centroid") files.push_back(e.path());
    std::sort(files.begin(), files.end(), snapshot_order);
    return files;
}

void CentroidAccumulator::merge_and_write(int k, const std::string& out_path) {
    if (snapshots_.empty()) {
        for (const auto& p : snapshot_files(dir_)) {
            std::ifstream f(p, std::ios::binary);
            int32_t d = 0;
            f.read(reinterpret_cast<char*>(&d), sizeof d);
            if (!f || d != D_) continue;
            std::vector<float> c(d);
            f.read(reinterpret_cast<char*>(c.data()), (std::streamsize)(d * sizeof(float)));
            if (f) snapshots_.push_back(std::move(c));
        }
    }
    if (snapshots_.empty()) {
        std::cerr << "[centroid] no snapshots to merge\n";
        return;
    }
    const int N = (int)snapshots_.size();
    k = std::min(k, N);
    if (k <= 0) throw std::runtime_error("CentroidAccumulator::merge_and_write: k must be > 0");

    int dev = device_;
    if (dev < 0 && hipGetDevice(&dev) != hipSuccess) throw CudaError("merge_and_write: no device");
    if (hipSetDevice(dev) != hipSuccess) throw CudaError("merge_and_write: hipSetDevice failed");
    std::vector<float> flat((size_t)N * D_);
    for (int n = 0; n < N; n++)
        std::memcpy(flat.data() + (size_t)n * D_, snapshots_[n].data(), D_ * sizeof(float));
    void *d_snap = nullptr, *d_cent = nullptr, *d_asg = nullptr;
    auto release = [&]() {
        (void)hipDeviceSynchronize();
        (void)ta_mem_free(d_snap, dev);
        (void)ta_mem_free(d_cent, dev);
        (void)ta_mem_free(d_asg, dev);
    };
    std::vector<float> centers((size_t)k * D_);
    try {
        check_status(ta_mem_alloc(&d_snap, (int64_t)flat.size() * 4, dev), "merge_and_write");
        check_status(ta_mem_alloc(&d_cent, (int64_t)centers.size() * 4, dev), "merge_and_write");
        check_status(ta_mem_alloc(&d_asg, (int64_t)N * 4, dev), "merge_and_write");
        if (hipMemcpy(d_snap, flat.data(), flat.size() * 4, hipMemcpyHostToDevice) != hipSuccess)
            throw CudaError("merge_and_write: upload failed");
        check_status(ta_kmeans_ref((const float*)d_snap, N, D_, k, 50, (float*)d_cent,
                                   (int32_t*)d_asg, nullptr, nullptr),
                     "merge_and_write");
        if (hipMemcpy(centers.data(), d_cent, centers.size() * 4, hipMemcpyDeviceToHost) !=
            hipSuccess)
            throw CudaError("merge_and_write: download failed");
    } catch (...) {
        release();
        throw;
    }
    release();
    std::ofstream f(out_path, std::ios::binary);
    if (!f) throw std::runtime_error("CentroidAccumulator: cannot write " + out_path);
    int32_t kk = k, D = D_;
    f.write(reinterpret_cast<const char*>(&kk), sizeof kk);
    f.write(reinterpret_cast<const char*>(&D), sizeof D);
    f.write(reinterpret_cast<const char*>(centers.data()),
            (std::streamsize)(centers.size() * sizeof(float)));
    std::cerr << "[centroid] merged " << N << " snapshots -> k=" << k << " clusters, " << out_path
              << "\n";
}

void CentroidMerge::run(const std::string& dir, const std::string& out_path, int k) {
    int32_t D = 0;
    for (const auto& p : snapshot_files(dir)) {
        std::ifstream f(p, std::ios::binary);
        f.read(reinterpret_cast<char*>(&D), sizeof D);
        break;
    }
    if (D == 0) throw std::runtime_error("No .centroid files in " + dir);
    CentroidAccumulator acc(D, dir);
    acc.merge_and_write(k, out_path);
}

}  // namespace tensor::centroid

// ── Dataset ─────────────────────────────────────────────────────────────
namespace tensor::data {

Dataset Dataset::load(const std::string& dir) {
    fs::path d(dir);
    if (!fs::exists(d)) throw DataError("path not found: " + dir);
    std::vector<fs::path> files;
    if (fs::is_regular_file(d) && d.extension() == ".bin") {
        files.push_back(d);
    } else if (fs::is_directory(d)) {
        for (const auto& e : fs::directory_iterator(d))
            if (e.is_regular_file() && e.path().extension() == ".bin") files.push_back(e.path());
        std::sort(files.begin(), files.end());
    } else {
        throw DataError("expected a .bin file or directory of .bin files: " + dir);
    }
    if (files.empty()) throw DataError("no .bin files in: " + dir);
    Dataset ds;
    for (const auto& f : files) {
        std::ifstream in(f, std::ios::binary | std::ios::ate);
        if (!in) throw DataError("cannot open: " + f.string());
        size_t n = (size_t)in.tellg() / sizeof(uint32_t);
        in.seekg(0);
        size_t old = ds.tokens_.size();
        ds.tokens_.resize(old + n);
        in.read(reinterpret_cast<char*>(ds.tokens_.data() + old), (std::streamsize)(n * 4));
        std::cerr << "[data] loaded " << f.filename() << " (" << n << " tokens)\n";
    }
    std::cerr << "[data] total tokens: " << ds.total_tokens() << "\n";
    return ds;
}

std::pair<std::vector<int32_t>, std::vector<int32_t>> Dataset::next_batch(int B, int T) {
    const size_t n = tokens_.size();
    if (n == 0) throw DataError("next_batch on an empty dataset");
    std::vector<int32_t> in((size_t)B * T), tg((size_t)B * T);
    for (int b = 0; b < B; b++) {
        for (int t = 0; t < T; t++) {
            size_t i = (pos_ + t) % n;
            in[(size_t)b * T + t] = (int32_t)tokens_[i];
            tg[(size_t)b * T + t] = (int32_t)tokens_[(i + 1) % n];
        }
        pos_ = (pos_ + T) % n;
    }
    consumed_ += (size_t)B * T;
    return {std::move(in), std::move(tg)};
}

}  // namespace tensor::data
