// CentroidAccumulator — the training step's side channel: per token t,
// C += h_t * ||g_t||_2 and W += ||g_t||_2, summed over every layer and step;
// snapshots C / W to <dir>/step-<N>.centroid; k-means over the snapshots at
// the end.  Same API and file formats as the reference's
// include/tensor/centroid/centroid_accumulator.hpp
// (src/centroid/centroid_accumulator.cpp:17-168):
//   snapshot  step-<N>.centroid : int32 D, D x f32 centroid, f32 W
//   merged    out_path          : int32 k, int32 D, k x D f32 centers
// Differences, by design: the sum runs on the device into an F64 vector
// (no per-layer synchronisation or host copy); accumulate() reads BF16
// or F32 h/g as they are typed (the reference reinterprets F32 buffers as
// BF16, its defect D1); snapshots found on disk are merged in step order
// (the reference used directory order); k-means runs on the device with
// the reference's init, tie rule, empty-cluster rule and 50-pass cap.
#pragma once
#include <cstddef>
#include <string>
#include <vector>

#include <tensor/backend/cuda/device.hpp>
#include <tensor/backend/cuda/tensor.hpp>

namespace tensor::centroid {

class CentroidAccumulator {
public:
    CentroidAccumulator(int hidden_dim, const std::string& snapshot_dir);
    ~CentroidAccumulator();
    CentroidAccumulator(const CentroidAccumulator&) = delete;
    CentroidAccumulator& operator=(const CentroidAccumulator&) = delete;

    // hidden, grad_signal: [BT, D], both BF16 or both F32, on dev.
    // Asynchronous on dev's stream.  Tensors whose D differs are ignored.
    void accumulate(const backend::cuda::Tensor& hidden,
                    const backend::cuda::Tensor& grad_signal,
                    const backend::cuda::Device& dev);

    // Writes step-<step>.centroid (nothing while W == 0).  Writing the same
    // step again replaces that snapshot, as rewriting its file does.
    void write_snapshot(std::size_t step);

    // k-means over the snapshots taken (or, if none, those in the
    // directory) and writes the merged file.
    void merge_and_write(int k, const std::string& out_path);

    // Current sums (C[0..D-1], W) as F64; waits for the device.
    std::vector<double> sums() const;

    // The device F64 vector [D + 1] (sums, then W) that accumulate() adds
    // into, allocated and zeroed on dev at the first call; for producers
    // that add into it on dev's stream (the step engine behind AdaptTrainer).
    double* device_sums(const backend::cuda::Device& dev);

private:
    int D_;
    std::string dir_;
    int device_ = -1;
    hipStream_t stream_ = nullptr;
    double* acc_ = nullptr;  // device [D + 1]
    std::vector<std::vector<float>> snapshots_;
    std::vector<std::size_t> snapshot_steps_;
};

}  // namespace tensor::centroid
