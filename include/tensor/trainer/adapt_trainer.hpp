// AdaptTrainer — the LoRA training loop (include/tensor/trainer/
// adapt_trainer.hpp:18-78 and src/trainer/adapt_trainer.cu in the
// reference, with the same types, methods and meaning): each step takes the
// next batch from the Dataset, runs forward, loss, backward, the centroid
// side channel, gradient norm and clip and AdamW, and every
// checkpoint_every steps writes a centroid snapshot and a checkpoint; run()
// trains until `tokens` tokens are consumed and saves the adapter.
//
// The whole step runs in the MI355X step engine (include/ta_engine.h) on the
// Device's stream; the base weights are copied from the FrozenBase's device
// tensors once, at create().  Injection follows every AdapterConfig flag (the
// reference always trains q, k, v, o).  AdaptOptions::resume_from, when set,
// names a checkpoint directory written by save_checkpoint; the trainer then
// continues from its step, optimiser state, token count, data position and
// centroid sums (the reference accepts the option and ignores it).
#pragma once
#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>

#include <tensor/adapter/adapter_config.hpp>
#include <tensor/adapter/adapter_model.hpp>
#include <tensor/backend/cuda/device.hpp>
#include <tensor/base/frozen_base.hpp>
#include <tensor/data/dataset.hpp>

namespace tensor::trainer {

struct StepMetrics {
    std::size_t step;
    std::size_t tokens_consumed;
    float loss;
    float learning_rate;
    float grad_norm;        // min(||g||, grad_clip)
    double step_ms;         // wall-clock time of this step
    double ema_ms;          // exponential moving average of step_ms (alpha 0.1)
    double tokens_per_sec;  // from ema_ms
};

struct AdaptOptions {
    std::string domain;
    std::string output_dir;
    std::size_t checkpoint_every = 1000;
    std::string resume_from;  // "" = start fresh
    std::string device = "cuda:0";
    uint64_t seed = 42;
    bool log_to_stdout = true;
    std::size_t tokens = 50'000'000;
};

class AdaptTrainer {
public:
    static AdaptTrainer create(const base::FrozenBase& base, const adapter::AdapterConfig& cfg,
                               data::Dataset& dataset, const AdaptOptions& opts,
                               const backend::cuda::Device& dev);

    void run();
    bool done() const;
    StepMetrics step();

    void save_checkpoint(const std::string& dir);
    void save_adapter(const std::string& dir);

    // the step engine (include/ta_engine.h) behind this trainer, for
    // inspection (ta_engine_read_adapter and the like)
    void* engine() const;

    ~AdaptTrainer();
    AdaptTrainer(AdaptTrainer&&) noexcept;
    AdaptTrainer& operator=(AdaptTrainer&&) noexcept;
    AdaptTrainer(const AdaptTrainer&) = delete;
    AdaptTrainer& operator=(const AdaptTrainer&) = delete;

private:
    struct Impl;
    std::unique_ptr<Impl> impl_;
    explicit AdaptTrainer(std::unique_ptr<Impl>);
};

}  // namespace tensor::trainer
