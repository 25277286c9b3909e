// AdamW over an AdapterModel's pairs, one tensor at a time
// (include/tensor/trainer/adamw.hpp and src/trainer/adamw.cu:9-38 in the
// reference; same struct, fields and methods).  Like the reference it takes
// beta1, beta2 and weight decay from the AdapterConfig and keeps eps at
// 1e-8.  The fused step engine runs the same update over one flat arena
// with the gradient clip folded in (ops::adamw_fused).
#pragma once
#include <tensor/adapter/adapter_model.hpp>
#include <tensor/backend/cuda/device.hpp>

namespace tensor::trainer {

struct AdamW {
    float beta1 = 0.9f;
    float beta2 = 0.999f;
    float eps = 1e-8f;
    float weight_decay = 0.f;

    explicit AdamW(const adapter::AdapterConfig& cfg)
        : beta1(cfg.adam_beta1), beta2(cfg.adam_beta2), weight_decay(cfg.weight_decay) {}

    // A then B of one pair from its gA / gB; step is 1-based (bias
    // correction exponent).
    void step(adapter::LoraPair& lp, float lr, int step, const backend::cuda::Device& dev) const;

    // Every pair of every layer, q, k, v, o in order.
    void step_all(adapter::AdapterModel& model, float lr, int step,
                  const backend::cuda::Device& dev) const;
};

}  // namespace tensor::trainer
