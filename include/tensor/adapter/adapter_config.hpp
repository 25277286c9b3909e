// AdapterConfig — LoRA capacity, injection targets, optimiser and batch
// settings of one training run.  Same fields, defaults and factory as the
// reference's include/tensor/adapter/adapter_config.hpp:25-70
// (src/adapter/adapter_config.cpp), plus inject_gate: the reference has no
// gate-projection flag and trains q, k, v and o whatever the flags say; here
// every flag selects its projection (inject_gate defaults to off, so a
// configuration the reference accepts trains what its flags name).
#pragma once
#include <cstddef>
#include <string>

#include <tensor/backend/cuda/device.hpp>
#include <tensor/base/frozen_base.hpp>

namespace tensor::adapter {

struct AdapterConfig {
    // LoRA capacity: rank ladder by base size in for_base()
    int rank = 16;
    float alpha = 16.f;  // effective scale alpha / rank
    float scale() const { return alpha / (float)rank; }

    bool inject_q = true;
    bool inject_k = true;
    bool inject_v = true;
    bool inject_o = true;
    bool inject_up = false;
    bool inject_down = false;
    bool inject_gate = false;  // extension (no reference counterpart)

    // optimiser
    float lr = 2e-4f;
    float grad_clip = 1.f;
    std::size_t warmup_steps = 200;
    float adam_beta1 = 0.9f;
    float adam_beta2 = 0.999f;
    float adam_eps = 1e-8f;
    float weight_decay = 0.f;

    // batch / sequence
    std::size_t batch_size = 4;
    std::size_t seq_len = 2048;

    // metadata, filled by for_base()
    std::string architecture;
    std::size_t base_parameters = 0;

    // inject_q .. inject_down as the step engine's mask (bits q,k,v,o,gate,up,down)
    int inject_mask() const {
        return (inject_q ? 1 : 0) | (inject_k ? 2 : 0) | (inject_v ? 4 : 0) | (inject_o ? 8 : 0) |
               (inject_gate ? 16 : 0) | (inject_up ? 32 : 0) | (inject_down ? 64 : 0);
    }

    // Rank, alpha, up/down injection and warmup from the base's parameter
    // count; batch and sequence from the device memory left free after the
    // base is loaded (src/adapter/adapter_config.cpp:50-120).
    static AdapterConfig for_base(const base::FrozenBase& base, const backend::cuda::Device& dev);
};

}  // namespace tensor::adapter
