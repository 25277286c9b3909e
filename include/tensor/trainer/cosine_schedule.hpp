// Learning-rate schedule of the trainer: linear warmup over warmup_steps,
// then cosine decay from base_lr to base_lr * floor_frac at total_steps
// (reference: include/tensor/trainer/cosine_schedule.hpp:18-29; `step` is the
// 0-based optimizer step, as adapt_trainer.cu:252 passes it).  F32
// arithmetic in the reference's order, so the values agree bit for bit.
#pragma once
#include <algorithm>
#include <cmath>
#include <cstddef>

namespace tensor::trainer {

struct CosineSchedule {
    float base_lr;
    std::size_t warmup_steps;
    std::size_t total_steps;
    float floor_frac = 0.1f;

    float lr_at(std::size_t step) const {
        if (step < warmup_steps) return base_lr * (float)(step + 1) / (float)warmup_steps;
        float t = (float)(step - warmup_steps) / (float)(total_steps - warmup_steps);
        t = std::min(t, 1.f);
        const float pi = 3.14159265358979323846f;
        float c = 0.5f * (1.f + std::cos(pi * t));
        float lo = base_lr * floor_frac;
        return lo + (base_lr - lo) * c;
    }
};

}  // namespace tensor::trainer
