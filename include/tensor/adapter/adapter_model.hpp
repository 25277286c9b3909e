// AdapterModel — the per-op LoRA adapter: per layer a LoRA pair for each of
// q, k, v and o, with BF16 working weights, F32 masters, AdamW moments and
// F32 gradient accumulators.  Same types, fields and signatures as the
// reference's include/tensor/adapter/adapter_model.hpp:18-95
// (src/adapter/adapter_model.cu:15-229), on this backend's GEMMs and ops.
//
// As in the reference, this per-op model always holds q, k, v and o pairs
// (AdapterConfig's inject flags do not change it); the step engine behind
// AdaptTrainer honours every flag, gate, up and down included.  A starts
// from the reference's hashed Kaiming-uniform values (the same for every
// pair), B from zeros; scale = alpha / rank.
#pragma once
#include <cstddef>
#include <string>
#include <vector>

#include <tensor/adapter/adapter_config.hpp>
#include <tensor/backend/cuda/device.hpp>
#include <tensor/backend/cuda/tensor.hpp>
#include <tensor/base/arch/qwen2.hpp>
#include <tensor/base/frozen_base.hpp>

namespace tensor::adapter {

using backend::cuda::Device;
using backend::cuda::Tensor;

// One projection's pair: delta = scale * (x A^T) B^T.
struct LoraPair {
    Tensor A_bf16, B_bf16;  // working weights, BF16: A [rank, in], B [out, rank]
    Tensor A_f32, B_f32;    // F32 masters
    Tensor mA, vA;          // AdamW moments of A
    Tensor mB, vB;          // ... of B
    Tensor gA, gB;          // F32 gradient accumulators

    int in_dim = 0;
    int out_dim = 0;
    int rank = 0;
};

struct LayerAdapter {
    LoraPair lora_q;
    LoraPair lora_k;
    LoraPair lora_v;
    LoraPair lora_o;
};

class AdapterModel {
public:
    static AdapterModel create(const base::FrozenBase& base, const AdapterConfig& cfg,
                               const Device& dev);

    // out[BT, out_dim] = bf16(out + scale * bf16(bf16(x A^T) B^T)), in place.
    void apply_lora_fwd(std::size_t layer, LoraPair& lp, const Tensor& x, Tensor& out, int BT,
                        const Device& dev);

    // With h = bf16(x A^T) recomputed and dh = bf16(grad_out B):
    //   gB += scale * grad_out^T h,  gA += scale * dh^T x   (F32 GEMMs)
    //   grad_x = bf16(grad_x + scale * dh A)                 (accumulated)
    void apply_lora_bwd(LoraPair& lp, const Tensor& x, const Tensor& grad_out, Tensor& grad_x,
                        int BT, const Device& dev);

    void zero_grad(const Device& dev);

    // rank * (in_dim + out_dim) summed over every pair
    std::size_t param_count() const;

    const AdapterConfig& config() const { return cfg_; }

    std::vector<LayerAdapter> layers;

private:
    AdapterConfig cfg_;

    static LoraPair make_pair(int in_dim, int out_dim, int rank, const Device& dev);
};

}  // namespace tensor::adapter
