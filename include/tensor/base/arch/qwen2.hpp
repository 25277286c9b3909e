// Qwen2Base — the per-op forward and backward of the frozen Qwen2 base, with
// the LoRA pairs of an AdapterModel applied when one is given.  Same types,
// fields and signatures as the reference's include/tensor/base/arch/qwen2.hpp
// (17-74; src/base/arch/qwen2.cu:47-308), for callers that build the
// training step from these classes instead of AdaptTrainer.
//
// Every op runs on this backend's kernels (ops::, gemm_bf16) on the
// Device's stream, in the reference's order and with its BF16 rounding
// points; the forward keeps every activation the backward reads in the
// layer cache, attention probabilities included ([B, Hq, T, T] F32 per
// layer, zero above the diagonal).  The fused step engine behind
// AdaptTrainer (include/ta_engine.h) computes the same step without those
// caches and is the fast path; this one is the reference's composition.
// Tensors returned here come from the backend's caching allocator.
#pragma once
#include <vector>

#include <tensor/backend/cuda/device.hpp>
#include <tensor/backend/cuda/tensor.hpp>
#include <tensor/base/frozen_base.hpp>

namespace tensor::adapter {
class AdapterModel;
}

namespace tensor::base::arch {

using backend::cuda::Device;
using backend::cuda::Tensor;

// What one layer's backward reads, saved by the forward.
struct Qwen2LayerCache {
    Tensor pre_attn_res;  // layer input (residual stream), BF16 [BT, H]
    Tensor in_norm_rms;   // inverse RMS of the input norm, F32 [BT]
    Tensor x_normed;      // input norm output, BF16 [BT, H]

    Tensor Q, K, V;       // after bias, LoRA and RoPE
    Tensor attn_out;      // BF16 [BT, Hq*hd]
    Tensor attn_w;        // probabilities, F32 [B, Hq, T, T]
    Tensor h_mid;         // o projection output (with its LoRA delta)

    Tensor pre_ffn_res;   // residual after attention
    Tensor post_norm_rms;
    Tensor x_normed2;

    Tensor gate_out;      // BF16 [BT, I]
    Tensor up_out;
    Tensor act_out;       // silu(gate) * up
    Tensor ffn_out;       // down projection output, BF16 [BT, H]
};

struct Qwen2ForwardResult {
    Tensor embed_in;  // embedding rows of the tokens
    std::vector<Qwen2LayerCache> layer_cache;

    Tensor x_final;    // residual after the last layer
    Tensor final_rms;  // inverse RMS of the final norm

    Tensor logits;   // BF16 [BT, V]
    Tensor dlogits;  // BF16 [BT, V], allocated here and filled by the caller's loss
};

class Qwen2Base {
public:
    // Per-layer input gradients the backward returns.
    struct LayerGrads {
        Tensor dQ;  // after RoPE backward (pre-RoPE gradient)
        Tensor dK;
        Tensor dV;
        Tensor do_proj;  // gradient of the o projection's output

        Tensor dx_attn_in;  // gradient at the input norm's output
        Tensor dx_ffn_in;   // gradient at the post-attention norm's output
    };

    // tokens: I32 [B*T] on the device.  adapter (may be null): its q, k, v
    // and o pairs are added to the projections (AdapterModel::apply_lora_fwd).
    static Qwen2ForwardResult forward(const FrozenBase& base, const Tensor& tokens, int B, int T,
                                      const Device& dev, adapter::AdapterModel* adapter = nullptr);

    // From fwd.dlogits down to the first layer; the adapter's pairs
    // accumulate their gA and gB (AdapterModel::apply_lora_bwd) and add
    // their input gradients into the layer's.
    static std::vector<LayerGrads> backward(const FrozenBase& base, const Qwen2ForwardResult& fwd,
                                            int B, int T, const Device& dev,
                                            adapter::AdapterModel* adapter = nullptr);
};

}  // namespace tensor::base::arch
