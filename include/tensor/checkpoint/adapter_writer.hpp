// AdapterWriter — the adapter artefacts of a run, in the reference's formats
// (src/checkpoint/adapter_writer.cpp:30-150):
//   adapter.safetensors  every LoRA A and B, F32 masters rounded to BF16
//                        (round to nearest even), flat 1-D shapes, header
//                        keys in sorted order, data in tensor order
//                        (layer by layer; q, k, v, o, then gate, up, down;
//                        lora_A before lora_B), header padded with spaces to
//                        a multiple of 8 bytes; the tensor set is the
//                        projections the AdapterConfig's inject flags name
//                        (the reference writes q, k, v and o whatever they
//                        say, so a configuration with MLP targets or without
//                        one of q, k, v, o writes a different set);
//   adapter.json         run metadata, 2-space indented, keys sorted;
//   train_state.json     {"step", "tokens_consumed"} (checkpoints only).
// A checkpoint here also stores optimizer.safetensors: each tensor's F32
// master and AdamW moments (names <name>, <name>.exp_avg, <name>.exp_avg_sq)
// and the centroid sums (centroid.sums, F64 [hidden + 1]), which
// AdaptTrainer reads back when AdaptOptions::resume_from names the
// checkpoint.  The reference declares resume_from but never reads it, and
// its checkpoint holds no optimiser state.
#pragma once
#include <cstddef>
#include <string>
#include <vector>

#include <tensor/adapter/adapter_config.hpp>
#include <tensor/base/frozen_base.hpp>

namespace tensor::checkpoint {

// One adapter tensor as the writer stores it.
struct AdapterTensor {
    std::string name;                         // e.g. "layers.3.self_attn.q_proj.lora_A"
    std::vector<float> value;                 // F32 master
    std::vector<float> exp_avg, exp_avg_sq;   // AdamW m, v (checkpoints)
};

// safetensors name prefix of projection p (0..6 = q,k,v,o,gate,up,down) in layer l
std::string lora_prefix(std::size_t layer, int proj);

class AdapterWriter {
public:
    explicit AdapterWriter(const std::string& base_output_dir);

    // adapter.safetensors, adapter.json, train_state.json and
    // optimizer.safetensors (with the centroid sums) into ckpt_dir.
    void save_checkpoint(const std::vector<AdapterTensor>& tensors,
                         const std::vector<double>& centroid_sums,
                         const adapter::AdapterConfig& cfg, const base::FrozenBase& base,
                         const std::string& domain, std::size_t step, std::size_t tokens,
                         const std::string& ckpt_dir);

    // adapter.safetensors and adapter.json into out_dir.
    void save_final(const std::vector<AdapterTensor>& tensors, const adapter::AdapterConfig& cfg,
                    const base::FrozenBase& base, const std::string& domain, std::size_t step,
                    std::size_t tokens, const std::string& out_dir);

private:
    std::string base_dir_;
};

// The three files, one at a time (the writer's building blocks; also used
// by tests).
void write_adapter_safetensors(const std::string& path, const std::vector<AdapterTensor>& tensors);
void write_optimizer_safetensors(const std::string& path,
                                 const std::vector<AdapterTensor>& tensors,
                                 const std::vector<double>& centroid_sums);
std::string adapter_json(const adapter::AdapterConfig& cfg, const base::BaseConfig& bc,
                         const std::string& domain, std::size_t step, std::size_t tokens);

// A checkpoint's optimiser state and counters, as save_checkpoint wrote them.
struct TrainState {
    std::size_t step = 0, tokens_consumed = 0;
    std::vector<AdapterTensor> tensors;  // value, exp_avg, exp_avg_sq filled
    std::vector<double> centroid_sums;
};
// Throws std::runtime_error when a file is missing or malformed.
TrainState load_checkpoint(const std::string& ckpt_dir);

}  // namespace tensor::checkpoint
