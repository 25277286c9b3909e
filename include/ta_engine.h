/* ta_engine.h — C-ABI of the MI355X step engine: one LoRA training step
 * (forward, cross entropy, backward with frozen-base input gradients and
 * LoRA A/B gradients, centroid side channel, grad-norm/clip, AdamW) over a
 * frozen BF16 Qwen2 base resident in HBM.
 *
 * It replaces the device-side body of AdaptTrainer::Impl::do_step
 * (src/trainer/adapt_trainer.cu:130-277) together with Qwen2Base::forward /
 * backward (src/base/arch/qwen2.cu:47-308), AdapterModel::apply_lora_fwd /
 * apply_lora_bwd / zero_grad (src/adapter/adapter_model.cu:96-229),
 * AdamW::step_all (src/trainer/adamw.cu:9-38) and the trainer's feed of
 * CentroidAccumulator::accumulate (adapt_trainer.cu:210-232).  The host
 * parts the reference keeps on the CPU (assistant-span masking, loss mean,
 * cosine schedule) run here on the host in the same order.
 *
 * Extension (the reference always trains q,k,v,o and has no MLP LoRA):
 * inject_mask bits 0..6 select {q,k,v,o,gate,up,down}; gate/up LoRA is added
 * before SiLU, down LoRA before the residual add; absent pairs take no part
 * in forward, backward, grad norm or AdamW.
 *
 * All calls return 0 on success or a negative status (ta_last_error()).
 */
#ifndef TA_ENGINE_H
#define TA_ENGINE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Qwen2 shape — BaseConfig (include/tensor/base/frozen_base.hpp:15-56). */
typedef struct ta_model_config {
    int vocab, hidden, layers, n_q, n_kv, head_dim, inter;
    float rms_eps, rope_theta;
    int tie; /* 1: LM head = embedding (qwen2.cu:163) */
} ta_model_config;

/* AdapterConfig fields used by the step (include/tensor/adapter/adapter_config.hpp:25-70). */
typedef struct ta_adapt_config {
    int rank;
    float alpha;
    int inject_mask;
    float lr, grad_clip;
    int64_t warmup, total_steps;
    float b1, b2, eps, wd;
} ta_adapt_config;

/* StepMetrics (include/tensor/trainer/adapt_trainer.hpp:18-27) plus the raw norm. */
typedef struct ta_step_metrics {
    float loss, lr, gnorm, gnorm_raw;
    int valid_tokens, step;
    double step_ms;
} ta_step_metrics;

/* Allocates the base (W and W^T of every projection), the adapter arena and
 * every activation buffer for batch B x T once; nothing is allocated per
 * step.  stream: hipStream_t (NULL = a stream the engine creates).
 * Returns NULL on failure. */
void* ta_engine_create(const ta_model_config* model, const ta_adapt_config* adapt, int B, int T,
                       void* stream);
int ta_engine_destroy(void* engine);

/* Upload one base tensor by its HF name (e.g. "model.layers.3.mlp.up_proj.weight"),
 * BF16 bits from host memory, n elements (BaseLoader::load, src/base/base_loader.cpp:75-172). */
int ta_engine_set_weight(void* engine, const char* name, const uint16_t* host_data, int64_t n);

/* Synthetic base on the device: every linear weight and the embedding
 * ~ N(0, std) from `seed` (per-tensor streams), norm weights 1, biases 0. */
int ta_engine_init_random(void* engine, uint64_t seed, float std);

/* One training step on host token ids [B*T] (inputs and next-token
 * targets as Dataset::next_batch gives them).  lr_override > 0 replaces the
 * cosine schedule.  metrics may be NULL. */
int ta_engine_step(void* engine, const int32_t* inputs, const int32_t* targets,
                   float lr_override, ta_step_metrics* metrics);

/* Copy adapter state to host memory.  target: 0..6 = q,k,v,o,gate,up,down;
 * which: 0 A master, 1 B master, 2 mA, 3 vA, 4 mB, 5 vB, 6 gA, 7 gB (F32),
 * 8 A shadow, 9 B shadow (BF16).  n must equal the tensor's element count. */
int ta_engine_read_adapter(void* engine, int layer, int target, int which, void* host_dst,
                           int64_t n);
/* Overwrite adapter state from host memory (same indexing as read); used to
 * resume from a saved state or to align two implementations before a step.
 * Writing a master does not refresh its BF16 shadow: write both. */
int ta_engine_write_adapter(void* engine, int layer, int target, int which, const void* host_src,
                            int64_t n);

/* Centroid accumulator (F64 [hidden + 1]: weighted sums, then total weight). */
int ta_engine_centroid(void* engine, double* host_out);

/* Device pointer of a cached activation, for parity checks: "l3.x_normed",
 * "l3.Q", "l3.attn_w", "logits" (holds dlogits after a step), "loss_tok", ... */
void* ta_engine_buffer(void* engine, const char* name, int64_t* n_elems, int* is_f32);
/* Copy n elements of a named buffer to host memory (2 bytes each for BF16
 * buffers, 4 for F32), after the engine's stream is idle. */
int ta_engine_read_buffer(void* engine, const char* name, void* host_dst, int64_t n);

/* Per-phase timing of the last step in ms (forward, backward, tail), measured
 * with events on the engine's stream. */
int ta_engine_phase_ms(void* engine, float* fwd_ms, float* bwd_ms, float* tail_ms);

#ifdef __cplusplus
}
#endif
#endif /* TA_ENGINE_H */
