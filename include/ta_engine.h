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

/* AdapterConfig fields used by the step (include/tensor/adapter/adapter_config.hpp:25-70).
 * rank: 1..64 (the reference's rank ladder tops out at 64); any rank in that
 * range trains exactly that rank, laid out internally at the next multiple
 * of 16 with zero extra rows of A and columns of B. */
typedef struct ta_adapt_config {
    int rank;
    float alpha;
    int inject_mask;
    float lr, grad_clip;
    int64_t warmup, total_steps;
    float b1, b2, eps, wd;
} ta_adapt_config;

/* StepMetrics (include/tensor/trainer/adapt_trainer.hpp:18-27) plus the raw
 * norm and nonfinite_logits: the number of NaN and Inf logits of the step
 * when it was the engine's first (step count 0 before it; the reference
 * checks the logits at step 0 only, adapt_trainer.cu:76-91,196-198), -1 on
 * later steps, which do not count them. */
typedef struct ta_step_metrics {
    float loss, lr, gnorm, gnorm_raw;
    int valid_tokens, step;
    double step_ms;
    int nonfinite_logits;
} ta_step_metrics;

/* Allocates the base (W and W^T of every projection), the adapter arena and
 * every activation buffer for batch B x T once; nothing is allocated per
 * step.  stream: hipStream_t (NULL = a stream the engine creates).
 * Returns NULL on failure. */
void* ta_engine_create(const ta_model_config* model, const ta_adapt_config* adapt, int B, int T,
                       void* stream);

/* ta_engine_create with creation flags.  No counterpart in the reference,
 * which caches every layer's activations (Qwen2LayerCache,
 * include/tensor/base/arch/qwen2.hpp:17-35); it is for long-sequence and
 * large-model runs such as the Qwen2-7B-shaped config at B=4 x T=2048.
 *   TA_ENGINE_RECOMPUTE: keep only each layer's input per layer; the
 *   backward reruns a layer's forward into one shared activation set just
 *   before that layer's backward.  Results are bit-identical to the cached
 *   step; the cost is one more forward of every layer but the last.
 * Named buffers of the shared set read as "work.<name>" ("work.x_normed").
 *   TA_ENGINE_CE_IN_DX: the cross entropy writes no dlogits, only the loss
 *   and each row's normaliser; the LM head's input-gradient GEMM forms
 *   dlogits from the logits as it reads them (bit-identical results; the
 *   "logits" buffer then keeps the logits).  Measured slower than the
 *   default two-pass form on MI355X (the exponentials run once per output
 *   column tile instead of once); kept as the measured alternative.  Needs
 *   vocab % 64 == 0, vocab <= 163840, hidden >= 192 and B*T >= 256, else the
 *   step uses the default form. */
enum { TA_ENGINE_RECOMPUTE = 1, TA_ENGINE_CE_IN_DX = 2 };
void* ta_engine_create_ex(const ta_model_config* model, const ta_adapt_config* adapt, int B, int T,
                          void* stream, int flags);
int ta_engine_destroy(void* engine);

/* Upload one base tensor by its HF name (e.g. "model.layers.3.mlp.up_proj.weight"),
 * BF16 bits from host memory, n elements (BaseLoader::load, src/base/base_loader.cpp:75-172). */
int ta_engine_set_weight(void* engine, const char* name, const uint16_t* host_data, int64_t n);

/* ta_engine_set_weight from device memory: n BF16 elements at src, copied on
 * the engine's stream (the caller makes sure src is ready on that stream;
 * the C++ AdaptTrainer loads its FrozenBase's device tensors this way). */
int ta_engine_set_weight_device(void* engine, const char* name, const uint16_t* src, int64_t n);

/* Add the centroid side channel of every later step into the caller's
 * device F64 vector [hidden + 1] (sums, then total weight) instead of the
 * engine's own; NULL returns to the engine's own.  The vector is updated on
 * the engine's stream.  (AdaptTrainer points it at its CentroidAccumulator,
 * as the reference's trainer feeds CentroidAccumulator::accumulate,
 * src/trainer/adapt_trainer.cu:210-232.) */
int ta_engine_set_centroid(void* engine, double* d_acc);

/* Set the number of steps already taken (0 after create): the next step
 * uses the schedule's lr_at(step) and AdamW's t = step + 1
 * (adapt_trainer.cu:252-253).  For resuming from a saved state. */
int ta_engine_set_step(void* engine, int64_t step);

/* Synthetic base on the device: every linear weight and the embedding
 * ~ N(0, std) from `seed` (per-tensor streams), norm weights 1, biases 0. */
int ta_engine_init_random(void* engine, uint64_t seed, float std);

/* One training step on host token ids [B*T] (inputs and next-token
 * targets as Dataset::next_batch gives them).  lr_override > 0 replaces the
 * cosine schedule.  metrics may be NULL. */
int ta_engine_step(void* engine, const int32_t* inputs, const int32_t* targets,
                   float lr_override, ta_step_metrics* metrics);

/* Same step with the batch already resident in device memory (int32 [B*T]
 * each; the assistant-span masking runs on the device).  No host-to-device
 * transfer happens inside the step.  Token ids are checked on the device:
 * an id outside [0, vocab) is never used as an index, and the call then
 * returns an error with the adapter state, the step count and the centroid
 * sums unchanged (targets outside [0, vocab) contribute only logsumexp to
 * the loss, as target -1 does). */
int ta_engine_step_resident(void* engine, const int32_t* d_inputs, const int32_t* d_targets,
                            float lr_override, ta_step_metrics* metrics);

/* Kernel-class timing during real steps.  category (TA_CAT_*) selects which
 * launches are bracketed with HIP events on the engine's stream (-1: none);
 * each step then adds their summed duration, launch count and algorithmic
 * work (flops for MFMA GEMMs and attention, HBM bytes for streaming
 * kernels) to the totals, which ta_engine_profile_read returns and clears. */
enum {
    TA_CAT_GEMM_FWD = 0, /* frozen-base projections, forward: x W^T        */
    TA_CAT_GEMM_DX = 1,  /* frozen-base input gradients: dY W              */
    TA_CAT_LMHEAD = 2,   /* LM head forward GEMM (logits)                 */
    TA_CAT_LORA = 3,     /* every LoRA GEMM (fwd h, delta; bwd gB, dh, gA, dx) */
    TA_CAT_ATTN_FWD = 4,
    TA_CAT_ATTN_BWD = 5,
    TA_CAT_NORM = 6,     /* RMSNorm forward + backward                    */
    TA_CAT_ELEMWISE = 7, /* SiLU fwd/bwd, RoPE, residual/LoRA adds        */
    TA_CAT_CE = 8,
    TA_CAT_TAIL = 9,     /* grad norm + clip + AdamW                      */
    TA_CAT_CENTROID = 10,
    TA_CAT_LMHEAD_BWD = 11, /* LM head input-gradient GEMM: dlogits W     */
    TA_NCAT = 12
};
int ta_engine_profile(void* engine, int category);
int ta_engine_profile_read(void* engine, double* total_ms, int64_t* launches, double* flops,
                           double* bytes);

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
 * "l3.Q", "l3.attn_stats" (each attention row's max in base-2 units and
 * 1/sum: the probabilities are recomputed from them, not stored), "logits"
 * (holds dlogits after a step), "loss_tok",
 * "targets" (the masked int32 targets of the last step; is_f32 = 1 marks its
 * 4-byte elements), ... */
void* ta_engine_buffer(void* engine, const char* name, int64_t* n_elems, int* is_f32);
/* Copy n elements of a named buffer to host memory (2 bytes each for BF16
 * buffers, 4 for F32), after the engine's stream is idle. */
int ta_engine_read_buffer(void* engine, const char* name, void* host_dst, int64_t n);

/* Per-phase timing of the last step in ms (forward, backward, tail), measured
 * with events on the engine's stream. */
int ta_engine_phase_ms(void* engine, float* fwd_ms, float* bwd_ms, float* tail_ms);

/* The step's learning rate: CosineSchedule::lr_at
 * (include/tensor/trainer/cosine_schedule.hpp:18-29) for the 0-based step,
 * as the engine applies it (adapt_trainer.cu:252).  Host only. */
float ta_cosine_lr(float base_lr, int64_t warmup, int64_t total, float floor_frac, int64_t step);

#ifdef __cplusplus
}
#endif
#endif /* TA_ENGINE_H */
