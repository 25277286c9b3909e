// ops:: — the kernel entry points the training step calls, with the
// reference's names, argument order and meaning
// (include/tensor/backend/cuda/ops.hpp:12-154), on HIP streams.  Each call
// launches asynchronously on `stream` and throws CudaError if the backend
// rejects the arguments or the launch fails (the reference returned void and
// left launches unchecked).  BF16 tensors are uint16_t bit patterns.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdint>

#include <tensor/backend/cuda/device.hpp>

namespace tensor::backend::cuda::ops {

using bf16_t = std::uint16_t;

// RMSNorm; rms_out receives the inverse RMS per row (ops.cu:84-86).
void rms_norm_fwd(const bf16_t* x, const bf16_t* w, bf16_t* out, float* rms_out, int B, int T,
                  int D, float eps, hipStream_t stream);
// dw (may be null) is accumulated (+=) in a fixed order.
void rms_norm_bwd(const bf16_t* dy, const bf16_t* x, const bf16_t* w, const float* rms_saved,
                  bf16_t* dx, float* dw, int B, int T, int D, float eps, hipStream_t stream);

// RoPE on interleaved pairs, in place.
void rope_fwd(bf16_t* x, int B, int T, int H, int head_dim, float theta, hipStream_t stream);
void rope_bwd(bf16_t* dx, int B, int T, int H, int head_dim, float theta, hipStream_t stream);

// Causal GQA attention; attn_w [B*Hq, T, T] F32 probabilities.
void sdpa_fwd(const bf16_t* Q, const bf16_t* K, const bf16_t* V, bf16_t* out, float* attn_w,
              int B, int T, int Hq, int Hkv, int head_dim, const Device& dev);
// dQ, dK, dV are overwritten.
void sdpa_bwd(const bf16_t* dout, const bf16_t* Q, const bf16_t* K, const bf16_t* V,
              const float* attn_w, bf16_t* dQ, bf16_t* dK, bf16_t* dV, int B, int T, int Hq,
              int Hkv, int head_dim, const Device& dev);

void silu_mul_fwd(const bf16_t* gate, const bf16_t* up, bf16_t* out, int N, hipStream_t stream);
void silu_mul_bwd(const bf16_t* dout, const bf16_t* gate, const bf16_t* up, bf16_t* dgate,
                  bf16_t* dup, int N, hipStream_t stream);

// Per-row loss (target < 0: logsumexp) and dlogits = (softmax - onehot)/N.
void cross_entropy_fwd(const bf16_t* logits, const int* targets, float* loss_out,
                       bf16_t* dlogits, int N, int V, hipStream_t stream);

void embed_fwd(const bf16_t* table, const int* tokens, bf16_t* out, int BT, int D,
               hipStream_t stream);
void embed_bwd(const bf16_t* dout, const int* tokens, float* dtable, int BT, int D,
               hipStream_t stream);

void add_bias(bf16_t* out, const bf16_t* bias, int BT, int D, hipStream_t stream);
void add_inplace(bf16_t* out, const bf16_t* delta, int N, hipStream_t stream);
void lora_add(bf16_t* out, const bf16_t* lora_delta, float scale, int N, hipStream_t stream);

void cast_bf16_to_f32(const bf16_t* src, float* dst, int N, hipStream_t s);
void cast_f32_to_bf16(const float* src, bf16_t* dst, int N, hipStream_t s);

// AdamW on one tensor; step is the 1-based bias-correction exponent.
void adamw_step(float* master, bf16_t* working, float* m, float* v, const float* grad, int N,
                float lr, float beta1, float beta2, float eps, float weight_decay, int step,
                hipStream_t stream);

// *accum += sum g^2 (fixed-order reduction, no atomics).
void sum_sq_into(const float* g, float* accum, int N, hipStream_t s);

// ── additions of this backend (no reference counterpart) ──────────────
// Grad norm, clip and AdamW over one flat parameter arena in one pass
// (replaces compute_grad_norm + clip_gradients + AdamW::step_all).
void adamw_fused(float* master, bf16_t* working, float* m, float* v, float* grad,
                 std::int64_t N, float lr, float beta1, float beta2, float eps,
                 float weight_decay, int step, float max_norm, float* norm_out,
                 hipStream_t stream);
// acc[d] += h[t,d] * ||g_t||, acc[D] += ||g_t|| over BT tokens (F64 acc).
void centroid_accumulate(const bf16_t* h, const bf16_t* g, std::int64_t BT, int D, double* acc,
                         hipStream_t stream);

}  // namespace tensor::backend::cuda::ops
