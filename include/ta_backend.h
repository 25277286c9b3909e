/* ta_backend.h — C-ABI of the MI355X (gfx950) backend for tensor-adapt's
 * LoRA training step.
 *
 * Every entry point is `extern "C"`, takes plain device pointers, sizes and
 * scalars, launches asynchronously on `stream` (a hipStream_t passed as
 * void*, NULL = the default stream) and returns 0 on success or a negative
 * status; ta_last_error() then holds the message.  BF16 tensors are passed as
 * uint16_t bit patterns.  Nothing here allocates on the caller's behalf unless
 * the comment says so; ops that need scratch memory draw it from the
 * library's pool, one set of grow-only buffers per (device, stream), so
 * calls on different streams never share scratch.  A stream's buffers live
 * until ta_scratch_release(stream) or the process ends: release them before
 * destroying a stream (a new stream may get the old handle value).
 *
 * Each declaration names the reference function it replaces (paths are in
 * carbon-os/tensor-adapt).  Layout conventions are the reference's: activations
 * row-major [B*T, features], attention probabilities [B*Hq, T, T] F32,
 * GEMMs in cuBLAS column-major semantics.
 */
#ifndef TA_BACKEND_H
#define TA_BACKEND_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ── status ─────────────────────────────────────────────────────────── */
/* Message of the most recent failing call on this thread ("" if none). */
const char* ta_last_error(void);
/* Library version string (build date + target). */
const char* ta_version(void);

/* ── RMSNorm ────────────────────────────────────────────────────────
 * replaces ops::rms_norm_fwd  include/tensor/backend/cuda/ops.hpp:12-18
 *          (kernel src/backend/cuda/ops.cu:59-107).
 * rms_out[row] receives the INVERSE rms, as in the reference. */
int ta_rms_norm_fwd(const uint16_t* x, const uint16_t* w, uint16_t* out, float* rms_out,
                    int B, int T, int D, float eps, void* stream);

/* replaces ops::rms_norm_bwd  ops.hpp:20-27 (ops.cu:113-170).
 * dw may be NULL (the trainer's weights are frozen); when given it is
 * accumulated (+=) with a fixed-order reduction instead of F32 atomics. */
int ta_rms_norm_bwd(const uint16_t* dy, const uint16_t* x, const uint16_t* w,
                    const float* rms_saved, uint16_t* dx, float* dw,
                    int B, int T, int D, float eps, void* stream);

/* ── RoPE (interleaved pairs) ───────────────────────────────────────
 * replaces ops::rope_fwd / ops::rope_bwd  ops.hpp:30-40 (ops.cu:176-204). In place. */
int ta_rope_fwd(uint16_t* x, int B, int T, int H, int head_dim, float theta, void* stream);
int ta_rope_bwd(uint16_t* dx, int B, int T, int H, int head_dim, float theta, void* stream);

/* ── causal GQA attention with saved probabilities ──────────────────
 * replaces ops::sdpa_fwd  ops.hpp:49-56 (ops.cu:578-681).
 * attn_w: [B*Hq, T, T] F32 probabilities (zeros above the diagonal). */
int ta_sdpa_fwd(const uint16_t* Q, const uint16_t* K, const uint16_t* V, uint16_t* out,
                float* attn_w, int B, int T, int Hq, int Hkv, int head_dim, void* stream);

/* replaces ops::sdpa_bwd  ops.hpp:58-69 (ops.cu:707-870).  dQ/dK/dV are
 * overwritten, as in the reference's batched path. */
int ta_sdpa_bwd(const uint16_t* dout, const uint16_t* Q, const uint16_t* K,
                const uint16_t* V, const float* attn_w, uint16_t* dQ, uint16_t* dK,
                uint16_t* dV, int B, int T, int Hq, int Hkv, int head_dim, void* stream);

/* The step engine's attention, which keeps no probabilities (no
 * counterpart in the reference, whose sdpa_fwd stores P for sdpa_bwd):
 * the forward writes O [B*T, Hq*hd] BF16, its F32 copy O32 (may be NULL)
 * and, per (b, hq, query row), the row's score maximum in base-2 units and
 * 1/sum of its exponentials as an F32 pair in stats [B*Hq*T][2]; the
 * backward recomputes P = exp2(S*scale*log2(e) - max) * (1/sum) from Q, K
 * and those pairs, takes the row dots dO.O from O32 (required), and
 * overwrites dQ/dK/dV as ta_sdpa_bwd does. */
int ta_attn_fwd_rowstats(const uint16_t* Q, const uint16_t* K, const uint16_t* V, uint16_t* O,
                         float* O32, float* stats, int B, int T, int Hq, int Hkv, int head_dim,
                         void* stream);
int ta_attn_bwd_rowstats(const uint16_t* dout, const uint16_t* Q, const uint16_t* K,
                         const uint16_t* V, const float* stats, const float* O32, uint16_t* dQ,
                         uint16_t* dK, uint16_t* dV, int B, int T, int Hq, int Hkv, int head_dim,
                         void* stream);

/* ── gated SiLU ─────────────────────────────────────────────────────
 * replaces ops::silu_mul_fwd / silu_mul_bwd  ops.hpp:72-86 (ops.cu:913-952). */
int ta_silu_mul_fwd(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t N,
                    void* stream);
int ta_silu_mul_bwd(const uint16_t* dout, const uint16_t* gate, const uint16_t* up,
                    uint16_t* dgate, uint16_t* dup, int64_t N, void* stream);

/* ── cross entropy ──────────────────────────────────────────────────
 * replaces ops::cross_entropy_fwd  ops.hpp:89-95 (ops.cu:958-1020).
 * target < 0 still reports logsumexp and receives softmax/N gradient; the
 * gradient divisor N counts every row, masked or not (ops.cu:997-1009). */
int ta_cross_entropy_fwd(const uint16_t* logits, const int32_t* targets, float* loss_out,
                         uint16_t* dlogits, int N, int V, void* stream);

/* ── embedding ──────────────────────────────────────────────────────
 * replaces ops::embed_fwd / embed_bwd  ops.hpp:98-110 (ops.cu:1026-1051).
 * embed_bwd accumulates (+=) into the F32 dtable with atomics, as the
 * reference does (its trainer never calls it: the embedding is frozen). */
int ta_embed_fwd(const uint16_t* table, const int32_t* tokens, uint16_t* out, int BT, int D,
                 void* stream);
int ta_embed_bwd(const uint16_t* dout, const int32_t* tokens, float* dtable, int BT, int D,
                 void* stream);

/* ── adds ───────────────────────────────────────────────────────────
 * replace ops::add_bias / add_inplace / lora_add  ops.hpp:113-132
 * (ops.cu:1062-1113). Each rounds to BF16 once per output, like the reference. */
int ta_add_bias(uint16_t* out, const uint16_t* bias, int BT, int D, void* stream);
int ta_add_inplace(uint16_t* out, const uint16_t* delta, int64_t N, void* stream);
int ta_lora_add(uint16_t* out, const uint16_t* delta, float scale, int64_t N, void* stream);

/* ── LoRA A initialisation ── replaces the k_kaiming_init / k_kaiming_init_f32
 * pair of AdapterModel::make_pair (src/adapter/adapter_model.cu:15-39,44-50):
 * element i of A ([rank, in_dim] row-major, n = rank * in_dim) is
 * u(i) * sqrt(1 / in_dim), u the reference's 24-bit integer hash of i (seed
 * 0x1234) mapped to [-1, 1]; a32 gets the F32 value, a16 its BF16 rounding
 * (either may be NULL). */
int ta_lora_kaiming_init(float* a32, uint16_t* a16, int64_t n, int in_dim, void* stream);

/* ── casts ── replace ops::cast_bf16_to_f32 / cast_f32_to_bf16  ops.hpp:135-136 */
int ta_cast_bf16_to_f32(const uint16_t* src, float* dst, int64_t N, void* stream);
int ta_cast_f32_to_bf16(const float* src, uint16_t* dst, int64_t N, void* stream);

/* ── AdamW ──────────────────────────────────────────────────────────
 * replaces ops::adamw_step  ops.hpp:139-147 (ops.cu:1139-1169); step is the
 * 1-based bias-correction exponent, as in adamw.cu:9-38. */
int ta_adamw_step(float* master, uint16_t* working, float* m, float* v, const float* grad,
                  int64_t N, float lr, float beta1, float beta2, float eps, float weight_decay,
                  int step, void* stream);

/* replaces ops::sum_sq_into  ops.hpp:153 (ops.cu:1175-1193): *accum += sum g^2.
 * Fixed-order two-level reduction (no F32 atomics). */
int ta_sum_sq_into(const float* g, float* accum, int64_t N, void* stream);

/* Fused multi-tensor tail of the step over ONE flat parameter arena
 * (replaces compute_grad_norm + clip_gradients + AdamW::step_all,
 * src/trainer/adapt_trainer.cu:32-70,248-253 and src/trainer/adamw.cu:9-38):
 *   norm = ||grad||_2 over all n elements;
 *   if norm > max_norm: grad is scaled by max_norm/(norm+1e-6) IN PLACE,
 *     as clip_gradients leaves gA/gB (adapt_trainer.cu:55-70);
 *   AdamW on every element; BF16 shadow written.
 * norm_out (device float, may be NULL) receives the unclipped norm.  The
 * whole tail runs on the device: no host synchronisation. */
int ta_adamw_fused(float* master, uint16_t* working, float* m, float* v, float* grad,
                   int64_t N, float lr, float beta1, float beta2, float eps,
                   float weight_decay, int step, float max_norm, float* norm_out,
                   void* stream);

/* ── GEMM ───────────────────────────────────────────────────────────
 * replaces gemm_bf16 / gemm_f32  include/tensor/backend/cuda/tensor.hpp:79-101
 * (src/backend/cuda/tensor.cu:144-182).  cuBLAS column-major semantics:
 *   C(MxN, ldc) = alpha * op(A) * op(B) + beta * C,
 *   op(A)(i,k) = transA ? A[k + i*lda] : A[i + k*lda]
 *   op(B)(k,j) = transB ? B[j + k*ldb] : B[k + j*ldb]
 * gemm_bf16: BF16 inputs, FP32 accumulation on MFMA, output rounded once
 * to BF16.  gemm_f32: F32 inputs and output with F32 accuracy (cublasSgemm
 * semantics): each operand is split into three BF16 parts carrying its 24
 * significand bits and the six part products down to 2^-24 relative are
 * accumulated in F32 on the BF16 MFMA; it stages the split operands in the
 * scratch pool (at most 256 MB per call, K taken in chunks).
 * Returns -1 for M,N,K,ld <= 0 (tensor.cu:134-142). */
int ta_gemm_bf16(int transA, int transB, int M, int N, int K, float alpha,
                 const uint16_t* A, int lda, const uint16_t* B, int ldb, float beta,
                 uint16_t* C, int ldc, void* stream);
int ta_gemm_f32(int transA, int transB, int M, int N, int K, float alpha, const float* A,
                int lda, const float* B, int ldb, float beta, float* C, int ldc, void* stream);

/* Row-major convenience form used by the step engine (no reference
 * counterpart; it is gemm_bf16 with the operands named the row-major way):
 *   C[m, n] = bf16(alpha * sum_k X(m,k) Y(k,n) + beta * C[m, n] (+ bias[n]))
 *   X(m,k) = x_kmajor ? X[m*ldx + k] : X[k*ldx + m]
 *   Y(k,n) = y_kmajor ? Y[n*ldy + k] : Y[k*ldy + n]
 * bias (may be NULL) is added after the first BF16 rounding and rounded
 * again, which is the reference's gemm + ops::add_bias sequence. */
int ta_gemm_rm(int x_kmajor, int y_kmajor, int M, int N, int K, float alpha,
               const uint16_t* X, int ldx, const uint16_t* Y, int ldy, float beta,
               uint16_t* C, int ldc, const uint16_t* bias, void* stream);

/* ta_gemm_rm with the kernel of the large K-contiguous GEMMs chosen for this
 * one call (tuning sweeps and the kernel-form tests); other calls, on this
 * thread or any other, keep the default:
 * 0 = the default (the pipelined kernel, 192- or 256-wide tiles by N),
 * 7..11 = the 8-/4-wave direct-to-LDS kernel shapes, 12/13 = the 4-wave
 * pipelined kernel with 192/256-wide tiles, 14/15 = its 8-wave 4x2 layout
 * with 256/192-wide tiles, 16 = its 8-wave 2x4 layout (256-wide), 17/18 =
 * the forms of 15/16 with 64-k stages (whole 128-byte operand lines per
 * direct-to-LDS row), 19/20 = the 128-row-tile kernel with 128/64-wide
 * tiles; + 100 x s forces s K splits on the 256-row kernels (F32 partials
 * and an ordered reduce).  Other values return an error.
 * No reference counterpart. */
int ta_gemm_rm_variant(int variant, int x_kmajor, int y_kmajor, int M, int N, int K, float alpha,
                       const uint16_t* X, int ldx, const uint16_t* Y, int ldy, float beta,
                       uint16_t* C, int ldc, const uint16_t* bias, void* stream);

/* ── centroid accumulator ───────────────────────────────────────────
 * replaces CentroidAccumulator::accumulate  src/centroid/centroid_accumulator.cpp:23-70
 * (intended math, see defect D1 there): for each token t,
 *   n_t = ||g_t||_2 ;  acc[d] += h[t,d] * n_t ;  acc[D] += n_t
 * h, g are BF16 [BT, D] (the trainer's x_normed and dx_attn_in, read
 * directly instead of through an F32 cast + host copy).  acc is a device
 * F64 vector of D+1 entries, accumulated in a fixed order. */
int ta_centroid_accumulate_bf16(const uint16_t* h, const uint16_t* g, int64_t BT, int D,
                                double* acc, void* stream);
/* ta_centroid_accumulate_bf16 without any allocation: no counterpart in the
 * reference.  It is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same kernels, same order, same bits as
 * ta_centroid_accumulate_bf16; its partial rows live in a static 8 MiB device
 * array per GPU, held until the process ends, so ceil(BT/16) * (D+1) * 4
 * bytes must fit 8 MiB (BT <= 21824 at D = 1536, 9360 at D = 3584), else it
 * returns an error before launching anything.  The GPU is the stream's
 * (the current device for the null stream); the caller's current device is
 * left as it was.  Every call on one GPU shares
 * that array: calls that overlap on one GPU (on different streams, or from
 * different threads) race and must be ordered by the caller. */
int ta_centroid_accumulate_bf16_noalloc(const uint16_t* h, const uint16_t* g, int64_t BT, int D,
                                        double* acc, void* stream);
/* Same with F32 h and g (the dtype the reference trainer hands over,
 * adapt_trainer.cu:215-231). */
int ta_centroid_accumulate_f32(const float* h, const float* g, int64_t BT, int D, double* acc,
                               void* stream);
/* Same with F32 h and given per-token norms n (the stress configuration). */
int ta_centroid_accumulate_f32n(const float* h, const float* n, int64_t BT, int D,
                                double* acc, void* stream);

/* ── centroid merge (k-means) ───────────────────────────────────────
 * replaces the Lloyd loop of CentroidAccumulator::merge_and_write
 * src/centroid/centroid_accumulator.cpp:114-157: init center i =
 * snaps[(i*N)/k], <= max_iters iterations, strict-< ties, stop when no
 * assignment changes, empty cluster -> zero vector.  One device launch.
 * k is clamped to N (centers then holds min(k, N) rows); iters_out (device
 * int, may be NULL) receives the number of assignment passes that changed
 * something, as the reference's loop counter. */
int ta_kmeans_ref(const float* snaps, int N, int D, int k, int max_iters, float* centers,
                  int32_t* assign, int32_t* iters_out, void* stream);
/* Stress mode (k-means++ seeding with splitmix64(seed), exactly `iters`
 * Lloyd iterations, clusters ranked by total weight of member snapshots).
 * No reference counterpart (the reference has only the mode above). */
int ta_kmeans_pp(const float* snaps, const float* weights, int N, int D, int k, int iters,
                 uint64_t seed, float* centers, int32_t* assign, double* mass,
                 int32_t* seeds, void* stream);

/* ── device memory (the host API's Tensor storage) ───────────────────
 * Caching allocator replacing the reference's one cudaMalloc/cudaFree per
 * Tensor (src/backend/cuda/tensor.cu:18-27,115-122).  Blocks are rounded to
 * a size class and recycled per device; ta_mem_free returns a block to the
 * cache (no hipFree), so it must only be called once the work using the
 * block has been enqueued on the stream that later users of the cache are
 * ordered on.  ta_mem_trim synchronises the device and releases the cache. */
int ta_mem_alloc(void** ptr, int64_t bytes, int device);
int ta_mem_free(void* ptr, int device);
int ta_mem_stats(int device, int64_t* in_use, int64_t* cached);
int ta_mem_trim(int device);
/* Waits for `stream` (on the current device) and frees the scratch buffers
 * the library keeps for it; the next op on that stream allocates afresh.
 * For hosts that create and destroy streams (one per request, say): call
 * it before hipStreamDestroy.  No reference counterpart (the reference
 * allocates per call). */
int ta_scratch_release(void* stream);

/* ── kernel-level timing (measurement; no reference counterpart) ─────
 * ta_kprof_select(kid) starts timing every launch of one kernel (ids: 0 the
 * large K-contiguous GEMM, 1 its wide-N tile shape, 2 attention forward,
 * 3 attention backward dQ pass, 4 attention backward dK/dV pass, 5 the LoRA
 * skinny products h = xA^T / dh = goB, 6 the LoRA weight gradients with
 * their reduction, 7 the chained input-gradient GEMMs, 8 the gate/up
 * projections with the SwiGLU product; -1 stops)
 * with start and stop events carried by the launch's own dispatch on its
 * stream.  ta_kprof_pause(1) leaves the selection and the recorded launches
 * as they are but times no further launch until ta_kprof_pause(0) (timing
 * costs a few microseconds of idle GPU around each timed launch, so a
 * measurement can time a sample of steps).  ta_kprof_read waits for
 * the recorded launches and returns their summed time, count, algorithmic
 * flops and HBM bytes, then clears them; ta_kprof_name gives the timed
 * kernel's symbol as a profiler prints it ("" before its first launch). */
int ta_kprof_select(int kid);
int ta_kprof_pause(int paused);
int ta_kprof_read(double* ms, int64_t* launches, double* flops, double* bytes);
const char* ta_kprof_name(int kid);

#ifdef __cplusplus
}
#endif
#endif /* TA_BACKEND_H */
