// ta_internal.hpp — launchers shared between the backend's translation units
// (not part of the C-ABI).
#pragma once
#include <hip/hip_ext.h>

#include <vector>

#include "ta_common.hpp"

// s_waitcnt vmcnt(n) with the other counters left free (gfx9 encoding)
#define TA_WAIT_VMCNT(n) \
    __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

namespace ta {

void* scratch_get(size_t bytes, hipStream_t s, int slot = 0);

// Kernel ids of the kernel-level timer (ta_kprof_select).
enum KernelId {
    KP_GEMM_BIG = 0,       // large K-contiguous GEMM, N <= 3072 tile shape
    KP_GEMM_BIG_WIDE = 1,  // large K-contiguous GEMM, N > 3072 tile shape
    KP_ATTN_FWD = 2,
    KP_ATTN_BWD_DQ = 3,
    KP_ATTN_BWD_DKV = 4,
    KP_LORA_SKINNY = 5,  // h = x A^T / dh = go B
    KP_LORA_WGRAD = 6,   // gB = go^T h / gA = dh^T x partials
    KP_GEMM_CHAIN = 7,   // chained input-gradient GEMMs (k_gemm_pipe_chain)
    KP_GEMM_SWIGLU = 8,  // gate/up projections with act (k_gemm_pipe_swiglu)
    KP_COUNT = 9
};
// Bracket one launch of kernel `kid` on stream s when that kernel is being
// timed; name is the kernel's symbol as a profiler prints it.  The launches
// in the bracket go through tlaunch, which hands them the bracket's events.
bool kprof_begin(int kid, hipStream_t s);
void kprof_end(int kid, hipStream_t s, double flops, double bytes, const char* name);

// Launch timing armed on this thread.  kprof: the event pair of the
// current kprof bracket (stop null: none).  pool: per-launch pairs for the
// engine's class profiling (each launch takes the next pair of *pool,
// counted in *npairs; null: off).  A launch carries at most one pair: a
// kprof bracket wins over the pool.
struct KpArm {
    hipEvent_t start = nullptr, stop = nullptr;
    bool used = false;
    size_t slot = 0;  // the kernel-timing slot kprof_begin reserved
    std::vector<hipEvent_t>* pool = nullptr;
    size_t* npairs = nullptr;
};
KpArm& kprof_arm();
// the next pair of the armed pool (created as needed); false: none
bool kprof_pool_pair(hipEvent_t* start, hipEvent_t* stop);

// Launch kernel<<<grid, block, 0, s>>>(args...).  When timing is armed the
// launch records the events in its own dispatch: inside a kprof bracket the
// first launch the bracket's start, every launch its stop (so the last
// one's end stands); under the class profiling a start/stop pair of its
// own.  No event packets go between the kernels (they would add idle GPU
// time to what is measured).
template <typename... KArgs, typename... Args>
inline void tlaunch(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t s,
                    Args&&... args) {
    KpArm& k = kprof_arm();
    hipEvent_t a = nullptr, b = nullptr;
    if (k.stop) {
        a = k.used ? nullptr : k.start;
        b = k.stop;
        k.used = true;
    } else if (k.pool) {
        (void)kprof_pool_pair(&a, &b);
    }
    if (b)
        hipExtLaunchKernelGGL(kernel, grid, block, 0, s, a, b, 0, static_cast<KArgs>(args)...);
    else
        kernel<<<grid, block, 0, s>>>(static_cast<KArgs>(args)...);
}

// sum_{z < splits} part[z * stride + idx], added in z order (deterministic);
// the loads of 8 splits are issued together so their latencies overlap.
__device__ __forceinline__ float sum_splits(const float* __restrict__ part, int splits,
                                            int64_t stride, int64_t idx) {
    float s = 0.f;
    int z = 0;
    for (; z + 8 <= splits; z += 8) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = part[(int64_t)(z + i) * stride + idx];
#pragma unroll
        for (int i = 0; i < 8; i++) s += v[i];
    }
    for (; z < splits; z++) s += part[(int64_t)z * stride + idx];
    return s;
}

// LoRA terms for gemm_dispatch.  After the base epilogue, for each pair p
// in order, with D_p = U_p V_p^T (U_p [M x r], V_p [N x r]):
//   delta: C = bf16(C + s * bf16(D_p))   (apply_lora_fwd's add)
//   else : C = bf16(s * D_p + C)         (apply_lora_bwd's dx GEMM, beta 1)
// v_nk: V_p as [N x r] rows (B for the delta, A^T for the dx update);
// v_alt: the same operand in k_rank_update's layout (B [N x r] / A [r x N]).
struct LoraEpi {
    int n, r;
    bool delta;
    float s;
    const bf16* u[3];
    int64_t ldu[3];
    const bf16* v_nk[3];
    const bf16* v_alt[3];
};

int gemm_dispatch(bool xk, bool yk, int M, int N, int K, float alpha, const bf16* X, int64_t ldx,
                  const bf16* Y, int64_t ldy, float beta, void* C, int64_t ldc, const bf16* bias,
                  bool out_f32, hipStream_t s, int force_splits, const LoraEpi* lora);
// one of up to three GEMMs sharing X in gemm_groups: C = bf16(X Y^T (+ bias))
// (+ LoRA delta), N output columns, row stride ldc
struct GemmGroup {
    int N;
    const bf16* Y;
    bf16* C;
    int64_t ldc;
    const bf16* bias;
    const LoraEpi* lora;
    bool rope = false;  // rotated when gemm_groups gets a RopeSpec
};
// one GEMM of a gemm_chain: X [M x K] (row stride ldx) times Y [N x K]^T
struct GemmSeg {
    int K;
    const bf16* X;
    int64_t ldx;
    const bf16* Y;
    int64_t ldy;
};
// C = bf16(X_0 Y_0^T), then C = bf16(X_s Y_s^T + C), then the LoRA terms, in
// one launch over the concatenated K (rounded to BF16 between the GEMMs)
int gemm_chain(int M, int N, const GemmSeg* sg, int ns, bf16* C, int64_t ldc, const LoraEpi* lora,
               hipStream_t s);
// RoPE of a layer's Q ([BT, Hq * hd]) and K ([BT, Hk * hd]) in one launch
// (sign +1 forward, -1 the inverse rotation of the backward)
int rope_qk(bf16* q, int Hq, bf16* k, int Hk, int B, int T, int hd, float theta, float sign,
            hipStream_t s);
// (cos, sin) of sign * t * theta^(-2i/hd) for t < T, i < hd/2 ([T][hd/2]),
// built once per (device, T, hd, theta, sign) on the caller's stream and
// kept for the process; NULL if the allocation fails
const float2* rope_table(int T, int hd, float theta, float sign, hipStream_t s);
// RoPE applied by the GEMM that writes Q and K (gemm_groups): rows are
// positions t = row % T, the output columns are heads of hd
struct RopeSpec {
    int B, T, hd;
    float theta;
};
// gate/up projections (+ LoRA deltas) and act = silu(gate) up in one launch
// over Wgu, the gate/up weights interleaved in 128-row blocks ([2I x K]);
// falls back to gemm_groups + silu_mul_fwd for other shapes (Wgu may be NULL)
int gemm_swiglu(int M, int K, const bf16* X, int64_t ldx, const bf16* Wgu, const bf16* Wg,
                const bf16* Wu, bf16* gate, bf16* up, bf16* act, int I, const LoraEpi* lg,
                const LoraEpi* lu, hipStream_t s);
// the groups' GEMMs in one launch over the N-concatenated tile grid; with
// rope, the groups whose `rope` flag is set are rotated after their final
// rounding (ops::rope_fwd of the written output, the same bits)
int gemm_groups(int M, int K, const bf16* X, int64_t ldx, int64_t ldy, const GemmGroup* gr,
                int ng, hipStream_t s, const RopeSpec* rope = nullptr);
// causal GQA attention; P [B*Hq, T, T] F32 probabilities, or (P NULL) only
// the rows' (max, 1/sum) in stats [B*Hq*T] float pairs, from which the
// backward recomputes P
int attn_fwd(const bf16* Q, const bf16* K, const bf16* V, bf16* O, float* O32, float* P,
             float* stats, int B, int T, int Hq, int Hkv, int hd, bool zero_fill, hipStream_t s);
// Dbuf: attn_bwd_rowbuf_floats(B, T, Hq) floats of per-query values; part:
// 2 B T Hq hd floats of dK/dV partials (each drawn from the scratch pool
// when NULL)
// rtab (may be NULL; the recompute path only): a rope_table(T, hd, theta,
// -1) whose inverse rotation dQ and dK take after their BF16 rounding, as
// ops::rope_bwd applied to the written dQ and dK would
int attn_bwd(const bf16* dO, const bf16* Q, const bf16* K, const bf16* V, const float* P,
             const float* stats, const float* O32, bf16* dQ, bf16* dK, bf16* dV, int B, int T,
             int Hq, int Hkv, int hd, float* Dbuf, float* part, hipStream_t s,
             const float2* rtab = nullptr);
int64_t attn_bwd_rowbuf_floats(int B, int T, int Hq);
int transpose_bf16(const bf16* in, bf16* out, int64_t rows, int64_t cols, hipStream_t s);
// cross_entropy_fwd (ops.cu:958-1020) that also adds the number of NaN and
// Inf logits to *nonfinite when it is not null (a device int32 the caller
// zeroes)
int cross_entropy(const bf16* logits, const int32_t* targets, float* loss_out, bf16* dlogits,
                  int N, int V, int32_t* nonfinite, hipStream_t s, float* lse2_out = nullptr);
// whether cross_entropy can write the row normalisers for these logits
bool cross_entropy_lse_ok(const bf16* logits, int V);
// dX = dlogits W of the LM head with dlogits formed from the logits inside
// the GEMM's operand reads: dlogits[t][v] = bf16((exp2(l log2(e) - lse2[t])
// - [v == tgt[t]]) / N), the bits cross_entropy writes (X = logits [M x K],
// Y = W^T [N x K], C = dX [M x N], all K-contiguous, beta 0).
int gemm_ce_dx(int M, int N, int K, const bf16* logits, const bf16* Wt, bf16* C,
               const float* lse2, const int32_t* tgt, float inv_n, hipStream_t s);
int fill_normal_bf16(bf16* out, int64_t n, uint64_t seed, uint64_t sid, float std, hipStream_t s);
int fill_bf16(bf16* out, int64_t n, float v, hipStream_t s);
int kaiming_init(float* a32, bf16* a16, int64_t n, int in_dim, hipStream_t s);
int add2_bf16(bf16* out, const bf16* a, const bf16* b, int64_t n, hipStream_t s);
// xs = bf16(a + b), then the RMSNorm forward of xs (out, inverse rms), in one pass
int rms_fwd_res(const bf16* a, const bf16* b, bf16* xs, const bf16* w, bf16* out, float* rms_out,
                int64_t rows, int D, float eps, hipStream_t s);
// acc = bf16(acc + bf16(RMSNorm backward dx)), in one pass (tmp: fallback scratch)
int rms_bwd_acc(const bf16* dy, const bf16* x, const bf16* w, const float* rms, bf16* acc,
                bf16* tmp, int64_t rows, int D, hipStream_t s);
// embedding gather that checks ids against V: an id outside [0, V) gets a
// zero row and sets *bad = 1 (ids resident in device memory)
int embed_fwd_checked(const bf16* table, const int32_t* tokens, bf16* out, int64_t BT, int D,
                      int V, int32_t* bad, hipStream_t s);
// One adapter tensor of the engine's arena for adamw_tiles_impl: [R x C]
// row-major at element offset off (the transposed copy [C x R] at the same
// offset of the transposed arena); a_side: A [r, in], tiled by 2^lw columns,
// else B [out, r], tiled by 2^lw rows (r <= 64, r x 2^lw <= 4096 and
// 2^lw <= 256); blk0: its first tile.
struct AdamTensor {
    int64_t off, blk0;
    int R, C, a_side, lw;
};
int adamw_tiles_impl(float* master, bf16* working, bf16* workingT, float* m, float* v,
                     float* grad, int64_t N, const AdamTensor* tens, int ntens, int64_t ntiles,
                     bool update, float lr, float beta1, float beta2, float eps,
                     float weight_decay, int step, float max_norm, float* norm_out,
                     const int32_t* skip, hipStream_t s);
// the fused norm / clip / AdamW tail; when skip (device int, may be NULL)
// holds a nonzero value the norm is still reported but no state changes
int adamw_fused_impl(float* master, bf16* working, float* m, float* v, float* grad, int64_t N,
                     float lr, float b1, float b2, float eps, float wd, int step, float max_norm,
                     float* norm_out, const int32_t* skip, hipStream_t s);
// centroid accumulate of BF16 h, g; when skip (device int, may be NULL) holds
// a nonzero value nothing is added
int centroid_acc_bf16(const bf16* h, const bf16* g, int64_t BT, int D, double* acc,
                      const int32_t* skip, hipStream_t s);
int mask_targets_dev(const int32_t* in, const int32_t* tgt_in, int32_t* tgt, int B, int T,
                     hipStream_t s);
int lora_skinny_nt(const bf16* X, int64_t ldx, int M, int K, int r, const bf16* const* Y,
                   bf16* const* C, int64_t ldc, int n, hipStream_t s);
int lora_rank_update(bool delta, bf16* Y, int64_t ldy, int M, int N, int r, float scale,
                     const bf16* const* U, const int64_t* ldu, const bf16* const* V, int n,
                     hipStream_t s);
// Weight-gradient products of the LoRA backward, reduced once per step:
// lora_wgrad_part writes split partials of L^T Sm into part; one
// lora_wgrad_reduce_jobs launch then adds scale * (ordered sum of each job's
// partials) into its gradient (see k_wgrad_reduce_jobs).
struct WgradJob {
    const float* part;
    float* g[3];
    int64_t n;     // NL * NS
    int64_t blk0;  // first block of this job in the reduce launch
    int splits, NL, NS, r, trans;
    float scale;
};
int lora_wgrad_splits(int NL, int T, int* per);
int lora_wgrad_part(const bf16* L, int64_t ldl, int NL, const bf16* Sm, int64_t lds, int NS, int T,
                    float* part, hipStream_t s);
// Fused SwiGLU backward + gate/up LoRA backward (rank 16): dgate/dup as
// silu_mul_bwd, the dh products of both pairs as column-split partials
// (dh_part [S_o][2][BT][16]) and their gB products as token-split partials
// (gb_g/gb_u [S_t][I][16], deferred-reduce layout); with dh_d/ga_d also the
// down pair's gA product act^T dh_down (act recomputed from gate and up) as
// token-split partials ga_d [S_t][I][16].  BT and I multiples of 64.
int silu_lora_splits(int BT, int I, int* s_t, int* s_o);
int silu_bwd_lora(const bf16* dact, const bf16* gate, const bf16* up, bf16* dgate, bf16* dup,
                  const bf16* bt_g, const bf16* bt_u, const bf16* h_g, const bf16* h_u,
                  float* dh_part, float* gb_g, float* gb_u, const bf16* dh_d, float* ga_d, int BT,
                  int I, hipStream_t s);
// dh[t][p*16 + j] = bf16(sum over the S_o column splits of dh_part[s][p][t][j]), p = 0, 1
int dh_reduce2(const float* dh_part, int s_o, int BT, bf16* dh, int64_t ldh, hipStream_t s);
// dh_p = bf16(go_p B_p) into dh (columns 16p.., row stride ldh) and the gB
// partials gb_p [S_t][N_p][16] of up to three rank-16 pairs in one pass over
// their go_p [BT x N_p] (N_p multiples of 64, BT a multiple of 32); bt_p the
// B^T shadows [16 x N_p], h_p [BT x 16]; dh_part: [S_o][3][BT][16] F32
int go_lora_splits(int BT, int ntot, int* s_t, int* s_o);
int go_lora(const bf16* const* go, const int64_t* ldgo, const bf16* const* bt, const bf16* const* h,
            float* const* gb, const int* n, int np, int BT, float* dh_part, bf16* dh, int64_t ldh,
            hipStream_t s);
int lora_wgrad_reduce_jobs(const WgradJob* jobs, int njobs, int64_t total_blocks, double elems,
                           hipStream_t s);

}  // namespace ta
