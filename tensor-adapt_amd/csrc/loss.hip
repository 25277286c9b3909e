// loss.hip — per-token cross entropy with the reference's gradient
// convention (src/backend/cuda/ops.cu:958-1020).
//
// k_cross_entropy_reg: one 1024-thread block per token row holds the whole
// row in registers (16-byte loads, all issued at once: up to 20 x 8 values
// per lane, V <= 163840), takes the block max, then the sum of exp, then
// writes dlogits = bf16((softmax - onehot) / N): the logits are read once
// and dlogits written once (the reference reads the row three times).
// k_cross_entropy (one 512-thread block per row, online max/sum, two reads)
// serves rows too long for registers and unaligned or ragged V.
#include <float.h>

#include "ta_internal.hpp"

namespace ta {

__device__ __forceinline__ void lse_merge(float& m, float& s, float m2, float s2) {
    float mn = fmaxf(m, m2);
    // exp2 of (-inf) - finite is 0; guard the (-inf,-inf) case
    float a = (m == -FLT_MAX) ? 0.f : s * exp2f((m - mn) * kLog2e);
    float b = (m2 == -FLT_MAX) ? 0.f : s2 * exp2f((m2 - mn) * kLog2e);
    m = mn;
    s = a + b;
}

template <bool VEC>
__global__ __launch_bounds__(512) void k_cross_entropy(const bf16* __restrict__ logits,
                                                       const int32_t* __restrict__ targets,
                                                       float* __restrict__ loss,
                                                       bf16* __restrict__ dlogits, int V,
                                                       float inv_N,
                                                       int32_t* __restrict__ nonfinite) {
    int64_t n = blockIdx.x;
    const bf16* L = logits + n * (int64_t)V;
    bf16* dL = dlogits ? dlogits + n * (int64_t)V : nullptr;
    int tgt = targets[n];
    if (nonfinite) {
        // Inf or NaN logits of the row (the reference's step-0 check,
        // adapt_trainer.cu:76-91), read before dlogits may overwrite them
        int bad = 0;
        for (int i = threadIdx.x; i < V; i += blockDim.x) bad += (L[i] & 0x7f80u) == 0x7f80u;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) bad += __shfl_xor(bad, o, 64);
        if ((threadIdx.x & 63) == 0 && bad) atomicAdd(nonfinite, bad);
        __syncthreads();
    }
    float m = -FLT_MAX, s = 0.f;
    int nv = VEC ? (V >> 3) : 0;
    if (VEC) {
        for (int c = threadIdx.x; c < nv; c += blockDim.x) {
            float f[8];
            unpack8(((const bf16x8v*)L)[c], f);
            float cm = f[0];
#pragma unroll
            for (int e = 1; e < 8; e++) cm = fmaxf(cm, f[e]);
            float cs = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) cs += exp2f((f[e] - cm) * kLog2e);
            lse_merge(m, s, cm, cs);
        }
    }
    for (int i = nv * 8 + threadIdx.x; i < V; i += blockDim.x) lse_merge(m, s, bf2f(L[i]), 1.f);
    // wave then block combine (fixed order)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        float m2 = __shfl_xor(m, o, 64), s2 = __shfl_xor(s, o, 64);
        lse_merge(m, s, m2, s2);
    }
    __shared__ float sm[8], ss[8], lsum;
    int wv = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sm[wv] = m;
        ss[wv] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float M = sm[0], S = ss[0];
        for (int k = 1; k < (int)(blockDim.x >> 6); k++) lse_merge(M, S, sm[k], ss[k]);
        float log_sum = logf(S) + M;
        // a target outside [0, V) reads nothing (the reference would read out
        // of bounds for tgt >= V; ids come from a vocab-sized tokenizer)
        float tl = (tgt >= 0 && tgt < V) ? bf2f(L[tgt]) : 0.f;
        loss[n] = -(tl - log_sum);
        lsum = log_sum;
    }
    __syncthreads();
    if (!dL) return;
    float ls = lsum;
    if (VEC) {
        for (int c = threadIdx.x; c < nv; c += blockDim.x) {
            float f[8];
            unpack8(((const bf16x8v*)L)[c], f);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                float p = exp2f((f[e] - ls) * kLog2e);
                float d = p - (float)(c * 8 + e == tgt);
                f[e] = d * inv_N;
            }
            ((bf16x8v*)dL)[c] = pack8(f);
        }
    }
    for (int i = nv * 8 + threadIdx.x; i < V; i += blockDim.x) {
        float p = exp2f((bf2f(L[i]) - ls) * kLog2e);
        dL[i] = f2bf((p - (float)(i == tgt)) * inv_N);
    }
}

// block-wide reductions over 16 waves, in wave order
__device__ __forceinline__ float block_max16(float v, float* red) {
    v = wave_max(v);
    __syncthreads();  // red is free (a previous reduction's readers are done)
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int k = 1; k < 16; k++) r = fmaxf(r, red[k]);
    return r;
}
__device__ __forceinline__ float block_sum16(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int k = 1; k < 16; k++) r += red[k];
    return r;
}

// COUNT: also add the row's NaN and Inf logits to *nonfinite (the
// reference's step-0 check, adapt_trainer.cu:76-91)
template <int CPT, bool COUNT>  // 16-byte chunks per lane: V <= 8 * 1024 * CPT, V % 8 == 0
__global__ __launch_bounds__(1024) void k_cross_entropy_reg(const bf16* __restrict__ logits,
                                                            const int32_t* __restrict__ targets,
                                                            float* __restrict__ loss,
                                                            bf16* __restrict__ dlogits, int V,
                                                            float inv_N,
                                                            int32_t* __restrict__ nonfinite,
                                                            float* __restrict__ lse2_out) {
    __shared__ float red[16], tls;
    const int64_t n = blockIdx.x;
    const bf16x8v* L = (const bf16x8v*)(logits + n * (int64_t)V);
    const int nv = V >> 3, tgt = targets[n];
    bf16x8v r[CPT];
#pragma unroll
    for (int k = 0; k < CPT; k++) {
        const int c = threadIdx.x + 1024 * k;
        if (c < nv) r[k] = L[c];
    }
    float m = -FLT_MAX;
#pragma unroll
    for (int k = 0; k < CPT; k++) {
        const int c = threadIdx.x + 1024 * k;
        if (c < nv) {
            float f[8];
            unpack8(r[k], f);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                m = fmaxf(m, f[e]);
                // the target's logit, from the lane that holds it (dlogits may
                // overwrite the row in place once the sums are known)
                if (c * 8 + e == tgt) tls = f[e];
            }
        }
    }
    if (COUNT) {
        // exponent bits all ones: Inf or NaN
        float bad = 0.f;
#pragma unroll
        for (int k = 0; k < CPT; k++)
            if (threadIdx.x + 1024 * k < nv)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const uint32_t w = r[k].w[e];
                    bad += (float)((w & 0x7f80u) == 0x7f80u) +
                           (float)((w & 0x7f800000u) == 0x7f800000u);
                }
        const float nb = block_sum16(bad, red);  // exact: at most V < 2^24
        if (threadIdx.x == 0 && nb > 0.f) atomicAdd(nonfinite, (int32_t)nb);
    }
    // exp as one v_exp_f32 of x log2(e) - M log2(e) (results below the
    // normal range flush to zero, as the reference's fast-math __expf does)
    const float M = block_max16(m, red);
    const float M2 = M * kLog2e;
    float sum = 0.f;
#pragma unroll
    for (int k = 0; k < CPT; k++) {
        if (threadIdx.x + 1024 * k < nv) {
            float f[8];
            unpack8(r[k], f);
#pragma unroll
            for (int e = 0; e < 8; e++) sum += __builtin_amdgcn_exp2f(fmaf(f[e], kLog2e, -M2));
        }
    }
    const float S = block_sum16(sum, red);
    const float log_sum = logf(S) + M;
    const float ls2 = log_sum * kLog2e;
    if (threadIdx.x == 0) {
        // a target outside [0, V) reads nothing (the reference would read out
        // of bounds for tgt >= V; ids come from a vocab-sized tokenizer)
        const float tl = (tgt >= 0 && tgt < V) ? tls : 0.f;
        loss[n] = -(tl - log_sum);
        // the row's base-2 normaliser, from which dlogits can be formed
        // elsewhere with the same bits (ce_dlogit8)
        if (lse2_out) lse2_out[n] = ls2;
    }
    if (!dlogits) return;
    bf16x8v* dL = (bf16x8v*)(dlogits + n * (int64_t)V);
#pragma unroll
    for (int k = 0; k < CPT; k++) {
        const int c = threadIdx.x + 1024 * k;
        if (c < nv) {
            float f[8];
            unpack8(r[k], f);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float p = __builtin_amdgcn_exp2f(fmaf(f[e], kLog2e, -ls2));
                f[e] = (p - (float)(c * 8 + e == tgt)) * inv_N;
            }
            dL[c] = pack8(f);
        }
    }
}

// cross_entropy_fwd that also adds the count of NaN and Inf logits to
// *nonfinite when it is not null (a device int32 the caller zeroes), and
// writes each row's base-2 normaliser to lse2_out when it is not null (then
// the row-in-registers kernel must take the shape: cross_entropy_lse_ok)
bool cross_entropy_lse_ok(const bf16* logits, int V) {
    return (V & 7) == 0 && ((uintptr_t)logits & 15u) == 0 && (V / 8 + 1023) / 1024 <= 20;
}
int cross_entropy(const bf16* logits, const int32_t* targets, float* loss_out, bf16* dlogits,
                  int N, int V, int32_t* nonfinite, hipStream_t s, float* lse2_out) {
    TA_REQUIRE(N >= 0 && V > 0, "cross_entropy_fwd: bad shape N=%d V=%d", N, V);
    TA_REQUIRE(!lse2_out || cross_entropy_lse_ok(logits, V),
               "cross_entropy: row normalisers need V %% 8 == 0 and V <= 163840");
    if (N == 0) return 0;
    // divisor = number of rows, masked rows included (gridDim.x in ops.cu:1005)
    float inv_N = 1.f / (float)N;
    bool vec = (V & 7) == 0 && (((uintptr_t)logits | (uintptr_t)dlogits) & 15u) == 0;
    const int cpt = (V / 8 + 1023) / 1024;
    // dlogits may overwrite logits in place: every lane reads its whole row
    // share before the block's first barrier, and writes only its own chunks
    // (up to 20 chunks per lane fit the 128 registers of a 16-wave block)
    if (vec && cpt <= 20) {
#define CE(C, K)                                                                      \
    tlaunch(k_cross_entropy_reg<C, K>, dim3(N), dim3(1024), s, logits, targets, loss_out, dlogits, V, inv_N, \
                                                 nonfinite, lse2_out)
#define CE2(C) \
    if (nonfinite) CE(C, true); else CE(C, false)
        if (cpt <= 4) { CE2(4); }
        else if (cpt <= 8) { CE2(8); }
        else if (cpt <= 16) { CE2(16); }
        else { CE2(20); }
#undef CE2
#undef CE
    } else if (vec) {
        tlaunch(k_cross_entropy<true>, dim3(N), dim3(512), s, logits, targets, loss_out, dlogits, V, inv_N,
                                                nonfinite);
    } else {
        tlaunch(k_cross_entropy<false>, dim3(N), dim3(512), s, logits, targets, loss_out, dlogits, V, inv_N,
                                                 nonfinite);
    }
    return check_launch("cross_entropy_fwd");
}

}  // namespace ta

using namespace ta;

extern "C" int ta_cross_entropy_fwd(const uint16_t* logits, const int32_t* targets,
                                    float* loss_out, uint16_t* dlogits, int N, int V,
                                    void* stream) {
    return cross_entropy(logits, targets, loss_out, dlogits, N, V, nullptr, (hipStream_t)stream,
                         nullptr);
}
