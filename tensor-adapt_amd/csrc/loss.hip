// loss.hip — per-token cross entropy with the reference's gradient
// convention (src/backend/cuda/ops.cu:958-1020).
//
// One 512-thread block per token row.  Pass 1 is an online max/sum over the
// row (each lane keeps a running max and a rescaled sum of exp, 16-byte
// loads), so the row is read twice in total instead of the reference's
// three times; pass 2 writes dlogits = bf16((softmax - onehot) / N).
#include <float.h>

#include "ta_common.hpp"

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
                                                       float inv_N) {
    int64_t n = blockIdx.x;
    const bf16* L = logits + n * (int64_t)V;
    bf16* dL = dlogits ? dlogits + n * (int64_t)V : nullptr;
    int tgt = targets[n];
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

}  // namespace ta

using namespace ta;

extern "C" int ta_cross_entropy_fwd(const uint16_t* logits, const int32_t* targets,
                                    float* loss_out, uint16_t* dlogits, int N, int V,
                                    void* stream) {
    TA_REQUIRE(N >= 0 && V > 0, "cross_entropy_fwd: bad shape N=%d V=%d", N, V);
    if (N == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    // divisor = number of rows, masked rows included (gridDim.x in ops.cu:1005)
    float inv_N = 1.f / (float)N;
    bool vec = (V & 7) == 0 && (((uintptr_t)logits | (uintptr_t)dlogits) & 15u) == 0;
    if (vec)
        k_cross_entropy<true><<<N, 512, 0, s>>>(logits, targets, loss_out, dlogits, V, inv_N);
    else
        k_cross_entropy<false><<<N, 512, 0, s>>>(logits, targets, loss_out, dlogits, V, inv_N);
    return check_launch("cross_entropy_fwd");
}
