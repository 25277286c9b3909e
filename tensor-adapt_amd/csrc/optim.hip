// optim.hip — AdamW, gradient sum of squares, and the fused optimizer tail.
//
// The step engine keeps every adapter tensor in ONE flat arena (master F32,
// m, v, grad F32, BF16 shadow), so the reference's per-tensor loops
// (392 sum_sq launches, a host read-back, 392 scale launches and 392 AdamW
// launches at the headline shape — src/trainer/adapt_trainer.cu:32-70,
// src/trainer/adamw.cu:9-38) become two launches with no host sync:
//   1. k_sumsq_partials: fixed grid, each block writes sum(g^2) of its
//      grid-stride slice (deterministic order);
//   2. k_adamw_fused: every block re-reduces the partials in the same order
//      (so all blocks agree on the norm bit for bit), derives the clip
//      factor, and applies AdamW (ops.cu:1139-1158) to its elements.  When
//      the clip fires, the scaled gradient is also stored back, so the
//      gradient arena ends the step holding what clip_gradients leaves in
//      gA/gB (adapt_trainer.cu:55-70: g *= clip / (norm + 1e-6) in place).
#include <algorithm>

#include "ta_internal.hpp"

namespace ta {

constexpr int kNormBlocks = 1024;

__global__ __launch_bounds__(256) void k_sumsq_partials(const float* __restrict__ g, int64_t N,
                                                         float* __restrict__ part) {
    float acc = 0.f;
    // float4 body when g is 16-byte aligned, scalar otherwise
    int64_t nv = (((uintptr_t)g & 15u) == 0) ? (N >> 2) : 0;
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < nv; i += (int64_t)gridDim.x * 256) {
        float4 v = ((const float4*)g)[i];
        acc += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    if (blockIdx.x == 0)
        for (int64_t i = (nv << 2) + threadIdx.x; i < N; i += 256) acc += g[i] * g[i];
    acc = wave_sum(acc);
    __shared__ float red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) part[blockIdx.x] = ((red[0] + red[1]) + red[2]) + red[3];
}

// sum of the kNormBlocks partials in double, fixed order; every caller gets
// the identical value.
__device__ double reduce_partials(const float* __restrict__ part, int nparts) {
    __shared__ double dred[4];
    double a = 0.0;
    for (int i = threadIdx.x; i < nparts; i += 256) a += (double)part[i];
    a = wave_sum_d(a);
    if ((threadIdx.x & 63) == 0) dred[threadIdx.x >> 6] = a;
    __syncthreads();
    double t = ((dred[0] + dred[1]) + dred[2]) + dred[3];
    __syncthreads();
    return t;
}

__global__ void k_accum_sumsq(const float* __restrict__ part, int nparts,
                              float* __restrict__ accum) {
    double t = reduce_partials(part, nparts);
    if (threadIdx.x == 0) *accum += (float)t;
}

// AdamW element update — ops.cu:1139-1158 (bias corrections passed in).
__device__ __forceinline__ float adamw_elem(float p, float g, float& m, float& v, float lr,
                                            float b1, float b2, float eps, float wd, float bc1,
                                            float bc2) {
    float mi = b1 * m + (1.f - b1) * g;
    float vi = b2 * v + (1.f - b2) * g * g;
    m = mi;
    v = vi;
    float mhat = mi / bc1, vhat = vi / bc2;
    return p - lr * (mhat / (sqrtf(vhat) + eps) + wd * p);
}

__global__ __launch_bounds__(256) void k_adamw(float* __restrict__ master, bf16* __restrict__ work,
                                               float* __restrict__ m, float* __restrict__ v,
                                               float* __restrict__ grad, int64_t N,
                                               float lr, float b1, float b2, float eps, float wd,
                                               float bc1, float bc2,
                                               const float* __restrict__ part, int nparts,
                                               float max_norm, float* __restrict__ norm_out,
                                               const int32_t* __restrict__ skip) {
    float gscale = 1.f;
    if (part) {
        double ss = reduce_partials(part, nparts);
        float norm = (float)sqrt(ss);
        if (norm_out && blockIdx.x == 0 && threadIdx.x == 0) *norm_out = norm;
        if (skip && *skip) return;  // a failed step: report the norm, change nothing
        // clip_gradients, adapt_trainer.cu:55-70
        if (norm > max_norm) gscale = max_norm / (norm + 1e-6f);
    }
    const bool clipped = gscale != 1.f;
    for (int64_t i = blockIdx.x * 256ll + threadIdx.x; i < N; i += (int64_t)gridDim.x * 256) {
        float g = grad[i];
        if (clipped) {
            g = g * gscale;
            grad[i] = g;
        }
        float mi = m[i], vi = v[i];
        float p = adamw_elem(master[i], g, mi, vi, lr, b1, b2, eps, wd, bc1, bc2);
        m[i] = mi;
        v[i] = vi;
        master[i] = p;
        if (work) work[i] = f2bf(p);
    }
}

// AdamW over the step engine's adapter arena, one tensor tile at a time,
// that also writes each updated BF16 shadow transposed (A^T [in, r], B^T
// [r, out]: the K-contiguous operands of the LoRA backward products) into a
// second arena at the same offsets.  A tile is W columns x all r rows of
// an A [r, in] or W rows x all r columns of a B [out, r] (W = 256 for
// r <= 16, else 64: at most 4096 elements): its state is read as whole row
// segments, and the transposed tile leaves through LDS as contiguous runs
// (W x r elements for A, r runs of W for B).  Blocks take
// tiles grid-stride; every block derives the clip factor from the norm
// partials as k_adamw does.  update = false: no AdamW, the shadow is only
// copied into its transposed arena (after a shadow is written from outside).
__global__ __launch_bounds__(256) void k_adamw_tiles(
    float* __restrict__ master, bf16* __restrict__ work, bf16* __restrict__ workT,
    float* __restrict__ m, float* __restrict__ v, float* __restrict__ grad,
    const AdamTensor* __restrict__ tens, int ntens, int64_t ntiles, bool update, float lr,
    float b1, float b2, float eps, float wd, float bc1, float bc2, const float* __restrict__ part,
    int nparts, float max_norm, float* __restrict__ norm_out, const int32_t* __restrict__ skip) {
    __shared__ uint16_t lt[256 * 17];  // [tile column (A) or row (B)][rank index], padded
    float gscale = 1.f;
    if (update && part) {
        double ss = reduce_partials(part, nparts);
        float norm = (float)sqrt(ss);
        if (norm_out && blockIdx.x == 0 && threadIdx.x == 0) *norm_out = norm;
        if (skip && *skip) return;  // a failed step: report the norm, change nothing
        // clip_gradients, adapt_trainer.cu:55-70
        if (norm > max_norm) gscale = max_norm / (norm + 1e-6f);
    }
    const bool clipped = gscale != 1.f;
    auto elem = [&](int64_t i) -> uint16_t {
        if (!update) return work[i];
        float g = grad[i];
        if (clipped) {
            g = g * gscale;
            grad[i] = g;
        }
        float mi = m[i], vi = v[i];
        const float p = adamw_elem(master[i], g, mi, vi, lr, b1, b2, eps, wd, bc1, bc2);
        m[i] = mi;
        v[i] = vi;
        master[i] = p;
        const uint16_t h = f2bf(p);
        work[i] = h;
        return h;
    };
    // elements i .. i + 3 (i a multiple of 4: every tensor starts on a
    // 64-element boundary), each with elem's arithmetic, moved as 16-byte
    // F32 and 8-byte BF16 vectors
    auto elem4 = [&](int64_t i, uint16_t (&h)[4]) {
        if (!update) {
            const uint2 w = *(const uint2*)(work + i);
            h[0] = (uint16_t)w.x, h[1] = (uint16_t)(w.x >> 16);
            h[2] = (uint16_t)w.y, h[3] = (uint16_t)(w.y >> 16);
            return;
        }
        float4 g = *(const float4*)(grad + i);
        if (clipped) {
            g.x *= gscale, g.y *= gscale, g.z *= gscale, g.w *= gscale;
            *(float4*)(grad + i) = g;
        }
        float4 mi = *(const float4*)(m + i), vi = *(const float4*)(v + i);
        float4 pm = *(const float4*)(master + i);
        pm.x = adamw_elem(pm.x, g.x, mi.x, vi.x, lr, b1, b2, eps, wd, bc1, bc2);
        pm.y = adamw_elem(pm.y, g.y, mi.y, vi.y, lr, b1, b2, eps, wd, bc1, bc2);
        pm.z = adamw_elem(pm.z, g.z, mi.z, vi.z, lr, b1, b2, eps, wd, bc1, bc2);
        pm.w = adamw_elem(pm.w, g.w, mi.w, vi.w, lr, b1, b2, eps, wd, bc1, bc2);
        *(float4*)(m + i) = mi;
        *(float4*)(v + i) = vi;
        *(float4*)(master + i) = pm;
        const uint2 w = make_uint2(pack2(pm.x, pm.y), pack2(pm.z, pm.w));
        *(uint2*)(work + i) = w;
        h[0] = (uint16_t)w.x, h[1] = (uint16_t)(w.x >> 16);
        h[2] = (uint16_t)w.y, h[3] = (uint16_t)(w.y >> 16);
    };
    for (int64_t b = blockIdx.x; b < ntiles; b += gridDim.x) {
        int lo = 0, hi = ntens - 1;  // last tensor with blk0 <= b
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (tens[mid].blk0 <= b) lo = mid; else hi = mid - 1;
        }
        const AdamTensor T = tens[lo];
        const int t = (int)(b - T.blk0);
        __syncthreads();  // the previous tile's transposed reads are done
        const int lw = T.lw, W = 1 << lw, P = (T.a_side ? T.R : T.C) + 1;  // LDS row pitch
        if ((T.R & 3) == 0 && (T.C & 3) == 0) {
            // four consecutive elements per thread, in memory and in the
            // transposed copy (both dimensions multiples of 4)
            if (T.a_side) {
                const int c0 = W * t, nc = min(W, T.C - c0);  // nc: a multiple of 4
                for (int e = threadIdx.x; e < T.R << (lw - 2); e += 256) {
                    const int rr = e >> (lw - 2), cc = (e & ((W >> 2) - 1)) << 2;
                    if (cc < nc) {
                        uint16_t h[4];
                        elem4(T.off + (int64_t)rr * T.C + c0 + cc, h);
#pragma unroll
                        for (int k = 0; k < 4; k++) lt[(cc + k) * P + rr] = h[k];
                    }
                }
                __syncthreads();
                bf16* dst = workT + T.off + (int64_t)c0 * T.R;
                for (int e = 4 * threadIdx.x; e < nc * T.R; e += 1024) {
                    const int cc = e / T.R, rr = e - cc * T.R;  // rr .. rr + 3 in one row
                    const int q = cc * P + rr;
                    *(uint2*)(dst + e) = make_uint2((uint32_t)lt[q] | ((uint32_t)lt[q + 1] << 16),
                                                    (uint32_t)lt[q + 2] | ((uint32_t)lt[q + 3] << 16));
                }
            } else {
                const int r0 = W * t, nr = min(W, T.R - r0);  // nr: a multiple of 4
                const int64_t base = T.off + (int64_t)r0 * T.C;
                for (int e = 4 * threadIdx.x; e < nr * T.C; e += 1024) {
                    const int rr = e / T.C, cc = e - rr * T.C;
                    uint16_t h[4];
                    elem4(base + e, h);
#pragma unroll
                    for (int k = 0; k < 4; k++) lt[rr * P + cc + k] = h[k];
                }
                __syncthreads();
                for (int e = threadIdx.x; e < T.C << (lw - 2); e += 256) {
                    const int cc = e >> (lw - 2), rr = (e & ((W >> 2) - 1)) << 2;
                    if (rr < nr)
                        *(uint2*)(workT + T.off + (int64_t)cc * T.R + r0 + rr) = make_uint2(
                            (uint32_t)lt[rr * P + cc] | ((uint32_t)lt[(rr + 1) * P + cc] << 16),
                            (uint32_t)lt[(rr + 2) * P + cc] | ((uint32_t)lt[(rr + 3) * P + cc] << 16));
                }
            }
        } else if (T.a_side) {
            // A [R = r, C = in]: columns [c0, c0 + nc), all R rows
            const int c0 = W * t, nc = min(W, T.C - c0);
            for (int e = threadIdx.x; e < T.R << lw; e += 256) {
                const int rr = e >> lw, cc = e & (W - 1);
                if (cc < nc) lt[cc * P + rr] = elem(T.off + (int64_t)rr * T.C + c0 + cc);
            }
            __syncthreads();
            // A^T [C, R]: rows c0 .. c0 + nc, one contiguous run
            bf16* dst = workT + T.off + (int64_t)c0 * T.R;
            for (int e = threadIdx.x; e < nc * T.R; e += 256) {
                const int cc = e / T.R, rr = e - cc * T.R;
                dst[e] = lt[cc * P + rr];
            }
        } else {
            // B [R = out, C = r]: rows [r0, r0 + nr), all C columns (contiguous)
            const int r0 = W * t, nr = min(W, T.R - r0);
            const int64_t base = T.off + (int64_t)r0 * T.C;
            for (int e = threadIdx.x; e < nr * T.C; e += 256) {
                const int rr = e / T.C, cc = e - rr * T.C;
                lt[rr * P + cc] = elem(base + e);
            }
            __syncthreads();
            // B^T [C, R]: row cc gets columns r0 .. r0 + nr
            for (int e = threadIdx.x; e < T.C << lw; e += 256) {
                const int cc = e >> lw, rr = e & (W - 1);
                if (rr < nr) workT[T.off + (int64_t)cc * T.R + r0 + rr] = lt[rr * P + cc];
            }
        }
    }
}

}  // namespace ta

using namespace ta;

static inline int adam_blocks(int64_t N) {
    int64_t b = (N + 255) / 256;
    if (b > 4096) b = 4096;
    return (int)(b < 1 ? 1 : b);
}

extern "C" {

int ta_adamw_step(float* master, uint16_t* working, float* m, float* v, const float* grad,
                  int64_t N, float lr, float beta1, float beta2, float eps, float weight_decay,
                  int step, void* stream) {
    TA_REQUIRE(N >= 0 && step >= 1, "adamw_step: bad N=%lld step=%d", (long long)N, step);
    if (N == 0) return 0;
    float bc1 = 1.f - powf(beta1, (float)step);
    float bc2 = 1.f - powf(beta2, (float)step);
    tlaunch(k_adamw, dim3(adam_blocks(N)), dim3(256), (hipStream_t)stream, master, working, m, v,
                                                             const_cast<float*>(grad), N, lr,
                                                             beta1, beta2, eps, weight_decay,
                                                             bc1, bc2, nullptr, 0, 0.f, nullptr,
                                                             nullptr);
    return check_launch("adamw_step");
}

int ta_sum_sq_into(const float* g, float* accum, int64_t N, void* stream) {
    TA_REQUIRE(N >= 0, "sum_sq_into: N < 0");
    if (N == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    float* part = (float*)scratch_get(kNormBlocks * sizeof(float), s);
    TA_REQUIRE(part, "sum_sq_into: scratch allocation failed");
    tlaunch(k_sumsq_partials, dim3(kNormBlocks), dim3(256), s, g, N, part);
    tlaunch(k_accum_sumsq, dim3(1), dim3(256), s, part, kNormBlocks, accum);
    return check_launch("sum_sq_into");
}

int ta_adamw_fused(float* master, uint16_t* working, float* m, float* v, float* grad,
                   int64_t N, float lr, float beta1, float beta2, float eps,
                   float weight_decay, int step, float max_norm, float* norm_out,
                   void* stream) {
    return adamw_fused_impl(master, working, m, v, grad, N, lr, beta1, beta2, eps, weight_decay,
                            step, max_norm, norm_out, nullptr, (hipStream_t)stream);
}

}  // extern "C"

namespace ta {

int adamw_fused_impl(float* master, bf16* working, float* m, float* v, float* grad, int64_t N,
                     float lr, float beta1, float beta2, float eps, float weight_decay, int step,
                     float max_norm, float* norm_out, const int32_t* skip, hipStream_t s) {
    TA_REQUIRE(N >= 0 && step >= 1, "adamw_fused: bad N=%lld step=%d", (long long)N, step);
    if (N == 0) return 0;
    float* part = (float*)scratch_get(kNormBlocks * sizeof(float), s);
    TA_REQUIRE(part, "adamw_fused: scratch allocation failed");
    float bc1 = 1.f - powf(beta1, (float)step);
    float bc2 = 1.f - powf(beta2, (float)step);
    tlaunch(k_sumsq_partials, dim3(kNormBlocks), dim3(256), s, grad, N, part);
    tlaunch(k_adamw, dim3(adam_blocks(N)), dim3(256), s, master, working, m, v, grad, N, lr, beta1, beta2,
                                           eps, weight_decay, bc1, bc2, part, kNormBlocks,
                                           max_norm, norm_out, skip);
    return check_launch("adamw_fused");
}

// The engine's tail with the transposed shadows: norm partials, then the
// tiled AdamW (update) or only the shadow transposes (!update; the other
// arguments past tiles are then unused).
int adamw_tiles_impl(float* master, bf16* working, bf16* workingT, float* m, float* v,
                     float* grad, int64_t N, const AdamTensor* tens, int ntens, int64_t ntiles,
                     bool update, float lr, float beta1, float beta2, float eps,
                     float weight_decay, int step, float max_norm, float* norm_out,
                     const int32_t* skip, hipStream_t s) {
    if (ntiles <= 0) return 0;
    TA_REQUIRE(ntens > 0 && (!update || step >= 1), "adamw_tiles: bad arguments");
    const int blocks = (int)std::min<int64_t>(ntiles, 2048);
    if (!update) {
        tlaunch(k_adamw_tiles, dim3(blocks), dim3(256), s, master, working, workingT, m, v, grad, tens, ntens,
                                             ntiles, false, 0.f, 0.f, 0.f, 0.f, 0.f, 1.f, 1.f,
                                             nullptr, 0, 0.f, nullptr, nullptr);
        return check_launch("adamw_tiles");
    }
    float* part = (float*)scratch_get(kNormBlocks * sizeof(float), s);
    TA_REQUIRE(part, "adamw_tiles: scratch allocation failed");
    float bc1 = 1.f - powf(beta1, (float)step);
    float bc2 = 1.f - powf(beta2, (float)step);
    tlaunch(k_sumsq_partials, dim3(kNormBlocks), dim3(256), s, grad, N, part);
    tlaunch(k_adamw_tiles, dim3(blocks), dim3(256), s, master, working, workingT, m, v, grad, tens, ntens, ntiles,
                                         true, lr, beta1, beta2, eps, weight_decay, bc1, bc2, part,
                                         kNormBlocks, max_norm, norm_out, skip);
    return check_launch("adamw_tiles");
}

}  // namespace ta
