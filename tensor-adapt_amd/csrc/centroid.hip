// centroid.hip — the Centroid Accumulator's per-token gradient-norm weighted
// sum and the centroid-merge k-means, on the device.
//
// Accumulate (src/centroid/centroid_accumulator.cpp:54-69, intended math):
//   n_t = ||g_t||_2 ; C[d] += h[t,d] * n_t ; W += n_t.
// The reference synchronises, copies two [BT, D] F32 tensors to the host per
// layer and loops on one core.  Here one launch reads h and g once (BF16,
// straight from the step's activations, no cast kernels), each block folds
// 16 (BF16) or 64 (F32) tokens into an F32 partial row, and a second launch
// adds the partial rows in block order into an F64 accumulator [D+1] (entry
// D holds W).  The result is deterministic and within 1e-7 relative of an
// F64 evaluation.
//
// k-means (centroid_accumulator.cpp:114-157 and the stress mode): one
// workgroup runs every iteration in a single launch.  Squared distances are
// summed sequentially over d in F32 with no contraction (__fmul_rn/__fadd_rn),
// exactly like a scalar CPU loop, so assignments are bit-reproducible; center
// sums run sequentially over snapshots in index order.  Every loop is bounded
// by max_iters / iters, so the launch always drains.
#include <float.h>

#include <mutex>

#include "ta_internal.hpp"

// Partial rows of ta_centroid_accumulate_bf16_noalloc, in a file-scope device
// array instead of allocated memory: every GPU the library runs on holds its
// own copy until the process ends.  In host code this name is a host-side
// stand-in, not a device address; host code uses only the per-device address
// from hipGetSymbolAddress (noalloc_scratch below).
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace ta {

constexpr int kTok = 16;   // tokens per block, BF16 inputs (512 blocks at BT = 8192)
constexpr int kTokF = 64;  // tokens per block, F32 inputs (1024 blocks per 65536 tokens)

// Per-block partial row: part[blk][d] = sum_{t in block} h[t][d] * n_t,
// part[blk][D] = sum n_t.  Rows move as 16-byte vectors when D % 8 == 0.
template <bool BF16IN, int KT = BF16IN ? kTok : kTokF>
__global__ __launch_bounds__(256) void k_centroid_part(const void* __restrict__ hv,
                                                       const void* __restrict__ gv,
                                                       const float* __restrict__ nv,
                                                       int64_t BT, int D,
                                                       float* __restrict__ part) {
    __shared__ float nrm[KT];
    int64_t t0 = (int64_t)blockIdx.x * KT;
    int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const bool v8 = BF16IN && (D & 7) == 0;
    const bool v4 = !BF16IN && (D & 3) == 0;
    // 1. per-token gradient norms (one wave per token; a wave's 16-byte
    // loads of its rows are issued together)
    for (int j = wv; j < KT; j += 4) {
        int64_t t = t0 + j;
        float ss = 0.f;
        if (t < BT && !nv) {
            if (v8) {
                const bf16x8v* g = (const bf16x8v*)((const bf16*)gv + t * D);
                constexpr int U = 4;
                for (int c0 = lane; c0 < (D >> 3); c0 += 64 * U) {
                    bf16x8v gg[U];
#pragma unroll
                    for (int u = 0; u < U; u++) {
                        const int c = c0 + 64 * u;
                        gg[u] = g[c < (D >> 3) ? c : c0];
                    }
#pragma unroll
                    for (int u = 0; u < U; u++) {
                        if (c0 + 64 * u >= (D >> 3)) continue;
                        float f[8];
                        unpack8(gg[u], f);
#pragma unroll
                        for (int e = 0; e < 8; e++) ss += f[e] * f[e];
                    }
                }
            } else if (BF16IN) {
                const bf16* g = (const bf16*)gv + t * D;
                for (int d = lane; d < D; d += 64) {
                    float f = bf2f(g[d]);
                    ss += f * f;
                }
            } else if (v4) {
                const float4* g = (const float4*)((const float*)gv + t * D);
                for (int c = lane; c < (D >> 2); c += 64) {
                    const float4 f = g[c];
                    ss += f.x * f.x;
                    ss += f.y * f.y;
                    ss += f.z * f.z;
                    ss += f.w * f.w;
                }
            } else {
                const float* g = (const float*)gv + t * D;
                for (int d = lane; d < D; d += 64) ss += g[d] * g[d];
            }
        }
        ss = wave_sum(ss);
        if (lane == 0) nrm[j] = (t < BT) ? (nv ? nv[t] : sqrtf(ss)) : 0.f;
    }
    __syncthreads();
    // 2. weighted column sums over this block's tokens
    float* out = part + (int64_t)blockIdx.x * (D + 1);
    if (v8) {
        for (int c = threadIdx.x; c < (D >> 3); c += 256) {
            float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            // all KT row loads first (rows past BT re-read the last row;
            // their weight is 0), then the sums in token order
            bf16x8v hh[KT];
#pragma unroll
            for (int j = 0; j < KT; j++) {
                const int64_t t = min(t0 + j, BT - 1);
                hh[j] = ((const bf16x8v*)((const bf16*)hv + t * D))[c];
            }
#pragma unroll
            for (int j = 0; j < KT; j++) {
                float f[8];
                unpack8(hh[j], f);
#pragma unroll
                for (int e = 0; e < 8; e++) acc[e] += f[e] * nrm[j];
            }
#pragma unroll
            for (int e = 0; e < 8; e++) out[c * 8 + e] = acc[e];
        }
    } else if (v4) {
        // F32 rows as 16-byte vectors.  When D/4 columns leave threads over
        // (D = 512: 128 columns), the block's G = 256 / (D/4) thread groups
        // take consecutive token ranges of KT/G tokens each; each group sums
        // its range in token order (16 row loads in flight per batch) and the
        // group sums are added in group order.
        __shared__ float4 gsum[256];
        const int nc4 = D >> 2;
        const int G = (nc4 <= 128 && 256 % nc4 == 0 && KT % (16 * (256 / nc4)) == 0)
                          ? 256 / nc4 : 1;
        const int TG = KT / G;
        for (int base = 0; base < nc4 * G; base += 256) {
            const int q = base + threadIdx.x, c = q % nc4, g = q / nc4;
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
            if (q < nc4 * G) {
                for (int j0 = g * TG; j0 < (g + 1) * TG; j0 += 16) {
                    float4 hh[16];
#pragma unroll
                    for (int j = 0; j < 16; j++) {
                        const int64_t t = min(t0 + j0 + j, BT - 1);
                        hh[j] = ((const float4*)((const float*)hv + t * D))[c];
                    }
#pragma unroll
                    for (int j = 0; j < 16; j++) {
                        const float w = nrm[j0 + j];
                        acc.x += hh[j].x * w;
                        acc.y += hh[j].y * w;
                        acc.z += hh[j].z * w;
                        acc.w += hh[j].w * w;
                    }
                }
            }
            if (G > 1) {
                gsum[threadIdx.x] = acc;
                __syncthreads();
                if (threadIdx.x < nc4) {
                    acc = gsum[threadIdx.x];
                    for (int gg = 1; gg < G; gg++) {
                        const float4 o = gsum[gg * nc4 + threadIdx.x];
                        acc.x += o.x;
                        acc.y += o.y;
                        acc.z += o.z;
                        acc.w += o.w;
                    }
                }
            }
            if ((G > 1 ? threadIdx.x < nc4 : q < nc4)) {
                const int cc = G > 1 ? threadIdx.x : c;
                // (partial rows are D + 1 floats apart: 4-byte stores)
                out[4 * cc + 0] = acc.x;
                out[4 * cc + 1] = acc.y;
                out[4 * cc + 2] = acc.z;
                out[4 * cc + 3] = acc.w;
            }
        }
    } else {
        for (int d = threadIdx.x; d < D; d += 256) {
            float acc = 0.f;
            for (int j = 0; j < KT; j++) {
                int64_t t = t0 + j;
                if (t >= BT) break;
                float h = BF16IN ? bf2f(((const bf16*)hv)[t * D + d]) : ((const float*)hv)[t * D + d];
                acc += h * nrm[j];
            }
            out[d] = acc;
        }
    }
    if (threadIdx.x == 0) {
        float w = 0.f;
        for (int j = 0; j < KT; j++) w += nrm[j];
        out[D] = w;
    }
}

// acc[d] += sum over blocks of part[b][d], in F64: 64 columns per block
// (lane = column), wave w of kRW sums the blocks of its slice in block order
// and the slice sums are added in wave order — a fixed order, so the result
// is deterministic.
constexpr int kRW = 16;
__global__ __launch_bounds__(64 * kRW) void k_centroid_reduce(const float* __restrict__ part,
                                                              int nblk, int D1,
                                                              double* __restrict__ acc,
                                                              const int32_t* __restrict__ skip) {
    if (skip && *skip) return;
    __shared__ double q[kRW][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int d = blockIdx.x * 64 + lane;
    const int per = (nblk + kRW - 1) / kRW, b0 = w * per, b1 = min(nblk, b0 + per);
    double s = 0.0;
    if (d < D1) {
#pragma unroll 8
        for (int b = b0; b < b1; b++) s += (double)part[(int64_t)b * D1 + d];
    }
    q[w][lane] = s;
    __syncthreads();
    if (w == 0 && d < D1) {
        double t = q[0][lane];
        for (int i = 1; i < kRW; i++) t += q[i][lane];
        acc[d] += t;
    }
}

// ── k-means ────────────────────────────────────────────────────────────
// Squared distance summed sequentially over i in F32 without contraction.
// Operands are loaded 32 elements at a time (independent loads in flight)
// before the dependent chain over them; the order of the additions is the
// plain loop's.
__device__ __forceinline__ float sqdist_seq(const float* __restrict__ a,
                                           const float* __restrict__ b, int D) {
    // hipcc would contract v * v + d into one FMA (one rounding where the
    // sequential form rounds twice): each product passes through an empty
    // asm statement, which no instruction combiner can look through
    constexpr int CH = 32;
    float d = 0.f;
    int i = 0;
    for (; i + CH <= D; i += CH) {
        float av[CH], bv[CH];
#pragma unroll
        for (int j = 0; j < CH; j++) {
            av[j] = a[i + j];
            bv[j] = b[i + j];
        }
#pragma unroll
        for (int j = 0; j < CH; j++) {
            float v = __fsub_rn(av[j], bv[j]);
            float q = __fmul_rn(v, v);
            asm volatile("" : "+v"(q));
            d = __fadd_rn(d, q);
        }
    }
    for (; i < D; i++) {
        float v = __fsub_rn(a[i], b[i]);
        float q = __fmul_rn(v, v);
        asm volatile("" : "+v"(q));
        d = __fadd_rn(d, q);
    }
    return d;
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__device__ __forceinline__ double u01(uint64_t& s) {
    return (double)(splitmix64(s) >> 11) * (1.0 / 9007199254740992.0);
}

// Up to J distance chains against one center b (rows a0 + i * astride,
// i < na), each chain in the order of sqdist_seq: every center chunk is
// loaded once for all rows.
template <int J>
__device__ __forceinline__ void sqdist_seq_rows(const float* __restrict__ a0, int64_t astride,
                                                int na, const float* __restrict__ b, int D,
                                                float* __restrict__ out) {
    constexpr int CH = 32;
    float d[J];
#pragma unroll
    for (int r = 0; r < J; r++) d[r] = 0.f;
    int i = 0;
    for (; i + CH <= D; i += CH) {
        float bv[CH];
#pragma unroll
        for (int j = 0; j < CH; j++) bv[j] = b[i + j];
#pragma unroll
        for (int r = 0; r < J; r++) {
            if (r >= na) break;
            const float* a = a0 + r * astride + i;
            float av[CH];
#pragma unroll
            for (int j = 0; j < CH; j++) av[j] = a[j];
#pragma unroll
            for (int j = 0; j < CH; j++) {
                float v = __fsub_rn(av[j], bv[j]);
                float q = __fmul_rn(v, v);
                asm volatile("" : "+v"(q));
                d[r] = __fadd_rn(d[r], q);
            }
        }
    }
    for (; i < D; i++)
#pragma unroll
        for (int r = 0; r < J; r++) {
            if (r >= na) break;
            float v = __fsub_rn(a0[r * astride + i], b[i]);
            float q = __fmul_rn(v, v);
            asm volatile("" : "+v"(q));
            d[r] = __fadd_rn(d[r], q);
        }
#pragma unroll
    for (int r = 0; r < J; r++)
        if (r < na) out[r] = d[r];
}

// assignment pass: dist[n*k + c] for all pairs, then argmin per n (strict <)
__device__ __forceinline__ int kmeans_assign(const float* __restrict__ X, const float* __restrict__ C, int N,
                             int D, int k, float* __restrict__ dist, int32_t* __restrict__ asg) {
    const int nt = blockDim.x;
    if (nt % k == 0 && (int64_t)N * k <= 2ll * nt) {
        // a thread's pairs p = tid + j * nt share the center c = tid % k:
        // rows n0 and n0 + nt / k
        const int c = threadIdx.x % k, n0 = threadIdx.x / k, st = nt / k;
        const int na = n0 < N ? (n0 + st < N ? 2 : 1) : 0;
        float dd[2];
        if (na > 0)
            sqdist_seq_rows<2>(X + (int64_t)n0 * D, (int64_t)st * D, na, C + (int64_t)c * D, D, dd);
        if (na > 0) dist[(int64_t)n0 * k + c] = dd[0];
        if (na > 1) dist[(int64_t)(n0 + st) * k + c] = dd[1];
    } else {
        for (int p = threadIdx.x; p < N * k; p += blockDim.x)
            dist[p] = sqdist_seq(X + (int64_t)(p / k) * D, C + (int64_t)(p % k) * D, D);
    }
    __syncthreads();
    int changed = 0;
    for (int n = threadIdx.x; n < N; n += blockDim.x) {
        float best = 1e38f;
        int bk = 0;
        for (int c = 0; c < k; c++) {
            float d = dist[(int64_t)n * k + c];
            if (d < best) {
                best = d;
                bk = c;
            }
        }
        if (asg[n] != bk) {
            asg[n] = bk;
            changed = 1;
        }
    }
    return __syncthreads_or(changed);
}

// update pass: center c = mean of members (sequential over n); empty ->
// zero (reference mode) or unchanged (stress mode)
__device__ __forceinline__ void kmeans_update(const float* __restrict__ X, float* __restrict__ C, int N, int D,
                              int k, const int32_t* __restrict__ asg, bool empty_to_zero) {
    for (int p = threadIdx.x; p < k * D; p += blockDim.x) {
        int c = p / D, d = p % D;
        float s = 0.f;
        int cnt = 0;
        // members' values loaded 16 snapshots at a time, added in index order
        constexpr int CH = 16;
        int n = 0;
        for (; n + CH <= N; n += CH) {
            float xv[CH];
            int av[CH];
#pragma unroll
            for (int j = 0; j < CH; j++) {
                xv[j] = X[(int64_t)(n + j) * D + d];
                av[j] = asg[n + j];
            }
#pragma unroll
            for (int j = 0; j < CH; j++)
                if (av[j] == c) {
                    s = __fadd_rn(s, xv[j]);
                    cnt++;
                }
        }
        for (; n < N; n++)
            if (asg[n] == c) {
                s = __fadd_rn(s, X[(int64_t)n * D + d]);
                cnt++;
            }
        if (cnt > 0)
            C[p] = s / (float)cnt;
        else if (empty_to_zero)
            C[p] = 0.f;
    }
    __syncthreads();
}

// Snapshots that fit kXs floats are copied into LDS once (XL): the
// distance chains and the center sums then read them from LDS.
constexpr int kXs = 32768;  // 128 KB
constexpr int kDs = 4096;   // distances held in LDS by k_kmeans_pp<true>

template <bool XL>
__device__ __forceinline__ const float* stage_snapshots(const float* __restrict__ Xg, float* xs,
                                                        int N, int D) {
    if constexpr (!XL) return Xg;
    for (int p = threadIdx.x; p < N * D; p += blockDim.x) xs[p] = Xg[p];
    __syncthreads();
    return xs;
}

template <bool XL>
__global__ __launch_bounds__(1024) void k_kmeans_ref(const float* __restrict__ Xg, int N, int D,
                                                     int k, int max_iters,
                                                     float* __restrict__ C,
                                                     int32_t* __restrict__ asg,
                                                     float* __restrict__ dist,
                                                     int32_t* __restrict__ iters_out) {
    __shared__ float xs[XL ? kXs : 1];
    const float* __restrict__ X = stage_snapshots<XL>(Xg, xs, N, D);
    for (int p = threadIdx.x; p < k * D; p += blockDim.x) {
        int c = p / D, d = p % D;
        C[p] = X[(int64_t)(((int64_t)c * N) / k) * D + d];
    }
    for (int n = threadIdx.x; n < N; n += blockDim.x) asg[n] = 0;
    __syncthreads();
    int it = 0;
    for (; it < max_iters; it++) {
        int changed = kmeans_assign(X, C, N, D, k, dist, asg);
        if (!changed) break;
        kmeans_update(X, C, N, D, k, asg, true);
    }
    if (threadIdx.x == 0 && iters_out) *iters_out = it;
}

template <bool XL>
__global__ __launch_bounds__(1024) void k_kmeans_pp(const float* __restrict__ Xg,
                                                    const float* __restrict__ W, int N, int D,
                                                    int k, int iters, uint64_t seed,
                                                    float* __restrict__ Cw,  // [k*D] work
                                                    float* __restrict__ d2g,  // [N]
                                                    float* __restrict__ distg,  // [N*k]
                                                    int32_t* __restrict__ asgg,  // [N]
                                                    float* __restrict__ C_out,
                                                    int32_t* __restrict__ asg_out,
                                                    double* __restrict__ mass_out,
                                                    int32_t* __restrict__ seeds_out) {
    // XL (N*D <= kXs, N <= 1024, N*k <= kDs): snapshots, assignments,
    // distances and the seeding distances in LDS; the ranking arrays reuse
    // the snapshot region once the last assignment pass has read it
    __shared__ int chosen[1024];
    __shared__ uint64_t rng;
    __shared__ __attribute__((aligned(16))) float xs[XL ? kXs : 1];
    __shared__ int sasg[XL ? 1024 : 1];
    __shared__ float sdist[XL ? kDs : 1];
    __shared__ float sd2[XL ? 1024 : 1];
    __shared__ double smass[XL ? 1 : 1024];
    __shared__ int sorder[XL ? 1 : 1024], srank[XL ? 1 : 1024];
    const float* __restrict__ X = stage_snapshots<XL>(Xg, xs, N, D);
    int32_t* asg = XL ? sasg : asgg;
    float* dist = XL ? sdist : distg;
    float* d2 = XL ? sd2 : d2g;
    double* mass = XL ? (double*)xs : smass;
    int* order = XL ? (int*)(xs + 2 * 1024) : sorder;
    int* rank_of = XL ? (int*)(xs + 3 * 1024) : srank;
    if (threadIdx.x == 0) {
        rng = seed;
        int first = (int)(u01(rng) * N);
        if (first >= N) first = N - 1;
        chosen[0] = first;
    }
    for (int n = threadIdx.x; n < N; n += blockDim.x) d2[n] = FLT_MAX;
    __syncthreads();
    // k-means++ seeding
    for (int m = 1; m < k; m++) {
        const float* c = X + (int64_t)chosen[m - 1] * D;
        for (int n = threadIdx.x; n < N; n += blockDim.x) {
            float d = sqdist_seq(X + (int64_t)n * D, c, D);
            if (d < d2[n]) d2[n] = d;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            double total = 0.0;
            for (int n = 0; n < N; n++) total += (double)d2[n];
            double target = u01(rng) * total;
            int pick = -1, last_pos = -1;
            double run = 0.0;
            for (int n = 0; n < N; n++) {
                run += (double)d2[n];
                if (d2[n] > 0.f) last_pos = n;
                if (pick < 0 && run > target && d2[n] > 0.f) pick = n;
            }
            if (pick < 0) pick = (last_pos >= 0) ? last_pos : m % N;
            chosen[m] = pick;
        }
        __syncthreads();
    }
    for (int p = threadIdx.x; p < k * D; p += blockDim.x)
        Cw[p] = X[(int64_t)chosen[p / D] * D + (p % D)];
    for (int n = threadIdx.x; n < N; n += blockDim.x) asg[n] = 0;
    __syncthreads();
    for (int it = 0; it < iters; it++) {
        kmeans_assign(X, Cw, N, D, k, dist, asg);
        kmeans_update(X, Cw, N, D, k, asg, false);
    }
    kmeans_assign(X, Cw, N, D, k, dist, asg);
    // rank by member weight (F64, index order), stable descending
    if (threadIdx.x == 0) {
        for (int c = 0; c < k; c++) mass[c] = 0.0;
        for (int n = 0; n < N; n++) mass[asg[n]] += (double)W[n];
        for (int c = 0; c < k; c++) order[c] = c;
        for (int i = 1; i < k; i++) {  // insertion sort: stable
            int v = order[i];
            int j = i - 1;
            while (j >= 0 && mass[order[j]] < mass[v]) {
                order[j + 1] = order[j];
                j--;
            }
            order[j + 1] = v;
        }
        for (int r = 0; r < k; r++) rank_of[order[r]] = r;
    }
    __syncthreads();
    for (int p = threadIdx.x; p < k * D; p += blockDim.x)
        C_out[p] = Cw[(int64_t)order[p / D] * D + (p % D)];
    for (int n = threadIdx.x; n < N; n += blockDim.x) asg_out[n] = rank_of[asg[n]];
    for (int r = threadIdx.x; r < k; r += blockDim.x) {
        if (mass_out) mass_out[r] = mass[order[r]];
        if (seeds_out) seeds_out[r] = chosen[r];
    }
}

}  // namespace ta

using namespace ta;

static int centroid_acc(const void* h, const void* g, const float* n, int64_t BT, int D,
                        double* acc, bool bf16in, void* stream, const int32_t* skip = nullptr) {
    TA_REQUIRE(BT >= 0 && D > 0, "centroid_accumulate: bad shape BT=%lld D=%d", (long long)BT, D);
    if (BT == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    const int kt = bf16in ? kTok : kTokF;
    int64_t nblk = (BT + kt - 1) / kt;
    TA_REQUIRE(nblk < (1ll << 31), "centroid_accumulate: BT too large");
    float* part = (float*)scratch_get((size_t)nblk * (D + 1) * sizeof(float), s);
    TA_REQUIRE(part, "centroid_accumulate: scratch allocation failed");
    if (bf16in)
        k_centroid_part<true><<<(int)nblk, 256, 0, s>>>(h, g, nullptr, BT, D, part);
    else
        k_centroid_part<false><<<(int)nblk, 256, 0, s>>>(h, g, n, BT, D, part);
    k_centroid_reduce<<<(D + 1 + 63) / 64, 64 * kRW, 0, s>>>(part, (int)nblk, D + 1, acc, skip);
    return check_launch("centroid_accumulate");
}

namespace ta {
int centroid_acc_bf16(const bf16* h, const bf16* g, int64_t BT, int D, double* acc,
                      const int32_t* skip, hipStream_t s) {
    return centroid_acc(h, g, nullptr, BT, D, acc, true, s, skip);
}
}  // namespace ta

// Device address of `scratch` on device dev, looked up once per device with
// that device current and kept.
static std::mutex g_na_mu;
static float* g_na_ptr[64];

static int noalloc_scratch(int dev, float** out) {
    TA_REQUIRE(dev >= 0 && dev < 64, "centroid_accumulate_bf16_noalloc: device %d out of range", dev);
    std::lock_guard<std::mutex> lk(g_na_mu);
    if (!g_na_ptr[dev]) {
        void* p = nullptr;
        TA_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        TA_REQUIRE(p, "centroid_accumulate_bf16_noalloc: no device address for the scratch");
        g_na_ptr[dev] = (float*)p;
    }
    *out = g_na_ptr[dev];
    return 0;
}

// Makes `dev` the current device for the lifetime of the object and restores
// the caller's device afterwards.
struct DeviceScope {
    int prev = -1;
    hipError_t err = hipSuccess;
    explicit DeviceScope(int dev) {
        err = hipGetDevice(&prev);
        if (err == hipSuccess && prev != dev) err = hipSetDevice(dev);
    }
    ~DeviceScope() {
        if (prev >= 0) (void)hipSetDevice(prev);
    }
};

extern "C" {

int ta_centroid_accumulate_bf16(const uint16_t* h, const uint16_t* g, int64_t BT, int D,
                                double* acc, void* stream) {
    return centroid_acc(h, g, nullptr, BT, D, acc, true, stream);
}

int ta_centroid_accumulate_bf16_noalloc(const uint16_t* h, const uint16_t* g, int64_t BT, int D,
                                        double* acc, void* stream) {
    TA_REQUIRE(h && g && acc, "centroid_accumulate_bf16_noalloc: null argument");
    TA_REQUIRE(BT >= 0 && D > 0, "centroid_accumulate_bf16_noalloc: bad shape BT=%lld D=%d",
               (long long)BT, D);
    if (BT == 0) return 0;
    const int64_t nblk = (BT + kTok - 1) / kTok;
    const int64_t max_blk = (int64_t)(kNoAllocScratchBytes / sizeof(float)) / (D + 1);
    TA_REQUIRE(nblk <= max_blk,
               "centroid_accumulate_bf16_noalloc: BT=%lld at D=%d needs %lld partial rows of "
               "D+1 floats, over the %zu-byte static scratch (at most BT=%lld at this D)",
               (long long)BT, D, (long long)nblk, kNoAllocScratchBytes,
               (long long)(max_blk * kTok));
    hipStream_t s = (hipStream_t)stream;
    // the stream's device (the current one for the null stream) holds the
    // scratch copy and runs the kernels
    int dev = 0;
    if (s)
        TA_HIP(hipStreamGetDevice(s, &dev));
    else
        TA_HIP(hipGetDevice(&dev));
    DeviceScope scope(dev);
    TA_HIP(scope.err);
    float* part = nullptr;
    const int rc = noalloc_scratch(dev, &part);
    if (rc != 0) return rc;
    // the same kernels and order as ta_centroid_accumulate_bf16: every
    // partial row is written in full before the reduce reads it
    k_centroid_part<true><<<(int)nblk, 256, 0, s>>>(h, g, nullptr, BT, D, part);
    k_centroid_reduce<<<(D + 1 + 63) / 64, 64 * kRW, 0, s>>>(part, (int)nblk, D + 1, acc,
                                                             nullptr);
    return check_launch("centroid_accumulate_bf16_noalloc");
}

int ta_centroid_accumulate_f32(const float* h, const float* g, int64_t BT, int D, double* acc,
                               void* stream) {
    TA_REQUIRE(h && g && acc, "centroid_accumulate_f32: null argument");
    return centroid_acc(h, g, nullptr, BT, D, acc, false, stream);
}

int ta_centroid_accumulate_f32n(const float* h, const float* n, int64_t BT, int D, double* acc,
                                void* stream) {
    return centroid_acc(h, nullptr, n, BT, D, acc, false, stream);
}

int ta_kmeans_ref(const float* snaps, int N, int D, int k, int max_iters, float* centers,
                  int32_t* assign, int32_t* iters_out, void* stream) {
    TA_REQUIRE(N > 0 && D > 0 && k > 0 && max_iters >= 0, "kmeans_ref: bad N=%d D=%d k=%d", N, D,
               k);
    if (k > N) k = N;
    hipStream_t s = (hipStream_t)stream;
    float* dist = (float*)scratch_get((size_t)N * k * sizeof(float), s);
    TA_REQUIRE(dist, "kmeans_ref: scratch allocation failed");
    if ((int64_t)N * D <= kXs)
        k_kmeans_ref<true><<<1, 1024, 0, s>>>(snaps, N, D, k, max_iters, centers, assign, dist,
                                              iters_out);
    else
        k_kmeans_ref<false><<<1, 1024, 0, s>>>(snaps, N, D, k, max_iters, centers, assign, dist,
                                               iters_out);
    return check_launch("kmeans_ref");
}

int ta_kmeans_pp(const float* snaps, const float* weights, int N, int D, int k, int iters,
                 uint64_t seed, float* centers, int32_t* assign, double* mass, int32_t* seeds,
                 void* stream) {
    TA_REQUIRE(N > 0 && D > 0 && k > 0 && iters >= 0, "kmeans_pp: bad N=%d D=%d k=%d", N, D, k);
    if (k > N) k = N;
    TA_REQUIRE(k <= 1024, "kmeans_pp: k=%d exceeds 1024", k);
    hipStream_t s = (hipStream_t)stream;
    size_t off_d2 = (size_t)k * D * sizeof(float);
    off_d2 = (off_d2 + 255) & ~(size_t)255;
    size_t off_dist = off_d2 + (((size_t)N * sizeof(float) + 255) & ~(size_t)255);
    size_t off_asg = off_dist + (((size_t)N * k * sizeof(float) + 255) & ~(size_t)255);
    size_t total = off_asg + (size_t)N * sizeof(int32_t);
    char* base = (char*)scratch_get(total, s);
    TA_REQUIRE(base, "kmeans_pp: scratch allocation failed");
    if ((int64_t)N * D <= kXs && N <= 1024 && (int64_t)N * k <= kDs)
        k_kmeans_pp<true><<<1, 1024, 0, s>>>(snaps, weights, N, D, k, iters, seed, (float*)base,
                                             (float*)(base + off_d2), (float*)(base + off_dist),
                                             (int32_t*)(base + off_asg), centers, assign, mass,
                                             seeds);
    else
        k_kmeans_pp<false><<<1, 1024, 0, s>>>(snaps, weights, N, D, k, iters, seed, (float*)base,
                                              (float*)(base + off_d2), (float*)(base + off_dist),
                                              (int32_t*)(base + off_asg), centers, assign, mass,
                                              seeds);
    return check_launch("kmeans_pp");
}

}  // extern "C"
