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
// sums run over each center's members in snapshot index order.  Every loop
// is bounded by max_iters / iters, so the launch always drains.
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
// Squared distances are sums over i = 0 .. D-1 in order, in F32, each term
// (a_i - b_i)^2 rounded before it is added (no contraction), like the
// reference's scalar loop.
//
// Snapshots staged in LDS keep row n's 16-byte chunks XOR-permuted by
// n & sw (sw + 1: the largest power of two up to 16 dividing D / 4):
// element (n, i) sits at n * D + snap_col(n, i, sw).  Rows read at one
// chunk by the lanes (the distance chains, one row per lane) then fall in
// distinct bank groups, and 64 consecutive columns of one row (the center
// sums, one column per lane) in distinct banks; every chain still visits i
// in order.  Snapshots read from global memory are not permuted (sw = 0).
__device__ __forceinline__ int snap_swizzle(int D) {
    return D % 4 == 0 ? min(16, (D >> 2) & -(D >> 2)) - 1 : 0;
}
__device__ __forceinline__ int snap_col(int n, int i, int sw) {
    return ((((i >> 2) ^ (n & sw))) << 2) | (i & 3);
}

// (a - b)^2 as the reference rounds it: hipcc would contract v * v + d into
// one FMA (one rounding where the sequential form rounds twice), so each
// product passes through an empty asm statement, which no instruction
// combiner can look through
__device__ __forceinline__ float sq_term(float a, float b) {
    const float v = __fsub_rn(a, b);
    float q = __fmul_rn(v, v);
    asm volatile("" : "+v"(q));
    return q;
}

// J distance chains: row n[r] of the snapshots X (permuted by sw) against
// the center at cb[r] (its chunks permuted by kb[r]).  With vec (D % 4 == 0,
// rows and centers 16-byte aligned) the operands move as 16-byte chunks, CH
// elements of every chain loaded before the dependent chains over them.
template <int J, int CH>
__device__ __forceinline__ void sqdist_chains(const float* __restrict__ X, int D, int sw, bool vec,
                                              const int (&n)[J], const float* const (&cb)[J],
                                              const int (&kb)[J], float (&out)[J]) {
    static_assert(CH % 4 == 0, "whole chunks");
    float d[J];
    int ka[J];
    const float* ar[J];
#pragma unroll
    for (int r = 0; r < J; r++) {
        d[r] = 0.f;
        ka[r] = n[r] & sw;
        ar[r] = X + (int64_t)n[r] * D;
    }
    int i = 0;
    if (vec) {
        for (; i + CH <= D; i += CH) {
            float4 av[J][CH / 4], bv[J][CH / 4];
#pragma unroll
            for (int r = 0; r < J; r++)
#pragma unroll
                for (int q = 0; q < CH / 4; q++) {
                    const int ch = (i >> 2) + q;
                    av[r][q] = *(const float4*)(ar[r] + ((ch ^ ka[r]) << 2));
                    bv[r][q] = *(const float4*)(cb[r] + ((ch ^ kb[r]) << 2));
                }
#pragma unroll
            for (int q = 0; q < CH / 4; q++)
#pragma unroll
                for (int r = 0; r < J; r++) {
                    d[r] = __fadd_rn(d[r], sq_term(av[r][q].x, bv[r][q].x));
                    d[r] = __fadd_rn(d[r], sq_term(av[r][q].y, bv[r][q].y));
                    d[r] = __fadd_rn(d[r], sq_term(av[r][q].z, bv[r][q].z));
                    d[r] = __fadd_rn(d[r], sq_term(av[r][q].w, bv[r][q].w));
                }
        }
    }
    for (; i < D; i++)
#pragma unroll
        for (int r = 0; r < J; r++)
            d[r] = __fadd_rn(d[r], sq_term(ar[r][snap_col(n[r], i, sw)], cb[r][snap_col(kb[r], i, sw)]));
#pragma unroll
    for (int r = 0; r < J; r++) out[r] = d[r];
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

// Assignment pass: every (center, snapshot) distance into dist [k][N], then
// each snapshot's argmin over the centers (strict <, so the first of equal
// distances).  A wave takes one center at a time (read at one address by all
// its lanes) against 64 snapshots (one per lane), two such units at once.
// C: the centers [k][D], not permuted.  Returns whether any assignment
// changed (block-wide).
__device__ __forceinline__ int kmeans_assign(const float* __restrict__ X, int sw, bool vec,
                                             const float* __restrict__ C, int N, int D, int k,
                                             float* __restrict__ dist, int32_t* __restrict__ asg) {
    const int lane = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
    const int nb = (N + 63) / 64, units = k * nb;
    for (int u = w; u < units; u += 2 * nw) {
        const int u1 = u + nw < units ? u + nw : u;
        const int c0 = u / nb, c1 = u1 / nb;
        const int r0 = (u % nb) * 64 + lane, r1 = (u1 % nb) * 64 + lane;
        const int n[2] = {min(r0, N - 1), min(r1, N - 1)};
        const float* const cb[2] = {C + (int64_t)c0 * D, C + (int64_t)c1 * D};
        const int kb[2] = {0, 0};
        float d[2];
        sqdist_chains<2, 16>(X, D, sw, vec, n, cb, kb, d);
        if (r0 < N) dist[(int64_t)c0 * N + r0] = d[0];
        if (u1 != u && r1 < N) dist[(int64_t)c1 * N + r1] = d[1];
    }
    __syncthreads();
    int changed = 0;
    for (int n = threadIdx.x; n < N; n += blockDim.x) {
        float best = 1e38f;
        int bk = 0;
        for (int c = 0; c < k; c++) {
            const float d = dist[(int64_t)c * N + n];
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

// Update pass: center c = the mean of its members, summed in snapshot index
// order; an empty center becomes zero (reference mode) or stays (stress
// mode).  When every wave's 64 outputs belong to one center (D a multiple of
// 64), a ballot over 64 assignments at a time gives its members in index
// order and only their values are read; otherwise each output scans every
// snapshot.  Either way the same chain of additions.
__device__ __forceinline__ void kmeans_update(const float* __restrict__ X, int sw,
                                              float* __restrict__ C, int N, int D, int k,
                                              const int32_t* __restrict__ asg,
                                              bool empty_to_zero) {
    const bool ballot = D % 64 == 0 && blockDim.x % 64 == 0;
    const int lane = threadIdx.x & 63;
    // the first 256 assignments stay in registers for every output
    int a4[4];
#pragma unroll
    for (int q = 0; q < 4; q++) a4[q] = ballot && 64 * q + lane < N ? asg[64 * q + lane] : -1;
    for (int p = threadIdx.x; p < k * D; p += blockDim.x) {
        const int c = p / D, d = p % D;
        float s = 0.f;
        int cnt = 0;
        if (ballot) {
            for (int n0 = 0; n0 < N; n0 += 64) {
                const int a = n0 < 256 ? a4[n0 >> 6] : n0 + lane < N ? asg[n0 + lane] : -1;
                uint64_t mem = __ballot(a == c);
                // up to four members' values loaded together, then added in
                // index order
                while (mem) {
                    float xv[4];
                    int nm = 0;
#pragma unroll
                    for (int u = 0; u < 4; u++) {
                        if (!mem) break;
                        const int n = n0 + __builtin_ctzll(mem);
                        mem &= mem - 1;
                        xv[u] = X[(int64_t)n * D + snap_col(n, d, sw)];
                        nm++;
                    }
#pragma unroll
                    for (int u = 0; u < 4; u++)
                        if (u < nm) s = __fadd_rn(s, xv[u]);
                    cnt += nm;
                }
            }
        } else {
            for (int n = 0; n < N; n++)
                if (asg[n] == c) {
                    s = __fadd_rn(s, X[(int64_t)n * D + snap_col(n, d, sw)]);
                    cnt++;
                }
        }
        if (cnt > 0)
            C[p] = s / (float)cnt;
        else if (empty_to_zero)
            C[p] = 0.f;
    }
    __syncthreads();
}

// Snapshots that fit kXs floats are copied into LDS once (XL, permuted as
// above): the distance chains and the center sums then read them from LDS.
constexpr int kXs = 32768;  // 128 KB
constexpr int kDs = 4096;   // distances held in LDS by k_kmeans_pp<true>

template <bool XL>
__device__ __forceinline__ const float* stage_snapshots(const float* __restrict__ Xg, float* xs,
                                                        int N, int D, int& sw) {
    if constexpr (!XL) {
        sw = 0;
        return Xg;
    }
    sw = snap_swizzle(D);
    for (int p = threadIdx.x; p < N * D; p += blockDim.x) {
        const int n = p / D, d = p % D;
        xs[(int64_t)n * D + snap_col(n, d, sw)] = Xg[p];
    }
    __syncthreads();
    return xs;
}

template <bool XL>
__global__ __launch_bounds__(1024) void k_kmeans_ref(const float* __restrict__ Xg, int N, int D,
                                                     int k, int max_iters,
                                                     float* __restrict__ C,
                                                     int32_t* __restrict__ asg,
                                                     float* __restrict__ dist,
                                                     int32_t* __restrict__ iters_out, bool vec) {
    __shared__ __attribute__((aligned(16))) float xs[XL ? kXs : 1];
    int sw = 0;
    const float* __restrict__ X = stage_snapshots<XL>(Xg, xs, N, D, sw);
    for (int p = threadIdx.x; p < k * D; p += blockDim.x) {
        const int c = p / D, d = p % D, n = (int)(((int64_t)c * N) / k);
        C[p] = X[(int64_t)n * D + snap_col(n, d, sw)];
    }
    for (int n = threadIdx.x; n < N; n += blockDim.x) asg[n] = 0;
    __syncthreads();
    int it = 0;
    for (; it < max_iters; it++) {
        int changed = kmeans_assign(X, sw, vec, C, N, D, k, dist, asg);
        if (!changed) break;
        kmeans_update(X, sw, C, N, D, k, asg, true);
    }
    if (threadIdx.x == 0 && iters_out) *iters_out = it;
}

// Phases of k_kmeans_pp: the whole merge in one launch, or (the Lloyd
// iterations spread over many workgroups in launches of their own,
// k_kmeans_dist + k_kmeans_step) the seeding up to the initial centers and
// zero assignments, and the ranking after the last assignment.
enum KmPhase { KM_ALL = 0, KM_SEED = 1, KM_RANK = 2 };

template <bool XL, int PH = KM_ALL>
__global__ __launch_bounds__(1024) void k_kmeans_pp(const float* __restrict__ Xg,
                                                    const float* __restrict__ W, int N, int D,
                                                    int k, int iters, uint64_t seed,
                                                    float* __restrict__ Cw,  // [k*D] work
                                                    float* __restrict__ d2g,  // [N]
                                                    float* __restrict__ distg,  // [k*N]
                                                    int32_t* __restrict__ asgg,  // [N]
                                                    int32_t* __restrict__ chosen_g,  // [k]
                                                    float* __restrict__ C_out,
                                                    int32_t* __restrict__ asg_out,
                                                    double* __restrict__ mass_out,
                                                    int32_t* __restrict__ seeds_out, bool vec) {
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
    int sw = 0;
    const float* __restrict__ X =
        PH == KM_RANK ? Xg : stage_snapshots<XL>(Xg, xs, N, D, sw);
    // (the split phases keep the assignments in global memory)
    int32_t* asg = XL && PH == KM_ALL ? sasg : asgg;
    float* dist = XL ? sdist : distg;
    float* d2 = XL ? sd2 : d2g;
    double* mass = XL ? (double*)xs : smass;
    int* order = XL ? (int*)(xs + 2 * 1024) : sorder;
    int* rank_of = XL ? (int*)(xs + 3 * 1024) : srank;
    if constexpr (PH != KM_RANK) {
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
        const int cm = chosen[m - 1];
        for (int n = threadIdx.x; n < N; n += blockDim.x) {
            const int nn[1] = {n};
            const float* const cb[1] = {X + (int64_t)cm * D};
            const int kb[1] = {cm & sw};
            float d[1];
            sqdist_chains<1, 32>(X, D, sw, vec, nn, cb, kb, d);
            if (d[0] < d2[n]) d2[n] = d[0];
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
    for (int p = threadIdx.x; p < k * D; p += blockDim.x) {
        const int n = chosen[p / D], d = p % D;
        Cw[p] = X[(int64_t)n * D + snap_col(n, d, sw)];
    }
    for (int n = threadIdx.x; n < N; n += blockDim.x) asg[n] = 0;
    if constexpr (PH == KM_SEED) {
        for (int r = threadIdx.x; r < k; r += blockDim.x) chosen_g[r] = chosen[r];
        return;
    }
    __syncthreads();
    for (int it = 0; it < iters; it++) {
        kmeans_assign(X, sw, vec, Cw, N, D, k, dist, asg);
        kmeans_update(X, sw, Cw, N, D, k, asg, false);
    }
    kmeans_assign(X, sw, vec, Cw, N, D, k, dist, asg);
    } else {
        for (int r = threadIdx.x; r < k; r += blockDim.x) chosen[r] = chosen_g[r];
        __syncthreads();
    }
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

// One Lloyd assignment pass spread over the GPU: block (c, j) is one wave
// with center c against snapshots 64 j .. 64 j + 63 (one distance chain per
// lane, the order of sqdist_chains), into dist [k][N].
__global__ __launch_bounds__(64) void k_kmeans_dist(const float* __restrict__ X,
                                                    const float* __restrict__ C, int N, int D,
                                                    bool vec, float* __restrict__ dist) {
    const int c = blockIdx.x, n = blockIdx.y * 64 + threadIdx.x;
    const int nn[1] = {min(n, N - 1)};
    const float* const cb[1] = {C + (int64_t)c * D};
    const int kb[1] = {0};
    float d[1];
    sqdist_chains<1, 64>(X, D, 0, vec, nn, cb, kb, d);
    if (n < N) dist[(int64_t)c * N + n] = d[0];
}

// Then each snapshot's argmin over dist (strict <, as kmeans_assign) and,
// with update, the centers' member means (kmeans_update, stress mode).
__global__ __launch_bounds__(1024) void k_kmeans_step(const float* __restrict__ X,
                                                      float* __restrict__ C, int N, int D, int k,
                                                      const float* __restrict__ dist,
                                                      int32_t* __restrict__ asg, bool update) {
    for (int n = threadIdx.x; n < N; n += blockDim.x) {
        // (the distances come from global memory: 16 loads in flight)
        float best = 1e38f;
        int bk = 0;
        for (int c0 = 0; c0 < k; c0 += 16) {
            float v[16];
#pragma unroll
            for (int u = 0; u < 16; u++) v[u] = c0 + u < k ? dist[(int64_t)(c0 + u) * N + n] : 0.f;
#pragma unroll
            for (int u = 0; u < 16; u++)
                if (c0 + u < k && v[u] < best) {
                    best = v[u];
                    bk = c0 + u;
                }
        }
        asg[n] = bk;
    }
    if (!update) return;
    __syncthreads();
    kmeans_update(X, 0, C, N, D, k, asg, false);
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
        tlaunch(k_centroid_part<true>, dim3((int)nblk), dim3(256), s, h, g, nullptr, BT, D, part);
    else
        tlaunch(k_centroid_part<false>, dim3((int)nblk), dim3(256), s, h, g, n, BT, D, part);
    tlaunch(k_centroid_reduce, dim3((D + 1 + 63) / 64), dim3(64 * kRW), s, part, (int)nblk, D + 1, acc, skip);
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
    tlaunch(k_centroid_part<true>, dim3((int)nblk), dim3(256), s, h, g, nullptr, BT, D, part);
    tlaunch(k_centroid_reduce, dim3((D + 1 + 63) / 64), dim3(64 * kRW), s, part, (int)nblk, D + 1, acc,
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
    // 16-byte operand loads: whole chunks, and aligned snapshots (when read
    // from global memory) and centers
    const bool xl = (int64_t)N * D <= kXs;
    const bool vec = D % 4 == 0 && ((uintptr_t)centers & 15) == 0 &&
                     (xl || ((uintptr_t)snaps & 15) == 0);
    if (xl)
        tlaunch(k_kmeans_ref<true>, dim3(1), dim3(1024), s, snaps, N, D, k, max_iters, centers, assign, dist,
                                              iters_out, vec);
    else
        tlaunch(k_kmeans_ref<false>, dim3(1), dim3(1024), s, snaps, N, D, k, max_iters, centers, assign, dist,
                                               iters_out, vec);
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
    size_t off_ch = off_asg + (((size_t)N * sizeof(int32_t) + 255) & ~(size_t)255);
    size_t total = off_ch + (size_t)k * sizeof(int32_t);
    char* base = (char*)scratch_get(total, s);
    TA_REQUIRE(base, "kmeans_pp: scratch allocation failed");
    // (the work centers sit at the scratch's 256-byte aligned start)
    const bool xl = (int64_t)N * D <= kXs && N <= 1024 && (int64_t)N * k <= kDs;
    const bool vec = D % 4 == 0 && (xl || ((uintptr_t)snaps & 15) == 0);
    float* Cw = (float*)base;
    float* d2 = (float*)(base + off_d2);
    float* dist = (float*)(base + off_dist);
    int32_t* asg = (int32_t*)(base + off_asg);
    int32_t* ch = (int32_t*)(base + off_ch);
    // Lloyd iterations on one workgroup while their distance work is small
    // (each assignment pass: k N D chain steps on one CU); above that, each
    // pass in launches of its own: the distances over k x ceil(N / 64)
    // waves, then the argmin and the center sums on one workgroup (the same
    // arithmetic in the same order, so the same bits)
    const bool spread = (int64_t)k * N * D >= (int64_t(1) << 19) && iters > 0;
    if (!spread) {
        if (xl)
            tlaunch(k_kmeans_pp<true>, dim3(1), dim3(1024), s, snaps, weights, N, D, k, iters,
                    seed, Cw, d2, dist, asg, ch, centers, assign, mass, seeds, vec);
        else
            tlaunch(k_kmeans_pp<false>, dim3(1), dim3(1024), s, snaps, weights, N, D, k, iters,
                    seed, Cw, d2, dist, asg, ch, centers, assign, mass, seeds, vec);
        return check_launch("kmeans_pp");
    }
    if (xl)
        tlaunch(k_kmeans_pp<true, KM_SEED>, dim3(1), dim3(1024), s, snaps, weights, N, D, k, iters,
                seed, Cw, d2, dist, asg, ch, centers, assign, mass, seeds, vec);
    else
        tlaunch(k_kmeans_pp<false, KM_SEED>, dim3(1), dim3(1024), s, snaps, weights, N, D, k,
                iters, seed, Cw, d2, dist, asg, ch, centers, assign, mass, seeds, vec);
    // the passes read the snapshots from global memory: 16-byte loads need
    // them aligned
    const bool gvec = D % 4 == 0 && ((uintptr_t)snaps & 15) == 0;
    const dim3 dgrid(k, (N + 63) / 64);
    for (int it = 0; it <= iters; it++) {
        tlaunch(k_kmeans_dist, dgrid, dim3(64), s, snaps, Cw, N, D, gvec, dist);
        tlaunch(k_kmeans_step, dim3(1), dim3(1024), s, snaps, Cw, N, D, k, dist, asg, it < iters);
    }
    tlaunch(k_kmeans_pp<false, KM_RANK>, dim3(1), dim3(1024), s, snaps, weights, N, D, k, iters,
            seed, Cw, d2, dist, asg, ch, centers, assign, mass, seeds, vec);
    return check_launch("kmeans_pp");
}

}  // extern "C"
