// oracle.cpp — CPU restatement of tensor-adapt's LoRA training step.
//
// TEST INFRASTRUCTURE ONLY.  Nothing in the product links, loads or calls
// this file.  Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg may use it, and only as the checker / CPU baseline.
//
// Every function restates one piece of the reference, line by line, with the
// reference's rounding points (BF16 round-to-nearest-even after every kernel
// or GEMM output, FP32 element math).  Where the reference accumulates in FP32
// through cuBLAS or a tree reduction of unknown order, this file accumulates
// in FP64 and rounds once, so that it is the "exact" side of every parity
// check.  Math functions are libm calls (expf/logf/powf/sqrtf, sin/cos in
// double); the reference was built with --use_fast_math and its
// approximations are not imitated.
//
// Citations are into /root/reference (carbon-os/tensor-adapt).
//
// Build: oracle/build.sh  (g++ -O3 -march=x86-64-v3 -fopenmp -ffp-contract=off; a portable
// ISA level because the built library also runs on the GPU box's host CPU)
//
// How each function is pinned independently of its own formula is recorded
// in tests/test_oracle_*.py (torch float64 autograd, numpy matmul, closed
// forms, complex-number rotation, brute force).

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>
#include <omp.h>

typedef uint16_t bf16_t;
typedef int64_t i64;

// ─────────────────────────────────────────────────────────────
//  BF16 <-> F32 (IEEE RNE on the F32 bit pattern, NaN kept quiet).
//  Matches __float2bfloat16 / __bfloat162float semantics used throughout
//  ops.cu and base_loader.cpp:62-65.
// ─────────────────────────────────────────────────────────────
static inline float bf2f(bf16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
static inline bf16_t f2bf(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (bf16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (bf16_t)(u >> 16);
}

extern "C" void or_bf16_from_f32(const float* x, bf16_t* y, i64 n);
extern "C" void or_f32_from_bf16(const bf16_t* x, float* y, i64 n);

// ─────────────────────────────────────────────────────────────
//  GEMM core (FP64 accumulation, blocked; used by both GEMM entry points)
// ─────────────────────────────────────────────────────────────
template <typename LoadA, typename LoadB, typename Store>
static void gemm_core(int M, int N, int K, LoadA la, LoadB lb, Store st);

// Accumulation mode of the GEMM core and of the attention contractions.
//   0 (default): FP64 accumulation, rounded once — the exact side of every
//     parity check.
//   1: FP32 accumulators fed by 16-wide K blocks, each block's products
//     summed in k order in FP32 and added to the running FP32 sum (the
//     accumulation a tiled matrix-core GEMM performs, with every rounding
//     point of the reference unchanged).  It exists to measure how far two
//     FP32-accumulating implementations of the same step drift apart over
//     depth; no check uses it as the reference side.
static int g_accum = 0;
extern "C" void or_set_accum_mode(int mode) { g_accum = mode; }
extern "C" int or_get_accum_mode(void) { return g_accum; }

extern "C" {

void or_bf16_from_f32(const float* x, bf16_t* y, i64 n) {
    for (i64 i = 0; i < n; i++) y[i] = f2bf(x[i]);
}
void or_f32_from_bf16(const bf16_t* x, float* y, i64 n) {
    for (i64 i = 0; i < n; i++) y[i] = bf2f(x[i]);
}

// ─────────────────────────────────────────────────────────────
//  GEMM — cuBLAS column-major semantics.
//  gemm_bf16: tensor.cu:144-166 (cublasGemmEx, BF16 in/out, COMPUTE_32F)
//  gemm_f32 : tensor.cu:168-182 (cublasSgemm)
//  C_cm(i,j) = alpha * sum_k opA(i,k) * opB(k,j) + beta * C_cm(i,j)
//  opA(i,k) = transA ? A[k + i*lda] : A[i + k*lda]
//  opB(k,j) = transB ? B[j + k*ldb] : B[k + j*ldb]
//  Validation of M/N/K/ld > 0 follows tensor.cu:134-142 (returns -1).
// ─────────────────────────────────────────────────────────────
}  // extern "C"

template <typename LoadA, typename LoadB, typename Store>
static void gemm_core(int M, int N, int K, LoadA la, LoadB lb, Store st) {
    // Gather opA rows and opB columns into contiguous K-major float arrays.
    std::vector<float> Ar((size_t)M * K), Bc((size_t)N * K);
#pragma omp parallel for schedule(static)
    for (i64 i = 0; i < M; i++)
        for (i64 k = 0; k < K; k++) Ar[(size_t)i * K + k] = la(i, k);
#pragma omp parallel for schedule(static)
    for (i64 j = 0; j < N; j++)
        for (i64 k = 0; k < K; k++) Bc[(size_t)j * K + k] = lb(k, j);
    const int IB = 32, JB = 32, KB = 2048;
    i64 nib = (M + IB - 1) / IB, njb = (N + JB - 1) / JB;
    if (g_accum == 1) {
        // FP32 blocked accumulation: per output, acc += (sum of 16 products
        // in k order), block after block.  Vectorised across the 32 outputs
        // of a row of the tile; each output's own order is sequential.
        const int KS = 16;
#pragma omp parallel for schedule(dynamic)
        for (i64 blk = 0; blk < nib * njb; blk++) {
            i64 i0 = (blk / njb) * IB, j0 = (blk % njb) * JB;
            i64 i1 = std::min<i64>(i0 + IB, M), j1 = std::min<i64>(j0 + JB, N);
            std::vector<float> bt((size_t)K * JB, 0.f);
            for (i64 j = j0; j < j1; j++)
                for (i64 k = 0; k < K; k++) bt[(size_t)k * JB + (j - j0)] = Bc[(size_t)j * K + k];
            for (i64 i = i0; i < i1; i++) {
                const float* a = &Ar[(size_t)i * K];
                float acc[JB], s[JB];
                for (int b = 0; b < JB; b++) acc[b] = 0.f;
                for (i64 k0 = 0; k0 < K; k0 += KS) {
                    i64 k1 = std::min<i64>(k0 + KS, K);
                    for (int b = 0; b < JB; b++) s[b] = 0.f;
                    for (i64 k = k0; k < k1; k++) {
                        const float av = a[k];
                        const float* br = &bt[(size_t)k * JB];
#pragma omp simd
                        for (int b = 0; b < JB; b++) s[b] += av * br[b];
                    }
                    for (int b = 0; b < JB; b++) acc[b] += s[b];
                }
                for (i64 j = j0; j < j1; j++) st(i, j, (double)acc[j - j0]);
            }
        }
        return;
    }
#pragma omp parallel for schedule(dynamic)
    for (i64 blk = 0; blk < nib * njb; blk++) {
        i64 i0 = (blk / njb) * IB, j0 = (blk % njb) * JB;
        i64 i1 = std::min<i64>(i0 + IB, M), j1 = std::min<i64>(j0 + JB, N);
        double acc[IB][JB];
        for (int a = 0; a < IB; a++)
            for (int b = 0; b < JB; b++) acc[a][b] = 0.0;
        for (i64 k0 = 0; k0 < K; k0 += KB) {
            i64 k1 = std::min<i64>(k0 + KB, K);
            for (i64 i = i0; i < i1; i++) {
                const float* a = &Ar[(size_t)i * K];
                for (i64 j = j0; j < j1; j++) {
                    const float* b = &Bc[(size_t)j * K];
                    double s = 0.0;
#pragma omp simd reduction(+ : s)
                    for (i64 k = k0; k < k1; k++) s += (double)a[k] * (double)b[k];
                    acc[i - i0][j - j0] += s;
                }
            }
        }
        for (i64 i = i0; i < i1; i++)
            for (i64 j = j0; j < j1; j++) st(i, j, acc[i - i0][j - j0]);
    }
}

extern "C" {

int or_gemm_bf16(int transA, int transB, int M, int N, int K, float alpha,
                 const bf16_t* A, int lda, const bf16_t* B, int ldb, float beta,
                 bf16_t* C, int ldc) {
    if (M <= 0 || N <= 0 || K <= 0 || lda <= 0 || ldb <= 0 || ldc <= 0) return -1;
    auto la = [&](i64 i, i64 k) {
        return bf2f(transA ? A[k + i * (i64)lda] : A[i + k * (i64)lda]);
    };
    auto lb = [&](i64 k, i64 j) {
        return bf2f(transB ? B[j + k * (i64)ldb] : B[k + j * (i64)ldb]);
    };
    auto st = [&](i64 i, i64 j, double acc) {
        bf16_t* c = &C[i + j * (i64)ldc];
        float v = alpha * (float)acc;
        if (beta != 0.f) v += beta * bf2f(*c);
        *c = f2bf(v);
    };
    gemm_core(M, N, K, la, lb, st);
    return 0;
}

int or_gemm_f32(int transA, int transB, int M, int N, int K, float alpha,
                const float* A, int lda, const float* B, int ldb, float beta,
                float* C, int ldc) {
    if (M <= 0 || N <= 0 || K <= 0 || lda <= 0 || ldb <= 0 || ldc <= 0) return -1;
    auto la = [&](i64 i, i64 k) { return transA ? A[k + i * (i64)lda] : A[i + k * (i64)lda]; };
    auto lb = [&](i64 k, i64 j) { return transB ? B[j + k * (i64)ldb] : B[k + j * (i64)ldb]; };
    auto st = [&](i64 i, i64 j, double acc) {
        float* c = &C[i + j * (i64)ldc];
        float v = alpha * (float)acc;
        if (beta != 0.f) v += beta * (*c);
        *c = v;
    };
    gemm_core(M, N, K, la, lb, st);
    return 0;
}

// ─────────────────────────────────────────────────────────────
//  RMSNorm forward — ops.cu:59-107.  rms_out holds the INVERSE rms
//  (ops.cu:84-86).  out = bf16((x * inv) * w).
// ─────────────────────────────────────────────────────────────
void or_rms_norm_fwd(const bf16_t* x, const bf16_t* w, bf16_t* out, float* rms_out,
                     i64 rows, int D, float eps) {
#pragma omp parallel for schedule(static)
    for (i64 r = 0; r < rows; r++) {
        const bf16_t* xr = x + r * D;
        double ss = 0.0;
        for (int i = 0; i < D; i++) {
            float xi = bf2f(xr[i]);
            ss += (double)(xi * xi);
        }
        float inv = (float)(1.0 / std::sqrt((double)((float)ss / (float)D + eps)));
        rms_out[r] = inv;
        for (int i = 0; i < D; i++) out[r * D + i] = f2bf(bf2f(xr[i]) * inv * bf2f(w[i]));
    }
}

// ─────────────────────────────────────────────────────────────
//  RMSNorm backward — ops.cu:113-170.
//  dot = sum dy*w*x_hat ; dx = inv*(w*dy - x_hat*dot/D) ; dw += dy*x_hat.
//  dw may be null (the weights are frozen; qwen2.cu discards it).
// ─────────────────────────────────────────────────────────────
void or_rms_norm_bwd(const bf16_t* dy, const bf16_t* x, const bf16_t* w,
                     const float* rms_saved, bf16_t* dx, float* dw, i64 rows, int D) {
    std::vector<double> dwacc(dw ? D : 0, 0.0);
#pragma omp parallel
    {
        std::vector<double> dwl(dw ? D : 0, 0.0);
#pragma omp for schedule(static)
        for (i64 r = 0; r < rows; r++) {
            float inv = rms_saved[r];
            double dot = 0.0;
            for (int i = 0; i < D; i++) {
                float dyi = bf2f(dy[r * D + i]), xi = bf2f(x[r * D + i]), wi = bf2f(w[i]);
                float xh = xi * inv;
                dot += (double)(dyi * wi * xh);
            }
            float corr = (float)dot / (float)D;
            for (int i = 0; i < D; i++) {
                float dyi = bf2f(dy[r * D + i]), xi = bf2f(x[r * D + i]), wi = bf2f(w[i]);
                float xh = xi * inv;
                dx[r * D + i] = f2bf(inv * (wi * dyi - xh * corr));
                if (dw) dwl[i] += (double)(dyi * xh);
            }
        }
        if (dw) {
#pragma omp critical
            for (int i = 0; i < D; i++) dwacc[i] += dwl[i];
        }
    }
    if (dw)
        for (int i = 0; i < D; i++) dw[i] += (float)dwacc[i];
}

// ─────────────────────────────────────────────────────────────
//  RoPE — ops.cu:176-204.  Interleaved pairs (2i, 2i+1) of each head,
//  freq = theta^(-2i/hd) (float powf), angle = t*freq (float), inverse
//  rotates by -angle.  x is [B, T, H, hd] (row = b*T + t).
// ─────────────────────────────────────────────────────────────
void or_rope(bf16_t* x, int B, int T, int H, int hd, float theta, int inverse) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; b++)
        for (int t = 0; t < T; t++)
            for (int h = 0; h < H; h++) {
                i64 idx = ((i64)b * T * H + (i64)t * H + h) * hd;
                for (int i = 0; i < hd / 2; i++) {
                    float freq = powf(theta, -2.f * (float)i / (float)hd);
                    float angle = (float)t * freq;
                    if (inverse) angle = -angle;
                    float cs = (float)std::cos((double)angle), sn = (float)std::sin((double)angle);
                    float x0 = bf2f(x[idx + 2 * i]), x1 = bf2f(x[idx + 2 * i + 1]);
                    x[idx + 2 * i] = f2bf(x0 * cs - x1 * sn);
                    x[idx + 2 * i + 1] = f2bf(x0 * sn + x1 * cs);
                }
            }
}

// ─────────────────────────────────────────────────────────────
//  SDPA forward — sdpa_fwd_batched, ops.cu:578-681 (the sm>=80 path).
//  All GEMMs in FP32 on BF16-upcast operands; S = scale*Q.K^T;
//  causal softmax (ops.cu:352-396: max, expf(s-mx), multiply by 1/sum);
//  P saved to attn_w [B*Hq, T, T] (zeros above the diagonal);
//  O = P.V rounded to BF16 into out [BT, Hq*hd].  kv head = hq/(Hq/Hkv).
// ─────────────────────────────────────────────────────────────
}  // extern "C"

template <typename Acc>
static void sdpa_fwd_t(const bf16_t* Q, const bf16_t* K, const bf16_t* V, bf16_t* out,
                 float* attn_w, int B, int T, int Hq, int Hkv, int hd) {
    float scale = 1.f / sqrtf((float)hd);
    int grp = Hq / Hkv;
#pragma omp parallel for collapse(2) schedule(dynamic)
    for (int b = 0; b < B; b++)
        for (int hq = 0; hq < Hq; hq++) {
            int hkv = hq / grp;
            std::vector<float> s(T);
            float* P = attn_w + ((i64)b * Hq + hq) * T * T;
            for (int tq = 0; tq < T; tq++) {
                const bf16_t* q = Q + ((i64)(b * T + tq) * Hq + hq) * hd;
                for (int tk = 0; tk <= tq; tk++) {
                    const bf16_t* k = K + ((i64)(b * T + tk) * Hkv + hkv) * hd;
                    Acc d = 0;
                    for (int i = 0; i < hd; i++) d += (Acc)bf2f(q[i]) * (Acc)bf2f(k[i]);
                    s[tk] = scale * (float)d;
                }
                float mx = -3.402823466e38f;
                for (int tk = 0; tk <= tq; tk++) mx = std::max(mx, s[tk]);
                Acc sum = 0;
                for (int tk = 0; tk <= tq; tk++) {
                    s[tk] = expf(s[tk] - mx);
                    sum += s[tk];
                }
                float inv = 1.f / (float)sum;
                float* prow = P + (i64)tq * T;
                for (int tk = 0; tk < T; tk++) prow[tk] = (tk <= tq) ? s[tk] * inv : 0.f;
                bf16_t* o = out + ((i64)(b * T + tq) * Hq + hq) * hd;
                for (int i = 0; i < hd; i++) {
                    Acc acc = 0;
                    for (int tk = 0; tk <= tq; tk++)
                        acc += (Acc)prow[tk] * (Acc)bf2f(V[((i64)(b * T + tk) * Hkv + hkv) * hd + i]);
                    o[i] = f2bf((float)acc);
                }
            }
        }
}

// ─────────────────────────────────────────────────────────────
//  SDPA backward — sdpa_bwd_batched, ops.cu:707-870, softmax bwd
//  ops.cu:405-435, GQA contraction ops.cu:539-555.  dQ/dK/dV are
//  OVERWRITTEN (the batched path writes, it does not accumulate).
//  dV = sum_group P^T dO ; dP = dO V^T ; dS = P*(dP - sum_j P dP) ;
//  dQ = dS K / sqrt(hd) ; dK = sum_group dS^T Q / sqrt(hd).
// ─────────────────────────────────────────────────────────────
template <typename Acc>
static void sdpa_bwd_t(const bf16_t* dout, const bf16_t* Q, const bf16_t* K, const bf16_t* V,
                 const float* attn_w, bf16_t* dQ, bf16_t* dK, bf16_t* dV,
                 int B, int T, int Hq, int Hkv, int hd) {
    float rs = 1.f / sqrtf((float)hd);
    int grp = Hq / Hkv;
    i64 nkv = (i64)B * T * Hkv * hd;
    std::vector<double> dKacc(nkv, 0.0), dVacc(nkv, 0.0);
    auto qi = [&](int b, int t, int h) { return ((i64)(b * T + t) * Hq + h) * hd; };
    auto ki = [&](int b, int t, int h) { return ((i64)(b * T + t) * Hkv + h) * hd; };
    for (int b = 0; b < B; b++)
        for (int hkv = 0; hkv < Hkv; hkv++) {
            // per query head in the group: compute dS, dQ; accumulate dK, dV in Acc
            std::vector<std::vector<Acc>> dKh(grp), dVh(grp);
#pragma omp parallel for schedule(dynamic)
            for (int g = 0; g < grp; g++) {
                int hq = hkv * grp + g;
                const float* P = attn_w + ((i64)b * Hq + hq) * T * T;
                std::vector<Acc>& dKl = dKh[g];
                std::vector<Acc>& dVl = dVh[g];
                dKl.assign((size_t)T * hd, (Acc)0);
                dVl.assign((size_t)T * hd, (Acc)0);
                std::vector<float> dP(T), dS(T);
                for (int tq = 0; tq < T; tq++) {
                    const bf16_t* dO = dout + qi(b, tq, hq);
                    const float* prow = P + (i64)tq * T;
                    for (int tk = 0; tk <= tq; tk++) {
                        const bf16_t* v = V + ki(b, tk, hkv);
                        Acc d = 0;
                        for (int i = 0; i < hd; i++) d += (Acc)bf2f(dO[i]) * (Acc)bf2f(v[i]);
                        dP[tk] = (float)d;
                    }
                    Acc dot = 0;
                    for (int tk = 0; tk <= tq; tk++) dot += (Acc)prow[tk] * (Acc)dP[tk];
                    for (int tk = 0; tk < T; tk++)
                        dS[tk] = (tk <= tq) ? prow[tk] * (dP[tk] - (float)dot) : 0.f;
                    for (int i = 0; i < hd; i++) {
                        Acc acc = 0;
                        for (int tk = 0; tk <= tq; tk++)
                            acc += (Acc)dS[tk] * (Acc)bf2f(K[ki(b, tk, hkv) + i]);
                        dQ[qi(b, tq, hq) + i] = f2bf(rs * (float)acc);
                    }
                    float qv[1024];
                    for (int i = 0; i < hd; i++) qv[i] = bf2f(Q[qi(b, tq, hq) + i]);
                    for (int tk = 0; tk <= tq; tk++) {
                        float p = prow[tk], ds = dS[tk];
                        if (p == 0.f && ds == 0.f) continue;
                        for (int i = 0; i < hd; i++) {
                            dVl[(size_t)tk * hd + i] += (Acc)p * (Acc)bf2f(dO[i]);
                            dKl[(size_t)tk * hd + i] += (Acc)ds * (Acc)qv[i];
                        }
                    }
                }
            }
            for (int tk = 0; tk < T; tk++)
                for (int i = 0; i < hd; i++) {
                    Acc sv = 0, sk = 0;
                    for (int g = 0; g < grp; g++) {
                        sv += (Acc)(float)dVh[g][(size_t)tk * hd + i];
                        sk += (Acc)(rs * (float)dKh[g][(size_t)tk * hd + i]);
                    }
                    dVacc[ki(b, tk, hkv) + i] = sv;
                    dKacc[ki(b, tk, hkv) + i] = sk;
                }
        }
    for (i64 i = 0; i < nkv; i++) {
        dV[i] = f2bf((float)dVacc[i]);
        dK[i] = f2bf((float)dKacc[i]);
    }
}

extern "C" {

void or_sdpa_fwd(const bf16_t* Q, const bf16_t* K, const bf16_t* V, bf16_t* out,
                 float* attn_w, int B, int T, int Hq, int Hkv, int hd) {
    if (g_accum == 1) sdpa_fwd_t<float>(Q, K, V, out, attn_w, B, T, Hq, Hkv, hd);
    else sdpa_fwd_t<double>(Q, K, V, out, attn_w, B, T, Hq, Hkv, hd);
}
void or_sdpa_bwd(const bf16_t* dout, const bf16_t* Q, const bf16_t* K, const bf16_t* V,
                 const float* attn_w, bf16_t* dQ, bf16_t* dK, bf16_t* dV,
                 int B, int T, int Hq, int Hkv, int hd) {
    if (g_accum == 1) sdpa_bwd_t<float>(dout, Q, K, V, attn_w, dQ, dK, dV, B, T, Hq, Hkv, hd);
    else sdpa_bwd_t<double>(dout, Q, K, V, attn_w, dQ, dK, dV, B, T, Hq, Hkv, hd);
}

// ─────────────────────────────────────────────────────────────
//  SiLU-gated activation — ops.cu:913-952.
// ─────────────────────────────────────────────────────────────
void or_silu_mul_fwd(const bf16_t* gate, const bf16_t* up, bf16_t* out, i64 n) {
#pragma omp parallel for schedule(static)
    for (i64 i = 0; i < n; i++) {
        float g = bf2f(gate[i]), u = bf2f(up[i]);
        float s = g / (1.f + expf(-g));
        out[i] = f2bf(s * u);
    }
}
void or_silu_mul_bwd(const bf16_t* dout, const bf16_t* gate, const bf16_t* up,
                     bf16_t* dgate, bf16_t* dup, i64 n) {
#pragma omp parallel for schedule(static)
    for (i64 i = 0; i < n; i++) {
        float g = bf2f(gate[i]), u = bf2f(up[i]), d = bf2f(dout[i]);
        float sig = 1.f / (1.f + expf(-g));
        float s = g * sig;
        float ds = sig * (1.f + g * (1.f - sig));
        dgate[i] = f2bf(d * u * ds);
        dup[i] = f2bf(d * s);
    }
}

// ─────────────────────────────────────────────────────────────
//  Cross entropy — ops.cu:958-1020.  Per row: log_sum = log(sum exp(L-mx))+mx;
//  loss = -(L[tgt] - log_sum) with L[tgt] := 0 when tgt < 0 (so a masked
//  token still reports log_sum); dL = bf16((exp(L - log_sum) - [i==tgt]) / N)
//  with N = number of rows (gridDim.x), masked rows included.
// ─────────────────────────────────────────────────────────────
void or_cross_entropy(const bf16_t* logits, const int32_t* targets, float* loss,
                      bf16_t* dlogits, i64 N, i64 V) {
    float inv_N = 1.f / (float)N;
#pragma omp parallel for schedule(dynamic)
    for (i64 n = 0; n < N; n++) {
        const bf16_t* L = logits + n * V;
        int tgt = targets[n];
        float mx = -3.402823466e38f;
        for (i64 i = 0; i < V; i++) mx = std::max(mx, bf2f(L[i]));
        double sum = 0.0;
        for (i64 i = 0; i < V; i++) sum += (double)expf(bf2f(L[i]) - mx);
        float log_sum = logf((float)sum) + mx;
        float tl = (tgt >= 0) ? bf2f(L[tgt]) : 0.f;
        loss[n] = -(tl - log_sum);
        if (dlogits)
            for (i64 i = 0; i < V; i++) {
                float p = expf(bf2f(L[i]) - log_sum);
                float d = p - (float)(i == tgt);
                dlogits[n * V + i] = f2bf(d * inv_N);
            }
    }
}

// ─────────────────────────────────────────────────────────────
//  Embedding gather (ops.cu:1026-1051), bias add (1062-1081),
//  residual add (1087-1099), LoRA add (1101-1113), casts (1119-1133).
// ─────────────────────────────────────────────────────────────
void or_embed_fwd(const bf16_t* table, const int32_t* tokens, bf16_t* out, i64 BT, int D) {
    for (i64 t = 0; t < BT; t++) std::memcpy(out + t * D, table + (i64)tokens[t] * D, D * 2);
}
void or_add_bias(bf16_t* out, const bf16_t* bias, i64 BT, int D) {
    for (i64 t = 0; t < BT; t++)
        for (int i = 0; i < D; i++) out[t * D + i] = f2bf(bf2f(out[t * D + i]) + bf2f(bias[i]));
}
void or_add_inplace(bf16_t* out, const bf16_t* delta, i64 n) {
    for (i64 i = 0; i < n; i++) out[i] = f2bf(bf2f(out[i]) + bf2f(delta[i]));
}
void or_lora_add(bf16_t* out, const bf16_t* delta, float scale, i64 n) {
    for (i64 i = 0; i < n; i++) out[i] = f2bf(bf2f(out[i]) + scale * bf2f(delta[i]));
}

// ─────────────────────────────────────────────────────────────
//  AdamW — ops.cu:1139-1169 (k_adamw), driven by adamw.cu:9-38.
//  m = b1 m + (1-b1) g ; v = b2 v + (1-b2) g^2 ; bias-corrected with
//  powf(b, step); p = p - lr*(mhat/(sqrt(vhat)+eps) + wd*p); shadow = bf16(p).
// ─────────────────────────────────────────────────────────────
void or_adamw_step(float* master, bf16_t* working, float* m, float* v, const float* grad,
                   i64 n, float lr, float b1, float b2, float eps, float wd, int step) {
    float bc1 = 1.f - powf(b1, (float)step);
    float bc2 = 1.f - powf(b2, (float)step);
    for (i64 i = 0; i < n; i++) {
        float g = grad[i];
        float mi = b1 * m[i] + (1.f - b1) * g;
        float vi = b2 * v[i] + (1.f - b2) * g * g;
        m[i] = mi;
        v[i] = vi;
        float mhat = mi / bc1, vhat = vi / bc2;
        float p = master[i] - lr * (mhat / (sqrtf(vhat) + eps) + wd * master[i]);
        master[i] = p;
        if (working) working[i] = f2bf(p);
    }
}

// sum of squares — ops.cu:1175-1193 (evaluated in FP64 here)
double or_sum_sq(const float* g, i64 n) {
    double s = 0.0;
    for (i64 i = 0; i < n; i++) s += (double)g[i] * g[i];
    return s;
}

// ─────────────────────────────────────────────────────────────
//  LoRA A init — adapter_model.cu:15-39, seed 0x1234 (adapter_model.cu:53-54).
//  Integer hash of (seed, i); u in [-1,1]; A = u*sqrt(1/in).  Written with
//  IEEE division and sqrt (the reference's fast-math division may differ by
//  at most a couple of F32 ulps before BF16 rounding).
// ─────────────────────────────────────────────────────────────
void or_kaiming_init(bf16_t* A_bf16, float* A_f32, int in_dim, int rank, uint32_t seed) {
    i64 n = (i64)in_dim * rank;
    for (i64 i = 0; i < n; i++) {
        uint32_t r = seed ^ ((uint32_t)i * 2654435761u);
        r = r ^ (r >> 16);
        r *= 0x45d9f3bu;
        r ^= (r >> 16);
        float u = (float)(r & 0xFFFFFFu) / (float)0xFFFFFF * 2.f - 1.f;
        float bound = sqrtf(1.f / (float)in_dim);
        if (A_bf16) A_bf16[i] = f2bf(u * bound);
        if (A_f32) A_f32[i] = u * bound;
    }
}

// ─────────────────────────────────────────────────────────────
//  Assistant-span masking — adapt_trainer.cu:145-182 (in place on targets).
// ─────────────────────────────────────────────────────────────
void or_mask_targets(const int32_t* input_ids, int32_t* target_ids, int B, int T) {
    for (int b = 0; b < B; ++b) {
        bool in_asst = false;
        int off = b * T;
        for (int t = 0; t < T; ++t) {
            int idx = off + t, tok = input_ids[idx];
            if (tok == 151644) in_asst = (t + 1 < T && input_ids[off + t + 1] == 77091);
            bool mask = !in_asst;
            if (tok == 151644 || tok == 77091) mask = true;
            if (tok == 151645) {
                in_asst = false;
                mask = false;
            }
            if (mask) target_ids[idx] = -1;
        }
    }
}

// CosineSchedule::lr_at — cosine_schedule.hpp:18-29
float or_cosine_lr(float base_lr, i64 warmup, i64 total, float floor_frac, i64 step) {
    if (step < warmup) return base_lr * (float)(step + 1) / (float)warmup;
    float progress = (float)(step - warmup) / (float)(total - warmup);
    progress = std::min(progress, 1.f);
    float cos_val = 0.5f * (1.f + std::cos((float)M_PI * progress));
    float floor = base_lr * floor_frac;
    return floor + (base_lr - floor) * cos_val;
}

// Dataset::next_batch — dataset.cpp:56-71 (windows of T, stride T, wrap-around)
void or_next_batch(const uint32_t* tokens, i64 n_tokens, i64* pos, int B, int T,
                   int32_t* inputs, int32_t* targets) {
    for (int b = 0; b < B; b++) {
        for (int t = 0; t < T; t++) {
            i64 idx = (*pos + t) % n_tokens;
            inputs[b * T + t] = (int32_t)tokens[idx];
            targets[b * T + t] = (int32_t)tokens[(idx + 1) % n_tokens];
        }
        *pos = (*pos + T) % n_tokens;
    }
}

// ─────────────────────────────────────────────────────────────
//  Centroid accumulate — centroid_accumulator.cpp:54-69 applied to
//  correctly typed F32 h and g (the intended math C += h_t*||g_t||,
//  W += ||g_t||), evaluated in FP64.  n (optional) receives ||g_t||.
// ─────────────────────────────────────────────────────────────
void or_centroid_accumulate(const float* h, const float* g, i64 BT, int D, double* acc,
                            double* acc_w, double* n_out) {
    int nt = omp_get_max_threads();
    std::vector<std::vector<double>> part(nt, std::vector<double>(D + 1, 0.0));
#pragma omp parallel
    {
        std::vector<double>& p = part[omp_get_thread_num()];
#pragma omp for schedule(static)
        for (i64 t = 0; t < BT; t++) {
            double ss = 0.0;
            for (int d = 0; d < D; d++) ss += (double)g[t * D + d] * g[t * D + d];
            double gn = std::sqrt(ss);
            if (n_out) n_out[t] = gn;
            for (int d = 0; d < D; d++) p[d] += (double)h[t * D + d] * gn;
            p[D] += gn;
        }
    }
    for (int k = 0; k < nt; k++) {
        for (int d = 0; d < D; d++) acc[d] += part[k][d];
        *acc_w += part[k][D];
    }
}

// Same, with the per-token norms given directly (c5 stress inputs).
void or_centroid_accumulate_n(const float* h, const float* n, i64 BT, int D, double* acc,
                              double* acc_w) {
    int nt = omp_get_max_threads();
    std::vector<std::vector<double>> part(nt, std::vector<double>(D + 1, 0.0));
#pragma omp parallel
    {
        std::vector<double>& p = part[omp_get_thread_num()];
#pragma omp for schedule(static)
        for (i64 t = 0; t < BT; t++) {
            double gn = n[t];
            for (int d = 0; d < D; d++) p[d] += (double)h[t * D + d] * gn;
            p[D] += gn;
        }
    }
    for (int k = 0; k < nt; k++) {
        for (int d = 0; d < D; d++) acc[d] += part[k][d];
        *acc_w += part[k][D];
    }
}

// ─────────────────────────────────────────────────────────────
//  k-means merge, reference mode — centroid_accumulator.cpp:114-157.
//  Init center i = snapshot[(i*N)/k]; <= 50 Lloyd iterations; assignment by
//  squared L2 summed sequentially over d in F32 (no contraction), strict '<'
//  (lowest index wins ties); stop when no assignment changes; update zeroes
//  every center and averages its members (sequential F32 sums over n), so an
//  empty cluster becomes the zero vector.  Returns k actually used.
// ─────────────────────────────────────────────────────────────
static float sqdist_f32(const float* a, const float* b, int D) {
    float d = 0.f;
    for (int i = 0; i < D; i++) {
        float v = a[i] - b[i];
        d += v * v;
    }
    return d;
}

int or_kmeans_ref(const float* snaps, int N, int D, int k, float* centers_out,
                  int* assign_out, int* iters_out) {
    k = std::min(k, N);
    std::vector<float> C((size_t)k * D);
    for (int i = 0; i < k; i++)
        std::memcpy(&C[(size_t)i * D], snaps + (size_t)((i64)i * N / k) * D, D * 4);
    std::vector<int> asg(N, 0);
    int it = 0;
    for (; it < 50; it++) {
        bool changed = false;
        for (int n = 0; n < N; n++) {
            float best = 1e38f;
            int bk = 0;
            for (int c = 0; c < k; c++) {
                float d = sqdist_f32(snaps + (size_t)n * D, &C[(size_t)c * D], D);
                if (d < best) {
                    best = d;
                    bk = c;
                }
            }
            if (asg[n] != bk) {
                asg[n] = bk;
                changed = true;
            }
        }
        if (!changed) break;
        std::vector<int> cnt(k, 0);
        std::fill(C.begin(), C.end(), 0.f);
        for (int n = 0; n < N; n++) {
            int c = asg[n];
            for (int i = 0; i < D; i++) C[(size_t)c * D + i] += snaps[(size_t)n * D + i];
            cnt[c]++;
        }
        for (int c = 0; c < k; c++)
            if (cnt[c] > 0)
                for (int i = 0; i < D; i++) C[(size_t)c * D + i] /= (float)cnt[c];
    }
    std::memcpy(centers_out, C.data(), (size_t)k * D * 4);
    if (assign_out) std::memcpy(assign_out, asg.data(), (size_t)N * 4);
    if (iters_out) *iters_out = it;
    return k;
}

// ─────────────────────────────────────────────────────────────
//  k-means, stress mode (c5).  Not in the reference (which has only the
//  mode above); defined once here and matched bit-exactly by the device:
//   * RNG: splitmix64(seed), u = (x >> 11) * 2^-53.
//   * k-means++: first center = floor(u*N); each next center is drawn with
//     probability D2(n) / sum D2, D2(n) = min over chosen centers of the F32
//     sequential squared distance; the draw walks the running FP64 sum of
//     D2 in index order and takes the first n with running sum > u*total
//     (falls back to the last n with D2 > 0).
//   * exactly `iters` Lloyd iterations (assign: strict '<'; update: F32
//     sequential sums in n order divided by the count; an empty cluster
//     keeps its previous center).
//   * ranking: mass_c = sum of weights of member snapshots (FP64, n order);
//     clusters ordered by descending mass, ties by lower index.
//  Outputs centers in ranked order, assignments remapped to ranks, masses.
// ─────────────────────────────────────────────────────────────
static inline uint64_t splitmix64(uint64_t& s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static inline double u01(uint64_t& s) { return (double)(splitmix64(s) >> 11) * (1.0 / 9007199254740992.0); }

int or_kmeans_pp(const float* snaps, const float* weights, int N, int D, int k, int iters,
                 uint64_t seed, float* centers_out, int* assign_out, double* mass_out,
                 int* seeds_out) {
    k = std::min(k, N);
    uint64_t s = seed;
    std::vector<int> chosen;
    std::vector<float> d2(N, 3.402823466e38f);
    int first = (int)(u01(s) * N);
    if (first >= N) first = N - 1;
    chosen.push_back(first);
    while ((int)chosen.size() < k) {
        const float* c = snaps + (size_t)chosen.back() * D;
        for (int n = 0; n < N; n++) {
            float d = sqdist_f32(snaps + (size_t)n * D, c, D);
            if (d < d2[n]) d2[n] = d;
        }
        double total = 0.0;
        for (int n = 0; n < N; n++) total += (double)d2[n];
        double target = u01(s) * total;
        int pick = -1, last_pos = -1;
        double run = 0.0;
        for (int n = 0; n < N; n++) {
            run += (double)d2[n];
            if (d2[n] > 0.f) last_pos = n;
            if (pick < 0 && run > target && d2[n] > 0.f) pick = n;
        }
        if (pick < 0) pick = (last_pos >= 0) ? last_pos : (int)chosen.size() % N;
        chosen.push_back(pick);
    }
    std::vector<float> C((size_t)k * D);
    for (int c = 0; c < k; c++) std::memcpy(&C[(size_t)c * D], snaps + (size_t)chosen[c] * D, D * 4);
    std::vector<int> asg(N, 0);
    for (int it = 0; it < iters; it++) {
        for (int n = 0; n < N; n++) {
            float best = 1e38f;
            int bk = 0;
            for (int c = 0; c < k; c++) {
                float d = sqdist_f32(snaps + (size_t)n * D, &C[(size_t)c * D], D);
                if (d < best) {
                    best = d;
                    bk = c;
                }
            }
            asg[n] = bk;
        }
        std::vector<float> S((size_t)k * D, 0.f);
        std::vector<int> cnt(k, 0);
        for (int n = 0; n < N; n++) {
            int c = asg[n];
            for (int i = 0; i < D; i++) S[(size_t)c * D + i] += snaps[(size_t)n * D + i];
            cnt[c]++;
        }
        for (int c = 0; c < k; c++)
            if (cnt[c] > 0)
                for (int i = 0; i < D; i++) C[(size_t)c * D + i] = S[(size_t)c * D + i] / (float)cnt[c];
    }
    // final assignment against the final centers
    for (int n = 0; n < N; n++) {
        float best = 1e38f;
        int bk = 0;
        for (int c = 0; c < k; c++) {
            float d = sqdist_f32(snaps + (size_t)n * D, &C[(size_t)c * D], D);
            if (d < best) {
                best = d;
                bk = c;
            }
        }
        asg[n] = bk;
    }
    std::vector<double> mass(k, 0.0);
    for (int n = 0; n < N; n++) mass[asg[n]] += (double)weights[n];
    std::vector<int> order(k);
    for (int c = 0; c < k; c++) order[c] = c;
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) { return mass[a] > mass[b]; });
    std::vector<int> rank_of(k);
    for (int r = 0; r < k; r++) rank_of[order[r]] = r;
    for (int r = 0; r < k; r++) {
        std::memcpy(centers_out + (size_t)r * D, &C[(size_t)order[r] * D], D * 4);
        if (mass_out) mass_out[r] = mass[order[r]];
    }
    if (assign_out)
        for (int n = 0; n < N; n++) assign_out[n] = rank_of[asg[n]];
    if (seeds_out)
        for (int c = 0; c < k; c++) seeds_out[c] = chosen[c];
    return k;
}

}  // extern "C"

// ═════════════════════════════════════════════════════════════
//  Model-level oracle: one AdaptTrainer step (adapt_trainer.cu:130-277)
//  over Qwen2Base::forward/backward (qwen2.cu:47-308) with the adapter
//  (adapter_model.cu:96-220), following the reference op by op.
//
//  Extension (the reference always trains q,k,v,o and has no MLP LoRA):
//  inject_mask selects targets {q,k,v,o,gate,up,down} = bits 0..6.
//  gate/up: LoRA on x_normed2 added to gate_out/up_out before SiLU; grad_x
//  accumulates into dx_normed2 after the base gate/up input-gradients.
//  down: LoRA on act_out added to ffn_out before the residual add; grad_x
//  accumulates into dact after the base down input-gradient, before
//  silu_mul_bwd.  Absent targets are skipped in fwd, bwd, grad-norm, AdamW.
// ═════════════════════════════════════════════════════════════

namespace {

enum { TQ = 0, TK, TV, TO, TG, TU, TD, NTGT };

struct ModelCfg {
    int vocab, hidden, layers, n_q, n_kv, head_dim, inter;
    float rms_eps, rope_theta;
    int tie;
};
struct AdaptCfg {
    int rank;
    float alpha;
    int inject_mask;
    float lr, grad_clip;
    i64 warmup, total_steps;
    float b1, b2, eps, wd;
};
struct StepOut {
    float loss, lr, gnorm, gnorm_raw;
    int valid_tokens, step;
};

typedef std::vector<bf16_t> VB;
typedef std::vector<float> VF;

struct Pair {
    bool on = false;
    int in = 0, out = 0, r = 0;
    VF A32, B32, mA, vA, mB, vB, gA, gB;
    VB A16, B16;
};

struct LayerW {
    VB in_norm, q_w, q_b, k_w, k_b, v_w, v_b, o_w, post_norm, gate_w, up_w, down_w;
    Pair pr[NTGT];
};

struct Cache {
    VB pre_attn_res, x_normed, Q, K, V, attn_out, h_mid, pre_ffn_res, x_normed2, gate, up, act;
    VF in_rms, post_rms, attn_w;
};

struct Model {
    ModelCfg c;
    AdaptCfg a;
    VB embed, final_norm, lm_head;
    std::vector<LayerW> L;
    i64 step_count = 0;
    std::vector<double> cacc;
    double cacc_w = 0.0;
    std::map<std::string, VB> taps_b;
    std::map<std::string, VF> taps_f;
    bool keep_taps = false;
};

void gemm_b(int tA, int tB, int M, int N, int K, float al, const bf16_t* A, int lda,
            const bf16_t* B, int ldb, float be, bf16_t* C, int ldc) {
    or_gemm_bf16(tA, tB, M, N, K, al, A, lda, B, ldb, be, C, ldc);
}

// proj_fwd — qwen2.cu:21-30 ; y[BT,out] = x[BT,in] W^T
void proj_fwd(const VB& W, const bf16_t* x, bf16_t* y, int BT, int in, int out) {
    gemm_b(1, 0, out, BT, in, 1.f, W.data(), in, x, in, 0.f, y, out);
}
// proj_bwd_x — qwen2.cu:32-41 ; dx[BT,in] = bf16(dy W + beta dx)
void proj_bwd_x(const bf16_t* W, const bf16_t* dy, bf16_t* dx, int BT, int out, int in, float beta) {
    gemm_b(0, 0, in, BT, out, 1.f, W, in, dy, out, beta, dx, in);
}

// apply_lora_fwd — adapter_model.cu:96-129
void lora_fwd(const Model& m, const Pair& p, const bf16_t* x, bf16_t* out, int BT) {
    VB h((size_t)BT * p.r), delta((size_t)BT * p.out);
    gemm_b(1, 0, p.r, BT, p.in, 1.f, p.A16.data(), p.in, x, p.in, 0.f, h.data(), p.r);
    gemm_b(1, 0, p.out, BT, p.r, 1.f, p.B16.data(), p.r, h.data(), p.r, 0.f, delta.data(), p.out);
    float scale = m.a.alpha / (float)m.a.rank;
    or_lora_add(out, delta.data(), scale, (i64)BT * p.out);
}

// apply_lora_bwd — adapter_model.cu:131-220
void lora_bwd(const Model& m, Pair& p, const bf16_t* x, const bf16_t* go, bf16_t* gx, int BT) {
    float scale = m.a.alpha / (float)m.a.rank;
    VB h((size_t)BT * p.r);
    gemm_b(1, 0, p.r, BT, p.in, 1.f, p.A16.data(), p.in, x, p.in, 0.f, h.data(), p.r);
    VF h32((size_t)BT * p.r), go32((size_t)BT * p.out), x32((size_t)BT * p.in);
    or_f32_from_bf16(h.data(), h32.data(), (i64)h.size());
    or_f32_from_bf16(go, go32.data(), (i64)go32.size());
    or_f32_from_bf16(x, x32.data(), (i64)x32.size());
    or_gemm_f32(0, 1, p.r, p.out, BT, scale, h32.data(), p.r, go32.data(), p.out, 1.f, p.gB.data(), p.r);
    VB dh((size_t)BT * p.r);
    gemm_b(0, 0, p.r, BT, p.out, 1.f, p.B16.data(), p.r, go, p.out, 0.f, dh.data(), p.r);
    VF dh32((size_t)BT * p.r);
    or_f32_from_bf16(dh.data(), dh32.data(), (i64)dh.size());
    or_gemm_f32(0, 1, p.in, p.r, BT, scale, x32.data(), p.in, dh32.data(), p.r, 1.f, p.gA.data(), p.in);
    gemm_b(0, 0, p.in, BT, p.r, scale, p.A16.data(), p.in, dh.data(), p.r, 1.f, gx, p.in);
}

void make_pair(Pair& p, bool on, int in, int out, int r) {
    p.on = on;
    p.in = in;
    p.out = out;
    p.r = r;
    if (!on) return;
    size_t nA = (size_t)r * in, nB = (size_t)out * r;
    p.A16.assign(nA, 0);
    p.A32.assign(nA, 0.f);
    or_kaiming_init(p.A16.data(), p.A32.data(), in, r, 0x1234u);
    p.B16.assign(nB, 0);
    p.B32.assign(nB, 0.f);
    p.mA.assign(nA, 0.f);
    p.vA.assign(nA, 0.f);
    p.mB.assign(nB, 0.f);
    p.vB.assign(nB, 0.f);
    p.gA.assign(nA, 0.f);
    p.gB.assign(nB, 0.f);
}

float step_model(Model& m, const int32_t* in_ids, const int32_t* tgt_in, int B, int T, StepOut* so,
                 float lr_override) {
    const ModelCfg& c = m.c;
    int BT = B * T, H = c.hidden, I = c.inter, Hq = c.n_q, Hkv = c.n_kv, hd = c.head_dim, V = c.vocab;
    int qd = Hq * hd, kvd = Hkv * hd;
    float eps = c.rms_eps;
    // 2. masking (adapt_trainer.cu:145-182)
    std::vector<int32_t> tgt(tgt_in, tgt_in + BT);
    or_mask_targets(in_ids, tgt.data(), B, T);
    // 3. zero_grad (adapter_model.cu:222-229)
    for (auto& lw : m.L)
        for (auto& p : lw.pr)
            if (p.on) {
                std::fill(p.gA.begin(), p.gA.end(), 0.f);
                std::fill(p.gB.begin(), p.gB.end(), 0.f);
            }
    // 4. forward (qwen2.cu:47-178)
    std::vector<Cache> cache(c.layers);
    VB residual((size_t)BT * H);
    or_embed_fwd(m.embed.data(), in_ids, residual.data(), BT, H);
    for (int l = 0; l < c.layers; l++) {
        LayerW& lw = m.L[l];
        Cache& lc = cache[l];
        lc.pre_attn_res = residual;
        lc.in_rms.assign(BT, 0.f);
        lc.x_normed.assign((size_t)BT * H, 0);
        or_rms_norm_fwd(residual.data(), lw.in_norm.data(), lc.x_normed.data(), lc.in_rms.data(), BT, H, eps);
        lc.Q.assign((size_t)BT * qd, 0);
        lc.K.assign((size_t)BT * kvd, 0);
        lc.V.assign((size_t)BT * kvd, 0);
        proj_fwd(lw.q_w, lc.x_normed.data(), lc.Q.data(), BT, H, qd);
        or_add_bias(lc.Q.data(), lw.q_b.data(), BT, qd);
        proj_fwd(lw.k_w, lc.x_normed.data(), lc.K.data(), BT, H, kvd);
        or_add_bias(lc.K.data(), lw.k_b.data(), BT, kvd);
        proj_fwd(lw.v_w, lc.x_normed.data(), lc.V.data(), BT, H, kvd);
        or_add_bias(lc.V.data(), lw.v_b.data(), BT, kvd);
        if (lw.pr[TQ].on) lora_fwd(m, lw.pr[TQ], lc.x_normed.data(), lc.Q.data(), BT);
        if (lw.pr[TK].on) lora_fwd(m, lw.pr[TK], lc.x_normed.data(), lc.K.data(), BT);
        if (lw.pr[TV].on) lora_fwd(m, lw.pr[TV], lc.x_normed.data(), lc.V.data(), BT);
        or_rope(lc.Q.data(), B, T, Hq, hd, c.rope_theta, 0);
        or_rope(lc.K.data(), B, T, Hkv, hd, c.rope_theta, 0);
        lc.attn_out.assign((size_t)BT * qd, 0);
        lc.attn_w.assign((size_t)B * Hq * T * T, 0.f);
        or_sdpa_fwd(lc.Q.data(), lc.K.data(), lc.V.data(), lc.attn_out.data(), lc.attn_w.data(), B, T, Hq, Hkv, hd);
        lc.h_mid.assign((size_t)BT * H, 0);
        proj_fwd(lw.o_w, lc.attn_out.data(), lc.h_mid.data(), BT, qd, H);
        if (lw.pr[TO].on) lora_fwd(m, lw.pr[TO], lc.attn_out.data(), lc.h_mid.data(), BT);
        or_add_inplace(residual.data(), lc.h_mid.data(), (i64)BT * H);
        lc.pre_ffn_res = residual;
        lc.post_rms.assign(BT, 0.f);
        lc.x_normed2.assign((size_t)BT * H, 0);
        or_rms_norm_fwd(residual.data(), lw.post_norm.data(), lc.x_normed2.data(), lc.post_rms.data(), BT, H, eps);
        lc.gate.assign((size_t)BT * I, 0);
        lc.up.assign((size_t)BT * I, 0);
        proj_fwd(lw.gate_w, lc.x_normed2.data(), lc.gate.data(), BT, H, I);
        proj_fwd(lw.up_w, lc.x_normed2.data(), lc.up.data(), BT, H, I);
        if (lw.pr[TG].on) lora_fwd(m, lw.pr[TG], lc.x_normed2.data(), lc.gate.data(), BT);
        if (lw.pr[TU].on) lora_fwd(m, lw.pr[TU], lc.x_normed2.data(), lc.up.data(), BT);
        lc.act.assign((size_t)BT * I, 0);
        or_silu_mul_fwd(lc.gate.data(), lc.up.data(), lc.act.data(), (i64)BT * I);
        VB ffn((size_t)BT * H);
        proj_fwd(lw.down_w, lc.act.data(), ffn.data(), BT, I, H);
        if (lw.pr[TD].on) lora_fwd(m, lw.pr[TD], lc.act.data(), ffn.data(), BT);
        or_add_inplace(residual.data(), ffn.data(), (i64)BT * H);
    }
    VB x_final = residual;
    VF final_rms(BT);
    VB xfn((size_t)BT * H);
    or_rms_norm_fwd(residual.data(), m.final_norm.data(), xfn.data(), final_rms.data(), BT, H, eps);
    const VB& lm = c.tie ? m.embed : m.lm_head;
    VB logits((size_t)BT * V);
    gemm_b(1, 0, V, BT, H, 1.f, lm.data(), H, xfn.data(), H, 0.f, logits.data(), V);
    // 6. loss (adapt_trainer.cu:201-205; ops.cu:958-1020)
    VF loss_tok(BT);
    VB dlogits((size_t)BT * V);
    or_cross_entropy(logits.data(), tgt.data(), loss_tok.data(), dlogits.data(), BT, V);
    logits.clear();
    logits.shrink_to_fit();
    // 7. backward (qwen2.cu:184-308)
    VB dres((size_t)BT * H, 0);
    proj_bwd_x(lm.data(), dlogits.data(), dres.data(), BT, V, H, 0.f);
    dlogits.clear();
    dlogits.shrink_to_fit();
    VB grad((size_t)BT * H);
    or_rms_norm_bwd(dres.data(), x_final.data(), m.final_norm.data(), final_rms.data(), grad.data(), nullptr, BT, H);
    if (m.keep_taps) m.taps_b["dres"] = dres;
    std::vector<VB> dx_attn_in(c.layers);
    for (int l = c.layers - 1; l >= 0; l--) {
        LayerW& lw = m.L[l];
        Cache& lc = cache[l];
        // FFN backward
        VB dact((size_t)BT * I);
        proj_bwd_x(lw.down_w.data(), grad.data(), dact.data(), BT, H, I, 0.f);
        if (lw.pr[TD].on) lora_bwd(m, lw.pr[TD], lc.act.data(), grad.data(), dact.data(), BT);
        VB dgate((size_t)BT * I), dup((size_t)BT * I);
        or_silu_mul_bwd(dact.data(), lc.gate.data(), lc.up.data(), dgate.data(), dup.data(), (i64)BT * I);
        VB dxn2((size_t)BT * H, 0);
        proj_bwd_x(lw.gate_w.data(), dgate.data(), dxn2.data(), BT, I, H, 0.f);
        proj_bwd_x(lw.up_w.data(), dup.data(), dxn2.data(), BT, I, H, 1.f);
        if (lw.pr[TG].on) lora_bwd(m, lw.pr[TG], lc.x_normed2.data(), dgate.data(), dxn2.data(), BT);
        if (lw.pr[TU].on) lora_bwd(m, lw.pr[TU], lc.x_normed2.data(), dup.data(), dxn2.data(), BT);
        VB dffn_in((size_t)BT * H);
        or_rms_norm_bwd(dxn2.data(), lc.pre_ffn_res.data(), lw.post_norm.data(), lc.post_rms.data(), dffn_in.data(), nullptr, BT, H);
        or_add_inplace(grad.data(), dffn_in.data(), (i64)BT * H);
        // attention backward
        VB dao((size_t)BT * qd);
        proj_bwd_x(lw.o_w.data(), grad.data(), dao.data(), BT, H, qd, 0.f);
        if (lw.pr[TO].on) lora_bwd(m, lw.pr[TO], lc.attn_out.data(), grad.data(), dao.data(), BT);
        VB dQ((size_t)BT * qd, 0), dK((size_t)BT * kvd, 0), dV((size_t)BT * kvd, 0);
        or_sdpa_bwd(dao.data(), lc.Q.data(), lc.K.data(), lc.V.data(), lc.attn_w.data(), dQ.data(), dK.data(), dV.data(), B, T, Hq, Hkv, hd);
        or_rope(dQ.data(), B, T, Hq, hd, c.rope_theta, 1);
        or_rope(dK.data(), B, T, Hkv, hd, c.rope_theta, 1);
        VB dxn((size_t)BT * H, 0);
        proj_bwd_x(lw.q_w.data(), dQ.data(), dxn.data(), BT, qd, H, 0.f);
        proj_bwd_x(lw.k_w.data(), dK.data(), dxn.data(), BT, kvd, H, 1.f);
        proj_bwd_x(lw.v_w.data(), dV.data(), dxn.data(), BT, kvd, H, 1.f);
        if (lw.pr[TQ].on) lora_bwd(m, lw.pr[TQ], lc.x_normed.data(), dQ.data(), dxn.data(), BT);
        if (lw.pr[TK].on) lora_bwd(m, lw.pr[TK], lc.x_normed.data(), dK.data(), dxn.data(), BT);
        if (lw.pr[TV].on) lora_bwd(m, lw.pr[TV], lc.x_normed.data(), dV.data(), dxn.data(), BT);
        dx_attn_in[l] = dxn;
        if (m.keep_taps) {
            std::string p = "l" + std::to_string(l) + ".";
            m.taps_b[p + "dQ"] = dQ;
            m.taps_b[p + "dK"] = dK;
            m.taps_b[p + "dV"] = dV;
            m.taps_b[p + "dattn_out"] = dao;
            m.taps_b[p + "dx_normed"] = dxn;
            m.taps_b[p + "dx_normed2"] = dxn2;
            m.taps_b[p + "x_normed"] = lc.x_normed;
            m.taps_b[p + "attn_out"] = lc.attn_out;
            m.taps_b[p + "Q"] = lc.Q;
            m.taps_b[p + "act"] = lc.act;
            m.taps_b[p + "dgate"] = dgate;
        }
        VB dattn_in((size_t)BT * H);
        or_rms_norm_bwd(dxn.data(), lc.pre_attn_res.data(), lw.in_norm.data(), lc.in_rms.data(), dattn_in.data(), nullptr, BT, H);
        or_add_inplace(grad.data(), dattn_in.data(), (i64)BT * H);
    }
    if (m.keep_taps) {
        m.taps_b["dembed"] = grad;
        m.taps_f["loss_tok"] = loss_tok;
    }
    // centroid feed (adapt_trainer.cu:210-232), intended math in FP64
    for (int l = 0; l < c.layers; l++) {
        VF h32((size_t)BT * H), g32((size_t)BT * H);
        or_f32_from_bf16(cache[l].x_normed.data(), h32.data(), (i64)h32.size());
        or_f32_from_bf16(dx_attn_in[l].data(), g32.data(), (i64)g32.size());
        or_centroid_accumulate(h32.data(), g32.data(), BT, H, m.cacc.data(), &m.cacc_w, nullptr);
    }
    // 8. stats (adapt_trainer.cu:237-246)
    float mean_loss = 0.f;
    int valid = 0;
    for (float lv : loss_tok)
        if (lv > 1e-9f) {
            mean_loss += lv;
            valid++;
        }
    if (valid > 0) mean_loss /= (float)valid;
    // grad norm + clip (adapt_trainer.cu:32-70, 248-250)
    double ss = 0.0;
    for (auto& lw : m.L)
        for (auto& p : lw.pr)
            if (p.on) {
                ss += or_sum_sq(p.gA.data(), (i64)p.gA.size());
                ss += or_sum_sq(p.gB.data(), (i64)p.gB.size());
            }
    float gnorm = (float)std::sqrt(ss);
    float gnorm_raw = gnorm;
    if (gnorm > m.a.grad_clip) {
        float sc = m.a.grad_clip / (gnorm + 1e-6f);
        for (auto& lw : m.L)
            for (auto& p : lw.pr)
                if (p.on) {
                    for (auto& g : p.gA) g *= sc;
                    for (auto& g : p.gB) g *= sc;
                }
    }
    gnorm = std::min(gnorm, m.a.grad_clip);
    float lr = (lr_override > 0.f)
                   ? lr_override
                   : or_cosine_lr(m.a.lr, m.a.warmup, m.a.total_steps, 0.1f, m.step_count);
    int t = (int)m.step_count + 1;
    for (auto& lw : m.L)
        for (auto& p : lw.pr)
            if (p.on) {
                or_adamw_step(p.A32.data(), p.A16.data(), p.mA.data(), p.vA.data(), p.gA.data(), (i64)p.A32.size(), lr, m.a.b1, m.a.b2, m.a.eps, m.a.wd, t);
                or_adamw_step(p.B32.data(), p.B16.data(), p.mB.data(), p.vB.data(), p.gB.data(), (i64)p.B32.size(), lr, m.a.b1, m.a.b2, m.a.eps, m.a.wd, t);
            }
    m.step_count++;
    if (so) {
        so->loss = mean_loss;
        so->lr = lr;
        so->gnorm = gnorm;
        so->gnorm_raw = gnorm_raw;
        so->valid_tokens = valid;
        so->step = (int)m.step_count;
    }
    return mean_loss;
}

VB* weight_slot(Model& m, const std::string& name) {
    if (name == "model.embed_tokens.weight") return &m.embed;
    if (name == "model.norm.weight") return &m.final_norm;
    if (name == "lm_head.weight") return &m.lm_head;
    const std::string pre = "model.layers.";
    if (name.compare(0, pre.size(), pre) != 0) return nullptr;
    size_t dot = name.find('.', pre.size());
    int l = std::stoi(name.substr(pre.size(), dot - pre.size()));
    if (l < 0 || l >= (int)m.L.size()) return nullptr;
    std::string k = name.substr(dot + 1);
    LayerW& w = m.L[l];
    if (k == "input_layernorm.weight") return &w.in_norm;
    if (k == "self_attn.q_proj.weight") return &w.q_w;
    if (k == "self_attn.q_proj.bias") return &w.q_b;
    if (k == "self_attn.k_proj.weight") return &w.k_w;
    if (k == "self_attn.k_proj.bias") return &w.k_b;
    if (k == "self_attn.v_proj.weight") return &w.v_w;
    if (k == "self_attn.v_proj.bias") return &w.v_b;
    if (k == "self_attn.o_proj.weight") return &w.o_w;
    if (k == "post_attention_layernorm.weight") return &w.post_norm;
    if (k == "mlp.gate_proj.weight") return &w.gate_w;
    if (k == "mlp.up_proj.weight") return &w.up_w;
    if (k == "mlp.down_proj.weight") return &w.down_w;
    return nullptr;
}

}  // namespace

extern "C" {

void* or_model_create(const ModelCfg* c, const AdaptCfg* a) {
    Model* m = new Model();
    m->c = *c;
    m->a = *a;
    int H = c->hidden, kv = c->n_kv * c->head_dim, qd = c->n_q * c->head_dim, I = c->inter;
    m->L.resize(c->layers);
    for (auto& lw : m->L) {
        int mask = a->inject_mask;
        make_pair(lw.pr[TQ], mask & 1, H, qd, a->rank);
        make_pair(lw.pr[TK], mask & 2, H, kv, a->rank);
        make_pair(lw.pr[TV], mask & 4, H, kv, a->rank);
        make_pair(lw.pr[TO], mask & 8, qd, H, a->rank);
        make_pair(lw.pr[TG], mask & 16, H, I, a->rank);
        make_pair(lw.pr[TU], mask & 32, H, I, a->rank);
        make_pair(lw.pr[TD], mask & 64, I, H, a->rank);
    }
    m->cacc.assign(H, 0.0);
    return m;
}
void or_model_destroy(void* p) { delete (Model*)p; }

int or_model_set_weight(void* p, const char* name, const bf16_t* data, i64 n) {
    VB* s = weight_slot(*(Model*)p, name);
    if (!s) return -1;
    s->assign(data, data + n);
    return 0;
}

// which: 0 A_f32, 1 B_f32, 2 mA, 3 vA, 4 mB, 5 vB, 6 gA, 7 gB (float)
//        8 A_bf16, 9 B_bf16 (bf16)
void* or_model_adapter_ptr(void* p, int layer, int target, int which, i64* n) {
    Model* m = (Model*)p;
    if (layer < 0 || layer >= (int)m->L.size() || target < 0 || target >= NTGT) return nullptr;
    Pair& pr = m->L[layer].pr[target];
    if (!pr.on) return nullptr;
    VF* f[8] = {&pr.A32, &pr.B32, &pr.mA, &pr.vA, &pr.mB, &pr.vB, &pr.gA, &pr.gB};
    if (which >= 0 && which < 8) {
        *n = (i64)f[which]->size();
        return f[which]->data();
    }
    if (which == 8) {
        *n = (i64)pr.A16.size();
        return pr.A16.data();
    }
    if (which == 9) {
        *n = (i64)pr.B16.size();
        return pr.B16.data();
    }
    return nullptr;
}

int or_model_step(void* p, const int32_t* inputs, const int32_t* targets, int B, int T,
                  float lr_override, StepOut* out) {
    step_model(*(Model*)p, inputs, targets, B, T, out, lr_override);
    return 0;
}

void or_model_keep_taps(void* p, int on) { ((Model*)p)->keep_taps = on != 0; }

// copies a tap into dst; returns element count (0 if absent); kind 0 bf16, 1 f32
i64 or_model_tap(void* p, const char* name, void* dst, int* kind) {
    Model* m = (Model*)p;
    auto ib = m->taps_b.find(name);
    if (ib != m->taps_b.end()) {
        if (dst) std::memcpy(dst, ib->second.data(), ib->second.size() * 2);
        if (kind) *kind = 0;
        return (i64)ib->second.size();
    }
    auto jf = m->taps_f.find(name);
    if (jf != m->taps_f.end()) {
        if (dst) std::memcpy(dst, jf->second.data(), jf->second.size() * 4);
        if (kind) *kind = 1;
        return (i64)jf->second.size();
    }
    return 0;
}

void or_model_centroid(void* p, double* acc, double* acc_w) {
    Model* m = (Model*)p;
    std::memcpy(acc, m->cacc.data(), m->cacc.size() * 8);
    *acc_w = m->cacc_w;
}

}  // extern "C"
