// gemm.hip — BF16 GEMM on gfx950 matrix cores (v_mfma_f32_32x32x16_bf16).
//
// Row-major problem (every GEMM of the step is one of these):
//   C[m, n] = alpha * sum_k X(m,k) * Y(k,n) + beta * C[m, n]   (F32 accumulate)
//   X(m,k) = XK ? X[m*ldx + k] : X[k*ldx + m]
//   Y(k,n) = YK ? Y[n*ldy + k] : Y[k*ldy + n]
// The step engine stores every frozen weight twice (W [out,in] and W^T
// [in,out], 288 GB of HBM makes that cheap), so all large GEMMs — forward
// x*W^T and backward dY*W — run with XK = YK = true: both operands are
// K-contiguous, global loads are 16-byte vectors along K and LDS tiles are
// stored K-contiguous, which is exactly the per-lane operand shape of the
// MFMA (8 consecutive k of one row).  The K-strided layouts (LoRA weight
// gradients, whose reduction runs over tokens) transpose while staging into
// LDS.
//
// Tiling: block = 256 threads = 4 wave64s arranged WM x WN, block tile
// BM x BN x 64, wave tile (BM/WM) x (BN/WN) made of 32x32 MFMA tiles.  LDS
// rows are padded by 8 BF16 (144-byte stride) so the 16-byte fragment reads
// of 8 consecutive rows hit disjoint banks.  Two LDS stages: the next
// k-tile's global loads are in flight while the current one feeds the MFMAs,
// one barrier per k-tile.  Block ids are remapped so that each of the 8 XCDs
// (own L2 each) works a contiguous band of output tiles.
//
// Epilogues: BF16 (alpha, beta, optional bias added after the first
// rounding and rounded again — the reference's gemm + ops::add_bias), F32
// (gemm_f32 semantics), or F32 partials for split-K with a separate
// fixed-order reduction (deterministic).
#include <algorithm>
#include <numeric>
#include <type_traits>

#include "ta_backend.h"
#include "ta_internal.hpp"

namespace ta {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 16-byte output store with the non-temporal hint (global_store ... nt).
// A GEMM's output is written once and read by a later kernel; with the
// hint the c3 step ran 1.9% faster than with plain stores (the values
// stored are the same), although the GEMMs' L2 misses rose.
__device__ __forceinline__ void st_out16(void* p, const bf16x8v& v) {
    const u32x4_t x = {v.w[0], v.w[1], v.w[2], v.w[3]};
    __builtin_nontemporal_store(x, (u32x4_t*)p);
}

constexpr int BK = 64;
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row

enum Epi { EPI_BF16 = 0, EPI_F32 = 1, EPI_PARTIAL = 2 };

struct GemmArgs {
    int M, N, K;
    const bf16* X;
    int64_t ldx;
    const bf16* Y;
    int64_t ldy;
    void* C;
    int64_t ldc;
    float alpha, beta;
    const bf16* bias;
    float* part;     // split-K partials [splits][M][N]
    int k_per_split; // multiple of BK
    int tiles_m, tiles_n;
    // LoRA epilogue (k_gemm_big only): after the base rounding, for each
    // pair p in order, with D_p = U_p V_p^T (U_p [M x r], V_p [N x r]):
    //   delta: C = bf16(C + s * bf16(D_p))    (apply_lora_fwd)
    //   else : C = bf16(s * D_p + C)          (apply_lora_bwd's dx GEMM)
    int lora_n, lora_r, lora_delta;
    float lora_s;
    const bf16* lora_u[3];
    int64_t lora_ldu[3];
    const bf16* lora_v[3];
    // N-concatenated groups (k_gemm_pipe only; ngroups <= 1 otherwise):
    // tile columns [tn0[g], tn0[g + 1]) compute group g's own GEMM over the
    // same X: gN[g] output columns of gY[g], written to gC[g] (row stride
    // gldc[g]) with bias gbias[g] and, when glora[g], the LoRA pair gu/gv[g]
    // (rank lora_r <= 64, lora_delta and lora_s shared).  The fields above describe
    // group 0 only as far as they are shared (M, K, X, ldy, alpha, beta).
    int ngroups;
    int tn0[3];
    int gN[3];
    int glora[3];
    const bf16* gY[3];
    void* gC[3];
    int64_t gldc[3];
    const bf16* gbias[3];
    const bf16* gu[3];
    const bf16* gv[3];
    // K segments (k_gemm_pipe only; nseg <= 1 otherwise): k in [kseg[s],
    // kseg[s + 1]) runs over X_s Y_s^T (sX, sldx, sY, sldy; k relative to
    // kseg[s]) and the accumulators are rounded to BF16 where a segment
    // ends: the chain C = bf16(X_s Y_s^T + C), s = 0, 1, .., in one launch
    int nseg;
    int kseg[3];
    const bf16* sX[3];
    int64_t sldx[3];
    const bf16* sY[3];
    int64_t sldy[3];
    // cross-entropy gradient formed from X = logits in the operand reads
    // (k_gemm_pipe_ce): per-row base-2 normaliser, target id, 1 / N
    const float* ce_lse2;
    const int32_t* ce_tgt;
    float ce_inv_n;
    // RoPE of the output (k_gemm_pipe / k_gemm_mid epilogue; NULL: none):
    // rope_tab [rope_T][rope_hd / 2] (cos, sin); row m is position
    // m % rope_T and output column c pair (c % rope_hd) / 2 of its head.
    // Per group in grope (which the tile's group selects into rope_tab).
    const float2* rope_tab;
    int rope_T, rope_hd;
    const float2* grope[3];
};

// Load one 16-byte chunk (8 bf16) of a K-contiguous operand row with
// bounds guards; out-of-range elements are zero.
__device__ __forceinline__ bf16x8v load_k8(const bf16* __restrict__ P, int64_t ld, int row,
                                           int k, int rows, int kend, bool vec) {
    bf16x8v v;
    if (row < rows && vec && k + 8 <= kend) {
        v = *(const bf16x8v*)(P + (int64_t)row * ld + k);
    } else {
        uint16_t t[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
            t[e] = (row < rows && k + e < kend) ? P[(int64_t)row * ld + k + e] : (uint16_t)0;
#pragma unroll
        for (int e = 0; e < 4; e++) v.w[e] = (uint32_t)t[2 * e] | ((uint32_t)t[2 * e + 1] << 16);
    }
    return v;
}
// Load 8 consecutive rows at one k of a row-contiguous (K-strided) operand.
__device__ __forceinline__ bf16x8v load_r8(const bf16* __restrict__ P, int64_t ld, int row,
                                           int k, int rows, int kend, bool vec) {
    bf16x8v v;
    if (k < kend && vec && row + 8 <= rows) {
        v = *(const bf16x8v*)(P + (int64_t)k * ld + row);
    } else {
        uint16_t t[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
            t[e] = (k < kend && row + e < rows) ? P[(int64_t)k * ld + row + e] : (uint16_t)0;
#pragma unroll
        for (int e = 0; e < 4; e++) v.w[e] = (uint32_t)t[2 * e] | ((uint32_t)t[2 * e + 1] << 16);
    }
    return v;
}

// Stage a ROWS x BK tile of an operand into LDS (K-contiguous rows).
template <int ROWS, bool KMAJ>
struct TileLoader {
    static constexpr int CHUNKS = ROWS * BK / 8;
    static constexpr int PER_THREAD = (CHUNKS + 255) / 256;
    bf16x8v r[PER_THREAD];

    __device__ __forceinline__ void load(const bf16* __restrict__ P, int64_t ld, int row0, int k0,
                                         int rows, int kend, bool vec) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            int q = threadIdx.x + 256 * i;
            if (q < CHUNKS) {
                if (KMAJ) {
                    int rr = q / (BK / 8), kc = q % (BK / 8);
                    r[i] = load_k8(P, ld, row0 + rr, k0 + kc * 8, rows, kend, vec);
                } else {
                    int kk = q / (ROWS / 8), rc = q % (ROWS / 8);
                    r[i] = load_r8(P, ld, row0 + rc * 8, k0 + kk, rows, kend, vec);
                }
            }
        }
    }
    __device__ __forceinline__ void store(bf16* __restrict__ S) {
#pragma unroll
        for (int i = 0; i < PER_THREAD; i++) {
            int q = threadIdx.x + 256 * i;
            if (q < CHUNKS) {
                if (KMAJ) {
                    int rr = q / (BK / 8), kc = q % (BK / 8);
                    *(bf16x8v*)(S + rr * LDS_STRIDE + kc * 8) = r[i];
                } else {
                    int kk = q / (ROWS / 8), rc = q % (ROWS / 8);
#pragma unroll
                    for (int e = 0; e < 8; e++) {
                        uint16_t h = (uint16_t)(r[i].w[e >> 1] >> ((e & 1) * 16));
                        S[(rc * 8 + e) * LDS_STRIDE + kk] = h;
                    }
                }
            }
        }
    }
};

template <int BM, int BN, int WM, int WN, bool XK, bool YK, int EPI>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs a, bool vecx, bool vecy) {
    constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
    constexpr int TM = WTM / 32, TN = WTN / 32;  // MFMA tiles per wave
    static_assert(WM * WN == 4, "4 waves per block");
    static_assert(TM >= 1 && TN >= 1, "wave tile too small");
    __shared__ __attribute__((aligned(16))) bf16 sX[2][BM * LDS_STRIDE];
    __shared__ __attribute__((aligned(16))) bf16 sY[2][BN * LDS_STRIDE];

    // XCD-aware block order: hardware dispatches consecutive block ids
    // round-robin over 8 XCDs; give each XCD a contiguous band of tiles.
    int nt = a.tiles_m * a.tiles_n;
    int bid = blockIdx.x;
    if ((nt & 7) == 0) bid = (bid & 7) * (nt >> 3) + (bid >> 3);
    int tm_i = bid / a.tiles_n, tn_i = bid % a.tiles_n;
    int m0 = tm_i * BM, n0 = tn_i * BN;
    int kbeg = blockIdx.z * a.k_per_split;
    int kend = min(a.K, kbeg + a.k_per_split);

    int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int wm = wv / WN, wn = wv % WN;

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    TileLoader<BM, XK> lx;
    TileLoader<BN, YK> ly;
    int nk = (kend - kbeg + BK - 1) / BK;
    if (nk > 0) {
        lx.load(a.X, a.ldx, m0, kbeg, a.M, kend, vecx);
        ly.load(a.Y, a.ldy, n0, kbeg, a.N, kend, vecy);
        lx.store(sX[0]);
        ly.store(sY[0]);
    }
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        int cur = kt & 1;
        bool more = kt + 1 < nk;
        if (more) {
            int k0 = kbeg + (kt + 1) * BK;
            lx.load(a.X, a.ldx, m0, k0, a.M, kend, vecx);
            ly.load(a.Y, a.ldy, n0, k0, a.N, kend, vecy);
        }
        const bf16* SX = sX[cur] + (wm * WTM + (lane & 31)) * LDS_STRIDE + (lane >> 5) * 8;
        const bf16* SY = sY[cur] + (wn * WTN + (lane & 31)) * LDS_STRIDE + (lane >> 5) * 8;
#pragma unroll
        for (int kk = 0; kk < BK / 16; kk++) {
            bf16x8_t fx[TM], fy[TN];
#pragma unroll
            for (int i = 0; i < TM; i++)
                fx[i] = *(const bf16x8_t*)(SX + i * 32 * LDS_STRIDE + kk * 16);
#pragma unroll
            for (int j = 0; j < TN; j++)
                fy[j] = *(const bf16x8_t*)(SY + j * 32 * LDS_STRIDE + kk * 16);
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] =
                        __builtin_amdgcn_mfma_f32_32x32x16_bf16(fx[i], fy[j], acc[i][j], 0, 0, 0);
        }
        if (more) {
            lx.store(sX[cur ^ 1]);
            ly.store(sY[cur ^ 1]);
        }
        __syncthreads();
    }

    // epilogue: lane holds column n = lane%32 of each 32x32 tile and rows
    // 8*(r/4) + 4*(lane/32) + r%4
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            int n = n0 + wn * WTN + j * 32 + (lane & 31);
            if (n >= a.N) continue;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                int m = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m >= a.M) continue;
                float v = acc[i][j][r];
                if (EPI == EPI_BF16) {
                    bf16* C = (bf16*)a.C + (int64_t)m * a.ldc + n;
                    float o = a.alpha * v;
                    if (a.beta != 0.f) o += a.beta * bf2f(*C);
                    if (a.bias) o = bf2f(f2bf(o)) + bf2f(a.bias[n]);
                    *C = f2bf(o);
                } else if (EPI == EPI_F32) {
                    float* C = (float*)a.C + (int64_t)m * a.ldc + n;
                    float o = a.alpha * v;
                    if (a.beta != 0.f) o += a.beta * (*C);
                    *C = o;
                } else {
                    a.part[((int64_t)blockIdx.z * a.M + m) * a.N + n] = v;
                }
            }
        }
}

// ── Large K-contiguous GEMMs (every frozen-base projection, the LM head) ──
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Tile of a block for the large kernels.  Blocks are dealt round-robin to
// the 8 XCDs (each with its own L2); each XCD gets a contiguous range of
// tile indices, walked in groups of GM tile-rows column by column, so the
// ~32 tiles an XCD runs at once share GM row bands of X and a few column
// bands of Y in its L2 instead of streaming all of Y.  GM = 8 (8 x 4
// tiles at once) measured 0.4% faster on the c3 step than 4 (4 x 8) and
// 1% faster than 16.
constexpr int TILE_GM = 8;
__device__ __forceinline__ void big_tile(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
    int nt = tiles_m * tiles_n;
    if ((nt & 7) == 0) bid = (bid & 7) * (nt >> 3) + (bid >> 3);
    int gsz = TILE_GM * tiles_n;
    int g = bid / gsz, idx = bid % gsz;
    int rows = min(TILE_GM, tiles_m - g * TILE_GM);
    tm = g * TILE_GM + idx % rows;
    tn = idx / rows;
}

// Epilogue of the large GEMM kernels on the 32x32 MFMA accumulator layout
// (lane: column l%32, rows 8*(r/4) + 4*(l/32) + r%4 of each fragment).
template <int TM, int TN, int WTM, int WTN, int EPI>
__device__ __attribute__((always_inline)) inline void big_epilogue(floatx16 (&acc)[TM][TN],
                                                                   const GemmArgs& a, int m0,
                                                                   int n0, int wm, int wn,
                                                                   int lane) {
    if constexpr (EPI == EPI_PARTIAL) {
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                int n = n0 + wn * WTN + j * 32 + (lane & 31);
                if (n >= a.N) continue;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    int m = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (m < a.M) a.part[((int64_t)blockIdx.z * a.M + m) * a.N + n] = acc[i][j][r];
                }
            }
    } else {
        // three small unrolled passes keep acc in registers: (1) base
        // epilogue in place, (2) LoRA terms pair by pair, (3) store
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                int n = n0 + wn * WTN + j * 32 + (lane & 31);
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    int m = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    float o = a.alpha * acc[i][j][r];
                    if (a.beta != 0.f && m < a.M && n < a.N)
                        o += a.beta * bf2f(((const bf16*)a.C)[(int64_t)m * a.ldc + n]);
                    if (a.bias && n < a.N) o = bf2f(f2bf(o)) + bf2f(a.bias[n]);
                    acc[i][j][r] = bf2f(f2bf(o));
                }
            }
        // LoRA terms: D = U V^T on the same 32x32 MFMA layout as acc; static
        // pair indices (a runtime index into the by-value argument struct
        // would move it to scratch)
#pragma unroll
        for (int p = 0; p < 3; p++) {
            if (p >= a.lora_n) continue;
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++) {
                    int arow = min(m0 + wm * WTM + i * 32 + (lane & 31), a.M - 1);
                    int bcol = min(n0 + wn * WTN + j * 32 + (lane & 31), a.N - 1);
                    floatx16 d;
#pragma unroll
                    for (int r = 0; r < 16; r++) d[r] = 0.f;
                    for (int k = 0; k < a.lora_r; k += 16) {
                        int kk = k + 8 * (lane >> 5);
                        bf16x8_t fa, fb;
                        if (kk < a.lora_r) {
                            fa = *(const bf16x8_t*)(a.lora_u[p] + (int64_t)arow * a.lora_ldu[p] + kk);
                            fb = *(const bf16x8_t*)(a.lora_v[p] + (int64_t)bcol * a.lora_r + kk);
                        } else {
#pragma unroll
                            for (int e = 0; e < 8; e++) fa[e] = fb[e] = (__bf16)0.f;
                        }
                        d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa, fb, d, 0, 0, 0);
                    }
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        acc[i][j][r] = a.lora_delta
                                           ? bf2f(f2bf(acc[i][j][r] + a.lora_s * bf2f(f2bf(d[r]))))
                                           : bf2f(f2bf(a.lora_s * d[r] + acc[i][j][r]));
                }
        }
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                int n = n0 + wn * WTN + j * 32 + (lane & 31);
                if (n >= a.N) continue;
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    int m = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                    if (m < a.M) ((bf16*)a.C)[(int64_t)m * a.ldc + n] = f2bf(acc[i][j][r]);
                }
            }
    }
}

// BF16 epilogue through LDS for the direct-to-LDS kernel: each wave stages
// its own 64 x WTN output sub-tile in a private LDS region `wb` (row stride
// WTN), so C is read (beta != 0) and written with 16-byte row vectors
// instead of 2-byte column-layout accesses.  Same arithmetic as
// big_epilogue: (1) alpha acc + beta C (+ bias) rounded in place, (2) the
// LoRA terms pair by pair, (3) the store.  Only this wave touches wb, and a
// wave's LDS operations complete in order.
template <int TM, int TN, int WTM, int WTN>
__device__ __attribute__((always_inline)) inline void staged_epilogue(
    floatx16 (&acc)[TM][TN], const GemmArgs& a, int m0, int n0, int wm, int wn, int lane,
    bf16* __restrict__ wb) {
    constexpr int CPR = WTN / 8;  // 16-byte chunks per sub-tile row
    const int R0 = m0 + wm * WTM, C0 = n0 + wn * WTN;
    bf16* C = (bf16*)a.C;
    const bool vec = ((a.ldc & 7) == 0) && (((uintptr_t)C & 15) == 0);
    if (a.beta != 0.f) {
        for (int q = lane; q < WTM * CPR; q += 64) {
            int row = q / CPR, ch = q % CPR;
            int gm = R0 + row, gn = C0 + 8 * ch;
            bf16x8v v;
            if (gm < a.M && vec && gn + 8 <= a.N) {
                v = *(const bf16x8v*)(C + (int64_t)gm * a.ldc + gn);
            } else {
                uint16_t t[8];
#pragma unroll
                for (int e = 0; e < 8; e++)
                    t[e] = (gm < a.M && gn + e < a.N) ? C[(int64_t)gm * a.ldc + gn + e] : (uint16_t)0;
#pragma unroll
                for (int e = 0; e < 4; e++) v.w[e] = (uint32_t)t[2 * e] | ((uint32_t)t[2 * e + 1] << 16);
            }
            *(bf16x8v*)(wb + row * WTN + 8 * ch) = v;
        }
        __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            int lc = j * 32 + (lane & 31);
            int n = C0 + lc;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                int lr = i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                float o = a.alpha * acc[i][j][r];
                if (a.beta != 0.f) o += a.beta * bf2f(wb[lr * WTN + lc]);
                if (a.bias && n < a.N) o = bf2f(f2bf(o)) + bf2f(a.bias[n]);
                acc[i][j][r] = bf2f(f2bf(o));
            }
        }
#pragma unroll
    for (int p = 0; p < 3; p++) {
        if (p >= a.lora_n) continue;
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++) {
                int arow = min(R0 + i * 32 + (lane & 31), a.M - 1);
                int bcol = min(C0 + j * 32 + (lane & 31), a.N - 1);
                floatx16 d;
#pragma unroll
                for (int r = 0; r < 16; r++) d[r] = 0.f;
                for (int k = 0; k < a.lora_r; k += 16) {
                    int kk = k + 8 * (lane >> 5);
                    bf16x8_t fa, fb;
                    if (kk < a.lora_r) {
                        fa = *(const bf16x8_t*)(a.lora_u[p] + (int64_t)arow * a.lora_ldu[p] + kk);
                        fb = *(const bf16x8_t*)(a.lora_v[p] + (int64_t)bcol * a.lora_r + kk);
                    } else {
#pragma unroll
                        for (int e = 0; e < 8; e++) fa[e] = fb[e] = (__bf16)0.f;
                    }
                    d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa, fb, d, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 16; r++)
                    acc[i][j][r] = a.lora_delta
                                       ? bf2f(f2bf(acc[i][j][r] + a.lora_s * bf2f(f2bf(d[r]))))
                                       : bf2f(f2bf(a.lora_s * d[r] + acc[i][j][r]));
            }
    }
    __builtin_amdgcn_wave_barrier();  // the beta reads of wb are done
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) {
            int lc = j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r++) {
                int lr = i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                wb[lr * WTN + lc] = f2bf(acc[i][j][r]);
            }
        }
    __builtin_amdgcn_wave_barrier();
    for (int q = lane; q < WTM * CPR; q += 64) {
        int row = q / CPR, ch = q % CPR;
        int gm = R0 + row, gn = C0 + 8 * ch;
        if (gm >= a.M) continue;
        bf16x8v v = *(const bf16x8v*)(wb + row * WTN + 8 * ch);
        if (vec && gn + 8 <= a.N) {
            st_out16(C + (int64_t)gm * a.ldc + gn, v);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (gn + e < a.N) C[(int64_t)gm * a.ldc + gn + e] = (uint16_t)(v.w[e >> 1] >> ((e & 1) * 16));
        }
    }
}

// ── k_gemm_dma: the same tiles fed by direct global->LDS loads ────────────
// BK = 32 per stage (rows of 64 bytes = 4 chunks of 16 bytes) and NS stages
// in LDS, so the loads of tile k + NS - 1 are in flight while tile k
// computes, with no register staging.  One global_load_lds_dwordx4 fills 16
// consecutive rows of a stage; chunk c of row R sits in slot c ^ dswz(R),
// which keeps every 16-row fragment read free of bank conflicts.
constexpr int DBK = 32;
__device__ __forceinline__ int dswz(int R) { return ((R >> 1) ^ (R >> 3)) & 3; }

// Stage rows of KD = 32 k (64 bytes: 4 chunks, above) or KD = 64 k (128
// bytes, one whole line: 8 chunks, slot c ^ ((R ^ R >> 3) & 7); any 8 or 16
// consecutive rows then read one chunk each from distinct banks).  One
// DMA instruction fills 64 / (KD / 8) consecutive rows.
template <int KD>
__device__ __forceinline__ int stage_swz(int R) {
    if constexpr (KD == 32)
        return dswz(R);
    else
        return (R ^ (R >> 3)) & 7;
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// One direct-to-LDS load, global_load_lds_dwordx4 in its scalar-base form
// (wave-uniform 64-bit base, 32-bit byte offset per lane; lane i writes LDS
// bytes lds + 16 i .. + 15), issued from inline assembly: the compiler does
// not see it as a write to LDS, so it does not make the next LDS read wait
// for every load in flight (it cannot tell the stage buffers apart and
// would).  The kernels order these loads with explicit vmcnt waits and
// barriers.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, const void* lds) {
    const uint32_t la = (uint32_t)(uintptr_t)lds;
    const uint64_t ba = (uint64_t)(uintptr_t)base;
    // (readfirstlane returns int: each half goes through uint32_t so that the
    // low word is not sign-extended into the high one)
    const uint64_t bu =
        (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)ba) |
        ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(ba >> 32)) << 32);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(__builtin_amdgcn_readfirstlane(la)), "v"(off), "s"(bu)
                 : "memory", "m0");
#pragma clang diagnostic pop
}

// Issue this wave's share of the loads of one stage: operand rows
// [row0, row0 + ROWS) (clamped to rows - 1), k range [k0, k0 + 32).
// Wave-instruction j covers stage rows 16j..16j+15.  Every one of the NW
// waves issues the same number, PER = ceil(NI / NW), in straight-line code
// (so the compiler's wait bookkeeping stays exact): j = w + NW h; an index
// past the end repeats an instruction of a lower wave, writing the same
// bytes.
template <int ROWS, int NW, int KD = DBK>
__device__ __forceinline__ void dma_stage(const bf16* __restrict__ P, int64_t ld, int row0,
                                          int rows, int k0, bf16* stage, int w, int lane) {
    constexpr int LPR = KD / 8, RPI = 64 / LPR;  // lanes per row, rows per instruction
    constexpr int NI = ROWS / RPI;
    constexpr int PER = (NI + NW - 1) / NW;
    // a wave-uniform base (the tile's first row at k0) plus a 32-bit byte
    // offset per lane: the scalar-base address form (row0 < rows; the
    // hosts check that ROWS rows of an operand span less than 4 GB)
    const char* bs = (const char*)(P + (int64_t)row0 * ld + k0);
#pragma unroll
    for (int h = 0; h < PER; h++) {
        int j = w + NW * h;
        j = j < NI ? j : j - NW;
        int r = RPI * j + lane / LPR;
        int c = (lane % LPR) ^ stage_swz<KD>(r);
        int grow = min(row0 + r, rows - 1);
        const uint32_t off = (uint32_t)((int64_t)(grow - row0) * ld * 2) + 16u * (uint32_t)c;
        dma16(bs, off, stage + RPI * j * KD);
    }
}

// dma_stage split in two for operands whose base and row stride change
// during the loop (the K segments of a chain): dma_offsets computes, once,
// this lane's byte offset from the tile's first row (clamped row x ld +
// swizzled chunk) for each of the wave's PER instructions; dma_stage_at
// issues them for one stage from the wave-uniform address of the tile's
// first row at k0.  Same addresses as dma_stage.
template <int ROWS, int NW, int KD = DBK>
struct DmaOffs {
    static constexpr int LPR = KD / 8, RPI = 64 / LPR;
    static constexpr int NI = ROWS / RPI, PER = (NI + NW - 1) / NW;
    uint32_t o[PER];
};
template <int ROWS, int NW, int KD>
__device__ __forceinline__ void dma_offsets(DmaOffs<ROWS, NW, KD>& d, int64_t ld, int row0,
                                            int rows, int w, int lane) {
    using D = DmaOffs<ROWS, NW, KD>;
#pragma unroll
    for (int h = 0; h < D::PER; h++) {
        int j = w + NW * h;
        j = j < D::NI ? j : j - NW;
        const int r = D::RPI * j + lane / D::LPR;
        const int c = (lane % D::LPR) ^ stage_swz<KD>(r);
        d.o[h] = (uint32_t)((int64_t)(min(row0 + r, rows - 1) - row0) * ld * 2) + 16u * (uint32_t)c;
    }
}
template <int ROWS, int NW, int KD>
__device__ __forceinline__ void dma_stage_at(const bf16* __restrict__ base,
                                             const DmaOffs<ROWS, NW, KD>& d, bf16* stage, int w) {
    using D = DmaOffs<ROWS, NW, KD>;
#pragma unroll
    for (int h = 0; h < D::PER; h++) {
        int j = w + NW * h;
        j = j < D::NI ? j : j - NW;
        dma16(base, d.o[h], stage + D::RPI * j * KD);
    }
}

// One 32-wide k slice of MFMAs for a wave from a swizzled stage.
template <int TM, int TN, int WTM, int WTN>
__device__ __attribute__((always_inline)) inline void dma_mma(floatx16 (&acc)[TM][TN],
                                                              const bf16* sX, const bf16* sY,
                                                              int wm, int wn, int lane) {
#pragma unroll
    for (int kk = 0; kk < DBK / 16; kk++) {
        const int c = 2 * kk + (lane >> 5);
        bf16x8_t fx[TM], fy[TN];
#pragma unroll
        for (int i = 0; i < TM; i++) {
            int R = wm * WTM + i * 32 + (lane & 31);
            fx[i] = *(const bf16x8_t*)(sX + R * DBK + 8 * (c ^ dswz(R)));
        }
#pragma unroll
        for (int j = 0; j < TN; j++) {
            int R = wn * WTN + j * 32 + (lane & 31);
            fy[j] = *(const bf16x8_t*)(sY + R * DBK + 8 * (c ^ dswz(R)));
        }
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
            for (int j = 0; j < TN; j++)
                acc[i][j] =
                    __builtin_amdgcn_mfma_f32_32x32x16_bf16(fx[i], fy[j], acc[i][j], 0, 0, 0);
    }
}


// 1 KB of zeros: the source of the tiles that pad K up to a whole number
// of trips (they add exact zeros)
static __device__ __attribute__((aligned(16))) bf16 g_dma_zero[512] = {};

template <int BN, int EPI, int NS, int WMW, int WNW>
__global__ __launch_bounds__(WMW * WNW * 64) void k_gemm_dma(GemmArgs a) {
    static_assert(NS == 4 || NS == 5, "4 or 5 stages");
    constexpr int BM = 256, NW = WMW * WNW;
    // loads per stage per wave
    constexpr int LPS = (BM / 16 + NW - 1) / NW + (BN / 16 + NW - 1) / NW;
    constexpr int WTM = BM / WMW, WTN = BN / WNW;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    constexpr int SX = BM * DBK, SY = BN * DBK;  // elements per stage
    // one LDS object per stage and operand: the compiler then only waits for
    // the loads into the buffer a read touches
    __shared__ __attribute__((aligned(1024))) bf16 sX0[SX], sX1[SX], sX2[SX], sX3[SX];
    __shared__ __attribute__((aligned(1024))) bf16 sY0[SY], sY1[SY], sY2[SY], sY3[SY];
    __shared__ __attribute__((aligned(1024))) bf16 sX4[NS == 5 ? SX : 16], sY4[NS == 5 ? SY : 16];

    int tm_i, tn_i;
    big_tile(blockIdx.x, a.tiles_m, a.tiles_n, tm_i, tn_i);
    int m0 = tm_i * BM, n0 = tn_i * BN;
    int kbeg = blockIdx.z * a.k_per_split;
    int kend = min(a.K, kbeg + a.k_per_split);
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int wm = w / WNW, wn = w % WNW;
    w = __builtin_amdgcn_readfirstlane(w);  // wave-uniform

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    // K runs as tiles kt = -pad .. nk-1 (pad makes the count a multiple of
    // NS; padded tiles load zeros).  Every step issues one stage (tiles
    // past the end reload the last tile into a buffer that is never read),
    // so exactly NS - 2 stages are issued after the one a step computes:
    // LPS loads per stage per wave.
    const int nk = (kend - kbeg) / DBK;
    const int pad = (NS - nk % NS) % NS;
    // (a padded tile reads row 0 of the zero buffer with stride 0: uniform
    // selects, no branch)
#define DMA_ISSUE(SXB, SYB, KT)                                                          \
    do {                                                                                 \
        const int kq_ = (KT);                                                            \
        const bool z_ = kq_ < 0;                                                         \
        const int k_ = z_ ? 0 : kbeg + min(kq_, nk - 1) * DBK;                          \
        dma_stage<BM, NW>(z_ ? g_dma_zero : a.X, z_ ? 0 : a.ldx, m0, a.M, k_, SXB, w,    \
                          lane);                                                         \
        dma_stage<BN, NW>(z_ ? g_dma_zero : a.Y, z_ ? 0 : a.ldy, n0, a.N, k_, SYB, w,    \
                          lane);                                                         \
    } while (0)
    DMA_ISSUE(sX0, sY0, 0 - pad);
    DMA_ISSUE(sX1, sY1, 1 - pad);
    DMA_ISSUE(sX2, sY2, 2 - pad);
    if constexpr (NS == 5) DMA_ISSUE(sX3, sY3, 3 - pad);
    // step on stage buffer J: wait for its loads, barrier (also: every wave
    // is done reading buffer JN), refill JN with tile kt + NS - 1, compute J
    // (no branch inside the loop body keeps the compiler's wait bookkeeping
    // per buffer)
#define DMA_STEP(J, SXJ, SYJ, SXN, SYN)                                                  \
    do {                                                                                 \
        TA_WAIT_VMCNT(LPS * (NS - 2));                                                   \
        __builtin_amdgcn_s_barrier();                                                    \
        DMA_ISSUE(SXN, SYN, kt0 + (J) + NS - 1);                                         \
        dma_mma<TM, TN, WTM, WTN>(acc, SXJ, SYJ, wm, wn, lane);                          \
    } while (0)
    for (int kt0 = -pad; kt0 < nk; kt0 += NS) {
        if constexpr (NS == 4) {
            DMA_STEP(0, sX0, sY0, sX3, sY3);
            DMA_STEP(1, sX1, sY1, sX0, sY0);
            DMA_STEP(2, sX2, sY2, sX1, sY1);
            DMA_STEP(3, sX3, sY3, sX2, sY2);
        } else {
            DMA_STEP(0, sX0, sY0, sX4, sY4);
            DMA_STEP(1, sX1, sY1, sX0, sY0);
            DMA_STEP(2, sX2, sY2, sX1, sY1);
            DMA_STEP(3, sX3, sY3, sX2, sY2);
            DMA_STEP(4, sX4, sY4, sX3, sY3);
        }
    }
    TA_WAIT_VMCNT(0);  // the surplus loads have landed before the block ends
#undef DMA_STEP
#undef DMA_ISSUE
    if constexpr (EPI == EPI_BF16 && WMW * WNW == 8) {
        // every wave is done with the stage buffers: each takes one of the
        // eight as its private output staging region (64 x WTN BF16 fits)
        static_assert(64 * WTN * 2 <= SY * 2 && 64 * WTN * 2 <= SX * 2, "staging fits");
        __syncthreads();
        bf16* wb = w == 0 ? sX0 : w == 1 ? sX1 : w == 2 ? sX2 : w == 3 ? sX3
                 : w == 4 ? sY0 : w == 5 ? sY1 : w == 6 ? sY2 : sY3;
        staged_epilogue<TM, TN, WTM, WTN>(acc, a, m0, n0, wm, wn, lane, wb);
    } else {
        big_epilogue<TM, TN, WTM, WTN, EPI>(acc, a, m0, n0, wm, wn, lane);
    }
}

// ── k_gemm_pipe: fragment double buffering over direct-to-LDS stages ────
// The default kernel of the large GEMMs.  Block tile 256 x BN (BN = 192 or
// 256) split over WMW x WNW wave64s.  The default layouts use 8 waves (two
// per SIMD, 64 x 128 / 64 x 96 / 128 x 64 wave tiles, accumulators in VGPRs)
// so that one wave's MFMAs cover the other's LDS and barrier waits; the
// 4-wave layouts (128-row wave tiles, accumulators in AGPRs, one wave per
// SIMD) remain as variants.  The stages are the direct-to-LDS stages of
// k_gemm_dma (32-wide k slices, 4 stages in flight, swizzled rows).  Each
// step of the loop computes one stage in two 16-wide halves: the fragments
// of the second half are read from LDS while the first half's MFMAs run,
// and the fragments of the next stage's first half while the second half's
// run, so LDS latency never sits between two MFMA batches.  One barrier per
// stage, placed between the halves: after it the next stage has landed for
// every wave and the buffer read two stages ago is free for the next DMA.
template <int TM, int TN>
struct Frags {
    bf16x8_t a[TM], b[TN];
};

template <int TM, int TN, int WTM, int WTN, int KD = DBK>
__device__ __forceinline__ void pipe_frags(Frags<TM, TN>& f, const bf16* sX, const bf16* sY,
                                           int wm, int wn, int lane, int kk) {
    const int c = 2 * kk + (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; i++) {
        int R = wm * WTM + i * 32 + (lane & 31);
        f.a[i] = *(const bf16x8_t*)(sX + R * KD + 8 * (c ^ stage_swz<KD>(R)));
    }
#pragma unroll
    for (int j = 0; j < TN; j++) {
        int R = wn * WTN + j * 32 + (lane & 31);
        f.b[j] = *(const bf16x8_t*)(sY + R * KD + 8 * (c ^ stage_swz<KD>(R)));
    }
}

// The accumulators hold the transposed fragments (Y rows as the MFMA's A
// operand): lane l of acc[i][j] has output row 32i + l%32 and columns
// 32j + 8(r/4) + 4(l/32) + r%4, i.e. four consecutive columns per register
// group, which the epilogue packs into 8-byte words.
template <int TM, int TN>
__device__ __forceinline__ void pipe_mma(floatx16 (&acc)[TM][TN], const Frags<TM, TN>& f) {
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[j], f.a[i], acc[i][j], 0, 0, 0);
}

// scheduling hint for the region just emitted: alternate one MFMA with one
// LDS read while reads remain
template <int NM, int ND>
__device__ __forceinline__ void pipe_interleave() {
#pragma unroll
    for (int i = 0; i < NM; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                // MFMA
        if (i < ND) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);    // DS read
    }
}

// compile-time loop: f(integral_constant<0>) ... f(integral_constant<N-1>)
template <int N, typename F>
__device__ __attribute__((always_inline)) inline void static_for(F&& f) {
    if constexpr (N > 0) {
        static_for<N - 1>(f);
        f(std::integral_constant<int, N - 1>{});
    }
}

// Element offset of (row, col) in a wave's 64 x WTN BF16 output staging:
// 16-byte chunks XOR-swizzled by row bits 1..3 (1..2 for WTN = 96 and 32), so the
// 8-byte writes of 32 rows at one column land in distinct banks and every
// 16-byte chunk stays contiguous for the row read-out.
template <int WTN>
__device__ __forceinline__ int stg_off(int row, int col) {
    constexpr int X = (WTN == 96 || WTN == 32) ? 3 : 7;
    return row * WTN + ((((col >> 3) ^ ((row >> 1) & X)) << 3) | (col & 7));
}

// Epilogue of one 64-row half (row fragments I0, I0 + 1) of a wave tile,
// staged in the wave's private LDS region wb (64 x WTN BF16, stg_off
// layout).  Same arithmetic as big_epilogue, fragment by fragment: alpha acc
// + beta C (+ bias) rounded, then each LoRA term (one MFMA k step per 16
// of rank, up to 64; the first step's operand fragments loaded up front,
// the others' from global memory), then the BF16 values into
// wb, four columns per 8-byte write; the half leaves as 16-byte row vectors.
// A lane reads and writes the same wb words for a fragment, so only the
// final read-back needs the wave barrier.
//
// lu/lv/lb (may be null): the block's rank-16 LoRA operands of the first PF
// pairs (U rows, V rows; 16 BF16 per row) and its bias, staged in LDS at the
// start of the kernel; R0 - m0 / C0 - n0 index them.
template <int TM, int TN, int WTN, int I0, int PF>
__device__ __attribute__((always_inline)) inline void pipe_half_epilogue(
    floatx16 (&acc)[TM][TN], const GemmArgs& a, bf16* __restrict__ C, int R0, int C0, int lane,
    bf16* __restrict__ wb, const bf16* lu, const bf16* lv, const bf16* lb, int mloc, int nloc,
    int BMs, int BNs) {
    constexpr int CPR = WTN / 8;
    const bool vec = ((a.ldc & 7) == 0) && (((uintptr_t)C & 15) == 0);
    if (a.beta != 0.f) {
        for (int q = lane; q < 64 * CPR; q += 64) {
            int row = q / CPR, ch = q % CPR;
            int gm = R0 + row, gn = C0 + 8 * ch;
            bf16x8v v;
            if (gm < a.M && vec && gn + 8 <= a.N) {
                v = *(const bf16x8v*)(C + (int64_t)gm * a.ldc + gn);
            } else {
                uint16_t t[8];
#pragma unroll
                for (int e = 0; e < 8; e++)
                    t[e] = (gm < a.M && gn + e < a.N) ? C[(int64_t)gm * a.ldc + gn + e] : (uint16_t)0;
#pragma unroll
                for (int e = 0; e < 4; e++) v.w[e] = (uint32_t)t[2 * e] | ((uint32_t)t[2 * e + 1] << 16);
            }
            *(bf16x8v*)(wb + stg_off<WTN>(row, 8 * ch)) = v;
        }
        __builtin_amdgcn_wave_barrier();
    }
    const int kk = 8 * (lane >> 5);
    const bool kin = kk < a.lora_r;
    bf16x8_t fu[PF][2], fv[PF][TN];
#pragma unroll
    for (int p = 0; p < PF; p++) {
        if (p < a.lora_n && lu) {
#pragma unroll
            for (int i = 0; i < 2; i++)
                fu[p][i] = *(const bf16x8_t*)(lu + (p * BMs + mloc + 32 * i + (lane & 31)) * 16 + kk);
#pragma unroll
            for (int j = 0; j < TN; j++)
                fv[p][j] = *(const bf16x8_t*)(lv + (p * BNs + nloc + 32 * j + (lane & 31)) * 16 + kk);
        } else if (p < a.lora_n) {
#pragma unroll
            for (int i = 0; i < 2; i++) {
                int row = min(R0 + 32 * i + (lane & 31), a.M - 1);
                fu[p][i] = *(const bf16x8_t*)(a.lora_u[p] + (int64_t)row * a.lora_ldu[p] + (kin ? kk : 0));
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                int col = min(C0 + 32 * j + (lane & 31), a.N - 1);
                fv[p][j] = *(const bf16x8_t*)(a.lora_v[p] + (int64_t)col * a.lora_r + (kin ? kk : 0));
            }
            if (!kin) {
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    fu[p][0][e] = fu[p][1][e] = (__bf16)0.f;
#pragma unroll
                    for (int j = 0; j < TN; j++) fv[p][j][e] = (__bf16)0.f;
                }
            }
        }
    }
    const int c4 = 4 * (lane >> 5);  // first of the lane's 4 columns in each 8-column group
    static_for<2 * TN>([&](auto ij) {
        constexpr int i = decltype(ij)::value / TN, j = decltype(ij)::value % TN;
        const int lr = i * 32 + (lane & 31);
        // v[4g + e]: column 32j + 8g + c4 + e of row lr
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; r++) v[r] = a.alpha * acc[I0 + i][j][r];
        if (a.beta != 0.f) {
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint2 cw = *(const uint2*)(wb + stg_off<WTN>(lr, 32 * j + 8 * g + c4));
                v[4 * g] += a.beta * lo2f(cw.x);
                v[4 * g + 1] += a.beta * hi2f(cw.x);
                v[4 * g + 2] += a.beta * lo2f(cw.y);
                v[4 * g + 3] += a.beta * hi2f(cw.y);
            }
        }
        if (a.bias) {
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int lc = 32 * j + 8 * g + c4;
                float bb[4];
                if (lb) {
                    const uint2 bw = *(const uint2*)(lb + nloc + lc);
                    bb[0] = lo2f(bw.x), bb[1] = hi2f(bw.x), bb[2] = lo2f(bw.y), bb[3] = hi2f(bw.y);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) bb[e] = C0 + lc + e < a.N ? bf2f(a.bias[C0 + lc + e]) : 0.f;
                }
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float bias = C0 + lc + e < a.N ? bb[e] : 0.f;
                    v[4 * g + e] = bf2f(f2bf(v[4 * g + e])) + bias;
                }
            }
        }
        if (a.lora_n > 0) {
#pragma unroll
            for (int r = 0; r < 16; r++) v[r] = bf2f(f2bf(v[r]));
        }
#pragma unroll
        for (int p = 0; p < 3; p++) {
            if (p < a.lora_n) {
                floatx16 d;
#pragma unroll
                for (int r = 0; r < 16; r++) d[r] = 0.f;
                bf16x8_t ua, vb;
                if (p < PF) {
                    ua = fu[p < PF ? p : 0][i];
                    vb = fv[p < PF ? p : 0][j];
                } else {
                    const int row = min(R0 + 32 * i + (lane & 31), a.M - 1);
                    const int col = min(C0 + 32 * j + (lane & 31), a.N - 1);
                    ua = *(const bf16x8_t*)(a.lora_u[p] + (int64_t)row * a.lora_ldu[p] + (kin ? kk : 0));
                    vb = *(const bf16x8_t*)(a.lora_v[p] + (int64_t)col * a.lora_r + (kin ? kk : 0));
                    if (!kin) {
#pragma unroll
                        for (int e = 0; e < 8; e++) ua[e] = vb[e] = (__bf16)0.f;
                    }
                }
                // transposed like the accumulators: V rows as the A operand
                d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vb, ua, d, 0, 0, 0);
                // ranks above 16: one more k step per 16, operand rows from
                // global memory (rank k0 + kk .. + 7 of the lane's row/column)
                for (int k0 = 16; k0 < a.lora_r; k0 += 16) {
                    const int row = min(R0 + 32 * i + (lane & 31), a.M - 1);
                    const int col = min(C0 + 32 * j + (lane & 31), a.N - 1);
                    const bool kin2 = k0 + kk < a.lora_r;
                    bf16x8_t u2 = *(const bf16x8_t*)(a.lora_u[p] + (int64_t)row * a.lora_ldu[p] +
                                                     (kin2 ? k0 + kk : 0));
                    bf16x8_t v2 = *(const bf16x8_t*)(a.lora_v[p] + (int64_t)col * a.lora_r +
                                                     (kin2 ? k0 + kk : 0));
                    if (!kin2) {
#pragma unroll
                        for (int e = 0; e < 8; e++) u2[e] = v2[e] = (__bf16)0.f;
                    }
                    d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v2, u2, d, 0, 0, 0);
                }
#pragma unroll
                for (int r = 0; r < 16; r++)
                    v[r] = a.lora_delta ? bf2f(f2bf(v[r] + a.lora_s * bf2f(f2bf(d[r]))))
                                        : bf2f(f2bf(a.lora_s * d[r] + v[r]));
            }
        }
        if (a.rope_tab) {
            // RoPE of the values as written (ops::rope_fwd over the output):
            // the lane's columns d .. d + 3 of a head are pairs d/2, d/2 + 1
            // (d a multiple of 4), position t = row % T
            const int t = (R0 + lr) % a.rope_T;
            const float2* tr = a.rope_tab + (int64_t)t * (a.rope_hd >> 1);
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int d = (C0 + 32 * j + 8 * g + c4) % a.rope_hd;
                const float4 cs = *(const float4*)(tr + (d >> 1));
                const float x0 = bf2f(f2bf(v[4 * g])), x1 = bf2f(f2bf(v[4 * g + 1]));
                const float x2 = bf2f(f2bf(v[4 * g + 2])), x3 = bf2f(f2bf(v[4 * g + 3]));
                rope_rot(x0, x1, cs.x, cs.y, v[4 * g], v[4 * g + 1]);
                rope_rot(x2, x3, cs.z, cs.w, v[4 * g + 2], v[4 * g + 3]);
            }
        }
        // the packing rounds to BF16 (exact when v is a BF16 value already)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            uint2 w;
            w.x = pack2(v[4 * g], v[4 * g + 1]);
            w.y = pack2(v[4 * g + 2], v[4 * g + 3]);
            *(uint2*)(wb + stg_off<WTN>(lr, 32 * j + 8 * g + c4)) = w;
        }
    });
    __builtin_amdgcn_wave_barrier();
    for (int q = lane; q < 64 * CPR; q += 64) {
        int row = q / CPR, ch = q % CPR;
        int gm = R0 + row, gn = C0 + 8 * ch;
        if (gm >= a.M) continue;
        bf16x8v v = *(const bf16x8v*)(wb + stg_off<WTN>(row, 8 * ch));
        if (vec && gn + 8 <= a.N) {
            st_out16(C + (int64_t)gm * a.ldc + gn, v);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++)
                if (gn + e < a.N) C[(int64_t)gm * a.ldc + gn + e] = (uint16_t)(v.w[e >> 1] >> ((e & 1) * 16));
        }
    }
}

// accumulators rounded to BF16 values (the end of one GEMM of a chain)
template <int TM, int TN>
__device__ __forceinline__ void round_acc(floatx16 (&acc)[TM][TN]) {
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = bf2f(f2bf(acc[i][j][r]));
}

// dlogits from the logits of a wave's X fragments (k_gemm_pipe_ce): lane l
// holds 8 consecutive k (columns kb .. kb + 7) of the row whose normaliser
// and target are ls2[i], tg[i]; the same operations as k_cross_entropy_reg,
// so the same bits.  Stages before the first (kt < 0) hold zeros and stay.
template <int TM>
__device__ __forceinline__ void ce_frags(bf16x8_t (&fa)[TM], int kt, int kk, const float (&ls2)[TM],
                                         const int (&tg)[TM], float inv_n, int lane) {
    if (kt < 0) return;
    const int kb = kt * 64 + 16 * kk + 8 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < TM; i++) {
        const u32x4_t w = __builtin_bit_cast(u32x4_t, fa[i]);
        u32x4_t o;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float d[2];
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const float f = h ? hi2f(w[q]) : lo2f(w[q]);
                const float p = __builtin_amdgcn_exp2f(fmaf(f, kLog2e, -ls2[i]));
                d[h] = (p - (float)(kb + 2 * q + h == tg[i])) * inv_n;
            }
            o[q] = pack2(d[0], d[1]);
        }
        fa[i] = __builtin_bit_cast(bf16x8_t, o);
    }
}

// CHAIN: K segments (a.nseg > 1).  SWIGLU: Y is the gate/up weight pair
// interleaved in blocks of 128 rows, so tile tn holds gate and up columns
// [128 tn, 128 tn + 128); gate waves (wn < 2) write gate, up waves up, each
// with its pair's LoRA delta, and then every gate/up wave pair writes
// act = silu(gate) * up from the two staged BF16 halves (gC[0..2] = gate,
// up, act; gu/gv[0..1] the pairs' h and B; gN[0] = gldc[0] = I).
//
// KD: stage depth.  KD = 32: four stages of 32 k (rows of half a line).
// KD = 64: two stages of 64 k in the same LDS, rows of one whole 128-byte
// line, so every line of an operand is fetched once; the next stage's load
// has the same 64 k of compute to land in as with four 32-k stages.
// CEX: X holds logits and the MFMAs take dlogits formed from them (ce_frags).
// PART: split-K, split blockIdx.z over k [z k_per_split, +k_per_split): F32
// partials of the split into part[z][M][N], no epilogue arithmetic.
template <int BN, int WMW, int WNW, bool CHAIN, bool SWIGLU = false, int KD = 32, int BM = 256,
          bool CEX = false, bool PART = false>
__device__ __attribute__((always_inline)) inline void gemm_pipe_body(const GemmArgs& a0) {
    static_assert(!CEX || (KD == 64 && !CHAIN && !SWIGLU), "CE operand form");
    static_assert(!PART || (KD == 64 && !CHAIN && !SWIGLU && !CEX), "split-K partials form");
    static_assert(KD == 32 || KD == 64, "stage depth");
    constexpr int NS = KD == 32 ? 4 : 2, NW = WMW * WNW;
    constexpr int WTM = BM / WMW, WTN = BN / WNW;
    constexpr int TM = WTM / 32, TN = WTN / 32;
    static_assert(TM * 32 == WTM && TN * 32 == WTN && TM % 2 == 0, "wave tile");
    // 128-row tiles: four waves of 64-row wave tiles (k_gemm_mid)
    static_assert(BM == 256 || (BM == 128 && NW == 4 && KD == 64), "tile height");
    static_assert(KD == 32 || NW == 8 || BM == 128, "64-k stages: 8-wave layouts");
    // DMA instructions per stage per wave
    constexpr int RPI = 64 / (KD / 8);  // stage rows per DMA instruction
    constexpr int LPS = (BM / RPI + NW - 1) / NW + (BN / RPI + NW - 1) / NW;
    constexpr int SX = BM * KD, SY = BN * KD;
    static_assert(BN == 192 || BN == 256 || (BM == 128 && (BN == 64 || BN == 128)),
                  "tile width");
    __shared__ __attribute__((aligned(1024))) bf16 sXs[NS][SX];
    __shared__ __attribute__((aligned(1024))) bf16 sYs[NS][SY];
    bf16* const sX0 = sXs[0];
    bf16* const sX1 = sXs[1];
    bf16* const sY0 = sYs[0];
    bf16* const sY1 = sYs[1];
    // epilogue operands staged at the start: rank-16 LoRA U/V rows of the
    // first LP pairs and 512 bias entries (one DMA instruction)
    // (128 x 128 tiles stage one pair, so two blocks fit a CU's LDS)
    constexpr int LP = (BN == 256 || (BM == 128 && BN == 128)) ? 1 : 3;
    constexpr int LPU = SWIGLU ? 2 : LP;  // U rows: both pairs' h in the SwiGLU form
    static_assert(!SWIGLU || (BN == 256 && WNW == 4 && WMW == 2), "SwiGLU tile layout");
    __shared__ __attribute__((aligned(16))) bf16 sLU[LPU * BM * 16], sLV[LP * BN * 16], sB[512];

    int tm_i, tn_i;
    big_tile(blockIdx.x, a0.tiles_m, a0.tiles_n, tm_i, tn_i);
    // N-concatenated groups: this tile's group supplies Y, C, N, bias, LoRA
    GemmArgs a = a0;
    if (a0.ngroups > 1) {
        const int g = (a0.ngroups > 2 && tn_i >= a0.tn0[2]) ? 2 : tn_i >= a0.tn0[1] ? 1 : 0;
        tn_i -= g == 2 ? a0.tn0[2] : g == 1 ? a0.tn0[1] : 0;
        a.N = g == 2 ? a0.gN[2] : g == 1 ? a0.gN[1] : a0.gN[0];
        a.Y = g == 2 ? a0.gY[2] : g == 1 ? a0.gY[1] : a0.gY[0];
        a.C = g == 2 ? a0.gC[2] : g == 1 ? a0.gC[1] : a0.gC[0];
        a.ldc = g == 2 ? a0.gldc[2] : g == 1 ? a0.gldc[1] : a0.gldc[0];
        a.bias = g == 2 ? a0.gbias[2] : g == 1 ? a0.gbias[1] : a0.gbias[0];
        a.lora_n = g == 2 ? a0.glora[2] : g == 1 ? a0.glora[1] : a0.glora[0];
        a.lora_u[0] = g == 2 ? a0.gu[2] : g == 1 ? a0.gu[1] : a0.gu[0];
        a.lora_v[0] = g == 2 ? a0.gv[2] : g == 1 ? a0.gv[1] : a0.gv[0];
        a.rope_tab = g == 2 ? a0.grope[2] : g == 1 ? a0.grope[1] : a0.grope[0];
    }
    if constexpr (PART) {
        // the split's K range is the whole K of operands that start at its
        // first k (both are K-contiguous, k_per_split a multiple of 64)
        const int k0 = blockIdx.z * a0.k_per_split;
        a.X += k0;
        a.Y += k0;
        a.K = min(a0.K - k0, a0.k_per_split);
        a.lora_n = 0;
        a.bias = nullptr;
    }
    const int m0 = tm_i * BM, n0 = tn_i * BN;
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int wm = w / WNW, wn = w % WNW;
    w = __builtin_amdgcn_readfirstlane(w);
    float ce_l2[TM];
    int ce_t[TM];
    if constexpr (CEX) {
#pragma unroll
        for (int i = 0; i < TM; i++) {
            const int row = min(m0 + wm * WTM + i * 32 + (lane & 31), a0.M - 1);
            ce_l2[i] = a0.ce_lse2[row];
            ce_t[i] = a0.ce_tgt[row];
        }
    }
#define PIPE_CE(F, KT, KK)                                                       \
    do {                                                                         \
        if constexpr (CEX) ce_frags<TM>((F).a, (KT), (KK), ce_l2, ce_t, a0.ce_inv_n, lane); \
    } while (0)

    // these loads are older than every stage load, so the prologue's wait
    // for stage 0 covers them; the main loop's barriers publish them
    const bool lds_lora = a.lora_n > 0 && a.lora_r == 16;
    const bool lds_bias = a.bias != nullptr && (a.N & 7) == 0 && a.N >= 8;
    if (SWIGLU && lds_lora) {
        // U: gate then up h rows of the tile; V: gate B rows of columns
        // [128 tn, +128) then the up pair's (instruction q: 32 rows x 32 B)
        constexpr int UI = BM / 32, VI = BN / 32;
        const int cb = 128 * tn_i;
        for (int q = w; q < 2 * UI + VI; q += NW) {
            const bf16* src;
            bf16* dst;
            if (q < 2 * UI) {
                const int pp = q / UI, qi = q % UI;
                const int row = min(m0 + 32 * qi + (lane >> 1), a.M - 1);
                src = (pp ? a0.gu[1] : a0.gu[0]) + (int64_t)row * 16 + 8 * (lane & 1);
                dst = sLU + (pp * BM + 32 * qi) * 16;
            } else {
                const int qi = q - 2 * UI, r = 32 * qi + (lane >> 1);
                src = (qi < VI / 2 ? a0.gv[0] : a0.gv[1]) + (int64_t)(cb + (r & 127)) * 16 +
                      8 * (lane & 1);
                dst = sLV + 32 * qi * 16;
            }
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)dst, 16, 0, 0);
        }
    } else if (lds_lora) {
        // instruction q moves 32 rows x 32 bytes: lane l -> row l/2, half l%2
        constexpr int UI = BM / 32, VI = BN / 32;
        for (int q = w; q < LP * (UI + VI); q += NW) {
            const int p = q / (UI + VI), qi = q % (UI + VI);
            if (p >= a.lora_n) break;
            const bf16* u = p == 0 ? a.lora_u[0] : p == 1 ? a.lora_u[1] : a.lora_u[2];
            const bf16* v = p == 0 ? a.lora_v[0] : p == 1 ? a.lora_v[1] : a.lora_v[2];
            const int64_t ldu = p == 0 ? a.lora_ldu[0] : p == 1 ? a.lora_ldu[1] : a.lora_ldu[2];
            const bf16* src;
            bf16* dst;
            if (qi < UI) {
                const int row = min(m0 + 32 * qi + (lane >> 1), a.M - 1);
                src = u + (int64_t)row * ldu + 8 * (lane & 1);
                dst = sLU + (p * BM + 32 * qi) * 16;
            } else {
                const int row = min(n0 + 32 * (qi - UI) + (lane >> 1), a.N - 1);
                src = v + (int64_t)row * 16 + 8 * (lane & 1);
                dst = sLV + (p * BN + 32 * (qi - UI)) * 16;
            }
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)dst, 16, 0, 0);
        }
    }
    if (lds_bias && w == NW - 1) {
        const bf16* src = a.bias + min(n0 + 8 * lane, a.N - 8);
        __builtin_amdgcn_global_load_lds((const void*)src, (lds_ptr_t)sB, 16, 0, 0);
    }

    floatx16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    // K runs as stages kt = -pad .. nk-1 (pad zero stages make the count a
    // multiple of NS; stages past the end reload the last one into a buffer
    // that is never read), as in k_gemm_dma
    const int nk = a.K / KD;
    const int pad = (NS - nk % NS) % NS;
    // K segments: stage kt (global k) belongs to segment s; the accumulators
    // are rounded after the last stage of every segment but the last
    const int kb1 = CHAIN ? a.kseg[1] / KD : -99, kb2 = CHAIN && a.nseg > 2 ? a.kseg[2] / KD : -99;
    DmaOffs<BM, NW, KD> ox0, ox1, ox2;
    DmaOffs<BN, NW, KD> oy0, oy1, oy2;
    if constexpr (CHAIN) {
        dma_offsets<BM, NW>(ox0, a.sldx[0], m0, a.M, w, lane);
        dma_offsets<BN, NW>(oy0, a.sldy[0], n0, a.N, w, lane);
        dma_offsets<BM, NW>(ox1, a.sldx[1], m0, a.M, w, lane);
        dma_offsets<BN, NW>(oy1, a.sldy[1], n0, a.N, w, lane);
        dma_offsets<BM, NW>(ox2, a.nseg > 2 ? a.sldx[2] : 0, m0, a.M, w, lane);
        dma_offsets<BN, NW>(oy2, a.nseg > 2 ? a.sldy[2] : 0, n0, a.N, w, lane);
    }
    // each segment's operands at the tile's first row (wave-uniform)
    const bf16* xt0 = CHAIN ? a.sX[0] + (int64_t)m0 * a.sldx[0] : nullptr;
    const bf16* xt1 = CHAIN ? a.sX[1] + (int64_t)m0 * a.sldx[1] : nullptr;
    const bf16* xt2 = CHAIN && a.nseg > 2 ? a.sX[2] + (int64_t)m0 * a.sldx[2] : nullptr;
    const bf16* yt0 = CHAIN ? a.sY[0] + (int64_t)n0 * a.sldy[0] : nullptr;
    const bf16* yt1 = CHAIN ? a.sY[1] + (int64_t)n0 * a.sldy[1] : nullptr;
    const bf16* yt2 = CHAIN && a.nseg > 2 ? a.sY[2] + (int64_t)n0 * a.sldy[2] : nullptr;
#define PIPE_ISSUE_P(SXB, SYB, KT, DOX, DOY)                                                        \
    do {                                                                                   \
        const int kq_ = (KT);                                                              \
        const bool z_ = kq_ < 0;                                                           \
        int k_ = z_ ? 0 : min(kq_, nk - 1) * KD;                                           \
        const bf16* x_ = a.X;                                                              \
        const bf16* y_ = a.Y;                                                              \
        int64_t lx_ = a.ldx, ly_ = a.ldy;                                                  \
        if constexpr (CHAIN) {                                                             \
            /* the segment's precomputed row offsets: no per-stage multiply */             \
            const int s_ = (a.nseg > 2 && k_ >= a.kseg[2]) ? 2 : k_ >= a.kseg[1] ? 1 : 0;  \
            x_ = s_ == 2 ? xt2 : s_ == 1 ? xt1 : xt0;                                      \
            y_ = s_ == 2 ? yt2 : s_ == 1 ? yt1 : yt0;                                      \
            k_ -= s_ == 2 ? a.kseg[2] : s_ == 1 ? a.kseg[1] : 0;                           \
            if (z_) {                                                                      \
                if (DOX) dma_stage<BM, NW, KD>(g_dma_zero, 0, m0, a.M, 0, SXB, w, lane);            \
                if (DOY) dma_stage<BN, NW, KD>(g_dma_zero, 0, n0, a.N, 0, SYB, w, lane);            \
            } else {                                                                       \
                if (DOX) dma_stage_at<BM, NW, KD>(x_ + k_, s_ == 2 ? ox2 : s_ == 1 ? ox1 : ox0, SXB, \
                                         w);                                               \
                if (DOY) dma_stage_at<BN, NW, KD>(y_ + k_, s_ == 2 ? oy2 : s_ == 1 ? oy1 : oy0, SYB, \
                                         w);                                               \
            }                                                                              \
        } else {                                                                           \
            if (DOX) dma_stage<BM, NW, KD>(z_ ? g_dma_zero : x_, z_ ? 0 : lx_, m0, a.M, k_, SXB, w, \
                                  lane);                                                   \
            if (DOY) dma_stage<BN, NW, KD>(z_ ? g_dma_zero : y_, z_ ? 0 : ly_, n0, a.N, k_, SYB, w, \
                                  lane);                                                   \
        }                                                                                  \
    } while (0)
#define PIPE_ISSUE(SXB, SYB, KT) PIPE_ISSUE_P(SXB, SYB, KT, true, true)
// (chains start every segment on a loop trip of NS stages, which the host
// checks, so the rounding test sits between trips and the NS steps of a
// trip stay one straight-line region)
#define PIPE_ROUND(KT)                                                                     \
    do {                                                                                   \
        if constexpr (CHAIN)                                                               \
            if ((KT) + 1 == kb1 || (KT) + 1 == kb2) round_acc<TM, TN>(acc);                \
    } while (0)
    Frags<TM, TN> f0, f1;
    if constexpr (KD == 32) {
    bf16* const sX2 = sXs[2];
    bf16* const sX3 = sXs[3];
    bf16* const sY2 = sYs[2];
    bf16* const sY3 = sYs[3];
    PIPE_ISSUE(sX0, sY0, 0 - pad);
    PIPE_ISSUE(sX1, sY1, 1 - pad);
    PIPE_ISSUE(sX2, sY2, 2 - pad);
    TA_WAIT_VMCNT(LPS * (NS - 2));
    __builtin_amdgcn_s_barrier();
    pipe_frags<TM, TN, WTM, WTN>(f0, sX0, sY0, wm, wn, lane, 0);
    // step J: second-half fragments of stage J while the first half
    // computes; wait for stage J+1 (NS - 3 stages may stay in flight);
    // barrier; refill the buffer of stage J-1 with stage J+NS-1; first-half
    // fragments of stage J+1 while the second half computes
#define PIPE_STEP(J, SXJ, SYJ, SXN, SYN, SXR, SYR)                                         \
    do {                                                                                   \
        pipe_frags<TM, TN, WTM, WTN>(f1, SXJ, SYJ, wm, wn, lane, 1);                       \
        pipe_mma<TM, TN>(acc, f0);                                                         \
        pipe_interleave<TM * TN, TM + TN>();                                               \
        TA_WAIT_VMCNT(LPS * (NS - 3));                                                     \
        __builtin_amdgcn_s_barrier();                                                      \
        PIPE_ISSUE(SXR, SYR, kt0 + (J) + NS - 1);                                          \
        pipe_frags<TM, TN, WTM, WTN>(f0, SXN, SYN, wm, wn, lane, 0);                       \
        pipe_mma<TM, TN>(acc, f1);                                                         \
        pipe_interleave<TM * TN, TM + TN>();                                               \
    } while (0)
    for (int kt0 = -pad; kt0 < nk; kt0 += NS) {
        PIPE_STEP(0, sX0, sY0, sX1, sY1, sX3, sY3);
        PIPE_STEP(1, sX1, sY1, sX2, sY2, sX0, sY0);
        PIPE_STEP(2, sX2, sY2, sX3, sY3, sX1, sY1);
        PIPE_STEP(3, sX3, sY3, sX0, sY0, sX2, sY2);
        PIPE_ROUND(kt0 + 3);
    }
#undef PIPE_STEP
    } else {
    // 64-k stages: step J computes stage J (k steps 0..3) from buffer J % 2;
    // its k step 3 fragments are read before the barrier that frees the
    // buffer for stage J + 2 (waited for: the DMA must not overwrite them),
    // after which the next stage's first fragments are read while k step 3
    // computes.  The only loads in flight at a step's wait are stage J + 1's.
    // Every wave issues the X share of stage J + 2 right after the barrier
    // that frees the buffer and the Y share after the step's last MFMA batch
    // (stages past the last are not loaded; every step's wait is for all
    // loads in flight): the split keeps a wave from stalling at the issue
    // of all its loads behind the other waves' before its MFMAs (c3 step
    // -0.8% against issuing both shares at the barrier).  With the loads issued from
    // inline assembly (dma16) nothing else waits for them, so the wave goes
    // on to its MFMAs while the address unit works through the stage; with
    // the compiler's own form every LDS read after an issue waited for all
    // loads in flight, and staggering the issue across the wave halves was
    // needed to keep the matrix cores busy (4% slower per c3 step than this).
    PIPE_ISSUE(sX0, sY0, 0 - pad);
    PIPE_ISSUE(sX1, sY1, 1 - pad);
    TA_WAIT_VMCNT(LPS);
    __builtin_amdgcn_s_barrier();
    pipe_frags<TM, TN, WTM, WTN, KD>(f0, sX0, sY0, wm, wn, lane, 0);
    PIPE_CE(f0, -pad, 0);
#define PIPE_STEP(J, SXJ, SYJ, SXN, SYN)                                                   \
    do {                                                                                   \
        pipe_frags<TM, TN, WTM, WTN, KD>(f1, SXJ, SYJ, wm, wn, lane, 1);                   \
        PIPE_CE(f1, kt0 + (J), 1);                                                         \
        pipe_mma<TM, TN>(acc, f0);                                                         \
        pipe_interleave<TM * TN, TM + TN>();                                               \
        pipe_frags<TM, TN, WTM, WTN, KD>(f0, SXJ, SYJ, wm, wn, lane, 2);                   \
        PIPE_CE(f0, kt0 + (J), 2);                                                         \
        pipe_mma<TM, TN>(acc, f1);                                                         \
        pipe_interleave<TM * TN, TM + TN>();                                               \
        pipe_frags<TM, TN, WTM, WTN, KD>(f1, SXJ, SYJ, wm, wn, lane, 3);                   \
        PIPE_CE(f1, kt0 + (J), 3);                                                         \
        pipe_mma<TM, TN>(acc, f0);                                                         \
        pipe_interleave<TM * TN, TM + TN>();                                               \
        __builtin_amdgcn_s_waitcnt(0x0070); /* vmcnt(0) lgkmcnt(0) */                      \
        __builtin_amdgcn_s_barrier();                                                      \
        if (kt0 + (J) + 2 < nk) PIPE_ISSUE_P(SXJ, SYJ, kt0 + (J) + 2, true, false);        \
        pipe_frags<TM, TN, WTM, WTN, KD>(f0, SXN, SYN, wm, wn, lane, 0);                   \
        PIPE_CE(f0, kt0 + (J) + 1, 0);                                                     \
        pipe_mma<TM, TN>(acc, f1);                                                         \
        pipe_interleave<TM * TN, TM + TN>();                                               \
        if (kt0 + (J) + 2 < nk) PIPE_ISSUE_P(SXJ, SYJ, kt0 + (J) + 2, false, true);        \
    } while (0)
    for (int kt0 = -pad; kt0 < nk; kt0 += NS) {
        PIPE_STEP(0, sX0, sY0, sX1, sY1);
        PIPE_STEP(1, sX1, sY1, sX0, sY0);
        PIPE_ROUND(kt0 + 1);
    }
#undef PIPE_STEP
    }
    TA_WAIT_VMCNT(0);  // the surplus loads have landed before the buffers are reused
    if constexpr (PART) {
        // F32 partials through LDS, 32 rows of the wave tile at a time: lane
        // l of acc[i][j] holds row 32i + l%32, columns 32j + 8g + 4(l/32) + e
        // (register 4g + e); written as [32][WTN + 4] F32 into a wave-private
        // region of the stage buffers (free after the main loop), read back
        // as 16-byte row runs, so each global store covers whole row segments
        constexpr int LDW = WTN + 4, RB = 32 * LDW * 4;  // region bytes per wave
        constexpr int NXR = (int)sizeof(sXs) / RB;        // regions in the X buffers
        static_assert(NXR + (int)sizeof(sYs) / RB >= NW, "partial staging fits the stage buffers");
        __syncthreads();  // every wave is done with the stage buffers
        float* const st = (float*)(w < NXR ? (char*)&sXs[0][0] + w * RB
                                           : (char*)&sYs[0][0] + (w - NXR) * RB);
        float* const P = a0.part + (int64_t)blockIdx.z * a0.M * a0.N;
        const bool v4 = (a0.N & 3) == 0;
#pragma unroll
        for (int i = 0; i < TM; i++) {
#pragma unroll
            for (int j = 0; j < TN; j++)
#pragma unroll
                for (int g = 0; g < 4; g++)
                    *(float4*)(st + (lane & 31) * LDW + 32 * j + 8 * g + 4 * (lane >> 5)) =
                        make_float4(acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2],
                                    acc[i][j][4 * g + 3]);
            // one wave's LDS accesses execute in order
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
            __builtin_amdgcn_wave_barrier();
            const int r0 = m0 + wm * WTM + 32 * i, c0 = n0 + wn * WTN;
            for (int q = lane; q < 32 * (WTN / 4); q += 64) {
                const int rr = q / (WTN / 4), cc = 4 * (q % (WTN / 4));
                const int row = r0 + rr, col = c0 + cc;
                if (row >= a0.M) continue;
                const float4 v = *(const float4*)(st + rr * LDW + cc);
                float* d = P + (int64_t)row * a0.N + col;
                if (v4 && col + 3 < a0.N) {
                    *(float4*)d = v;
                } else {
                    const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (col + e < a0.N) d[e] = vv[e];
                }
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // the reads are done before the next chunk's writes
            __builtin_amdgcn_wave_barrier();
        }
        return;
    }
#undef PIPE_CE
#undef PIPE_ROUND
#undef PIPE_ISSUE
#undef PIPE_ISSUE_P
    __syncthreads();
    // each wave stages its 64-row halves in LDS of its own: the 4-wave
    // layouts use one X and one Y stage buffer per wave, the 8-wave layouts
    // one stage buffer per wave (split in two when it holds two halves)
    const bf16* lu = lds_lora ? sLU : nullptr;
    const bf16* lv = lds_lora ? sLV : nullptr;
    const bf16* lb = lds_bias ? sB : nullptr;
    // (64-k stages: two waves per stage buffer)
    auto wave_stage = [&](int v) -> bf16* {
        if constexpr (KD == 32) {
            return v == 0 ? sXs[0] : v == 1 ? sXs[1] : v == 2 ? sXs[2] : v == 3 ? sXs[3]
                 : v == 4 ? sYs[0] : v == 5 ? sYs[1] : v == 6 ? sYs[2] : sYs[3];
        } else {
            static_assert(2 * 64 * WTN * (TM / 2) <= SY, "staging fits half a stage buffer");
            bf16* b = (v >> 1) == 0 ? sXs[0] : (v >> 1) == 1 ? sXs[1] : (v >> 1) == 2 ? sYs[0] : sYs[1];
            return b + (v & 1) * (64 * WTN * (TM / 2));
        }
    };
    bf16 *wb0, *wb1;
    if constexpr (BM == 128) {
        // one 64-row half per wave (TM = 2), the four regions side by side
        // over the two X stage buffers
        static_assert(TM == 2 && 4 * 64 * WTN <= NS * SX, "staging fits the X stages");
        wb0 = &sXs[0][0] + w * 64 * WTN;
        wb1 = wb0;
    } else if constexpr (NW == 4) {
        wb0 = sXs[w];
        wb1 = sYs[w];
        static_assert(64 * WTN <= SX && 64 * WTN <= SY, "staging fits a stage buffer");
    } else {
        bf16* b = wave_stage(w);
        static_assert(64 * WTN * (TM / 2) <= SY, "staging fits a stage buffer");
        wb0 = b;
        wb1 = b + 64 * WTN;
    }
    if constexpr (SWIGLU) {
        // gate waves write gate, up waves up (I columns, row stride I), each
        // with its own pair's h rows
        const bool upw = wn >= 2;
        GemmArgs ae = a;
        ae.N = a0.gN[0];
        ae.ldc = a0.gldc[0];
        // (ranks other than 16 read the wave's pair from global memory)
        ae.lora_u[0] = upw ? a0.gu[1] : a0.gu[0];
        ae.lora_v[0] = upw ? a0.gv[1] : a0.gv[0];
        bf16* Cw = (bf16*)(upw ? a0.gC[1] : a0.gC[0]);
        const int cg = 128 * tn_i + 64 * (wn & 1);
        const bf16* luw = lu ? lu + (upw ? BM * 16 : 0) : nullptr;
        pipe_half_epilogue<TM, TN, WTN, 0, LP>(acc, ae, Cw, m0 + wm * WTM, cg, lane, wb0, luw, lv,
                                               nullptr, wm * WTM, wn * WTN, BM, BN);
        pipe_half_epilogue<TM, TN, WTN, 2, LP>(acc, ae, Cw, m0 + wm * WTM + 64, cg, lane, wb1, luw,
                                               lv, nullptr, wm * WTM + 64, wn * WTN, BM, BN);
        __syncthreads();  // the partner wave's halves are staged
        // act = silu(gate) * up: the gate wave takes the first 64 rows, the
        // up wave (w ^ 2) the second, each from both waves' staging
        bf16* pb = wave_stage(w ^ 2);
        const bf16* gst = upw ? pb + 64 * WTN : wb0;
        const bf16* ust = upw ? wb1 : pb;
        const int rb = m0 + wm * WTM + (upw ? 64 : 0);
        bf16* actp = (bf16*)a0.gC[2];
        const int64_t I = a0.gldc[0];
        for (int q = lane; q < 64 * (WTN / 8); q += 64) {
            const int row = q / (WTN / 8), ch = q % (WTN / 8);
            if (rb + row >= a.M) continue;
            float g[8], u[8], o[8];
            unpack8(*(const bf16x8v*)(gst + stg_off<WTN>(row, 8 * ch)), g);
            unpack8(*(const bf16x8v*)(ust + stg_off<WTN>(row, 8 * ch)), u);
#pragma unroll
            for (int e = 0; e < 8; e++) o[e] = silu_mul_f(g[e], u[e]);
            st_out16(actp + (int64_t)(rb + row) * I + cg + 8 * ch, pack8(o));
        }
    } else {
        pipe_half_epilogue<TM, TN, WTN, 0, LP>(acc, a, (bf16*)a.C, m0 + wm * WTM, n0 + wn * WTN,
                                               lane, wb0, lu, lv, lb, wm * WTM, wn * WTN, BM, BN);
        if constexpr (TM == 4)
            pipe_half_epilogue<TM, TN, WTN, 2, LP>(acc, a, (bf16*)a.C, m0 + wm * WTM + 64,
                                                   n0 + wn * WTN, lane, wb1, lu, lv, lb,
                                                   wm * WTM + 64, wn * WTN, BM, BN);
    }
}

template <int BN, int WMW, int WNW, int KD = 32>
__global__ __launch_bounds__(WMW * WNW * 64) __attribute__((amdgpu_waves_per_eu(
    WMW * WNW / 4, WMW * WNW / 4))) void k_gemm_pipe(GemmArgs a) {
    gemm_pipe_body<BN, WMW, WNW, false, false, KD>(a);
}
template <int BN, int WMW, int WNW, int KD = 32>
__global__ __launch_bounds__(WMW * WNW * 64) __attribute__((amdgpu_waves_per_eu(
    WMW * WNW / 4, WMW * WNW / 4))) void k_gemm_pipe_chain(GemmArgs a) {
    gemm_pipe_body<BN, WMW, WNW, true, false, KD>(a);
}
template <int BN, int WMW, int WNW, int KD = 32>
__global__ __launch_bounds__(WMW * WNW * 64) __attribute__((amdgpu_waves_per_eu(
    WMW * WNW / 4, WMW * WNW / 4))) void k_gemm_pipe_swiglu(GemmArgs a) {
    gemm_pipe_body<BN, WMW, WNW, false, true, KD>(a);
}
// split-K F32 partials (grid z = splits), reduced by k_splitk_reduce
template <int BN, int WMW, int WNW>
__global__ __launch_bounds__(WMW * WNW * 64) __attribute__((amdgpu_waves_per_eu(
    WMW * WNW / 4, WMW * WNW / 4))) void k_gemm_pipe_part(GemmArgs a) {
    gemm_pipe_body<BN, WMW, WNW, false, false, 64, 256, false, true>(a);
}
// The LM head's input gradient with the cross-entropy gradient formed in the
// operand reads (gemm_ce_dx).
template <int BN, int WMW, int WNW>
__global__ __launch_bounds__(WMW * WNW * 64) __attribute__((amdgpu_waves_per_eu(
    WMW * WNW / 4, WMW * WNW / 4))) void k_gemm_pipe_ce(GemmArgs a) {
    gemm_pipe_body<BN, WMW, WNW, false, false, 64, 256, true>(a);
}
// 128-row tiles (128 x BN, BN = 64 or 128; four waves of 64-row wave tiles,
// two 64-k stages): the same pipeline and epilogue for outputs too small to
// fill the chip with 256-row tiles (the Qwen2-0.5B shapes at B x T = 2048).
template <int BN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_mid(
    GemmArgs a) {
    gemm_pipe_body<BN, 2, 2, false, false, 64, 128>(a);
}
template <int BN>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_mid_chain(
    GemmArgs a) {
    gemm_pipe_body<BN, 2, 2, true, false, 64, 128>(a);
}

// Kernel variants of the large GEMMs (ta_gemm_rm_variant): 0 picks k_gemm_pipe
// with 8 waves and 64-k stages (256 x 192 tiles in a 4 x 2 wave layout up
// to N = 3072, 256 x 256 in a 2 x 4 layout above; N = 1536 then gives one
// block per CU at M = 8192): variants 17 and 18.  7..11 are k_gemm_dma
// shapes kept for sweeps and for the split-K partials; 12..16 force one
// k_gemm_pipe shape with 32-k stages (15, 16: the 32-k forms of 17, 18).
// 19 and 20 force k_gemm_mid with 128- and 64-wide tiles.
// The variant in force: 0 except inside a ta_gemm_rm_variant call on this
// thread, so no caller's GEMMs change kernel because of another's sweep;
// g_force_splits likewise (0: the dispatch's own split-K choice).
static thread_local int g_big_variant = 0;
static thread_local int g_force_splits = 0;
static bool variant_ok(int v) { return v == 0 || (v >= 7 && v <= 20); }
static bool is_pipe(int variant) { return variant >= 12 && variant <= 18; }
static int big_bn(int variant) {
    return (variant == 8 || variant == 10 || variant == 13 || variant == 14 || variant == 16 ||
            variant == 18)
               ? 256
               : 192;
}
// stage depth of a pipe variant (17, 18: the 64-k forms of 15, 16)
static int pipe_kd(int variant) { return variant >= 17 ? 64 : 32; }

// symbol of the unsplit BF16-output instance of each variant, as printed
// by the profiler
static const char* big_name(int variant) {
    switch (variant) {
        case 7: return "void ta::k_gemm_dma<192, 0, 4, 4, 2>(ta::GemmArgs)";
        case 8: return "void ta::k_gemm_dma<256, 0, 4, 4, 2>(ta::GemmArgs)";
        case 9: return "void ta::k_gemm_dma<192, 0, 5, 4, 2>(ta::GemmArgs)";
        case 10: return "void ta::k_gemm_dma<256, 0, 4, 2, 2>(ta::GemmArgs)";
        case 11: return "void ta::k_gemm_dma<192, 0, 4, 2, 2>(ta::GemmArgs)";
        case 13: return "void ta::k_gemm_pipe<256, 2, 2>(ta::GemmArgs)";
        case 14: return "void ta::k_gemm_pipe<256, 4, 2>(ta::GemmArgs)";
        case 15: return "void ta::k_gemm_pipe<192, 4, 2>(ta::GemmArgs)";
        case 16: return "void ta::k_gemm_pipe<256, 2, 4>(ta::GemmArgs)";
        case 17: return "void ta::k_gemm_pipe<192, 4, 2, 64>(ta::GemmArgs)";
        case 18: return "void ta::k_gemm_pipe<256, 2, 4, 64>(ta::GemmArgs)";
        default: return "void ta::k_gemm_pipe<192, 2, 2>(ta::GemmArgs)";
    }
}

template <int EPI>
static void launch_big(int variant, dim3 grid, const GemmArgs& a, hipStream_t s) {
    switch (variant) {
        case 8: tlaunch(k_gemm_dma<256, EPI, 4, 4, 2>, dim3(grid), dim3(512), s, a); break;
        case 9: tlaunch(k_gemm_dma<192, EPI, 5, 4, 2>, dim3(grid), dim3(512), s, a); break;
        case 10: tlaunch(k_gemm_dma<256, EPI, 4, 2, 2>, dim3(grid), dim3(256), s, a); break;
        case 11: tlaunch(k_gemm_dma<192, EPI, 4, 2, 2>, dim3(grid), dim3(256), s, a); break;
        default: tlaunch(k_gemm_dma<192, EPI, 4, 4, 2>, dim3(grid), dim3(512), s, a); break;
    }
}

// Split-K reduction: sum partials in split order, then the BF16 or F32
// epilogue.
template <bool OUT_BF16>
__global__ void k_splitk_reduce(const float* __restrict__ part, int splits, int M, int N,
                                void* __restrict__ Cv, int64_t ldc, float alpha, float beta,
                                const bf16* __restrict__ bias) {
    int64_t idx = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    int64_t MN = (int64_t)M * N;
    if (idx >= MN) return;
    float s = sum_splits(part, splits, MN, idx);
    int m = (int)(idx / N), n = (int)(idx % N);
    if (OUT_BF16) {
        bf16* C = (bf16*)Cv + (int64_t)m * ldc + n;
        float o = alpha * s;
        if (beta != 0.f) o += beta * bf2f(*C);
        if (bias) o = bf2f(f2bf(o)) + bf2f(bias[n]);
        *C = f2bf(o);
    } else {
        float* C = (float*)Cv + (int64_t)m * ldc + n;
        float o = alpha * s;
        if (beta != 0.f) o += beta * (*C);
        *C = o;
    }
}

template <int BM, int BN, int WM, int WN, int EPI>
static void launch_cfg(bool xk, bool yk, const GemmArgs& a, int splits, bool vx, bool vy,
                       hipStream_t s) {
    dim3 grid(a.tiles_m * a.tiles_n, 1, splits);
    if (xk && yk)
        tlaunch(k_gemm<BM, BN, WM, WN, true, true, EPI>, dim3(grid), dim3(256), s, a, vx, vy);
    else if (xk && !yk)
        tlaunch(k_gemm<BM, BN, WM, WN, true, false, EPI>, dim3(grid), dim3(256), s, a, vx, vy);
    else if (!xk && yk)
        tlaunch(k_gemm<BM, BN, WM, WN, false, true, EPI>, dim3(grid), dim3(256), s, a, vx, vy);
    else
        tlaunch(k_gemm<BM, BN, WM, WN, false, false, EPI>, dim3(grid), dim3(256), s, a, vx, vy);
}

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }
// row stride limit of the direct-to-LDS kernels: 256 rows of an operand
// must span less than 4 GB (32-bit byte offsets from the tile's first row)
constexpr int64_t kMaxStageLd = int64_t(1) << 23;

// Tile width of k_gemm_mid for an M x N output (0: the 256-row kernels).
// The 256-row tiles stay while they fill most of the chip (big_ok: that
// kernel can take the shape), and for long K (32 or more 64-k stages),
// where they run split-K: 128-row tiles reread each operand band twice as
// often, and at Qwen2-0.5B's K = 4864 .. 151936 the small tiles were bound
// by those rereads (measured 1.0-2.9x slower than 256-row split-K).
// Otherwise the 64-wide tiles while two blocks per CU hold them all (they
// measured fastest at M = 2048, N = 896 .. 1152, K <= 1152), then the
// 128-wide ones.  n_mult: every N (of every group) must be a multiple of
// the width.
static int mid_bn(int M, int N, int BNb, int ksteps, bool big_ok, int n_mult) {
    if (M < 128 || N < 64) return 0;
    const int big_tiles = ((M + 255) / 256) * ((N + BNb - 1) / BNb);
    if (big_ok && big_tiles >= 192) return 0;
    if (ksteps >= 32 && M >= 256 && N >= 128) return 0;
    const int t64 = ((M + 127) / 128) * ((N + 63) / 64);
    const int t128 = ((M + 127) / 128) * ((N + 127) / 128);
    if (n_mult % 64 == 0 && t64 <= 512) return 64;
    if (n_mult % 128 == 0 && t128 <= 512) return 128;
    if (big_ok) return 0;
    return n_mult % 128 == 0 ? 128 : n_mult % 64 == 0 ? 64 : 0;
}
static const char* mid_name(int bn, bool chain) {
    if (chain)
        return bn == 128 ? "void ta::k_gemm_mid_chain<128>(ta::GemmArgs)"
                         : "void ta::k_gemm_mid_chain<64>(ta::GemmArgs)";
    return bn == 128 ? "void ta::k_gemm_mid<128>(ta::GemmArgs)"
                     : "void ta::k_gemm_mid<64>(ta::GemmArgs)";
}

// Shape-driven dispatch.  out_f32: C is F32 (gemm_f32 semantics).  lora
// (may be NULL): rank-r terms applied to C after the base epilogue, fused
// into the large-GEMM kernel's epilogue when that kernel runs unsplit and
// applied by k_rank_update right after the GEMM otherwise.
int gemm_dispatch(bool xk, bool yk, int M, int N, int K, float alpha, const bf16* X, int64_t ldx,
                  const bf16* Y, int64_t ldy, float beta, void* C, int64_t ldc, const bf16* bias,
                  bool out_f32, hipStream_t s, int force_splits, const LoraEpi* lora) {
    GemmArgs a{};
    a.M = M;
    a.N = N;
    a.K = K;
    a.X = X;
    a.ldx = ldx;
    a.Y = Y;
    a.ldy = ldy;
    a.C = C;
    a.ldc = ldc;
    a.alpha = alpha;
    a.beta = beta;
    a.bias = bias;
    a.part = nullptr;
    a.lora_n = 0;
    a.lora_r = 0;
    a.lora_delta = 0;
    a.lora_s = 0.f;
    for (int p = 0; p < 3; p++) {
        a.lora_u[p] = a.lora_v[p] = nullptr;
        a.lora_ldu[p] = 0;
    }
    a.ngroups = 1;
    a.nseg = 1;
    if (lora && lora->n > 0) {
        if (out_f32 || lora->n > 3 || (lora->r & 7) != 0)
            return set_error(-1, "gemm: unsupported LoRA epilogue (n=%d r=%d)", lora->n, lora->r);
    }
    // runs the LoRA terms as a separate pass when the kernel did not fuse them
    auto lora_after = [&]() -> int {
        if (!lora || lora->n == 0) return 0;
        return lora_rank_update(lora->delta, (bf16*)C, ldc, M, N, lora->r, lora->s, lora->u,
                                lora->ldu, lora->v_alt, lora->n, s);
    };
    bool vx = al16(X) && (ldx % 8) == 0;
    bool vy = al16(Y) && (ldy % 8) == 0;

    // K-contiguous BF16 GEMMs too small to fill the chip with 256-row tiles:
    // k_gemm_mid (128-row tiles, LoRA terms in the epilogue)
    const bool pipe_ok = xk && yk && !out_f32 && (K % BK) == 0 && vx && vy &&
                         ldx < kMaxStageLd && ldy < kMaxStageLd;
    if (pipe_ok && ((g_big_variant == 0 && force_splits <= 0 && g_force_splits == 0) ||
                    g_big_variant == 19 || g_big_variant == 20)) {
        const bool big_ok = M >= 1024 && N >= 1024;
        const int bn = g_big_variant == 19   ? 128
                       : g_big_variant == 20 ? 64
                                             : mid_bn(M, N, N > 3072 ? 256 : 192, K / BK, big_ok, 128);
        if (bn) {
            a.tiles_m = (M + 127) / 128;
            a.tiles_n = (N + bn - 1) / bn;
            a.k_per_split = K;
            if (lora && lora->n > 0) {
                a.lora_n = lora->n;
                a.lora_r = lora->r;
                a.lora_delta = lora->delta ? 1 : 0;
                a.lora_s = lora->s;
                for (int p = 0; p < lora->n; p++) {
                    a.lora_u[p] = lora->u[p];
                    a.lora_ldu[p] = lora->ldu[p];
                    a.lora_v[p] = lora->v_nk[p];
                }
            }
            const bool timed = kprof_begin(KP_GEMM_BIG, s);
            dim3 grid(a.tiles_m * a.tiles_n);
            if (bn == 128)
                tlaunch(k_gemm_mid<128>, dim3(grid), dim3(256), s, a);
            else
                tlaunch(k_gemm_mid<64>, dim3(grid), dim3(256), s, a);
            if (timed) {
                double mn = (double)M * N;
                double fl = 2.0 * mn * K + 2.0 * mn * a.lora_r * a.lora_n;
                double by = 2.0 * ((double)M * K + (double)N * K + mn * (beta != 0.f ? 2 : 1)) +
                            2.0 * a.lora_n * (double)(M + N) * a.lora_r;
                kprof_end(KP_GEMM_BIG, s, fl, by, mid_name(bn, false));
            }
            return check_launch("gemm");
        }
    }
    // large K-contiguous BF16 GEMMs: k_gemm_pipe (k_gemm_dma for split-K)
    // (the stage loads address 256 operand rows with 32-bit byte offsets)
    // (smaller outputs take the 256-row tiles when a variant is forced, and
    // split-K when K is long: 32 or more 64-k stages)
    const int ksteps = (K + BK - 1) / BK;
    if (pipe_ok && ((M >= 1024 && N >= 1024) || (M >= 256 && N >= 128 && ksteps >= 32) ||
                    (g_big_variant != 0 && M >= 256 && N >= 128))) {
        int variant = g_big_variant;
        if (variant == 0) variant = N > 3072 ? 18 : 17;
        // up to N = 3072 the 256-wide tiles when they need fewer waves of 256
        // blocks (waves x tile area): N = 2048 at M = 8192 is one wave of
        // 256-wide tiles against 1.4 of 192-wide (48 against 73 us measured)
        if (g_big_variant == 0 && N <= 3072) {
            const int64_t tm = (M + 255) / 256;
            const int64_t w192 = (tm * ((N + 191) / 192) + 255) / 256;
            const int64_t w256 = (tm * ((N + 255) / 256) + 255) / 256;
            if (w256 * 256 < w192 * 192) variant = 18;
        }
        // split-K over few tiles: as many splits as keep the blocks within one
        // per CU (at least 8 stages each), with the tile width that gives the
        // most blocks (256-wide on a tie)
        auto split_for = [&](int tiles) {
            return std::max(1, std::min(256 / tiles, ksteps / 8));
        };
        const int t192 = ((M + 255) / 256) * ((N + 191) / 192);
        const int t256 = ((M + 255) / 256) * ((N + 255) / 256);
        const bool auto_split = force_splits <= 0 && g_force_splits == 0 && ksteps >= 32;
        if (g_big_variant == 0 && auto_split && (N > 3072 ? t256 : t192) < 192)
            variant = t192 * split_for(t192) > t256 * split_for(t256) ? 17 : 18;
        const int BNb = big_bn(variant);
        a.tiles_m = (M + 255) / 256;
        a.tiles_n = (N + BNb - 1) / BNb;
        int tiles = a.tiles_m * a.tiles_n;
        int splits = 1;
        if (force_splits > 0)
            splits = force_splits;
        else if (g_force_splits > 0)
            splits = g_force_splits;
        else if (tiles < 192 && ksteps >= 32)
            splits = split_for(tiles);
        if (splits < 1) splits = 1;
        // A last wave of at most half the CUs' blocks (M 8192 x N 8960: 4.375
        // waves of 256 x 256 tiles) runs as its own launch of 128-row tiles,
        // two blocks per CU at a quarter of the work each: the columns past
        // the last whole wave of 256-wide tiles go to k_gemm_mid.  Every
        // output element keeps its k order, so the result is the same.
        if (g_big_variant == 0 && force_splits <= 0 && g_force_splits == 0 && splits == 1 &&
            variant == 18 && !out_f32) {
            const int full = tiles / 256, rem = tiles % 256;
            if (full >= 1 && rem > 0 && rem <= 128 && (full * 256) % a.tiles_m == 0) {
                const int n_main = full * 256 / a.tiles_m * 256;
                if (n_main > 3072 && n_main < N &&
                    mid_bn(M, N - n_main, 256, ksteps, false, 128) != 0) {
                    const bool fz = lora && lora->n > 0;
                    LoraEpi lt{};
                    if (fz) {
                        lt = *lora;
                        for (int p = 0; p < lora->n; p++) {
                            lt.v_nk[p] = lora->v_nk[p] + (int64_t)n_main * lora->r;
                            lt.v_alt[p] = nullptr;  // the mid kernel fuses every rank here
                        }
                    }
                    int rc = gemm_dispatch(xk, yk, M, n_main, K, alpha, X, ldx, Y, ldy, beta, C,
                                           ldc, bias, false, s, 0, lora);
                    if (rc) return rc;
                    return gemm_dispatch(xk, yk, M, N - n_main, K, alpha, X, ldx,
                                         Y + (int64_t)n_main * ldy, ldy, beta,
                                         (bf16*)C + n_main, ldc, bias ? bias + n_main : nullptr,
                                         false, s, 0, fz ? &lt : nullptr);
                }
            }
        }
        int steps_per = (ksteps + splits - 1) / splits;
        a.k_per_split = steps_per * BK;
        splits = (ksteps + steps_per - 1) / steps_per;
        dim3 grid(tiles, 1, splits);
        if (splits > 1) {
            size_t bytes = (size_t)splits * M * N * sizeof(float);
            a.part = (float*)scratch_get(bytes, s);
            if (!a.part) return set_error(-2, "gemm: scratch allocation of %zu bytes failed", bytes);
            // F32 partials from the 64-k pipeline kernel of the tile width
            // when each split runs 32 or more stages (the LM head's input
            // gradient at B x T = 2048: 10% faster), else from the 8-wave
            // direct-to-LDS kernel, whose shorter prologue wins on splits of
            // about 10 stages (same bits either way)
            const bool long_split = steps_per >= 32;
            if (variant == 17 && long_split)
                tlaunch(k_gemm_pipe_part<192, 4, 2>, dim3(grid), dim3(512), s, a);
            else if (variant == 18 && long_split)
                tlaunch(k_gemm_pipe_part<256, 2, 4>, dim3(grid), dim3(512), s, a);
            else
                launch_big<EPI_PARTIAL>(is_pipe(variant) ? (BNb == 256 ? 8 : 7) : variant, grid,
                                        a, s);
            int64_t MN = (int64_t)M * N;
            tlaunch(k_splitk_reduce<true>, dim3((int)((MN + 255) / 256)), dim3(256), s, a.part, splits, M, N, C,
                                                                          ldc, alpha, beta, bias);
            int rc = check_launch("gemm");
            return rc ? rc : lora_after();
        }
        // LoRA terms fuse into the epilogue up to rank 64 for k_gemm_pipe (one
        // MFMA k step per 16) and at any rank for k_gemm_dma; otherwise they
        // run after the GEMM
        const bool fuse = lora && lora->n > 0 && (lora->r & 7) == 0 &&
                          (!is_pipe(variant) || lora->r <= 64);
        if (fuse) {
            a.lora_n = lora->n;
            a.lora_r = lora->r;
            a.lora_delta = lora->delta ? 1 : 0;
            a.lora_s = lora->s;
            for (int p = 0; p < lora->n; p++) {
                a.lora_u[p] = lora->u[p];
                a.lora_ldu[p] = lora->ldu[p];
                a.lora_v[p] = lora->v_nk[p];
            }
        }
        // measurement hook: algorithmic work of the launch (MNK product,
        // rank-r epilogue products; operands read once, C written once and
        // read once more when beta != 0)
        const int kid = BNb == 256 ? KP_GEMM_BIG_WIDE : KP_GEMM_BIG;
        const bool timed = kprof_begin(kid, s);
        if (variant == 12)
            tlaunch(k_gemm_pipe<192, 2, 2>, dim3(grid), dim3(256), s, a);
        else if (variant == 13)
            tlaunch(k_gemm_pipe<256, 2, 2>, dim3(grid), dim3(256), s, a);
        else if (variant == 14)
            tlaunch(k_gemm_pipe<256, 4, 2>, dim3(grid), dim3(512), s, a);
        else if (variant == 15)
            tlaunch(k_gemm_pipe<192, 4, 2>, dim3(grid), dim3(512), s, a);
        else if (variant == 16)
            tlaunch(k_gemm_pipe<256, 2, 4>, dim3(grid), dim3(512), s, a);
        else if (variant == 17)
            tlaunch(k_gemm_pipe<192, 4, 2, 64>, dim3(grid), dim3(512), s, a);
        else if (variant == 18)
            tlaunch(k_gemm_pipe<256, 2, 4, 64>, dim3(grid), dim3(512), s, a);
        else
            launch_big<EPI_BF16>(variant, grid, a, s);
        if (timed) {
            double mn = (double)M * N;
            double fl = 2.0 * mn * K + 2.0 * mn * a.lora_r * a.lora_n;
            double by = 2.0 * ((double)M * K + (double)N * K + mn * (beta != 0.f ? 2 : 1)) +
                        2.0 * a.lora_n * (double)(M + N) * a.lora_r;
            kprof_end(kid, s, fl, by, big_name(variant));
        }
        int rc = check_launch("gemm");
        return (rc || fuse) ? rc : lora_after();
    }

    // tile choice: wide-N tiles for big outputs, skinny tiles for N <= 32
    enum { CFG_256x128, CFG_128x128, CFG_128x32 } cfg;
    int BMv, BNv;
    if (N <= 32) {
        cfg = CFG_128x32;
        BMv = 128;
        BNv = 32;
    } else if ((int64_t)M * N >= (int64_t)256 * 128 * 512) {
        cfg = CFG_256x128;
        BMv = 256;
        BNv = 128;
    } else {
        cfg = CFG_128x128;
        BMv = 128;
        BNv = 128;
    }
    a.tiles_m = (M + BMv - 1) / BMv;
    a.tiles_n = (N + BNv - 1) / BNv;
    int tiles = a.tiles_m * a.tiles_n;
    // split K when the tile grid alone cannot fill the 256 CUs
    int splits = 1;
    if (force_splits > 0) {
        splits = force_splits;
    } else if (tiles < 256 && ksteps >= 16) {
        splits = (512 + tiles - 1) / tiles;
        if (splits > ksteps / 4) splits = ksteps / 4;
        if (splits < 1) splits = 1;
    }
    if (splits > ksteps) splits = ksteps > 0 ? ksteps : 1;
    int steps_per = (ksteps + splits - 1) / splits;
    a.k_per_split = steps_per * BK;
    splits = (ksteps + steps_per - 1) / steps_per;
    if (splits < 1) splits = 1;

    int epi;
    if (splits > 1) {
        size_t bytes = (size_t)splits * M * N * sizeof(float);
        a.part = (float*)scratch_get(bytes, s);
        if (!a.part) return set_error(-2, "gemm: scratch allocation of %zu bytes failed", bytes);
        epi = EPI_PARTIAL;
    } else {
        epi = out_f32 ? EPI_F32 : EPI_BF16;
    }
#define TA_LAUNCH(BM_, BN_, WM_, WN_)                                                   \
    do {                                                                                \
        if (epi == EPI_BF16)                                                            \
            launch_cfg<BM_, BN_, WM_, WN_, EPI_BF16>(xk, yk, a, splits, vx, vy, s);     \
        else if (epi == EPI_F32)                                                        \
            launch_cfg<BM_, BN_, WM_, WN_, EPI_F32>(xk, yk, a, splits, vx, vy, s);      \
        else                                                                            \
            launch_cfg<BM_, BN_, WM_, WN_, EPI_PARTIAL>(xk, yk, a, splits, vx, vy, s);  \
    } while (0)
    if (cfg == CFG_256x128)
        TA_LAUNCH(256, 128, 2, 2);
    else if (cfg == CFG_128x128)
        TA_LAUNCH(128, 128, 2, 2);
    else
        TA_LAUNCH(128, 32, 4, 1);
#undef TA_LAUNCH
    if (splits > 1) {
        int64_t MN = (int64_t)M * N;
        int blocks = (int)((MN + 255) / 256);
        if (out_f32)
            tlaunch(k_splitk_reduce<false>, dim3(blocks), dim3(256), s, a.part, splits, M, N, C, ldc, alpha,
                                                          beta, bias);
        else
            tlaunch(k_splitk_reduce<true>, dim3(blocks), dim3(256), s, a.part, splits, M, N, C, ldc, alpha,
                                                         beta, bias);
    }
    int rc = check_launch("gemm");
    return rc ? rc : lora_after();
}

// The chain C = bf16(X_0 Y_0^T), C = bf16(X_s Y_s^T + C) for s = 1, 2, then
// the LoRA terms (the q/k/v or gate/up input gradients, proj_bwd_x with
// beta 0, 1, 1: qwen2.cu:233-234, 283-285) as ONE k_gemm_pipe launch over
// the concatenated K: the accumulators are rounded to BF16 where each
// GEMM of the chain ends, so the rounding points are those of the
// separate GEMMs (only the F32 summation order inside a GEMM differs).
// Shapes the pipe kernel does not take run as separate gemm_dispatch calls.
int gemm_chain(int M, int N, const GemmSeg* sg, int ns, bf16* C, int64_t ldc, const LoraEpi* lora,
               hipStream_t s) {
    TA_REQUIRE(ns >= 1 && ns <= 3, "gemm_chain: %d segments", ns);
    int variant = g_big_variant;
    if (variant == 0) variant = N > 3072 ? 18 : 17;
    const int BNb = big_bn(variant);  // the chain kernel comes in the two default shapes
    int Ktot = 0;
    const int KD = pipe_kd(variant), NS = KD == 32 ? 4 : 2;
    bool ok = ns > 1 && variant >= 15 && variant <= 18 && M >= 1024 && N >= 1024;
    for (int q = 0; q < ns; q++) {
        Ktot += sg[q].K;
        ok &= sg[q].K % BK == 0 && al16(sg[q].X) && al16(sg[q].Y) && sg[q].ldx % 8 == 0 &&
              sg[q].ldy % 8 == 0;
        // the kernel keeps each segment's row offsets as 32-bit byte counts
        ok &= sg[q].ldx < kMaxStageLd && sg[q].ldy < kMaxStageLd;
    }
    const int tiles = ((M + 255) / 256) * ((N + BNb - 1) / BNb);
    // (as gemm_dispatch: few tiles and a long K go to split-K instead)
    ok &= tiles >= 192 || Ktot / BK < 32;
    // every segment must start on a loop trip of the kernel (4 stages of 32
    // k or 2 of 64 after the leading zero stages), where the kernel rounds
    {
        const int nk = Ktot / KD, pad = (NS - nk % NS) % NS;
        int kb = 0;
        for (int q = 0; q + 1 < ns; q++) {
            kb += sg[q].K;
            ok &= (kb / KD + pad) % NS == 0;
        }
    }
    ok &= !lora || lora->n == 0 || (lora->r <= 64 && (lora->r & 7) == 0);
    // 128-row tiles (k_gemm_mid_chain: two 64-k stages per trip) when the
    // 256-row chain cannot fill the chip
    // (long chains run per segment instead, where each takes split-K)
    int mid = 0;
    if (g_big_variant == 0 && ns > 1 && M >= 128 && N >= 64 && Ktot / BK < 32) {
        bool mok = !lora || lora->n == 0 || (lora->r <= 64 && (lora->r & 7) == 0);
        const int nk = Ktot / 64, pad = (2 - nk % 2) % 2;
        int kb = 0;
        for (int q = 0; q < ns; q++) {
            mok &= sg[q].K % BK == 0 && al16(sg[q].X) && al16(sg[q].Y) && sg[q].ldx % 8 == 0 &&
                   sg[q].ldy % 8 == 0 && sg[q].ldx < kMaxStageLd && sg[q].ldy < kMaxStageLd;
            kb += sg[q].K;
            if (q + 1 < ns) mok &= (kb / 64 + pad) % 2 == 0;
        }
        if (mok) mid = mid_bn(M, N, BNb, Ktot / BK, ok, 128);
    }
    if (!ok && !mid) {
        for (int q = 0; q < ns; q++) {
            int rc = gemm_dispatch(true, true, M, N, sg[q].K, 1.f, sg[q].X, sg[q].ldx, sg[q].Y,
                                   sg[q].ldy, q ? 1.f : 0.f, C, ldc, nullptr, false, s, 0,
                                   q == ns - 1 ? lora : nullptr);
            if (rc) return rc;
        }
        return 0;
    }
    GemmArgs a{};
    a.M = M;
    a.N = N;
    a.K = Ktot;
    a.X = sg[0].X;
    a.ldx = sg[0].ldx;
    a.Y = sg[0].Y;
    a.ldy = sg[0].ldy;
    a.C = C;
    a.ldc = ldc;
    a.alpha = 1.f;
    a.beta = 0.f;
    a.k_per_split = Ktot;
    a.tiles_m = mid ? (M + 127) / 128 : (M + 255) / 256;
    a.tiles_n = mid ? (N + mid - 1) / mid : (N + BNb - 1) / BNb;
    a.ngroups = 1;
    a.nseg = ns;
    int k = 0;
    for (int q = 0; q < ns; q++) {
        a.kseg[q] = k;
        k += sg[q].K;
        a.sX[q] = sg[q].X;
        a.sldx[q] = sg[q].ldx;
        a.sY[q] = sg[q].Y;
        a.sldy[q] = sg[q].ldy;
    }
    if (lora && lora->n > 0) {
        a.lora_n = lora->n;
        a.lora_r = lora->r;
        a.lora_delta = lora->delta ? 1 : 0;
        a.lora_s = lora->s;
        for (int p = 0; p < lora->n; p++) {
            a.lora_u[p] = lora->u[p];
            a.lora_ldu[p] = lora->ldu[p];
            a.lora_v[p] = lora->v_nk[p];
        }
    }
    dim3 grid(a.tiles_m * a.tiles_n);
    const bool timed = kprof_begin(KP_GEMM_CHAIN, s);
    if (mid == 128)
        tlaunch(k_gemm_mid_chain<128>, dim3(grid), dim3(256), s, a);
    else if (mid == 64)
        tlaunch(k_gemm_mid_chain<64>, dim3(grid), dim3(256), s, a);
    else if (BNb == 192 && KD == 64)
        tlaunch(k_gemm_pipe_chain<192, 4, 2, 64>, dim3(grid), dim3(512), s, a);
    else if (KD == 64)
        tlaunch(k_gemm_pipe_chain<256, 2, 4, 64>, dim3(grid), dim3(512), s, a);
    else if (BNb == 192)
        tlaunch(k_gemm_pipe_chain<192, 4, 2>, dim3(grid), dim3(512), s, a);
    else
        tlaunch(k_gemm_pipe_chain<256, 2, 4>, dim3(grid), dim3(512), s, a);
    if (timed) {
        // every link's operands read once, C written once, rank-r epilogue products
        double mn = (double)M * N;
        double fl = 2.0 * mn * Ktot + 2.0 * mn * a.lora_r * a.lora_n;
        double by = 2.0 * ((double)M * Ktot + (double)N * Ktot + mn) +
                    2.0 * a.lora_n * (double)(M + N) * a.lora_r;
        kprof_end(KP_GEMM_CHAIN, s, fl, by,
                  mid ? mid_name(mid, true)
                  : KD == 64 ? (BNb == 192 ? "void ta::k_gemm_pipe_chain<192, 4, 2, 64>(ta::GemmArgs)"
                                         : "void ta::k_gemm_pipe_chain<256, 2, 4, 64>(ta::GemmArgs)")
                           : (BNb == 192 ? "void ta::k_gemm_pipe_chain<192, 4, 2>(ta::GemmArgs)"
                                         : "void ta::k_gemm_pipe_chain<256, 2, 4>(ta::GemmArgs)"));
    }
    return check_launch("gemm_chain");
}

// Up to three GEMMs over the same X [M x K], C_g = bf16(X Y_g^T (+ bias_g))
// plus the LoRA delta of group g's pair (none, or one pair of rank <= 64;
// rank, delta kind and scale shared), as ONE k_gemm_pipe launch over the N-concatenated
// tile grid: q/k/v or gate/up projections.  Separate launches would each
// end on a partly filled wave of tiles, and the narrow k/v projections
// would run on the small-GEMM path; every output keeps its own epilogue, so
// the results are those of separate launches.  Shapes the pipe kernel does
// not take run as separate gemm_dispatch calls.
int gemm_groups(int M, int K, const bf16* X, int64_t ldx, int64_t ldy, const GemmGroup* gr,
                int ng, hipStream_t s, const RopeSpec* rope) {
    TA_REQUIRE(ng >= 1 && ng <= 3, "gemm_groups: %d groups", ng);
    TA_REQUIRE(!rope || (rope->T > 0 && rope->hd > 0 && rope->hd % 8 == 0 && rope->B * rope->T == M),
               "gemm_groups: bad RoPE shape (B %d, T %d, hd %d, M %d)", rope ? rope->B : 0,
               rope ? rope->T : 0, rope ? rope->hd : 0, M);
    // rope of the roped groups' outputs as separate passes (the other paths)
    auto rope_after = [&]() -> int {
        if (!rope) return 0;
        for (int g = 0; g < ng; g++)
            if (gr[g].rope) {
                TA_REQUIRE(gr[g].N % rope->hd == 0 && gr[g].ldc == gr[g].N,
                           "gemm_groups: RoPE needs whole heads in dense rows");
                if (int rc = ta_rope_fwd(gr[g].C, rope->B, rope->T, gr[g].N / rope->hd, rope->hd,
                                         rope->theta, s))
                    return rc;
            }
        return 0;
    };
    int Ntot = 0;
    bool all256 = true, all192 = true, lora_ok = true, vy = (ldy % 8) == 0;
    const LoraEpi* l0 = nullptr;
    for (int g = 0; g < ng; g++) {
        Ntot += gr[g].N;
        all256 &= gr[g].N % 256 == 0;
        all192 &= gr[g].N % 192 == 0;
        vy &= al16(gr[g].Y);
        const LoraEpi* l = gr[g].lora;
        if (l && l->n > 0) {
            lora_ok &= l->n == 1 && l->r <= 64 && (l->r & 7) == 0 && l->ldu[0] == l->r;
            if (l0) lora_ok &= l->r == l0->r;
            if (l0) lora_ok &= l->delta == l0->delta && l->s == l0->s;
            else l0 = l;
        }
    }
    int variant = g_big_variant;
    if (variant == 0) variant = all256 ? 18 : 17;
    const int BNb = big_bn(variant);
    const bool tiles_ok = BNb == 256 ? all256 : all192;
    const int tiles = ((M + 255) / 256) * (Ntot / BNb);
    const bool vx = al16(X) && (ldx % 8) == 0;
    // (as gemm_dispatch: few tiles and a long K go to split-K instead)
    const bool big = ng > 1 && is_pipe(variant) && tiles_ok && lora_ok && vx && vy && M >= 1024 &&
                     ldx < kMaxStageLd && ldy < kMaxStageLd && Ntot >= 1024 && (K % BK) == 0 &&
                     (tiles >= 192 || K / BK < 32);
    // 128-row tiles when the 256-row grid cannot fill the chip; every
    // group's N a multiple of the tile width
    int nmult = 0;
    for (int g = 0; g < ng; g++) nmult = std::gcd(nmult, gr[g].N);
    const int mid = (g_big_variant == 0 && ng > 1 && lora_ok && vx && vy && (K % BK) == 0 &&
                     ldx < kMaxStageLd && ldy < kMaxStageLd)
                        ? mid_bn(M, Ntot, BNb, K / BK, big, nmult)
                        : 0;
    const int TBN = mid ? mid : BNb;
    if (!big && !mid) {
        for (int g = 0; g < ng; g++) {
            int rc = gemm_dispatch(true, true, M, gr[g].N, K, 1.f, X, ldx, gr[g].Y, ldy, 0.f,
                                   gr[g].C, gr[g].ldc, gr[g].bias, false, s, 0, gr[g].lora);
            if (rc) return rc;
        }
        return rope_after();
    }
    GemmArgs a{};
    a.M = M;
    a.N = gr[0].N;
    a.K = K;
    a.X = X;
    a.ldx = ldx;
    a.Y = gr[0].Y;
    a.ldy = ldy;
    a.C = gr[0].C;
    a.ldc = gr[0].ldc;
    a.alpha = 1.f;
    a.beta = 0.f;
    a.bias = gr[0].bias;
    a.k_per_split = K;
    a.tiles_m = mid ? (M + 127) / 128 : (M + 255) / 256;
    a.tiles_n = Ntot / TBN;
    a.ngroups = ng;
    a.lora_r = l0 ? l0->r : 0;
    a.lora_delta = l0 && l0->delta ? 1 : 0;
    a.lora_s = l0 ? l0->s : 0.f;
    int tn = 0;
    for (int g = 0; g < ng; g++) {
        const LoraEpi* l = gr[g].lora;
        const bool on = l && l->n > 0;
        a.tn0[g] = tn;
        tn += gr[g].N / TBN;
        a.gN[g] = gr[g].N;
        a.gY[g] = gr[g].Y;
        a.gC[g] = gr[g].C;
        a.gldc[g] = gr[g].ldc;
        a.gbias[g] = gr[g].bias;
        a.glora[g] = on ? 1 : 0;
        a.gu[g] = on ? l->u[0] : nullptr;
        a.gv[g] = on ? l->v_nk[0] : nullptr;
        if (on) a.lora_ldu[0] = l->r;
    }
    a.lora_n = a.glora[0];
    a.lora_u[0] = a.gu[0];
    a.lora_v[0] = a.gv[0];
    if (rope) {
        // in the epilogue: every roped group holds whole heads
        const float2* tab = rope_table(rope->T, rope->hd, rope->theta, 1.f, s);
        TA_REQUIRE(tab, "gemm_groups: RoPE table allocation failed");
        a.rope_T = rope->T;
        a.rope_hd = rope->hd;
        for (int g = 0; g < ng; g++) {
            TA_REQUIRE(!gr[g].rope || gr[g].N % rope->hd == 0,
                       "gemm_groups: RoPE group of %d columns, not whole heads of %d", gr[g].N,
                       rope->hd);
            a.grope[g] = gr[g].rope ? tab : nullptr;
        }
        a.rope_tab = a.grope[0];
    }
    const int kid = BNb == 256 ? KP_GEMM_BIG_WIDE : KP_GEMM_BIG;
    const bool timed = kprof_begin(kid, s);
    dim3 grid(a.tiles_m * a.tiles_n);
    if (mid == 128)
        tlaunch(k_gemm_mid<128>, dim3(grid), dim3(256), s, a);
    else if (mid == 64)
        tlaunch(k_gemm_mid<64>, dim3(grid), dim3(256), s, a);
    else if (variant == 12)
        tlaunch(k_gemm_pipe<192, 2, 2>, dim3(grid), dim3(256), s, a);
    else if (variant == 13)
        tlaunch(k_gemm_pipe<256, 2, 2>, dim3(grid), dim3(256), s, a);
    else if (variant == 14)
        tlaunch(k_gemm_pipe<256, 4, 2>, dim3(grid), dim3(512), s, a);
    else if (variant == 15)
        tlaunch(k_gemm_pipe<192, 4, 2>, dim3(grid), dim3(512), s, a);
    else if (variant == 17)
        tlaunch(k_gemm_pipe<192, 4, 2, 64>, dim3(grid), dim3(512), s, a);
    else if (variant == 18)
        tlaunch(k_gemm_pipe<256, 2, 4, 64>, dim3(grid), dim3(512), s, a);
    else
        tlaunch(k_gemm_pipe<256, 2, 4>, dim3(grid), dim3(512), s, a);
    if (timed) {
        double mn = (double)M * Ntot, fl = 2.0 * mn * K, by = 2.0 * ((double)M * K + (double)Ntot * K + mn);
        for (int g = 0; g < ng; g++)
            if (a.glora[g]) {
                fl += 2.0 * M * gr[g].N * a.lora_r;
                by += 2.0 * (double)(M + gr[g].N) * a.lora_r;
            }
        kprof_end(kid, s, fl, by, mid ? mid_name(mid, false) : big_name(variant));
    }
    return check_launch("gemm_groups");
}

// gate = bf16(X Wg^T) + LoRA delta, up likewise, act = bf16(silu(gate) up)
// (qwen2.cu:21-30 twice, then silu_mul_fwd, ops.cu:913-923) as ONE launch
// over Wgu, the gate/up weights interleaved in blocks of 128 rows
// ([Wg rows 0..127; Wu rows 0..127; Wg rows 128..255; ...], [2I x K]): the
// act pass reads the BF16 gate/up tiles from LDS instead of HBM.  The
// LoRA pairs are both on (one rank <= 64) or both off.  Other shapes run as the
// grouped launch plus silu_mul_fwd.
int gemm_swiglu(int M, int K, const bf16* X, int64_t ldx, const bf16* Wgu, const bf16* Wg,
                const bf16* Wu, bf16* gate, bf16* up, bf16* act, int I, const LoraEpi* lg,
                const LoraEpi* lu, hipStream_t s) {
    const bool on = lg && lg->n > 0;
    const bool lora_ok = on ? (lu && lu->n == 1 && lg->n == 1 && lg->r <= 64 && (lg->r & 7) == 0 &&
                               lu->r == lg->r &&
                               lg->delta == lu->delta && lg->s == lu->s &&
                               lg->ldu[0] == lg->r && lu->ldu[0] == lu->r)
                            : !(lu && lu->n > 0);
    const int tiles = ((M + 255) / 256) * (2 * I / 256);
    const bool ok = Wgu && lora_ok &&
                    (g_big_variant == 0 || g_big_variant == 16 || g_big_variant == 18) && M >= 1024 &&
                    I % 128 == 0 && 2 * I >= 1024 && K % BK == 0 && al16(X) && ldx % 8 == 0 &&
                    al16(Wgu) && al16(gate) && al16(up) && al16(act) && I % 8 == 0 &&
                    ldx < kMaxStageLd && K < kMaxStageLd &&
                    (tiles >= 192 || K / BK < 32);
    if (!ok) {
        const GemmGroup gr[2] = {{I, Wg, gate, I, nullptr, lg}, {I, Wu, up, I, nullptr, lu}};
        if (int rc = gemm_groups(M, K, X, ldx, K, gr, 2, s)) return rc;
        return ta_silu_mul_fwd(gate, up, act, (int64_t)M * I, s);
    }
    GemmArgs a{};
    a.M = M;
    a.N = 2 * I;
    a.K = K;
    a.X = X;
    a.ldx = ldx;
    a.Y = Wgu;
    a.ldy = K;
    a.C = gate;
    a.ldc = I;
    a.alpha = 1.f;
    a.beta = 0.f;
    a.k_per_split = K;
    a.tiles_m = (M + 255) / 256;
    a.tiles_n = 2 * I / 256;
    a.ngroups = 1;
    a.nseg = 1;
    a.gN[0] = I;
    a.gldc[0] = I;
    a.gC[0] = gate;
    a.gC[1] = up;
    a.gC[2] = act;
    if (on) {
        a.lora_n = 1;
        a.lora_r = lg->r;
        a.lora_delta = lg->delta ? 1 : 0;
        a.lora_s = lg->s;
        a.lora_ldu[0] = lg->r;
        a.gu[0] = lg->u[0];
        a.gu[1] = lu->u[0];
        a.gv[0] = lg->v_nk[0];
        a.gv[1] = lu->v_nk[0];
    }
    const bool timed = kprof_begin(KP_GEMM_SWIGLU, s);
    const bool kd64 = g_big_variant != 16;
    if (kd64)
        tlaunch(k_gemm_pipe_swiglu<256, 2, 4, 64>, dim3(tiles), dim3(512), s, a);
    else
        tlaunch(k_gemm_pipe_swiglu<256, 2, 4>, dim3(tiles), dim3(512), s, a);
    if (timed) {
        // X and both weights read once; gate, up and act written once
        const double mn = 2.0 * M * I;
        const double fl = 2.0 * mn * K + (on ? 2.0 * mn * a.lora_r : 0.0);
        const double by = 2.0 * ((double)M * K + 2.0 * I * (double)K + 1.5 * mn) +
                          (on ? 2.0 * 2.0 * (M + I) * a.lora_r : 0.0);
        kprof_end(KP_GEMM_SWIGLU, s, fl, by,
                  kd64 ? "void ta::k_gemm_pipe_swiglu<256, 2, 4, 64>(ta::GemmArgs)"
                       : "void ta::k_gemm_pipe_swiglu<256, 2, 4>(ta::GemmArgs)");
    }
    return check_launch("gemm_swiglu");
}

// Operand staging of gemm_f32.  Each F32 value is split into three BF16
// parts, s0 = bf16(s), s1 = bf16(s - s0), s2 = bf16(s - s0 - s1), whose sum
// carries s to about 2^-24 relative (24 bits of significand).  A product
// a*b is formed as the six part products whose magnitude reaches 2^-24 of
// it, a2 b0 + a1 b1 + a0 b2 + a1 b0 + a0 b1 + a0 b0 (smallest first, so the
// F32 accumulator adds the small terms before the large ones); each part
// product is exact in the MFMA's F32 arithmetic.  The parts are laid out
// K-contiguous as six segments of kp columns per row (the segment q of a
// row holds part (code >> 2q) & 3 of columns k0 .. k0 + kc, zero padded to
// kp), so that one BF16 GEMM over K = 6 kp adds exactly those products.
__global__ void k_split3(const float* __restrict__ S, int64_t ld, bool kcontig, int rows,
                         int64_t k0, int kc, int kp, unsigned code, bf16* __restrict__ dst) {
    const int64_t n = (int64_t)rows * kp;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        int64_t r, k;
        if (kcontig) {
            r = i / kp;
            k = i - r * kp;
        } else {
            k = i / rows;
            r = i - k * rows;
        }
        float v = 0.f;
        if (k < kc) v = kcontig ? S[r * ld + k0 + k] : S[(k0 + k) * ld + r];
        bf16 p[3];
        p[0] = f2bf(v);
        const float r1 = v - bf2f(p[0]);
        p[1] = f2bf(r1);
        p[2] = f2bf(r1 - bf2f(p[1]));
        bf16* row = dst + r * (int64_t)(6 * kp) + k;
#pragma unroll
        for (int q = 0; q < 6; q++) row[(int64_t)q * kp] = p[(code >> (2 * q)) & 3u];
    }
}

int gemm_ce_dx(int M, int N, int K, const bf16* logits, const bf16* Wt, bf16* C,
               const float* lse2, const int32_t* tgt, float inv_n, hipStream_t s) {
    TA_REQUIRE(M >= 256 && N >= 192 && K % BK == 0 && al16(logits) && al16(Wt) && al16(C) &&
                   (N % 8) == 0 && K < kMaxStageLd && lse2 && tgt,
               "gemm_ce_dx: unsupported shape M=%d N=%d K=%d", M, N, K);
    GemmArgs a{};
    a.M = M;
    a.N = N;
    a.K = K;
    a.X = logits;
    a.ldx = K;
    a.Y = Wt;
    a.ldy = K;
    a.C = C;
    a.ldc = N;
    a.alpha = 1.f;
    a.beta = 0.f;
    a.k_per_split = K;
    a.ngroups = 1;
    a.nseg = 1;
    a.ce_lse2 = lse2;
    a.ce_tgt = tgt;
    a.ce_inv_n = inv_n;
    const int BNb = N > 3072 ? 256 : 192;
    a.tiles_m = (M + 255) / 256;
    a.tiles_n = (N + BNb - 1) / BNb;
    dim3 grid(a.tiles_m * a.tiles_n);
    if (BNb == 192)
        tlaunch(k_gemm_pipe_ce<192, 4, 2>, dim3(grid), dim3(512), s, a);
    else
        tlaunch(k_gemm_pipe_ce<256, 2, 4>, dim3(grid), dim3(512), s, a);
    return check_launch("gemm_ce_dx");
}

}  // namespace ta

using namespace ta;

extern "C" {


int ta_gemm_rm(int x_kmajor, int y_kmajor, int M, int N, int K, float alpha, const uint16_t* X,
               int ldx, const uint16_t* Y, int ldy, float beta, uint16_t* C, int ldc,
               const uint16_t* bias, void* stream) {
    TA_REQUIRE(M > 0 && N > 0 && K > 0 && ldx > 0 && ldy > 0 && ldc > 0,
               "gemm_rm: M/N/K and leading dims must be > 0");
    return gemm_dispatch(x_kmajor != 0, y_kmajor != 0, M, N, K, alpha, X, ldx, Y, ldy, beta, C,
                         ldc, bias, false, (hipStream_t)stream, 0, nullptr);
}

int ta_gemm_rm_variant(int variant, int x_kmajor, int y_kmajor, int M, int N, int K, float alpha,
                       const uint16_t* X, int ldx, const uint16_t* Y, int ldy, float beta,
                       uint16_t* C, int ldc, const uint16_t* bias, void* stream) {
    TA_REQUIRE(variant_ok(variant % 100) && variant >= 0 && variant / 100 <= 64,
               "gemm_rm_variant: %d is not a kernel variant (0, 7..20, + 100 x splits)", variant);
    struct Restore {
        int v, f;
        ~Restore() {
            g_big_variant = v;
            g_force_splits = f;
        }
    } restore{g_big_variant, g_force_splits};
    g_big_variant = variant % 100;
    g_force_splits = variant / 100;
    return ta_gemm_rm(x_kmajor, y_kmajor, M, N, K, alpha, X, ldx, Y, ldy, beta, C, ldc, bias,
                      stream);
}

// cuBLAS column-major C(MxN) = alpha op(A) op(B) + beta C  ==  row-major
// C^T(NxM) = op(B)^T op(A)^T: rows j come from op(B), columns i from op(A).
int ta_gemm_bf16(int transA, int transB, int M, int N, int K, float alpha, const uint16_t* A,
                 int lda, const uint16_t* B, int ldb, float beta, uint16_t* C, int ldc,
                 void* stream) {
    TA_REQUIRE(M > 0 && N > 0 && K > 0, "gemm_bf16: M/N/K must be > 0");
    TA_REQUIRE(lda > 0 && ldb > 0 && ldc > 0, "gemm_bf16: leading dims must be > 0");
    return gemm_dispatch(!transB, transA != 0, N, M, K, alpha, B, ldb, A, lda, beta, C, ldc,
                         nullptr, false, (hipStream_t)stream, 0, nullptr);
}

// cublasSgemm semantics (tensor.cu:168-182): F32 operands, F32 result.  The
// operands are split into BF16 parts (k_split3) and multiplied on the BF16
// MFMA with F32 accumulation, K in chunks whose staging stays within 256 MB;
// each chunk after the first adds into C (beta 1), as a split-K SGEMM does.
int ta_gemm_f32(int transA, int transB, int M, int N, int K, float alpha, const float* A, int lda,
                const float* B, int ldb, float beta, float* C, int ldc, void* stream) {
    TA_REQUIRE(M > 0 && N > 0 && K > 0, "gemm_f32: M/N/K must be > 0");
    TA_REQUIRE(lda > 0 && ldb > 0 && ldc > 0, "gemm_f32: leading dims must be > 0");
    hipStream_t s = (hipStream_t)stream;
    // rows of the row-major form: X = op(B) by output column j (N rows, K
    // contiguous when !transB), Y = op(A) by output row i (M rows, K
    // contiguous when transA); part codes pair a2 b0, a1 b1, a0 b2, a1 b0,
    // a0 b1, a0 b0 segment by segment
    const unsigned code_x = 0u | 1u << 2 | 2u << 4 | 0u << 6 | 1u << 8 | 0u << 10;
    const unsigned code_y = 2u | 1u << 2 | 0u << 4 | 1u << 6 | 0u << 8 | 0u << 10;
    const int64_t budget = (int64_t)256 << 20;
    int64_t kc_max = budget / (12 * ((int64_t)M + N));
    kc_max = kc_max < 32 ? 32 : (kc_max & ~(int64_t)31);
    const int kcap = (int)std::min<int64_t>(kc_max, ((int64_t)K + 31) & ~(int64_t)31);
    const size_t offy = ((size_t)N * 6 * kcap * 2 + 255) & ~(size_t)255;
    bf16* x16 = (bf16*)scratch_get(offy + (size_t)M * 6 * kcap * 2, s, 1);
    TA_REQUIRE(x16, "gemm_f32: scratch allocation failed");
    bf16* y16 = (bf16*)((char*)x16 + offy);
    for (int64_t k0 = 0; k0 < K; k0 += kcap) {
        const int kc = (int)std::min<int64_t>(kcap, K - k0);
        const int kp = (kc + 31) & ~31;
        const int64_t nx = (int64_t)N * kp, ny = (int64_t)M * kp;
        tlaunch(k_split3, dim3((int)std::min<int64_t>((nx + 255) / 256, 4096)), dim3(256), s, B, ldb, transB == 0, N, k0, kc, kp, code_x, x16);
        tlaunch(k_split3, dim3((int)std::min<int64_t>((ny + 255) / 256, 4096)), dim3(256), s, A, lda, transA != 0, M, k0, kc, kp, code_y, y16);
        const int rc = gemm_dispatch(true, true, N, M, 6 * kp, alpha, x16, 6 * kp, y16, 6 * kp,
                                     k0 == 0 ? beta : 1.f, C, ldc, nullptr, true, s, 0, nullptr);
        if (rc != 0) return rc;
    }
    return check_launch("gemm_f32");
}

}  // extern "C"
