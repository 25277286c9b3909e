// lora.hip — the LoRA products of apply_lora_fwd / apply_lora_bwd
// (src/adapter/adapter_model.cu:96-220) as purpose-built gfx950 kernels.
//
// At rank r = 8..64 every LoRA product is skinny: one side is r wide, the
// other is tokens (B*T) or a hidden/intermediate width.  They are HBM-bound
// (about r flops per byte), so the design goal is one pass over each large
// operand, not MFMA tile efficiency:
//
//   k_skinny_nt   C_p = bf16(X Y_p^T) for up to 3 pairs sharing X -
//                 h = x A^T for q,k,v (or gate,up) in ONE pass over x, and
//                 dh = go B (with the B^T shadow) — 16 tokens per block, the
//                 4 waves split K and reduce through LDS in a fixed order.
//   k_rank_update Y = Y (+) s * U_p V_p for up to 3 pairs applied in order
//                 on one [64 x 64] tile held in LDS:  the forward delta add
//                 y = bf16(y + s*bf16(h B^T)) (adapter_model.cu:108-127) and
//                 the input-gradient update gx = bf16(s*dh A + gx)
//                 (adapter_model.cu:210-219), so y / gx are read and written
//                 once per group instead of once per pair and GEMM.
//   k_wgrad       partial G = sum over a token range of P^T Q (gB = go^T h,
//                 gA = dh^T x), split over token ranges for parallelism;
//                 k_wgrad_reduce adds s * (sum of partials, fixed order) into
//                 the F32 gradients (the reference's gemm_f32 with beta = 1).
//
// All MFMAs are v_mfma_f32_16x16x32_bf16; rank dimensions are zero-padded to
// multiples of 32 (r = 8, 16) or looped (r = 64).
#include <algorithm>

#include "lds_tr.hpp"
#include "ta_internal.hpp"

namespace ta {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mf16(bf16x8_t a, bf16x8_t b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8_t zfrag() {
    bf16x8_t z;
#pragma unroll
    for (int e = 0; e < 8; e++) z[e] = (__bf16)0.f;
    return z;
}
// 8 consecutive k of a K-contiguous row, zero beyond kend
__device__ __forceinline__ bf16x8_t ld8(const bf16* __restrict__ row, int k, int kend) {
    if (k + 8 <= kend) return *(const bf16x8_t*)(row + k);
    bf16x8_t v = zfrag();
    for (int e = 0; e < 8; e++)
        if (k + e < kend) v[e] = __builtin_bit_cast(__bf16, row[k + e]);
    return v;
}
// 8 consecutive k at row + k when ok, zero otherwise.  The load is issued
// unconditionally (from row itself when !ok) and the zero is a select, so a
// wave's loads go out back to back instead of one branch-guarded load at a
// time.  row must be a valid 16-byte aligned address.
__device__ __forceinline__ bf16x8_t ld8s(const bf16* __restrict__ row, int k, bool ok) {
    bf16x8_t v = *(const bf16x8_t*)(row + (ok ? k : 0));
    return ok ? v : zfrag();
}

struct Pairs3 {
    const bf16* y[3];  // k_skinny_nt: Y_p [r x K]; k_rank_update: V_p
    bf16* c[3];        // k_skinny_nt outputs C_p [M x r] (ldc = r)
    const bf16* u[3];  // k_rank_update: U_p [M x r]
    int64_t ldu[3];
    int n;             // pairs
    int64_t ldc;       // k_skinny_nt: row stride of every C_p
};

// ── C_p = bf16(X Y_p^T) ───────────────────────────────────────────────────
// grid: ceil(M/32) blocks x 512 threads (8 waves).  Each wave covers all 32
// rows of the block (2 groups of 16) for runs of U consecutive 32-wide K
// chunks taken round robin, so one fragment of Y_p serves 32 rows; it
// issues the loads of its U chunks before their MFMAs (U 16-byte loads per
// lane and operand in flight).  The waves' partial sums are added in wave order through LDS.
// Column c of the concatenated output belongs to pair c / r, rank c % r.
constexpr int SK_W = 8, SK_RG = 2;  // waves, 16-row groups per block
template <int NT, int U>  // NT: 16-column tiles covering n*r columns
__global__ __launch_bounds__(SK_W * 64) void k_skinny_nt(const bf16* __restrict__ X, int64_t ldx,
                                                         int M, int K, int r, Pairs3 p) {
    __shared__ floatx4 red[SK_W / 2][SK_RG][NT][64];
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int m0 = blockIdx.x * 16 * SK_RG;
    int ncat = p.n * r;
    floatx4 acc[SK_RG][NT];
#pragma unroll
    for (int g = 0; g < SK_RG; g++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[g][t] = floatx4{0.f, 0.f, 0.f, 0.f};
    const bf16* xr[SK_RG];
    bool rin[SK_RG];
#pragma unroll
    for (int g = 0; g < SK_RG; g++) {
        int row = m0 + 16 * g + (lane & 15);
        rin[g] = row < M;
        xr[g] = X + (int64_t)(rin[g] ? row : 0) * ldx;
    }
    const bf16* yr[NT];
    bool yin[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        int c = 16 * t + (lane & 15);
        yin[t] = c < ncat;
        const int pr = c / r;
        yr[t] = yin[t] ? (pr == 0 ? p.y[0] : pr == 1 ? p.y[1] : p.y[2]) + (int64_t)(c - pr * r) * K
                       : p.y[0];
    }
    const int nks = (K + 31) / 32;
    const int ko = 8 * (lane >> 4);
    // K is a multiple of 8 (checked by the launcher): a chunk of 8 at k < K
    // is whole
    // each wave takes U consecutive chunks per trip (U * 64 contiguous bytes
    // of each of its rows), the waves interleaved at that granularity
    for (int ks0 = w * U; ks0 < nks; ks0 += SK_W * U) {
        bf16x8_t a[U][SK_RG], b[U][NT];
#pragma unroll
        for (int u = 0; u < U; u++) {
            int ks = ks0 + u;
            int k = 32 * ks + ko;
            bool in = ks < nks && k < K;
#pragma unroll
            for (int g = 0; g < SK_RG; g++) a[u][g] = ld8s(xr[g], k, in && rin[g]);
#pragma unroll
            for (int t = 0; t < NT; t++) b[u][t] = ld8s(yr[t], k, in && yin[t]);
        }
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int g = 0; g < SK_RG; g++)
#pragma unroll
                for (int t = 0; t < NT; t++) acc[g][t] = mf16(a[u][g], b[u][t], acc[g][t]);
    }
    // fixed-order tree over the waves: w += w + h for h = 4, 2, 1
#pragma unroll
    for (int h = SK_W / 2; h >= 1; h >>= 1) {
        if (w >= h && w < 2 * h)
#pragma unroll
            for (int g = 0; g < SK_RG; g++)
#pragma unroll
                for (int t = 0; t < NT; t++) red[w - h][g][t][lane] = acc[g][t];
        __syncthreads();
        if (w < h)
#pragma unroll
            for (int g = 0; g < SK_RG; g++)
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    floatx4 o = red[w][g][t][lane];
                    acc[g][t][0] += o[0];
                    acc[g][t][1] += o[1];
                    acc[g][t][2] += o[2];
                    acc[g][t][3] += o[3];
                }
        __syncthreads();
    }
    if (w == 0) {
#pragma unroll
        for (int g = 0; g < SK_RG; g++)
#pragma unroll
            for (int t = 0; t < NT; t++) {
                floatx4 v = acc[g][t];
                int c = 16 * t + (lane & 15);
                if (c >= ncat) continue;
                const int pr = c / r;  // selects, not an index into the argument struct
                bf16* out = (pr == 0 ? p.c[0] : pr == 1 ? p.c[1] : p.c[2]) + (c - pr * r);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    int m = m0 + 16 * g + 4 * (lane >> 4) + i;
                    if (m < M) out[(int64_t)m * p.ldc] = f2bf(v[i]);
                }
            }
    }
}

// ── C_p = bf16(X Y_p^T) with X and Y streamed through LDS ────────────────
// The same product for the common case (16-byte aligned rows, K a multiple
// of 8, n * r <= 64) with direct-to-LDS loads: K runs in stages of 256; one
// global_load_lds_dwordx4 moves 2 rows x 512 contiguous bytes (whole cache
// lines, where k_skinny_nt's fragment-shaped loads take 64 bytes of each of
// 16 rows), NS stage buffers (6 for one 16-column tile, 4 for two, 3 for
// three or four: as many as the LDS holds, since the kernel streams X with
// little compute per byte and is bound by the bytes it has in flight).  Block: 32 rows of X, 8 waves; in each
// stage wave w computes k chunk w (32 wide) for both 16-row groups and
// every 16-column tile of the concatenated Y.  16-byte unit u of row R sits
// in slot u ^ (R % 16), so the fragment reads of 16 consecutive rows hit
// distinct banks.  Partial sums are added in wave order through LDS, as in
// k_skinny_nt.  Stages before the first (padding K up to a multiple of
// NS stages) and chunks past K load a zero page.
constexpr int SKD_K = 256;  // k per stage
static __device__ __attribute__((aligned(16))) bf16 g_skd_zero[8] = {};

// One stage of DMA: NI instructions of 2 rows x 512 bytes, instruction i
// (rows 2i, 2i+1) issued by wave i % 8.  X rows are m0 + row (clamped, their
// products unused past M); Y rows are the concatenated rank rows c (pair
// c / r, rank c % r), zero past n * r.
template <int NI, bool ISX>
__device__ __forceinline__ void skd_stage(const bf16* __restrict__ X, int64_t ldx, int m0, int M,
                                          const Pairs3& p, int r, int kst, int K, bf16* buf, int w,
                                          int lane) {
    constexpr int PER = (NI + 7) / 8;
#pragma unroll
    for (int h = 0; h < PER; h++) {
        int i = w + 8 * h;
        i = i < NI ? i : i - 8;  // a surplus instruction repeats a lower wave's (same bytes)
        const int row = 2 * i + (lane >> 5), slot = lane & 31;
        const int k = kst + 8 * (slot ^ (row & 15));
        bool ok = kst >= 0 && k < K;
        const bf16* base;
        if constexpr (ISX) {
            base = X + (int64_t)min(m0 + row, M - 1) * ldx;
        } else {
            const int pr = row < r ? 0 : row < 2 * r ? 1 : 2;
            ok = ok && row < p.n * r;
            const bf16* y = pr == 0 ? p.y[0] : pr == 1 ? p.y[1] : p.y[2];
            base = (ok ? y : g_skd_zero) + (int64_t)(row - pr * r) * K;
        }
        const bf16* src = ok ? base + k : g_skd_zero;
        __builtin_amdgcn_global_load_lds((const void*)src,
                                         (__attribute__((address_space(3))) void*)(buf + 512 * i),
                                         16, 0, 0);
    }
}

// 16x16x32 operand of stage rows [R0, R0+16), k chunk c (32 wide)
__device__ __forceinline__ bf16x8_t skd_frag(const bf16* buf, int R0, int c, int lane) {
    const int row = R0 + (lane & 15), u = 4 * c + (lane >> 4);
    return *(const bf16x8_t*)(buf + row * SKD_K + 8 * (u ^ (row & 15)));
}

template <int NT, int NS>
__global__ __launch_bounds__(512) void k_skinny_dma(const bf16* __restrict__ X, int64_t ldx, int M,
                                                    int K, int r, Pairs3 p) {
    constexpr int XE = 32 * SKD_K, YE = 16 * NT * SKD_K;  // elements per stage
    constexpr int XI = 16, YI = 8 * NT;                   // DMA instructions per stage
    constexpr int LPS = (XI + 7) / 8 + (YI + 7) / 8;      // ... per wave
    static_assert(NS == 3 || NS == 4 || NS == 6, "3, 4 or 6 stages");
    __shared__ __attribute__((aligned(1024))) bf16 sX0[XE], sX1[XE], sX2[XE], sX3[NS >= 4 ? XE : 8],
        sX4[NS == 6 ? XE : 8], sX5[NS == 6 ? XE : 8];
    __shared__ __attribute__((aligned(1024))) bf16 sY0[YE], sY1[YE], sY2[YE], sY3[NS >= 4 ? YE : 8],
        sY4[NS == 6 ? YE : 8], sY5[NS == 6 ? YE : 8];
    // the partial sums' exchange; with four 16-column tiles it reuses stage
    // buffer sY0 (32 KB), which keeps the block within the LDS
    static_assert(NT < 4 || sizeof(floatx4) * SK_W / 2 * SK_RG * NT * 64 <= sizeof(bf16) * YE,
                  "exchange fits a Y stage buffer");
    __shared__ floatx4 red_own[NT < 4 ? SK_W / 2 : 1][SK_RG][NT][64];
    floatx4 (*const red)[SK_RG][NT][64] =
        NT < 4 ? red_own : reinterpret_cast<floatx4 (*)[SK_RG][NT][64]>(sY0);
    const int lane = threadIdx.x & 63;
    int w = threadIdx.x >> 6;
    w = __builtin_amdgcn_readfirstlane(w);
    const int m0 = blockIdx.x * 32;
    floatx4 acc[SK_RG][NT];
#pragma unroll
    for (int g = 0; g < SK_RG; g++)
#pragma unroll
        for (int t = 0; t < NT; t++) acc[g][t] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int nst = (K + SKD_K - 1) / SKD_K;
    const int pad = (NS - nst % NS) % NS;
#define SKD_ISSUE(SXB, SYB, KS)                                                            \
    do {                                                                                   \
        const int ks_ = (KS);                                                              \
        const int kst_ = ks_ < 0 ? -1 : min(ks_, nst - 1) * SKD_K;                         \
        skd_stage<XI, true>(X, ldx, m0, M, p, r, kst_, K, SXB, w, lane);                    \
        skd_stage<YI, false>(X, ldx, m0, M, p, r, kst_, K, SYB, w, lane);                   \
    } while (0)
#define SKD_STEP(J, SXJ, SYJ, SXN, SYN)                                                    \
    do {                                                                                   \
        TA_WAIT_VMCNT(LPS * (NS - 2));                                                     \
        __builtin_amdgcn_s_barrier();                                                      \
        SKD_ISSUE(SXN, SYN, ks0 + (J) + NS - 1);                                           \
        bf16x8_t a_[SK_RG], b_[NT];                                                        \
        _Pragma("unroll") for (int g = 0; g < SK_RG; g++) a_[g] = skd_frag(SXJ, 16 * g, w, lane); \
        _Pragma("unroll") for (int t = 0; t < NT; t++) b_[t] = skd_frag(SYJ, 16 * t, w, lane);    \
        _Pragma("unroll") for (int g = 0; g < SK_RG; g++)                                  \
            _Pragma("unroll") for (int t = 0; t < NT; t++) acc[g][t] = mf16(a_[g], b_[t], acc[g][t]); \
    } while (0)
    SKD_ISSUE(sX0, sY0, 0 - pad);
    SKD_ISSUE(sX1, sY1, 1 - pad);
    if constexpr (NS >= 4) SKD_ISSUE(sX2, sY2, 2 - pad);
    if constexpr (NS == 6) {
        SKD_ISSUE(sX3, sY3, 3 - pad);
        SKD_ISSUE(sX4, sY4, 4 - pad);
    }
    for (int ks0 = -pad; ks0 < nst; ks0 += NS) {
        if constexpr (NS == 6) {
            SKD_STEP(0, sX0, sY0, sX5, sY5);
            SKD_STEP(1, sX1, sY1, sX0, sY0);
            SKD_STEP(2, sX2, sY2, sX1, sY1);
            SKD_STEP(3, sX3, sY3, sX2, sY2);
            SKD_STEP(4, sX4, sY4, sX3, sY3);
            SKD_STEP(5, sX5, sY5, sX4, sY4);
        } else if constexpr (NS == 4) {
            SKD_STEP(0, sX0, sY0, sX3, sY3);
            SKD_STEP(1, sX1, sY1, sX0, sY0);
            SKD_STEP(2, sX2, sY2, sX1, sY1);
            SKD_STEP(3, sX3, sY3, sX2, sY2);
        } else {
            SKD_STEP(0, sX0, sY0, sX2, sY2);
            SKD_STEP(1, sX1, sY1, sX0, sY0);
            SKD_STEP(2, sX2, sY2, sX1, sY1);
        }
    }
    TA_WAIT_VMCNT(0);  // the surplus loads have landed before the block ends
    // (exchange in sY0: every wave's loads have landed and its fragment
    // reads are done before any wave writes there)
    if constexpr (NT == 4) __syncthreads();
#undef SKD_STEP
#undef SKD_ISSUE
    // fixed-order tree over the waves: w += w + h for h = 4, 2, 1
#pragma unroll
    for (int h = SK_W / 2; h >= 1; h >>= 1) {
        if (w >= h && w < 2 * h)
#pragma unroll
            for (int g = 0; g < SK_RG; g++)
#pragma unroll
                for (int t = 0; t < NT; t++) red[w - h][g][t][lane] = acc[g][t];
        __syncthreads();
        if (w < h)
#pragma unroll
            for (int g = 0; g < SK_RG; g++)
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    floatx4 o = red[w][g][t][lane];
                    acc[g][t][0] += o[0];
                    acc[g][t][1] += o[1];
                    acc[g][t][2] += o[2];
                    acc[g][t][3] += o[3];
                }
        __syncthreads();
    }
    if (w == 0) {
        const int ncat = p.n * r;
#pragma unroll
        for (int g = 0; g < SK_RG; g++)
#pragma unroll
            for (int t = 0; t < NT; t++) {
                floatx4 v = acc[g][t];
                int c = 16 * t + (lane & 15);
                if (c >= ncat) continue;
                const int pr = c / r;  // selects, not an index into the argument struct
                bf16* out = (pr == 0 ? p.c[0] : pr == 1 ? p.c[1] : p.c[2]) + (c - pr * r);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    int m = m0 + 16 * g + 4 * (lane >> 4) + i;
                    if (m < M) out[(int64_t)m * p.ldc] = f2bf(v[i]);
                }
            }
    }
}

// ── Y (+)= s * U_p V_p, pairs applied in order, one 64 x 64 tile of Y ─────
// DELTA: V_p is [N x r] (B of the pair): Y = bf16(Y + s * bf16(U V^T)).
// GEMM : V_p is [r x N] (A of the pair): Y = bf16(s * (U V) + Y).
constexpr int RU_LD = 64 + 8;
template <bool DELTA, int RK>  // RK: rank rounded up to a multiple of 32
__global__ __launch_bounds__(256) void k_rank_update(bf16* __restrict__ Y, int64_t ldy, int M, int N,
                                                     int r, float s, Pairs3 p) {
    __shared__ __attribute__((aligned(16))) bf16 sY[64 * RU_LD];
    __shared__ __attribute__((aligned(16))) bf16 sV[64 * (RK + 8)];  // [n][k]
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    bool vec = ((ldy & 7) == 0) && (((uintptr_t)Y & 15) == 0);
    // stage the Y tile (coalesced 16-byte rows)
    for (int q = threadIdx.x; q < 64 * 8; q += 256) {
        int rr = q >> 3, cc = (q & 7) * 8;
        int m = m0 + rr, n = n0 + cc;
        bf16x8v v;
        if (m < M && vec && n + 8 <= N) {
            v = *(const bf16x8v*)(Y + (int64_t)m * ldy + n);
        } else {
            uint16_t tt[8];
            for (int e = 0; e < 8; e++)
                tt[e] = (m < M && n + e < N) ? Y[(int64_t)m * ldy + n + e] : (uint16_t)0;
            for (int e = 0; e < 4; e++) v.w[e] = tt[2 * e] | ((uint32_t)tt[2 * e + 1] << 16);
        }
        *(bf16x8v*)(sY + rr * RU_LD + cc) = v;
    }
    for (int pi = 0; pi < p.n; pi++) {
        // stage V_p as [n][k] (k = rank index), zero-padded to RK
        __syncthreads();
        for (int q = threadIdx.x; q < 64 * RK; q += 256) {
            // DELTA reads B[n][k] (k contiguous), GEMM reads A[k][n] (n contiguous)
            int nn = DELTA ? q / RK : q % 64, kk = DELTA ? q % RK : q / 64;
            int n = n0 + nn;
            uint16_t v = 0;
            if (n < N && kk < r) v = DELTA ? p.y[pi][(int64_t)n * r + kk] : p.y[pi][(int64_t)kk * N + n];
            sV[nn * (RK + 8) + kk] = v;
        }
        __syncthreads();
        floatx4 acc[4];
#pragma unroll
        for (int t = 0; t < 4; t++) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
        int row = m0 + 16 * w + (lane & 15);
        const bf16* ur = p.u[pi] + (int64_t)(row < M ? row : 0) * p.ldu[pi];
#pragma unroll
        for (int kc = 0; kc < RK / 32; kc++) {
            int k = 32 * kc + 8 * (lane >> 4);
            bf16x8_t a = (row < M) ? ld8(ur, k, r) : zfrag();
#pragma unroll
            for (int t = 0; t < 4; t++) {
                bf16x8_t b = *(const bf16x8_t*)(sV + (16 * t + (lane & 15)) * (RK + 8) + k);
                acc[t] = mf16(a, b, acc[t]);
            }
        }
        // each lane owns column 16t + l%16, rows 4(l/16)+i of this wave's strip
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                int idx = (16 * w + 4 * (lane >> 4) + i) * RU_LD + 16 * t + (lane & 15);
                float y = bf2f(sY[idx]);
                float o = DELTA ? y + s * bf2f(f2bf(acc[t][i])) : s * acc[t][i] + y;
                sY[idx] = f2bf(o);
            }
    }
    __syncthreads();
    for (int q = threadIdx.x; q < 64 * 8; q += 256) {
        int rr = q >> 3, cc = (q & 7) * 8;
        int m = m0 + rr, n = n0 + cc;
        if (m >= M) continue;
        bf16x8v v = *(const bf16x8v*)(sY + rr * RU_LD + cc);
        if (vec && n + 8 <= N) {
            *(bf16x8v*)(Y + (int64_t)m * ldy + n) = v;
        } else {
            for (int e = 0; e < 8; e++)
                if (n + e < N) Y[(int64_t)m * ldy + n + e] = (uint16_t)(v.w[e >> 1] >> ((e & 1) * 16));
        }
    }
}

// ── weight gradients: partial[z][l][s] = sum_{t in range z} L[t][l] * Sm[t][s]
// L: [T x NL] (ldl), Sm: [T x NS] (lds), NS <= 192.  Block: 64 columns of L
// (4 waves x 16), one token range, token tiles of 64.  Both tiles sit in LDS
// in their natural layout ([token][column], 16-byte row chunks straight
// from the global rows) and the MFMA operands, which need 8 consecutive
// tokens per lane, come out of LDS through gfx950's transposing read
// (ds_read_b64_tr_b16: 16 lanes that each read 4 consecutive columns of
// rows k0 + lane/4 receive, lane i, column i of rows k0..k0+3).
constexpr int WG_TK = 64;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 8 consecutive BF16 of row `tok`, columns [c, c+8) (zero outside the
// matrix), as a 16-byte vector
__device__ __forceinline__ u32x4 ld8z(const bf16* __restrict__ P, int64_t ld, int tok, int t_end,
                                      int c, int ncols, bool vec) {
    if (vec) {
        // rows 16-byte aligned and ncols a multiple of 8: one unconditional
        // load (of row 0 when out of range) and a select, no branch
        const bool ok = tok < t_end && c < ncols;
        u32x4 v = *(const u32x4*)(P + (ok ? (int64_t)tok * ld + c : 0));
        return ok ? v : u32x4{0u, 0u, 0u, 0u};
    }
    uint16_t x[8];
#pragma unroll
    for (int e = 0; e < 8; e++)
        x[e] = (tok < t_end && c + e < ncols) ? P[(int64_t)tok * ld + c + e] : (uint16_t)0;
    u32x4 v;
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = x[2 * e] | ((uint32_t)x[2 * e + 1] << 16);
    return v;
}

template <int NST, bool VEC>  // 16-column tiles of the small side; VEC: 16-byte rows
__global__ __launch_bounds__(256) void k_wgrad(const bf16* __restrict__ L, int64_t ldl, int NL,
                                               const bf16* __restrict__ Sm, int64_t lds, int NS,
                                               int T, int tokens_per_split,
                                               float* __restrict__ part) {
    constexpr int NSTP = NST <= 1 ? 1 : NST <= 2 ? 2 : NST <= 4 ? 4 : NST <= 8 ? 8 : 16;
    __shared__ __attribute__((aligned(16))) char sL[WG_TK * 64 * 2];           // [t][l]
    __shared__ __attribute__((aligned(16))) char sS[WG_TK * NSTP * 16 * 2];    // [t][s]
    constexpr int SCPR = NST * 2;              // 16-byte chunks per small-tile row
    constexpr int SCH = SCPR * WG_TK;          // ... per tile
    constexpr int SPT = (SCH + 255) / 256;     // ... per thread
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int l0 = blockIdx.x * 64;
    int t_beg = blockIdx.y * tokens_per_split;
    int t_end = min(T, t_beg + tokens_per_split);
    floatx4 acc[NST];
#pragma unroll
    for (int t = 0; t < NST; t++) acc[t] = floatx4{0.f, 0.f, 0.f, 0.f};
    // staging registers: the next token tile is loaded while this one computes
    u32x4 rl[2], rs[SPT];
#define WG_LOAD(tb)                                                                         \
    do {                                                                                    \
        _Pragma("unroll") for (int i = 0; i < 2; i++) {                                     \
            int q = threadIdx.x + 256 * i;                                                  \
            rl[i] = ld8z(L, ldl, (tb) + (q >> 3), t_end, l0 + (q & 7) * 8, NL, VEC);        \
        }                                                                                   \
        _Pragma("unroll") for (int i = 0; i < SPT; i++) {                                   \
            int q = threadIdx.x + 256 * i;                                                  \
            if (q < SCH)                                                                    \
                rs[i] = ld8z(Sm, lds, (tb) + q / SCPR, t_end, (q % SCPR) * 8, NS, VEC);     \
        }                                                                                   \
    } while (0)
    if (t_beg < t_end) WG_LOAD(t_beg);
    for (int tb = t_beg; tb < t_end; tb += WG_TK) {
        __syncthreads();  // the previous tile's fragment reads are done
#pragma unroll
        for (int i = 0; i < 2; i++) {
            int q = threadIdx.x + 256 * i;
            *(u32x4*)(sL + tr_off<4>(q >> 3, (q & 7) * 8)) = rl[i];
        }
#pragma unroll
        for (int i = 0; i < SPT; i++) {
            int q = threadIdx.x + 256 * i;
            if (q < SCH) *(u32x4*)(sS + tr_off<NSTP>(q / SCPR, (q % SCPR) * 8)) = rs[i];
        }
        __syncthreads();
        if (tb + WG_TK < t_end) WG_LOAD(tb + WG_TK);
#pragma unroll
        for (int kc = 0; kc < WG_TK / 32; kc++) {
            bf16x8_t a = tr_frag<4>(sL, 32 * kc, 16 * w, lane);
#pragma unroll
            for (int t = 0; t < NST; t++) acc[t] = mf16(a, tr_frag<NSTP>(sS, 32 * kc, 16 * t, lane), acc[t]);
        }
    }
#undef WG_LOAD
    // C layout: column s = 16t + l%16, rows l = 16w + 4(l/16) + i
    float* out = part + (int64_t)blockIdx.y * NL * NS;
#pragma unroll
    for (int t = 0; t < NST; t++) {
        int sidx = 16 * t + (lane & 15);
        if (sidx >= NS) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int l = l0 + 16 * w + 4 * (lane >> 4) + i;
            if (l < NL) out[(int64_t)l * NS + sidx] = acc[t][i];
        }
    }
}

// Deferred reduction of every weight-gradient product of a step in one
// launch: job j adds scale * (sum of its partials, split order) into its
// gradient, G_p[l][s] for one pair (gB: [out x r], NS = r) or, TRANS,
// column s of pair s / r into G_p[s % r][l] (gA: [r x in]).  Jobs own
// disjoint gradient elements; job j covers blocks [blk0, blk0 + n / 1024),
// a thread four consecutive elements (one 16-byte load per split when n is
// a multiple of 4; the partial arrays start 256-byte aligned).
__device__ __forceinline__ void wgrad_reduce_store(const WgradJob& J, int64_t idx, float v) {
    const int l = (int)(idx / J.NS), sc = (int)(idx % J.NS);
    if (!J.trans) {
        J.g[0][(int64_t)l * J.NS + sc] += J.scale * v;
    } else {
        const int pp = sc / J.r, j = sc % J.r;
        float* g = pp == 0 ? J.g[0] : pp == 1 ? J.g[1] : J.g[2];
        g[(int64_t)j * J.NL + l] += J.scale * v;
    }
}
__global__ __launch_bounds__(256) void k_wgrad_reduce_jobs(const WgradJob* __restrict__ jobs,
                                                           int njobs) {
    const int64_t b = blockIdx.x;
    int lo = 0, hi = njobs - 1;  // last job with blk0 <= b
    while (lo < hi) {
        int mid = (lo + hi + 1) >> 1;
        if (jobs[mid].blk0 <= b) lo = mid; else hi = mid - 1;
    }
    const WgradJob& J = jobs[lo];
    const int64_t i0 = ((b - J.blk0) * 256 + threadIdx.x) * 4;
    if (i0 >= J.n) return;
    if ((J.n & 3) == 0) {
        // sum over the splits in split order, 8 loads in flight
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        int z = 0;
        for (; z + 8 <= J.splits; z += 8) {
            float4 v[8];
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = *(const float4*)(J.part + (int64_t)(z + i) * J.n + i0);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                acc.x += v[i].x;
                acc.y += v[i].y;
                acc.z += v[i].z;
                acc.w += v[i].w;
            }
        }
        for (; z < J.splits; z++) {
            const float4 v = *(const float4*)(J.part + (int64_t)z * J.n + i0);
            acc.x += v.x;
            acc.y += v.y;
            acc.z += v.z;
            acc.w += v.w;
        }
        wgrad_reduce_store(J, i0, acc.x);
        wgrad_reduce_store(J, i0 + 1, acc.y);
        wgrad_reduce_store(J, i0 + 2, acc.z);
        wgrad_reduce_store(J, i0 + 3, acc.w);
    } else {
        for (int e = 0; e < 4 && i0 + e < J.n; e++)
            wgrad_reduce_store(J, i0 + e, sum_splits(J.part, J.splits, J.n, i0 + e));
    }
}

// ── SwiGLU backward fused with the gate/up LoRA backward (rank 16) ───────
// One pass over dact, gate and up [BT x I] instead of silu_mul_bwd followed
// by two passes each over dgate and dup (the dh product and the gB product
// of adapter_model.cu:131-220 for the gate and up pairs):
//   dgate, dup = silu_mul_bwd(dact, gate, up)                  (ops.cu:925-940)
//   dh_p[t][j] partial over the block's columns of sum_c go_p[t][c] B_p[c][j]
//   gB_p[c][j] partial over the block's tokens  of sum_t go_p[t][c] h_p[t][j]
// with go_0 = bf16(dgate), go_1 = bf16(dup), as the reference's products see
// them.
//
// Block (x, y) of NW waves: columns [64 NW x, 64 NW (x + 1)) (wave w: 64 of
// them) and token range y, walked in 16-token tiles.  Every global load and store of a
// wave covers 8 rows x one whole 128-byte line (lane l: row l/8, columns
// 8 (l%8) .. + 7): lines split between two instructions cost about 20% of
// the bandwidth.  The go tile goes to wave-private LDS, from which the wave
// reads its MFMA operands: rows as the 16x16x32 A operand of the dh product
// (B^T shadow fragments of the wave's columns held in registers), columns
// through transposing reads as the 16x16x16 A operand of the gB product (h
// of the tile, also via wave-private LDS, as B).  gB accumulates in
// registers over the block's tokens (each wave owns its columns); the NW
// waves' dh partials of a tile are added in wave order through LDS (two
// buffers, one barrier per tile).  Inputs are loaded two tiles ahead.
typedef short s16x4_t __attribute__((ext_vector_type(4)));
// byte offset of (row r < 16, column c < 64) in a wave's [16][64] BF16 tile:
// 32-byte units XOR-permuted by (r >> 1) & 3 and their 16-byte halves by
// (r >> 3) & 1, so that row reads (16 rows, 16 B each), transposing reads
// (rows 4g'..4g'+3, g' = 0, 1) and line-shaped writes hit distinct banks
__device__ __forceinline__ int sw_off(int r, int c) {
    return r * 128 + 32 * ((c >> 4) ^ ((r >> 1) & 3)) + 16 * (((c >> 3) & 1) ^ ((r >> 3) & 1)) +
           (c & 7) * 2;
}
__device__ __forceinline__ s16x4_t tr4(const char* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_p)p);
}
__device__ __forceinline__ floatx4 mf16k16(s16x4_t a, s16x4_t b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ u32x4 silu_fwd8(u32x4 gt, u32x4 u) {
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; i++)
        o[i] = pack2(silu_mul_f(lo2f(gt[i]), lo2f(u[i])), silu_mul_f(hi2f(gt[i]), hi2f(u[i])));
    return o;
}
__device__ __forceinline__ void silu_bwd8(u32x4 d, u32x4 gt, u32x4 u, u32x4& dg, u32x4& du) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        float a0, b0, a1, b1;
        silu_bwd_f(lo2f(d[i]), lo2f(gt[i]), lo2f(u[i]), a0, b0);
        silu_bwd_f(hi2f(d[i]), hi2f(gt[i]), hi2f(u[i]), a1, b1);
        dg[i] = pack2(a0, a1);
        du[i] = pack2(b0, b1);
    }
}

template <int NW, bool DG>  // DG: also the down pair's gA partial act^T dh_down
__global__ __launch_bounds__(NW * 64) void k_silu_bwd_lora(
    const bf16* __restrict__ dact, const bf16* __restrict__ gate, const bf16* __restrict__ up,
    bf16* __restrict__ dgate, bf16* __restrict__ dup, const bf16* __restrict__ bt_g,
    const bf16* __restrict__ bt_u, const bf16* __restrict__ h_g, const bf16* __restrict__ h_u,
    float* __restrict__ dh_part, float* __restrict__ gb_g, float* __restrict__ gb_u,
    const bf16* __restrict__ dh_d, float* __restrict__ ga_d, int BT, int I, int per) {
    constexpr int NP = DG ? 3 : 2;  // transposed products: gate gB, up gB (, down gA)
    __shared__ __attribute__((aligned(16))) char sW[NW][NP][16 * 128];  // go (act) tiles per wave
    __shared__ __attribute__((aligned(16))) char sHw[NW][NP][16 * 32];  // h (dh_down) tiles per wave
    __shared__ __attribute__((aligned(16))) float sDh[2][NW][8][64];   // dh partials [buf][wave]
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int g = lane >> 4, j = lane & 15;
    const int t_beg = blockIdx.y * per, t_end = min(BT, t_beg + per);
    const int c0 = blockIdx.x * (NW * 64), cw = c0 + 64 * w;
    const bool act = cw < I;                    // wave-uniform: I is a multiple of 64
    const int nact = min(NW, (I - c0) >> 6);     // active waves of the block
    // line-shaped element of a tile at token tb: rows lane/8 (+ 8i), columns cw + 8 (lane%8)
    const int64_t lofs = (int64_t)(lane >> 3) * I + cw + 8 * (lane & 7);
    // h element of a tile: pair lane/32, row (lane/2)%16, half lane%2
    const int hp = lane >> 5, hrow = (lane >> 1) & 15, hh = lane & 1;
    const bf16* hsrc = (hp ? h_u : h_g) + hrow * 16 + 8 * hh;
    const bf16* dsrc = dh_d + hrow * 16 + 8 * hh;  // (lanes 32.. repeat lanes 0..31)
    char* const sw0 = sW[w][0];
    char* const sw1 = sW[w][1];
    char* const sw2 = sW[w][NP - 1];
    char* const shw = sHw[w][0];
    u32x4 ra[2][2], rg[2][2], ru[2][2], rh[2], rd[2];  // [buffer][row half]
#define SL_LOAD(B, tb)                                                        \
    do {                                                                      \
        const int64_t o_ = (int64_t)(tb) * I + lofs;                          \
        _Pragma("unroll") for (int i = 0; i < 2; i++) {                       \
            ra[B][i] = *(const u32x4*)(dact + o_ + 8 * (int64_t)I * i);       \
            rg[B][i] = *(const u32x4*)(gate + o_ + 8 * (int64_t)I * i);       \
            ru[B][i] = *(const u32x4*)(up + o_ + 8 * (int64_t)I * i);         \
        }                                                                     \
        rh[B] = *(const u32x4*)(hsrc + (int64_t)(tb) * 16);                   \
        if constexpr (DG) rd[B] = *(const u32x4*)(dsrc + (int64_t)(tb) * 16); \
    } while (0)
    bf16x8_t fb[2][2];  // B^T shadow: row j, columns cw + 32 kc + 8g .. + 7
    floatx4 gb[NP][4];  // [product][16-column group] over the block's tokens
#pragma unroll
    for (int q = 0; q < NP; q++)
#pragma unroll
        for (int ct = 0; ct < 4; ct++) gb[q][ct] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (act) {
#pragma unroll
        for (int kc = 0; kc < 2; kc++) {
            fb[0][kc] = *(const bf16x8_t*)(bt_g + (int64_t)j * I + cw + 32 * kc + 8 * g);
            fb[1][kc] = *(const bf16x8_t*)(bt_u + (int64_t)j * I + cw + 32 * kc + 8 * g);
        }
        if (t_beg < t_end) SL_LOAD(0, t_beg);
        if (t_beg + 16 < t_end) SL_LOAD(1, t_beg + 16);
    }
    // transposing-read lane offsets: row 4g + j/4, columns 4 (j%4) ..
    const int rr = 4 * g + (j >> 2), cc = 4 * (j & 3);
    for (int tb0 = t_beg; tb0 < t_end; tb0 += 32) {
#pragma unroll
        for (int B = 0; B < 2; B++) {
            const int tb = tb0 + 16 * B;
            if (tb < t_end) {  // block-uniform
                floatx4 dhw[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
                if (act) {
                    u32x4 og[2], ou[2], oa[2];
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        silu_bwd8(ra[B][i], rg[B][i], ru[B][i], og[i], ou[i]);
                        // act = silu_mul(gate, up) exactly as the forward computed it
                        if constexpr (DG) oa[i] = silu_fwd8(rg[B][i], ru[B][i]);
                    }
                    const u32x4 hv = rh[B];
                    const u32x4 dv = rd[B];
                    if (tb + 32 < t_end) SL_LOAD(B, tb + 32);
                    const int64_t o = (int64_t)tb * I + lofs;
                    const int lr = lane >> 3, lc = 8 * (lane & 7);
#pragma unroll
                    for (int i = 0; i < 2; i++) {
                        *(u32x4*)(dgate + o + 8 * (int64_t)I * i) = og[i];
                        *(u32x4*)(dup + o + 8 * (int64_t)I * i) = ou[i];
                        *(u32x4*)(sw0 + sw_off(lr + 8 * i, lc)) = og[i];
                        *(u32x4*)(sw1 + sw_off(lr + 8 * i, lc)) = ou[i];
                        if constexpr (DG) *(u32x4*)(sw2 + sw_off(lr + 8 * i, lc)) = oa[i];
                    }
                    *(u32x4*)(shw + hp * 512 + tr_off<1>(hrow, 8 * hh)) = hv;
                    if (DG && hp == 0) *(u32x4*)(shw + 1024 + tr_off<1>(hrow, 8 * hh)) = dv;
                    // one wave's LDS instructions execute in order, so the
                    // reads below see the writes above; keep the compiler
                    // from moving them across
                    asm volatile("" ::: "memory");
#pragma unroll
                    for (int kc = 0; kc < 2; kc++) {
                        const bf16x8_t a0 = *(const bf16x8_t*)(sw0 + sw_off(j, 32 * kc + 8 * g));
                        const bf16x8_t a1 = *(const bf16x8_t*)(sw1 + sw_off(j, 32 * kc + 8 * g));
                        dhw[0] = mf16(a0, fb[0][kc], dhw[0]);
                        dhw[1] = mf16(a1, fb[1][kc], dhw[1]);
                    }
                    const s16x4_t hb0 = tr4(shw + tr_off<1>(rr, cc));
                    const s16x4_t hb1 = tr4(shw + 512 + tr_off<1>(rr, cc));
#pragma unroll
                    for (int ct = 0; ct < 4; ct++) {
                        gb[0][ct] = mf16k16(tr4(sw0 + sw_off(rr, 16 * ct + cc)), hb0, gb[0][ct]);
                        gb[1][ct] = mf16k16(tr4(sw1 + sw_off(rr, 16 * ct + cc)), hb1, gb[1][ct]);
                    }
                    if constexpr (DG) {
                        const s16x4_t hb2 = tr4(shw + 1024 + tr_off<1>(rr, cc));
#pragma unroll
                        for (int ct = 0; ct < 4; ct++)
                            gb[NP - 1][ct] =
                                mf16k16(tr4(sw2 + sw_off(rr, 16 * ct + cc)), hb2, gb[NP - 1][ct]);
                    }
                    asm volatile("" ::: "memory");
                }
                // dh of the tile over the block's columns: waves' partials in wave order
#pragma unroll
                for (int pp = 0; pp < 2; pp++)
#pragma unroll
                    for (int i = 0; i < 4; i++) sDh[B][w][pp * 4 + i][lane] = dhw[pp][i];
                __syncthreads();
#pragma unroll
                for (int k = 0; k < 512 / (NW * 64); k++) {
                    const int e = threadIdx.x + NW * 64 * k;
                    const int pp = e >> 8, i = (e >> 6) & 3, ln = e & 63;
                    float v = sDh[B][0][pp * 4 + i][ln];
                    for (int ww = 1; ww < nact; ww++) v += sDh[B][ww][pp * 4 + i][ln];
                    dh_part[(((int64_t)blockIdx.x * 2 + pp) * BT + tb + 4 * (ln >> 4) + i) * 16 +
                            (ln & 15)] = v;
                }
            }
        }
    }
#undef SL_LOAD
    // gB partial of token range y: rows (columns of I) cw + 16ct + 4g + i, rank j
    if (act) {
#pragma unroll
        for (int ct = 0; ct < 4; ct++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t o = ((int64_t)blockIdx.y * I + cw + 16 * ct + 4 * g + i) * 16 + j;
                gb_g[o] = gb[0][ct][i];
                gb_u[o] = gb[1][ct][i];
                if constexpr (DG) ga_d[o] = gb[NP - 1][ct][i];
            }
    }
}

// ── one pass over go for the dh and gB products of up to three pairs ─────
// (adapter_model.cu:131-220, rank 16): dh_p = go_p B_p (column-split
// partials, dh_part [S_o][3][BT][16]) and gB_p = go_p^T h_p (token-split
// partials, gb_p [S_t][N_p][16]).  The pairs' columns are concatenated
// (pair p at columns [c0_p, c0_p + N_p), N_p a multiple of 64), so a wave's
// 64 columns belong to one pair: down or o alone (go = the residual
// gradient), or q, k, v with their own go = dQ, dK, dV.  Same tiling as
// k_silu_bwd_lora: 8 waves x 64 columns per block, 16-token tiles, whole-line
// global loads, wave-private LDS for the MFMA operands, the waves' dh
// partials of one pair added in wave order through LDS.
struct GoPairs {
    const bf16* go[3];
    int64_t ldgo[3];
    const bf16* bt[3];  // B^T shadow [16 x N_p]
    const bf16* h[3];   // [BT x 16]
    float* gb[3];       // [S_t][N_p][16]
    int n[3], c0[3], np, ntot;
};

template <int NW>
__global__ __launch_bounds__(NW * 64) void k_go_lora(GoPairs P, float* __restrict__ dh_part,
                                                     int BT, int per) {
    __shared__ __attribute__((aligned(16))) char sW[NW][16 * 128];  // go tile per wave
    __shared__ __attribute__((aligned(16))) char sHw[NW][16 * 32];  // h tile per wave
    __shared__ __attribute__((aligned(16))) float sDh[2][NW][4][64]; // dh partials [buf][wave]
    __shared__ int sPair[NW];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int g = lane >> 4, j = lane & 15;
    const int t_beg = blockIdx.y * per, t_end = min(BT, t_beg + per);
    const int cw = blockIdx.x * (NW * 64) + 64 * w;  // concatenated column of this wave
    const bool act = cw < P.ntot;                    // wave-uniform
    const int pp = (P.np > 2 && cw >= P.c0[2]) ? 2 : (P.np > 1 && cw >= P.c0[1]) ? 1 : 0;
    const bf16* go = pp == 2 ? P.go[2] : pp == 1 ? P.go[1] : P.go[0];
    const int64_t ld = pp == 2 ? P.ldgo[2] : pp == 1 ? P.ldgo[1] : P.ldgo[0];
    const bf16* bt = pp == 2 ? P.bt[2] : pp == 1 ? P.bt[1] : P.bt[0];
    const bf16* hh = pp == 2 ? P.h[2] : pp == 1 ? P.h[1] : P.h[0];
    float* gbp = pp == 2 ? P.gb[2] : pp == 1 ? P.gb[1] : P.gb[0];
    const int np_ = pp == 2 ? P.n[2] : pp == 1 ? P.n[1] : P.n[0];
    const int lc = cw - (pp == 2 ? P.c0[2] : pp == 1 ? P.c0[1] : P.c0[0]);  // column in pair
    if (lane == 0) sPair[w] = act ? pp : -1;
    // whole-line element of a tile at token tb: rows lane/8 (+ 8i), columns lc + 8 (lane%8)
    const int64_t lofs = (int64_t)(lane >> 3) * ld + lc + 8 * (lane & 7);
    const int hrow = (lane >> 1) & 15, hh8 = lane & 1;  // h tile: lanes 0..31 load
    char* const sw = sW[w];
    char* const shw = sHw[w];
    u32x4 rg[2][2], rh[2];
#define GO_LOAD(B, tb)                                                       \
    do {                                                                     \
        const int64_t o_ = (int64_t)(tb) * ld + lofs;                        \
        rg[B][0] = *(const u32x4*)(go + o_);                                 \
        rg[B][1] = *(const u32x4*)(go + o_ + 8 * ld);                        \
        rh[B] = *(const u32x4*)(hh + (int64_t)((tb) + hrow) * 16 + 8 * hh8); \
    } while (0)
    bf16x8_t fb[2];  // B^T: row j, columns lc + 32 kc + 8g .. + 7
    floatx4 gb[4];
#pragma unroll
    for (int ct = 0; ct < 4; ct++) gb[ct] = floatx4{0.f, 0.f, 0.f, 0.f};
    if (act) {
#pragma unroll
        for (int kc = 0; kc < 2; kc++)
            fb[kc] = *(const bf16x8_t*)(bt + (int64_t)j * np_ + lc + 32 * kc + 8 * g);
        if (t_beg < t_end) GO_LOAD(0, t_beg);
        if (t_beg + 16 < t_end) GO_LOAD(1, t_beg + 16);
    }
    __syncthreads();  // sPair
    const int rr = 4 * g + (j >> 2), cc = 4 * (j & 3);
    for (int tb0 = t_beg; tb0 < t_end; tb0 += 32) {
#pragma unroll
        for (int B = 0; B < 2; B++) {
            const int tb = tb0 + 16 * B;
            if (tb < t_end) {  // block-uniform
                floatx4 dhw = floatx4{0.f, 0.f, 0.f, 0.f};
                if (act) {
                    const u32x4 v0 = rg[B][0], v1 = rg[B][1], hv = rh[B];
                    if (tb + 32 < t_end) GO_LOAD(B, tb + 32);
                    const int lr = lane >> 3, lcc = 8 * (lane & 7);
                    *(u32x4*)(sw + sw_off(lr, lcc)) = v0;
                    *(u32x4*)(sw + sw_off(lr + 8, lcc)) = v1;
                    if (lane < 32) *(u32x4*)(shw + tr_off<1>(hrow, 8 * hh8)) = hv;
                    // one wave's LDS instructions execute in order
                    asm volatile("" ::: "memory");
#pragma unroll
                    for (int kc = 0; kc < 2; kc++)
                        dhw = mf16(*(const bf16x8_t*)(sw + sw_off(j, 32 * kc + 8 * g)), fb[kc], dhw);
                    const s16x4_t hb = tr4(shw + tr_off<1>(rr, cc));
#pragma unroll
                    for (int ct = 0; ct < 4; ct++)
                        gb[ct] = mf16k16(tr4(sw + sw_off(rr, 16 * ct + cc)), hb, gb[ct]);
                    asm volatile("" ::: "memory");
                }
                // dh of the tile per pair over the block's columns, waves in order
#pragma unroll
                for (int i = 0; i < 4; i++) sDh[B][w][i][lane] = dhw[i];
                __syncthreads();
                for (int e = threadIdx.x; e < 3 * 256; e += NW * 64) {
                    const int q = e >> 8, i = (e >> 6) & 3, ln = e & 63;
                    float v = 0.f;
                    bool any = false;
                    for (int ww = 0; ww < NW; ww++)
                        if (sPair[ww] == q) {
                            v = any ? v + sDh[B][ww][i][ln] : sDh[B][ww][i][ln];
                            any = true;
                        }
                    if (any)
                        dh_part[(((int64_t)blockIdx.x * 3 + q) * BT + tb + 4 * (ln >> 4) + i) * 16 +
                                (ln & 15)] = v;
                }
            }
        }
    }
#undef GO_LOAD
    if (act) {
#pragma unroll
        for (int ct = 0; ct < 4; ct++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                gbp[((int64_t)blockIdx.y * np_ + lc + 16 * ct + 4 * g + i) * 16 + j] = gb[ct][i];
    }
}

// dh[t][16p + j] = bf16(sum over the column blocks holding pair p, in order,
// of dh_part[s][p][t][j])
__global__ __launch_bounds__(256) void k_dh_reduce_go(const float* __restrict__ dh_part, GoPairs P,
                                                      int bcols, int BT, bf16* __restrict__ dh,
                                                      int64_t ldh) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= (int64_t)BT * 16 * P.np) return;
    const int64_t t = q / (16 * P.np);
    const int pp = (int)(q / 16 % P.np), jj = (int)(q & 15);
    const int c0 = pp == 2 ? P.c0[2] : pp == 1 ? P.c0[1] : P.c0[0];
    const int n = pp == 2 ? P.n[2] : pp == 1 ? P.n[1] : P.n[0];
    float v = 0.f;
    for (int sb = c0 / bcols; sb <= (c0 + n - 1) / bcols; sb++)
        v += dh_part[(((int64_t)sb * 3 + pp) * BT + t) * 16 + jj];
    dh[t * ldh + 16 * pp + jj] = f2bf(v);
}

// dh[t][16p + j] = bf16(sum over the column splits, in order, of dh_part[s][p][t][j])
__global__ __launch_bounds__(256) void k_dh_reduce2(const float* __restrict__ dh_part, int s_o,
                                                    int BT, bf16* __restrict__ dh, int64_t ldh) {
    const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (q >= (int64_t)BT * 32) return;
    const int64_t t = q >> 5;
    const int pp = (int)(q >> 4) & 1, jj = (int)q & 15;
    float v = 0.f;
    for (int s = 0; s < s_o; s++) v += dh_part[(((int64_t)s * 2 + pp) * BT + t) * 16 + jj];
    dh[t * ldh + 16 * pp + jj] = f2bf(v);
}

// ── host launchers ────────────────────────────────────────────────────────
int lora_skinny_nt(const bf16* X, int64_t ldx, int M, int K, int r, const bf16* const* Y,
                   bf16* const* C, int64_t ldc, int n, hipStream_t s) {
    TA_REQUIRE(n >= 1 && n <= 3 && r >= 1 && M > 0 && K > 0, "lora_skinny_nt: bad arguments");
    TA_REQUIRE(((uintptr_t)X & 15) == 0 && (ldx & 7) == 0 && (K & 7) == 0,
               "lora_skinny_nt: X rows must be 16-byte aligned and K a multiple of 8");
    Pairs3 p{};
    p.n = n;
    p.ldc = ldc;
    for (int i = 0; i < n; i++) {
        p.y[i] = Y[i];
        p.c[i] = C[i];
        TA_REQUIRE(((uintptr_t)Y[i] & 15) == 0, "lora_skinny_nt: Y must be 16-byte aligned");
    }
    int nt = (n * r + 15) / 16;
    dim3 grid((M + 16 * SK_RG - 1) / (16 * SK_RG));
    const bool timed = kprof_begin(KP_LORA_SKINNY, s);
    const bool dma = ((uintptr_t)X & 15) == 0 && (ldx & 7) == 0 && (K & 7) == 0 && nt <= 4;
    if (dma) {
        switch (nt) {
            case 1: tlaunch(k_skinny_dma<1, 6>, dim3(grid), dim3(SK_W * 64), s, X, ldx, M, K, r, p); break;
            case 2: tlaunch(k_skinny_dma<2, 4>, dim3(grid), dim3(SK_W * 64), s, X, ldx, M, K, r, p); break;
            case 3: tlaunch(k_skinny_dma<3, 3>, dim3(grid), dim3(SK_W * 64), s, X, ldx, M, K, r, p); break;
            default: tlaunch(k_skinny_dma<4, 3>, dim3(grid), dim3(SK_W * 64), s, X, ldx, M, K, r, p); break;
        }
    } else switch (nt) {
        case 1: tlaunch(k_skinny_nt<1, 4>, dim3(grid), dim3(SK_W * 64), s, X, ldx, M, K, r, p); break;
        case 2: tlaunch(k_skinny_nt<2, 4>, dim3(grid), dim3(SK_W * 64), s, X, ldx, M, K, r, p); break;
        case 3: tlaunch(k_skinny_nt<3, 3>, dim3(grid), dim3(SK_W * 64), s, X, ldx, M, K, r, p); break;
        case 4: tlaunch(k_skinny_nt<4, 2>, dim3(grid), dim3(SK_W * 64), s, X, ldx, M, K, r, p); break;
        case 6: tlaunch(k_skinny_nt<6, 2>, dim3(grid), dim3(SK_W * 64), s, X, ldx, M, K, r, p); break;
        case 8: tlaunch(k_skinny_nt<8, 1>, dim3(grid), dim3(SK_W * 64), s, X, ldx, M, K, r, p); break;
        case 12: tlaunch(k_skinny_nt<12, 1>, dim3(grid), dim3(SK_W * 64), s, X, ldx, M, K, r, p); break;
        default: return set_error(-1, "lora_skinny_nt: %d pairs x rank %d unsupported", n, r);
    }
    if (timed)  // X and the Y_p read once, C_p written once
        kprof_end(KP_LORA_SKINNY, s, 2.0 * M * K * n * r,
                  2.0 * ((double)M * K + (double)n * r * K + (double)M * n * r),
                  "ta::k_skinny_dma + ta::k_skinny_nt (all instances)");
    return check_launch("lora_skinny_nt");
}

int lora_rank_update(bool delta, bf16* Y, int64_t ldy, int M, int N, int r, float scale,
                     const bf16* const* U, const int64_t* ldu, const bf16* const* V, int n,
                     hipStream_t s) {
    TA_REQUIRE(n >= 1 && n <= 3 && r >= 1 && r <= 64, "lora_rank_update: bad arguments");
    Pairs3 p{};
    p.n = n;
    for (int i = 0; i < n; i++) {
        p.u[i] = U[i];
        p.ldu[i] = ldu[i];
        p.y[i] = V[i];
        TA_REQUIRE(((uintptr_t)U[i] & 15) == 0 && (ldu[i] & 7) == 0,
                   "lora_rank_update: U rows must be 16-byte aligned");
    }
    dim3 grid((N + 63) / 64, (M + 63) / 64);
    int rk = (r + 31) / 32 * 32;
#define RU(D, R) tlaunch(k_rank_update<D, R>, dim3(grid), dim3(256), s, Y, ldy, M, N, r, scale, p)
    if (delta) {
        if (rk == 32) RU(true, 32); else RU(true, 64);
    } else {
        if (rk == 32) RU(false, 32); else RU(false, 64);
    }
#undef RU
    return check_launch("lora_rank_update");
}

// Token splits of a weight-gradient product over T tokens with NL large-side
// columns: enough blocks (64 columns x one token range each) to fill the
// chip.  *per receives the tokens per split (a multiple of the tile).
int lora_wgrad_splits(int NL, int T, int* per) {
    int ltiles = (NL + 63) / 64;
    int tiles_t = (T + WG_TK - 1) / WG_TK;
    int splits = (768 + ltiles - 1) / ltiles;
    if (splits > tiles_t) splits = tiles_t;
    if (splits < 1) splits = 1;
    *per = (tiles_t + splits - 1) / splits * WG_TK;
    return (T + *per - 1) / *per;
}

// partials part[z][l][s] = sum over the tokens of split z of L[t][l] Sm[t][s]
// (part holds lora_wgrad_splits(NL, T) x NL x NS floats); the reduction into
// the gradient runs later, for all products of the step at once
// (lora_wgrad_reduce_jobs).
int lora_wgrad_part(const bf16* L, int64_t ldl, int NL, const bf16* Sm, int64_t lds, int NS, int T,
                    float* part, hipStream_t s) {
    TA_REQUIRE(NL > 0 && NS > 0 && NS <= 192 && T > 0 && part, "lora_wgrad_part: bad arguments");
    int per = 0;
    const int splits = lora_wgrad_splits(NL, T, &per);
    dim3 grid((NL + 63) / 64, splits);
    int nst = (NS + 15) / 16;
    const bool timed = kprof_begin(KP_LORA_WGRAD, s);
    // 16-byte row loads need aligned rows and column counts in whole chunks
    const bool vec = ((ldl & 7) == 0) && (((uintptr_t)L & 15) == 0) && ((lds & 7) == 0) &&
                     (((uintptr_t)Sm & 15) == 0) && (NL % 8) == 0 && (NS % 8) == 0;
#define WG(N)                                                                                  \
    do {                                                                                       \
        if (vec)                                                                               \
            tlaunch(k_wgrad<N, true>, dim3(grid), dim3(256), s, L, ldl, NL, Sm, lds, NS, T, per, part);      \
        else                                                                                   \
            tlaunch(k_wgrad<N, false>, dim3(grid), dim3(256), s, L, ldl, NL, Sm, lds, NS, T, per, part);     \
    } while (0)
    switch (nst) {
        case 1: WG(1); break;
        case 2: WG(2); break;
        case 3: WG(3); break;
        case 4: WG(4); break;
        case 6: WG(6); break;
        case 8: WG(8); break;
        case 9: WG(9); break;
        case 12: WG(12); break;
        default: return set_error(-1, "lora_wgrad_part: %d small columns unsupported", NS);
    }
#undef WG
    if (timed)  // L and Sm read once
        kprof_end(KP_LORA_WGRAD, s, 2.0 * T * NL * NS, 2.0 * ((double)T * NL + (double)T * NS),
                  "ta::k_wgrad + ta::k_wgrad_reduce_jobs (all instances)");
    return check_launch("lora_wgrad_part");
}

// jobs: device array of njobs WgradJob sorted by blk0, covering total_blocks
int lora_wgrad_reduce_jobs(const WgradJob* jobs, int njobs, int64_t total_blocks, double elems,
                           hipStream_t s) {
    if (njobs <= 0) return 0;
    TA_REQUIRE(total_blocks > 0 && total_blocks < (1ll << 31), "lora_wgrad_reduce_jobs: %lld blocks",
               (long long)total_blocks);
    const bool timed = kprof_begin(KP_LORA_WGRAD, s);
    tlaunch(k_wgrad_reduce_jobs, dim3((unsigned)total_blocks), dim3(256), s, jobs, njobs);
    if (timed)  // every gradient element read and written once (F32)
        kprof_end(KP_LORA_WGRAD, s, 0.0, 8.0 * elems,
                  "ta::k_wgrad + ta::k_wgrad_reduce_jobs (all instances)");
    return check_launch("lora_wgrad_reduce_jobs");
}

// k_silu_bwd_lora grid: SL_NW waves of 64 columns per block (512 columns:
// half the dh partials of 256-column blocks, measured a little faster); the
// tokens are cut into as many ranges (multiples of 32 tokens) as keep every
// block resident at once (blocks per CU from the occupancy query, once per
// process): more blocks in flight than that were measured slower
static constexpr int SL_NW = 8;
static int silu_lora_plan(int BT, int I, int* s_t, int* s_o, int* per) {
    static int resident = 0;
    if (!resident) {
        int nb = 0, dev = 0, ncu = 0;
        TA_HIP(hipGetDevice(&dev));
        TA_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
        TA_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_silu_bwd_lora<SL_NW, true>,
                                                            SL_NW * 64, 0));
        resident = std::max(1, nb) * std::max(1, ncu);
    }
    *s_o = (I + SL_NW * 64 - 1) / (SL_NW * 64);
    int ranges = std::max(1, std::min(resident / *s_o, BT / 32));
    *per = (BT / ranges + 31) / 32 * 32;
    *s_t = (BT + *per - 1) / *per;
    return 0;
}
int silu_lora_splits(int BT, int I, int* s_t, int* s_o) {
    int per = 0;
    return silu_lora_plan(BT, I, s_t, s_o, &per);
}

int silu_bwd_lora(const bf16* dact, const bf16* gate, const bf16* up, bf16* dgate, bf16* dup,
                  const bf16* bt_g, const bf16* bt_u, const bf16* h_g, const bf16* h_u,
                  float* dh_part, float* gb_g, float* gb_u, const bf16* dh_d, float* ga_d, int BT,
                  int I, hipStream_t s) {
    TA_REQUIRE(BT > 0 && I > 0 && BT % 64 == 0 && I % 64 == 0,
               "silu_bwd_lora: BT %d and I %d must be positive multiples of 64", BT, I);
    const void* ptrs[] = {dact, gate, up, dgate, dup, bt_g, bt_u, h_g, h_u, dh_part, gb_g, gb_u};
    for (const void* q : ptrs)
        TA_REQUIRE(q && ((uintptr_t)q & 15) == 0, "silu_bwd_lora: null or unaligned operand");
    TA_REQUIRE(!dh_d == !ga_d && ((uintptr_t)dh_d & 15) == 0 && ((uintptr_t)ga_d & 15) == 0,
               "silu_bwd_lora: the down pair's dh and gA partials come together, aligned");
    int s_t = 0, s_o = 0, per = 0;
    if (int rc = silu_lora_plan(BT, I, &s_t, &s_o, &per)) return rc;
    const dim3 grid(s_o, s_t);
    if (ga_d)
        tlaunch(k_silu_bwd_lora<SL_NW, true>, dim3(grid), dim3(SL_NW * 64), s, dact, gate, up, dgate, dup, bt_g, bt_u, h_g, h_u, dh_part, gb_g, gb_u, dh_d, ga_d, BT, I,
            per);
    else
        tlaunch(k_silu_bwd_lora<SL_NW, false>, dim3(grid), dim3(SL_NW * 64), s, dact, gate, up, dgate, dup, bt_g, bt_u, h_g, h_u, dh_part, gb_g, gb_u, dh_d, ga_d, BT, I,
            per);
    return check_launch("silu_bwd_lora");
}

int dh_reduce2(const float* dh_part, int s_o, int BT, bf16* dh, int64_t ldh, hipStream_t s) {
    TA_REQUIRE(dh_part && dh && s_o > 0 && BT > 0 && ldh >= 32, "dh_reduce2: bad arguments");
    const int64_t n = (int64_t)BT * 32;
    tlaunch(k_dh_reduce2, dim3((unsigned)((n + 255) / 256)), dim3(256), s, dh_part, s_o, BT, dh, ldh);
    return check_launch("dh_reduce2");
}

// k_go_lora grid: 8 waves x 64 columns per block over the pairs'
// concatenated columns; token ranges (multiples of 32) sized so that every
// block is resident at once.  *s_t: token splits (the gB partials' count),
// *s_o: column blocks.
static constexpr int GL_NW = 8;
static int go_lora_plan(int BT, int ntot, int* s_t, int* s_o, int* per) {
    static int resident = 0;
    if (!resident) {
        int nb = 0, dev = 0, ncu = 0;
        TA_HIP(hipGetDevice(&dev));
        TA_HIP(hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev));
        TA_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_go_lora<GL_NW>, GL_NW * 64, 0));
        resident = std::max(1, nb) * std::max(1, ncu);
    }
    *s_o = (ntot + GL_NW * 64 - 1) / (GL_NW * 64);
    const int ranges = std::max(1, std::min(resident / *s_o, BT / 32));
    *per = (BT / ranges + 31) / 32 * 32;
    *s_t = (BT + *per - 1) / *per;
    return 0;
}
int go_lora_splits(int BT, int ntot, int* s_t, int* s_o) {
    int per = 0;
    return go_lora_plan(BT, ntot, s_t, s_o, &per);
}

int go_lora(const bf16* const* go, const int64_t* ldgo, const bf16* const* bt, const bf16* const* h,
            float* const* gb, const int* n, int np, int BT, float* dh_part, bf16* dh, int64_t ldh,
            hipStream_t s) {
    TA_REQUIRE(np >= 1 && np <= 3 && BT > 0 && BT % 32 == 0 && dh_part && dh,
               "go_lora: bad arguments (np %d, BT %d)", np, BT);
    GoPairs P{};
    int c = 0;
    for (int q = 0; q < np; q++) {
        TA_REQUIRE(n[q] > 0 && n[q] % 64 == 0 && ldgo[q] % 8 == 0 && go[q] && bt[q] && h[q] &&
                       gb[q] && ((uintptr_t)go[q] & 15) == 0 && ((uintptr_t)bt[q] & 15) == 0 &&
                       ((uintptr_t)h[q] & 15) == 0,
                   "go_lora: pair %d: N %d must be a multiple of 64, operands 16-byte aligned", q,
                   n[q]);
        P.go[q] = go[q];
        P.ldgo[q] = ldgo[q];
        P.bt[q] = bt[q];
        P.h[q] = h[q];
        P.gb[q] = gb[q];
        P.n[q] = n[q];
        P.c0[q] = c;
        c += n[q];
    }
    P.np = np;
    P.ntot = c;
    int s_t = 0, s_o = 0, per = 0;
    if (int rc = go_lora_plan(BT, c, &s_t, &s_o, &per)) return rc;
    tlaunch(k_go_lora<GL_NW>, dim3(dim3(s_o, s_t)), dim3(GL_NW * 64), s, P, dh_part, BT, per);
    const int64_t nel = (int64_t)BT * 16 * np;
    tlaunch(k_dh_reduce_go, dim3((unsigned)((nel + 255) / 256)), dim3(256), s, dh_part, P, GL_NW * 64, BT, dh,
                                                                  ldh);
    return check_launch("go_lora");
}


}  // namespace ta
