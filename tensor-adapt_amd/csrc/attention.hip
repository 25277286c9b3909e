// attention.hip — causal GQA attention with saved probabilities on gfx950
// (v_mfma_f32_16x16x32_bf16), replacing sdpa_fwd_batched / sdpa_bwd_batched
// (src/backend/cuda/ops.cu:578-681, 707-870).
//
// Layouts are the reference's: Q/dO/dQ [B*T, Hq*hd], K/V/dK/dV
// [B*T, Hkv*hd] BF16, probabilities P [B*Hq, T, T] F32 (zeros above the
// diagonal); kv head = hq / (Hq/Hkv).  Nothing is packed, expanded or cast:
// kernels read the strided heads in place (the reference launches 6 layout
// kernels and allocates ~1.3 GB of temporaries per call at the headline
// shape).
//
// Tiles are 64 queries x 64 keys.  A block is 4 waves; in the forward and
// the dQ kernel wave w owns query rows 16w..16w+15 of the block's tile, so
// softmax row statistics reduce over 16 lanes with xor shuffles.  The MFMA
// C layout (lane: column l%16, rows 4*(l/16)+r) is converted to the A
// operand layout (row l%16, 8 consecutive k) through a per-wave LDS tile.
// Every loop over tiles loads the next tile's operands into registers while
// the current tile computes, so global latency overlaps the MFMAs.
//
// Forward with stored probabilities (the C-ABI's sdpa_fwd; per b, hq,
// query tile; heaviest tiles launch first; the engine's forward, which
// stores no P, is k_attn_fwd_t below):
//   pass 1: online row max / sum of exp over key tiles 0..diag;
//   pass 2: recompute S, P = exp(S - max) / sum (the reference's softmax,
//   ops.cu:352-396), store P (F32), O += P*V; O is stored in BF16 and, for
//   the backward's row dots, in F32.
// Every product whose left operand is an F32 quantity (P, dS) runs as two
// MFMAs on its BF16 hi/lo split, keeping ~16 mantissa bits: the reference
// computes these GEMMs in F32 (ops.cu:628-855).
// Backward:
//   row dots D = sum_k P dP (ops.cu:405-435) = dO . O with the F32 O of the
//   forward (k_attn_rowdot_o), or from P and dP = dO V^T when no F32 O is
//   at hand (k_attn_rowdot_p, the C-ABI's sdpa_bwd);
//   k_attn_bwd_dq (per b, hq, query tile): dS = P (dP - D), dQ = scale dS K;
//   k_attn_bwd_dkv (per b, hq, key tile): dV_h = P^T dO and
//   dK_h = scale dS^T Q for the query head as F32 partials, then
//   k_attn_dkv_reduce sums the heads of each GQA group in head order — the
//   group sum of ops.cu:539-555 without atomics, so dK/dV are deterministic.
#include <float.h>
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "lds_tr.hpp"
#include "ta_internal.hpp"

namespace ta {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int TQ = 64, TK = 64;
constexpr int LDT = TK + 8;  // stride of [hd][key] and [row][key] LDS tiles

__device__ __forceinline__ floatx4 mfma16(bf16x8_t a, bf16x8_t b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx4 zero4() {
    floatx4 z;
    z[0] = z[1] = z[2] = z[3] = 0.f;
    return z;
}
__device__ __forceinline__ bf16x8_t ld_frag(const bf16* p) { return *(const bf16x8_t*)p; }

// 16 bytes of a head row from global memory (row < T guarded, zero beyond).
__device__ __forceinline__ bf16x8_t ld_head8(const bf16* base, int64_t row_stride, int row,
                                             int T, int col) {
    if (row < T) return *(const bf16x8_t*)(base + (int64_t)row * row_stride + col);
    bf16x8_t z;
#pragma unroll
    for (int e = 0; e < 8; e++) z[e] = (__bf16)0.f;
    return z;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Rows [r0, r0+64) of one head ([row][HD] in global memory, row stride rs),
// held in registers between load() and store() so that the next tile's
// global loads overlap the current tile's MFMAs.  store() writes LDS
// [row][HD + 8] (K-contiguous rows for MFMA operands over hd).
template <int HD>
struct Rows64 {
    static constexpr int CPR = HD / 8;         // 16-byte chunks per row
    static constexpr int NR = 64 * CPR / 256;  // chunks per thread
    u32x4 v[NR];
    __device__ __forceinline__ void load(const bf16* __restrict__ g, int64_t rs, int r0, int T) {
#pragma unroll
        for (int i = 0; i < NR; i++) {
            int q = threadIdx.x + 256 * i;
            int r = q / CPR, c = (q % CPR) * 8;
            v[i] = (r0 + r < T) ? *(const u32x4*)(g + (int64_t)(r0 + r) * rs + c)
                                : u32x4{0u, 0u, 0u, 0u};
        }
    }
    __device__ __forceinline__ void store(bf16* __restrict__ s) const {
#pragma unroll
        for (int i = 0; i < NR; i++) {
            int q = threadIdx.x + 256 * i;
            *(u32x4*)(s + (q / CPR) * (HD + 8) + (q % CPR) * 8) = v[i];
        }
    }
};

// The same 64 rows loaded as 4 consecutive rows x 8 columns per thread, so
// they can be written transposed to LDS [HD][64 + 8] (row index contiguous)
// with one 8-byte word per column (store_t), and/or as rows (store_rows).
template <int HD>
struct Rows64T {
    static constexpr int NG = 16 * (HD / 8);  // 4-row x 8-column groups
    u32x4 v[4];
    __device__ __forceinline__ void load(const bf16* __restrict__ g, int64_t rs, int r0, int T) {
        int q = threadIdx.x;
        if (q >= NG) return;
        int rg = q & 15, c = (q >> 4) * 8;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            int row = r0 + 4 * rg + i;
            v[i] = (row < T) ? *(const u32x4*)(g + (int64_t)row * rs + c) : u32x4{0u, 0u, 0u, 0u};
        }
    }
    __device__ __forceinline__ void store_t(bf16* __restrict__ s) const {
        int q = threadIdx.x;
        if (q >= NG) return;
        int rg = q & 15, c = (q >> 4) * 8;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            int j = e >> 1, sh = (e & 1) * 16;
            uint64_t word = (uint64_t)((v[0][j] >> sh) & 0xffffu) |
                            ((uint64_t)((v[1][j] >> sh) & 0xffffu) << 16) |
                            ((uint64_t)((v[2][j] >> sh) & 0xffffu) << 32) |
                            ((uint64_t)((v[3][j] >> sh) & 0xffffu) << 48);
            *(uint64_t*)(s + (c + e) * LDT + 4 * rg) = word;
        }
    }
    __device__ __forceinline__ void store_rows(bf16* __restrict__ s) const {
        int q = threadIdx.x;
        if (q >= NG) return;
        int rg = q & 15, c = (q >> 4) * 8;
#pragma unroll
        for (int i = 0; i < 4; i++) *(u32x4*)(s + (4 * rg + i) * (HD + 8) + c) = v[i];
    }
};

// Orders this wave's LDS writes before its later LDS reads (a wave's LDS
// operations complete in order; this keeps the compiler from moving them).
__device__ __forceinline__ void wave_sync() { __builtin_amdgcn_wave_barrier(); }

// S (or dP) for one wave: 16 rows x 64 keys = 4 MFMA tiles, A fragments in
// registers (af[HD/32]), B rows from an LDS [key][HD+8] tile.
template <int HD>
__device__ __forceinline__ void wave_qk(floatx4 (&S)[4], const bf16x8_t (&af)[HD / 32],
                                        const bf16* __restrict__ sB, int lane) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
        S[t] = zero4();
        const bf16* rowp = sB + (16 * t + (lane & 15)) * (HD + 8) + 8 * (lane >> 4);
#pragma unroll
        for (int ks = 0; ks < HD / 32; ks++) S[t] = mfma16(af[ks], ld_frag(rowp + 32 * ks), S[t]);
    }
}

// acc[16 x HD] += A[16 x 64] * B[64 x HD]; A (an F32 quantity: P or dS)
// arrives as two BF16 tiles, hi = bf16(a) and lo = bf16(a - hi), in this
// wave's LDS slots sA[0], sA[1] ([16][LDT], k contiguous), so the product
// keeps ~16 mantissa bits of A like the reference's F32 GEMMs; B^T comes
// from LDS [HD][LDT] (exact BF16 values).
template <int HD>
__device__ __forceinline__ void wave_pv(floatx4 (&acc)[HD / 16], const bf16* __restrict__ sAhi,
                                        const bf16* __restrict__ sAlo,
                                        const bf16* __restrict__ sBt, int lane) {
#pragma unroll
    for (int kc = 0; kc < 2; kc++) {
        bf16x8_t ah = ld_frag(sAhi + (lane & 15) * LDT + 32 * kc + 8 * (lane >> 4));
        bf16x8_t al = ld_frag(sAlo + (lane & 15) * LDT + 32 * kc + 8 * (lane >> 4));
#pragma unroll
        for (int j = 0; j < HD / 16; j++) {
            bf16x8_t b = ld_frag(sBt + (16 * j + (lane & 15)) * LDT + 32 * kc + 8 * (lane >> 4));
            acc[j] = mfma16(al, b, acc[j]);
            acc[j] = mfma16(ah, b, acc[j]);
        }
    }
}

// store an F32 value as its hi/lo BF16 pair into two LDS tiles
__device__ __forceinline__ void put_split(bf16* hi, bf16* lo, int idx, float v) {
    bf16 h = f2bf(v);
    hi[idx] = h;
    lo[idx] = f2bf(v - bf2f(h));
}

__device__ __forceinline__ float red16_max(float v) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ float red16_sum(float v) {
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// ── forward ───────────────────────────────────────────────────────────────
// Scores are kept in base-2 units (S * scale * log2 e) so that every
// exponential is one v_exp_f32.  Only the diagonal key tile needs the causal
// (and T) mask: every key of an earlier tile precedes every query row.  P
// leaves as F32 rows to global memory and, split into BF16 hi/lo, into a
// per-wave LDS tile stored [key][row] (4 rows of one key per 8-byte write);
// the P·V MFMA operands (8 consecutive keys per lane) come out of that tile
// and out of V, staged in its natural [key][hd] layout, through the
// transposing LDS read.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

template <int HD, bool SP>  // SP: store P (else only the row statistics)
__global__ __launch_bounds__(256) void k_attn_fwd(const bf16* __restrict__ Q,
                                                  const bf16* __restrict__ K,
                                                  const bf16* __restrict__ V,
                                                  bf16* __restrict__ O, float* __restrict__ O32,
                                                  float* __restrict__ P, float2* __restrict__ stats,
                                                  int T, int Hq, int Hkv, float scale,
                                                  int zero_fill) {
    constexpr int VST = HD / 16;  // 32-byte units of a V row
    __shared__ __attribute__((aligned(16))) bf16 sK[TK * (HD + 8)];
    __shared__ __attribute__((aligned(16))) char sV[TK * HD * 2];
    __shared__ __attribute__((aligned(16))) char sP[4][2][TK * 16 * 2];
    int nqt = (T + TQ - 1) / TQ;
    int nbh = gridDim.x / nqt;
    int qt = nqt - 1 - (int)(blockIdx.x / nbh);  // longest rows launch first
    int bh = (int)(blockIdx.x % nbh);
    int b = bh / Hq, hq = bh % Hq, hkv = hq / (Hq / Hkv);
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int64_t qs = (int64_t)Hq * HD, ks_ = (int64_t)Hkv * HD;
    const bf16* Qh = Q + (int64_t)b * T * qs + hq * HD;
    const bf16* Kh = K + (int64_t)b * T * ks_ + hkv * HD;
    const bf16* Vh = V + (int64_t)b * T * ks_ + hkv * HD;
    float* Ph = SP ? P + (int64_t)bh * T * T : nullptr;
    int q0 = qt * TQ;
    int rowA = q0 + 16 * w + (lane & 15);  // A-operand row of this lane
    bf16x8_t qf[HD / 32];
#pragma unroll
    for (int ks = 0; ks < HD / 32; ks++) qf[ks] = ld_head8(Qh, qs, rowA, T, 32 * ks + 8 * (lane >> 4));
    const int rbase = q0 + 16 * w + 4 * (lane >> 4);  // C-layout rows rbase + r
    const float sl2 = scale * kLog2e;
    Rows64<HD> lk, lv;

    // pass 1: online max / sum of exp2 (per-lane partial sums, shared max)
    float m[4], l[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        m[r] = -INFINITY;
        l[r] = 0.f;
    }
    lk.load(Kh, ks_, 0, T);
    for (int kt = 0; kt <= qt; kt++) {
        __syncthreads();  // every wave is done with the previous tile
        lk.store(sK);
        __syncthreads();
        if (kt < qt) lk.load(Kh, ks_, (kt + 1) * TK, T);
        floatx4 S[4];
        wave_qk<HD>(S, qf, sK, lane);
        const bool diag = kt == qt;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int row = rbase + r;
            float v[4], tmax = -INFINITY;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int key = kt * TK + 16 * t + (lane & 15);
                v[t] = (!diag || (key <= row && key < T)) ? S[t][r] * sl2 : -INFINITY;
                tmax = fmaxf(tmax, v[t]);
            }
            const float mn = fmaxf(m[r], red16_max(tmax));
            float add = 0.f;
#pragma unroll
            for (int t = 0; t < 4; t++) add += exp2_fast(v[t] - mn);
            l[r] = (m[r] == -INFINITY ? 0.f : l[r] * exp2_fast(m[r] - mn)) + add;
            m[r] = mn;
        }
    }
    float inv[4];
    bool rowok[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        inv[r] = 1.f / red16_sum(l[r]);
        rowok[r] = rbase + r < T;
        // (max, 1 / sum) of the row: P = exp2(S scale log2e - max) / sum is
        // recomputed from them, bit for bit, where P is not stored
        if (stats && rowok[r] && (lane & 15) == 0)
            stats[(int64_t)bh * T + rbase + r] = make_float2(m[r], inv[r]);
    }

    // pass 2: P, O
    floatx4 acc[HD / 16];
#pragma unroll
    for (int j = 0; j < HD / 16; j++) acc[j] = zero4();
    lk.load(Kh, ks_, 0, T);
    lv.load(Vh, ks_, 0, T);
    char* sPh = sP[w][0];
    char* sPl = sP[w][1];
    for (int kt = 0; kt <= qt; kt++) {
        __syncthreads();
        lk.store(sK);
#pragma unroll
        for (int i = 0; i < Rows64<HD>::NR; i++) {
            int q = threadIdx.x + 256 * i;
            *(u32x4*)(sV + tr_off<VST>(q / (HD / 8), (q % (HD / 8)) * 8)) = lv.v[i];
        }
        __syncthreads();
        if (kt < qt) {
            lk.load(Kh, ks_, (kt + 1) * TK, T);
            lv.load(Vh, ks_, (kt + 1) * TK, T);
        }
        floatx4 S[4];
        wave_qk<HD>(S, qf, sK, lane);
        const bool diag = kt == qt;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int kl = 16 * t + (lane & 15);
            const int key = kt * TK + kl;
            float p[4];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                p[r] = exp2_fast(S[t][r] * sl2 - m[r]) * inv[r];
                if (diag && !(key <= rbase + r && key < T)) p[r] = 0.f;
                if constexpr (SP)
                    if (rowok[r] && (!diag || key < T)) Ph[(int64_t)(rbase + r) * T + key] = p[r];
            }
            uint2 hi, lo;
            hi.x = pack2(p[0], p[1]);
            hi.y = pack2(p[2], p[3]);
            lo.x = pack2(p[0] - lo2f(hi.x), p[1] - hi2f(hi.x));
            lo.y = pack2(p[2] - lo2f(hi.y), p[3] - hi2f(hi.y));
            const int off = tr_off<1>(kl, 4 * (lane >> 4));
            *(uint2*)(sPh + off) = hi;
            *(uint2*)(sPl + off) = lo;
        }
        wave_sync();  // sP[w] is this wave's own tile
#pragma unroll
        for (int kc = 0; kc < TK / 32; kc++) {
            const bf16x8_t ah = tr_frag<1>(sPh, 32 * kc, 0, lane);
            const bf16x8_t al = tr_frag<1>(sPl, 32 * kc, 0, lane);
#pragma unroll
            for (int j = 0; j < HD / 16; j++) {
                const bf16x8_t bv = tr_frag<VST>(sV, 32 * kc, 16 * j, lane);
                acc[j] = mfma16(al, bv, acc[j]);
                acc[j] = mfma16(ah, bv, acc[j]);
            }
        }
    }
    // zeros above the diagonal (ops.cu:352-396 leaves exact zeros there)
    if (SP && zero_fill) {
        int k0 = (qt + 1) * TK;
        int width = T - k0;
        if (width > 0) {
            for (int i = threadIdx.x; i < TQ * width; i += 256) {
                int r = i / width, c = i % width;
                if (q0 + r < T) Ph[(int64_t)(q0 + r) * T + k0 + c] = 0.f;
            }
        }
    }
    // O (bf16, and F32 when O32 is given) — lane holds column 16j + l%16 of
    // rows rbase + r
    bf16* Oh = O + (int64_t)b * T * qs + hq * HD;
    float* O32h = O32 ? O32 + (int64_t)b * T * qs + hq * HD : nullptr;
#pragma unroll
    for (int j = 0; j < HD / 16; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            int row = rbase + r;
            if (row < T) {
                Oh[(int64_t)row * qs + 16 * j + (lane & 15)] = f2bf(acc[j][r]);
                if (O32h) O32h[(int64_t)row * qs + 16 * j + (lane & 15)] = acc[j][r];
            }
        }
}

// ── forward, transposed scores (the engine's form: P not stored) ───────────
// Per block: 128 queries of one (b, hq), 4 waves of 32; key tiles of 64,
// staged in LDS in the xr_off layout.  Each wave computes
// S^T = K Q^T with 32x32x16 MFMAs (K rows as the A operand, the wave's Q
// rows as the B operand, held in registers): lane l then holds the scores
// of query l%32 for keys 8(r/4) + 4(l/32) + r%4 (r < 16) of each 32-key
// half of the tile, so a query's softmax statistics combine over its own
// registers and one exchange with lane l^32.  With the keys of a 16-wide
// k step taken in that order (r < 8: keys 0..15 of a half, r >= 8: keys
// 16..31), the probabilities in registers are directly the B operand of
// O^T += V^T P^T, whose A operand (V^T, the same key order) comes from the
// V tile through two transposing reads per fragment.  P never passes
// through LDS.  Single pass with an online softmax: O is rescaled by
// exp2(m_old - m_new) when some query's running max grows (skipped when
// none did: a factor of exactly 1); P = exp2(S scale log2(e) - m) enters the
// MFMAs as a BF16 hi/lo pair; the rows' final (max, 1/sum) are kept, and
// the backward recomputes P from them.
constexpr int TQ2 = 128;  // queries per block (4 waves x 32)
// per (b, hq) and 64-query tile, the backward's per-query values as one
// The inverse RoPE of a backward output (ops::rope_bwd applied to the
// written dQ / dK): four consecutive head dims d .. d + 3 (d a multiple of
// 4) of a row at position t, from their BF16 values, with the table of
// sign -1 ([T][hd / 2] (cos, sin)); returns the two packed words.
__device__ __forceinline__ uint2 rope4_packed(const float2* __restrict__ rtab, int t, int hd, int d,
                                              float a0, float a1, float a2, float a3) {
    const float4 cs = *(const float4*)(rtab + (int64_t)t * (hd >> 1) + (d >> 1));
    float o0, o1, o2, o3;
    rope_rot(bf2f(f2bf(a0)), bf2f(f2bf(a1)), cs.x, cs.y, o0, o1);
    rope_rot(bf2f(f2bf(a2)), bf2f(f2bf(a3)), cs.z, cs.w, o2, o3);
    uint2 pk;
    pk.x = pack2(o0, o1);
    pk.y = pack2(o2, o3);
    return pk;
}

// 1 KB block: [0, 64) the row's log2 normaliser lse2 = max + log2(sum) (so
// P = exp2(S scale log2(e) - lse2)), [64, 128) the row dot D
constexpr int QST = 256;

typedef float floatx16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ floatx16 mfma32(bf16x8_t a, bf16x8_t b, floatx16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ floatx16 zero16() {
    floatx16 z;
#pragma unroll
    for (int i = 0; i < 16; i++) z[i] = 0.f;
    return z;
}

typedef __attribute__((address_space(3))) void* lds_vptr_t;

// 8 F32 values as the BF16 pair hi = bf16(v), lo = bf16(v - hi) (round to
// nearest even), as MFMA operands; values converted two at a time (one
// v_cvt_pk_bf16_f32 per pair for hi and one for lo)
__device__ __forceinline__ void split8(const float* v, bf16x8_t& hi, bf16x8_t& lo) {
    u32x4 h, l;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        h[i] = pack2(v[2 * i], v[2 * i + 1]);
        l[i] = pack2(v[2 * i] - lo2f(h[i]), v[2 * i + 1] - hi2f(h[i]));
    }
    hi = __builtin_bit_cast(bf16x8_t, h);
    lo = __builtin_bit_cast(bf16x8_t, l);
}

// Loads of one 64-row x HD tile (rows row0.., row stride rs) from global
// memory straight into LDS in the xr_off (or tr_off) layout, as buffer
// loads: each buffer_load_dwordx4 ... lds fills 1 KB of the tile (lane i
// writes bytes 16i..16i+15, so lane i fetches the 16-byte chunk that the
// layout places there); wave w issues instructions w, w + 4, ...  Rows at or past T read
// as zeros through the buffer's bounds (the resource covers rows 0..T-1);
// the lane offsets are fixed for the kernel and a tile's row offset is one
// scalar.
typedef int i32x4_t __attribute__((ext_vector_type(4)));

// A second tile layout, [row][HD] BF16 with the 16-byte chunks of row r
// XOR-permuted by xr_g(r): over any 16 consecutive rows (HD 128; any 8 of
// one parity for HD 64) the permutation is a bijection, so 16 lanes reading
// the same chunk of 16 rows (the MFMA A/B operand of rows) hit 16 distinct
// bank groups; and any 4 consecutive rows x 4 aligned chunks land on
// distinct banks, which keeps the transposing reads of 4 rows x 32 columns
// per half-wave conflict free as well.
template <int NCH>  // 16-byte chunks per row (HD / 8)
__device__ __forceinline__ int xr_g(int r) {
    if constexpr (NCH == 16) return 4 * (r & 3) + ((r >> 2) & 3);
    else return 4 * ((r >> 1) & 1) + ((r >> 2) & 3);
}
template <int NCH>
__device__ __forceinline__ int xr_off(int r, int c) {
    return r * NCH * 16 + (((c >> 3) ^ xr_g<NCH>(r)) << 4) + (c & 7) * 2;
}

template <int HD, bool XR = false>  // XR: the xr_off layout (else tr_off)
struct AttnDma {
    static constexpr int RB = HD * 2, RPI = 1024 / RB, NI = 64 / RPI, PER = NI / 4;
    int voff[PER];
    __device__ __forceinline__ void init(int64_t rs, int w, int lane) {
#pragma unroll
        for (int h = 0; h < PER; h++) {
            const int r = (w + 4 * h) * RPI + (lane * 16) / RB, ib = (lane * 16) % RB;
            const int col = XR ? 8 * ((ib >> 4) ^ xr_g<HD / 8>(r))
                               : 16 * ((ib >> 5) ^ tr_x<HD / 16>(r)) + 8 * ((ib >> 4) & 1);
            voff[h] = (int)((r * rs + col) * 2);
        }
    }
    // tile rows row0 .. row0 + 63 of the buffer into `tile`.  The loads are
    // issued from inline assembly so that the compiler's wait insertion does
    // not pair later LDS reads of other tiles with them (it cannot tell the
    // buffers' loads apart and would wait for every one); the kernel orders
    // them with explicit vmcnt waits and barriers.
    __device__ __forceinline__ void issue(i32x4_t rsrc, int64_t rs, int row0, char* tile,
                                          int w) const {
        const int so = (int)(row0 * rs * 2);
#pragma unroll
        for (int h = 0; h < PER; h++) {
            const uint32_t la = (uint32_t)(uintptr_t)(tile + (w + 4 * h) * 1024);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                         :
                         : "s"(__builtin_amdgcn_readfirstlane(la)), "v"(voff[h]), "s"(rsrc),
                           "s"(so)
                         : "memory", "m0");
#pragma clang diagnostic pop
        }
    }
};

// Buffer resource over rows 0..T-1 of a [rows, rs] BF16 tensor at base:
// 64-bit base, stride 0, T*rs*2 bytes (reads past them return zeros).
__device__ __forceinline__ i32x4_t rows_rsrc(const bf16* base, int T, int64_t rs) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    i32x4_t r;
    r[0] = (int)(uint32_t)a;
    r[1] = (int)(uint32_t)(a >> 32);
    r[2] = (int)(T * rs * 2);
    r[3] = 0x00020000;
    return r;
}

template <int HD>
__global__ __launch_bounds__(256, 2) void k_attn_fwd_t(const bf16* __restrict__ Q,
                                                    const bf16* __restrict__ K,
                                                    const bf16* __restrict__ V,
                                                    bf16* __restrict__ O, float* __restrict__ O32,
                                                    float2* __restrict__ stats, int T, int Hq,
                                                    int Hkv, float scale) {
    constexpr int NST = HD / 16, NDB = HD / 32;
    // Two K/V buffer pairs (64 KB), each its own array (so the compiler can
    // match each LDS read with the loads that fill that buffer and waits for
    // no other), used alternately by a loop unrolled twice: tile kt + 1 is
    // loaded into the buffers of tile kt - 1 once every wave is done with
    // it.  Two blocks fit a CU (at most 256 registers per lane, from the
    // launch bounds), so each SIMD runs two waves whose softmax VALU work
    // and MFMAs overlap; measured 22% faster than one block per CU with
    // three buffer pairs.
    constexpr int TB = TK * HD * 2;
    __shared__ __attribute__((aligned(1024))) char sK0[TB], sK1[TB];
    __shared__ __attribute__((aligned(1024))) char sV0[TB], sV1[TB];
    const int nqt = (T + TQ2 - 1) / TQ2;
    const int nbh = gridDim.x / nqt;
    const int qt = nqt - 1 - (int)(blockIdx.x / nbh);  // longest rows launch first
    const int bh = (int)(blockIdx.x % nbh);
    const int b = bh / Hq, hq = bh % Hq, hkv = hq / (Hq / Hkv);
    // the wave index as a scalar: conditions on it are uniform branches
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t qs = (int64_t)Hq * HD, ks_ = (int64_t)Hkv * HD;
    const bf16* Qh = Q + (int64_t)b * T * qs + hq * HD;
    const bf16* Kh = K + (int64_t)b * T * ks_ + hkv * HD;
    const bf16* Vh = V + (int64_t)b * T * ks_ + hkv * HD;
    const int q0 = qt * TQ2, qw0 = q0 + 32 * w;
    const int qrow = qw0 + (lane & 31);  // this lane's query
    bf16x8_t qf[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) qf[st] = ld_head8(Qh, qs, qrow, T, 16 * st + 8 * (lane >> 5));
    // per-lane LDS offsets within a tile (the tile-, half- and step-dependent
    // parts are multiples of 16 rows, which the row XOR of xr_off ignores):
    // K rows for S^T, and the two transposing reads of each 32-wide V^T block
    int koff[NST], voff[NDB][2];
#pragma unroll
    for (int st = 0; st < NST; st++) koff[st] = xr_off<HD / 8>(lane & 31, 16 * st + 8 * (lane >> 5));
    {
        const int g = lane >> 4, j = lane & 15;
        const int r = 4 * (g >> 1) + (j >> 2), c = 16 * (g & 1) + 4 * (j & 3);
#pragma unroll
        for (int db = 0; db < NDB; db++) {
            voff[db][0] = xr_off<HD / 8>(r, 32 * db + c);
            voff[db][1] = xr_off<HD / 8>(r + 8, 32 * db + c);
        }
    }
    const float sl2 = scale * kLog2e;
    float m = -INFINITY, l = 0.f;
    floatx16 acc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; db++) acc[db] = zero16();
    // key tiles holding keys <= the block's last query
    const int nkt = min((T + TK - 1) / TK, (min(q0 + TQ2, T) - 1) / TK + 1);
    // tiles past the last one reload it into a buffer that is never read,
    // so every wave issues the same number of loads per step
    AttnDma<HD, true> dma;
    dma.init(ks_, w, lane);
    const i32x4_t rK = rows_rsrc(Kh, T, ks_), rV = rows_rsrc(Vh, T, ks_);
    auto issueK = [&](int kt, char* dK) { dma.issue(rK, ks_, min(kt, nkt - 1) * TK, dK, w); };
    auto issueV = [&](int kt, char* dV) { dma.issue(rV, ks_, min(kt, nkt - 1) * TK, dV, w); };
    auto issue = [&](int kt, char* dK, char* dV) {
        issueK(kt, dK);
        issueV(kt, dV);
    };
    // tile kt; the next tile's V loads go out after this tile's first MFMAs
    auto tile = [&](const char* __restrict__ sK, const char* __restrict__ sV, int kt,
                    char* nV) {
        const int k0 = kt * TK;
        if (k0 > qw0 + 31 || qw0 >= T) {  // every key follows every query of this wave
            issueV(kt + 1, nV);
            return;
        }
        floatx16 s[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            s[h] = zero16();
#pragma unroll
            for (int st = 0; st < NST; st++)
                s[h] = mfma32(*(const bf16x8_t*)(sK + h * 32 * 32 * NST + koff[st]), qf[st], s[h]);
        }
        issueV(kt + 1, nV);
        // scores in base-2 units; on a tile reaching past this wave's first
        // query, keys after the query are masked (which covers keys past T
        // for every row below T; rows past T are never stored).  The mask
        // is a real branch: the empty asm keeps its compares from being
        // speculated into every tile.
        float mx = -INFINITY;
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int r = 0; r < 16; r++) s[h][r] *= sl2;
        if (k0 + TK - 1 > qw0) {
            int kq = qrow - k0 - 4 * (lane >> 5);  // query - key of register 0
            asm volatile("" : "+v"(kq));
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    s[h][r] = 32 * h + 8 * (r >> 2) + (r & 3) <= kq ? s[h][r] : -INFINITY;
        }
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int r = 0; r < 16; r++) mx = fmaxf(mx, s[h][r]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mn = fmaxf(m, mx);
        const float al = m == -INFINITY ? 0.f : exp2_fast(m - mn);
        m = mn;
        // rescaling by exactly 1 changes nothing: skipped unless some query's
        // running max grew
        if (__ballot(al != 1.f) != 0) {
#pragma unroll
            for (int db = 0; db < NDB; db++)
#pragma unroll
                for (int r = 0; r < 16; r++) acc[db][r] *= al;
        }
        float add = 0.f;
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                // k step (h, hf): keys 32h + 16hf .. +15, registers r = 8hf .. 8hf + 7
                float p[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    p[e] = exp2_fast(s[h][8 * hf + e] - m);  // 0 where masked
                    add += p[e];
                }
                bf16x8_t ph, pl;
                split8(p, ph, pl);
                const char* vt = sV + (32 * h + 16 * hf) * 32 * NST;
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_i16x4_p)(vt + voff[db][0]));
                    i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_i16x4_p)(vt + voff[db][1]));
                    const bf16x8_t va = __builtin_bit_cast(
                        bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                    acc[db] = mfma32(va, pl, acc[db]);
                    acc[db] = mfma32(va, ph, acc[db]);
                }
            }
        l = l * al + add;
    };
    TA_WAIT_VMCNT(0);  // the Q fragments are in; only tile loads are counted below
    issue(0, sK0, sV0);
    // one step: wait for this wave's loads of the tile, barrier (after it
    // every wave's loads have landed and every wave is done reading the
    // previous tile's buffers), refill the K buffer with the next tile,
    // compute (the next tile's V loads go out after the first MFMAs, so a
    // wave starts its MFMAs before it has issued every load of the step)
#define ATT_STEP(KT, SK, SV, RK, RV)          \
    if ((KT) < nkt) {                         \
        TA_WAIT_VMCNT(0);                     \
        __builtin_amdgcn_s_barrier();         \
        issueK((KT) + 1, RK);                 \
        tile(SK, SV, (KT), RV);               \
    }
    for (int kt = 0; kt < nkt; kt += 2) {
        ATT_STEP(kt, sK0, sV0, sK1, sV1);
        ATT_STEP(kt + 1, sK1, sV1, sK0, sV0);
    }
#undef ATT_STEP
    TA_WAIT_VMCNT(0);  // the surplus loads have landed before the block ends
    if (qw0 >= T) return;
    const float inv = 1.f / (l + __shfl_xor(l, 32, 64));
    if (qrow < T && lane < 32) stats[(int64_t)bh * T + qrow] = make_float2(m, inv);
    if (qrow >= T) return;
    bf16* orow = O + ((int64_t)b * T + qrow) * qs + hq * HD;
    float* o32row = O32 ? O32 + ((int64_t)b * T + qrow) * qs + hq * HD : nullptr;
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            // d = 32 db + 8 j + 4 (lane / 32) + 0..3
            const int d = 32 * db + 8 * j + 4 * (lane >> 5);
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] = acc[db][4 * j + i] * inv;
            uint2 pk;
            pk.x = pack2(o[0], o[1]);
            pk.y = pack2(o[2], o[3]);
            *(uint2*)(orow + d) = pk;
            if (o32row) *(float4*)(o32row + d) = make_float4(o[0], o[1], o[2], o[3]);
        }
}

// ── backward dQ, transposed scores (the engine's form: P recomputed) ─────
// Per block: 128 queries of one (b, hq), 4 waves of 32; key tiles of 64 in
// two LDS buffer pairs, two blocks per CU, as in k_attn_fwd_t (measured 12%
// faster than one block per CU with three pairs).  Per tile each wave forms
// S^T = K Q^T exactly as the forward did (same operands, same MFMA order,
// so the same bits) and dP^T = V dO^T, both with lane l holding query l%32;
// P = exp2(S scale log2(e) - lse2), lse2 = max + log2(sum) from the forward's
// row statistics, and dS = P (dP - D) (ops.cu:405-435) stay in registers and enter
// dQ^T += K^T dS^T as its B operand (BF16 hi/lo), K^T coming from the K tile
// through transposing reads in the scores' key order.  The row dots
// D = dO . O are formed at the start from the dO fragments and the forward's
// F32 output, and stored with the row statistics for the dK/dV pass.
template <int HD>
__global__ __launch_bounds__(256, 2) void k_attn_bwd_dq_t(const bf16* __restrict__ dO,
                                                       const bf16* __restrict__ Q,
                                                       const bf16* __restrict__ K,
                                                       const bf16* __restrict__ V,
                                                       const float2* __restrict__ stats,
                                                       float* __restrict__ qst,
                                                       const float* __restrict__ O32,
                                                       bf16* __restrict__ dQ, int T, int Hq,
                                                       int Hkv, float scale,
                                                       const float2* __restrict__ rtab) {
    constexpr int NST = HD / 16, NDB = HD / 32;
    constexpr int TB = TK * HD * 2;
    __shared__ __attribute__((aligned(1024))) char sK0[TB], sK1[TB];
    __shared__ __attribute__((aligned(1024))) char sV0[TB], sV1[TB];
    const int nqt = (T + TQ2 - 1) / TQ2;
    const int nbh = gridDim.x / nqt;
    const int qt = nqt - 1 - (int)(blockIdx.x / nbh);  // longest rows launch first
    const int bh = (int)(blockIdx.x % nbh);
    const int b = bh / Hq, hq = bh % Hq, hkv = hq / (Hq / Hkv);
    // the wave index as a scalar: conditions on it are uniform branches
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t qs = (int64_t)Hq * HD, ks_ = (int64_t)Hkv * HD;
    const bf16* Qh = Q + (int64_t)b * T * qs + hq * HD;
    const bf16* dOh = dO + (int64_t)b * T * qs + hq * HD;
    const bf16* Kh = K + (int64_t)b * T * ks_ + hkv * HD;
    const bf16* Vh = V + (int64_t)b * T * ks_ + hkv * HD;
    const int q0 = qt * TQ2, qw0 = q0 + 32 * w;
    const int qrow = qw0 + (lane & 31);
    bf16x8_t qf[NST], of[NST];
#pragma unroll
    for (int st = 0; st < NST; st++) {
        qf[st] = ld_head8(Qh, qs, qrow, T, 16 * st + 8 * (lane >> 5));
        of[st] = ld_head8(dOh, qs, qrow, T, 16 * st + 8 * (lane >> 5));
    }
    // row dot D = dO . O (F32 O of the forward) over this lane's half of the
    // head dims, then the other half from lane l ^ 32; the row's log2
    // normaliser from its statistics (+inf past T: P = 0 there)
    float D = 0.f, lse = INFINITY;
    if (qrow < T) {
        const float* orow = O32 + ((int64_t)b * T + qrow) * qs + hq * HD;
#pragma unroll
        for (int st = 0; st < NST; st++) {
            const float4 o0 = *(const float4*)(orow + 16 * st + 8 * (lane >> 5));
            const float4 o1 = *(const float4*)(orow + 16 * st + 8 * (lane >> 5) + 4);
            const float ov[8] = {o0.x, o0.y, o0.z, o0.w, o1.x, o1.y, o1.z, o1.w};
#pragma unroll
            for (int e = 0; e < 8; e++) D += (float)of[st][e] * ov[e];
        }
        const float2 st = stats[(int64_t)bh * T + qrow];
        lse = st.x - __builtin_amdgcn_logf(st.y);
    }
    D += __shfl_xor(D, 32, 64);
    // the dK/dV pass reads (lse2, D) per 64-query tile; rows past T inside
    // the last tile get (+inf, 0), which make their P and dS zero there
    const int nq64 = (T + TQ - 1) / TQ;
    if (lane < 32 && qrow < nq64 * TQ) {
        float* t = qst + ((int64_t)bh * nq64 + (qrow >> 6)) * QST + (qrow & 63);
        t[0] = lse;
        t[64] = D;
    }
    int koff[NST], voff[NDB][2];
#pragma unroll
    for (int st = 0; st < NST; st++) koff[st] = xr_off<HD / 8>(lane & 31, 16 * st + 8 * (lane >> 5));
    {
        const int g = lane >> 4, j = lane & 15;
        const int r = 4 * (g >> 1) + (j >> 2), c = 16 * (g & 1) + 4 * (j & 3);
#pragma unroll
        for (int db = 0; db < NDB; db++) {
            voff[db][0] = xr_off<HD / 8>(r, 32 * db + c);
            voff[db][1] = xr_off<HD / 8>(r + 8, 32 * db + c);
        }
    }
    const float sl2 = scale * kLog2e;
    floatx16 acc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; db++) acc[db] = zero16();
    const int nkt = min((T + TK - 1) / TK, (min(q0 + TQ2, T) - 1) / TK + 1);
    AttnDma<HD, true> dma;
    dma.init(ks_, w, lane);
    const i32x4_t rK = rows_rsrc(Kh, T, ks_), rV = rows_rsrc(Vh, T, ks_);
    auto issueK = [&](int kt, char* dK) { dma.issue(rK, ks_, min(kt, nkt - 1) * TK, dK, w); };
    auto issueV = [&](int kt, char* dV) { dma.issue(rV, ks_, min(kt, nkt - 1) * TK, dV, w); };
    auto issue = [&](int kt, char* dK, char* dV) {
        issueK(kt, dK);
        issueV(kt, dV);
    };
    // tile kt; the next tile's V loads go out after this tile's first MFMAs
    auto tile = [&](const char* __restrict__ sK, const char* __restrict__ sV, int kt,
                    char* nV) {
        const int k0 = kt * TK;
        if (k0 > qw0 + 31 || qw0 >= T) {  // every key follows every query of this wave
            issueV(kt + 1, nV);
            return;
        }
        floatx16 sT[2], dp[2];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            sT[h] = zero16();
            dp[h] = zero16();
#pragma unroll
            for (int st = 0; st < NST; st++)
                sT[h] = mfma32(*(const bf16x8_t*)(sK + h * 32 * 32 * NST + koff[st]), qf[st], sT[h]);
#pragma unroll
            for (int st = 0; st < NST; st++)
                dp[h] = mfma32(*(const bf16x8_t*)(sV + h * 32 * 32 * NST + koff[st]), of[st], dp[h]);
        }
        issueV(kt + 1, nV);
        // P exactly as the forward's statistics define it (keys after the
        // query masked on a tile reaching past the wave's first query, a
        // real branch as in the forward); dS = P (dP - D)
        float p[2][16];
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int r = 0; r < 16; r++) p[h][r] = exp2_fast(sT[h][r] * sl2 - lse);
        if (k0 + TK - 1 > qw0) {
            int kq = qrow - k0 - 4 * (lane >> 5);  // query - key of register 0
            asm volatile("" : "+v"(kq));
#pragma unroll
            for (int h = 0; h < 2; h++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    p[h][r] = 32 * h + 8 * (r >> 2) + (r & 3) <= kq ? p[h][r] : 0.f;
        }
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int r = 0; r < 16; r++) dp[h][r] = p[h][r] * (dp[h][r] - D);
#pragma unroll
        for (int h = 0; h < 2; h++)
#pragma unroll
            for (int hf = 0; hf < 2; hf++) {
                bf16x8_t dh, dl;
                float d8[8];
#pragma unroll
                for (int e = 0; e < 8; e++) d8[e] = dp[h][8 * hf + e];
                split8(d8, dh, dl);
                const char* kt_ = sK + (32 * h + 16 * hf) * 32 * NST;
#pragma unroll
                for (int db = 0; db < NDB; db++) {
                    i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_i16x4_p)(kt_ + voff[db][0]));
                    i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                        (lds_i16x4_p)(kt_ + voff[db][1]));
                    const bf16x8_t ka = __builtin_bit_cast(
                        bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                    acc[db] = mfma32(ka, dl, acc[db]);
                    acc[db] = mfma32(ka, dh, acc[db]);
                }
            }
    };
    TA_WAIT_VMCNT(0);  // Q, dO, O and the statistics are in; only tile loads are counted below
    issue(0, sK0, sV0);
    // one step as in the forward kernel: K of the next tile at the barrier,
    // its V after this tile's score and dP MFMAs
#define ATT_STEP(KT, SK, SV, RK, RV)          \
    if ((KT) < nkt) {                         \
        TA_WAIT_VMCNT(0);                     \
        __builtin_amdgcn_s_barrier();         \
        issueK((KT) + 1, RK);                 \
        tile(SK, SV, (KT), RV);               \
    }
    for (int kt = 0; kt < nkt; kt += 2) {
        ATT_STEP(kt, sK0, sV0, sK1, sV1);
        ATT_STEP(kt + 1, sK1, sV1, sK0, sV0);
    }
#undef ATT_STEP
    TA_WAIT_VMCNT(0);  // the surplus loads have landed before the block ends
    if (qrow >= T) return;
    bf16* drow = dQ + ((int64_t)b * T + qrow) * qs + hq * HD;
#pragma unroll
    for (int db = 0; db < NDB; db++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int d = 32 * db + 8 * j + 4 * (lane >> 5);
            uint2 pk;
            if (rtab) {
                pk = rope4_packed(rtab, qrow, HD, d, scale * acc[db][4 * j + 0],
                                  scale * acc[db][4 * j + 1], scale * acc[db][4 * j + 2],
                                  scale * acc[db][4 * j + 3]);
            } else {
                pk.x = pack2(scale * acc[db][4 * j + 0], scale * acc[db][4 * j + 1]);
                pk.y = pack2(scale * acc[db][4 * j + 2], scale * acc[db][4 * j + 3]);
            }
            *(uint2*)(drow + d) = pk;
        }
}

// ── backward dK/dV, keys on the lanes (the engine's form: P recomputed) ───
// Per block: 128 keys of one (b, kv head) and a run of the query heads of
// its GQA group [h0, h1).  The block walks (head, 64-query tile) steps; each
// step's Q and dO tiles (xr_off layout) and the tile's 1 KB of per-query
// values come straight into LDS by buffer-load DMA, three stages deep, as
// the K/V tiles of k_attn_fwd_t (the Q tile and the per-query block of step
// j + 2 go out at step j's barrier, its dO tile after the V role's first
// score MFMAs of step j).  S = Q K^T and dP = dO V^T run as 32
// queries x 32 keys MFMA tiles with the keys' rows as B operands held in
// accumulation registers, so lane l holds key l%32 and queries
// 8(r/4) + 4(l/32) + r%4 of each 32-query half.  P = exp2(S scale log2(e) -
// lse2), exactly as the dQ pass forms it, and dS = P (dP - D)
// (ops.cu:405-435), with the queries of a 16-wide k step taken in that
// order, are the B operands (BF16 hi/lo) of dV^T += dO^T P and
// dK^T += Q^T dS, whose A operands come from the same tiles through
// transposing reads.
// The work of each 32-key group is split between two waves of different
// roles, so that two waves share each SIMD and one's VALU work overlaps the
// other's MFMAs.  Block: 8 waves; waves w and w + 4 own keys
// kb*128 + 32w .. +31.
//   V role (w < 4): S, P (masked on the diagonal), P to LDS; then dV^T.  It
//     also issues the tile DMA.
//   K role (w >= 4): dP; then, with P from LDS, dS and dK^T.
// Per 32-query half each role runs 8 MFMAs before a block barrier (the V
// role's exponentials overlap the K role's dP) and 16 after it; each
// accumulator takes, per half, the lo then the hi product of the first
// 16-query k step, then those of the second.  The barriers are reached by
// every wave on every half, whether or not its keys take part in it.  P
// travels in a buffer per half parity ([pair][4 row groups][64 lanes]
// float4): a half's K-role reads end before the next half's barrier, which
// the V role passes before it writes the same parity again.
// The run's heads accumulate in registers; a run covering the whole group
// writes dK (times scale) and dV in BF16, otherwise each run writes F32
// partials that k_attn_dkv_sum adds in run order — the group sum of
// ops.cu:539-555 with no atomics, so dK/dV are deterministic.
template <int HD>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_attn_bwd_dkv_r(
    const bf16* __restrict__ dO, const bf16* __restrict__ Q, const bf16* __restrict__ K,
    const bf16* __restrict__ V, const float* __restrict__ qst, float* __restrict__ part,
    bf16* __restrict__ dK, bf16* __restrict__ dV, int T, int Hq, int Hkv, int nsplit,
    float scale, const float2* __restrict__ rtab) {
    constexpr int NST = HD / 16, NDB = HD / 32;
    constexpr int TB = TQ * HD * 2;
    // DMA instructions per V-role wave per step: Q and dO tiles, a quarter of
    // the per-query block
    constexpr int LPT = 2 * (TB / 1024) / 4 + 1;
    // three stages of Q tile, dO tile and per-query block, addressed from a
    // stage index that is not a compile-time constant, so that the compiler
    // keeps one base per tile instead of a hoisted address per stage and
    // fragment
    __shared__ __attribute__((aligned(1024))) char sQ[3][TB];
    __shared__ __attribute__((aligned(1024))) char sO[3][TB];
    __shared__ __attribute__((aligned(1024))) float sS[3][QST];
    __shared__ __attribute__((aligned(16))) float4 sP[2][4][4][64];
    const int nkb = (T + 127) / 128, nqt = (T + TQ - 1) / TQ, grp = Hq / Hkv;
    const int per = gridDim.x / nkb;               // B * Hkv * nsplit blocks per key block
    const int kb = (int)(blockIdx.x / per);       // low kb = most query tiles: launch first
    const int rem = (int)(blockIdx.x % per);
    const int sp = rem % nsplit, bkv = rem / nsplit;
    const int B = per / (Hkv * nsplit), b = bkv / Hkv, hkv = bkv % Hkv;
    const int h0 = sp * grp / nsplit, h1 = (sp + 1) * grp / nsplit;
    // wave index and role as scalars: conditions on them are uniform branches
    const int lane = threadIdx.x & 63, w8 = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int w = w8 & 3;
    const bool vrole = w8 < 4;
    const int64_t qs = (int64_t)Hq * HD, ks_ = (int64_t)Hkv * HD;
    const int kw0 = kb * 128 + 32 * w, key = kw0 + (lane & 31);
    // K rows (V role, the B operand of S) or V rows (K role, of dP)
    bf16x8_t kv[NST];
    {
        const bf16* src = (vrole ? K : V) + (int64_t)b * T * ks_ + hkv * HD;
#pragma unroll
        for (int st = 0; st < NST; st++) kv[st] = ld_head8(src, ks_, key, T, 16 * st + 8 * (lane >> 5));
#pragma unroll
        for (int st = 0; st < NST; st++) asm volatile("" : "+a"(kv[st]));
    }
    int qoff[NST], toff[NDB][2];
#pragma unroll
    for (int st = 0; st < NST; st++) qoff[st] = xr_off<HD / 8>(lane & 31, 16 * st + 8 * (lane >> 5));
    {
        const int g = lane >> 4, j = lane & 15;
        const int r = 4 * (g >> 1) + (j >> 2), c = 16 * (g & 1) + 4 * (j & 3);
#pragma unroll
        for (int db = 0; db < NDB; db++) {
            toff[db][0] = xr_off<HD / 8>(r, 32 * db + c);
            toff[db][1] = xr_off<HD / 8>(r + 8, 32 * db + c);
        }
    }
    // dV^T (V role) or unscaled dK^T (K role): rows are head dims
    floatx16 acc[NDB];
#pragma unroll
    for (int db = 0; db < NDB; db++) acc[db] = zero16();
    const int qt0 = (kb * 128) / TQ, nqh = nqt - qt0, nst = (h1 - h0) * nqh;
    AttnDma<HD, true> dma;
    dma.init(qs, w, lane);
    const bf16* Qb = Q + (int64_t)b * T * qs;
    const bf16* Ob = dO + (int64_t)b * T * qs;
    const float* Sb = qst + (int64_t)b * Hq * nqt * QST;
    const int soff = 4 * (64 * w + 4 * lane);
    auto step_head = [&](int j, int& qt) {
        const int jj = min(j, nst - 1);
        qt = qt0 + jj % nqh;
        return hkv * grp + h0 + jj / nqh;
    };
    // the loads of step j (V-role waves only; past the last step the last is
    // loaded again into a buffer that is never read)
    auto issueO = [&](int j, char* tO) {
        if (!vrole) return;
        int qt;
        const int hq = step_head(j, qt);
        dma.issue(rows_rsrc(Ob + hq * HD, T, qs), qs, qt * TQ, tO, w);
    };
    auto issueQ = [&](int j, char* tQ, float* tS) {
        if (!vrole) return;
        int qt;
        const int hq = step_head(j, qt);
        dma.issue(rows_rsrc(Qb + hq * HD, T, qs), qs, qt * TQ, tQ, w);
        const uint64_t a = (uint64_t)(uintptr_t)(Sb + ((int64_t)hq * nqt + qt) * QST);
        i32x4_t rs;
        rs[0] = (int)(uint32_t)a;
        rs[1] = (int)(uint32_t)(a >> 32);
        rs[2] = QST * 4;
        rs[3] = 0x00020000;
        const uint32_t la = (uint32_t)(uintptr_t)(tS + 64 * w);
        const int zero = 0;
        if (lane < 16) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
            asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                         :
                         : "s"(__builtin_amdgcn_readfirstlane(la)), "v"(soff), "s"(rs),
                           "s"(zero)
                         : "memory", "m0");
#pragma clang diagnostic pop
        }
    };
    auto issue = [&](int j, char* tQ, char* tO, float* tS) {
        issueQ(j, tQ, tS);
        issueO(j, tO);
    };
    const float sl2 = scale * kLog2e;
    // first phase of half h: S (V role) or dP (K role) over the tile's
    // 32 query rows, the A operands read from the Q or dO tile
    auto mm1 = [&](const char* __restrict__ tA, int h) {
        bf16x8_t fa[NST];
#pragma unroll
        for (int st = 0; st < NST; st++)
            fa[st] = *(const bf16x8_t*)(tA + h * 32 * 32 * NST + qoff[st]);
        __builtin_amdgcn_sched_barrier(0);
        floatx16 r = zero16();
#pragma unroll
        for (int st = 0; st < NST; st++) r = mfma32(fa[st], kv[st], r);
        return r;
    };
    // second phase: acc += A^T X over the half's two 16-query k steps, X the
    // BF16 hi/lo split of P (V role) or dS (K role), A^T read transposed
    // from the dO or Q tile; per accumulator the lo product precedes the hi
    // one in each k step
    auto mm2 = [&](const char* __restrict__ tA, int h, const bf16x8_t (&xb)[2][2]) {
        bf16x8_t fa[2][NDB];
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
            const char* at = tA + (32 * h + 16 * hf) * 32 * NST;
#pragma unroll
            for (int db = 0; db < NDB; db++) {
                i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_p)(at + toff[db][0]));
                i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_p)(at + toff[db][1]));
                fa[hf][db] = __builtin_bit_cast(
                    bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int hf = 0; hf < 2; hf++) {
#pragma unroll
            for (int db = 0; db < NDB; db++) acc[db] = mfma32(fa[hf][db], xb[hf][1], acc[db]);
#pragma unroll
            for (int db = 0; db < NDB; db++) acc[db] = mfma32(fa[hf][db], xb[hf][0], acc[db]);
        }
    };
    // the role as a compile-time constant (RT: std::true_type for the V role),
    // so that each role's loop is compiled and register-allocated on its own
    auto step = [&](auto RT, const char* __restrict__ tQ, const char* __restrict__ tO,
                    const float* __restrict__ tS, int j, int jn, char* nO) {
        constexpr bool VR = decltype(RT)::value;
        const int q0 = (qt0 + j % nqh) * TQ;
        // every key follows every query of the tile: no work, barriers only
        const bool any = kw0 <= q0 + TQ - 1 && kw0 < T;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int qh0 = q0 + 32 * h;
            const bool act = any && kw0 <= qh0;
            float4* pb = &sP[h][w][0][0];
            float p[16];
            floatx16 dP;
            if constexpr (VR) {
                if (h == 0 && !act) issueO(jn, nO);
            }
            if (act) {
                if constexpr (VR) {
                    const floatx16 S = mm1(tQ, h);
                    if (h == 0) issueO(jn, nO);
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const float4 lx = *(const float4*)(tS + 32 * h + 8 * c + 4 * (lane >> 5));
                        const float l4[4] = {lx.x, lx.y, lx.z, lx.w};
#pragma unroll
                        for (int e = 0; e < 4; e++) p[4 * c + e] = exp2_fast(S[4 * c + e] * sl2 - l4[e]);
                    }
                    if (kw0 == qh0) {
                        int kq = (lane & 31) - 4 * (lane >> 5);
                        asm volatile("" : "+v"(kq));
#pragma unroll
                        for (int r = 0; r < 16; r++) p[r] = kq <= 8 * (r >> 2) + (r & 3) ? p[r] : 0.f;
                    }
#pragma unroll
                    for (int c = 0; c < 4; c++)
                        pb[64 * c + lane] = make_float4(p[4 * c], p[4 * c + 1], p[4 * c + 2], p[4 * c + 3]);
                } else {
                    dP = mm1(tO, h);
                }
            }
            // the V role's P stores are complete before any wave passes
            // (the asm's memory clobber also keeps the compiler from moving
            // LDS accesses across it)
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (act) {
                bf16x8_t xb[2][2];
                if constexpr (VR) {
#pragma unroll
                    for (int hf = 0; hf < 2; hf++) split8(p + 8 * hf, xb[hf][0], xb[hf][1]);
                    mm2(tO, h, xb);
                } else {
                    float d[16];
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const float4 pv = pb[64 * c + lane];
                        const float4 dd = *(const float4*)(tS + 64 + 32 * h + 8 * c + 4 * (lane >> 5));
                        d[4 * c] = pv.x * (dP[4 * c] - dd.x);
                        d[4 * c + 1] = pv.y * (dP[4 * c + 1] - dd.y);
                        d[4 * c + 2] = pv.z * (dP[4 * c + 2] - dd.z);
                        d[4 * c + 3] = pv.w * (dP[4 * c + 3] - dd.w);
                    }
#pragma unroll
                    for (int hf = 0; hf < 2; hf++) split8(d + 8 * hf, xb[hf][0], xb[hf][1]);
                    mm2(tQ, h, xb);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    TA_WAIT_VMCNT(0);  // K or V rows are in; only tile loads are counted below
    issue(0, sQ[0], sO[0], sS[0]);
    issue(1, sQ[1], sO[1], sS[1]);
    auto loop = [&](auto RT) {
        constexpr bool VR = decltype(RT)::value;
        int cur = 0, nxt = 2;  // stage of step j, stage that step j + 2 loads into
#pragma nounroll
        for (int j = 0; j < nst; j++) {
            if constexpr (VR) TA_WAIT_VMCNT(LPT);
            __builtin_amdgcn_s_barrier();
            if constexpr (VR) issueQ(j + 2, sQ[nxt], sS[nxt]);
            step(RT, sQ[cur], sO[cur], sS[cur], j, j + 2, sO[nxt]);
            cur = cur == 2 ? 0 : cur + 1;
            nxt = nxt == 2 ? 0 : nxt + 1;
        }
    };
    if (vrole)
        loop(std::true_type{});
    else
        loop(std::false_type{});
    TA_WAIT_VMCNT(0);  // the surplus loads have landed before the block ends
    if (key >= T) return;
    // accumulator rows are head dims 32 db + 8 j + 4 (lane / 32) + 0..3
    const float os = vrole ? 1.f : scale;
    if (nsplit == 1) {
        bf16* row = (vrole ? dV : dK) + ((int64_t)b * T + key) * ks_ + hkv * HD;
#pragma unroll
        for (int db = 0; db < NDB; db++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int d = 32 * db + 8 * j + 4 * (lane >> 5);
                uint2 pk;
                if (rtab && !vrole) {
                    pk = rope4_packed(rtab, key, HD, d, os * acc[db][4 * j], os * acc[db][4 * j + 1],
                                      os * acc[db][4 * j + 2], os * acc[db][4 * j + 3]);
                } else {
                    pk.x = pack2(os * acc[db][4 * j], os * acc[db][4 * j + 1]);
                    pk.y = pack2(os * acc[db][4 * j + 2], os * acc[db][4 * j + 3]);
                }
                *(uint2*)(row + d) = pk;
            }
    } else {
        // partials [nsplit][2][B*T][Hkv*HD]: dK (unscaled) then dV of run sp
        const int64_t n = (int64_t)B * T * ks_;
        float* row = part + (2 * sp + (vrole ? 1 : 0)) * n + ((int64_t)b * T + key) * ks_ + hkv * HD;
#pragma unroll
        for (int db = 0; db < NDB; db++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int d = 32 * db + 8 * j + 4 * (lane >> 5);
                *(float4*)(row + d) = make_float4(acc[db][4 * j], acc[db][4 * j + 1],
                                                  acc[db][4 * j + 2], acc[db][4 * j + 3]);
            }
    }
}

// dK = bf16(scale * sum_s partK[s]), dV = bf16(sum_s partV[s]), runs added
// in order; n4 groups of 4 elements.
__global__ __launch_bounds__(256) void k_attn_dkv_sum(const float4* __restrict__ part,
                                                      uint2* __restrict__ dK,
                                                      uint2* __restrict__ dV, int64_t n4,
                                                      int nsplit, float scale,
                                                      const float2* __restrict__ rtab, int T,
                                                      int kvw, int hd) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n4;
         i += (int64_t)gridDim.x * blockDim.x) {
        float4 k = part[i], v = part[n4 + i];
        for (int sp = 1; sp < nsplit; sp++) {
            const float4 a = part[2 * sp * n4 + i], c = part[(2 * sp + 1) * n4 + i];
            k.x += a.x;
            k.y += a.y;
            k.z += a.z;
            k.w += a.w;
            v.x += c.x;
            v.y += c.y;
            v.z += c.z;
            v.w += c.w;
        }
        uint2 pk;
        if (rtab) {
            // element 4i: row 4i / kvw (position row % T), head dim (4i % kvw) % hd
            // (32-bit: the host keeps 4 n4 below 2^31)
            const uint32_t e = 4u * (uint32_t)i, row = e / (uint32_t)kvw;
            pk = rope4_packed(rtab, (int)(row % (uint32_t)T), hd,
                              (int)((e - row * (uint32_t)kvw) % (uint32_t)hd), scale * k.x,
                              scale * k.y, scale * k.z, scale * k.w);
        } else {
            pk.x = pack2(scale * k.x, scale * k.y);
            pk.y = pack2(scale * k.z, scale * k.w);
        }
        dK[i] = pk;
        pk.x = pack2(v.x, v.y);
        pk.y = pack2(v.z, v.w);
        dV[i] = pk;
    }
}

// ── backward: the row dots D = sum_k P * dP ──────────────────────────────
// From the forward's F32 output: D[bh, t] = dO[t, h, :] . O[t, h, :], since
// sum_k P dP = sum_k P (dO V_k) = dO (sum_k P V_k).  HD/8 lanes per row.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_rowdot_o(const bf16* __restrict__ dO,
                                                       const float* __restrict__ O32,
                                                       float* __restrict__ D, int B, int T,
                                                       int Hq) {
    constexpr int LPR = HD / 8;  // lanes per (token, head)
    int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    int64_t pr = gid / LPR;  // (b, t, h) in dO's row-major order
    int sub = (int)(gid % LPR);
    int64_t npr = (int64_t)B * T * Hq;
    float s = 0.f;
    if (pr < npr) {
        const bf16* o = dO + pr * HD + sub * 8;
        const float* f = O32 + pr * HD + sub * 8;
        bf16x8v a = *(const bf16x8v*)o;
        float4 f0 = *(const float4*)f, f1 = *(const float4*)(f + 4);
        float x[8];
        unpack8(a, x);
        s = x[0] * f0.x + x[1] * f0.y + x[2] * f0.z + x[3] * f0.w + x[4] * f1.x + x[5] * f1.y +
            x[6] * f1.z + x[7] * f1.w;
    }
#pragma unroll
    for (int o = 1; o < LPR; o <<= 1) s += __shfl_xor(s, o, 64);
    if (sub == 0 && pr < npr) {
        int h = (int)(pr % Hq);
        int64_t bt = pr / Hq;
        int t = (int)(bt % T), b = (int)(bt / T);
        D[((int64_t)b * Hq + h) * T + t] = s;
    }
}

// Without the F32 output (the C-ABI's sdpa_bwd): D = sum_k P * dP with
// dP = dO V^T recomputed on MFMA, per (b, hq, query tile).
template <int HD>
__global__ __launch_bounds__(256) void k_attn_rowdot_p(const bf16* __restrict__ dO,
                                                       const bf16* __restrict__ V,
                                                       const float* __restrict__ P,
                                                       float* __restrict__ Dout, int T, int Hq,
                                                       int Hkv) {
    __shared__ __attribute__((aligned(16))) bf16 sV[TK * (HD + 8)];
    int nqt = (T + TQ - 1) / TQ;
    int nbh = gridDim.x / nqt;
    int qt = nqt - 1 - (int)(blockIdx.x / nbh);
    int bh = (int)(blockIdx.x % nbh);
    int b = bh / Hq, hq = bh % Hq, hkv = hq / (Hq / Hkv);
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int64_t qs = (int64_t)Hq * HD, ks_ = (int64_t)Hkv * HD;
    const bf16* dOh = dO + (int64_t)b * T * qs + hq * HD;
    const bf16* Vh = V + (int64_t)b * T * ks_ + hkv * HD;
    const float* Ph = P + (int64_t)bh * T * T;
    int q0 = qt * TQ;
    int rowA = q0 + 16 * w + (lane & 15);
    bf16x8_t of[HD / 32];
#pragma unroll
    for (int ks = 0; ks < HD / 32; ks++)
        of[ks] = ld_head8(dOh, qs, rowA, T, 32 * ks + 8 * (lane >> 4));
    int rbase = q0 + 16 * w + 4 * (lane >> 4);
    float dsum[4] = {0.f, 0.f, 0.f, 0.f};
    Rows64<HD> lv;
    lv.load(Vh, ks_, 0, T);
    for (int kt = 0; kt <= qt; kt++) {
        __syncthreads();
        lv.store(sV);
        __syncthreads();
        if (kt < qt) lv.load(Vh, ks_, (kt + 1) * TK, T);
        floatx4 dP[4];
        wave_qk<HD>(dP, of, sV, lane);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            int key = kt * TK + 16 * t + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int row = rbase + r;
                if (key <= row && key < T && row < T)
                    dsum[r] += Ph[(int64_t)row * T + key] * dP[t][r];
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float d = red16_sum(dsum[r]);
        int row = rbase + r;
        if ((lane & 15) == 0 && row < T) Dout[(int64_t)bh * T + row] = d;
    }
}

// P values a lane needs for one key tile in the C layout of a 16 x 64 wave
// tile: p[t][r] = P[row0 + r][key0 + 16t + l%16] for keys <= row (0 above).
__device__ __forceinline__ void load_p_rows(float (&p)[4][4], const float* __restrict__ Ph, int T,
                                            int row0, int key0, int lane) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
        int key = key0 + 16 * t + (lane & 15);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            int row = row0 + r;
            p[t][r] = (key <= row && key < T && row < T) ? Ph[(int64_t)row * T + key] : 0.f;
        }
    }
}

// ── backward: dQ ──────────────────────────────────────────────────────────
// Per (b, hq, query tile), one pass over the key tiles at or below the
// diagonal: dP = dO V^T, dS = P (dP - D) (ops.cu:405-435), dQ = scale dS K.
// The next tile's V, K and P are loaded while the current one computes.
// K is staged once, in its natural layout, and read as the dS·K operand
// through the transposing LDS read; dS (hi/lo) goes to a per-wave
// [key][row] tile like P in the forward.
template <int HD>
__global__ __launch_bounds__(256) void k_attn_bwd_dq(const bf16* __restrict__ dO,
                                                     const bf16* __restrict__ K,
                                                     const bf16* __restrict__ V,
                                                     const float* __restrict__ P,
                                                     const float* __restrict__ Dq,
                                                     bf16* __restrict__ dQ, int T, int Hq, int Hkv,
                                                     float scale) {
    constexpr int VST = HD / 16;
    __shared__ __attribute__((aligned(16))) bf16 sV[TK * (HD + 8)];
    __shared__ __attribute__((aligned(16))) char sK[TK * HD * 2];
    __shared__ __attribute__((aligned(16))) char sS[4][2][TK * 16 * 2];
    int nqt = (T + TQ - 1) / TQ;
    int nbh = gridDim.x / nqt;
    int qt = nqt - 1 - (int)(blockIdx.x / nbh);  // longest rows launch first
    int bh = (int)(blockIdx.x % nbh);
    int b = bh / Hq, hq = bh % Hq, hkv = hq / (Hq / Hkv);
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int64_t qs = (int64_t)Hq * HD, ks_ = (int64_t)Hkv * HD;
    const bf16* dOh = dO + (int64_t)b * T * qs + hq * HD;
    const bf16* Kh = K + (int64_t)b * T * ks_ + hkv * HD;
    const bf16* Vh = V + (int64_t)b * T * ks_ + hkv * HD;
    const float* Ph = P + (int64_t)bh * T * T;
    int q0 = qt * TQ;
    int rowA = q0 + 16 * w + (lane & 15);
    bf16x8_t of[HD / 32];
#pragma unroll
    for (int ks = 0; ks < HD / 32; ks++)
        of[ks] = ld_head8(dOh, qs, rowA, T, 32 * ks + 8 * (lane >> 4));
    int rbase = q0 + 16 * w + 4 * (lane >> 4);
    float D[4];
#pragma unroll
    for (int r = 0; r < 4; r++) D[r] = (rbase + r < T) ? Dq[(int64_t)bh * T + rbase + r] : 0.f;

    floatx4 acc[HD / 16];
#pragma unroll
    for (int j = 0; j < HD / 16; j++) acc[j] = zero4();
    Rows64<HD> lv, lk;
    float pn[4][4];
    lv.load(Vh, ks_, 0, T);
    lk.load(Kh, ks_, 0, T);
    load_p_rows(pn, Ph, T, rbase, 0, lane);
    char* sSh = sS[w][0];
    char* sSl = sS[w][1];
    for (int kt = 0; kt <= qt; kt++) {
        __syncthreads();
        lv.store(sV);
#pragma unroll
        for (int i = 0; i < Rows64<HD>::NR; i++) {
            int q = threadIdx.x + 256 * i;
            *(u32x4*)(sK + tr_off<VST>(q / (HD / 8), (q % (HD / 8)) * 8)) = lk.v[i];
        }
        float pc[4][4];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) pc[t][r] = pn[t][r];
        __syncthreads();
        if (kt < qt) {
            lv.load(Vh, ks_, (kt + 1) * TK, T);
            lk.load(Kh, ks_, (kt + 1) * TK, T);
            load_p_rows(pn, Ph, T, rbase, (kt + 1) * TK, lane);
        }
        floatx4 dP[4];
        wave_qk<HD>(dP, of, sV, lane);
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int kl = 16 * t + (lane & 15);
            float d[4];
#pragma unroll
            for (int r = 0; r < 4; r++) d[r] = pc[t][r] * (dP[t][r] - D[r]);
            uint2 hi, lo;
            hi.x = pack2(d[0], d[1]);
            hi.y = pack2(d[2], d[3]);
            lo.x = pack2(d[0] - lo2f(hi.x), d[1] - hi2f(hi.x));
            lo.y = pack2(d[2] - lo2f(hi.y), d[3] - hi2f(hi.y));
            const int off = tr_off<1>(kl, 4 * (lane >> 4));
            *(uint2*)(sSh + off) = hi;
            *(uint2*)(sSl + off) = lo;
        }
        wave_sync();
#pragma unroll
        for (int kc = 0; kc < TK / 32; kc++) {
            const bf16x8_t ah = tr_frag<1>(sSh, 32 * kc, 0, lane);
            const bf16x8_t al = tr_frag<1>(sSl, 32 * kc, 0, lane);
#pragma unroll
            for (int j = 0; j < HD / 16; j++) {
                const bf16x8_t bk = tr_frag<VST>(sK, 32 * kc, 16 * j, lane);
                acc[j] = mfma16(al, bk, acc[j]);
                acc[j] = mfma16(ah, bk, acc[j]);
            }
        }
    }
    bf16* dQh = dQ + (int64_t)b * T * qs + hq * HD;
#pragma unroll
    for (int j = 0; j < HD / 16; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            int row = rbase + r;
            if (row < T) dQh[(int64_t)row * qs + 16 * j + (lane & 15)] = f2bf(scale * acc[j][r]);
        }
}

// P^T values for the dK/dV kernel: p[t][r] = P[q0 + 16t + l%16][kbase + r]
// for keys <= query (0 above the diagonal).
__device__ __forceinline__ void load_p_cols(float (&p)[4][4], const float* __restrict__ Ph, int T,
                                            int q0, int kbase, int lane) {
#pragma unroll
    for (int t = 0; t < 4; t++) {
        int q = q0 + 16 * t + (lane & 15);
        const float* prow = Ph + (int64_t)q * T;
        if ((T & 3) == 0 && q < T && kbase + 3 < T && kbase + 3 <= q) {  // 16-byte aligned
            float4 v4 = *(const float4*)(prow + kbase);
            p[t][0] = v4.x;
            p[t][1] = v4.y;
            p[t][2] = v4.z;
            p[t][3] = v4.w;
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int key = kbase + r;
                p[t][r] = (q < T && key < T && key <= q) ? prow[key] : 0.f;
            }
        }
    }
}

// ── backward: dK, dV contributions of one query head, one key tile ─────────
// Wave w owns keys 16w..16w+15 of the tile; for each query tile qt >= kt:
// dP^T = V dO^T (keys x queries), dS^T = P^T (dP^T - D), dV_h += P^T dO,
// dK_h += dS^T Q.  The head's F32 contributions go to part[bh] ([T][hd] for
// dK then dV); k_attn_dkv_reduce sums the GQA group in head order — the
// group sum of ops.cu:539-555 without atomics, so dK/dV are deterministic.
// The next query tile's dO, Q, D and P are loaded while this one computes.
// dO is staged twice: padded rows for dP^T (16-byte fragment reads) and in
// the transposing-read layout for the P^T·dO operand, like Q for dS^T·Q;
// P^T and dS^T (hi/lo) go to a per-wave [query][key] tile.
template <int HD>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_attn_bwd_dkv(
    const bf16* __restrict__ dO, const bf16* __restrict__ Q, const bf16* __restrict__ V,
    const float* __restrict__ P, const float* __restrict__ Dq, float* __restrict__ part, int T,
    int Hq, int Hkv) {
    constexpr int VST = HD / 16;
    __shared__ __attribute__((aligned(16))) bf16 sO[TQ * (HD + 8)];  // dO [q][hd], padded
    __shared__ __attribute__((aligned(16))) char sOn[TQ * HD * 2];   // dO, tr_off layout
    __shared__ __attribute__((aligned(16))) char sQn[TQ * HD * 2];   // Q, tr_off layout
    __shared__ __attribute__((aligned(16))) char sA[4][2][TQ * 16 * 2];  // per wave [q][key] hi,lo
    __shared__ float sD[TQ];
    int nkt = (T + TK - 1) / TK;
    int nbh = gridDim.x / nkt;
    int kt = (int)(blockIdx.x / nbh);  // low kt = most query tiles: they launch first
    int bh = (int)(blockIdx.x % nbh);
    int b = bh / Hq, hq = bh % Hq, hkv = hq / (Hq / Hkv);
    int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int64_t qs = (int64_t)Hq * HD, ks_ = (int64_t)Hkv * HD;
    const bf16* Vh = V + (int64_t)b * T * ks_ + hkv * HD;
    const bf16* dOh = dO + (int64_t)b * T * qs + hq * HD;
    const bf16* Qh = Q + (int64_t)b * T * qs + hq * HD;
    const float* Ph = P + (int64_t)bh * T * T;
    const float* Dh = Dq + (int64_t)bh * T;
    int k0 = kt * TK;
    int keyA = k0 + 16 * w + (lane & 15);  // A-operand row (key) of this lane
    bf16x8_t vf[HD / 32];
#pragma unroll
    for (int s = 0; s < HD / 32; s++) vf[s] = ld_head8(Vh, ks_, keyA, T, 32 * s + 8 * (lane >> 4));
    int kbase = k0 + 16 * w + 4 * (lane >> 4);  // C-layout key rows kbase + r

    floatx4 accK[HD / 16], accV[HD / 16];
#pragma unroll
    for (int j = 0; j < HD / 16; j++) {
        accK[j] = zero4();
        accV[j] = zero4();
    }
    int nqt = (T + TQ - 1) / TQ;
    Rows64<HD> ldo, lq;
    float pn[4][4];
    float dn = 0.f;
    ldo.load(dOh, qs, kt * TQ, T);
    lq.load(Qh, qs, kt * TQ, T);
    load_p_cols(pn, Ph, T, kt * TQ, kbase, lane);
    if (threadIdx.x < TQ) dn = (kt * TQ + threadIdx.x < T) ? Dh[kt * TQ + threadIdx.x] : 0.f;
    char* sAh = sA[w][0];
    char* sAl = sA[w][1];
    for (int qt = kt; qt < nqt; qt++) {
        __syncthreads();
        ldo.store(sO);
#pragma unroll
        for (int i = 0; i < Rows64<HD>::NR; i++) {
            int q = threadIdx.x + 256 * i;
            const int off = tr_off<VST>(q / (HD / 8), (q % (HD / 8)) * 8);
            *(u32x4*)(sOn + off) = ldo.v[i];
            *(u32x4*)(sQn + off) = lq.v[i];
        }
        if (threadIdx.x < TQ) sD[threadIdx.x] = dn;
        float pv[4][4];
#pragma unroll
        for (int t = 0; t < 4; t++)
#pragma unroll
            for (int r = 0; r < 4; r++) pv[t][r] = pn[t][r];
        __syncthreads();
        if (qt + 1 < nqt) {
            int qn = (qt + 1) * TQ;
            ldo.load(dOh, qs, qn, T);
            lq.load(Qh, qs, qn, T);
            load_p_cols(pn, Ph, T, qn, kbase, lane);
            if (threadIdx.x < TQ) dn = (qn + threadIdx.x < T) ? Dh[qn + threadIdx.x] : 0.f;
        }
        floatx4 dPt[4];
        wave_qk<HD>(dPt, vf, sO, lane);  // rows = keys, cols = queries
        // dV += P^T dO: lane holds keys kbase + r (4 consecutive) of query 16t + l%16
#pragma unroll
        for (int t = 0; t < 4; t++) {
            uint2 hi, lo;
            hi.x = pack2(pv[t][0], pv[t][1]);
            hi.y = pack2(pv[t][2], pv[t][3]);
            lo.x = pack2(pv[t][0] - lo2f(hi.x), pv[t][1] - hi2f(hi.x));
            lo.y = pack2(pv[t][2] - lo2f(hi.y), pv[t][3] - hi2f(hi.y));
            const int off = tr_off<1>(16 * t + (lane & 15), 4 * (lane >> 4));
            *(uint2*)(sAh + off) = hi;
            *(uint2*)(sAl + off) = lo;
        }
        wave_sync();
#pragma unroll
        for (int kc = 0; kc < TQ / 32; kc++) {
            const bf16x8_t ah = tr_frag<1>(sAh, 32 * kc, 0, lane);
            const bf16x8_t al = tr_frag<1>(sAl, 32 * kc, 0, lane);
#pragma unroll
            for (int j = 0; j < HD / 16; j++) {
                const bf16x8_t bo = tr_frag<VST>(sOn, 32 * kc, 16 * j, lane);
                accV[j] = mfma16(al, bo, accV[j]);
                accV[j] = mfma16(ah, bo, accV[j]);
            }
        }
        wave_sync();
        // dK += dS^T Q
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const int ql = 16 * t + (lane & 15);
            const float dq = sD[ql];
            float d[4];
#pragma unroll
            for (int r = 0; r < 4; r++) d[r] = pv[t][r] * (dPt[t][r] - dq);
            uint2 hi, lo;
            hi.x = pack2(d[0], d[1]);
            hi.y = pack2(d[2], d[3]);
            lo.x = pack2(d[0] - lo2f(hi.x), d[1] - hi2f(hi.x));
            lo.y = pack2(d[2] - lo2f(hi.y), d[3] - hi2f(hi.y));
            const int off = tr_off<1>(ql, 4 * (lane >> 4));
            *(uint2*)(sAh + off) = hi;
            *(uint2*)(sAl + off) = lo;
        }
        wave_sync();
#pragma unroll
        for (int kc = 0; kc < TQ / 32; kc++) {
            const bf16x8_t ah = tr_frag<1>(sAh, 32 * kc, 0, lane);
            const bf16x8_t al = tr_frag<1>(sAl, 32 * kc, 0, lane);
#pragma unroll
            for (int j = 0; j < HD / 16; j++) {
                const bf16x8_t bq = tr_frag<VST>(sQn, 32 * kc, 16 * j, lane);
                accK[j] = mfma16(al, bq, accK[j]);
                accK[j] = mfma16(ah, bq, accK[j]);
            }
        }
    }
    float* pK = part + (int64_t)bh * T * HD;
    float* pV = part + ((int64_t)gridDim.x / nkt + bh) * T * HD;
#pragma unroll
    for (int j = 0; j < HD / 16; j++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            int key = kbase + r;
            if (key < T) {
                pK[(int64_t)key * HD + 16 * j + (lane & 15)] = accK[j][r];
                pV[(int64_t)key * HD + 16 * j + (lane & 15)] = accV[j][r];
            }
        }
}

// dK[b,t,hkv,:] = bf16(scale * sum_g part_K[b, hkv*grp+g, t, :]) and dV
// likewise without the scale; heads summed in order.
__global__ void k_attn_dkv_reduce(const float* __restrict__ part, bf16* __restrict__ dK,
                                  bf16* __restrict__ dV, int B, int T, int Hq, int Hkv, int HD,
                                  float scale) {
    int64_t n = (int64_t)B * T * Hkv * HD;
    int64_t nbh = (int64_t)B * Hq;
    int grp = Hq / Hkv;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        int d = (int)(i % HD);
        int64_t r = i / HD;
        int hkv = (int)(r % Hkv);
        int64_t bt = r / Hkv;
        int t = (int)(bt % T), b = (int)(bt / T);
        float sk = 0.f, sv = 0.f;
        for (int g = 0; g < grp; g++) {
            int64_t bh = (int64_t)b * Hq + hkv * grp + g;
            sk += part[(bh * T + t) * HD + d];
            sv += part[((nbh + bh) * T + t) * HD + d];
        }
        dK[i] = f2bf(scale * sk);
        dV[i] = f2bf(sv);
    }
}

static inline bool a16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int attn_fwd(const bf16* Q, const bf16* K, const bf16* V, bf16* O, float* O32, float* P,
             float* stats, int B, int T, int Hq, int Hkv, int hd, bool zero_fill, hipStream_t s) {
    TA_REQUIRE(B > 0 && T > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0,
               "sdpa_fwd: bad shape B=%d T=%d Hq=%d Hkv=%d", B, T, Hq, Hkv);
    TA_REQUIRE(P || stats, "sdpa_fwd: neither probabilities nor row statistics requested");
    TA_REQUIRE(hd == 64 || hd == 128, "sdpa_fwd: head_dim %d not supported (64 or 128)", hd);
    TA_REQUIRE(a16(Q) && a16(K) && a16(V) && a16(O), "sdpa_fwd: tensors must be 16-byte aligned");
    int nqt = (T + TQ - 1) / TQ;
    int64_t blocks = (int64_t)B * Hq * nqt;
    float scale = 1.f / sqrtf((float)hd);
    const bool timed = kprof_begin(KP_ATTN_FWD, s);
    float2* st = (float2*)stats;
#define AF(H) \
    tlaunch(k_attn_fwd<H, true>, dim3((int)blocks), dim3(256), s, Q, K, V, O, O32, P, st, T, Hq, Hkv, scale, zero_fill)
#define AF1(H)                                                                             \
    tlaunch(k_attn_fwd_t<H>, dim3((int)((int64_t)B * Hq * ((T + TQ2 - 1) / TQ2))), dim3(256), s, \
        Q, K, V, O, O32, st, T, Hq, Hkv, scale)
    // with P: two passes (P normalised when it is written); without: one
    if (hd == 64) {
        if (P) AF(64); else AF1(64);
    } else {
        if (P) AF(128); else AF1(128);
    }
#undef AF
#undef AF1
    if (timed) {
        // causal S = QK^T and O = PV; Q, K, V read, O written (and O32),
        // P written (causal half, or all of it when the upper triangle is
        // zero-filled)
        double tri = (double)B * Hq * T * (T + 1) / 2.0, bt = (double)B * T;
        double pbytes = !P ? 8.0 * B * Hq * (double)T : zero_fill ? 4.0 * B * Hq * (double)T * T : 4.0 * tri;
        kprof_end(KP_ATTN_FWD, s, 4.0 * hd * tri,
                  2.0 * bt * hd * (2.0 * Hq + 2.0 * Hkv) + (O32 ? 4.0 * bt * Hq * hd : 0.0) +
                      pbytes,
                  hd == 64 ? (P ? "void ta::k_attn_fwd<64, true>" : "void ta::k_attn_fwd_t<64>")
                           : (P ? "void ta::k_attn_fwd<128, true>" : "void ta::k_attn_fwd_t<128>"));
    }
    return check_launch("sdpa_fwd");
}

int64_t attn_bwd_rowbuf_floats(int B, int T, int Hq) {
    return (int64_t)B * Hq * ((T + TQ - 1) / TQ) * QST;
}

// Dbuf: attn_bwd_rowbuf_floats(B, T, Hq) floats: the row dots [B*Hq*T], or
// on the recompute path the per-tile (max, 1/sum, D) blocks; part: up to
// [2*B*Hq*T*hd] F32 dK/dV partials (both drawn from the scratch pool when
// NULL).  O32: the forward's F32 output [B*T, Hq*hd] (NULL: the row dots
// are formed from P).  P NULL: the probabilities are recomputed from Q, K
// and the forward's row statistics (stats, [B*Hq*T] (max, 1/sum) pairs),
// which needs O32.
int attn_bwd(const bf16* dO, const bf16* Q, const bf16* K, const bf16* V, const float* P,
             const float* stats, const float* O32, bf16* dQ, bf16* dK, bf16* dV, int B, int T,
             int Hq, int Hkv, int hd, float* Dbuf, float* part, hipStream_t s,
             const float2* rtab) {
    TA_REQUIRE(P || (stats && O32), "sdpa_bwd: without P, the row statistics and O32 are needed");
    TA_REQUIRE(!rtab || !P, "sdpa_bwd: the fused inverse RoPE is for the recompute path");
    TA_REQUIRE(B > 0 && T > 0 && Hq > 0 && Hkv > 0 && Hq % Hkv == 0,
               "sdpa_bwd: bad shape B=%d T=%d Hq=%d Hkv=%d", B, T, Hq, Hkv);
    TA_REQUIRE(hd == 64 || hd == 128, "sdpa_bwd: head_dim %d not supported (64 or 128)", hd);
    TA_REQUIRE(a16(dO) && a16(Q) && a16(K) && a16(V) && a16(dQ) && a16(dK) && a16(dV),
               "sdpa_bwd: tensors must be 16-byte aligned");
    TA_REQUIRE(!O32 || a16(O32), "sdpa_bwd: O32 must be 16-byte aligned");
    if (!Dbuf) {
        Dbuf = (float*)scratch_get((size_t)attn_bwd_rowbuf_floats(B, T, Hq) * sizeof(float), s);
        TA_REQUIRE(Dbuf, "sdpa_bwd: scratch allocation failed");
    }
    int nqt = (T + TQ - 1) / TQ;
    float scale = 1.f / sqrtf((float)hd);
    int64_t b1 = (int64_t)B * Hq * nqt;
    const bool rc = P == nullptr;
    const int grp = Hq / Hkv, nkb = (T + 127) / 128;
    // recompute path: the query heads of a GQA group split into runs so that
    // the grid holds about 384 blocks (1.5 per CU); one run per group writes
    // dK/dV directly, several add their F32 partials afterwards
    const int nsplit = rc ? std::max(1, std::min(grp, (int)((384 + (int64_t)B * Hkv * nkb - 1) /
                                                           ((int64_t)B * Hkv * nkb))))
                          : grp;
    if (!part && (!rc || nsplit > 1)) {
        part = (float*)scratch_get((size_t)2 * B * Hq * T * hd * sizeof(float), s, 2);
        TA_REQUIRE(part, "sdpa_bwd: scratch allocation failed");
    }
    // row dots D: formed inside the dQ pass on the recompute path; otherwise here
    if (rc) {
    } else if (O32) {
        int64_t thr = (int64_t)B * T * Hq * (hd / 8);
        int blocks = (int)((thr + 255) / 256);
        if (hd == 64)
            tlaunch(k_attn_rowdot_o<64>, dim3(blocks), dim3(256), s, dO, O32, Dbuf, B, T, Hq);
        else
            tlaunch(k_attn_rowdot_o<128>, dim3(blocks), dim3(256), s, dO, O32, Dbuf, B, T, Hq);
    } else {
        if (hd == 64)
            tlaunch(k_attn_rowdot_p<64>, dim3((int)b1), dim3(256), s, dO, V, P, Dbuf, T, Hq, Hkv);
        else
            tlaunch(k_attn_rowdot_p<128>, dim3((int)b1), dim3(256), s, dO, V, P, Dbuf, T, Hq, Hkv);
    }
    // algorithmic work (causal half): dq pass dP = dO V^T, dQ = dS K; dkv
    // pass dP again, dV = P^T dO, dK = dS^T Q.  Bytes: BF16 operands, P and
    // the row dots read once, outputs written once (stored-P dkv: F32
    // partials)
    const double tri = (double)B * Hq * T * (T + 1) / 2.0, bt = (double)B * T;
    const float2* st = (const float2*)stats;
    // with recomputation each pass also forms S = QK^T again (2 hd flops per
    // causal element) and reads the row statistics instead of P
    const double pb = rc ? 8.0 * B * Hq * (double)T : 4.0 * tri, rf = rc ? 2.0 * hd * tri : 0.0;
    bool timed = kprof_begin(KP_ATTN_BWD_DQ, s);
    // stored P: the reference's form (64-query tiles); recompute: the
    // transposed-score kernel (128-query blocks)
#define DQ(H)                                                                             \
    tlaunch(k_attn_bwd_dq<H>, dim3((int)b1), dim3(256), s, dO, K, V, P, Dbuf, dQ, T, Hq, Hkv, scale)
#define DQT(H)                                                                            \
    tlaunch(k_attn_bwd_dq_t<H>, dim3((int)((int64_t)B * Hq * ((T + TQ2 - 1) / TQ2))), dim3(256), s, \
        dO, Q, K, V, st, Dbuf, O32, dQ, T, Hq, Hkv, scale, rtab)
    if (hd == 64) {
        if (rc) DQT(64); else DQ(64);
    } else {
        if (rc) DQT(128); else DQ(128);
    }
#undef DQ
#undef DQT
    if (timed)
        kprof_end(KP_ATTN_BWD_DQ, s, 4.0 * hd * tri + rf,
                  pb + 2.0 * bt * hd * (2.0 * Hq + 2.0 * Hkv) + 4.0 * bt * Hq,
                  hd == 64 ? (rc ? "void ta::k_attn_bwd_dq_t<64>" : "void ta::k_attn_bwd_dq<64>")
                           : (rc ? "void ta::k_attn_bwd_dq_t<128>" : "void ta::k_attn_bwd_dq<128>"));
    timed = kprof_begin(KP_ATTN_BWD_DKV, s);
    if (rc) {
        const int blocks = nkb * B * Hkv * nsplit;
        if (hd == 64)
            tlaunch(k_attn_bwd_dkv_r<64>, dim3(blocks), dim3(512), s, dO, Q, K, V, Dbuf, part, dK, dV, T, Hq,
                                                         Hkv, nsplit, scale, rtab);
        else
            tlaunch(k_attn_bwd_dkv_r<128>, dim3(blocks), dim3(512), s, dO, Q, K, V, Dbuf, part, dK, dV, T, Hq,
                                                          Hkv, nsplit, scale, rtab);
    } else if (hd == 64) {
        tlaunch(k_attn_bwd_dkv<64>, dim3((int)b1), dim3(256), s, dO, Q, V, P, Dbuf, part, T, Hq, Hkv);
    } else {
        tlaunch(k_attn_bwd_dkv<128>, dim3((int)b1), dim3(256), s, dO, Q, V, P, Dbuf, part, T, Hq, Hkv);
    }
    if (timed)
        kprof_end(KP_ATTN_BWD_DKV, s, 6.0 * hd * tri + rf,
                  rc ? 12.0 * B * Hq * (double)T + 2.0 * bt * hd * (2.0 * Hq + 4.0 * Hkv)
                     : pb + 2.0 * bt * hd * (2.0 * Hq + Hkv) + 4.0 * bt * Hq + 8.0 * bt * Hq * hd,
                  hd == 64 ? (rc ? "void ta::k_attn_bwd_dkv_r<64>" : "void ta::k_attn_bwd_dkv<64>")
                           : (rc ? "void ta::k_attn_bwd_dkv_r<128>" : "void ta::k_attn_bwd_dkv<128>"));
    if (!rc) {
        int64_t n = (int64_t)B * T * Hkv * hd;
        int rb = (int)std::min<int64_t>((n + 255) / 256, 4096);
        tlaunch(k_attn_dkv_reduce, dim3(rb), dim3(256), s, part, dK, dV, B, T, Hq, Hkv, hd, scale);
    } else if (nsplit > 1) {
        const int64_t n4 = (int64_t)B * T * Hkv * hd / 4;
        TA_REQUIRE(!rtab || 4 * n4 < (int64_t(1) << 31), "sdpa_bwd: %lld dK elements for the fused RoPE",
                   (long long)(4 * n4));
        const int rb = (int)std::min<int64_t>((n4 + 255) / 256, 4096);
        tlaunch(k_attn_dkv_sum, dim3(rb), dim3(256), s, (const float4*)part, (uint2*)dK, (uint2*)dV, n4,
                                          nsplit, scale, rtab, T, Hkv * hd, hd);
    }
    return check_launch("sdpa_bwd");
}

}  // namespace ta

extern "C" {

int ta_sdpa_fwd(const uint16_t* Q, const uint16_t* K, const uint16_t* V, uint16_t* out,
                float* attn_w, int B, int T, int Hq, int Hkv, int head_dim, void* stream) {
    return ta::attn_fwd(Q, K, V, out, nullptr, attn_w, nullptr, B, T, Hq, Hkv, head_dim, true,
                        (hipStream_t)stream);
}

int ta_attn_fwd_rowstats(const uint16_t* Q, const uint16_t* K, const uint16_t* V, uint16_t* O,
                         float* O32, float* stats, int B, int T, int Hq, int Hkv, int head_dim,
                         void* stream) {
    TA_REQUIRE(Q && K && V && O && stats, "attn_fwd_rowstats: null argument");
    return ta::attn_fwd(Q, K, V, O, O32, nullptr, stats, B, T, Hq, Hkv, head_dim, false,
                    (hipStream_t)stream);
}

int ta_attn_bwd_rowstats(const uint16_t* dout, const uint16_t* Q, const uint16_t* K,
                         const uint16_t* V, const float* stats, const float* O32, uint16_t* dQ,
                         uint16_t* dK, uint16_t* dV, int B, int T, int Hq, int Hkv, int head_dim,
                         void* stream) {
    TA_REQUIRE(dout && Q && K && V && stats && O32 && dQ && dK && dV,
               "attn_bwd_rowstats: null argument");
    return ta::attn_bwd(dout, Q, K, V, nullptr, stats, O32, dQ, dK, dV, B, T, Hq, Hkv, head_dim,
                    nullptr, nullptr, (hipStream_t)stream);
}

int ta_sdpa_bwd(const uint16_t* dout, const uint16_t* Q, const uint16_t* K, const uint16_t* V,
                const float* attn_w, uint16_t* dQ, uint16_t* dK, uint16_t* dV, int B, int T,
                int Hq, int Hkv, int head_dim, void* stream) {
    return ta::attn_bwd(dout, Q, K, V, attn_w, nullptr, nullptr, dQ, dK, dV, B, T, Hq, Hkv,
                        head_dim, nullptr, nullptr, (hipStream_t)stream);
}

}  // extern "C"
