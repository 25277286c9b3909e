// norm.hip — RMSNorm forward/backward and interleaved RoPE on gfx950.
//
// RMSNorm: one wave64 per row, 4 rows per 256-thread block.  A row is held in
// registers as 16-byte chunks (8 BF16) — D <= 64*8*MAXC — so x (and dy) are
// read from HBM exactly once; the row reduction is a 64-lane xor butterfly,
// no LDS and no block barrier.  Rows whose D is not a multiple of 8 take a
// scalar one-wave path.
//
// RoPE: one thread per (token, 4 consecutive pairs) computes the 4 angles
// once and rotates that slice of every head of the token, so sincos work is
// amortised over H heads and the data moves as 16-byte vectors.
#include <mutex>
#include <vector>

#include "ta_backend.h"
#include "ta_internal.hpp"

namespace ta {

constexpr int kMaxChunks = 8;  // 8 chunks x 8 elems x 64 lanes = D <= 4096 in registers

// ── RMSNorm forward — ops.cu:59-97 ──────────────────────────────────────
// inv = 1/sqrt(mean(x^2) + eps) is stored (the reference stores the inverse,
// ops.cu:84-86); out = bf16(x * inv * w).
// RES: the normalised row is x = bf16(x + x2), the residual add of
// qwen2.cu (add2, ops.cu:1087-1094) fused in; x is also written to xs.
template <int MAXC, bool RES = false>
__global__ __launch_bounds__(256) void k_rms_fwd_v8(const bf16* __restrict__ x,
                                                    const bf16* __restrict__ w,
                                                    bf16* __restrict__ out,
                                                    float* __restrict__ rms_out, int64_t rows,
                                                    int D, float eps,
                                                    const bf16* __restrict__ x2 = nullptr,
                                                    bf16* __restrict__ xs = nullptr) {
    int lane = threadIdx.x & 63;
    int64_t row = blockIdx.x * 4ll + (threadIdx.x >> 6);
    if (row >= rows) return;
    const bf16x8v* xr = (const bf16x8v*)(x + row * D);
    int nc = D >> 3;
    bf16x8v v[MAXC];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < MAXC; j++) {
        int c = lane + 64 * j;
        if (c < nc) {
            v[j] = xr[c];
            if constexpr (RES) {
                float a[8], b[8];
                unpack8(v[j], a);
                unpack8(((const bf16x8v*)(x2 + row * D))[c], b);
#pragma unroll
                for (int e = 0; e < 8; e++) a[e] = a[e] + b[e];
                v[j] = pack8(a);
                ((bf16x8v*)(xs + row * D))[c] = v[j];
            }
            float f[8];
            unpack8(v[j], f);
#pragma unroll
            for (int e = 0; e < 8; e++) ss += f[e] * f[e];
        }
    }
    ss = wave_sum(ss);
    float inv = 1.f / sqrtf(ss / (float)D + eps);
    if (lane == 0) rms_out[row] = inv;
    bf16x8v* orow = (bf16x8v*)(out + row * D);
#pragma unroll
    for (int j = 0; j < MAXC; j++) {
        int c = lane + 64 * j;
        if (c < nc) {
            float f[8], g[8];
            unpack8(v[j], f);
            unpack8(((const bf16x8v*)w)[c], g);
#pragma unroll
            for (int e = 0; e < 8; e++) f[e] = f[e] * inv * g[e];
            orow[c] = pack8(f);
        }
    }
}

__global__ __launch_bounds__(256) void k_rms_fwd_scalar(const bf16* __restrict__ x,
                                                        const bf16* __restrict__ w,
                                                        bf16* __restrict__ out,
                                                        float* __restrict__ rms_out,
                                                        int64_t rows, int D, float eps) {
    int lane = threadIdx.x & 63;
    int64_t row = blockIdx.x * 4ll + (threadIdx.x >> 6);
    if (row >= rows) return;
    const bf16* xr = x + row * D;
    float ss = 0.f;
    for (int i = lane; i < D; i += 64) {
        float f = bf2f(xr[i]);
        ss += f * f;
    }
    ss = wave_sum(ss);
    float inv = 1.f / sqrtf(ss / (float)D + eps);
    if (lane == 0) rms_out[row] = inv;
    for (int i = lane; i < D; i += 64) out[row * D + i] = f2bf(bf2f(xr[i]) * inv * bf2f(w[i]));
}

// ── RMSNorm backward — ops.cu:113-158 ───────────────────────────────────
// dot = sum dy*w*xhat ; dx = inv*(w*dy - xhat*dot/D) ; dw += dy*xhat.
// With dw requested, each block folds its rows' dy*xhat into a per-block
// partial row (fixed order: waves, then rows) and a second kernel sums the
// partials in block order, so dw is deterministic.
// ACC: dx is not stored but added into the residual gradient,
// dx_acc = bf16(dx_acc + bf16(dx)) (add_inplace, ops.cu:1087-1094, fused in).
template <int MAXC, bool DW, bool ACC = false>
__global__ __launch_bounds__(256) void k_rms_bwd_v8(const bf16* __restrict__ dy,
                                                    const bf16* __restrict__ x,
                                                    const bf16* __restrict__ w,
                                                    const float* __restrict__ rms,
                                                    bf16* __restrict__ dx,
                                                    float* __restrict__ dw_part, int64_t rows,
                                                    int D, int rows_per_block) {
    int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    int nc = D >> 3;
    float dwacc[DW ? MAXC * 8 : 1];
    if (DW)
#pragma unroll
        for (int i = 0; i < MAXC * 8; i++) dwacc[i] = 0.f;
    int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    for (int rr = wv; rr < rows_per_block; rr += 4) {
        int64_t row = r0 + rr;
        if (row >= rows) break;
        float inv = rms[row];
        const bf16x8v* dyr = (const bf16x8v*)(dy + row * D);
        const bf16x8v* xr = (const bf16x8v*)(x + row * D);
        bf16x8v vd[MAXC], vx[MAXC];
        float dot = 0.f;
#pragma unroll
        for (int j = 0; j < MAXC; j++) {
            int c = lane + 64 * j;
            if (c < nc) {
                vd[j] = dyr[c];
                vx[j] = xr[c];
                float a[8], b[8], g[8];
                unpack8(vd[j], a);
                unpack8(vx[j], b);
                unpack8(((const bf16x8v*)w)[c], g);
#pragma unroll
                for (int e = 0; e < 8; e++) dot += a[e] * g[e] * (b[e] * inv);
            }
        }
        dot = wave_sum(dot);
        float corr = dot / (float)D;
        bf16x8v* dxr = (bf16x8v*)(dx + row * D);
#pragma unroll
        for (int j = 0; j < MAXC; j++) {
            int c = lane + 64 * j;
            if (c < nc) {
                float a[8], b[8], g[8], o[8];
                unpack8(vd[j], a);
                unpack8(vx[j], b);
                unpack8(((const bf16x8v*)w)[c], g);
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float xh = b[e] * inv;
                    o[e] = inv * (g[e] * a[e] - xh * corr);
                    if (DW) dwacc[j * 8 + e] += a[e] * xh;
                }
                if constexpr (ACC) {
                    float q[8];
                    unpack8(pack8(o), o);
                    unpack8(dxr[c], q);
#pragma unroll
                    for (int e = 0; e < 8; e++) o[e] = q[e] + o[e];
                }
                dxr[c] = pack8(o);
            }
        }
    }
    if (DW) {
        // fold the 4 waves in order through LDS, then write the block partial
        __shared__ float red[4][64 * 8];
        float* out = dw_part + (int64_t)blockIdx.x * D;
        for (int j = 0; j < MAXC; j++) {
            int c = lane + 64 * j;
#pragma unroll
            for (int e = 0; e < 8; e++) red[wv][lane * 8 + e] = dwacc[j * 8 + e];
            __syncthreads();
            if (wv == 0 && c < nc)
                for (int e = 0; e < 8; e++)
                    out[c * 8 + e] = ((red[0][lane * 8 + e] + red[1][lane * 8 + e]) +
                                      red[2][lane * 8 + e]) +
                                     red[3][lane * 8 + e];
            __syncthreads();
        }
    }
}

__global__ __launch_bounds__(256) void k_rms_bwd_scalar(const bf16* __restrict__ dy,
                                                        const bf16* __restrict__ x,
                                                        const bf16* __restrict__ w,
                                                        const float* __restrict__ rms,
                                                        bf16* __restrict__ dx,
                                                        float* __restrict__ dw_part,
                                                        int64_t rows, int D) {
    // one block per row (used for odd D only); dw partial = this row's term
    int64_t row = blockIdx.x;
    if (row >= rows) return;
    __shared__ float red[4];
    float inv = rms[row];
    float dot = 0.f;
    for (int i = threadIdx.x; i < D; i += 256)
        dot += bf2f(dy[row * D + i]) * bf2f(w[i]) * (bf2f(x[row * D + i]) * inv);
    dot = wave_sum(dot);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = dot;
    __syncthreads();
    dot = ((red[0] + red[1]) + red[2]) + red[3];
    float corr = dot / (float)D;
    for (int i = threadIdx.x; i < D; i += 256) {
        float a = bf2f(dy[row * D + i]), xh = bf2f(x[row * D + i]) * inv;
        dx[row * D + i] = f2bf(inv * (bf2f(w[i]) * a - xh * corr));
        if (dw_part) dw_part[row * D + i] = a * xh;
    }
}

__global__ void k_sum_partials(const float* __restrict__ part, float* __restrict__ dw,
                               int nparts, int D) {
    int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= D) return;
    float s = 0.f;
    for (int p = 0; p < nparts; p++) s += part[(int64_t)p * D + d];
    dw[d] += s;
}

// ── RoPE — ops.cu:176-192 ───────────────────────────────────────────────
// Pairs (2i, 2i+1) of each head rotate by angle = t * theta^(-2i/hd)
// (negated for the backward).  x is [B*T, H*hd]; t = row % T.
__global__ __launch_bounds__(256) void k_rope_v8(bf16* __restrict__ x, int64_t rows, int T,
                                                 int H, int hd, float theta, float sign) {
    int qpr = hd >> 3;  // 16-byte chunks per head (4 pairs each)
    int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    int64_t row = gid / qpr;
    int q = (int)(gid % qpr);
    if (row >= rows) return;
    int t = (int)(row % T);
    float cs[4], sn[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        int i = q * 4 + p;
        float freq = powf(theta, -2.f * (float)i / (float)hd);
        float angle = (float)t * freq * sign;
        sincosf(angle, &sn[p], &cs[p]);
    }
    bf16x8v* base = (bf16x8v*)(x + row * (int64_t)H * hd) + q;
    for (int h = 0; h < H; h++) {
        bf16x8v v = base[h * qpr];
        float f[8], o[8];
        unpack8(v, f);
#pragma unroll
        for (int p = 0; p < 4; p++) {
            o[2 * p] = f[2 * p] * cs[p] - f[2 * p + 1] * sn[p];
            o[2 * p + 1] = f[2 * p] * sn[p] + f[2 * p + 1] * cs[p];
        }
        base[h * qpr] = pack8(o);
    }
}

// The same rotation from a table of (cos, sin) per (t, pair), built once per
// (T, hd, theta, sign) with exactly the per-element expressions above, so
// the results are the same bits; one thread per 16-byte chunk of a head.
__global__ void k_rope_table(float2* __restrict__ tab, int T, int hd, float theta, float sign) {
    int half = hd >> 1;
    int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (gid >= (int64_t)T * half) return;
    int t = (int)(gid / half), i = (int)(gid % half);
    float freq = powf(theta, -2.f * (float)i / (float)hd);
    float angle = (float)t * freq * sign;
    float sn, cs;
    sincosf(angle, &sn, &cs);
    tab[gid] = make_float2(cs, sn);
}
// chunk gid of x ([rows, H * hd]): 16 bytes of one head of one row
__device__ __forceinline__ void rope_chunk(bf16* __restrict__ x, int64_t gid, int64_t rows, int T,
                                           int H, int hd, const float4* __restrict__ tab) {
    const int qpr = hd >> 3;  // 16-byte chunks per head (4 pairs each)
    int64_t row = gid / (H * qpr);
    int hq = (int)(gid % (H * qpr)), q = hq % qpr;
    if (row >= rows) return;
    int t = (int)(row % T);
    // pairs 4q .. 4q+3 of position t: two float4 of (cos, sin, cos, sin)
    const float4* tp = tab + ((int64_t)t * (hd >> 1) + 4 * q) / 2;
    float4 c01 = tp[0], c23 = tp[1];
    bf16x8v* p = (bf16x8v*)(x + row * (int64_t)H * hd) + hq;
    float f[8], o[8];
    unpack8(*p, f);
    const float cs[4] = {c01.x, c01.z, c23.x, c23.z}, sn[4] = {c01.y, c01.w, c23.y, c23.w};
#pragma unroll
    for (int e = 0; e < 4; e++) rope_rot(f[2 * e], f[2 * e + 1], cs[e], sn[e], o[2 * e], o[2 * e + 1]);
    *p = pack8(o);
}
__global__ __launch_bounds__(256) void k_rope_tab(bf16* __restrict__ x, int64_t rows, int T,
                                                  int H, int hd, const float4* __restrict__ tab) {
    rope_chunk(x, blockIdx.x * (int64_t)blockDim.x + threadIdx.x, rows, T, H, hd, tab);
}
// Q and K of a layer in one launch: chunks [0, n0) of the grid rotate x0
// (H0 heads), the rest x1 (H1 heads); K alone is too small to fill the chip
__global__ __launch_bounds__(256) void k_rope_tab2(bf16* __restrict__ x0, int H0,
                                                   bf16* __restrict__ x1, int H1, int64_t rows,
                                                   int T, int hd, int64_t n0,
                                                   const float4* __restrict__ tab) {
    const int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    if (gid < n0) rope_chunk(x0, gid, rows, T, H0, hd, tab);
    else rope_chunk(x1, gid - n0, rows, T, H1, hd, tab);
}

// Tables live for the process, one per (device, T, hd, theta, sign), built on
// first use on the caller's stream.
struct RopeTab {
    int dev, T, hd;
    float theta, sign;
    float2* tab;
};
static std::vector<RopeTab> g_rope_tabs;
static std::mutex g_rope_mu;
const float2* rope_table(int T, int hd, float theta, float sign, hipStream_t s) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lk(g_rope_mu);
    for (const RopeTab& r : g_rope_tabs)
        if (r.dev == dev && r.T == T && r.hd == hd && r.theta == theta && r.sign == sign)
            return r.tab;
    float2* tab = nullptr;
    int64_t n = (int64_t)T * (hd >> 1);
    if (hipMalloc((void**)&tab, n * sizeof(float2)) != hipSuccess) return nullptr;
    tlaunch(k_rope_table, dim3((int)((n + 255) / 256)), dim3(256), s, tab, T, hd, theta, sign);
    g_rope_tabs.push_back({dev, T, hd, theta, sign, tab});
    return tab;
}

__global__ void k_rope_scalar(bf16* __restrict__ x, int64_t rows, int T, int H, int hd,
                              float theta, float sign) {
    int half = hd >> 1;
    int64_t gid = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
    int64_t row = gid / half;
    int i = (int)(gid % half);
    if (row >= rows) return;
    int t = (int)(row % T);
    float freq = powf(theta, -2.f * (float)i / (float)hd);
    float angle = (float)t * freq * sign;
    float sn, cs;
    sincosf(angle, &sn, &cs);
    for (int h = 0; h < H; h++) {
        bf16* p = x + (row * H + h) * hd + 2 * i;
        float o0, o1;
        rope_rot(bf2f(p[0]), bf2f(p[1]), cs, sn, o0, o1);
        p[0] = f2bf(o0);
        p[1] = f2bf(o1);
    }
}

}  // namespace ta

using namespace ta;

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

namespace ta {
// xs = bf16(a + b); out = rms_norm(xs) (add2 then rms_norm_fwd in one pass)
int rms_fwd_res(const bf16* a, const bf16* b, bf16* xs, const bf16* w, bf16* out, float* rms_out,
                int64_t rows, int D, float eps, hipStream_t s) {
    if (rows == 0) return 0;
    if (!((D & 7) == 0 && D <= 64 * 8 * kMaxChunks && al16(a) && al16(b) && al16(xs) && al16(w) &&
          al16(out))) {
        if (int rc = add2_bf16(xs, a, b, rows * D, s)) return rc;
        return ta_rms_norm_fwd(xs, w, out, rms_out, 1, (int)rows, D, eps, s);
    }
    tlaunch(k_rms_fwd_v8<kMaxChunks, true>, dim3((int)((rows + 3) / 4)), dim3(256), s, a, w, out, rms_out, rows,
                                                                       D, eps, b, xs);
    return check_launch("rms_fwd_res");
}
// acc = bf16(acc + bf16(rms_norm_bwd(dy))) (rms_norm_bwd then add_inplace in
// one pass); tmp: [rows x D] scratch for shapes the fused kernel does not take
int rms_bwd_acc(const bf16* dy, const bf16* x, const bf16* w, const float* rms, bf16* acc,
                bf16* tmp, int64_t rows, int D, hipStream_t s) {
    if (rows == 0) return 0;
    if (!((D & 7) == 0 && D <= 64 * 8 * kMaxChunks && al16(dy) && al16(x) && al16(w) &&
          al16(acc))) {
        if (int rc = ta_rms_norm_bwd(dy, x, w, rms, tmp, nullptr, 1, (int)rows, D, 0.f, s))
            return rc;
        return ta_add_inplace(acc, tmp, rows * D, s);
    }
    tlaunch(k_rms_bwd_v8<kMaxChunks, false, true>, dim3((int)((rows + 3) / 4)), dim3(256), s, dy, x, w, rms, acc, nullptr, rows, D, 4);
    return check_launch("rms_bwd_acc");
}
}  // namespace ta

extern "C" {

int ta_rms_norm_fwd(const uint16_t* x, const uint16_t* w, uint16_t* out, float* rms_out, int B,
                    int T, int D, float eps, void* stream) {
    TA_REQUIRE(B >= 0 && T >= 0 && D > 0, "rms_norm_fwd: bad shape B=%d T=%d D=%d", B, T, D);
    int64_t rows = (int64_t)B * T;
    if (rows == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    int blocks = (int)((rows + 3) / 4);
    if ((D & 7) == 0 && D <= 64 * 8 * kMaxChunks && al16(x) && al16(w) && al16(out))
        tlaunch(k_rms_fwd_v8<kMaxChunks>, dim3(blocks), dim3(256), s, x, w, out, rms_out, rows, D, eps,
                nullptr, nullptr);
    else
        tlaunch(k_rms_fwd_scalar, dim3(blocks), dim3(256), s, x, w, out, rms_out, rows, D, eps);
    return check_launch("rms_norm_fwd");
}

int ta_rms_norm_bwd(const uint16_t* dy, const uint16_t* x, const uint16_t* w,
                    const float* rms_saved, uint16_t* dx, float* dw, int B, int T, int D,
                    float eps, void* stream) {
    (void)eps;  // the saved inverse rms already holds eps (ops.cu:113-158 ignores it too)
    TA_REQUIRE(B >= 0 && T >= 0 && D > 0, "rms_norm_bwd: bad shape B=%d T=%d D=%d", B, T, D);
    int64_t rows = (int64_t)B * T;
    if (rows == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    bool vec = (D & 7) == 0 && D <= 64 * 8 * kMaxChunks && al16(dy) && al16(x) && al16(w) &&
               al16(dx);
    if (vec) {
        int rpb = dw ? 64 : 4;  // with dw: fewer, fuller blocks keep the partials small
        int blocks = (int)((rows + rpb - 1) / rpb);
        if (!dw) {
            tlaunch(k_rms_bwd_v8<kMaxChunks, false>, dim3(blocks), dim3(256), s, dy, x, w, rms_saved, dx, nullptr, rows, D, rpb);
        } else {
            float* part = (float*)scratch_get((size_t)blocks * D * sizeof(float), s);
            TA_REQUIRE(part, "rms_norm_bwd: scratch allocation failed");
            tlaunch(k_rms_bwd_v8<kMaxChunks, true>, dim3(blocks), dim3(256), s, dy, x, w, rms_saved, dx, part, rows, D, rpb);
            tlaunch(k_sum_partials, dim3((D + 255) / 256), dim3(256), s, part, dw, blocks, D);
        }
    } else {
        float* part = nullptr;
        if (dw) {
            part = (float*)scratch_get((size_t)rows * D * sizeof(float), s);
            TA_REQUIRE(part, "rms_norm_bwd: scratch allocation failed");
        }
        tlaunch(k_rms_bwd_scalar, dim3((int)rows), dim3(256), s, dy, x, w, rms_saved, dx, part, rows, D);
        if (dw) tlaunch(k_sum_partials, dim3((D + 255) / 256), dim3(256), s, part, dw, (int)rows, D);
    }
    return check_launch("rms_norm_bwd");
}

static int rope(uint16_t* x, int B, int T, int H, int hd, float theta, float sign,
                void* stream) {
    TA_REQUIRE(B >= 0 && T >= 0 && H > 0 && hd > 0 && (hd % 2) == 0,
               "rope: bad shape B=%d T=%d H=%d hd=%d", B, T, H, hd);
    int64_t rows = (int64_t)B * T;
    if (rows == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    if ((hd & 7) == 0 && al16(x)) {
        const float2* tab = rope_table(T, hd, theta, sign, s);
        TA_REQUIRE(tab, "rope: table allocation failed");
        int64_t n = rows * H * (hd >> 3);
        tlaunch(k_rope_tab, dim3((int)((n + 255) / 256)), dim3(256), s, x, rows, T, H, hd, (const float4*)tab);
    } else {
        int64_t n = rows * (hd >> 1);
        tlaunch(k_rope_scalar, dim3((int)((n + 255) / 256)), dim3(256), s, x, rows, T, H, hd, theta, sign);
    }
    return check_launch("rope");
}

}  // extern "C"

namespace ta {
// rope of Q (Hq heads) and K (Hk heads) of one layer, one launch when
// both take the table path (the same bits as two rope calls)
int rope_qk(bf16* q, int Hq, bf16* k, int Hk, int B, int T, int hd, float theta, float sign,
            hipStream_t s) {
    if (B <= 0 || T <= 0 || Hq <= 0 || Hk <= 0 || hd <= 0 || (hd & 7) != 0 || !al16(q) ||
        !al16(k)) {
        if (int rc = rope(q, B, T, Hq, hd, theta, sign, s)) return rc;
        return rope(k, B, T, Hk, hd, theta, sign, s);
    }
    const int64_t rows = (int64_t)B * T;
    const float2* tab = rope_table(T, hd, theta, sign, s);
    TA_REQUIRE(tab, "rope: table allocation failed");
    const int64_t n0 = rows * Hq * (hd >> 3), n = n0 + rows * Hk * (hd >> 3);
    tlaunch(k_rope_tab2, dim3((int)((n + 255) / 256)), dim3(256), s, q, Hq, k, Hk, rows, T, hd, n0,
                                                       (const float4*)tab);
    return check_launch("rope_qk");
}
}  // namespace ta

extern "C" {

int ta_rope_fwd(uint16_t* x, int B, int T, int H, int head_dim, float theta, void* stream) {
    return rope(x, B, T, H, head_dim, theta, 1.f, stream);
}
int ta_rope_bwd(uint16_t* dx, int B, int T, int H, int head_dim, float theta, void* stream) {
    return rope(dx, B, T, H, head_dim, theta, -1.f, stream);
}

}  // extern "C"
