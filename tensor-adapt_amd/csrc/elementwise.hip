// elementwise.hip — HBM-bound streaming kernels: gated SiLU fwd/bwd, residual,
// bias and LoRA adds, casts, embedding gather/scatter.
//
// Every kernel moves 16-byte vectors (8 BF16) per lane with a grid-stride loop
// sized to fill the 256 CUs a few times over; a scalar tail handles N % 8.
// Element math follows src/backend/cuda/ops.cu line for line (cited per
// kernel); rounding to BF16 happens exactly where the reference rounds.
#include "ta_internal.hpp"

namespace ta {

static inline int stream_blocks(int64_t nvec, int threads) {
    int64_t b = (nvec + threads - 1) / threads;
    if (b > 8192) b = 8192;  // 256 CUs x 32 resident blocks: enough to saturate HBM
    if (b < 1) b = 1;
    return (int)b;
}
static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// ── SiLU-gated activation forward — ops.cu:913-923 ──────────────────────
// silu_mul_f: ta_internal.hpp
__global__ void k_silu_mul_fwd(const bf16* __restrict__ gate, const bf16* __restrict__ up,
                               bf16* __restrict__ out, int64_t N) {
    int64_t nv = N >> 3;
    const bf16x8v* g8 = (const bf16x8v*)gate;
    const bf16x8v* u8 = (const bf16x8v*)up;
    bf16x8v* o8 = (bf16x8v*)out;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nv;
         i += (int64_t)gridDim.x * blockDim.x) {
        float g[8], u[8], o[8];
        unpack8(g8[i], g);
        unpack8(u8[i], u);
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = silu_mul_f(g[e], u[e]);
        o8[i] = pack8(o);
    }
    if (blockIdx.x == 0)
        for (int64_t i = (nv << 3) + threadIdx.x; i < N; i += blockDim.x)
            out[i] = f2bf(silu_mul_f(bf2f(gate[i]), bf2f(up[i])));
}

// ── SiLU-gated activation backward — ops.cu:925-940 ─────────────────────
// silu_bwd_f: ta_internal.hpp
__global__ void k_silu_mul_bwd(const bf16* __restrict__ dout, const bf16* __restrict__ gate,
                               const bf16* __restrict__ up, bf16* __restrict__ dgate,
                               bf16* __restrict__ dup, int64_t N) {
    int64_t nv = N >> 3;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nv;
         i += (int64_t)gridDim.x * blockDim.x) {
        float d[8], g[8], u[8], a[8], b[8];
        unpack8(((const bf16x8v*)dout)[i], d);
        unpack8(((const bf16x8v*)gate)[i], g);
        unpack8(((const bf16x8v*)up)[i], u);
#pragma unroll
        for (int e = 0; e < 8; e++) silu_bwd_f(d[e], g[e], u[e], a[e], b[e]);
        ((bf16x8v*)dgate)[i] = pack8(a);
        ((bf16x8v*)dup)[i] = pack8(b);
    }
    if (blockIdx.x == 0)
        for (int64_t i = (nv << 3) + threadIdx.x; i < N; i += blockDim.x) {
            float a, b;
            silu_bwd_f(bf2f(dout[i]), bf2f(gate[i]), bf2f(up[i]), a, b);
            dgate[i] = f2bf(a);
            dup[i] = f2bf(b);
        }
}

// ── out = bf16(out + scale * delta) — add_inplace (scale 1, ops.cu:1087-1094)
//    and lora_add (ops.cu:1101-1108).  For scale == 1 the product is exact,
//    so one kernel serves both.
__global__ void k_axpy_bf16(bf16* __restrict__ out, const bf16* __restrict__ delta, float scale,
                            int64_t N) {
    int64_t nv = N >> 3;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nv;
         i += (int64_t)gridDim.x * blockDim.x) {
        float o[8], d[8];
        unpack8(((const bf16x8v*)out)[i], o);
        unpack8(((const bf16x8v*)delta)[i], d);
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = o[e] + scale * d[e];
        ((bf16x8v*)out)[i] = pack8(o);
    }
    if (blockIdx.x == 0)
        for (int64_t i = (nv << 3) + threadIdx.x; i < N; i += blockDim.x)
            out[i] = f2bf(bf2f(out[i]) + scale * bf2f(delta[i]));
}

// scalar fallbacks for unaligned pointers (every element on its own)
__global__ void k_axpy_bf16_scalar(bf16* out, const bf16* delta, float scale, int64_t N) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < N;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = f2bf(bf2f(out[i]) + scale * bf2f(delta[i]));
}
__global__ void k_silu_fwd_scalar(const bf16* gate, const bf16* up, bf16* out, int64_t N) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < N;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = f2bf(silu_mul_f(bf2f(gate[i]), bf2f(up[i])));
}
__global__ void k_silu_bwd_scalar(const bf16* dout, const bf16* gate, const bf16* up, bf16* dgate,
                                  bf16* dup, int64_t N) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < N;
         i += (int64_t)gridDim.x * blockDim.x) {
        float a, b;
        silu_bwd_f(bf2f(dout[i]), bf2f(gate[i]), bf2f(up[i]), a, b);
        dgate[i] = f2bf(a);
        dup[i] = f2bf(b);
    }
}

// ── bias add over rows — ops.cu:1062-1073 ───────────────────────────────
__global__ void k_add_bias(bf16* __restrict__ out, const bf16* __restrict__ bias, int64_t BT,
                           int D) {
    int64_t n = BT * (int64_t)D;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        int d = (int)(i % D);
        out[i] = f2bf(bf2f(out[i]) + bf2f(bias[d]));
    }
}
__global__ void k_add_bias_v8(bf16* __restrict__ out, const bf16* __restrict__ bias, int64_t BT,
                              int D) {
    int dv = D >> 3;
    int64_t nv = BT * (int64_t)dv;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nv;
         i += (int64_t)gridDim.x * blockDim.x) {
        int c = (int)(i % dv);
        float o[8], b[8];
        unpack8(((const bf16x8v*)out)[i], o);
        unpack8(((const bf16x8v*)bias)[c], b);
#pragma unroll
        for (int e = 0; e < 8; e++) o[e] = o[e] + b[e];
        ((bf16x8v*)out)[i] = pack8(o);
    }
}

// ── casts — ops.cu:1119-1126 ─────────────────────────────────────────────
__global__ void k_bf16_to_f32(const bf16* __restrict__ s, float* __restrict__ d, int64_t N) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < N;
         i += (int64_t)gridDim.x * blockDim.x)
        d[i] = bf2f(s[i]);
}
__global__ void k_f32_to_bf16(const float* __restrict__ s, bf16* __restrict__ d, int64_t N) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < N;
         i += (int64_t)gridDim.x * blockDim.x)
        d[i] = f2bf(s[i]);
}

// ── embedding gather — ops.cu:1026-1035 (one wave per token row) ─────────
__global__ void k_embed_fwd(const bf16* __restrict__ table, const int32_t* __restrict__ tokens,
                            bf16* __restrict__ out, int64_t BT, int D, bool vec) {
    int lane = threadIdx.x & 63;
    int64_t row = blockIdx.x * (int64_t)(blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= BT) return;
    int64_t tok = tokens[row];
    const bf16* src = table + tok * D;
    bf16* dst = out + row * D;
    if (vec) {
        for (int c = lane; c < (D >> 3); c += 64)
            ((bf16x8v*)dst)[c] = ((const bf16x8v*)src)[c];
    } else {
        for (int c = lane; c < D; c += 64) dst[c] = src[c];
    }
}

// The step engine's embedding gather for token ids that no host has
// checked (ids resident in device memory): an id outside [0, V) reads
// nothing, its row is written as zeros and *bad is set to 1 (a plain store;
// every writer stores the same value).
__global__ void k_embed_fwd_checked(const bf16* __restrict__ table,
                                    const int32_t* __restrict__ tokens, bf16* __restrict__ out,
                                    int64_t BT, int D, int V, bool vec, int32_t* __restrict__ bad) {
    int lane = threadIdx.x & 63;
    int64_t row = blockIdx.x * (int64_t)(blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= BT) return;
    int64_t tok = tokens[row];
    bf16* dst = out + row * D;
    if (tok < 0 || tok >= V) {
        if (lane == 0) *bad = 1;
        for (int c = lane; c < D; c += 64) dst[c] = 0;
        return;
    }
    const bf16* src = table + tok * D;
    if (vec) {
        for (int c = lane; c < (D >> 3); c += 64)
            ((bf16x8v*)dst)[c] = ((const bf16x8v*)src)[c];
    } else {
        for (int c = lane; c < D; c += 64) dst[c] = src[c];
    }
}

int embed_fwd_checked(const bf16* table, const int32_t* tokens, bf16* out, int64_t BT, int D,
                      int V, int32_t* bad, hipStream_t s) {
    TA_REQUIRE(BT >= 0 && D > 0 && V > 0 && bad, "embed_fwd_checked: bad arguments");
    if (BT == 0) return 0;
    bool vec = (D & 7) == 0 && aligned16(table) && aligned16(out);
    tlaunch(k_embed_fwd_checked, dim3((int)((BT + 3) / 4)), dim3(256), s, table, tokens, out, BT, D, V, vec,
                                                            bad);
    return check_launch("embed_fwd_checked");
}

// ── embedding scatter-add — ops.cu:1037-1046 (F32 atomics, as the reference;
//    dead code in the reference trainer, kept for API completeness) ────────
__global__ void k_embed_bwd(const bf16* __restrict__ dout, const int32_t* __restrict__ tokens,
                            float* __restrict__ dtable, int64_t BT, int D) {
    int lane = threadIdx.x & 63;
    int64_t row = blockIdx.x * (int64_t)(blockDim.x >> 6) + (threadIdx.x >> 6);
    if (row >= BT) return;
    int64_t tok = tokens[row];
    for (int c = lane; c < D; c += 64) atomicAdd(&dtable[tok * D + c], bf2f(dout[row * D + c]));
}

}  // namespace ta

using namespace ta;

extern "C" {

int ta_silu_mul_fwd(const uint16_t* gate, const uint16_t* up, uint16_t* out, int64_t N,
                    void* stream) {
    TA_REQUIRE(N >= 0, "silu_mul_fwd: N < 0");
    if (N == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    if (aligned16(gate) && aligned16(up) && aligned16(out))
        tlaunch(k_silu_mul_fwd, dim3(stream_blocks(N >> 3, 256)), dim3(256), s, gate, up, out, N);
    else
        tlaunch(k_silu_fwd_scalar, dim3(stream_blocks(N, 256)), dim3(256), s, gate, up, out, N);
    return check_launch("silu_mul_fwd");
}

int ta_silu_mul_bwd(const uint16_t* dout, const uint16_t* gate, const uint16_t* up,
                    uint16_t* dgate, uint16_t* dup, int64_t N, void* stream) {
    TA_REQUIRE(N >= 0, "silu_mul_bwd: N < 0");
    if (N == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    if (aligned16(dout) && aligned16(gate) && aligned16(up) && aligned16(dgate) && aligned16(dup))
        tlaunch(k_silu_mul_bwd, dim3(stream_blocks(N >> 3, 256)), dim3(256), s, dout, gate, up, dgate, dup, N);
    else
        tlaunch(k_silu_bwd_scalar, dim3(stream_blocks(N, 256)), dim3(256), s, dout, gate, up, dgate, dup, N);
    return check_launch("silu_mul_bwd");
}

static int axpy(uint16_t* out, const uint16_t* delta, float scale, int64_t N, void* stream,
                const char* name) {
    TA_REQUIRE(N >= 0, "%s: N < 0", name);
    if (N == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    if (aligned16(out) && aligned16(delta))
        tlaunch(k_axpy_bf16, dim3(stream_blocks(N >> 3, 256)), dim3(256), s, out, delta, scale, N);
    else
        tlaunch(k_axpy_bf16_scalar, dim3(stream_blocks(N, 256)), dim3(256), s, out, delta, scale, N);
    return check_launch(name);
}

int ta_add_inplace(uint16_t* out, const uint16_t* delta, int64_t N, void* stream) {
    return axpy(out, delta, 1.f, N, stream, "add_inplace");
}

int ta_lora_add(uint16_t* out, const uint16_t* delta, float scale, int64_t N, void* stream) {
    return axpy(out, delta, scale, N, stream, "lora_add");
}

int ta_add_bias(uint16_t* out, const uint16_t* bias, int BT, int D, void* stream) {
    TA_REQUIRE(BT >= 0 && D > 0, "add_bias: bad shape BT=%d D=%d", BT, D);
    if (BT == 0) return 0;
    hipStream_t s = (hipStream_t)stream;
    if ((D & 7) == 0 && aligned16(out) && aligned16(bias))
        tlaunch(k_add_bias_v8, dim3(stream_blocks((int64_t)BT * (D >> 3), 256)), dim3(256), s, out, bias, BT, D);
    else
        tlaunch(k_add_bias, dim3(stream_blocks((int64_t)BT * D, 256)), dim3(256), s, out, bias, BT, D);
    return check_launch("add_bias");
}

int ta_cast_bf16_to_f32(const uint16_t* src, float* dst, int64_t N, void* stream) {
    TA_REQUIRE(N >= 0, "cast_bf16_to_f32: N < 0");
    if (N == 0) return 0;
    tlaunch(k_bf16_to_f32, dim3(stream_blocks(N, 256)), dim3(256), (hipStream_t)stream, src, dst, N);
    return check_launch("cast_bf16_to_f32");
}

int ta_cast_f32_to_bf16(const float* src, uint16_t* dst, int64_t N, void* stream) {
    TA_REQUIRE(N >= 0, "cast_f32_to_bf16: N < 0");
    if (N == 0) return 0;
    tlaunch(k_f32_to_bf16, dim3(stream_blocks(N, 256)), dim3(256), (hipStream_t)stream, src, dst, N);
    return check_launch("cast_f32_to_bf16");
}

int ta_embed_fwd(const uint16_t* table, const int32_t* tokens, uint16_t* out, int BT, int D,
                 void* stream) {
    TA_REQUIRE(BT >= 0 && D > 0, "embed_fwd: bad shape BT=%d D=%d", BT, D);
    if (BT == 0) return 0;
    bool vec = (D & 7) == 0 && aligned16(table) && aligned16(out);
    int blocks = (BT + 3) / 4;
    tlaunch(k_embed_fwd, dim3(blocks), dim3(256), (hipStream_t)stream, table, tokens, out, BT, D, vec);
    return check_launch("embed_fwd");
}

int ta_embed_bwd(const uint16_t* dout, const int32_t* tokens, float* dtable, int BT, int D,
                 void* stream) {
    TA_REQUIRE(BT >= 0 && D > 0, "embed_bwd: bad shape BT=%d D=%d", BT, D);
    if (BT == 0) return 0;
    int blocks = (BT + 3) / 4;
    tlaunch(k_embed_bwd, dim3(blocks), dim3(256), (hipStream_t)stream, dout, tokens, dtable, BT, D);
    return check_launch("embed_bwd");
}

}  // extern "C"
