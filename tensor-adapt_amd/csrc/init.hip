// init.hip — device-side set-up kernels of the step engine: weight
// transposes (the engine keeps W and W^T resident), synthetic base weights,
// the LoRA A initialisation, and the out-of-place residual add.
#include <string.h>

#include "ta_internal.hpp"

namespace ta {

// out[c][r] = in[r][c] for a rows x cols BF16 matrix (64x64 LDS tiles).
__global__ __launch_bounds__(256) void k_transpose(const bf16* __restrict__ in,
                                                   bf16* __restrict__ out, int64_t rows,
                                                   int64_t cols) {
    __shared__ bf16 tile[64][65];
    int64_t tr = (int64_t)blockIdx.y * 64, tc = (int64_t)blockIdx.x * 64;
    int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int r = ty; r < 64; r += 4)
        if (tr + r < rows && tc + tx < cols) tile[r][tx] = in[(tr + r) * cols + tc + tx];
    __syncthreads();
    for (int c = ty; c < 64; c += 4)
        if (tc + c < cols && tr + tx < rows) out[(tc + c) * rows + tr + tx] = tile[tx][c];
}

int transpose_bf16(const bf16* in, bf16* out, int64_t rows, int64_t cols, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return 0;
    TA_REQUIRE((cols + 63) / 64 < (1ll << 31) && (rows + 63) / 64 < 65536,
               "transpose: matrix too large (%lld x %lld)", (long long)rows, (long long)cols);
    dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
    tlaunch(k_transpose, dim3(grid), dim3(256), s, in, out, rows, cols);
    return check_launch("transpose");
}

// Synthetic weights: element i of tensor `stream_id` is
// bf16(std * N(0,1)), the normal drawn by Box-Muller from two uniforms of
// splitmix64(seed ^ golden * (stream_id + 1) + 2i, +1).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
__global__ void k_fill_normal(bf16* __restrict__ out, int64_t n, uint64_t seed, uint64_t sid,
                              float std) {
    uint64_t base = seed ^ (0x9E3779B97F4A7C15ull * (sid + 1));
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        uint64_t a = mix64(base + 2 * (uint64_t)i), b = mix64(base + 2 * (uint64_t)i + 1);
        double u1 = ((double)(a >> 11) + 0.5) * (1.0 / 9007199254740992.0);
        double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);
        double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
        out[i] = f2bf((float)(z * std));
    }
}
int fill_normal_bf16(bf16* out, int64_t n, uint64_t seed, uint64_t sid, float std,
                     hipStream_t s) {
    if (n <= 0) return 0;
    tlaunch(k_fill_normal, dim3(2048), dim3(256), s, out, n, seed, sid, std);
    return check_launch("fill_normal");
}

__global__ void k_fill_bf16(bf16* __restrict__ out, int64_t n, bf16 v) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x)
        out[i] = v;
}
int fill_bf16(bf16* out, int64_t n, float v, hipStream_t s) {
    if (n <= 0) return 0;
    uint32_t u;
    memcpy(&u, &v, 4);  // host-side RNE to BF16 (finite v)
    bf16 h = (bf16)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    tlaunch(k_fill_bf16, dim3(1024), dim3(256), s, out, n, h);
    return check_launch("fill_bf16");
}

// LoRA A init — src/adapter/adapter_model.cu:15-39 with the fixed seed 0x1234
// (adapter_model.cu:53-54): integer hash of (seed, i), u in [-1, 1],
// A = u * sqrt(1/in).  Exact integer math; IEEE division and sqrt.
__global__ void k_kaiming(float* __restrict__ a32, bf16* __restrict__ a16, int64_t n, int in_dim,
                          uint32_t seed) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        uint32_t r = seed ^ ((uint32_t)i * 2654435761u);
        r = r ^ (r >> 16);
        r *= 0x45d9f3bu;
        r ^= (r >> 16);
        float u = (float)(r & 0xFFFFFFu) / (float)0xFFFFFF * 2.f - 1.f;
        float bound = sqrtf(1.f / (float)in_dim);
        float v = u * bound;
        if (a32) a32[i] = v;
        if (a16) a16[i] = f2bf(v);
    }
}
int kaiming_init(float* a32, bf16* a16, int64_t n, int in_dim, hipStream_t s) {
    if (n <= 0) return 0;
    tlaunch(k_kaiming, dim3(256), dim3(256), s, a32, a16, n, in_dim, 0x1234u);
    return check_launch("kaiming_init");
}

// out = bf16(a + b): the reference's in-place residual add
// (ops::add_inplace, ops.cu:1087-1094) written out of place, so each layer's
// residual input stays cached without a device-to-device copy.
__global__ void k_add2(bf16* __restrict__ out, const bf16* __restrict__ a,
                       const bf16* __restrict__ b, int64_t n) {
    int64_t nv = n >> 3;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < nv;
         i += (int64_t)gridDim.x * blockDim.x) {
        float x[8], y[8];
        unpack8(((const bf16x8v*)a)[i], x);
        unpack8(((const bf16x8v*)b)[i], y);
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = x[e] + y[e];
        ((bf16x8v*)out)[i] = pack8(x);
    }
    if (blockIdx.x == 0)
        for (int64_t i = (nv << 3) + threadIdx.x; i < n; i += blockDim.x)
            out[i] = f2bf(bf2f(a[i]) + bf2f(b[i]));
}
int add2_bf16(bf16* out, const bf16* a, const bf16* b, int64_t n, hipStream_t s) {
    if (n <= 0) return 0;
    TA_REQUIRE((((uintptr_t)out | (uintptr_t)a | (uintptr_t)b) & 15u) == 0,
               "add2: pointers must be 16-byte aligned");
    int64_t blocks = ((n >> 3) + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks < 1) blocks = 1;
    tlaunch(k_add2, dim3((int)blocks), dim3(256), s, out, a, b, n);
    return check_launch("add2");
}

// Assistant-span masking of src/trainer/adapt_trainer.cu:145-182 on device
// tokens.  The reference's state machine is sequential along t, but its
// state after token t depends only on the last event e <= t (a token
// 151644, which sets in_asst = (tokens[e + 1] == 77091), or 151645, which
// clears it; false before any event).  One 1024-thread block per batch row
// takes e as an inclusive prefix max of the event positions (wave shuffles,
// then the waves in order), 1024 tokens at a time with the running e
// carried over; every thread then applies the reference's per-token rule.
// Targets outside assistant spans become -1.
__global__ __launch_bounds__(1024) void k_mask_targets(const int32_t* __restrict__ in,
                                                       const int32_t* __restrict__ tgt_in,
                                                       int32_t* __restrict__ tgt, int B, int T) {
    __shared__ int wmax[16];
    __shared__ int carry_s;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t off = (int64_t)blockIdx.x * T;
    int carry = -1;  // last event before this chunk
    for (int c0 = 0; c0 < T; c0 += 1024) {
        const int t = c0 + (int)threadIdx.x;
        const int tok = t < T ? in[off + t] : 0;
        int v = (t < T && (tok == 151644 || tok == 151645)) ? t : -1;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int u = __shfl_up(v, o, 64);
            if (lane >= o) v = max(v, u);
        }
        if (lane == 63) wmax[wv] = v;
        __syncthreads();
        int pre = carry;
        for (int k = 0; k < wv; k++) pre = max(pre, wmax[k]);
        v = max(v, pre);
        bool in_asst = false;
        if (v >= 0) in_asst = in[off + v] == 151644 && v + 1 < T && in[off + v + 1] == 77091;
        bool mask = !in_asst;
        if (tok == 151644 || tok == 77091) mask = true;
        if (tok == 151645) mask = false;
        if (t < T) tgt[off + t] = mask ? -1 : tgt_in[off + t];
        if (threadIdx.x == 1023) carry_s = v;
        __syncthreads();  // carry_s written, wmax free for the next chunk
        carry = carry_s;
    }
}
int mask_targets_dev(const int32_t* in, const int32_t* tgt_in, int32_t* tgt, int B, int T,
                     hipStream_t s) {
    if (B <= 0 || T <= 0) return 0;
    tlaunch(k_mask_targets, dim3(B), dim3(1024), s, in, tgt_in, tgt, B, T);
    return check_launch("mask_targets");
}

}  // namespace ta

extern "C" int ta_lora_kaiming_init(float* a32, uint16_t* a16, int64_t n, int in_dim,
                                    void* stream) {
    TA_REQUIRE(n >= 0 && in_dim > 0, "lora_kaiming_init: bad arguments (n=%lld in_dim=%d)",
               (long long)n, in_dim);
    return ta::kaiming_init(a32, a16, n, in_dim, (hipStream_t)stream);
}
