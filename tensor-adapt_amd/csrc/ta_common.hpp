// ta_common.hpp — device helpers shared by every gfx950 kernel of the backend.
//
// BF16 values travel as raw uint16_t bit patterns (the C-ABI has no HIP
// types in it).  Conversions are IEEE round-to-nearest-even on the F32 bit
// pattern with NaN kept quiet, which is what __float2bfloat16 does on the
// reference side (src/backend/cuda/ops.cu, every kernel output).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace ta {

typedef uint16_t bf16;

__device__ __forceinline__ float bf2f(bf16 h) {
    return __uint_as_float((uint32_t)h << 16);
}
// gfx950's v_cvt_pk_bf16_f32 rounds to nearest even and keeps NaNs quiet
// (sign and top payload bits kept, quiet bit set): the same bits as the
// integer formulation u + 0x7fff + lsb, checked over 5M patterns including
// ties, denormals and NaNs.  One instruction, no branch.
__device__ __forceinline__ bf16 f2bf(float f) {
    return __builtin_bit_cast(uint16_t, (__bf16)f);
}
// two bf16 packed in one 32-bit word (low half = first element)
__device__ __forceinline__ float lo2f(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi2f(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
typedef __bf16 ta_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float ta_floatx2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((ta_floatx2_t){a, b}, ta_bf16x2_t));
}

// 8 bf16 = 16 bytes, the natural global/LDS vector on CDNA.
struct alignas(16) bf16x8v { uint32_t w[4]; };

__device__ __forceinline__ void unpack8(const bf16x8v& v, float* f) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = lo2f(v.w[i]);
        f[2 * i + 1] = hi2f(v.w[i]);
    }
}
__device__ __forceinline__ bf16x8v pack8(const float* f) {
    bf16x8v v;
#pragma unroll
    for (int i = 0; i < 4; i++) v.w[i] = pack2(f[2 * i], f[2 * i + 1]);
    return v;
}

// wave64 reductions (xor butterflies over all 64 lanes)
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

constexpr float kLog2e = 1.4426950408889634f;

// RoPE rotation of one interleaved pair (x0, x1) by (cs, sn) = (cos, sin) of
// its angle (ops.cu:176-204): x0 cs - x1 sn and x0 sn + x1 cs, written as
// the contracted form fma(x0, cs, -(x1 sn)) and fma(x1, cs, x0 sn), the
// products with sn rounded on their own (the empty asm statement keeps the
// compiler from fusing them elsewhere).  Every kernel that rotates uses
// this, so a rotation gives the same bits in whichever kernel it runs.
__device__ __forceinline__ void rope_rot(float x0, float x1, float cs, float sn, float& o0,
                                         float& o1) {
    float b = x1 * sn, c = x0 * sn;
    asm volatile("" : "+v"(b), "+v"(c));
    o0 = __builtin_fmaf(x0, cs, -b);
    o1 = __builtin_fmaf(x1, cs, c);
}

// ── SwiGLU math (ops.cu:913-940), shared by the elementwise kernels and the
// fused SwiGLU-backward + LoRA kernel.  exp(-g) as v_exp_f32 of -g log2(e)
// and the quotient as v_rcp_f32 (each within 1 ulp of F32; the reference is
// built with --use_fast_math, whose __expf and division are approximations
// of the same kind).
__device__ __forceinline__ float sigmoid_f(float g) {
    return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-g * kLog2e));
}
__device__ __forceinline__ float silu_mul_f(float g, float u) {
    float s = g * sigmoid_f(g);
    return s * u;
}
__device__ __forceinline__ void silu_bwd_f(float d, float g, float u, float& dg, float& du) {
    float sig = sigmoid_f(g);
    float s = g * sig;
    float ds = sig * (1.f + g * (1.f - sig));
    dg = d * u * ds;
    du = d * s;
}

}  // namespace ta

// Launch-status plumbing for the C-ABI: every entry point returns 0 or a
// negative code and leaves a message for ta_last_error().
namespace ta {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
}  // namespace ta

#define TA_REQUIRE(cond, ...)                                     \
    do {                                                          \
        if (!(cond)) return ::ta::set_error(-1, __VA_ARGS__);     \
    } while (0)

#define TA_HIP(call)                                                              \
    do {                                                                          \
        hipError_t _e = (call);                                                   \
        if (_e != hipSuccess)                                                     \
            return ::ta::set_error(-2, "%s: %s", #call, hipGetErrorString(_e));   \
    } while (0)
