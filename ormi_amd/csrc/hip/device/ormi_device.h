// Device helpers shared by the kernels compiled into libormi_hip.so and the
// kernels the hipRTC code generator emits (the generator embeds this file's
// text ahead of every generated kernel). Written for gfx950: wave64, DPP
// cross-lane moves, 128-bit global accesses.
//
// Numeric contract with the CPU oracle: generated code is compiled with
// -ffp-contract=off and IEEE division, so the user-visible + - * / agree bit
// for bit; the helpers below are the oracle's fp32 formulas, with the device
// math library for transcendentals (expf, tanhf, erff: a few ulp from the
// host's). One deliberate difference: sigmoid takes 1/(1+e) with the hardware
// reciprocal V_RCP_F32 (1 ulp) instead of an IEEE divide, which costs ten
// VALU instructions per element in a VALU-bound kernel; the result stays
// within 2 ulp of the oracle's.
#pragma once
#ifndef __HIPCC_RTC__
#include <hip/hip_runtime.h>
#endif

typedef float ormi_f4 __attribute__((ext_vector_type(4)));
typedef unsigned short ormi_u16x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------ conversions --
__device__ __forceinline__ float ormi_bf16_to_f32(unsigned short h) {
    return __uint_as_float((unsigned)h << 16);
}
// Round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ unsigned short ormi_f32_to_bf16(float f) {
    unsigned u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (unsigned short)(u >> 16);
}
__device__ __forceinline__ float ormi_f16_to_f32(unsigned short h) {
    _Float16 x;
    __builtin_memcpy(&x, &h, 2);
    return (float)x;
}
__device__ __forceinline__ unsigned short ormi_f32_to_f16(float f) {
    _Float16 x = (_Float16)f;
    unsigned short h;
    __builtin_memcpy(&h, &x, 2);
    return h;
}
__device__ __forceinline__ float ormi_round_bf16(float f) { return ormi_bf16_to_f32(ormi_f32_to_bf16(f)); }
__device__ __forceinline__ float ormi_round_f16(float f) { return ormi_f16_to_f32(ormi_f32_to_f16(f)); }
// float -> int64 truncates toward zero; NaN gives 0, out-of-range values saturate.
__device__ __forceinline__ long long ormi_f32_to_i64(float f) {
    if (f != f) return 0;
    if (f >= 9.2233720368547758e18f) return 0x7fffffffffffffffLL;
    if (f <= -9.2233720368547758e18f) return (long long)0x8000000000000000ULL;
    return (long long)f;
}

// ------------------------------------------------------- element-wise ops --
__device__ __forceinline__ float ormi_relu(float a) { return a > 0.0f ? a : 0.0f; }
__device__ __forceinline__ float ormi_step(float a) { return a > 0.0f ? 1.0f : 0.0f; }
__device__ __forceinline__ float ormi_tanh_grad(float y) { return 1.0f - y * y; }
// 1 + e >= 1 (or inf, or NaN), so the reciprocal never sees a denormal.
__device__ __forceinline__ float ormi_sigmoid(float a) { return __builtin_amdgcn_rcpf(1.0f + expf(-a)); }
__device__ __forceinline__ float ormi_sigmoid_grad(float y) { return y * (1.0f - y); }
// GELU, erf form: 0.5 x (1 + erf(x / sqrt 2)).
__device__ __forceinline__ float ormi_gelu(float a) {
    return (0.5f * a) * (1.0f + erff(a * 0.70710678118654752f));
}
// d/dx GELU = Phi(x) + x phi(x).
__device__ __forceinline__ float ormi_gelu_grad(float a) {
    const float cdf = 0.5f * (1.0f + erff(a * 0.70710678118654752f));
    const float pdf = 0.39894228040143268f * expf((-0.5f * a) * a);
    return cdf + a * pdf;
}
__device__ __forceinline__ float ormi_eq(float a, float b) { return a == b ? 1.0f : 0.0f; }

// ------------------------------------------------------- index arithmetic --
// Division by a run-time invariant d for dividends n < 2^31:
//   s = ceil(log2 d), m = floor(2^32 (2^s - d) / d) + 1, q = (mulhi(n, m) + n) >> s.
// The host computes (m, s) once per launch (ormi::hip::make_fastdiv).
__device__ __forceinline__ unsigned ormi_fdiv(unsigned n, unsigned m, unsigned s) {
    return (__umulhi(n, m) + n) >> s;
}

// ------------------------------------------------- wave64 reductions (DPP) --
// DPP controls (GFX9 encoding): quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] = 0x4E,
// row_half_mirror = 0x141, row_mirror = 0x140. After these four steps every
// lane holds its 16-lane row's result; two xor-shuffles across rows finish the
// wave. Each step pairs lanes symmetrically, so every lane ends with the same
// bits and the combination order is fixed (deterministic sums).
template <int CTRL>
__device__ __forceinline__ float ormi_dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int ormi_dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

__device__ __forceinline__ float ormi_wave_sum(float v) {
    v += ormi_dpp_f<0xB1>(v);
    v += ormi_dpp_f<0x4E>(v);
    v += ormi_dpp_f<0x141>(v);
    v += ormi_dpp_f<0x140>(v);
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// Ordering for max/argmax: NaN above every number; equal values (+0 == -0)
// prefer the smaller index. It is a total order on (value, index) pairs, so
// the reduced pair is the first occurrence of the maximum whatever the tree.
__device__ __forceinline__ bool ormi_am_better(float a, int ia, float b, int ib) {
    const bool an = a != a, bn = b != b;
    if (an || bn) return (an && bn) ? (ia < ib) : an;
    if (a != b) return a > b;
    return ia < ib;
}

__device__ __forceinline__ void ormi_am_take(float& v, int& i, float ov, int oi) {
    if (ormi_am_better(ov, oi, v, i)) { v = ov; i = oi; }
}

template <int CTRL>
__device__ __forceinline__ void ormi_am_dpp_step(float& v, int& i) {
    const float ov = ormi_dpp_f<CTRL>(v);
    const int oi = ormi_dpp_i<CTRL>(i);
    ormi_am_take(v, i, ov, oi);
}

__device__ __forceinline__ void ormi_wave_argmax(float& v, int& i) {
    ormi_am_dpp_step<0xB1>(v, i);
    ormi_am_dpp_step<0x4E>(v, i);
    ormi_am_dpp_step<0x141>(v, i);
    ormi_am_dpp_step<0x140>(v, i);
    ormi_am_take(v, i, __shfl_xor(v, 16, 64), __shfl_xor(i, 16, 64));
    ormi_am_take(v, i, __shfl_xor(v, 32, 64), __shfl_xor(i, 32, 64));
}
