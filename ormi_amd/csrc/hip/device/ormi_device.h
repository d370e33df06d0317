// Device helpers shared by the kernels compiled into libormi_hip.so and the
// kernels the hipRTC code generator emits (the generator embeds this file's
// text ahead of every generated kernel). Written for gfx950: wave64, DPP
// cross-lane moves, 128-bit global accesses.
//
// Numeric contract with the CPU oracle: generated code is compiled with
// -ffp-contract=off and IEEE division, so the user-visible + - * / agree bit
// for bit; the helpers below are the oracle's fp32 formulas, with the device
// math library for log, sin, cos and erf (a few ulp from the host's). exp,
// tanh and sigmoid, which dominate VALU-bound fused chains, are written here
// from the hardware V_EXP_F32 / V_RCP_F32 in about half the instructions of
// the library versions, within 3 ulp of the exact values (the oracle's glibc
// results are within 1 ulp), so parity holds at rtol 1e-6.
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
// float -> int32 the same way: truncation toward zero, NaN gives 0, values
// outside [-2^31, 2^31 - 1] saturate.
__device__ __forceinline__ int ormi_f32_to_i32(float f) {
    if (f != f) return 0;
    if (f >= 2147483648.0f) return 2147483647;
    if (f <= -2147483648.0f) return (int)0x80000000u;
    return (int)f;
}

// ------------------------------------------------------- element-wise ops --
__device__ __forceinline__ float ormi_relu(float a) { return a > 0.0f ? a : 0.0f; }
__device__ __forceinline__ float ormi_step(float a) { return a > 0.0f ? 1.0f : 0.0f; }
__device__ __forceinline__ float ormi_tanh_grad(float y) { return 1.0f - y * y; }

// tanh in about 15 VALU instructions (the device library's tanhf takes about 27
// and branches), branch-free, within 3 ulp of the exact value:
//   |y| <  0.625: y + y^3 P(y^2), P of degree 4 fitted here by Remez exchange on
//                 the relative error of tanh over [0, 0.625] (fit error 4.4e-9;
//                 tests/test_tanh_fit.py re-derives the fit on the host);
//   |y| >= 0.625: 1 - 2 / (1 + 2^(2|y| log2 e)) with the hardware V_EXP_F32
//                 (2^x) and V_RCP_F32; at |y| >= 0.625 the subtraction loses at
//                 most one bit.
// Infinite |y| gives 1 through exp -> inf, rcp -> 0; NaN takes the second branch
// and stays NaN. The sign is restored last (tanh is odd).
__device__ __forceinline__ float ormi_tanh(float y) {
    const float a = __builtin_fabsf(y);
    const float e = __builtin_amdgcn_exp2f(a * 2.88539004f);
    const float big = __builtin_fmaf(__builtin_amdgcn_rcpf(1.0f + e), -2.0f, 1.0f);
    const float u = a * a;
    float p = -0.00570498733f;
    p = __builtin_fmaf(p, u, 0.0206390880f);
    p = __builtin_fmaf(p, u, -0.0537397154f);
    p = __builtin_fmaf(p, u, 0.133314416f);
    p = __builtin_fmaf(p, u, -0.333332807f);
    const float small = __builtin_fmaf(a * u, p, a);
    return __builtin_copysignf(a < 0.625f ? small : big, y);
}

// sigmoid(x) = 1 / (1 + e^-x) in about 10 VALU instructions, within 3 ulp for
// every finite x. e^-x = 2^hi e^r with hi = fl(-x log2 e) and r = -x - hi ln 2
// (Cody-Waite: two FMAs against ln 2 split into an fp32 head and tail), so the
// rounding of hi costs nothing: s = rcp(1 + 2^hi) is corrected to first order,
// 1 / (1 + 2^hi (1 + r)) = s - s (1 - s) r. 1 + 2^hi >= 1 (or inf, or NaN), so
// the reciprocal never sees a denormal. For x = +-inf, r is NaN and s (1 or 0)
// is already exact; NaN x gives NaN through s.
__device__ __forceinline__ float ormi_sigmoid(float x) {
    const float hi = x * -1.44269502f;
    float r = __builtin_fmaf(-hi, 0.693147182f, -x);
    r = __builtin_fmaf(-hi, -1.90465432e-09f, r);
    const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(hi));
    const float c = __builtin_fmaf(-__builtin_fmaf(-s, s, s), r, s);
    return r == r ? c : s;
}
__device__ __forceinline__ float ormi_sigmoid_grad(float y) { return y * (1.0f - y); }

// e^x in about 7 VALU instructions (the device library's expf takes about 13),
// within 2 ulp for results in the normal range: e^x = 2^hi e^r with
// hi = fl(x log2 e), r = x - hi ln 2 from two FMAs (Cody-Waite, ln 2 split into
// an fp32 head and tail), and e^r = 1 + r to within r^2/2 < 2^-34. When the
// correction is NaN (x = +-inf, where r is NaN, or 2^hi = inf times a negative
// r) the uncorrected 2^hi is already the answer (inf or 0); NaN x stays NaN.
// Results below the normal range (x < -87.3) come from V_EXP_F32 as they are.
__device__ __forceinline__ float ormi_exp(float x) {
    const float hi = x * 1.44269502f;
    float r = __builtin_fmaf(-hi, 0.693147182f, x);
    r = __builtin_fmaf(-hi, -1.90465432e-09f, r);
    const float e = __builtin_amdgcn_exp2f(hi);
    const float c = __builtin_fmaf(e, r, e);
    return c == c ? c : e;
}
// GELU, erf form: 0.5 x (1 + erf(x / sqrt 2)).
__device__ __forceinline__ float ormi_gelu(float a) {
    return (0.5f * a) * (1.0f + erff(a * 0.70710678118654752f));
}
// d/dx GELU = Phi(x) + x phi(x).
__device__ __forceinline__ float ormi_gelu_grad(float a) {
    const float cdf = 0.5f * (1.0f + erff(a * 0.70710678118654752f));
    const float pdf = 0.39894228040143268f * ormi_exp((-0.5f * a) * a);
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
// Written as one boolean expression so it compiles to compares and selects,
// not to divergent branches.
__device__ __forceinline__ bool ormi_am_better(float a, int ia, float b, int ib) {
    const bool an = a != a, bn = b != b, earlier = ia < ib;
    return an ? (!bn | earlier) : (!bn & ((a > b) | ((a == b) & earlier)));
}

__device__ __forceinline__ void ormi_am_take(float& v, int& i, float ov, int oi) {
    const bool t = ormi_am_better(ov, oi, v, i);
    v = t ? ov : v;
    i = t ? oi : i;
}

// One element of a chain whose indices increase (a lane's own elements):
// only a strictly larger value, or the first NaN, replaces the current pair,
// so ties keep the earlier element without comparing indices. !(x <= v) is
// "x > v, or either is NaN"; (v == v) keeps a NaN already held. A chain
// starts at (-inf, 0x7fffffff); one whose elements are all -inf keeps that
// index, and the caller replaces it with the chain's first index after the loop.
__device__ __forceinline__ void ormi_am_step(float& v, int& i, float x, int ix) {
    const bool t = !(x <= v) & (v == v);
    v = t ? x : v;
    i = t ? ix : i;
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
