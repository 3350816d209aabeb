// common.h -- device helpers shared by the gfx950 kernels of the cuda_inf
// attention path: fp16 / OCP-E4M3 conversions, the deterministic exp, wave64
// reductions, and the status plumbing of the C-ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cuda_inf_attn.h"

namespace cia {

constexpr int NH = CIA_NH;
constexpr int NKV = CIA_NKV;
constexpr int GQA = CIA_GQA;
constexpr int D = CIA_HEAD_DIM;
constexpr int G = CIA_KVGROUP;
constexpr int WAVE = 64;

// ---------------------------------------------------------------- status
// Records the HIP error of the last failing call (per host thread).
void set_hip_error(hipError_t e);
// After a launch: CIA_ERR_HIP if the launch failed.
int launch_status();

#define CIA_REQUIRE(cond, code) \
  do {                          \
    if (!(cond)) return (code); \
  } while (0)

inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// ---------------------------------------------------------------- types
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- fp16
__device__ __forceinline__ float h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
// round-to-nearest-even (the MODE register's default rounding)
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
// a - b, never fused with the multiply that produced a: the result is the
// same whether or not the compiler can see that product (a select it folds
// away would otherwise decide between v_fma and v_mul + v_sub)
__device__ __forceinline__ float sub_rn(float a, float b) {
#pragma clang fp contract(off)
  return a - b;
}

// ---------------------------------------------------------------- E4M3
// gfx950's fp8 conversions use the OCP E4M3 format (bias 7, max 448,
// S.1111.111 = NaN).  Decoding is exact.
template <int kByte>
__device__ __forceinline__ float e4m3_to_f32(uint32_t word) {
  return __builtin_amdgcn_cvt_f32_fp8(word, kByte);
}
// bytes 0,1 (kHi = false) or 2,3 (kHi = true) of `word` -> two fp32
template <bool kHi>
__device__ __forceinline__ f32x2 e4m3x2_to_f32(uint32_t word) {
  return __builtin_amdgcn_cvt_pk_f32_fp8(word, kHi);
}

// Encode with SATFINITE: finite values and infinities beyond +-448 clamp to
// +-448, NaN keeps its sign as S.1111.111; the hardware conversion rounds to
// nearest even.
__device__ __forceinline__ float sat448(float x) {
  return __builtin_fminf(__builtin_fmaxf(x, -448.0f), 448.0f);
}
__device__ __forceinline__ uint32_t nan_code(float x) {
  return ((__builtin_bit_cast(uint32_t, x) >> 24) & 0x80u) | 0x7Fu;
}
// packs e4m3(a) into byte 0 and e4m3(b) into byte 1
__device__ __forceinline__ uint32_t e4m3x2(float a, float b) {
  uint32_t r = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(sat448(a), sat448(b), 0, false) & 0xFFFFu;
  if (__builtin_isnan(a)) r = (r & 0xFF00u) | nan_code(a);
  if (__builtin_isnan(b)) r = (r & 0x00FFu) | (nan_code(b) << 8);
  return r;
}
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
  return e4m3x2(a, b) | (e4m3x2(c, d) << 16);
}

// The quantisation scale of the reference, amax/448 + 1e-12 in fp32 with an
// IEEE division (hipcc's default fp32 division is correctly rounded).
__device__ __forceinline__ float quant_scale(float amax) {
  return amax / 448.0f + 1e-12f;
}
// x / s as the IEEE division rounds it, for a scale s = quant_scale(amax)
// and r = 1 / s (IEEE), with s passed through quant_div_s: q0 = x r, the
// exact remainder e = x - q0 s by fma, one correction q0 + e r (Markstein's
// final step), and x's sign back for x = -0 (the correction gives +0
// there).  Three operations instead of a division's ten, with r computed
// once per scale.  Equal to x / s in every bit for every fp16 x and the
// scale of every finite fp16 amax (2.0e9 pairs), and for every finite x
// when amax is infinite (an inf in the group: s = inf, r = 0, passed as
// s = 0, gives x r = +-0 as x / inf does); an infinite x there gives a NaN
// of its own sign.  All of it is checked on the CPU by
// tests/quant_div_check.c.
__device__ __forceinline__ float quant_div_s(float s) {
  return s == __builtin_inff() ? 0.f : s;
}
__device__ __forceinline__ float quant_div(float x, float s, float r) {
#pragma clang fp contract(off)
  const float q0 = x * r;
  const float e = __builtin_fmaf(-q0, s, x);
  return __builtin_copysignf(__builtin_fmaf(e, r, q0), x);
}

// ---------------------------------------------------------------- exp
// Deterministic exp used for the H2O attention mass: Cody-Waite reduction by
// ln2 (two constants), degree-7 Taylor polynomial in Horner form with
// explicit fma, exact power-of-two scale.  Inputs below -60 give 0.  Every
// operation is a single IEEE-rounded op, so the result is bit-identical on
// any IEEE-754 machine with the same sequence.
__device__ __forceinline__ float exp_det(float x) {
  if (!(x >= -60.0f)) return (x != x) ? x : 0.0f;
  if (x > 88.0f) return __builtin_inff();
  float kf = __builtin_rintf(x * 1.44269502162933349609375f);
  float r = __builtin_fmaf(-kf, 0.693145751953125f, x);
  r = __builtin_fmaf(-kf, 1.428606765330187045e-06f, r);
  float p = 1.98412701138295233249664306640625e-04f;
  p = __builtin_fmaf(p, r, 1.38888892810791730880737304687500e-03f);
  p = __builtin_fmaf(p, r, 8.33333376795053482055664062500000e-03f);
  p = __builtin_fmaf(p, r, 4.16666679084300994873046875000000e-02f);
  p = __builtin_fmaf(p, r, 1.66666671633720397949218750000000e-01f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int k = (int)kf;
  return p * __builtin_bit_cast(float, (uint32_t)(k + 127) << 23);
}

// fast exp for the tolerance-checked softmax (v_exp_f32 is exp2)
__device__ __forceinline__ float fast_exp(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896340736f);
}

// ---------------------------------------------------------------- waves
// Cross-lane steps without the LDS unit: DPP row rotations within each
// 16-lane row, then v_permlane16_swap / v_permlane32_swap across rows.  Each
// swap returns a pair holding, per lane, its own value and that of lane
// l ^ 16 / l ^ 32: the partner is the second element in the lower row of
// each swapped pair of rows (lanes 0-15, 32-47 / lanes 0-31) and the first
// element in the upper one.
template <int kN>
__device__ __forceinline__ float row_ror(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x120 + kN, 0xF, 0xF, false));
}
__device__ __forceinline__ f32x2 swap16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, v),
                                                  __builtin_bit_cast(uint32_t, v), false, false);
  return f32x2{__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
__device__ __forceinline__ f32x2 swap32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, v),
                                                  __builtin_bit_cast(uint32_t, v), false, false);
  return f32x2{__builtin_bit_cast(float, (uint32_t)r[0]), __builtin_bit_cast(float, (uint32_t)r[1])};
}
// max / sum over the lanes {l, l^16, l^32, l^48} (one MFMA column)
__device__ __forceinline__ float col4_max(float v) {
  f32x2 r = swap16(v);
  v = __builtin_fmaxf(r[0], r[1]);
  r = swap32(v);
  return __builtin_fmaxf(r[0], r[1]);
}
__device__ __forceinline__ float col4_sum(float v) {
  f32x2 r = swap16(v);
  v = r[0] + r[1];
  r = swap32(v);
  return r[0] + r[1];
}
// col4_sum of four registers at once: lane l of the result holds register
// (l >> 4)'s sum for column l & 15 (a, b, c, d for lane blocks 0..3).  The
// same additions in the same order as col4_sum, with 3 swaps and 3 adds
// where four col4_sum take 8 of each.
__device__ __forceinline__ float col4_sum4(float a, float b, float c, float d) {
  // permlane16_swap(x, y): x gets rows (x0, y0, x2, y2), y rows (x1, y1, x3, y3)
  const auto ab = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, a), __builtin_bit_cast(uint32_t, b),
                                                   false, false);
  const auto cd = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, c), __builtin_bit_cast(uint32_t, d),
                                                   false, false);
  const float x = __builtin_bit_cast(float, (uint32_t)ab[0]) + __builtin_bit_cast(float, (uint32_t)ab[1]);
  const float y = __builtin_bit_cast(float, (uint32_t)cd[0]) + __builtin_bit_cast(float, (uint32_t)cd[1]);
  // permlane32_swap(x, y): x gets halves (x_lo, y_lo), y (x_hi, y_hi)
  const auto xy = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x), __builtin_bit_cast(uint32_t, y),
                                                   false, false);
  return __builtin_bit_cast(float, (uint32_t)xy[0]) + __builtin_bit_cast(float, (uint32_t)xy[1]);
}
// max over the wave (exact in any order)
__device__ __forceinline__ float wave_max_fast(float v) {
  v = __builtin_fmaxf(v, row_ror<8>(v));
  v = __builtin_fmaxf(v, row_ror<4>(v));
  v = __builtin_fmaxf(v, row_ror<2>(v));
  v = __builtin_fmaxf(v, row_ror<1>(v));
  return col4_max(v);
}
// sum over the wave (every lane gets the same value; the order differs from
// wave_sum's butterfly, so this is not for the deterministic mass)
__device__ __forceinline__ float wave_sum_fast(float v) {
  v += row_ror<8>(v);
  v += row_ror<4>(v);
  v += row_ror<2>(v);
  v += row_ror<1>(v);
  return col4_sum(v);
}

// Sum over the wave in the tree order red[d] += red[d + s], s = 32, 16, ..,
// 1 (the shared-memory reduction of engine.cu:153-154), every add "lower
// lane + upper lane"; lanes d < s hold the tree's values at each level and
// lane 0's total is broadcast.  No LDS traffic.  The same bits as wave_sum:
// IEEE addition is commutative, so after each butterfly level lanes d and
// d ^ off hold equal values, and lane 0's butterfly is this tree.
__device__ __forceinline__ float wave_tree_sum(float v) {
  // (a row rotation by 16 - k hands lane i the value of lane i + k of its
  // 16-lane row for i < 16 - k)
  v = v + swap32(v)[1];    // lane d < 32: v[d] + v[d + 32]
  v = v + swap16(v)[1];    // lane d < 16: + (v[d + 16] + v[d + 48])
  v = v + row_ror<8>(v);   // lane d < 8: + lane d + 8
  v = v + row_ror<12>(v);  // lane d < 4: + lane d + 4
  v = v + row_ror<14>(v);  // lane d < 2: + lane d + 2
  v = v + row_ror<15>(v);  // lane 0: + lane 1
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}

// butterfly max / sum (xor 32, 16, ..., 1): the fixed order of the
// deterministic attention mass (wave_tree_sum gives the same sum without
// LDS permutes)
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, off));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off);
  return v;
}

}  // namespace cia
