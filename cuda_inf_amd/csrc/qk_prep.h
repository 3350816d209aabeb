// qk_prep.h -- the QK producers of the attention branch (engine.cu:148-182,
// called at 799-801): per-head RMSNorm, then rotate-half RoPE, on one
// 64-dim head row held one value per lane of a wave.  Every operation is a
// single IEEE-rounded op in a fixed order, so the result is bit-identical
// to the CPU restatement:
//   ss  = sum of x^2 in the reference's tree order (pairs d, d + s for
//         s = 32..1, lower + upper), broadcast from lane 0
//   inv = 1 / sqrt(ss / 64 + eps)          (IEEE sqrt and division)
//   y   = fp16((x * inv) * w)
//   for d < 32: ang = pos * invf[d], (sn, cs) = sincos_det(ang),
//   y0' = fp16(y0 * cs - y1 * sn), y1' = fp16(y1 * cs + y0 * sn)
// sincos_det replaces the reference's sinf/cosf with a fixed sequence:
// k = rint(x * 2/pi), x - k pi/2 in three fma steps, Taylor polynomials of
// degree 9 and 8 in Horner form with fma, the quadrant from k & 3 (about
// 1e-7 absolute error up to |x| = 2.6e5).
#pragma once

#include "common.h"

namespace cia {

// RoPE inverse frequencies theta^(-2i/64), computed on the host in double
// and rounded to fp32
struct RopeTable {
  float invf[D / 2];
};

__device__ __forceinline__ void sincos_det(float x, float& s, float& c) {
#pragma clang fp contract(off)
  const float kf = __builtin_rintf(x * 0x1.45f306p-1f);
  float r = __builtin_fmaf(-kf, 0x1.921fb6p+0f, x);
  r = __builtin_fmaf(-kf, -0x1.777a5cp-25f, r);
  r = __builtin_fmaf(-kf, -0x1.ee59dap-50f, r);
  const float r2 = r * r;
  float ps = __builtin_fmaf(r2, 0x1.71de3ap-19f, -0x1.a01a02p-13f);
  ps = __builtin_fmaf(r2, ps, 0x1.111112p-7f);
  ps = __builtin_fmaf(r2, ps, -0x1.555556p-3f);
  const float sr = __builtin_fmaf(r * r2, ps, r);
  float pc = __builtin_fmaf(r2, 0x1.a01a02p-16f, -0x1.6c16c2p-10f);
  pc = __builtin_fmaf(r2, pc, 0x1.555556p-5f);
  pc = __builtin_fmaf(r2, pc, -0x1p-1f);
  const float cr = __builtin_fmaf(r2, pc, 1.0f);
  const int q = ((int)kf) & 3;
  const float a = (q & 1) ? cr : sr, b = (q & 1) ? sr : cr;
  s = (q & 2) ? -a : a;
  c = (q == 1 || q == 2) ? -b : b;
}

// an fp32 value the compiler must materialise before it is narrowed, so
// the fp32 rounding and then the fp16 rounding both happen (no fused
// multiply-and-narrow)
__device__ __forceinline__ float fp32_round(float v) {
  asm volatile("" : "+v"(v));
  return v;
}

// The rotation of frequency invf at position pos
__device__ __forceinline__ void rope_sincos_f(float invf, int pos, float& sn, float& cs) {
#pragma clang fp contract(off)
  sincos_det((float)pos * invf, sn, cs);
}

// The rotation of lane d's frequency (d mod 32) at position pos
__device__ __forceinline__ void rope_sincos(int d, int pos, const RopeTable& rt, float& sn,
                                            float& cs) {
  rope_sincos_f(rt.invf[d & 31], pos, sn, cs);
}

// One head row, lane d holding x = row[d] and w = weight[d], (sn, cs) the
// rotation of lane d's frequency: returns the fp16 bits of the normalised,
// rotated value of dim d.  Called by all 64 lanes of a wave together.
__device__ __forceinline__ uint16_t qk_norm_rope_sc(float x, float w, int d, float sn, float cs,
                                                    float eps) {
#pragma clang fp contract(off)
  const float ss = wave_tree_sum(x * x);
  const float inv = 1.0f / __builtin_sqrtf(ss / (float)D + eps);
  const float y = h2f(f2h(fp32_round((x * inv) * w)));
  // dim d ^ 32: the swap hands lanes below 32 their partner in the second
  // register and lanes from 32 in the first
  const f32x2 sw = swap32(y);
  const float other = d < 32 ? sw[1] : sw[0];
  const float r = d < 32 ? y * cs - other * sn : y * cs + other * sn;
  return f2h(fp32_round(r));
}

__device__ __forceinline__ uint16_t qk_norm_rope_lane(float x, float w, int d, int pos,
                                                      float eps, const RopeTable& rt) {
  float sn, cs;
  rope_sincos(d, pos, rt, sn, cs);
  return qk_norm_rope_sc(x, w, d, sn, cs, eps);
}

// What the decode kernels need to run the QK producers on the raw q / fresh
// k themselves; qw == nullptr: q and k arrive prepared.
struct QkPrep {
  const uint16_t* qw;
  const uint16_t* kw;
  float eps;
  RopeTable rt;
};

}  // namespace cia
