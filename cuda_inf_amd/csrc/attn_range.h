// attn_range.h -- block-level online-softmax attention of one GQA group (the
// 4 query heads of one kv head) over a contiguous key range of the group-64
// FP8 cache.  Shared by the flash-decoding split kernel, the one-launch
// decode and the fused prefill.
//
// Block = 256 threads = 4 waves.  In a wave, lane quad (lane >> 2) owns one
// key per iteration and lane part (lane & 3) owns dims 16*part .. +15, so a
// key row of one kv head (64 bytes FP8 / 128 bytes fp16) is read with one
// 16-byte load per lane and shared by the 4 query heads.  Keys advance by 64
// per iteration (16 per wave).  Each lane keeps the running (m, l, o) of its
// keys; the block merges them at the end.
#pragma once
#include "common.h"

namespace cia {

struct Group64Cache {
  const uint8_t* kc8;
  const uint8_t* vc8;
  const uint16_t* ksc;
  const uint16_t* vsc;
  const uint16_t* ktail;
  const uint16_t* vtail;
  int committed;
};

// 16 dequantised values of key/value row t (kv head kvh), dims d0..d0+15
__device__ __forceinline__ void load_row16(const uint8_t* c8, const uint16_t* sc,
                                           const uint16_t* tail, int committed, int t,
                                           int kvh, int d0, float* x) {
  if (t < committed) {
    const u32x4 b = *(const u32x4*)(c8 + ((size_t)t * NKV + kvh) * D + d0);
    const float s = h2f(sc[(t / G) * NKV + kvh]);
#pragma unroll
    for (int w = 0; w < 4; w++) {
      f32x2 lo = e4m3x2_to_f32<false>(b[w]), hi = e4m3x2_to_f32<true>(b[w]);
      x[4 * w + 0] = lo[0] * s;
      x[4 * w + 1] = lo[1] * s;
      x[4 * w + 2] = hi[0] * s;
      x[4 * w + 3] = hi[1] * s;
    }
  } else {
    const uint16_t* p = tail + ((size_t)(t - committed) * NKV + kvh) * D + d0;
    const u32x4 a = *(const u32x4*)p, b = *(const u32x4*)(p + 8);
#pragma unroll
    for (int w = 0; w < 4; w++) {
      x[2 * w] = h2f((uint16_t)a[w]);
      x[2 * w + 1] = h2f((uint16_t)(a[w] >> 16));
      x[8 + 2 * w] = h2f((uint16_t)b[w]);
      x[8 + 2 * w + 1] = h2f((uint16_t)(b[w] >> 16));
    }
  }
}

// LDS needed by attend_range (floats)
constexpr int kRangeLds = 4 * 4 * D + 4 * 4 + 4 * 4;

// Computes the block-merged state of heads 4*kvh..4*kvh+3 of query row q
// (fp16 [32][64]) over keys [kstart, kend).  On return (after a barrier)
// sM[j], sL[j], sO[j*64+d] hold max, sum and unnormalised output of head j.
// kend <= kstart gives m = -1e30, l = 0, o = 0.
__device__ __forceinline__ void attend_range(const uint16_t* __restrict__ q,
                                             const Group64Cache& c, int kvh, float scale,
                                             int kstart, int kend, float* lds, float* sM,
                                             float* sL, float* sO) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int quad = lane >> 2, d0 = (lane & 3) * 16;
  float qr[4][16];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint16_t* qp = q + (size_t)(kvh * GQA + j) * D + d0;
    const u32x4 a = *(const u32x4*)qp, b = *(const u32x4*)(qp + 8);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      qr[j][2 * i] = h2f((uint16_t)a[i]);
      qr[j][2 * i + 1] = h2f((uint16_t)(a[i] >> 16));
      qr[j][8 + 2 * i] = h2f((uint16_t)b[i]);
      qr[j][8 + 2 * i + 1] = h2f((uint16_t)(b[i] >> 16));
    }
  }
  float m[4], l[4], o[4][16];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    m[j] = -1e30f;
    l[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) o[j][i] = 0.f;
  }
  for (int t = kstart + w * 16 + quad; t < kend; t += 64) {
    float kx[16], vx[16];
    load_row16(c.kc8, c.ksc, c.ktail, c.committed, t, kvh, d0, kx);
    load_row16(c.vc8, c.vsc, c.vtail, c.committed, t, kvh, d0, vx);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 16; i++) acc = __builtin_fmaf(qr[j][i], kx[i], acc);
      acc += __shfl_xor(acc, 1);
      acc += __shfl_xor(acc, 2);
      const float s = acc * scale;
      const float mnew = __builtin_fmaxf(m[j], s);
      const float cc = fast_exp(m[j] - mnew), p = fast_exp(s - mnew);
      l[j] = __builtin_fmaf(l[j], cc, p);
#pragma unroll
      for (int i = 0; i < 16; i++) o[j][i] = __builtin_fmaf(p, vx[i], o[j][i] * cc);
      m[j] = mnew;
    }
  }
  // ---- merge: lanes -> wave -> block
  float* sOw = lds;                  // [4 waves][4 heads][64]
  float* sMw = lds + 4 * 4 * D;      // [4][4]
  float* sLw = sMw + 16;             // [4][4]
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const float wm = wave_max(m[j]);
    if (lane == 0) sMw[w * 4 + j] = wm;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const float bm = __builtin_fmaxf(__builtin_fmaxf(sMw[j], sMw[4 + j]),
                                     __builtin_fmaxf(sMw[8 + j], sMw[12 + j]));
    const float alpha = fast_exp(m[j] - bm);
    float lj = l[j] * alpha;
#pragma unroll
    for (int off = 4; off <= 32; off <<= 1) lj += __shfl_xor(lj, off);
    if (lane == 0) sLw[w * 4 + j] = lj;
#pragma unroll
    for (int i = 0; i < 16; i++) {
      float v = o[j][i] * alpha;
#pragma unroll
      for (int off = 4; off <= 32; off <<= 1) v += __shfl_xor(v, off);
      o[j][i] = v;
    }
    if (quad == 0) {
#pragma unroll
      for (int i = 0; i < 16; i++) sOw[(w * 4 + j) * D + d0 + i] = o[j][i];
    }
    if (tid == 0) sM[j] = bm;
  }
  __syncthreads();
  {
    const int j = tid >> 6, d = tid & 63;
    sO[j * D + d] = sOw[(0 * 4 + j) * D + d] + sOw[(1 * 4 + j) * D + d] +
                    sOw[(2 * 4 + j) * D + d] + sOw[(3 * 4 + j) * D + d];
    if (tid < 4) sL[tid] = sLw[tid] + sLw[4 + tid] + sLw[8 + tid] + sLw[12 + tid];
  }
  __syncthreads();
}

}  // namespace cia
