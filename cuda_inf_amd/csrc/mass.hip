// mass.hip -- the attn_sum option of attention_fused (engine.cu:291-307) on
// gfx950: the attention mass of every (query, head) added per key of the
// group-64 cache.
//
// The reference adds every (query, head) probability into attn_sum with
// atomicAdd in an undefined order and with an approximate __expf.  Here the
// mass is computed with the fixed rule of the H2O path, which gives
// identical bits on any IEEE-754 machine (the CPU restatement follows the
// same rule):
//   s(t) = fma chain over d = 0..63 of q[d]*k(t)[d] from 0, times scale
//   (keys in blocks b of 64: t = 64b + j)
//   m_b  = max s over the eligible keys of block b;  m = max of the m_b
//   e(t) = exp_det(s(t) - m_b)        (0 for ineligible keys)
//   l_b  = lane j of a wave holds e(64b + j) (0 past the end), the
//          butterfly v = v + v[lane ^ off], off = 32..1, gives l_b
//   c_b  = exp_det(m_b - m), 0 for a block with no eligible key
//   l    = l_b * c_b added in ascending b from 0
//   p(t) = e(t) * (c_b * (1/l))
//   attn_sum[t] += p(t), one add per (query, head), queries then heads
//                  ascending -- one of the orders the reference's atomics
//                  can take.
// Every product, sum and fma above is a single IEEE-rounded operation;
// contraction is off in this file so the compiler adds no fusions.
#pragma clang fp contract(off)

#include "common.h"

namespace cia {

// group-64 cache: keys 0..qpos are visible; FP8 below `committed`
struct Group64Src {
  const uint8_t* kc8;
  const uint16_t* ksc;
  const uint16_t* ktail;
  int committed;
  __device__ int count(int qpos) const { return qpos + 1; }
  __device__ bool ok(int, int) const { return true; }
  __device__ void key(int t, int kvh, float* x) const {
    if (t < committed) {
      const u32x4* p = (const u32x4*)(kc8 + ((size_t)t * NKV + kvh) * D);
      const float s = h2f(ksc[(t / G) * NKV + kvh]);
#pragma unroll
      for (int c = 0; c < 4; c++) {
        const u32x4 b = p[c];
#pragma unroll
        for (int w = 0; w < 4; w++) {
          f32x2 lo = e4m3x2_to_f32<false>(b[w]), hi = e4m3x2_to_f32<true>(b[w]);
          x[16 * c + 4 * w + 0] = lo[0] * s;
          x[16 * c + 4 * w + 1] = lo[1] * s;
          x[16 * c + 4 * w + 2] = hi[0] * s;
          x[16 * c + 4 * w + 3] = hi[1] * s;
        }
      }
    } else {
      const u32x4* p = (const u32x4*)(ktail + ((size_t)(t - committed) * NKV + kvh) * D);
#pragma unroll
      for (int c = 0; c < 8; c++) {
        const u32x4 b = p[c];
#pragma unroll
        for (int w = 0; w < 4; w++) {
          x[8 * c + 2 * w] = h2f((uint16_t)b[w]);
          x[8 * c + 2 * w + 1] = h2f((uint16_t)(b[w] >> 16));
        }
      }
    }
  }
};

__device__ __forceinline__ void load_q(const uint16_t* q, float* x) {
  const u32x4* p = (const u32x4*)q;
#pragma unroll
  for (int c = 0; c < 8; c++) {
    const u32x4 b = p[c];
#pragma unroll
    for (int w = 0; w < 4; w++) {
      x[8 * c + 2 * w] = h2f((uint16_t)b[w]);
      x[8 * c + 2 * w + 1] = h2f((uint16_t)(b[w] >> 16));
    }
  }
}

__device__ __forceinline__ float dot_chain(const float* q, const float* k) {
  float acc = 0.0f;
#pragma unroll
  for (int d = 0; d < D; d++) acc = __builtin_fmaf(q[d], k[d], acc);
  return acc;
}

// Per (query i, kv head): wave w handles query head 4*kvh+w.  Writes
// stats[(i*32+h)*2] = m, [..+1] = 1/l.  block = 256, grid = (S, 8).
template <class Src>
__global__ __launch_bounds__(256) void k_mass_stats(const uint16_t* __restrict__ q, Src src,
                                                    int past, float scale,
                                                    float* __restrict__ stats) {
  const int i = blockIdx.x, kvh = blockIdx.y;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int h = kvh * GQA + w, qpos = past + i;
  float qr[D];
  load_q(q + ((size_t)i * NH + h) * D, qr);
  const int n = src.count(qpos);
  float mx = -__builtin_inff();
  for (int t = lane; t < n; t += 64) {
    if (!src.ok(t, qpos)) continue;
    float kx[D];
    src.key(t, kvh, kx);
    mx = __builtin_fmaxf(mx, dot_chain(qr, kx) * scale);
  }
  mx = wave_max(mx);
  float l = 0.0f;
  for (int t0 = 0; t0 < n; t0 += 64) {
    const int t = t0 + lane;
    const bool ok = t < n && src.ok(t, qpos);
    float sv = -__builtin_inff();
    if (ok) {
      float kx[D];
      src.key(t, kvh, kx);
      sv = dot_chain(qr, kx) * scale;
    }
    const float mb = wave_max_fast(sv);
    const float e = ok ? exp_det(sv - mb) : 0.0f;
    const float cb = mb == -__builtin_inff() ? 0.0f : exp_det(mb - mx);
    l = l + wave_tree_sum(e) * cb;  // the block's butterfly, then the ordered total
  }
  if (lane == 0) {
    stats[((size_t)i * NH + h) * 2] = mx;
    stats[((size_t)i * NH + h) * 2 + 1] = 1.0f / l;
  }
}

// attn_sum[t] += p for every (query, head) in order.  grid = ceil(n/64),
// block = 64: one wave per 64-key block, lane j owns key 64b + j; the wave
// takes the block's maximum m_b itself, so every lane runs every reduction.
template <class Src>
__global__ __launch_bounds__(64) void k_mass_accum(const uint16_t* __restrict__ q, Src src, int S,
                                                   int past, float scale,
                                                   const float* __restrict__ stats,
                                                   float* __restrict__ attn_sum, int nkeys) {
  const int t0 = blockIdx.x * 64, t = t0 + threadIdx.x;
  const bool live = t < nkeys;
  const int tc = live ? t : t0;  // (key t0 < nkeys exists in every block)
  float a = live ? attn_sum[t] : 0.0f;
  for (int i = 0; i < S; i++) {
    const int qpos = past + i;
    if (t0 >= src.count(qpos)) continue;  // uniform: the block has no visible key
    const bool ok = live && t < src.count(qpos) && src.ok(t, qpos);
    for (int kvh = 0; kvh < NKV; kvh++) {
      float kx[D];
      src.key(tc, kvh, kx);
      for (int j = 0; j < GQA; j++) {
        const int h = kvh * GQA + j;
        float qr[D];
        load_q(q + ((size_t)i * NH + h) * D, qr);
        const float m = stats[((size_t)i * NH + h) * 2];
        const float inv = stats[((size_t)i * NH + h) * 2 + 1];
        const float sv = ok ? dot_chain(qr, kx) * scale : -__builtin_inff();
        const float mb = wave_max_fast(sv);
        const float w = exp_det(mb - m) * inv;  // mb is finite: key t0 is visible
        if (ok) a = a + exp_det(sv - mb) * w;
      }
    }
  }
  if (live) attn_sum[t] = a;
}

}  // namespace cia

using namespace cia;

extern "C" int64_t cia_mass_workspace_bytes(int S) {
  return S < 0 ? 0 : (int64_t)S * NH * 2 * (int64_t)sizeof(float);
}

// attn_sum of attention_fused over the group-64 cache (called after the
// output kernel by cia_attention_fused).
extern "C" __attribute__((visibility("hidden"))) int cia_mass_group64(const uint16_t* q, const uint8_t* kc8, const uint16_t* ksc,
                                const uint16_t* ktail, int committed, float* attn_sum, int S,
                                int past, float scale, void* ws, void* stream) {
  CIA_REQUIRE(ws, CIA_ERR_NULL);
  CIA_REQUIRE(aligned(ws, 8), CIA_ERR_ALIGN);
  Group64Src src{kc8, ksc, ktail, committed};
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL((k_mass_stats<Group64Src>), dim3(S, NKV), dim3(256), 0, s, q, src, past,
                     scale, (float*)ws);
  int st = launch_status();
  if (st) return st;
  const int nkeys = past + S;
  hipLaunchKernelGGL((k_mass_accum<Group64Src>), dim3((nkeys + 63) / 64), dim3(64), 0, s, q, src,
                     S, past, scale, (const float*)ws, attn_sum, nkeys);
  return launch_status();
}
