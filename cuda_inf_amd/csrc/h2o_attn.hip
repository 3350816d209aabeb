// h2o_attn.hip -- attention_h2o (engine.cu:337-384) on gfx950: attention of
// S queries over the H2O slot buffer (per-slot FP8 K/V, one fp16 scale per
// slot and kv head, causal mask via slot_pos) and the attention mass added
// to attn_sum.
//
// The reference runs one thread per (query, head) over every slot and adds
// the mass with atomicAdd, in an undefined order and with __expf.  Here the
// mass follows a fixed rule that gives identical bits on any IEEE-754
// machine (the CPU restatement follows the same rule):
//   s(t) = fma chain over d = 0..63 of q[d]*k(t)[d] from 0, times scale,
//          with k(t)[d] = e4m3(byte d) * fp32(scale of slot t)
//   m    = max s over eligible slots (slot_pos[t] <= qpos, t < n_live)
//   e(t) = exp_det(s(t) - m), 0 for ineligible slots
//   l    = lane j of a wave sums e(j), e(j+64), ... in order, then the
//          butterfly v = v + v[lane ^ off], off = 32..1
//   p(t) = e(t) * (1/l)
//   attn_sum[t] += p(t), one add per (query, head), queries then heads
//                  ascending -- one of the orders the reference's atomics
//                  can take.
// Every product, sum and fma above is a single IEEE-rounded operation;
// contraction is off in this file so the compiler adds no fusions.
//
// Three launches per chunk of up to kChunk queries, each spread over the
// whole chip (the reference's one block of 32 threads per query scans the
// buffer serially):
//   k_h2o_scores  (64-slot block, kv head, query): one wave per query head
//                 of the GQA group, lane = slot.  s(t) into scratch, and the
//                 block's partial softmax (max, sum, V-weighted sum) for
//                 the output, with fast exp -- the output is held to a
//                 tolerance, not to bits.
//   k_h2o_exp     same grid: m from the partial maxima (an exact max), e(t)
//                 over s(t) in place; the first block of every head merges
//                 the partials into the output row.
//   k_h2o_mass    1024 slots per block: l and 1/l of every (query, head),
//                 then attn_sum[t] += p(t) in the rule's order.
#pragma clang fp contract(off)

#include <algorithm>

#include "common.h"

namespace cia {

constexpr int kChunk = 16;  // queries per pass (bounds the scratch)
constexpr float kNegInf = -__builtin_inff();

struct H2oArgs {
  const uint16_t* q;  // first query row of the chunk, [Sq][32][64]
  const uint8_t* kf;
  const uint8_t* vf;
  const uint16_t* ks;
  const uint16_t* vs;
  const int32_t* slot_pos;
  uint16_t* out;  // first output row of the chunk
  float* attn_sum;
  float* sc;       // [Sq][32][nblk * 64]: s(t), then e(t)
  float* part_o;   // [Sq][32][nblk][64]
  float* part_ml;  // [Sq][32][nblk][2]: block max, block sum
  int n_live, nblk, qpos0, Sq;
  float scale;
};

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// grid = (nblk, 8, Sq), block = 256 (wave w: query head 4 kvh + w).  All
// global loads are issued before the first use, so the kernel waits on
// memory once.
__global__ __launch_bounds__(256) void k_h2o_scores(H2oArgs a) {
  __shared__ uint8_t vl[64 * D];  // V rows of the block's slots, this kv head
  const int blk = blockIdx.x, kvh = blockIdx.y, i = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, h = kvh * GQA + wave_id();
  const int qpos = a.qpos0 + i, t0 = blk * 64, t = t0 + lane;
  const int row = tid >> 2, c4 = tid & 3;
  const bool live = t < a.n_live;
  const u32x4* qp = (const u32x4*)(a.q + ((size_t)i * NH + h) * D);
  u32x4 qv[8];
#pragma unroll
  for (int c = 0; c < 8; c++) qv[c] = qp[c];
  u32x4 vst = {0u, 0u, 0u, 0u};
  if (t0 + row < a.n_live)
    vst = *(const u32x4*)(a.vf + ((size_t)(t0 + row) * NKV + kvh) * D + c4 * 16);
  int sp = 0x7FFFFFFF;
  uint16_t ks16 = 0, vs16 = 0;
  u32x4 kr[4] = {};
  if (live) {
    sp = a.slot_pos[t];
    ks16 = a.ks[t * NKV + kvh];
    vs16 = a.vs[t * NKV + kvh];
    const u32x4* kp = (const u32x4*)(a.kf + ((size_t)t * NKV + kvh) * D);
#pragma unroll
    for (int c = 0; c < 4; c++) kr[c] = kp[c];
  }
  *(u32x4*)(vl + row * D + c4 * 16) = vst;
  const bool ok = live && sp <= qpos;
  float s = kNegInf;
  if (ok) {
    const float ksc = h2f(ks16);
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const f32x2 lo = e4m3x2_to_f32<false>(kr[c][w]), hi = e4m3x2_to_f32<true>(kr[c][w]);
        const uint32_t q01 = qv[2 * c + w / 2][2 * (w % 2)];
        const uint32_t q23 = qv[2 * c + w / 2][2 * (w % 2) + 1];
        acc = __builtin_fmaf(h2f((uint16_t)q01), lo[0] * ksc, acc);
        acc = __builtin_fmaf(h2f((uint16_t)(q01 >> 16)), lo[1] * ksc, acc);
        acc = __builtin_fmaf(h2f((uint16_t)q23), hi[0] * ksc, acc);
        acc = __builtin_fmaf(h2f((uint16_t)(q23 >> 16)), hi[1] * ksc, acc);
      }
    }
    s = acc * a.scale;
  }
  a.sc[((size_t)i * NH + h) * (a.nblk * 64) + t] = s;
  // the block's partial softmax for the output
  const float mb = wave_max_fast(s);
  const float e = ok ? fast_exp(s - mb) : 0.0f;
  const float lb = wave_sum_fast(e);
  const float wgt = ok ? e * h2f(vs16) : 0.0f;
  __syncthreads();  // V rows staged
  float o = 0.0f;
#pragma unroll 16
  for (int j = 0; j < 64; j++) {
    const float wj = __builtin_bit_cast(
        float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wgt), j));
    o = __builtin_fmaf(wj, e4m3_to_f32<0>(vl[j * D + lane]), o);
  }
  const size_t pi = ((size_t)i * NH + h) * a.nblk + blk;
  a.part_o[pi * D + lane] = o;
  if (lane == 0) {
    a.part_ml[pi * 2] = mb;
    a.part_ml[pi * 2 + 1] = lb;
  }
}

// grid = (nblk, 8, Sq), block = 256
__global__ __launch_bounds__(256) void k_h2o_exp(H2oArgs a) {
  const int blk = blockIdx.x, kvh = blockIdx.y, i = blockIdx.z;
  const int lane = threadIdx.x & 63, h = kvh * GQA + wave_id();
  const int qpos = a.qpos0 + i, t = blk * 64 + lane;
  const size_t ph = ((size_t)i * NH + h) * a.nblk;
  const bool live = t < a.n_live;
  const int sp = live ? a.slot_pos[t] : 0x7FFFFFFF;
  float* scp = a.sc + ((size_t)i * NH + h) * (a.nblk * 64) + t;
  const float sv = *scp;
  float m = kNegInf;
  for (int b = lane; b < a.nblk; b += 64) m = __builtin_fmaxf(m, a.part_ml[(ph + b) * 2]);
  m = wave_max_fast(m);  // the exact maximum of s over eligible slots
  *scp = (live && sp <= qpos) ? exp_det(sv - m) : 0.0f;
  if (blk != 0) return;
  // output row of head h: merge the blocks' partial softmaxes.  Lane b
  // weighs block b; lane d then sums the weighted partial rows.
  float L = 0.0f, O = 0.0f;
  for (int b0 = 0; b0 < a.nblk; b0 += 64) {
    const int nb = min(64, a.nblk - b0);
    float cb = 0.0f, lb = 0.0f;
    if (lane < nb) {
      const float mb = a.part_ml[(ph + b0 + lane) * 2];
      lb = a.part_ml[(ph + b0 + lane) * 2 + 1];
      cb = mb > kNegInf ? fast_exp(mb - m) : 0.0f;
    }
    L += wave_sum_fast(cb * lb);
    const float* po = a.part_o + (ph + b0) * D + lane;
    for (int j = 0; j < nb; j += 16) {
      float ov[16];
#pragma unroll
      for (int u = 0; u < 16; u++) ov[u] = j + u < nb ? po[(j + u) * D] : 0.0f;
#pragma unroll
      for (int u = 0; u < 16; u++) {
        const float cj = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cb), j + u));
        O = __builtin_fmaf(cj, ov[u], O);
      }
    }
  }
  a.out[((size_t)i * NH + h) * D + lane] = f2h(O / L);
}

// grid = ceil(n_live / 1024), block = 1024: every block derives 1/l of
// every (query, head) of the chunk (the same bits), then owns 1024 slots.
// Loads are batched ahead of the in-order sums.
__global__ __launch_bounds__(1024) void k_h2o_mass(H2oArgs a) {
  __shared__ float inv[kChunk * NH];
  const int tid = threadIdx.x, lane = tid & 63, w = wave_id();
  const size_t cp = (size_t)a.nblk * 64;
  for (int pr = w; pr < a.Sq * NH; pr += 16) {
    const float* e = a.sc + pr * cp;
    float acc = 0.0f;
    int t = lane;
    for (; t + 64 * 15 < a.n_live; t += 64 * 16) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; u++) v[u] = e[t + 64 * u];
#pragma unroll
      for (int u = 0; u < 16; u++) acc = acc + v[u];
    }
    for (; t < a.n_live; t += 64) acc = acc + e[t];
    const float l = wave_sum(acc);  // the butterfly of the rule
    if (lane == 0) inv[pr] = 1.0f / l;
  }
  __syncthreads();
  const int t = blockIdx.x * 1024 + tid;
  if (t >= a.n_live) return;
  const int sp = a.slot_pos[t];
  float acc = a.attn_sum[t];
  for (int i = 0; i < a.Sq; i++) {
    if (sp > a.qpos0 + i) continue;
    float ev[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) ev[h] = a.sc[(size_t)(i * NH + h) * cp + t];
#pragma unroll
    for (int h = 0; h < NH; h++) acc = acc + ev[h] * inv[i * NH + h];
  }
  a.attn_sum[t] = acc;
}

int64_t h2o_ws_bytes(int S, int C) {
  const int64_t sq = std::min(S, kChunk), nblk = (C + 63) / 64;
  return sq * NH * (2 * nblk * 64 + 2 * nblk) * (int64_t)sizeof(float);
}

}  // namespace cia

using namespace cia;

extern "C" int64_t cia_h2o_workspace_bytes(int S, int C) {
  return (S < 0 || C < 0) ? 0 : h2o_ws_bytes(S, C);
}

extern "C" int cia_attention_h2o(const uint16_t* q, const uint8_t* kf, const uint8_t* vf,
                                 const uint16_t* ks, const uint16_t* vs,
                                 const int32_t* slot_pos, int n_live, uint16_t* out,
                                 float* attn_sum, int S, int past, float scale, void* ws,
                                 int64_t ws_bytes, void* stream) {
  CIA_REQUIRE(S >= 0 && past >= 0 && n_live >= 0, CIA_ERR_ARG);
  if (S == 0) return CIA_OK;
  CIA_REQUIRE(q && kf && vf && ks && vs && slot_pos && out && attn_sum && ws, CIA_ERR_NULL);
  CIA_REQUIRE(n_live >= 1 && ws_bytes >= h2o_ws_bytes(S, n_live), CIA_ERR_ARG);
  CIA_REQUIRE(aligned(q, 16) && aligned(kf, 16) && aligned(vf, 16) && aligned(ws, 16) &&
                  aligned(ks, 2) && aligned(vs, 2) && aligned(out, 2) && aligned(attn_sum, 4) &&
                  aligned(slot_pos, 4),
              CIA_ERR_ALIGN);
  hipStream_t s = (hipStream_t)stream;
  const int nblk = (n_live + 63) / 64;
  for (int c0 = 0; c0 < S; c0 += kChunk) {
    const int sq = std::min(kChunk, S - c0);
    H2oArgs a;
    a.q = q + (size_t)c0 * NH * D;
    a.kf = kf;
    a.vf = vf;
    a.ks = ks;
    a.vs = vs;
    a.slot_pos = slot_pos;
    a.out = out + (size_t)c0 * NH * D;
    a.attn_sum = attn_sum;
    a.sc = (float*)ws;
    a.part_o = a.sc + (size_t)sq * NH * nblk * 64;
    a.part_ml = a.part_o + (size_t)sq * NH * nblk * 64;
    a.n_live = n_live;
    a.nblk = nblk;
    a.qpos0 = past + c0;
    a.Sq = sq;
    a.scale = scale;
    hipLaunchKernelGGL(k_h2o_scores, dim3(nblk, NKV, sq), dim3(256), 0, s, a);
    int st = launch_status();
    if (st) return st;
    hipLaunchKernelGGL(k_h2o_exp, dim3(nblk, NKV, sq), dim3(256), 0, s, a);
    if ((st = launch_status())) return st;
    hipLaunchKernelGGL(k_h2o_mass, dim3((n_live + 1023) / 1024), dim3(1024), 0, s, a);
    if ((st = launch_status())) return st;
  }
  return CIA_OK;
}
