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
//   l    = for each 64-slot block b ascending: lane j of a wave holds
//          e(64b + j) (0 past the end), the butterfly v = v + v[lane ^ off],
//          off = 32..1, gives the block's total; the totals are added in
//          ascending b from 0
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
//                 over s(t) in place and the block's total of the rule's l;
//                 the first block of every head merges the partials into
//                 the output row.
//   k_h2o_mass    1024 slots per block: l (the block totals in order) and
//                 1/l of every (query, head), then attn_sum[t] += p(t) in
//                 the rule's order.
#pragma clang fp contract(off)

#include <algorithm>

#include "common.h"
#include "h2o_place.h"

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
  float* part_l;   // [Sq][32][nblk]: the block's total of the rule's l
  int n_live, nblk, qpos0, Sq;
  float scale;
  // single-token step that evicted a slot (placement in the scores launch):
  // the slot (read from *placed), whose mass restarts from 0 and whose
  // position becomes posj in the mass launch; null otherwise
  const int32_t* placed;
  int32_t* slotpos_w;
  int posj;
};

// Placement of a single fresh token inside the scores launch (the
// reference's host loop, engine.cu:808-826, for one token).  Every
// workgroup derives the same slot: n0 while the buffer fills, else the
// minimum (mass, slot) key outside the window, else over all slots -- the
// rule of k_h2o_place.  Masses and positions are only read in this launch,
// so every workgroup sees the same values: the evicted slot's mass reset
// and new position are written by the mass launch (the position cannot
// change eligibility within the step: old and new positions are both <=
// the query's).  The workgroup whose 64-slot block holds the slot quantises
// the token for its kv head (engine.cu:317-333), writes the bytes and
// scales, and uses them in place of the slot's old ones; for a filling slot
// it also writes the position.
struct H2oPlace {
  const uint16_t* k;  // the token's K and V [8][64] fp16
  const uint16_t* v;
  uint8_t* kf;
  uint8_t* vf;
  uint16_t* ks;
  uint16_t* vs;
  const float* attn;
  int32_t* slotpos;
  int32_t* dst;  // dst[0] = the slot, -1 when none can be taken
  int n0, C, W, posj;
};

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

// grid = (nblk, 8, Sq), block = 256 (wave w: query head 4 kvh + w).  All
// global loads are issued before the first use, so the kernel waits on
// memory once.  kPlace (Sq = 1): the token is placed here (H2oPlace).
template <bool kPlace>
__global__ __launch_bounds__(256) void k_h2o_scores(H2oArgs a, H2oPlace pl) {
  __shared__ __attribute__((aligned(16))) uint8_t vl[64 * D];  // V rows of the block's slots, this kv head
  __shared__ __attribute__((aligned(16))) uint8_t newkv[2][D];  // kPlace: the token's K / V bytes
  __shared__ uint16_t newsc[2];
  __shared__ uint64_t red[2][4];
  const int blk = blockIdx.x, kvh = blockIdx.y, i = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, h = kvh * GQA + wave_id();
  const int qpos = a.qpos0 + i, t0 = blk * 64, t = t0 + lane;
  const int row = tid >> 2, c4 = tid & 3;
  const bool live = t < a.n_live;
  // ---- placement loads first: the token's row of this kv head, masses
  // and positions (each thread 8 slots of a 2048-slot buffer)
  int slot = -1;
  float tk = 0.f, tv = 0.f;
  uint64_t kwin = ~0ull, kall = ~0ull;
  if constexpr (kPlace) {
    tk = h2f(pl.k[kvh * D + lane]);
    tv = h2f(pl.v[kvh * D + lane]);
    if (pl.n0 >= pl.C) {
      const int lim = pl.posj - pl.W;
      for (int u0 = tid; u0 < pl.C; u0 += 256 * 8) {
        float m[8];
        int sp[8];
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int u = u0 + 256 * e;
          m[e] = u < pl.C ? pl.attn[u] : kPicked;
          sp[e] = u < pl.C ? a.slot_pos[u] : 0;
        }
#pragma unroll
        for (int e = 0; e < 8; e++)
          if (m[e] < kPicked) {
            const uint64_t key = place_key(m[e], u0 + 256 * e);
            kall = min_u64(kall, key);
            if (sp[e] <= lim) kwin = min_u64(kwin, key);
          }
      }
    }
  }
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
  if constexpr (kPlace) {
    // ---- the slot (the same in every workgroup)
    if (pl.n0 < pl.C) {
      slot = pl.n0;
    } else {
      kwin = wave_min_u64(kwin);
      kall = wave_min_u64(kall);
      if (lane == 0) {
        red[0][wave_id()] = kwin;
        red[1][wave_id()] = kall;
      }
      __syncthreads();
#pragma unroll
      for (int w = 0; w < 4; w++) {
        kwin = min_u64(kwin, red[0][w]);
        kall = min_u64(kall, red[1][w]);
      }
      const uint64_t kb = kwin != ~0ull ? kwin : kall;
      slot = kb != ~0ull ? (int)(uint32_t)kb : -1;
    }
    if (blk == 0 && kvh == 0 && tid == 0) pl.dst[0] = slot;
    if (slot >= t0 && slot < t0 + 64) {
      // this block holds the slot: quantise the token's kv head (wave 0),
      // write it, and use it for the slot's key, value and scales
      if (wave_id() == 0) {
        const float sck = quant_scale(wave_max_fast(__builtin_fabsf(tk)));
        const float scv = quant_scale(wave_max_fast(__builtin_fabsf(tv)));
        const uint32_t kb = e4m3x2(tk / sck, 0.f) & 0xFFu, vb = e4m3x2(tv / scv, 0.f) & 0xFFu;
        newkv[0][lane] = (uint8_t)kb;
        newkv[1][lane] = (uint8_t)vb;
        const size_t o = ((size_t)slot * NKV + kvh) * D + lane;
        pl.kf[o] = (uint8_t)kb;
        pl.vf[o] = (uint8_t)vb;
        if (lane == 0) {
          newsc[0] = f2h(sck);
          newsc[1] = f2h(scv);
          pl.ks[slot * NKV + kvh] = newsc[0];
          pl.vs[slot * NKV + kvh] = newsc[1];
          if (kvh == 0 && pl.n0 < pl.C) pl.slotpos[slot] = pl.posj;
        }
      }
      __syncthreads();
      if (t == slot) {
#pragma unroll
        for (int c = 0; c < 4; c++) kr[c] = *(const u32x4*)(newkv[0] + 16 * c);
        ks16 = newsc[0];
        vs16 = newsc[1];
        sp = pl.posj;
      }
      if (t0 + row == slot) vst = *(const u32x4*)(newkv[1] + 16 * c4);
    }
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
  const float e = (live && sp <= qpos) ? exp_det(sv - m) : 0.0f;
  *scp = e;
  const float etot = wave_sum(e);  // the rule's butterfly over this block
  if (lane == 0) a.part_l[ph + blk] = etot;
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
// every (query, head) of the chunk (the same bits) from the block totals,
// then owns 1024 slots.  The first query's numerators of the thread's slot
// are loaded before the totals are summed.
__global__ __launch_bounds__(1024) void k_h2o_mass(H2oArgs a) {
  __shared__ float inv[kChunk * NH];
  const int tid = threadIdx.x;
  const size_t cp = (size_t)a.nblk * 64;
  const int t = blockIdx.x * 1024 + tid;
  const int tc = t < a.n_live ? t : 0;  // (slot 0 exists whenever a block runs)
  float ev0[NH];
#pragma unroll
  for (int h = 0; h < NH; h++) ev0[h] = a.sc[(size_t)h * cp + tc];
  const int npr = a.Sq * NH;
  if (tid < npr) {
    // thread pr: the totals of row pr in ascending block order, 16 loads in
    // flight at a time
    const float* pt = a.part_l + (size_t)tid * a.nblk;
    float l = 0.0f;
    for (int b0 = 0; b0 < a.nblk; b0 += 16) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; u++) v[u] = b0 + u < a.nblk ? pt[b0 + u] : 0.0f;
#pragma unroll
      for (int u = 0; u < 16; u++)
        if (b0 + u < a.nblk) l = l + v[u];
    }
    inv[tid] = 1.0f / l;
  }
  __syncthreads();
  if (t >= a.n_live) return;
  const bool re = a.placed && t == *a.placed;  // the slot evicted by this step
  const int sp = re ? a.posj : a.slot_pos[t];
  float acc = re ? 0.0f : a.attn_sum[t];
  if (sp <= a.qpos0) {
#pragma unroll
    for (int h = 0; h < NH; h++) acc = acc + ev0[h] * inv[h];
  }
  for (int i = 1; i < a.Sq; i++) {
    if (sp > a.qpos0 + i) continue;
    float ev[NH];
#pragma unroll
    for (int h = 0; h < NH; h++) ev[h] = a.sc[(size_t)(i * NH + h) * cp + t];
#pragma unroll
    for (int h = 0; h < NH; h++) acc = acc + ev[h] * inv[i * NH + h];
  }
  a.attn_sum[t] = acc;
  if (re) a.slotpos_w[t] = a.posj;
}

int64_t h2o_ws_bytes(int S, int C) {
  const int64_t sq = std::min(S, kChunk), nblk = (C + 63) / 64;
  return sq * NH * (2 * nblk * 64 + 3 * nblk) * (int64_t)sizeof(float);
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
    a.part_l = a.part_ml + (size_t)sq * NH * nblk * 2;
    a.n_live = n_live;
    a.nblk = nblk;
    a.qpos0 = past + c0;
    a.Sq = sq;
    a.scale = scale;
    a.placed = nullptr;
    a.slotpos_w = nullptr;
    a.posj = 0;
    hipLaunchKernelGGL(k_h2o_scores<false>, dim3(nblk, NKV, sq), dim3(256), 0, s, a, H2oPlace{});
    int st = launch_status();
    if (st) return st;
    hipLaunchKernelGGL(k_h2o_exp, dim3(nblk, NKV, sq), dim3(256), 0, s, a);
    if ((st = launch_status())) return st;
    hipLaunchKernelGGL(k_h2o_mass, dim3((n_live + 1023) / 1024), dim3(1024), 0, s, a);
    if ((st = launch_status())) return st;
  }
  return CIA_OK;
}

// One decode step of an H2O layer in three launches: the token placed and
// quantised inside the scores launch (H2oPlace), then exp and mass.  The
// same slots, positions, bytes and masses as cia_h2o_place followed by
// cia_attention_h2o for S = 1.  mid_event (may be NULL) is recorded after
// the scores launch.
extern "C" __attribute__((visibility("hidden"))) int cia_h2o_decode_step(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, uint8_t* kf, uint8_t* vf,
    uint16_t* ks, uint16_t* vs, float* attn_sum, int32_t* slot_pos, int32_t* dst_slots,
    int* n_live, int C, int W, int past, uint16_t* out, float scale, void* ws, int64_t ws_bytes,
    void* stream, void* mid_event) {
  CIA_REQUIRE(n_live, CIA_ERR_NULL);
  CIA_REQUIRE(past >= 0 && C >= 1 && W >= 0 && *n_live >= 0 && *n_live <= C, CIA_ERR_ARG);
  CIA_REQUIRE(q && k && v && kf && vf && ks && vs && attn_sum && slot_pos && dst_slots && out && ws,
              CIA_ERR_NULL);
  const int n0 = *n_live, n1 = n0 < C ? n0 + 1 : C;
  CIA_REQUIRE(ws_bytes >= h2o_ws_bytes(1, n1), CIA_ERR_ARG);
  CIA_REQUIRE(aligned(q, 16) && aligned(kf, 16) && aligned(vf, 16) && aligned(ws, 16) &&
                  aligned(ks, 2) && aligned(vs, 2) && aligned(out, 2) && aligned(attn_sum, 4) &&
                  aligned(slot_pos, 4) && aligned(dst_slots, 4) && aligned(k, 2) && aligned(v, 2),
              CIA_ERR_ALIGN);
  hipStream_t s = (hipStream_t)stream;
  const int nblk = (n1 + 63) / 64;
  H2oArgs a;
  a.q = q;
  a.kf = kf;
  a.vf = vf;
  a.ks = ks;
  a.vs = vs;
  a.slot_pos = slot_pos;
  a.out = out;
  a.attn_sum = attn_sum;
  a.sc = (float*)ws;
  a.part_o = a.sc + (size_t)NH * nblk * 64;
  a.part_ml = a.part_o + (size_t)NH * nblk * 64;
  a.part_l = a.part_ml + (size_t)NH * nblk * 2;
  a.n_live = n1;
  a.nblk = nblk;
  a.qpos0 = past;
  a.Sq = 1;
  a.scale = scale;
  a.placed = nullptr;
  a.slotpos_w = nullptr;
  a.posj = past;
  const H2oPlace pl{k, v, kf, vf, ks, vs, attn_sum, slot_pos, dst_slots, n0, C, W, past};
  hipLaunchKernelGGL(k_h2o_scores<true>, dim3(nblk, NKV, 1), dim3(256), 0, s, a, pl);
  int st = launch_status();
  if (st) return st;
  if (mid_event) {
    const hipError_t e = hipEventRecord((hipEvent_t)mid_event, s);
    if (e != hipSuccess) {
      set_hip_error(e);
      return CIA_ERR_HIP;
    }
  }
  hipLaunchKernelGGL(k_h2o_exp, dim3(nblk, NKV, 1), dim3(256), 0, s, a);
  if ((st = launch_status())) return st;
  if (n0 >= C) {
    a.placed = dst_slots;
    a.slotpos_w = slot_pos;
  }
  hipLaunchKernelGGL(k_h2o_mass, dim3((n1 + 1023) / 1024), dim3(1024), 0, s, a);
  if ((st = launch_status())) return st;
  *n_live = n1;
  return CIA_OK;
}
