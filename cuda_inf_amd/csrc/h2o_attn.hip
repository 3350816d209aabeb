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
//   (slots in blocks b of 64: t = 64b + j)
//   m_b  = max s over the eligible slots of block b (slot_pos[t] <= qpos,
//          t < n_live), -inf if none;  m = max of the m_b
//   e(t) = exp_det(s(t) - m_b), 0 for ineligible slots
//   l_b  = lane j of a wave holds e(64b + j) (0 past the end), the
//          butterfly v = v + v[lane ^ off], off = 32..1, gives l_b
//   c_b  = exp_det(m_b - m), 0 for a block with no eligible slot
//   l    = l_b * c_b added in ascending b from 0;  w_b = c_b * (1/l)
//   p(t) = e(t) * w_b
//   attn_sum[t] += p(t), one add per (query, head), queries then heads
//                  ascending -- one of the orders the reference's atomics
//                  can take.
// Every product, sum and fma above is a single IEEE-rounded operation;
// contraction is off in this file so the compiler adds no fusions.
//
// Two launches per chunk of up to kChunk queries, each spread over the
// whole chip (the reference's one block of 32 threads per query scans the
// buffer serially):
//   k_h2o_scores  (64-slot block, kv head, query): one wave per query head
//                 of the GQA group, lane = slot.  s(t), the block's maximum,
//                 e(t) into scratch and the block's l_b; and the block's
//                 partial softmax (max, sum, V-weighted sum) for the output,
//                 with fast exp -- the output is held to a tolerance, not to
//                 bits.
//   k_h2o_mass    256-slot groups: m, l and the weights w_b of every
//                 (query, head), attn_sum[t] += p(t) in the rule's order;
//                 and, in workgroups of their own, the output rows merged
//                 from the blocks' partials.
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
  float* sc;       // [Sq][32][nblk * 64]: e(t) = exp_det(s(t) - m_b)
  float* part_o;   // [Sq][32][nblk][64]
  float* part_ml;  // [Sq][32][nblk][2]: block max, block sum
  float* part_l;   // [Sq][32][nblk]: l_b, the block's butterfly total of e
  int n_live, nblk, qpos0, Sq;
  float scale;
  // single-token step that evicted a slot (placement in the scores launch):
  // the slot (read from *placed), whose mass restarts from 0 and whose
  // position becomes posj in the mass launch; null otherwise
  const int32_t* placed;
  int32_t* slotpos_w;
  int posj;
  // single-token step: the placement keys of the next step, per slot-owning
  // wave (min (mass, slot) key among its slots with position <= klim, and
  // among all), for a next step at posj + 1 (klim = posj + 1 - W); null: none
  uint64_t* keys;
  int klim;
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
  // the previous step's mass launch's keys of this step's buffer (nkw
  // pairs), or null: then every workgroup reads all masses and positions.
  // The keys are used only when the tag the mass launch stored beside them
  // (keys[kKeyTag], keys[kKeyTag + 1]) equals (tag0, tag1): this buffer's
  // attn_sum address and posj; else (a workspace shared with another layer,
  // or a step in between) every slot is read.
  const uint64_t* keys;
  int nkw;
  uint64_t tag0, tag1;
};
// index of the tag in the keys region, after the keys of up to 256 slot
// workgroups x 4 waves (kMassMaxWg)
constexpr int kKeyTag = 256 * 4 * 2;

__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
}

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2_t;

// piece swizzle of V row r in LDS (4 pieces of 16 bytes per 64-byte row): a
// read of rows 8k + j (k = 0..3, j = 0..7) is served 32 lanes (512 bytes of
// banks) or 16 lanes at a time; bit 0 = bit 2 ^ bit 4 of r and bit 1 = bit
// 3 make the rows that share banks in either grouping take distinct pieces
__device__ __forceinline__ int vsw(int r) { return (((r >> 2) ^ (r >> 4)) & 1) | ((r >> 2) & 2); }

// ds_read_b64_tr_b8: within each 16-lane block, lane i receives byte i mod 8
// of the 8-byte rows addressed by lanes 2j + (i div 8), j = 0..7
__device__ __forceinline__ u32x2 lds_read_tr8(const uint8_t* p) {
  const i32x2 v = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2_t*)p);
  return u32x2{(uint32_t)v[0], (uint32_t)v[1]};
}

// 8 E4M3 bytes -> fp16, exactly (scale 1)
__device__ __forceinline__ f16x8 e4m3x8_to_f16(uint32_t w0, uint32_t w1) {
  const f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false);
  const f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true);
  const f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false);
  const f16x2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true);
  return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// grid = (nblk, 8, Sq), block = 256 (wave w: query head 4 kvh + w).  All
// global loads are issued before the first use, so the kernel waits on
// memory once.  kPlace (Sq = 1): the token is placed here (H2oPlace).
template <bool kPlace>
__global__ __launch_bounds__(256) void k_h2o_scores(H2oArgs a, H2oPlace pl) {
  // V rows of the block's slots, this kv head: row r's 16-byte piece c at
  // c ^ vsw(r), so the transposing reads of 32 rows (one piece each) hit
  // distinct banks
  __shared__ __attribute__((aligned(16))) uint8_t vl[64 * D];
  __shared__ __attribute__((aligned(16))) _Float16 wl[GQA][64];  // each head's numerators (fp16)
  __shared__ __attribute__((aligned(16))) _Float16 vsl[64];      // the slots' V scales
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
    const bool use_keys = pl.n0 >= pl.C && pl.keys && pl.keys[kKeyTag] == pl.tag0 &&
                          pl.keys[kKeyTag + 1] == pl.tag1;
    if (use_keys) {
      for (int x = tid; x < pl.nkw; x += 256) {
        kwin = min_u64(kwin, pl.keys[2 * x]);
        kall = min_u64(kall, pl.keys[2 * x + 1]);
      }
    } else if (pl.n0 >= pl.C) {
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
        const uint32_t kb = e4m3x2(quant_div(tk, quant_div_s(sck), 1.0f / sck), 0.f) & 0xFFu;
        const uint32_t vb = e4m3x2(quant_div(tv, quant_div_s(scv), 1.0f / scv), 0.f) & 0xFFu;
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
  *(u32x4*)(vl + row * D + 16 * (c4 ^ vsw(row))) = vst;
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
  // the block's maximum m_b; the rule's numerators and l_b
  const float mb = wave_max_fast(s);
  const float ed = ok ? exp_det(s - mb) : 0.0f;
  a.sc[((size_t)i * NH + h) * (a.nblk * 64) + t] = ed;
  const float lbd = wave_tree_sum(ed);  // the rule's butterfly total
  // the block's partial softmax for the output: numerators e in fp16 (the
  // sum taken over the same fp16 values), o = sum_t e(t) (V(t) * scale(t))
  // on the matrix cores with each V row times its slot's scale in fp16
  const _Float16 e16 = (_Float16)(ok ? fast_exp(s - mb) : 0.0f);
  const float lb = wave_sum_fast((float)e16);
  wl[wave_id()][lane] = e16;
  if (wave_id() == 0) vsl[lane] = __builtin_bit_cast(_Float16, vs16);
  __syncthreads();  // V rows, numerators and scales in LDS
  // O (16 rows, all the same) = W (64 numerators in every row) x V' (64
  // slots x 64 dims): A lane (r, kg) holds slots 32 s + 8 kg .. +7, B lane
  // (n, kg) the same slots of dim 16 dt + n (a transposing read), so lane l
  // ends with dim l in element 0 of product dt = l / 16
  const int kg = lane >> 4, ln = lane & 15;
  f32x4 acc[4];
#pragma unroll
  for (int dt = 0; dt < 4; dt++) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 2; ks++) {
    const int sl0 = 32 * ks + 8 * kg;
    const f16x8 wa = *(const f16x8*)&wl[wave_id()][sl0];
    const f16x8 sc8 = *(const f16x8*)&vsl[sl0];
#pragma unroll
    for (int dt = 0; dt < 4; dt++) {
      const int vr = sl0 + (ln >> 1);
      const u32x2 raw = lds_read_tr8(vl + vr * D + 16 * (dt ^ vsw(vr)) + 8 * (ln & 1));
      const f16x8 vb = e4m3x8_to_f16(raw[0], raw[1]) * sc8;
      acc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, vb, acc[dt], 0, 0, 0);
    }
  }
  const float o = kg == 0 ? acc[0][0] : (kg == 1 ? acc[1][0] : (kg == 2 ? acc[2][0] : acc[3][0]));
  const size_t pi = ((size_t)i * NH + h) * a.nblk + blk;
  a.part_o[pi * D + lane] = o;
  if (lane == 0) {
    a.part_ml[pi * 2] = mb;
    a.part_ml[pi * 2 + 1] = lb;
    a.part_l[pi] = lbd;
  }
}

constexpr int kMassBlk = 4;         // 64-slot blocks per slot group (256 slots)
constexpr int kMassMaxWg = 256;     // slot workgroups at most
constexpr int kMassWaves = 16;      // waves per mass workgroup
constexpr int kPwStride = 68;       // floats per row of a wave's block products

// One output row of the chunk: the 64-slot blocks' partial softmaxes merged
// (lane b weighs block b, lane d then sums dim d); 32 blocks' loads at a time.
__device__ __forceinline__ void h2o_out_row(const H2oArgs& a, int pr, int lane) {
  const size_t ph = (size_t)pr * a.nblk;
  float m = kNegInf, L = 0.0f, O = 0.0f;
  for (int c0 = 0; c0 < a.nblk; c0 += 32) {
    const int nb = min(32, a.nblk - c0);
    const bool in = lane < nb;
    const float mb = in ? a.part_ml[(ph + c0 + lane) * 2] : kNegInf;
    const float lb = in ? a.part_ml[(ph + c0 + lane) * 2 + 1] : 0.0f;
    const float* po = a.part_o + (ph + c0) * D + lane;
    float ov[32];
#pragma unroll
    for (int u = 0; u < 32; u++) ov[u] = u < nb ? po[u * D] : 0.0f;
    const float mn = __builtin_fmaxf(m, wave_max_fast(mb));
    if (mn == kNegInf) continue;
    const float r = m == kNegInf ? 0.0f : fast_exp(m - mn);
    const float cb = mb > kNegInf ? fast_exp(mb - mn) : 0.0f;
    L = L * r + wave_sum_fast(cb * lb);
    O = O * r;
#pragma unroll
    for (int u = 0; u < 32; u++) {
      const float cj = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, cb), u));
      O = __builtin_fmaf(cj, ov[u], O);
    }
    m = mn;
  }
  a.out[(size_t)pr * D + lane] = f2h(O / L);
}

// grid = nsw + ceil(Sq * 32 / 16), block = 1024.  Workgroups below nsw are
// slot workgroups: their 16 waves take m and 1/l of every (query, head) row
// of the chunk, kRowPass rows per wave at a time (lane = block: the maxima
// and c_b wave-parallel; then one lane per row adds the row's l_b c_b in
// block order from LDS).  The first 256 threads then own the 256-slot
// groups g = blockIdx, blockIdx + nsw, ..: the weights w_b of the group's 4
// blocks, then attn_sum[t] += e(t) w_b in (query, head) order.  The other
// workgroups merge the output rows, one per wave, alongside.
template <int kRowPass>
__global__ __launch_bounds__(1024) void k_h2o_mass(H2oArgs a, int nsw) {
  __shared__ float wsh[kChunk * NH * kMassBlk];  // w_b of the group's blocks
  __shared__ float mi[kChunk * NH][2];           // m, 1/l per row
  __shared__ __attribute__((aligned(16))) float pw[kMassWaves][kRowPass * kPwStride];
  const int tid = threadIdx.x, lane = tid & 63, wv = wave_id();
  const int npr = a.Sq * NH;
  if ((int)blockIdx.x >= nsw) {
    const int pr = ((int)blockIdx.x - nsw) * kMassWaves + wv;
    if (pr < npr) h2o_out_row(a, pr, lane);
    return;
  }
  const size_t cp = (size_t)a.nblk * 64;
  const int ng = (a.n_live + 255) / 256;
  const int placed = a.placed ? *a.placed : -1;  // the slot evicted by this step
  int g = blockIdx.x;
  int b0 = g * kMassBlk;
  // a group's loads that do not wait for the weights: the numerators of the
  // first query, the slot's position and mass (threads below 256)
  float ev0[NH] = {}, acc = 0.0f;
  int sp = 0;
  auto fetch = [&](int gg) {
    if (wv >= 4) return;
    const int t = gg * 256 + tid;
    const int tc = t < a.n_live ? t : 0;
#pragma unroll
    for (int h = 0; h < NH; h++) ev0[h] = a.sc[(size_t)h * cp + tc];
    sp = a.slot_pos[tc];
    acc = a.attn_sum[tc];
  };
  fetch(g);
  // ---- m and 1/l of every row (lane = block); the first group's w_b
  if (a.nblk <= 64) {
    const bool in = lane < a.nblk;
    for (int r0 = wv; r0 < npr; r0 += kMassWaves * kRowPass) {
      float mbv[kRowPass], lt[kRowPass], cb[kRowPass], m[kRowPass];
#pragma unroll
      for (int k = 0; k < kRowPass; k++) {
        const int r = r0 + kMassWaves * k;
        const bool ok = in && r < npr;
        mbv[k] = ok ? a.part_ml[((size_t)r * a.nblk + lane) * 2] : kNegInf;
        lt[k] = ok ? a.part_l[(size_t)r * a.nblk + lane] : 0.0f;
      }
      float* pwr = pw[wv];
#pragma unroll
      for (int k = 0; k < kRowPass; k++) {
        m[k] = wave_max_fast(mbv[k]);
        cb[k] = mbv[k] == kNegInf ? 0.0f : exp_det(mbv[k] - m[k]);
        pwr[k * kPwStride + lane] = lt[k] * cb[k];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // lane k: l of row r0 + 16k in block order, 32 blocks per read.
      // Entries past nblk up to the next multiple of 4 are +0 (0 * 0),
      // which leave a sum of non-negative terms unchanged.
      float lk = 0.0f;
      if (lane < kRowPass) {
        const f32x4* row = (const f32x4*)(pwr + lane * kPwStride);
        const int nc = (a.nblk + 3) >> 2;
        for (int h = 0; h < nc; h += 8) {
          f32x4 rv[8];
#pragma unroll
          for (int c = 0; c < 8; c++) rv[c] = row[h + c];
#pragma unroll
          for (int c = 0; c < 8; c++) {
            if (h + c < nc) {
              lk = lk + rv[c][0];
              lk = lk + rv[c][1];
              lk = lk + rv[c][2];
              lk = lk + rv[c][3];
            }
          }
        }
      }
      const float invk = 1.0f / lk;
#pragma unroll
      for (int k = 0; k < kRowPass; k++) {
        const int r = r0 + kMassWaves * k;
        const float inv = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, invk), k));
        if (r < npr) {
          if (lane == 0) {
            mi[r][0] = m[k];
            mi[r][1] = inv;
          }
          if (lane >= b0 && lane < b0 + kMassBlk) wsh[r * kMassBlk + (lane - b0)] = cb[k] * inv;
        }
      }
    }
  } else {
    for (int r = wv; r < npr; r += kMassWaves) {
      const size_t rb = (size_t)r * a.nblk;
      float m = kNegInf;
      for (int c0 = 0; c0 < a.nblk; c0 += 64)
        m = __builtin_fmaxf(m, c0 + lane < a.nblk ? a.part_ml[(rb + c0 + lane) * 2] : kNegInf);
      m = wave_max_fast(m);
      float l = 0.0f, cw = 0.0f;
      for (int c0 = 0; c0 < a.nblk; c0 += 64) {
        const int b = c0 + lane;
        const float mb = b < a.nblk ? a.part_ml[(rb + b) * 2] : kNegInf;
        const float lt = b < a.nblk ? a.part_l[rb + b] : 0.0f;
        const float cb = mb == kNegInf ? 0.0f : exp_det(mb - m);
        const float prod = lt * cb;
        const int nb = min(64, a.nblk - c0);
        for (int u = 0; u < nb; u++)
          l = l + __builtin_bit_cast(
                      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, prod), u));
        if (b >= b0 && b < b0 + kMassBlk) cw = cb;
      }
      const float inv = 1.0f / l;
      if (lane == 0) {
        mi[r][0] = m;
        mi[r][1] = inv;
      }
      const int bl = (b0 & 63) + (lane & 3);  // lanes 0..3: the first group's blocks
      const float cwl = __builtin_bit_cast(
          float, __builtin_amdgcn_ds_bpermute(bl << 2, __builtin_bit_cast(int, cw)));
      if (lane < kMassBlk) wsh[r * kMassBlk + lane] = cwl * inv;
    }
  }
  __syncthreads();
  uint64_t kwin = ~0ull, kall = ~0ull;  // the next step's placement keys (a.keys)
  for (;;) {
    const int t = g * 256 + tid;
    if (tid < 256 && t < a.n_live) {
      const int bl = (t >> 6) - b0;
      const bool re = t == placed;
      const int spt = re ? a.posj : sp;
      float x = re ? 0.0f : acc;
      if (spt <= a.qpos0) {
#pragma unroll
        for (int h = 0; h < NH; h++) x = x + ev0[h] * wsh[h * kMassBlk + bl];
      }
      for (int i = 1; i < a.Sq; i++) {
        if (spt > a.qpos0 + i) continue;
        float ev[NH];
#pragma unroll
        for (int h = 0; h < NH; h++) ev[h] = a.sc[(size_t)(i * NH + h) * cp + t];
#pragma unroll
        for (int h = 0; h < NH; h++) x = x + ev[h] * wsh[(i * NH + h) * kMassBlk + bl];
      }
      a.attn_sum[t] = x;
      if (re) a.slotpos_w[t] = a.posj;
      if (a.keys && x < kPicked) {
        const uint64_t key = place_key(x, t);
        kall = min_u64(kall, key);
        if (spt <= a.klim) kwin = min_u64(kwin, key);
      }
    }
    g += nsw;
    if (g >= ng) break;
    // the next group: its loads, then its w_b
    b0 = g * kMassBlk;
    fetch(g);
    __syncthreads();  // the previous group's weights are read
    for (int x = tid; x < npr * kMassBlk; x += kMassWaves * 64) {
      const int r = x / kMassBlk, b = b0 + x % kMassBlk;
      const float mb = b < a.nblk ? a.part_ml[((size_t)r * a.nblk + b) * 2] : kNegInf;
      const float cb = mb == kNegInf ? 0.0f : exp_det(mb - mi[r][0]);
      wsh[x] = cb * mi[r][1];
    }
    __syncthreads();
  }
  if (a.keys && blockIdx.x == 0 && tid == 0) {
    // the tag of these keys: this buffer, for a next step at posj + 1
    a.keys[kKeyTag] = (uint64_t)(uintptr_t)a.attn_sum;
    a.keys[kKeyTag + 1] = (uint64_t)(a.posj + 1);
  }
  if (a.keys && wv < 4) {
    // each slot-owning wave's minimum keys
    kwin = wave_min_u64(kwin);
    kall = wave_min_u64(kall);
    if (lane == 0) {
      a.keys[2 * (blockIdx.x * 4 + wv)] = kwin;
      a.keys[2 * (blockIdx.x * 4 + wv) + 1] = kall;
    }
  }
}

// the placement keys' region after the partials (16-byte aligned)
int64_t h2o_keys_offset(int S, int C) {
  const int64_t sq = std::min(S, kChunk), nblk = (C + 63) / 64;
  return (sq * NH * (2 * nblk * 64 + 3 * nblk) * (int64_t)sizeof(float) + 15) / 16 * 16;
}

int64_t h2o_ws_bytes(int S, int C) {
  static_assert(kKeyTag == kMassMaxWg * 4 * 2, "key tag index");
  return h2o_keys_offset(S, C) + (int64_t)(kKeyTag + 2) * sizeof(uint64_t);
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
    a.keys = nullptr;
    a.klim = 0;
    hipLaunchKernelGGL(k_h2o_scores<false>, dim3(nblk, NKV, sq), dim3(256), 0, s, a,
                       H2oPlace{nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                                nullptr, nullptr, 0, 0, 0, 0, nullptr, 0, 0, 0});
    int st = launch_status();
    if (st) return st;
    const int nsw = std::min((n_live + 255) / 256, kMassMaxWg);
    hipLaunchKernelGGL(k_h2o_mass<8>, dim3(nsw + (sq * NH + kMassWaves - 1) / kMassWaves),
                       dim3(kMassWaves * 64), 0, s, a, nsw);
    if ((st = launch_status())) return st;
  }
  return CIA_OK;
}

// One decode step of an H2O layer in two launches: the token placed and
// quantised inside the scores launch (H2oPlace), then the mass launch.  The
// same slots, positions, bytes and masses as cia_h2o_place followed by
// cia_attention_h2o for S = 1.  mid_event (may be NULL) is recorded after
// the scores launch.  When the buffer is full after the step, the mass
// launch also leaves in ws the placement keys of a next step at past + 1
// with the same window; keys_valid says that the previous call on this
// layer was such a step at past - 1 (and nothing else has touched the
// buffer since), so the scores launch reads those keys instead of every
// slot's mass and position.
extern "C" __attribute__((visibility("hidden"))) int cia_h2o_decode_step(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, uint8_t* kf, uint8_t* vf,
    uint16_t* ks, uint16_t* vs, float* attn_sum, int32_t* slot_pos, int32_t* dst_slots,
    int* n_live, int C, int W, int past, uint16_t* out, float scale, void* ws, int64_t ws_bytes,
    void* stream, void* mid_event, int keys_valid) {
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
  uint64_t* keys = (uint64_t*)((char*)ws + h2o_keys_offset(1, n1));
  a.keys = n1 >= C ? keys : nullptr;
  a.klim = past + 1 - W;
  const H2oPlace pl{k,  v,  kf, vf, ks,   vs,
                    attn_sum, slot_pos, dst_slots, n0, C, W, past,
                    keys_valid && n0 >= C ? keys : nullptr,
                    4 * std::min((n0 + 255) / 256, kMassMaxWg),
                    (uint64_t)(uintptr_t)attn_sum, (uint64_t)past};
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
  if (n0 >= C) {
    a.placed = dst_slots;
    a.slotpos_w = slot_pos;
  }
  const int nsw = std::min((n1 + 255) / 256, kMassMaxWg);
  hipLaunchKernelGGL(k_h2o_mass<2>, dim3(nsw + NH / kMassWaves), dim3(kMassWaves * 64), 0, s, a,
                     nsw);
  if ((st = launch_status())) return st;
  *n_live = n1;
  return CIA_OK;
}
