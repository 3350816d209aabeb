// prefill_fp8.hip -- the OCP-fp8 matrix-core variant of the causal attention
// of attention_fused (engine.cu:236-308).  Both products run on gfx950's
// v_mfma_scale_f32_16x16x128_f8f6f4 with E4M3 operands -- the cache's own
// format, read as bytes with no conversion -- and per-32-element power-of-two
// operand scales.
//
// An MFMA of this shape sums over 128 elements; a head has 64 dims and a
// tile 64 keys, so each product carries a second fp8 term in the other 64:
//   S^T = K Q^T: A = [K | K], B = [Q_hi | Q_lo] with Q = sq (Q_hi + Q_lo/16),
//        Q_hi = e4m3(Q / sq), Q_lo = e4m3(16 (Q / sq - Q_hi)), sq = amax/448
//        per (query, head); the scale 2^-4 rides on Q_lo's 32-element blocks.
//        Scores carry about 8 bits of Q precision instead of 4.
//   O^T += V^T P^T: A = [V^T | V^T] with the tile's V scale exponent as A's
//        block scale, B = [P_hi | P_lo], P_hi = e4m3(P'), P_lo = e4m3(P' -
//        P_hi): the numerators keep about 8 bits too.
// K/V enter with the cache's own FP8 rounding only; the remaining extra
// error (Q and P to ~2^-8) is measured against the fp32 restatement and
// reported, not held to the fp16 kernel's tolerance.
//
// Operand layout of the 16x16x128 fp8 form (measured): lane (n, g), n = l &
// 15, g = l >> 4, holds row/column n at k = 16 g + j (bytes 0..15) and
// k = 64 + 16 g + j (bytes 16..31); the block scale of lane (n, g) covers
// k in [32 g, 32 g + 32).  K-index k < 64 maps to key / dim
// pi(16 g + j) = 16 (j / 4) + 4 g + (j % 4), the keys a lane holds in the
// S^T accumulators, so P needs no movement between the two products.
//
// Work split, heavy/light block pairing, the two-deep prefetch and the lazy
// running max follow the fp16 kernel; numerators are P' = 2^(s c - m + 3) *
// mant(V scale), at most 2^8.5 while s c - m <= 4.5, so they stay in E4M3's
// range, and keys 12 binades below the running max still register.  The fp16 tail tile (keys not yet committed) runs on the fp16
// tile with the running max offset by the bias: tail keys carry no rounding
// beyond the fp16 kernel's.
#include "prefill_tile.h"

namespace cia {

constexpr int kF8Q = 64;              // queries per block
constexpr int kF8Tile = 4096;         // one fp8 64 x 64 tile
constexpr float kF8Log2e = 1.44269504088896340736f;
constexpr float kF8Bias = 3.0f;       // P' = 2^(t + 3) * mant
constexpr float kF8Remax = 4.5f;      // largest t kept without moving the max
constexpr int kE8One = 127;           // E8M0 encoding of 1.0

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;

// K tile: 64-byte key rows, 16-byte chunk c at c ^ (((key >> 1) ^ (key >> 2)) & 3):
// the rows n = 0..15 of one operand read cover all 64 banks, each group of 8
// of them all banks of a 128-byte half
__device__ __forceinline__ int f8_kaddr(int key, int c16) {
  return key * 64 + ((c16 ^ (((key >> 1) ^ (key >> 2)) & 3)) << 4);
}
// V tile: 64-byte key rows, 8-byte chunk c at c ^ f(key), f = 2 ((key >> 1
// ^ key >> 2) & 1) + 4 ((key >> 4) & 1): the keys of one transposed read
// (4g + {0..3}, 16 + 4g + {0..3}, and those of the next lane group) take
// distinct bank pairs within 16 and within 32 lanes
__device__ __forceinline__ int f8_vaddr(int key, int c8) {
  const int f = ((((key >> 1) ^ (key >> 2)) & 1) << 1) | (((key >> 4) & 1) << 2);
  return key * 64 + ((c8 ^ f) << 3);
}
// K-index x < 64 of lane group g -> key (or dim) of the tile
__device__ __forceinline__ int f8_pi(int g, int x) { return 16 * (x >> 2) + 4 * g + (x & 3); }

// a thread's share of a tile in flight: key tid >> 3, bytes 8 (tid & 7) .. +7
struct F8Stage {
  u32x2 k, v;
  uint16_t ks, vs;
};

__device__ __forceinline__ void f8_load(const PrefillArgs& a, int g, int j, int tid,
                                        F8Stage& st) {
  // the group's rows from a uniform base, this thread's bytes at a 32-bit
  // offset (one address register per load)
  const size_t grp = (size_t)j * (64 * NKV * D);
  const uint32_t row = (uint32_t)(((tid >> 3) * NKV + g) * D + 8 * (tid & 7));
  st.ks = a.ksc[j * NKV + g];
  st.vs = a.vsc[j * NKV + g];
  st.k = *(const u32x2*)(a.kc8 + grp + row);
  st.v = *(const u32x2*)(a.vc8 + grp + row);
}

__device__ __forceinline__ void f8_store(uint8_t* buf, int tid, u32x2 k, u32x2 v) {
  const int key = tid >> 3, c8 = tid & 7;
  *(u32x2*)(buf + f8_kaddr(key, c8 >> 1) + 8 * (c8 & 1)) = k;
  *(u32x2*)(buf + kF8Tile + f8_vaddr(key, c8)) = v;
}

// opaque to the uniformity analysis (keeps a late-used scale load from
// being waited for the moment it is issued)
__device__ __forceinline__ uint32_t f8_late(uint16_t x) {
  uint32_t v = x;
  asm volatile("" : "+v"(v));
  return v;
}

// e4m3 of four floats (no saturation: callers keep them in range).  The
// first conversion writes the low word over a's own bits, which the second
// replaces in the high word, so no register has to be cleared first.
__device__ __forceinline__ uint32_t f8_pack4(float a, float b, float c, float d) {
  const uint32_t w =
      (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, __builtin_bit_cast(int, a), false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
}

// an LDS address the compiler cannot equate with another, so that two
// reads of the same bytes land in the two halves of an operand without
// register copies
__device__ __forceinline__ const uint8_t* f8_opaque(const uint8_t* p) {
  asm volatile("" : "+v"(p));
  return p;
}

// A tile's V scale as 2^e * mant, mant in [1, 2): e goes to the MFMA's
// block scale, log2(mant) into the numerators.  A zero scale (a group of
// zeros) keeps e = 0, mant = 1.
struct F8VScale {
  int e8;        // E8M0 byte: 127 + e
  float lmant;   // log2(mant)
  float imant;   // 1 / mant
};
__device__ __forceinline__ F8VScale f8_vscale(float vs) {
  F8VScale r{kE8One, 0.0f, 1.0f};
  if (vs > 0.0f) {
    const int e = __builtin_amdgcn_frexp_expf(vs) - 1;  // vs = mant * 2^e
    const float mant = __builtin_ldexpf(vs, -e);
    r.e8 = kE8One + e;
    r.lmant = __builtin_amdgcn_logf(mant);
    r.imant = 1.0f / mant;
  }
  return r;
}

// numerators P' = 2^(s c + off) of one 16-query tile as the [P_hi | P_lo]
// B operand; returns the lane's fp32 sum of P'
template <bool kMask>
__device__ __forceinline__ float f8_exp(const f32x4 (&S)[4], float c, float off, int key0,
                                        int qpos, i32x8& P) {
  float p[4][4];
  float rs = 0.0f;
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float t = __builtin_fmaf(S[kt][i], c, off);
      if (kMask && key0 + 16 * kt + i > qpos) t = -__builtin_inff();
      p[kt][i] = __builtin_amdgcn_exp2f(t);
      rs += p[kt][i];
    }
#pragma unroll
  for (int kt = 0; kt < 4; kt++) {
    const uint32_t hi = f8_pack4(p[kt][0], p[kt][1], p[kt][2], p[kt][3]);
    const f32x2 h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, false);
    const f32x2 h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hi, true);
    P[kt] = (int)hi;
    P[4 + kt] = (int)f8_pack4(p[kt][0] - h01[0], p[kt][1] - h01[1], p[kt][2] - h23[0],
                              p[kt][3] - h23[1]);
  }
  return rs;
}

// largest s c - m over the lane's unmasked keys
template <bool kMask>
__device__ __forceinline__ float f8_tmax(const f32x4 (&S)[4], float c, float m, int key0,
                                         int qpos) {
  float mx = -__builtin_inff();
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const bool out = kMask && key0 + 16 * kt + i > qpos;
      mx = __builtin_fmaxf(mx, out ? -__builtin_inff() : S[kt][i]);
    }
  return mx * c - m;
}

// softmax of one query tile with the lazy running max: the lane's largest
// exponent is checked first, the max moved (on the column's first tile, or
// when a numerator would leave the fp8 range) with O and l rescaled, and the
// numerators computed once
template <bool kMask>
__device__ __forceinline__ void f8_softmax(const f32x4 (&S)[4], float c, const F8VScale& vsc,
                                           bool first, int key0, int qpos, float& m, float& l,
                                           f32x4 (&O)[4][2], int qt, i32x8& P) {
  const float tm = f8_tmax<kMask>(S, c, 0.0f, key0, qpos);  // largest s c of the lane
  if (first || __any(tm - m > kF8Remax)) {
    // the column's largest score of this tile (finite on a first tile: key
    // 0 is never masked; c > 0)
    const float mt = col4_max(tm);
    if (first) {
      m = mt;
    } else if (mt > m) {
      const float corr = __builtin_amdgcn_exp2f(m - mt);
      m = mt;
      l *= corr;
#pragma unroll
      for (int dt = 0; dt < 4; dt++)
#pragma unroll
        for (int i = 0; i < 4; i++) O[dt][qt][i] *= corr;
    }
  }
  const float rs = f8_exp<kMask>(S, c, kF8Bias + vsc.lmant - m, key0, qpos, P);
  l = __builtin_fmaf(rs, vsc.imant, l);
}

// One 64-key tile for the wave's two 16-query tiles
template <bool kMask>
__device__ __forceinline__ void f8_tile(const uint8_t* kt_lds, const uint8_t* vt_lds,
                                        const i32x8 (&qop)[2], int qsc, const float (&c)[2],
                                        const F8VScale& vsc, bool first, int key0, int qpos0,
                                        int n, int g, f32x4 (&O)[4][2], float (&mrun)[2],
                                        float (&lrun)[2]) {
  // A = [K | K]: key 16 kt + n, dims 16 g .. +15, twice
  i32x8 kop[4];
#pragma unroll
  for (int kt = 0; kt < 4; kt++) {
    const int off = f8_kaddr(16 * kt + n, g);
    const u32x4 r = *(const u32x4*)(kt_lds + off);
    const u32x4 r2 = *(const u32x4*)(f8_opaque(kt_lds) + off);
    kop[kt] = i32x8{(int)r[0], (int)r[1], (int)r[2], (int)r[3],
                    (int)r2[0], (int)r2[1], (int)r2[2], (int)r2[3]};
  }
  f32x4 S0[4], S1[4];
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
    S0[kt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
        kop[kt], qop[0], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, kE8One, 0, qsc);
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
    S1[kt] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
        kop[kt], qop[1], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, kE8One, 0, qsc);
  // A = [V^T | V^T]: dim 16 dt + n of keys pi(g, 0..15).  Lane j of a
  // 16-lane group loads key pi(g, 8 r + (j >> 1)), bytes 16 dt + 8 (j & 1)
  // .. +7; the transposed read hands lane n byte i = V[pi(g, 8 r + i)][16 dt + n].
  i32x8 vop[4];
#pragma unroll
  for (int dt = 0; dt < 4; dt++) {
    const int o0 = f8_vaddr(f8_pi(g, n >> 1), 2 * dt + (n & 1));
    const int o1 = f8_vaddr(f8_pi(g, 8 + (n >> 1)), 2 * dt + (n & 1));
    const uint8_t* vt2 = f8_opaque(vt_lds);
    const i32x2 r0 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(vt_lds + o0));
    const i32x2 r1 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(vt_lds + o1));
    const i32x2 r2 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(vt2 + o0));
    const i32x2 r3 = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(vt2 + o1));
    vop[dt] = i32x8{r0[0], r0[1], r1[0], r1[1], r2[0], r2[1], r3[0], r3[1]};
  }
  const int kb0 = key0 + 4 * g;
  i32x8 P0, P1;
  f8_softmax<kMask>(S0, c[0], vsc, first, kb0, qpos0, mrun[0], lrun[0], O, 0, P0);
#pragma unroll
  for (int dt = 0; dt < 4; dt++)
    O[dt][0] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(vop[dt], P0, O[dt][0], 0, 0, 0,
                                                                vsc.e8, 0, kE8One);
  f8_softmax<kMask>(S1, c[1], vsc, first, kb0, qpos0 + 16, mrun[1], lrun[1], O, 1, P1);
#pragma unroll
  for (int dt = 0; dt < 4; dt++)
    O[dt][1] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(vop[dt], P1, O[dt][1], 0, 0, 0,
                                                                vsc.e8, 0, kE8One);
}

// grid = 8 * ceil(nblk / 2), block = 512
__global__ __launch_bounds__(512) void k_prefill_fp8(PrefillArgs a) {
  // two fp8 tile buffers; the fp16 tail tile uses the whole array
  static_assert(2 * 2 * kF8Tile == 2 * kPfTileBytes, "fp16 tail tile size");
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2 * kF8Tile];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, n = l & 15, g16 = l >> 4;
  const int g = blockIdx.x & 7, pr = blockIdx.x >> 3;
  const int h = g * GQA + (w & 3);
  const int nvalid_tail = a.past + a.S - a.committed;
  const int nfp8 = a.committed >> 6;
  // Q_lo's 32-element blocks (lane groups 2, 3) carry 2^-4
  const int qsc = g16 >= 2 ? kE8One - 4 : kE8One;

  for (int phase = 0; phase < 2; phase++) {
    const int blk = phase == 0 ? a.nblk - 1 - pr : pr;
    if (phase == 1 && pr >= a.nblk - 1 - pr) break;  // the middle block runs once
    const int q0 = blk * kF8Q + 32 * (w >> 2);
    const int kend = a.past + min(a.S, (blk + 1) * kF8Q);
    const int ntile = (kend + 63) >> 6;
    const int qmin = a.past + q0;
    const int qlast = a.past + min(q0 + 31, a.S - 1);
    const bool wave_live = q0 < a.S;

    // B = [Q_hi | Q_lo]: lane (n, g16) holds query q0 + 16 qt + n, dims
    // 16 g16 .. +15 of both terms
    i32x8 qop[2];
    float qs[2];
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
      const int s = q0 + 16 * qt + n;
      u32x4 r[2] = {{0u, 0u, 0u, 0u}, {0u, 0u, 0u, 0u}};
      if (s < a.S) {
        const u32x4* qp = (const u32x4*)(a.q + ((size_t)s * NH + h) * D + 16 * g16);
        r[0] = qp[0];
        r[1] = qp[1];
      }
      float x[16];
      float mx = 0.0f;
#pragma unroll
      for (int i = 0; i < 16; i++) {
        x[i] = h2f((uint16_t)(r[i >> 3][(i >> 1) & 3] >> (16 * (i & 1))));
        mx = __builtin_fmaxf(mx, __builtin_fabsf(x[i]));
      }
      const float sq = quant_scale(col4_max(mx));
      const float iq = 1.0f / sq;
#pragma unroll
      for (int c4 = 0; c4 < 4; c4++) {
        float y[4], lo[4];
#pragma unroll
        for (int i = 0; i < 4; i++) y[i] = x[4 * c4 + i] * iq;
        const uint32_t hw = e4m3x4(y[0], y[1], y[2], y[3]);
        const f32x2 h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hw, false);
        const f32x2 h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)hw, true);
        lo[0] = 16.0f * (y[0] - h01[0]);
        lo[1] = 16.0f * (y[1] - h01[1]);
        lo[2] = 16.0f * (y[2] - h23[0]);
        lo[3] = 16.0f * (y[3] - h23[1]);
        qop[qt][c4] = (int)hw;
        qop[qt][4 + c4] = (int)e4m3x4(lo[0], lo[1], lo[2], lo[3]);
      }
      qs[qt] = sq * a.qscale;
    }
    f32x4 O[4][2];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
      for (int qt = 0; qt < 2; qt++) O[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrun[2] = {0.f, 0.f}, lrun[2] = {0.f, 0.f};

    const int nf = min(ntile, nfp8);
    const int qpos0 = a.past + q0 + n;
    F8Stage st;
    float kc_cur = 1.0f, vs_cur = 1.0f, kc_next = 1.0f, vs_next = 1.0f;
    if (nf > 0) {
      f8_load(a, g, 0, tid, st);
      kc_cur = h2f((uint16_t)f8_late(st.ks));
      vs_cur = h2f((uint16_t)f8_late(st.vs));
      f8_store(lds[0], tid, st.k, st.v);
      if (nf > 1) f8_load(a, g, 1, tid, st);
    }
    __syncthreads();
    for (int j = 0; j < nf; j++) {
      if (j + 1 < nf) {
        kc_next = h2f((uint16_t)f8_late(st.ks));
        vs_next = h2f((uint16_t)f8_late(st.vs));
        f8_store(lds[(j + 1) & 1], tid, st.k, st.v);
        if (j + 2 < nf) f8_load(a, g, j + 2, tid, st);
      }
      if (wave_live && 64 * j <= qlast) {
        // multiplier >= 1e-30 keeps masked keys at -inf for a zero K scale
        const float c[2] = {__builtin_fmaxf(kc_cur * qs[0], 1e-30f),
                            __builtin_fmaxf(kc_cur * qs[1], 1e-30f)};
        const F8VScale vsc = f8_vscale(vs_cur);
        if (64 * j + 63 > qmin)
          f8_tile<true>(lds[j & 1], lds[j & 1] + kF8Tile, qop, qsc, c, vsc, j == 0, 64 * j,
                        qpos0, n, g16, O, mrun, lrun);
        else
          f8_tile<false>(lds[j & 1], lds[j & 1] + kF8Tile, qop, qsc, c, vsc, j == 0, 64 * j,
                         qpos0, n, g16, O, mrun, lrun);
      }
      kc_cur = kc_next;
      vs_cur = vs_next;
      __syncthreads();
    }
    if (ntile > nf) {
      // the fp16 tail on the fp16 tile (fp16 Q operands, numerators
      // 2^(s c - (m - 3)) so that O and l keep this kernel's scale)
      uint8_t* buf = &lds[0][0];
      const uint32_t sel01 = ((tid >> 5) & 1) ? 0x07060302u : 0x05040100u;
      const uint32_t sel10 = ((tid >> 5) & 1) ? 0x05040100u : 0x07060302u;
      PfStage16 s16;
      pf_load16(a, g, nvalid_tail, tid, s16);
      pf_store16(buf, tid, s16, sel01, sel10);
      __syncthreads();
      if (wave_live && 64 * nf <= qlast) {
        f16x8 qh[2][2];
#pragma unroll
        for (int qt = 0; qt < 2; qt++) {
          const int s = q0 + 16 * qt + n;
#pragma unroll
          for (int kb = 0; kb < 2; kb++)
            qh[qt][kb] = s < a.S ? *(const f16x8*)(a.q + ((size_t)s * NH + h) * D + 32 * kb + 8 * g16)
                                 : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
        }
        float m16[2] = {mrun[0] - kF8Bias, mrun[1] - kF8Bias};
        pf_tile<true>(buf, buf + kPfTileBytes, qh, __builtin_fmaxf(a.qscale, 1e-30f), nf == 0,
                      64 * nf, qpos0, n, g16, O, m16, lrun);
      }
      __syncthreads();
    }
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
      const float L = col4_sum(lrun[qt]);
      const int s = q0 + 16 * qt + n;
      if (s < a.S) {
        const float inv = 1.0f / L;
        uint16_t* op = a.out + ((size_t)s * NH + h) * D + 4 * g16;
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
          u32x2 r;
          r[0] = (uint32_t)f2h(O[dt][qt][0] * inv) | ((uint32_t)f2h(O[dt][qt][1] * inv) << 16);
          r[1] = (uint32_t)f2h(O[dt][qt][2] * inv) | ((uint32_t)f2h(O[dt][qt][3] * inv) << 16);
          *(u32x2*)(op + 16 * dt) = r;
        }
      }
    }
  }
}

}  // namespace cia

using namespace cia;

extern "C" int cia_attention_fused_fp8(const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8,
                                       const uint16_t* ksc, const uint16_t* vsc,
                                       const uint16_t* ktail, const uint16_t* vtail,
                                       int committed, uint16_t* out, int S, int past, float scale,
                                       void* stream) {
  CIA_REQUIRE(S >= 0 && past >= 0 && committed >= 0 && committed % G == 0, CIA_ERR_ARG);
  if (S == 0) return CIA_OK;
  CIA_REQUIRE(q && kc8 && vc8 && ksc && vsc && ktail && vtail && out, CIA_ERR_NULL);
  CIA_REQUIRE(past + S - 1 - committed < G, CIA_ERR_STATE);  // the tail holds at most 64 keys
  CIA_REQUIRE(scale >= 0.0f && scale < __builtin_inff(), CIA_ERR_ARG);
  CIA_REQUIRE(aligned(q, 16) && aligned(kc8, 16) && aligned(vc8, 16) && aligned(ktail, 16) &&
                  aligned(vtail, 16) && aligned(out, 8) && aligned(ksc, 2) && aligned(vsc, 2),
              CIA_ERR_ALIGN);
  const int nblk = (S + kF8Q - 1) / kF8Q;
  PrefillArgs fa{q, kc8, vc8, ksc, vsc, ktail, vtail, committed, out, S, past, scale * kF8Log2e,
                 nblk};
  hipLaunchKernelGGL(k_prefill_fp8, dim3(8 * ((nblk + 1) / 2)), dim3(512), 0,
                     (hipStream_t)stream, fa);
  return launch_status();
}
