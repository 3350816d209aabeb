// prefill_tile.h -- the fp16 matrix-core tile of the causal prefill: the
// LDS layouts, staging, softmax and products of one 64-key tile for a
// wave's two 16-query tiles.  Used by the fp16 kernel for every tile and by
// the OCP-fp8 kernel for the fp16 tail tile.
#pragma once

#include "common.h"

namespace cia {


constexpr int kPfWaves = 8;
constexpr int kPfQ = 64;            // queries per block
constexpr int kPfTileBytes = 8192;  // one fp16 64 x 64 tile
constexpr float kPfLog2e = 1.44269504088896340736f;

struct PrefillArgs {
  const uint16_t* q;  // [S][32][64]
  const uint8_t* kc8;
  const uint8_t* vc8;
  const uint16_t* ksc;
  const uint16_t* vsc;
  const uint16_t* ktail;
  const uint16_t* vtail;
  int committed;
  uint16_t* out;  // [S][32][64]
  int S, past;
  float qscale;   // softmax scale * log2(e)
  int nblk;       // ceil(S / 64)
};

// K tile: key row of 128 bytes, 16-byte chunk c stored at c ^ ((key >> 1) & 7)
__device__ __forceinline__ int pf_kaddr(int key, int c) {
  return key * 128 + ((c ^ ((key >> 1) & 7)) << 4);
}
// V^T tile: dim row of 128 bytes (64 key slots), same chunk swizzle
__device__ __forceinline__ int pf_vaddr(int dim, int slot) {
  return dim * 128 + ((((slot >> 3) ^ ((dim >> 1) & 7))) << 4) + (slot & 7) * 2;
}
// key t (0..63) of a tile -> its V^T slot
__device__ __forceinline__ int pf_vslot(int t) {
  const int r = t & 31;
  return (t & 32) + 8 * ((r >> 2) & 3) + 4 * (r >> 4) + (r & 3);
}

__device__ __forceinline__ f16x8 pf_cvt8(uint32_t w0, uint32_t w1) {
  const f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false);
  const f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true);
  const f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false);
  const f16x2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true);
  return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// One thread's share of a tile in flight: K key tid >> 3, dims 8 (tid & 7)
// .. +7; V keys 2 (tid & 31) and +1, dims 4 (tid >> 5) .. +3.  FP8 tiles and
// the fp16 tail use separate registers, so a prefetch never waits on the
// previous one.
struct PfStage8 {
  u32x2 k;           // 8 fp8 K bytes
  uint32_t v0, v1;   // 4 fp8 V bytes of keys 2kp, 2kp+1
  uint16_t ks, vs;   // group scales (fp16 bits)
};
struct PfStage16 {
  u32x4 k;           // 8 fp16 K values
  u32x2 v0, v1;      // 4 fp16 V values of keys 2kp, 2kp+1
};

__device__ __forceinline__ void pf_load8(const PrefillArgs& a, int g, int j, int tid,
                                         PfStage8& st) {
  const int kkey = tid >> 3, kch = tid & 7, kp = tid & 31, dc = tid >> 5;
  st.ks = a.ksc[j * NKV + g];
  st.vs = a.vsc[j * NKV + g];
  // the group's rows from a uniform base, this thread's bytes at a 32-bit
  // offset (one address register per load)
  const uint8_t* kg = a.kc8 + (size_t)j * (64 * NKV * D);
  const uint8_t* vg = a.vc8 + (size_t)j * (64 * NKV * D);
  st.k = *(const u32x2*)(kg + (uint32_t)((kkey * NKV + g) * D + 8 * kch));
  const uint32_t v0 = (uint32_t)((2 * kp * NKV + g) * D + 4 * dc);
  st.v0 = *(const uint32_t*)(vg + v0);
  st.v1 = *(const uint32_t*)(vg + v0 + NKV * D);
}

// tail rows 0..nvalid-1 (keys committed..); the others stage as zeros
__device__ __forceinline__ void pf_load16(const PrefillArgs& a, int g, int nvalid, int tid,
                                          PfStage16& st) {
  const int kkey = tid >> 3, kch = tid & 7, kp = tid & 31, dc = tid >> 5;
  st.k = u32x4{0u, 0u, 0u, 0u};
  st.v0 = st.v1 = u32x2{0u, 0u};
  if (kkey < nvalid) st.k = *(const u32x4*)(a.ktail + ((size_t)kkey * NKV + g) * D + 8 * kch);
  if (2 * kp < nvalid) st.v0 = *(const u32x2*)(a.vtail + ((size_t)(2 * kp) * NKV + g) * D + 4 * dc);
  if (2 * kp + 1 < nvalid)
    st.v1 = *(const u32x2*)(a.vtail + ((size_t)(2 * kp + 1) * NKV + g) * D + 4 * dc);
}

// K row chunk and the V^T words of this thread (dims 4dc..4dc+3, each the
// pair key 2kp, key 2kp+1).  The upper half-wave writes its dims in the
// order 1,0,3,2, which spreads the writes over all LDS banks: the byte
// selectors sel01 / sel10 pick dims (0,1) / (1,0) of a pair of f16x2 words.
__device__ __forceinline__ void pf_store(uint8_t* buf, int tid, u32x4 kw, u32x2 va, u32x2 vb,
                                         uint32_t sel01, uint32_t sel10) {
  const int kkey = tid >> 3, kch = tid & 7, kp = tid & 31, dc = tid >> 5;
  *(u32x4*)(buf + pf_kaddr(kkey, kch)) = kw;
  const int slot = pf_vslot(2 * kp);
  const int flip = (tid >> 5) & 1;
  uint8_t* vt = buf + kPfTileBytes;
  // word for dim 4dc + d: (va half d, vb half d); v_perm picks bytes of
  // {vb, va} (va = bytes 0-3, vb = bytes 4-7)
  *(uint32_t*)(vt + pf_vaddr(4 * dc + (0 ^ flip), slot)) = __builtin_amdgcn_perm(vb[0], va[0], sel01);
  *(uint32_t*)(vt + pf_vaddr(4 * dc + (1 ^ flip), slot)) = __builtin_amdgcn_perm(vb[0], va[0], sel10);
  *(uint32_t*)(vt + pf_vaddr(4 * dc + (2 ^ flip), slot)) = __builtin_amdgcn_perm(vb[1], va[1], sel01);
  *(uint32_t*)(vt + pf_vaddr(4 * dc + (3 ^ flip), slot)) = __builtin_amdgcn_perm(vb[1], va[1], sel10);
}

// A group scale loaded two tiles ahead, read when its tile is staged.  The
// empty asm makes the value opaque to the compiler's uniformity analysis, so
// it is not moved into a scalar register (which would wait for the load the
// moment it is issued).
__device__ __forceinline__ uint32_t pf_late(uint16_t x) {
  uint32_t v = x;
  asm volatile("" : "+v"(v));
  return v;
}

// K scale -> score multiplier base (times scale * log2e where it is used)
__device__ __forceinline__ float pf_scale(uint16_t ks) { return h2f((uint16_t)pf_late(ks)); }

// K is staged exactly (fp8 -> fp16), V as V * V scale (one fp16 rounding)
__device__ __forceinline__ void pf_store8(uint8_t* buf, int tid, const PfStage8& st,
                                          uint32_t sel01, uint32_t sel10) {
  const u32x4 kw = __builtin_bit_cast(u32x4, pf_cvt8(st.k[0], st.k[1]));
  const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)pf_late(st.vs));
  const f16x2 s2 = f16x2{s, s};
  const f16x2 a0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(st.v0, 1.0f, false) * s2;
  const f16x2 a1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(st.v0, 1.0f, true) * s2;
  const f16x2 b0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(st.v1, 1.0f, false) * s2;
  const f16x2 b1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(st.v1, 1.0f, true) * s2;
  pf_store(buf, tid, kw,
           u32x2{__builtin_bit_cast(uint32_t, a0), __builtin_bit_cast(uint32_t, a1)},
           u32x2{__builtin_bit_cast(uint32_t, b0), __builtin_bit_cast(uint32_t, b1)}, sel01, sel10);
}

__device__ __forceinline__ void pf_store16(uint8_t* buf, int tid, const PfStage16& st,
                                           uint32_t sel01, uint32_t sel10) {
  pf_store(buf, tid, st.k, st.v0, st.v1, sel01, sel10);
}

// max over the 4 lanes {l, l^16, l^32, l^48} that hold one query column
__device__ __forceinline__ float pf_colmax(float v) { return col4_max(v); }
__device__ __forceinline__ float pf_colsum(float v) { return col4_sum(v); }

// Softmax numerators of one 16-query tile: exponents s * c - m (log2
// units) of the scores S[kt] (rows = keys key0 + 16 kt + i, column = query
// qpos).  P[u] is the B operand of key block u; returns this lane's sum of
// the fp16 numerators, which is infinite once a numerator overflows fp16,
// i.e. once a score exceeds the running max by about 16.
template <bool kMask>
__device__ __forceinline__ float pf_exp(const f32x4 (&S)[4], float c, float m, int key0, int qpos,
                                        f16x8 (&P)[2]) {
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float t = __builtin_fmaf(S[kt][i], c, -m);
      if (kMask && key0 + 16 * kt + i > qpos) t = -__builtin_inff();
      P[kt >> 1][4 * (kt & 1) + i] = (_Float16)__builtin_amdgcn_exp2f(t);
    }
  const f16x2 one = f16x2{(_Float16)1.0f, (_Float16)1.0f};
  float rs = 0.f;
#pragma unroll
  for (int u = 0; u < 2; u++)
#pragma unroll
    for (int e = 0; e < 4; e++)
      rs = __builtin_amdgcn_fdot2(f16x2{P[u][2 * e], P[u][2 * e + 1]}, one, rs, false);
  return rs;
}

// Moves the running max of a query column to the column's largest score of
// this tile: always on the column's first tile (no max yet), otherwise when
// that score is above it (a numerator overflowed).  Rescales O and l and
// recomputes the numerators.
template <bool kMask>
__device__ __forceinline__ float pf_remax(const f32x4 (&S)[4], float c, bool first, float& m,
                                          float& l, f32x4 (&O)[4], int key0, int qpos,
                                          f16x8 (&P)[2]) {
  float cm = -__builtin_inff();
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const bool out = kMask && key0 + 16 * kt + i > qpos;
      cm = __builtin_fmaxf(cm, out ? -__builtin_inff() : S[kt][i]);
    }
  // finite on a first tile (key 0 is never masked); c > 0
  const float mt = pf_colmax(cm) * c;
  if (first) {
    m = mt;
  } else if (mt > m) {
    const float corr = __builtin_amdgcn_exp2f(m - mt);
    m = mt;
    l *= corr;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
      for (int i = 0; i < 4; i++) O[dt][i] *= corr;
  }
  return pf_exp<kMask>(S, c, m, key0, qpos, P);
}

// exponentials of one query tile, with the re-max path when needed.  The
// running max only moves when a numerator would overflow fp16, so between
// moves the exponents stay below 16 (fp16 numerators, fp32 sums are safe).
template <bool kMask>
__device__ __forceinline__ void pf_softmax(const f32x4 (&S)[4], float c, bool first, int key0,
                                           int qpos, float& m, float& l, f32x4 (&O)[4][2],
                                           int qt, f16x8 (&P)[2]) {
  float rs = first ? __builtin_inff() : pf_exp<kMask>(S, c, m, key0, qpos, P);
  if (__any(!(rs < 3.0e38f))) {
    f32x4 Oq[4] = {O[0][qt], O[1][qt], O[2][qt], O[3][qt]};
    rs = pf_remax<kMask>(S, c, first, m, l, Oq, key0, qpos, P);
#pragma unroll
    for (int dt = 0; dt < 4; dt++) O[dt][qt] = Oq[dt];
  }
  l += rs;
}

// One 64-key tile for the wave's two 16-query tiles.  The second query
// tile's products are issued before the first tile's exponentials, and the
// first tile's P V before the second tile's exponentials, so the matrix
// cores and the vector unit of one wave overlap.
template <bool kMask>
__device__ __forceinline__ void pf_tile(const uint8_t* kt_lds, const uint8_t* vt_lds,
                                        const f16x8 (&qop)[2][2], float c, bool first, int key0,
                                        int qpos0, int n, int b, f32x4 (&O)[4][2],
                                        float (&mrun)[2], float (&lrun)[2]) {
  f16x8 kop[4][2];
#pragma unroll
  for (int kt = 0; kt < 4; kt++)
#pragma unroll
    for (int kb = 0; kb < 2; kb++)
      kop[kt][kb] = *(const f16x8*)(kt_lds + pf_kaddr(16 * kt + n, 4 * kb + b));
  f32x4 S0[4], S1[4];
#pragma unroll
  for (int kt = 0; kt < 4; kt++) {
    S0[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[kt][0], qop[0][0], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    S0[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[kt][1], qop[0][1], S0[kt], 0, 0, 0);
  }
#pragma unroll
  for (int kt = 0; kt < 4; kt++) {
    S1[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[kt][0], qop[1][0], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    S1[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop[kt][1], qop[1][1], S1[kt], 0, 0, 0);
  }
  const int kb0 = key0 + 4 * b;
  f16x8 P0[2], P1[2];
  pf_softmax<kMask>(S0, c, first, kb0, qpos0, mrun[0], lrun[0], O, 0, P0);
  f16x8 vop[4][2];
#pragma unroll
  for (int dt = 0; dt < 4; dt++)
#pragma unroll
    for (int u = 0; u < 2; u++)
      vop[dt][u] = *(const f16x8*)(vt_lds + pf_vaddr(16 * dt + n, 32 * u + 8 * b));
#pragma unroll
  for (int dt = 0; dt < 4; dt++)
#pragma unroll
    for (int u = 0; u < 2; u++)
      O[dt][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop[dt][u], P0[u], O[dt][0], 0, 0, 0);
  pf_softmax<kMask>(S1, c, first, kb0, qpos0 + 16, mrun[1], lrun[1], O, 1, P1);
#pragma unroll
  for (int dt = 0; dt < 4; dt++)
#pragma unroll
    for (int u = 0; u < 2; u++)
      O[dt][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop[dt][u], P1[u], O[dt][1], 0, 0, 0);
}

}  // namespace cia
