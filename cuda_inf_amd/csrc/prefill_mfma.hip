// prefill_mfma.hip -- causal attention over the group-64 cache on the gfx950
// matrix cores: the output of attention_fused (engine.cu:236-308) for S
// queries at positions past..past+S-1, every key 0..pos of each query.
//
// Work unit: one kv head g and a block of 64 queries.  A workgroup of 8 waves
// serves the 4 query heads of g for those 64 queries (wave w: query head
// 4g + (w & 3), queries 32 (w >> 2) .. +31), so every K/V tile staged in LDS
// feeds 8 waves.  Workgroups take one heavy and one light block (blocks nb-1-p
// and p), which evens out the causal work; workgroup i serves kv head i mod 8,
// and workgroups are handed to the 8 XCDs round-robin, so one XCD's L2 holds
// one kv head's cache.
//
// Tiles are the cache's own 64-key groups: K and V of committed group j are
// FP8 with one fp16 scale each per kv head; the last tile may be the fp16
// tail.  Per tile:
//   staging   K -> fp16 [64 keys][64 dims] (exact: scale 1 conversion),
//             V -> fp16 V^T [64 dims][64 key slots], times the group's V
//             scale (one fp16 rounding), both XOR-swizzled so that operand
//             reads and staging writes are free of LDS bank conflicts;
//   S^T = K Q^T on v_mfma_f32_16x16x32_f16 (A = K rows from LDS, B = Q^T
//             held in registers): a lane holds 16 keys x 1 query per
//             16-query tile, so the softmax max is per-lane work plus two
//             cross-lane steps;
//   softmax   exp2 of (s * K scale * scale * log2e - m), online, with the
//             running max only moved when a tile exceeds it by more than 8
//             (values stay below 2^8, so fp16 P and fp32 sums cannot
//             overflow); row sums by v_dot2_f32_f16 on the fp16 P;
//   O^T += V^T P^T on the matrix cores: the S^T registers, packed to fp16,
//             are the B operand as they stand; V^T slots are ordered to
//             match (slot 8b + e of 32-key block u holds key
//             32u + (e < 4 ? 4b + e : 16 + 4b + e - 4)).
// K/V of tile j+1 are loaded into registers while tile j is computed, and
// written to the second LDS buffer afterwards: one barrier per tile.
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
  st.k = *(const u32x2*)(a.kc8 + ((size_t)(64 * j + kkey) * NKV + g) * D + 8 * kch);
  const size_t v0 = (size_t)(64 * j + 2 * kp) * NKV + g;
  st.v0 = *(const uint32_t*)(a.vc8 + v0 * D + 4 * dc);
  st.v1 = *(const uint32_t*)(a.vc8 + (v0 + NKV) * D + 4 * dc);
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

// grid = 8 * ceil(nblk / 2), block = 512
__global__ __launch_bounds__(64 * kPfWaves) void k_prefill_mfma(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2 * kPfTileBytes];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, n = l & 15, b = l >> 4;
  const int g = blockIdx.x & 7, pr = blockIdx.x >> 3;
  const int h = g * GQA + (w & 3);
  const int nvalid_tail = a.past + a.S - a.committed;  // tail keys 0..63
  const int nfp8 = a.committed >> 6;
  // v_perm selectors of this lane's V^T word pairs (see pf_store)
  const uint32_t sel01 = ((tid >> 5) & 1) ? 0x07060302u : 0x05040100u;
  const uint32_t sel10 = ((tid >> 5) & 1) ? 0x05040100u : 0x07060302u;

  for (int phase = 0; phase < 2; phase++) {
    const int blk = phase == 0 ? a.nblk - 1 - pr : pr;
    if (phase == 1 && pr >= a.nblk - 1 - pr) break;  // the middle block runs once
    const int q0 = blk * kPfQ + 32 * (w >> 2);        // this wave's first query
    const int kend = a.past + min(a.S, (blk + 1) * kPfQ);  // keys 0..kend-1 for the block
    const int ntile = (kend + 63) >> 6;
    const int qmin = a.past + q0;                      // wave's first position
    const int qlast = a.past + min(q0 + 31, a.S - 1);  // wave's last valid position
    const bool wave_live = q0 < a.S;

    // Q^T as the B operand: lane (n, b) holds query q0 + 16 qt + n, dims 32 kb + 8 b .. +7
    f16x8 qop[2][2];
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
      const int s = q0 + 16 * qt + n;
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
        qop[qt][kb] = s < a.S ? *(const f16x8*)(a.q + ((size_t)s * NH + h) * D + 32 * kb + 8 * b)
                              : f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    }
    f32x4 O[4][2];
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
      for (int qt = 0; qt < 2; qt++) O[dt][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrun[2] = {-__builtin_inff(), -__builtin_inff()}, lrun[2] = {0.f, 0.f};

    // Q must have arrived before the loop: an explicit vmcnt(0) here keeps
    // the loop's waits for the K/V prefetch from covering it
    __builtin_amdgcn_s_waitcnt(0x0F70);

    // FP8 tiles 0..nf-1 with a two-deep prefetch, then at most one fp16
    // tail tile (the last one)
    const int nf = min(ntile, nfp8);
    const int qpos0 = a.past + q0 + n;
    PfStage8 s8;
    float c_cur = 1.0f, c_next = 1.0f;  // K scale of the tile being computed / staged
    if (nf > 0) {
      pf_load8(a, g, 0, tid, s8);
      c_cur = pf_scale(s8.ks);
      pf_store8(lds[0], tid, s8, sel01, sel10);
      if (nf > 1) pf_load8(a, g, 1, tid, s8);
    }
    __syncthreads();
    for (int j = 0; j < nf; j++) {
      // stage tile j+1 (loaded during tile j-1) into the free buffer, then
      // start loading tile j+2
      if (j + 1 < nf) {
        c_next = pf_scale(s8.ks);
        pf_store8(lds[(j + 1) & 1], tid, s8, sel01, sel10);
        if (j + 2 < nf) pf_load8(a, g, j + 2, tid, s8);
      }
      // tiles past the wave's last query are skipped (wave-uniform).  The
      // score multiplier is kept >= 1e-30 so that masked keys (-inf) stay
      // -inf when a group's K scale is 0 (its scores are then ~0, as they
      // should be).
      if (wave_live && 64 * j <= qlast) {
        const float c = __builtin_fmaxf(c_cur * a.qscale, 1e-30f);
        if (64 * j + 63 > qmin)
          pf_tile<true>(lds[j & 1], lds[j & 1] + kPfTileBytes, qop, c, j == 0, 64 * j, qpos0, n,
                        b, O, mrun, lrun);
        else
          pf_tile<false>(lds[j & 1], lds[j & 1] + kPfTileBytes, qop, c, j == 0, 64 * j, qpos0,
                         n, b, O, mrun, lrun);
      }
      c_cur = c_next;
      __syncthreads();
    }
    if (ntile > nf) {
      PfStage16 s16;
      pf_load16(a, g, nvalid_tail, tid, s16);
      pf_store16(lds[nf & 1], tid, s16, sel01, sel10);
      __syncthreads();
      if (wave_live && 64 * nf <= qlast)
        pf_tile<true>(lds[nf & 1], lds[nf & 1] + kPfTileBytes, qop,
                      __builtin_fmaxf(a.qscale, 1e-30f), nf == 0, 64 * nf, qpos0, n, b, O, mrun,
                      lrun);
      __syncthreads();
    }
    // ---- normalise and store: lane holds query q0 + 16 qt + n, dims 16 dt + 4 b .. +3
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
      const float L = pf_colsum(lrun[qt]);
      const int s = q0 + 16 * qt + n;
      if (s < a.S) {
        const float inv = 1.0f / L;
        uint16_t* op = a.out + ((size_t)s * NH + h) * D + 4 * b;
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

// Internal entry used by cia_attention_fused once its arguments are checked.
extern "C" __attribute__((visibility("hidden"))) int cia_prefill_mfma(
    const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8, const uint16_t* ksc,
    const uint16_t* vsc, const uint16_t* ktail, const uint16_t* vtail, int committed,
    uint16_t* out, int S, int past, float scale, void* stream) {
  const int nblk = (S + kPfQ - 1) / kPfQ;
  PrefillArgs pa{q, kc8, vc8, ksc, vsc, ktail, vtail, committed, out, S, past,
                 scale * kPfLog2e, nblk};
  hipLaunchKernelGGL(k_prefill_mfma, dim3(8 * ((nblk + 1) / 2)), dim3(64 * kPfWaves), 0,
                     (hipStream_t)stream, pa);
  return launch_status();
}
