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
constexpr float kPfLazy = 8.0f;     // log2 headroom before the running max moves

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
// .. +7; V keys 2 (tid & 31) and +1, dims 4 (tid >> 5) .. +3.
struct PfStage {
  u32x4 k;        // 8 fp8 bytes (k.x, k.y) or 8 fp16 values
  u32x2 v0, v1;   // 4 fp8 bytes (v0.x) or 4 fp16 values, keys 2kp and 2kp+1
  uint16_t vs;    // V scale (fp16 bits); 0x3C00 = 1 for the tail
  bool fp8;
};

__device__ __forceinline__ void pf_load(const PrefillArgs& a, int g, int j, int nvalid, int tid,
                                        PfStage& st) {
  const int kkey = tid >> 3, kch = tid & 7, kp = tid & 31, dc = tid >> 5;
  st.fp8 = (j << 6) < a.committed;
  if (st.fp8) {
    const size_t kb = (size_t)(64 * j + kkey) * NKV + g;
    const u32x2 kk = *(const u32x2*)(a.kc8 + kb * D + 8 * kch);
    st.k = u32x4{kk[0], kk[1], 0u, 0u};
    const size_t v0 = (size_t)(64 * j + 2 * kp) * NKV + g;
    st.v0 = u32x2{*(const uint32_t*)(a.vc8 + v0 * D + 4 * dc), 0u};
    st.v1 = u32x2{*(const uint32_t*)(a.vc8 + (v0 + NKV) * D + 4 * dc), 0u};
    st.vs = a.vsc[j * NKV + g];
  } else {
    // tail rows 0..nvalid-1 (keys committed..); others stage as zeros
    const u32x4 z4 = u32x4{0u, 0u, 0u, 0u};
    const u32x2 z2 = u32x2{0u, 0u};
    st.k = kkey < nvalid ? *(const u32x4*)(a.ktail + ((size_t)kkey * NKV + g) * D + 8 * kch) : z4;
    st.v0 = 2 * kp < nvalid
                ? *(const u32x2*)(a.vtail + ((size_t)(2 * kp) * NKV + g) * D + 4 * dc) : z2;
    st.v1 = 2 * kp + 1 < nvalid
                ? *(const u32x2*)(a.vtail + ((size_t)(2 * kp + 1) * NKV + g) * D + 4 * dc) : z2;
    st.vs = 0x3C00;
  }
}

__device__ __forceinline__ void pf_store(uint8_t* buf, int tid, const PfStage& st) {
  const int kkey = tid >> 3, kch = tid & 7, kp = tid & 31, dc = tid >> 5;
  u32x4 kw = st.k;
  f16x4 va, vb;
  if (st.fp8) {
    kw = __builtin_bit_cast(u32x4, pf_cvt8(st.k[0], st.k[1]));
    const _Float16 s = __builtin_bit_cast(_Float16, st.vs);
    const f16x2 s2 = f16x2{s, s};
    const f16x2 a0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(st.v0[0], 1.0f, false) * s2;
    const f16x2 a1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(st.v0[0], 1.0f, true) * s2;
    const f16x2 b0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(st.v1[0], 1.0f, false) * s2;
    const f16x2 b1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(st.v1[0], 1.0f, true) * s2;
    va = f16x4{a0[0], a0[1], a1[0], a1[1]};
    vb = f16x4{b0[0], b0[1], b1[0], b1[1]};
  } else {
    va = __builtin_bit_cast(f16x4, st.v0);
    vb = __builtin_bit_cast(f16x4, st.v1);
  }
  *(u32x4*)(buf + pf_kaddr(kkey, kch)) = kw;
  // V^T: dims 4dc + e, the pair (key 2kp, key 2kp+1) as one 32-bit word;
  // the upper half-wave writes its dims in the order 1,0,3,2 (bank spread)
  const int slot = pf_vslot(2 * kp);
  const int flip = (tid >> 5) & 1;
  uint8_t* vt = buf + kPfTileBytes;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int ee = e ^ flip;
    const _Float16 x0 = flip ? va[e ^ 1] : va[e];
    const _Float16 x1 = flip ? vb[e ^ 1] : vb[e];
    const uint32_t word = (uint32_t)__builtin_bit_cast(uint16_t, x0) |
                          ((uint32_t)__builtin_bit_cast(uint16_t, x1) << 16);
    *(uint32_t*)(vt + pf_vaddr(4 * dc + ee, slot)) = word;
  }
}

// grid = 8 * ceil(nblk / 2), block = 512
__global__ __launch_bounds__(64 * kPfWaves) void k_prefill_mfma(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[2][2 * kPfTileBytes];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63, n = l & 15, b = l >> 4;
  const int g = blockIdx.x & 7, pr = blockIdx.x >> 3;
  const int h = g * GQA + (w & 3);
  const int nvalid_tail = a.past + a.S - a.committed;  // tail keys 0..63

  for (int phase = 0; phase < 2; phase++) {
    const int blk = phase == 0 ? a.nblk - 1 - pr : pr;
    if (phase == 1 && pr >= a.nblk - 1 - pr) break;  // the middle block runs once
    const int q0 = blk * kPfQ + 32 * (w >> 2);        // this wave's first query
    const int kend = a.past + min(a.S, (blk + 1) * kPfQ);  // keys 0..kend-1 for the block
    const int ntile = (kend + 63) >> 6;
    const int qmin = a.past + q0;                                 // wave's first position
    const int qlast = a.past + min(q0 + 31, a.S - 1);             // wave's last valid position
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

    PfStage st;
    pf_load(a, g, 0, nvalid_tail, tid, st);
    pf_store(lds[0], tid, st);
    __syncthreads();
    for (int j = 0; j < ntile; j++) {
      if (j + 1 < ntile) pf_load(a, g, j + 1, nvalid_tail, tid, st);
      const uint8_t* kt_lds = lds[j & 1];
      const uint8_t* vt_lds = lds[j & 1] + kPfTileBytes;
      // tiles past the wave's last query are skipped (wave-uniform)
      if (wave_live && 64 * j <= qlast) {
        // score multiplier; kept >= 1e-30 so that masked keys (-inf) stay
        // -inf when a group's K scale is 0 (its scores are then ~0, as they
        // should be)
        const float c = __builtin_fmaxf(
            (64 * j < a.committed ? h2f(a.ksc[j * NKV + g]) : 1.0f) * a.qscale, 1e-30f);
        // ---- S^T = K Q^T: Sc[kt][qt] rows = keys 16 kt + 4 b + i, column = query n
        f32x4 Sc[4][2];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
          Sc[kt][0] = Sc[kt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kb = 0; kb < 2; kb++) {
            const f16x8 kop = *(const f16x8*)(kt_lds + pf_kaddr(16 * kt + n, 4 * kb + b));
#pragma unroll
            for (int qt = 0; qt < 2; qt++)
              Sc[kt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kop, qop[qt][kb], Sc[kt][qt], 0, 0, 0);
          }
        }
        // ---- causal mask (only tiles that reach past the wave's first query)
        const bool diag = 64 * j + 63 > qmin;
        if (diag) {
#pragma unroll
          for (int qt = 0; qt < 2; qt++) {
            const int qpos = a.past + q0 + 16 * qt + n;
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
              for (int i = 0; i < 4; i++)
                if (64 * j + 16 * kt + 4 * b + i > qpos) Sc[kt][qt][i] = -__builtin_inff();
          }
        }
        // ---- tile max per query column, lazily moved running max
        float mt[2];
        bool need[2];
#pragma unroll
        for (int qt = 0; qt < 2; qt++) {
          float cm = __builtin_fmaxf(__builtin_fmaxf(Sc[0][qt][0], Sc[0][qt][1]),
                                     __builtin_fmaxf(Sc[0][qt][2], Sc[0][qt][3]));
#pragma unroll
          for (int kt = 1; kt < 4; kt++)
            cm = __builtin_fmaxf(cm, __builtin_fmaxf(__builtin_fmaxf(Sc[kt][qt][0], Sc[kt][qt][1]),
                                                     __builtin_fmaxf(Sc[kt][qt][2], Sc[kt][qt][3])));
          cm = __builtin_fmaxf(cm, __shfl_xor(cm, 16));
          cm = __builtin_fmaxf(cm, __shfl_xor(cm, 32));
          mt[qt] = cm == -__builtin_inff() ? cm : cm * c;
          need[qt] = mt[qt] > mrun[qt] + kPfLazy;
        }
        if (__any(need[0] || need[1])) {
#pragma unroll
          for (int qt = 0; qt < 2; qt++) {
            const float corr = need[qt] ? __builtin_amdgcn_exp2f(mrun[qt] - mt[qt]) : 1.0f;
            if (need[qt]) mrun[qt] = mt[qt];
            lrun[qt] *= corr;
#pragma unroll
            for (int dt = 0; dt < 4; dt++)
#pragma unroll
              for (int i = 0; i < 4; i++) O[dt][qt][i] *= corr;
          }
        }
        // ---- P (fp16), row sums, O^T += V^T P^T
        f16x8 pop[2][2];  // [key block u][qt]
#pragma unroll
        for (int qt = 0; qt < 2; qt++) {
          const float nm = -mrun[qt];
#pragma unroll
          for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++)
              pop[kt >> 1][qt][4 * (kt & 1) + i] =
                  (_Float16)__builtin_amdgcn_exp2f(__builtin_fmaf(Sc[kt][qt][i], c, nm));
          float rs = lrun[qt];
#pragma unroll
          for (int u = 0; u < 2; u++)
#pragma unroll
            for (int e = 0; e < 4; e++)
              rs = __builtin_amdgcn_fdot2(f16x2{pop[u][qt][2 * e], pop[u][qt][2 * e + 1]},
                                          f16x2{(_Float16)1.0f, (_Float16)1.0f}, rs, false);
          lrun[qt] = rs;
        }
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
          for (int u = 0; u < 2; u++) {
            const f16x8 vop = *(const f16x8*)(vt_lds + pf_vaddr(16 * dt + n, 32 * u + 8 * b));
#pragma unroll
            for (int qt = 0; qt < 2; qt++)
              O[dt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop[u][qt], O[dt][qt], 0, 0, 0);
          }
      }
      if (j + 1 < ntile) pf_store(lds[(j + 1) & 1], tid, st);
      __syncthreads();
    }
    // ---- normalise and store: lane holds query q0 + 16 qt + n, dims 16 dt + 4 b .. +3
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
      float L = lrun[qt];
      L += __shfl_xor(L, 16);
      L += __shfl_xor(L, 32);
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
