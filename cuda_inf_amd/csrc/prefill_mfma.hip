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
// K/V of tile j+2 are loaded into registers while tile j is computed; tile
// j+1 (loaded during tile j-1) is written to the second LDS buffer after
// tile j's products, by waves 0-3 alone (of the two waves of a SIMD, the
// older one's products finish first): one barrier per tile.
#include "prefill_tile.h"

namespace cia {

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
    // waves 0-3 (the older wave of each SIMD, whose products finish first)
    // stage whole tiles: thread tid its own half and that of tid + 256;
    // waves 4-7 fetch only the group's K scale
    struct Stage2 {
      PfStage8 lo, hi;
    };
    const bool stager = w < 4;
    auto load2 = [&](int j, Stage2& st) {
      if (stager) {
        pf_load8(a, g, j, tid, st.lo);
        pf_load8(a, g, j, tid + 256, st.hi);
      } else {
        st.lo.ks = a.ksc[j * NKV + g];
      }
    };
    auto store2 = [&](uint8_t* buf, const Stage2& st) {
      if (stager) {
        pf_store8(buf, tid, st.lo, sel01, sel10);
        pf_store8(buf, tid + 256, st.hi, sel01, sel10);
      }
    };
    Stage2 sa, sb;
    float c_cur = 1.0f, c_next = 1.0f;  // K scale of the tile being computed / staged
    if (nf > 0) {
      load2(0, sa);
      c_cur = pf_scale(sa.lo.ks);
      store2(lds[0], sa);
      if (nf > 1) load2(1, sb);
    }
    __syncthreads();
    // tile j: start loading tile j+2 (into ld), compute tile j, then stage
    // tile j+1 (loaded during tile j-1, in st) into the free buffer, so a
    // wave that finishes its products early stages while the other wave of
    // its SIMD still computes
    auto step = [&](int j, Stage2& ld, Stage2& st) {
      if (j + 2 < nf) load2(j + 2, ld);
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
      __builtin_amdgcn_sched_barrier(0);
      if (j + 1 < nf) {
        c_next = pf_scale(st.lo.ks);
        store2(lds[(j + 1) & 1], st);
      }
      c_cur = c_next;
      __syncthreads();
    };
    for (int j = 0; j < nf; j += 2) {
      step(j, sa, sb);
      if (j + 1 < nf) step(j + 1, sb, sa);
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
