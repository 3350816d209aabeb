// gemv_int4.hip -- the attention layer's INT4 group-128 projections
// (gemv_int4, engine.cu:83-109, launched by run_gemv_int4 at 626-630 for
// q/k/v_proj at 792-797 and out_proj at 858) on gfx950.
//
// Weight format (tools/export_weights.py:64-79): packed u8 [N][K/2], k even
// in the low nibble, w = (nibble - 8) * scale[n][k/128], scales fp16.
//
// Few rows of x (decode): the launch is bound by the packed weights in HBM
// (N*K/2 bytes plus N*K/64 bytes of scales) and, at the attention layer's
// sizes (3 and 2 MiB), by latency.  One wave per weight row, 8 per
// workgroup; lane l reads 16-byte chunk l of the row (32 nibbles, k = 32l ..
// 32l+31, all inside group l/4) with one 128-bit load, so one instruction
// covers a 2048-wide row.  The workgroup stages its rows of x in LDS once
// (the weight loads are already in flight) and every lane reads its 64-byte
// slice from there; the four 16-byte pieces of a slice are rotated by
// (chunk >> 2) & 3 so that each read of a 16-lane pass hits 16 distinct
// bank groups.  A nibble pair becomes two exact fp16 values nibble - 8 by
// or-ing it under the exponent of 1024 (0x6400) and subtracting 1032;
// v_dot2_f32_f16 accumulates nibble * x in fp32, and the group scale
// multiplies each lane's 32-term sum once.  One DPP / permlane reduction per
// output.  (Measured at 3072 and 2048 rows: one row per wave beats 2, 4 or
// 8; the staged x beats per-wave x loads.)
#include "common.h"

namespace cia {

struct Int4Mat {
  const uint8_t* packed;  // [N][K/2]
  const uint16_t* scales; // [N][K/128]
  int N;
  float* y32;     // fp32 output [M][N], or null
  uint16_t* y16;  // fp16 output [M][N], or null
};

struct GemvArgs {
  const uint16_t* x;  // [M][K]
  int K, M;
  int add;   // y32 += sum instead of y32 = sum
  int rows;  // total weight rows over the matrices
  Int4Mat mat[3];  // rows of mat[1] follow those of mat[0], then mat[2]
};

constexpr int kGemvWaves = 8;
constexpr int kGemmMinM = 56;  // rows of x from which the matrix-core GEMM runs (measured crossover)

// nibbles sh..sh+3 and sh+16..sh+19 of w as fp16 (nibble - 8), exact
__device__ __forceinline__ f16x2 nib_pair(uint32_t w, int sh) {
  const uint32_t v = ((w >> sh) & 0x000F000Fu) | 0x64006400u;  // 1024 + nibble
  return __builtin_bit_cast(f16x2, v) - f16x2{(_Float16)1032.0f, (_Float16)1032.0f};
}

// The x pairs matching nib_pair(w_j, 0/4/8/12) of weight word j (k = 8j ..
// 8j+7): {x0, x4}, {x1, x5}, {x2, x6}, {x3, x7} out of the x words
// 4j..4j+3 (word i holds x[2i] low, x[2i+1] high).
__device__ __forceinline__ void x_pairs(const u32x4 (&xv)[4], f16x2 (&p)[16]) {
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const u32x4 X = xv[j];
    p[4 * j + 0] = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(X[2], X[0], 0x05040100u));
    p[4 * j + 1] = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(X[2], X[0], 0x07060302u));
    p[4 * j + 2] = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(X[3], X[1], 0x05040100u));
    p[4 * j + 3] = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(X[3], X[1], 0x07060302u));
  }
}

// sum over one 16-byte weight chunk of (nibble - 8) * x
__device__ __forceinline__ float chunk_dot(const u32x4& w, const f16x2 (&p)[16]) {
  float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    d0 = __builtin_amdgcn_fdot2(nib_pair(w[j], 0), p[4 * j + 0], d0, false);
    d1 = __builtin_amdgcn_fdot2(nib_pair(w[j], 4), p[4 * j + 1], d1, false);
    d0 = __builtin_amdgcn_fdot2(nib_pair(w[j], 8), p[4 * j + 2], d0, false);
    d1 = __builtin_amdgcn_fdot2(nib_pair(w[j], 12), p[4 * j + 3], d1, false);
  }
  return d0 + d1;
}

// LDS element offset of piece p (8 fp16) of chunk c of a staged x row
__device__ __forceinline__ int xs_off(int c, int p) { return c * 32 + 8 * ((p + (c >> 2)) & 3); }

// row of the staged block holding element e (no division: kM <= 4)
template <int kM>
__device__ __forceinline__ int stage_row(int e, int K) {
  int mm = 0;
#pragma unroll
  for (int j = 1; j < kM; j++) mm += e >= j * K ? 1 : 0;
  return mm;
}

// grid = (ceil(rows / kGemvWaves), ceil(M / kM)), block = 64 * kGemvWaves.
// kStage > 0: x rows m0..m0+kM-1 (kM * K <= kStage * 4096 elements) are
// staged in LDS; 0: every lane loads its x slices itself.
template <int kM, int kStage>
__global__ __launch_bounds__(64 * kGemvWaves) void k_gemv_int4(GemvArgs a) {
  constexpr int kPer = 8 * 64 * kGemvWaves;  // elements staged per pass
  // (+8: the drop slot of the stores past the block)
  __shared__ __attribute__((aligned(16))) uint16_t xs[kStage > 0 ? kStage * kPer + 8 : 8];
  const int l = threadIdx.x & 63;
  const int row = blockIdx.x * kGemvWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int m0 = blockIdx.y * kM;
  const int K = a.K, nch = K >> 5, ng = K >> 7;
  // this wave's row (uniform): matrix and local row; waves past the last
  // row read it again and write nothing
  int n = row < a.rows ? row : a.rows - 1, mi = 0;
  if (n >= a.mat[0].N) {
    n -= a.mat[0].N;
    mi = 1;
    if (n >= a.mat[1].N) {
      n -= a.mat[1].N;
      mi = 2;
    }
  }
  const uint8_t* packed = mi == 0 ? a.mat[0].packed : (mi == 1 ? a.mat[1].packed : a.mat[2].packed);
  const uint16_t* scales = mi == 0 ? a.mat[0].scales : (mi == 1 ? a.mat[1].scales : a.mat[2].scales);
  const uint8_t* wp = packed + (size_t)n * (K >> 1);
  const uint16_t* sp = scales + (size_t)n * ng;
  // Loads, all branch-free so that each wait counts exactly: x first
  // (elements past the block load element 0 and are dropped), then this
  // lane's first weight chunk and its scale (lanes past the row's last
  // chunk load that chunk and discard it).  The LDS stores wait only for
  // the x loads, and the barrier only for the LDS stores.
  u32x4 st[kStage > 0 ? kStage : 1];
  if constexpr (kStage > 0) {
#pragma unroll
    for (int i = 0; i < kStage; i++) {
      int e = i * kPer + (int)threadIdx.x * 8;
      e = e < kM * K ? e : 0;
      const int mm = stage_row<kM>(e, K);
      const int src = m0 + mm < a.M ? m0 + mm : a.M - 1;
      st[i] = *(const u32x4*)(a.x + (size_t)src * K + (e - mm * K));
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  const int c0 = l < nch ? l : nch - 1;
  u32x4 wv = *(const u32x4*)(wp + 16 * c0);
  uint32_t sv = sp[c0 >> 2];  // (32-bit holder: no early wait)
  float* y32 = mi == 0 ? a.mat[0].y32 : (mi == 1 ? a.mat[1].y32 : a.mat[2].y32);
  uint16_t* y16 = mi == 0 ? a.mat[0].y16 : (mi == 1 ? a.mat[1].y16 : a.mat[2].y16);
  const int N = mi == 0 ? a.mat[0].N : (mi == 1 ? a.mat[1].N : a.mat[2].N);
  // the residual (add): fetched with the weights, so the epilogue does not
  // wait a round trip for it (the wave's lanes share the address; without
  // add, a harmless read of x[0])
  float yold[kM];
#pragma unroll
  for (int m = 0; m < kM; m++) {
    const int mm = m0 + m < a.M ? m0 + m : a.M - 1;
    const float* ysrc = a.add && y32 ? y32 + (size_t)mm * N + n : (const float*)a.x;
    yold[m] = *ysrc;
  }
  if constexpr (kStage > 0) {
#pragma unroll
    for (int i = 0; i < kStage; i++) {
      const int e = i * kPer + (int)threadIdx.x * 8;
      const int mm = stage_row<kM>(e, K), k = e - mm * K;
      *(u32x4*)(xs + (e < kM * K ? mm * K + xs_off(k >> 5, (k >> 3) & 3) : kStage * kPer)) = st[i];
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS stores
    __builtin_amdgcn_s_barrier();
  }
  float acc[kM];
#pragma unroll
  for (int m = 0; m < kM; m++) acc[m] = 0.0f;
  for (int c = l; c < nch; c += 64) {
    if (c != l) {
      wv = *(const u32x4*)(wp + 16 * c);
      sv = sp[c >> 2];
    }
#pragma unroll
    for (int m = 0; m < kM; m++) {
      u32x4 xv[4];
      if constexpr (kStage > 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) xv[i] = *(const u32x4*)(xs + m * K + xs_off(c, i));
      } else {
        const uint16_t* xr = a.x + (size_t)(m0 + m < a.M ? m0 + m : a.M - 1) * K + 32 * c;
#pragma unroll
        for (int i = 0; i < 4; i++) xv[i] = *(const u32x4*)(xr + 8 * i);
      }
      f16x2 p[16];
      x_pairs(xv, p);
      acc[m] = __builtin_fmaf(chunk_dot(wv, p), h2f((uint16_t)sv), acc[m]);
    }
  }
#pragma unroll
  for (int m = 0; m < kM; m++) {
    const float v = wave_sum_fast(acc[m]);
    if (l == 0 && row < a.rows && m0 + m < a.M) {
      const size_t o = (size_t)(m0 + m) * N + n;
      if (y32) y32[o] = a.add ? yold[m] + v : v;
      if (y16) y16[o] = f2h(v);
    }
  }
}

// ---------------------------------------------------------------- GEMM
// Many rows of x (prefill): Y = X W^T on the fp16 matrix cores
// (v_mfma_f32_16x16x32_f16).  A workgroup computes a 128 (x rows) x 128
// (weight rows) tile with 8 waves (two per SIMD, so one wave's matrix
// products overlap another's dequantisation) in a 2 x 4 grid of 64 x 32
// wave tiles (4 x 2 MFMA tiles).  The K loop runs over the 128-wide scale groups: the
// products of one group accumulate from zero on the matrix cores and are
// then added with the group scale of their column in fp32, so the weights
// enter the MFMA as exact fp16 (nibble - 8) values.
//   Inside a group the k order of the four 32-k MFMA steps is permuted the
//   same way for both operands: lane group q = l >> 4 holds k = 32q + 8s ..
//   32q + 8s + 7 at step s, so one 16-byte read per lane and column tile
//   brings the nibbles of all four steps (word s is step s).
//   Operands reach LDS by DMA (global_load_lds_dwordx4: lane i's 16 bytes
//   land at the instruction's LDS base + 16 i, so the swizzles are made by
//   choosing which global chunk each lane fetches), in a ring of 3 slots
//   filled two groups ahead: per group one wait for the group's own DMA,
//   one barrier, and no staging registers.
//     X slot: 128 rows x 16 chunks; row r's chunk c at c ^ xsw(r).  A
//       16-byte read is served 32 lanes (512 bytes of banks) at a time:
//       lanes 16q + n (q = 0, 1 or 2, 3) read row n's chunks 4q + s, and
//       two rows of one parity share a 512-byte bank window, so xsw maps
//       the 8 rows of a parity to distinct offsets whose bit 2 is the
//       parity: chunk 4q + s of one q and of the other never land on one
//       bank (and the 16 rows of a read take 16 distinct offsets).
//     W slot: 128 columns x 4 chunks of nibbles; column c's chunk q at
//       q ^ ((c >> 2) & 3) (16 consecutive columns hit distinct banks).
//     scale slot: the 128 columns' fp16 scales of the group, one per dword
//       (a 2-byte LDS DMA writes each lane's value zero-extended to a dword).
constexpr int kTile = 128;
constexpr int kRing = 3;
constexpr int kGemmWaves = 8;
constexpr int kXSlot = kTile * 256;            // bytes: 128 rows x 128 fp16
constexpr int kWSlot = kTile * 64;             // bytes: 128 columns x 128 nibbles
constexpr int kSSlot = 2 * kTile * 4;          // bytes: 128 scale dwords + a drop area
constexpr int kSlot = kXSlot + kWSlot + kSSlot;

typedef __attribute__((address_space(3))) void lds_void_t;

// X slot chunk swizzle of row r: bits 1-2 of r to bits 0-1, bit 0 to bit 2,
// bit 3 stays
__device__ __forceinline__ int xsw(int r) { return ((r >> 1) & 3) | ((r & 1) << 2) | (r & 8); }
typedef __attribute__((address_space(1))) void gbl_void_t;

// 8 nibbles (one u32, k even in the low nibble) -> 8 fp16 (nibble - 8), in k order
__device__ __forceinline__ f16x8 nib8(uint32_t u) {
  const uint32_t x = u & 0x0F0F0F0Fu, y = (u >> 4) & 0x0F0F0F0Fu;
  const f16x2 off = f16x2{(_Float16)1032.0f, (_Float16)1032.0f};
  f16x8 r;
#pragma unroll
  for (int b = 0; b < 4; b++) {
    // {lo_b, hi_b} as 16-bit values, then under the exponent of 1024
    const uint32_t sel = 0x0C000C00u | (uint32_t)(4 + b) << 16 | (uint32_t)b;
    const f16x2 h =
        __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(y, x, sel) | 0x64006400u) - off;
    r[2 * b] = h[0];
    r[2 * b + 1] = h[1];
  }
  return r;
}

// weight row of global column col (clamped), across the up to 3 matrices
struct ColRef {
  const uint8_t* packed;
  const uint16_t* scales;
};
__device__ __forceinline__ ColRef col_ref(const GemvArgs& a, int col, int K) {
  int n = col < a.rows ? col : a.rows - 1, mi = 0;
  if (n >= a.mat[0].N) {
    n -= a.mat[0].N;
    mi = 1;
    if (n >= a.mat[1].N) {
      n -= a.mat[1].N;
      mi = 2;
    }
  }
  const uint8_t* pk = mi == 0 ? a.mat[0].packed : (mi == 1 ? a.mat[1].packed : a.mat[2].packed);
  const uint16_t* sc = mi == 0 ? a.mat[0].scales : (mi == 1 ? a.mat[1].scales : a.mat[2].scales);
  return ColRef{pk + (size_t)n * (K >> 1), sc + (size_t)n * (K >> 7)};
}

// grid = (ceil(rows / 128), ceil(M / 128)), block = 64 * kGemmWaves.
// (Giving each XCD a contiguous run of tiles, so its L2 sees a few row
// blocks of X rather than all, measured no faster.)
__global__ __launch_bounds__(64 * kGemmWaves) void k_gemm_int4(GemvArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[kRing * kSlot];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int wm = w >> 2, wn = w & 3, n16 = l & 15, q = l >> 4;
  const int m0 = blockIdx.y * kTile, r0 = blockIdx.x * kTile;
  const int K = a.K, ng = K >> 7;
  // DMA sources of this lane (fixed across groups; + 256 g bytes for X,
  // + 64 g for W, + 2 g for the scales)
  //   X: instruction t of wave w fills rows 4 (4w + t) .. +3; lane l takes
  //      row 4 (4w + t) + (l >> 4), physical chunk l & 15
  const uint8_t* xsrc[4];
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const int r = 4 * (4 * w + t) + (l >> 4), m = m0 + r;
    const int lc = (l & 15) ^ xsw(r);
    xsrc[t] = (const uint8_t*)(a.x + (size_t)(m < a.M ? m : a.M - 1) * K) + 16 * lc;
  }
  //   W: wave w fills columns 16 w .. +15; lane l takes column 16 w + (l >> 2),
  //      physical chunk l & 3
  const int wcol = 16 * w + (l >> 2);
  const uint8_t* wsrc = col_ref(a, r0 + wcol, K).packed + 16 * ((l & 3) ^ ((wcol >> 2) & 3));
  //   scales: waves 0, 1 fill columns 64 w + l; the others the drop area
  const uint16_t* ssrc = col_ref(a, r0 + 64 * (w & 1) + l, K).scales;
  const int sdst = kXSlot + kWSlot + (w < 2 ? 256 * w : 512);
  auto issue = [&](int g) {
    uint8_t* slot = ring + (g % kRing) * kSlot;
    const int gg = g < ng ? g : ng - 1;  // past the end: a harmless refetch
#pragma unroll
    for (int t = 0; t < 4; t++)
      __builtin_amdgcn_global_load_lds((gbl_void_t*)(xsrc[t] + 256 * gg),
                                       (lds_void_t*)(slot + (4 * w + t) * 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((gbl_void_t*)(wsrc + 64 * gg),
                                     (lds_void_t*)(slot + kXSlot + w * 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((gbl_void_t*)(ssrc + gg), (lds_void_t*)(slot + sdst), 2, 0,
                                     0);
  };
  f32x4 C[4][2];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) C[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  issue(0);
  issue(1);
  for (int g = 0; g < ng; g++) {
    // this group's 6 DMAs are done once at most the next group's 6 remain
    __builtin_amdgcn_s_waitcnt(0x0F76);  // vmcnt(6)
    __builtin_amdgcn_s_barrier();        // every wave's DMA landed; slot g-1 is free
    issue(g + 2);
    const uint8_t* slot = ring + (g % kRing) * kSlot;
    const uint16_t* xs = (const uint16_t*)slot;
    const uint8_t* ws = slot + kXSlot;
    const uint32_t* ss = (const uint32_t*)(slot + kXSlot + kWSlot);
    u32x4 wq[2];
    float scl[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int c = 32 * wn + 16 * j + n16;
      wq[j] = *(const u32x4*)(ws + c * 64 + 16 * (q ^ ((c >> 2) & 3)));
      scl[j] = h2f((uint16_t)ss[c]);
    }
    f32x4 P[4][2];
#pragma unroll
    for (int s2 = 0; s2 < 4; s2++) {
      f16x8 A[4], B[2];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = 64 * wm + 16 * i + n16;
        A[i] = *(const f16x8*)(xs + r * 128 + 8 * ((4 * q + s2) ^ xsw(n16)));
      }
#pragma unroll
      for (int j = 0; j < 2; j++) B[j] = nib8(wq[j][s2]);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
          P[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              A[i], B[j], s2 == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : P[i][j], 0, 0, 0);
    }
    // C += P * scale of the column (the lane's column is n16 of tile j)
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) C[i][j][e] = __builtin_fmaf(P[i][j][e], scl[j], C[i][j][e]);
  }
  // outputs: lane holds rows 4q + e of tile i, column n16 of tile j
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int col = r0 + 32 * wn + 16 * j + n16;
    if (col >= a.rows) continue;
    int n = col, mi = 0;
    if (n >= a.mat[0].N) {
      n -= a.mat[0].N;
      mi = 1;
      if (n >= a.mat[1].N) {
        n -= a.mat[1].N;
        mi = 2;
      }
    }
    float* y32 = mi == 0 ? a.mat[0].y32 : (mi == 1 ? a.mat[1].y32 : a.mat[2].y32);
    uint16_t* y16 = mi == 0 ? a.mat[0].y16 : (mi == 1 ? a.mat[1].y16 : a.mat[2].y16);
    const int N = mi == 0 ? a.mat[0].N : (mi == 1 ? a.mat[1].N : a.mat[2].N);
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int m = m0 + 64 * wm + 16 * i + 4 * q + e;
        if (m >= a.M) continue;
        const size_t o = (size_t)m * N + n;
        const float v = C[i][j][e];
        if (y32) y32[o] = a.add ? y32[o] + v : v;
        if (y16) y16[o] = f2h(v);
      }
  }
  // (the last two DMAs refetch the final group into free slots; let them
  // land before the workgroup's LDS is released)
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
}

template <int kM>
static void gemv_launch(const GemvArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)((a.rows + kGemvWaves - 1) / kGemvWaves),
                  (unsigned)((a.M + kM - 1) / kM));
  const dim3 block(64 * kGemvWaves);
  const int per = 8 * 64 * kGemvWaves, need = (kM * a.K + per - 1) / per;
  if (need <= 1)
    hipLaunchKernelGGL((k_gemv_int4<kM, 1>), grid, block, 0, s, a);
  else if (need <= 2)
    hipLaunchKernelGGL((k_gemv_int4<kM, 2>), grid, block, 0, s, a);
  else if (need <= 4)
    hipLaunchKernelGGL((k_gemv_int4<kM, 4>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((k_gemv_int4<kM, 0>), grid, block, 0, s, a);
}

static int gemv_run(GemvArgs& a, void* stream) {
  a.rows = a.mat[0].N + a.mat[1].N + a.mat[2].N;
  hipStream_t s = (hipStream_t)stream;
  if (a.M >= kGemmMinM) {
    hipLaunchKernelGGL(k_gemm_int4, dim3((unsigned)((a.rows + kTile - 1) / kTile),
                       (unsigned)((a.M + kTile - 1) / kTile)), dim3(64 * kGemmWaves), 0, s, a);
  } else if (a.M == 1)
    gemv_launch<1>(a, s);
  else if (a.M == 2)
    gemv_launch<2>(a, s);
  else
    gemv_launch<4>(a, s);
  return launch_status();
}

static bool mat_ok(const uint8_t* packed, const uint16_t* scales) {
  return aligned(packed, 16) && aligned(scales, 2);
}

}  // namespace cia

using namespace cia;

static int gemv_common(const uint16_t* x, const uint8_t* packed, const uint16_t* scales, float* y,
                       int N, int K, int M, int add, void* stream) {
  CIA_REQUIRE(N > 0 && K > 0 && K % 128 == 0 && M >= 0, CIA_ERR_ARG);
  if (M == 0) return CIA_OK;
  CIA_REQUIRE(x && packed && scales && y, CIA_ERR_NULL);
  CIA_REQUIRE(aligned(x, 16) && mat_ok(packed, scales) && aligned(y, 4), CIA_ERR_ALIGN);
  GemvArgs a{};
  a.x = x;
  a.K = K;
  a.M = M;
  a.add = add;
  a.mat[0] = Int4Mat{packed, scales, N, y, nullptr};
  return gemv_run(a, stream);
}

extern "C" int cia_gemv_int4(const uint16_t* x, const uint8_t* packed, const uint16_t* scales,
                             float* y, int N, int K, int M, void* stream) {
  return gemv_common(x, packed, scales, y, N, K, M, 0, stream);
}

extern "C" int cia_gemv_int4_add(const uint16_t* x, const uint8_t* packed,
                                 const uint16_t* scales, float* y, int N, int K, int M,
                                 void* stream) {
  return gemv_common(x, packed, scales, y, N, K, M, 1, stream);
}

extern "C" int cia_qkv_proj_int4(const uint16_t* x, const uint8_t* wq_packed,
                                 const uint16_t* wq_scales, int Nq, const uint8_t* wk_packed,
                                 const uint16_t* wk_scales, const uint8_t* wv_packed,
                                 const uint16_t* wv_scales, int Nkv, int K, int M, uint16_t* q,
                                 uint16_t* k, uint16_t* v, void* stream) {
  CIA_REQUIRE(Nq > 0 && Nkv > 0 && K > 0 && K % 128 == 0 && M >= 0, CIA_ERR_ARG);
  if (M == 0) return CIA_OK;
  CIA_REQUIRE(x && wq_packed && wq_scales && wk_packed && wk_scales && wv_packed && wv_scales &&
                  q && k && v,
              CIA_ERR_NULL);
  CIA_REQUIRE(aligned(x, 16) && mat_ok(wq_packed, wq_scales) && mat_ok(wk_packed, wk_scales) &&
                  mat_ok(wv_packed, wv_scales) && aligned(q, 2) && aligned(k, 2) && aligned(v, 2),
              CIA_ERR_ALIGN);
  GemvArgs a{};
  a.x = x;
  a.K = K;
  a.M = M;
  a.mat[0] = Int4Mat{wq_packed, wq_scales, Nq, nullptr, q};
  a.mat[1] = Int4Mat{wk_packed, wk_scales, Nkv, nullptr, k};
  a.mat[2] = Int4Mat{wv_packed, wv_scales, Nkv, nullptr, v};
  return gemv_run(a, stream);
}
