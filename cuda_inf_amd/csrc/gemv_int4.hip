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
constexpr int kGemmMinM = 80;  // rows of x from which the matrix-core GEMM runs (measured crossover)

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
  float* y32 = mi == 0 ? a.mat[0].y32 : (mi == 1 ? a.mat[1].y32 : a.mat[2].y32);
  uint16_t* y16 = mi == 0 ? a.mat[0].y16 : (mi == 1 ? a.mat[1].y16 : a.mat[2].y16);
  const int N = mi == 0 ? a.mat[0].N : (mi == 1 ? a.mat[1].N : a.mat[2].N);
#pragma unroll
  for (int m = 0; m < kM; m++) {
    const float v = wave_sum_fast(acc[m]);
    if (l == 0 && row < a.rows && m0 + m < a.M) {
      const size_t o = (size_t)(m0 + m) * N + n;
      if (y32) y32[o] = a.add ? y32[o] + v : v;
      if (y16) y16[o] = f2h(v);
    }
  }
}

// ---------------------------------------------------------------- GEMM
// Many rows of x (prefill): Y = X W^T on the fp16 matrix cores
// (v_mfma_f32_16x16x32_f16).  A workgroup computes a 128 (x rows) x 128
// (weight rows) tile with 4 waves in a 2 x 2 grid of 64 x 64 wave tiles
// (4 x 4 MFMA tiles).  The K loop runs over the 128-wide scale groups: the
// products of one group accumulate from zero on the matrix cores and are
// then added with the group scale of their column in fp32, so the weights
// enter the MFMA as exact fp16 (nibble - 8) values.
//   Inside a group the k order of the four 32-k MFMA steps is permuted the
//   same way for both operands: lane group q = l >> 4 holds k = 32q + 8s ..
//   32q + 8s + 7 at step s.  So one 16-byte load per lane and column tile
//   brings the nibbles of all four steps (k = 32q .. 32q+31), word s being
//   step s.
//   X tiles go through LDS (two buffers, 32 KiB each): row r, 16-byte chunk
//   c at chunk c ^ (r & 15), so the 16 rows of an MFMA read hit distinct
//   banks.  The next group's X and weights are loaded while this group
//   computes; one barrier per group.
constexpr int kTile = 128;

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

// grid = (ceil(rows / 128), ceil(M / 128)), block = 256
__global__ __launch_bounds__(256) void k_gemm_int4(GemvArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][kTile * 128];
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int wm = w >> 1, wn = w & 1, n16 = l & 15, q = l >> 4;
  const int m0 = blockIdx.y * kTile, r0 = blockIdx.x * kTile;
  const int K = a.K, ng = K >> 7;
  // this lane's weight row in each of the wave's 4 column tiles
  const uint8_t* wrow[4];
  const uint16_t* srow[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    int n = r0 + 64 * wn + 16 * j + n16;
    n = n < a.rows ? n : a.rows - 1;
    int mi = 0;
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
    wrow[j] = pk + (size_t)n * (K >> 1) + 16 * q;
    srow[j] = sc + (size_t)n * ng;
  }
  // X staging: pass p moves rows 16p + (tid >> 4), chunk tid & 15
  const int sr = tid >> 4, sc16 = tid & 15;
  const uint16_t* xrow[8];
#pragma unroll
  for (int p = 0; p < 8; p++) {
    const int m = m0 + 16 * p + sr;
    xrow[p] = a.x + (size_t)(m < a.M ? m : a.M - 1) * K + 8 * sc16;
  }
  const int xdst = sr * 128 + 8 * (sc16 ^ (sr & 15));  // + 16 * 128 * p
  u32x4 xv[8], wv[4];
  uint32_t sv[4];
  auto load = [&](int g) {
#pragma unroll
    for (int p = 0; p < 8; p++) xv[p] = *(const u32x4*)(xrow[p] + 128 * g);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      wv[j] = *(const u32x4*)(wrow[j] + 64 * g);
      sv[j] = srow[j][g];
    }
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int p = 0; p < 8; p++) *(u32x4*)(&xs[buf][16 * 128 * p + xdst]) = xv[p];
  };
  f32x4 C[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) C[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  load(0);
  stage(0);
  __syncthreads();
  for (int g = 0; g < ng; g++) {
    const int buf = g & 1;
    u32x4 wc[4];
    float scl[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      wc[j] = wv[j];
      scl[j] = h2f((uint16_t)sv[j]);
    }
    if (g + 1 < ng) load(g + 1);
    f32x4 P[4][4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
      f16x8 A[4], B[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = 64 * wm + 16 * i + n16;
        A[i] = *(const f16x8*)(&xs[buf][r * 128 + 8 * ((4 * q + s) ^ n16)]);
      }
#pragma unroll
      for (int j = 0; j < 4; j++) B[j] = nib8(wc[j][s]);
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
          P[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              A[i], B[j], s == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : P[i][j], 0, 0, 0);
    }
    // C += P * scale of the column (the lane's column is n16 of tile j)
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int e = 0; e < 4; e++) C[i][j][e] = __builtin_fmaf(P[i][j][e], scl[j], C[i][j][e]);
    if (g + 1 < ng) {
      stage(buf ^ 1);
      __syncthreads();
    }
  }
  // outputs: lane holds rows 4q + e of tile i, column n16 of tile j
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int col = r0 + 64 * wn + 16 * j + n16;
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
                       (unsigned)((a.M + kTile - 1) / kTile)), dim3(256), 0, s, a);
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
