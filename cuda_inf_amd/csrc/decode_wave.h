// decode_wave.h -- pieces shared by the matrix-core decode kernels
// (decode_kv.hip: one layer per launch; decode_tok.hip: every layer of a
// token in one launch): the FP8 wave's LDS unit geometry, the partial-state
// rows and the workspace layout, operand conversions and cross-lane steps,
// LDS transposing reads, buffer resources, the publication of a partial to
// other workgroups, and the host-side choice of key ranges.
#pragma once

#include <algorithm>

#include "common.h"

namespace cia {

constexpr int kFpWaves = 8;                // FP8 waves per workgroup
constexpr int kMaxRanges = 44;             // workgroups per kv head (32 on average)
constexpr int kBlkB = 16 * 64 + 16;        // 16 keys x 64 B + 16 B pad
constexpr int kTileB = 4 * kBlkB;          // one 64-key group of one kv head
constexpr int kHalfB = 2 * kTileB;         // K (or V) of a unit
constexpr int kScaleB = 256;               // K (or V) scales of a unit: 64 dwords, 2 used
constexpr int kPartRow = 4 + D;            // one head's partial: m, l, -, -, o[64]
constexpr int kPartF = GQA * kPartRow;     // floats of one workgroup partial
constexpr int kCntStride = 64;             // uint32 between two counters (256 B)
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLn2 = 0.69314718055994530942f;

// Decode workspace (cia_decode_workspace_bytes):
//   partials  f32 [8 kv heads][kMaxRanges][4 heads][kPartRow]
//   counters of the one-layer decode: [8 kv heads], kCntStride apart
//   multi-layer decode: tickets [kTokMaxLayers][8 kv heads][4 heads] and
//   layer-done counters [kTokMaxLayers], kCntStride apart, a fault word,
//   then one go word per workgroup (kTokGoStride apart)
// Every counter and go word is zero between calls; the fault word is sticky.
constexpr int kTokMaxLayers = 8;
constexpr int64_t kPartBytes = (int64_t)NKV * kMaxRanges * kPartF * sizeof(float);
constexpr int64_t kCntBytes = (int64_t)NKV * kCntStride * sizeof(uint32_t);
constexpr int64_t kTokTickOff = kPartBytes + kCntBytes;
constexpr int64_t kTokDoneOff = kTokTickOff + (int64_t)kTokMaxLayers * NKV * GQA * kCntStride * 4;
constexpr int64_t kTokErrOff = kTokDoneOff + (int64_t)kTokMaxLayers * kCntStride * 4;
// per-workgroup go words of the multi-layer decode, 128 B apart
constexpr int kTokGoStride = 32;
constexpr int64_t kTokGoOff = kTokErrOff + kCntStride * 4;
constexpr int64_t kWsBytes = kTokGoOff + (int64_t)NKV * kMaxRanges * kTokGoStride * 4;

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void gbl_void_t;

__device__ __forceinline__ f16x8 cvt8(uint32_t w0, uint32_t w1) {
  const f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false);
  const f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true);
  const f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false);
  const f16x2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true);
  return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// max / sum over the 16 lanes of one head (lane bits 2..5; bits 0, 1 = head)
__device__ __forceinline__ float head_max(float v) {
  v = __builtin_fmaxf(v, row_ror<4>(v));
  v = __builtin_fmaxf(v, row_ror<8>(v));
  return col4_max(v);
}
__device__ __forceinline__ float head_sum(float v) {
  v += row_ror<4>(v);
  v += row_ror<8>(v);
  return col4_sum(v);
}

// ds_read_b64_tr_b8 (within each 16-lane block, lane i receives byte i mod 8
// of the 8-byte rows addressed by lanes 2k + (i div 8), k = 0..7), issued as
// inline assembly: the compiler treats the builtin as touching every LDS
// byte a pending DMA may write and would wait for all of them.  The result is
// used only after lds_wait4.
template <int kOff>
__device__ __forceinline__ u32x2 ds_read_tr8_at(const uint8_t* p) {
  u32x2 v;
  asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2"
               : "=v"(v)
               : "v"((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p), "i"(kOff));
  return v;
}
#define ds_read_tr8(p, off) ds_read_tr8_at<off>(p)
// waits for the LDS reads above and ties their results to the wait, so no
// use is scheduled before it
__device__ __forceinline__ void lds_wait4(u32x2& a, u32x2& b, u32x2& c, u32x2& d) {
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}
// the same, leaving the kN LDS reads issued after these four in flight (LDS
// reads complete in order; another pending lgkm operation only makes the
// wait longer)
template <int kN>
__device__ __forceinline__ void lds_wait4_but(u32x2& a, u32x2& b, u32x2& c, u32x2& d) {
  asm volatile("s_waitcnt lgkmcnt(%4)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d) : "i"(kN));
}

// P V of one unit into T (zeroed by the caller): in product mu the k-group
// c of V^T holds key block (c + mu) & 3, so A = P on the lanes whose block
// that is and zero elsewhere; V^T comes from LDS at vw + vrd[mu] through
// the transposing read.  The reads of two products are in flight at once,
// each product issued as soon as its four reads are in.
__device__ __forceinline__ void unit_pv(f32x4 (&T)[4], const f16x8& P, const uint8_t* vw, const int (&vrd)[4],
                                        int n, int c) {
  const f16x8 zero8 = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
  u32x2 rw[4][4];
  auto rd = [&](int mu) __attribute__((always_inline)) {
    rw[mu][0] = ds_read_tr8(vw + vrd[mu], 0);
    rw[mu][1] = ds_read_tr8(vw + vrd[mu], 16);
    rw[mu][2] = ds_read_tr8(vw + vrd[mu], 32);
    rw[mu][3] = ds_read_tr8(vw + vrd[mu], 48);
  };
  auto mma = [&](int mu) __attribute__((always_inline)) {
    const f16x8 A = ((n >> 2) == ((c + mu) & 3)) ? P : zero8;
#pragma unroll
    for (int j = 0; j < 4; j++)
      T[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, cvt8(rw[mu][j][0], rw[mu][j][1]), T[j], 0, 0, 0);
  };
  rd(0);
  rd(1);
  lds_wait4_but<4>(rw[0][0], rw[0][1], rw[0][2], rw[0][3]);
  mma(0);
  rd(2);
  lds_wait4_but<4>(rw[1][0], rw[1][1], rw[1][2], rw[1][3]);
  mma(1);
  rd(3);
  lds_wait4_but<4>(rw[2][0], rw[2][1], rw[2][2], rw[2][3]);
  mma(2);
  lds_wait4(rw[3][0], rw[3][1], rw[3][2], rw[3][3]);
  mma(3);
}

// Publishing a partial to the other workgroups: its agent-coherent stores
// (relaxed agent-scope atomics) are acknowledged -- vmcnt(0): a store's
// count drops when the L2 of this XCD has written it through -- before the
// caller's barrier and its relaxed ticket increment, which another
// workgroup's coherent loads then follow.  The wait builtin has no memory
// semantics for the compiler, so compiler-only fences (no instruction) keep
// the stores above it and the ticket below it.
__device__ __forceinline__ void stores_acked() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  asm volatile("" ::: "memory");
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// A polled word read on the scalar path: one s_load_dword with glc (a miss
// in the scalar cache, read from L2), then its wait.  The vector memory
// requests of a compute unit are served in order, so a vector poll waits
// behind the DMAs the workgroup's other waves have just sent; this load
// does not.  The word is written by agent-coherent stores from any XCD;
// the caller's wait is bounded and records a fault if the value never
// arrives.  p must be uniform and 4-byte aligned.
__device__ __forceinline__ uint32_t scalar_poll(const uint32_t* p) {
  uint32_t v;
  asm volatile("s_load_dword %0, %1, 0x0 glc\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return v;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p, uint32_t nrec) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, nrec, 0x00020000);
}
constexpr int kCoherent = 16;  // sc1: agent-scope coherent access (L2 write-through / miss)

// ---- the fp16 tail in a tail wave (one query head; scores with lane = key)
// The old rows 0..nold-1 of kv head g in registers, each array loaded in one
// batch: kq = the K row of key `lane`; vr[k] = dims 2j, 2j + 1 (j = lane &
// 31) of the V row 2k + (lane >> 5).  Rows from nold on read as zero (the
// buffer resource ends at row nold - 1 of the head); the row goes in the
// scalar offset.
constexpr uint32_t kTailRow = NKV * D * 2;  // bytes between two tail rows
__device__ __forceinline__ uint32_t tail_nrec(int nold) {
  return nold > 0 ? (uint32_t)(nold - 1) * kTailRow + D * 2 : 0u;
}
__device__ __forceinline__ void tail_k_load(const uint16_t* ktail, int g, int nold, u32x4 (&kq)[8]) {
  const int l = threadIdx.x & 63;
  const __amdgpu_buffer_rsrc_t rk = buf_rsrc(ktail + g * D, tail_nrec(nold));
#pragma unroll
  for (int cc = 0; cc < 8; cc++)
    kq[cc] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rk, l * kTailRow + 16 * cc, 0, 0));
}
__device__ __forceinline__ void tail_v_load(const uint16_t* vtail, int g, int nold, uint32_t (&vr)[G / 2]) {
  const int l = threadIdx.x & 63;
  const __amdgpu_buffer_rsrc_t rv = buf_rsrc(vtail + g * D, tail_nrec(nold));
  const int vo = (l & 31) * 4 + (l >> 5) * kTailRow;
#pragma unroll
  for (int k = 0; k < G / 2; k++) vr[k] = __builtin_amdgcn_raw_buffer_load_b32(rv, vo, k * 2 * kTailRow, 0);
}
// P V over the tail rows (p: lane = key, 0 past the tail; rows from nold
// on zero in vr) with the fresh row t (its dims 2j, 2j + 1 in fv; t >= nold):
// o of dims 2j (x) and 2j + 1 (y), lanes j and j + 32 alike.  Each lane
// sums its rows' parity in row order, and row t is the last nonzero term of
// its parity's chain, so it is added after the loop; then the even rows'
// sum plus the odd rows'.
__device__ __forceinline__ f32x2 tail_pv(const uint32_t (&vr)[G / 2], float p, int t, uint32_t fv) {
  const int h = (threadIdx.x >> 5) & 1;
  float o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int k = 0; k < G / 2; k++) {
    const float pe = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), 2 * k));
    const float po = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), 2 * k + 1));
    const float pr = h ? po : pe;
    o0 = __builtin_fmaf(pr, h2f((uint16_t)vr[k]), o0);
    o1 = __builtin_fmaf(pr, h2f((uint16_t)(vr[k] >> 16)), o1);
  }
  if (t >= 0) {
    const float pt = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), t));
    if (h == (t & 1)) {
      o0 = __builtin_fmaf(pt, h2f((uint16_t)fv), o0);
      o1 = __builtin_fmaf(pt, h2f((uint16_t)(fv >> 16)), o1);
    }
  }
  const f32x2 a = swap32(o0), b = swap32(o1);
  return f32x2{a[0] + a[1], b[0] + b[1]};
}
// ---------------------------------------------------------------- host side
// compute units of the current device (0 if unknown)
inline int device_cus() {
  static int cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cus[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev] = n;
  }
  return cus[dev];
}

// workgroups per kv head: about two groups per FP8 wave, 1 or even, <= 32,
// and at most one workgroup per compute unit over the 8 kv heads (a
// workgroup fills a CU's LDS; the cap keeps the whole grid resident at once)
inline int dec_ranges(int ng) {
  int R = (ng + 2 * kFpWaves - 1) / (2 * kFpWaves);
  if (R <= 1) return 1;
  R += R & 1;
  int cap = kMaxRanges;
  const int cus = device_cus();
  if (cus > 0 && cus / NKV < cap) cap = (cus / NKV) & ~1;
  if (cap < 2) return 1;
  return R > cap ? cap : R;
}

// The head pair whose bytes sit at 384..511 of each 512-byte block of the
// cache (kv heads 2p and 2p + 1 own bytes 128p .. 128p + 127 of a key's
// 512-byte row).  Measured on MI355X with per-wave timestamps: the
// workgroups reading that quarter get their first data 1-1.5 us later and
// take about a third longer over the same bytes (stream ends 24.5 against
// 18.5 us at 131072 keys), from HBM and from the Infinity Cache alike; the
// slow heads move with the buffers' base address (bases 128 or 256 bytes
// further on make heads 4-5 or 2-3 the slow pair instead of 6-7).  -1 when K and V disagree or a base
// is not 128-byte aligned.
inline int slow_pair(const void* kc8, const void* vc8) {
  const uintptr_t k = (uintptr_t)kc8 & 511, v = (uintptr_t)vc8 & 511;
  if (k != v || (k & 127)) return -1;
  return (int)(((384 - k) & 511) >> 7);
}

// Workgroups per head pair for R per kv head on average (4R units of two
// workgroups), once the stream is long (2 or more two-group units per FP8
// wave on average: a workgroup's time then follows its bytes, its waves
// sharing the CU's bandwidth): the slow pair gets rs, the others
// (4R - rs) / 3, with rs the feasible count that minimises the costliest
// workgroup's groups weighed 7/5 for the slow pair.  Shorter streams, or no
// slow pair: equal ranges (rp[0] = 0).  nep[p]: the extra groups of pair p
// (one each to the extra wave of workgroups 1..nep[p]); up: prefix sums.
inline void pair_ranges(int ng, int R, int slow, int* rp, int* up, int* nep) {
  rp[0] = 0;
  if (slow < 0 || R < 8 || ng < 4 * kFpWaves * R) return;
  int best_rs = R;
  double best = 7.0 / R;
  for (int rs = R + 3; rs <= kMaxRanges && 4 * R - rs >= 3; rs += 3) {
    const int rf = (4 * R - rs) / 3;
    const double c = std::max(5.0 / rf, 7.0 / rs);
    if (c < best) {
      best = c;
      best_rs = rs;
    }
  }
  if (best_rs == R) return;
  const int rf = (4 * R - best_rs) / 3;
  int acc = 0;
  for (int p = 0; p < 4; p++) {
    rp[p] = p == slow ? best_rs : rf;
    nep[p] = std::min(std::max(ng - 16 * rp[p], 0), rp[p] - 1);
    up[p] = acc;
    acc += rp[p];
  }
  up[4] = acc;
}

}  // namespace cia
