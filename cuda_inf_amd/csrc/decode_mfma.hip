// decode_mfma.hip -- flash-decoding of one query over the group-64 FP8 cache
// on gfx950 matrix cores (replaces the pair attn_decode_split ->
// attn_decode_combine, engine.cu:386-480, for the library's own split; the
// fresh token's tail write, engine.cu:190-198, rides along).  Two launches:
//
// k_decode_attend covers the committed FP8 keys.  They are cut into "pairs":
// 32 keys (half a 64-key group) x 4 kv heads (one half of the 8).  The pairs
// of a half are spread evenly over the 8*nwg waves of its nwg workgroups; a
// wave takes one pair per round and two waves share a SIMD, so one computes
// while the other waits for memory.
//   Loads: every 16-byte global load of a wave covers 4 keys x one 256-byte
//     half-row, so each 16 lanes read 256 contiguous bytes.  K and V land in
//     per-wave LDS tiles [32 keys][16 chunks of 16 B] with an XOR swizzle of
//     the chunk index so the MFMA-layout reads below are conflict-free.
//   S^T = K Q^T on v_mfma_f32_16x16x32_f16: A = K (lane l: key l & 15 of a
//     16-key tile, kv head l >> 4, 8 dims, read as 16 bytes per two MFMAs and
//     converted fp8 -> fp16 exactly); B = Q^T block-diagonal over the 4 kv
//     heads, so all 16 output columns (4 kv heads x 4 query heads) are real.
//     Lane l = 16b + 4a + j then holds keys 4b..4b+3 (+16 per tile) of
//     column (a, j).
//   Online softmax per round in registers (scale folded in, log2 units).
//   O = P V, block-diagonal with the kv head of k-group b rotated per MFMA
//     (sigma_mu(b) = (b + mu) & 3) so each lane's P registers are its A
//     operand as they stand (zero when its kv head is not sigma_mu(b)).  V
//     comes back from LDS through ds_read_b64_tr_b8: 8 keys of one dim per
//     lane.  Each pair's V scale multiplies its own PV product.
//   The waves merge in LDS into one partial (m in log2 units, l, o[64]) per
//   query head of the half.
// k_decode_finish: one single-wave workgroup per item (query head, 8 dims).
//   It issues every load at once -- the head's FP8 partials and the fp16 tail
//   (keys committed..qpos; the fresh token is read from knew/vnew and written
//   into the tail) -- then merges them and writes its 8 output values.
//   (Workgroup-to-workgroup synchronisation inside one launch costs more on
//   this part than a kernel boundary, hence the second launch.)
#include "attn_range.h"
#include "qk_prep.h"

namespace cia {

constexpr int kDecWaves = 8;        // waves per workgroup
constexpr int kMaxWgPerHalf = 128;  // at most one workgroup per CU of a 256-CU part
constexpr int kPart = 4 + D;        // m (log2 units), l, 2 unused, o[64]: 16-byte rows
constexpr int kItems = NH * 8;      // merge items: (query head, 8 dims)
constexpr float kLog2e = 1.44269504088896340736f;
typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;

__device__ __forceinline__ f16x8 cvt8(uint32_t w0, uint32_t w1) {
  const f16x2 a = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false);
  const f16x2 b = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true);
  const f16x2 c = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false);
  const f16x2 d = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true);
  return f16x8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// LDS tiles of a pair: 32 keys x 256 bytes, rows padded to 272 bytes and
// keys 16..31 shifted by a further 64 bytes.  Row r starts 16 r bytes into a
// 128-byte bank cycle, so each 8-lane group of a 16-byte access (K/V stores:
// one key row; K operand reads: 8 keys, one chunk) and each 16-lane group of
// the transposed V reads (keys 4b..4b+3 and 16+4b..16+4b+3, the second four
// moved to the other half of the cycle by the shift) touches distinct banks,
// and every address is a per-lane base plus an immediate.
constexpr int kRowB = 272;
constexpr int kTileB = 16 * kRowB + 64;  // byte offset of keys 16..31
constexpr int kPairB = 2 * kTileB;       // 8832 bytes per wave and operand
constexpr int kQRowsB = 16 * D * 2;      // q rows of a half (fp16)
constexpr int kQBytes = kQRowsB + 128;   // + 128 zero bytes (inactive operand lanes)
constexpr int kMRow = D + 4;             // merge rows (floats)
__device__ __forceinline__ int lds_row(int key) { return key * kRowB + (key >> 4) * 64; }

struct DecodeArgs {
  const uint16_t* q;  // [32][64]
  uint8_t* kc8;    // written only when the fresh token completes a group
  uint8_t* vc8;
  uint16_t* ksc;
  uint16_t* vsc;
  uint16_t* ktail;
  uint16_t* vtail;
  const uint16_t* knew;  // fresh token [8][64] (key qpos), or null: it is in the tail
  const uint16_t* vnew;
  int committed, qpos;
  float scale;
  float* part;    // [32][nwg][kPart]: m, l, -, -, o[64]
  int npairs;     // committed / 32
  int nwg;        // workgroups per half
  uint16_t* out;  // [32][64]
  QkPrep prep;    // prep.qw != null: q and the fresh k arrive raw and are
                  // normalised and rotated here (engine.cu:799-801)
  uint16_t* prepq;  // with prep: the prepared q [32][64] and fresh k [8][64]
                    // rows, written by the attend for the finish
};

// ---------------------------------------------------------------- attend
// grid = (nwg, 2 halves), block = 64 * kDecWaves
// kPrep: q arrives raw and the QK producers run here (a.prep)
template <bool kPrep>
__global__ __launch_bounds__(64 * kDecWaves) void k_decode_attend(DecodeArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t klds[kDecWaves][kPairB];
  __shared__ __attribute__((aligned(16))) uint8_t vlds[kDecWaves][kPairB];
  // q rows of the half (fp16) + zeros: the wave's own copy (prepared q), or
  // one copy the producers fill (raw q)
  __shared__ __attribute__((aligned(16))) uint8_t qlds[kPrep ? 1 : kDecWaves][kQBytes];
  const int half = blockIdx.y;
  const int tid = threadIdx.x, l = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = l & 15, b = l >> 4;  // MFMA column / k-group of this lane
  uint8_t* kw = klds[w];
  uint8_t* vw = vlds[w];
  uint8_t* qb = qlds[kPrep ? 0 : w];
  // this wave's pairs: an even share of the half's pairs
  const int nwaves = a.nwg * kDecWaves;
  const int wid = blockIdx.x * kDecWaves + w;
  // (wid * npairs < 2^31: at most 1024 waves per half, 2^21 pairs)
  const int p0 = (int)(((unsigned)wid * (unsigned)a.npairs) / (unsigned)nwaves);
  const int p1 = (int)(((unsigned)(wid + 1) * (unsigned)a.npairs) / (unsigned)nwaves);
  // Q^T as the block-diagonal B operand, fp16, read from LDS: lane (n, b)
  // holds query head n of the half when its k-group b is that head's kv head
  // (n >> 2), zeros otherwise.  Prepared q: the half's 2 KiB arrive in two
  // full-wave loads issued before the first pair (eight 16-lane operand loads
  // per wave measurably slow the K/V stream behind them).  Raw q (with the
  // QK producers) is loaded first too, but normalised and rotated while the
  // first pair's K/V loads are in flight.
  uint32_t qraw[4] = {0u, 0u, 0u, 0u}, wraw = 0u, kraw = 0u, wkraw = 0u;
  u32x4 qrow2[2];
  float invf = 0.0f;
  if constexpr (kPrep) {
    // (every wave loads four raw q rows, rows 4 (w mod 4) + r of the half,
    // and the fresh raw k row of kv head 4 half + (w mod 4); waves 0-3 use
    // them)
    invf = a.prep.rt.invf[l & 31];
    wraw = a.prep.qw[l];
#pragma unroll
    for (int r = 0; r < 4; r++)
      qraw[r] = a.q[(size_t)(half * 16 + 4 * (w & 3) + r) * D + l];
    // (unconditional: a load under a branch makes the wave wait for it at
    // the join, before the pair's loads are issued; without a fresh k the
    // row is a q row and unused)
    const uint16_t* kn = a.knew ? a.knew : a.q;
    kraw = kn[(size_t)(half * 4 + (w & 3)) * D + l];
    wkraw = a.prep.kw[l];
  } else {
#pragma unroll
    for (int r = 0; r < 2; r++)
      qrow2[r] = *(const u32x4*)(a.q + (size_t)half * 16 * D + (size_t)(r * 64 + l) * 8);
  }
  // per-lane address parts (bytes): global rows of a pair, K/V stores,
  // K operand reads, V transposed reads
  const uint32_t goff = (uint32_t)(b * 512 + n * 16);
  const int wr = b * kRowB + n * 16;  // store i -> key 4i + b, chunk n
  const int krd = n * kRowB + b * 64;  // tile t, MFMA pair m2 -> key 16t + n, chunk 4b + m2
  const int kk8 = n >> 1;
  const int vkey = kk8 < 4 ? 4 * b + kk8 : 16 + 4 * b + (kk8 - 4);
  int vrd[4];  // MFMA mu reads kv head (b + mu) & 3; + nu * 16
#pragma unroll
  for (int mu = 0; mu < 4; mu++) vrd[mu] = lds_row(vkey) + 8 * (n & 1) + ((b + mu) & 3) * 64;
  // loads of a pair: instruction i covers keys 4i..4i+3, lane -> (key 4i + b,
  // chunk n); the group scales first (both for this lane's column kv head),
  // then all K, then all V, so S^T and the softmax run while V is still
  // arriving
  uint16_t ksc_h = 0, vsc_h = 0;
  u32x4 kr[8], vr[8];
  auto load_k = [&](int p, const uint8_t* kc8) {
    const uint8_t* kb = kc8 + (size_t)p * (32 * 512) + half * 256;
    ksc_h = a.ksc[(p >> 1) * NKV + half * 4 + (n >> 2)];
#pragma unroll
    for (int i = 0; i < 8; i++) kr[i] = *(const u32x4*)(kb + goff + i * 2048);
  };
  auto load_v = [&](int p, const uint8_t* vc8) {
    const uint8_t* vb = vc8 + (size_t)p * (32 * 512) + half * 256;
    vsc_h = a.vsc[(p >> 1) * NKV + half * 4 + (n >> 2)];
#pragma unroll
    for (int i = 0; i < 8; i++) vr[i] = *(const u32x4*)(vb + goff + i * 2048);
  };
  // The first pair is loaded whether or not the wave has one (a wave
  // without pairs reads pair 0, or with no committed pair at all the first
  // 16 KiB of the tail buffers, and never uses the values).  It is issued
  // in two phases per workgroup: waves 0-3, a barrier, then waves 4-7.  With
  // every wave's loads issued at once, each wave's last bytes land at the
  // end of the launch and all arithmetic queues behind them; staggered,
  // the first half computes while the second half streams in.
  {
    const bool cache = p0 < p1 || a.npairs > 0;
    const int pf = p0 < p1 ? p0 : 0;
    const uint8_t* k8 = cache ? a.kc8 : (const uint8_t*)a.ktail;
    const uint8_t* v8 = cache ? a.vc8 : (const uint8_t*)a.vtail;
    // One load in straight-line code, the barrier on either side of it by
    // wave (each wave executes one barrier; the hardware counts arrivals).
    // Loads under two conditional branches would merge at the joins into a
    // conservative count, and every later wait on a pair register would
    // become a wait for all of the wave's loads.
    if (w >= kDecWaves / 2) __builtin_amdgcn_s_barrier();
    load_k(pf, k8);
    load_v(pf, v8);
    if (w < kDecWaves / 2) {
      if constexpr (kPrep) {
        // The QK producers: waves 0-3 prepare the half's 16 q rows (four
        // each) while their pair streams in (their raw rows were loaded
        // ahead of it), and before the barrier, so the rows are in LDS for
        // every wave after it.  Workgroup 0 of the half also prepares the
        // fresh k rows of the half's kv heads (one per wave) and stores
        // both for the finish launch.
        // (keeps the producers' arithmetic behind the pair's loads, so it
        // waits only for its own older loads)
        __builtin_amdgcn_sched_barrier(0);
        float sn, cs;
        rope_sincos_f(invf, a.qpos, sn, cs);
        const float wq = h2f((uint16_t)wraw);
        uint16_t* qrows = (uint16_t*)qb;
        uint16_t qp[4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
          qp[r] = qk_norm_rope_sc(h2f((uint16_t)qraw[r]), wq, l, sn, cs, a.prep.eps);
          qrows[(4 * w + r) * D + l] = qp[r];
        }
        if (w == 0 && l < 8) *(u32x4*)(qb + kQRowsB + 16 * l) = u32x4{0u, 0u, 0u, 0u};
        if (blockIdx.x == 0) {
#pragma unroll
          for (int r = 0; r < 4; r++) a.prepq[(size_t)(half * 16 + 4 * w + r) * D + l] = qp[r];
          if (a.knew)
            a.prepq[(size_t)(NH + half * 4 + w) * D + l] = qk_norm_rope_sc(
                h2f((uint16_t)kraw), h2f((uint16_t)wkraw), l, sn, cs, a.prep.eps);
        }
        // LDS writes done, then the barrier alone: a full __syncthreads
        // would also wait for the pair's K/V loads
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      }
      __builtin_amdgcn_s_barrier();
    }
  }
  if constexpr (!kPrep) {
    // (one wave writes and reads its own copy: LDS executes a wave's
    // instructions in order, the wave barrier keeps the compiler from
    // reordering them)
#pragma unroll
    for (int r = 0; r < 2; r++) *(u32x4*)(qb + (r * 64 + l) * 16) = qrow2[r];
    if (l < 8) *(u32x4*)(qb + kQRowsB + 16 * l) = u32x4{0u, 0u, 0u, 0u};
    __builtin_amdgcn_wave_barrier();
  }
  f16x8 qop[8];
  {
    const int qoff = (n >> 2) == b ? n * (2 * D) : kQRowsB;
#pragma unroll
    for (int mu = 0; mu < 8; mu++) qop[mu] = *(const f16x8*)(qb + qoff + 16 * mu);
  }
  const float qscale = a.scale * kLog2e;
  const f16x2 one2 = f16x2{(_Float16)1.0f, (_Float16)1.0f};
  float mx = -1e30f, lsum = 0.f;  // column (a, j) = n: running max (log2) and sum
  f32x4 O[4];                     // rows (kv head b, query head i), dims 16 nu + n
#pragma unroll
  for (int v = 0; v < 4; v++) O[v] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int p = p0; p < p1; p++) {
    // K scale of this lane's column kv head (times scale*log2e); V scale of
    // the same kv head, folded into P
    const float ksc = h2f(ksc_h) * qscale;
    const _Float16 vsc = __builtin_bit_cast(_Float16, vsc_h);
    // ---- S^T = K Q^T for the pair's two tiles; tile t (keys 16t..16t+15)
    // needs only load instructions 4t..4t+3
    f32x4 S[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
      // (the scheduling barriers keep later tiles' LDS stores, which wait
      // for their loads, behind this tile's matrix products)
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 4 * t; i < 4 * t + 4; i++)
        *(u32x4*)(kw + wr + (i & 3) * (4 * kRowB) + (i >> 2) * kTileB) = kr[i];
      S[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m2 = 0; m2 < 4; m2++) {
        const u32x4 kk = *(const u32x4*)(kw + krd + t * kTileB + 16 * m2);
        S[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cvt8(kk[0], kk[1]), qop[2 * m2], S[t], 0, 0, 0);
        S[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cvt8(kk[2], kk[3]), qop[2 * m2 + 1], S[t], 0, 0, 0);
      }
    }
    // the next pair's K loads go out as soon as this pair's K is in LDS
    const bool more = p + 1 < p1;
    if (more) load_k(p + 1, a.kc8);
    // ---- online softmax (column (a, j) = n: 4 lanes x 4 keys per tile)
    float rmx = -1e30f;
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        S[t][i] *= ksc;
        rmx = __builtin_fmaxf(rmx, S[t][i]);
      }
    rmx = col4_max(rmx);
    const float mnew = __builtin_fmaxf(mx, rmx);
    const float corr = __builtin_amdgcn_exp2f(mx - mnew);  // rescales earlier rounds
    mx = mnew;
    f16x8 P;
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) P[t * 4 + i] = (_Float16)__builtin_amdgcn_exp2f(S[t][i] - mnew);
    // row sum of the fp16 numerators (the weights P V uses, before the V scale)
    float rs = 0.f;
#pragma unroll
    for (int e = 0; e < 4; e++) rs = __builtin_amdgcn_fdot2(f16x2{P[2 * e], P[2 * e + 1]}, one2, rs, false);
    rs = col4_sum(rs);
    lsum = __builtin_fmaf(lsum, corr, rs);
    P = P * vsc;
    // this lane's O rows are (kv head b, query head i); the correction of
    // column (b, i) lives in lane 4b + i
    float oc[4];
#pragma unroll
    for (int i = 0; i < 4; i++) oc[i] = __shfl(corr, 4 * b + i);
    // ---- O = O * corr + (P sv) V
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < 8; i++)
      *(u32x4*)(vw + wr + (i & 3) * (4 * kRowB) + (i >> 2) * kTileB) = vr[i];
    const f16x8 zero8 = f16x8{0, 0, 0, 0, 0, 0, 0, 0};
    f32x4 T[4];
#pragma unroll
    for (int nu = 0; nu < 4; nu++) T[nu] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mu = 0; mu < 4; mu++) {
      const int sg = (b + mu) & 3;
      const f16x8 A = ((n >> 2) == sg) ? P : zero8;
#pragma unroll
      for (int nu = 0; nu < 4; nu++) {
        const u32x2 raw = __builtin_bit_cast(
            u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(vw + vrd[mu] + 16 * nu)));
        T[nu] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, cvt8(raw[0], raw[1]), T[nu], 0, 0, 0);
      }
    }
    if (more) load_v(p + 1, a.vc8);
#pragma unroll
    for (int nu = 0; nu < 4; nu++)
#pragma unroll
      for (int i = 0; i < 4; i++) O[nu][i] = __builtin_fmaf(O[nu][i], oc[i], T[nu][i]);
  }
  // ---- merge the waves: O per wave in the V tiles, rows of 68 floats (the
  // readers' 8-byte loads of one row are contiguous; the stores of a fixed
  // (nu, i) conflict at most 2 ways); (m, l) per row in the K tiles
  __syncthreads();
  float* sO = (float*)&vlds[0][0];
  f32x2* sml = (f32x2*)&klds[0][0];
#pragma unroll
  for (int nu = 0; nu < 4; nu++)
#pragma unroll
    for (int i = 0; i < 4; i++) sO[(w * 16 + 4 * b + i) * kMRow + 16 * nu + n] = O[nu][i];
  if (l < 16) sml[w * 16 + l] = f32x2{mx, lsum};
  __syncthreads();
  // thread: row r, dims d0 and d0 + 1
  const int r = tid >> 5, d0 = (tid & 31) * 2;
  f32x2 ml[kDecWaves];  // (m, l) of row r per wave
#pragma unroll
  for (int v = 0; v < kDecWaves; v++) ml[v] = sml[v * 16 + r];
  float M = ml[0][0];
#pragma unroll
  for (int v = 1; v < kDecWaves; v++) M = __builtin_fmaxf(M, ml[v][0]);
  float L = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int v = 0; v < kDecWaves; v++) {
    const float al = __builtin_amdgcn_exp2f(ml[v][0] - M);
    L = __builtin_fmaf(ml[v][1], al, L);
    const f32x2 o2 = *(const f32x2*)(sO + (v * 16 + r) * kMRow + d0);
    a0 = __builtin_fmaf(o2[0], al, a0);
    a1 = __builtin_fmaf(o2[1], al, a1);
  }
  float* pp = a.part + ((size_t)(half * 16 + r) * a.nwg + blockIdx.x) * kPart;
  *(f32x2*)(pp + 4 + d0) = f32x2{a0, a1};
  if (d0 == 0) *(f32x2*)pp = f32x2{M, L};
}

// Wave sums of 8 values by recursive halving: a permlane32 swap pairs value e
// of the lower half with value 4 + e of the upper half (each side adds its
// partner's copy of the value it keeps), a permlane16 swap does the same for
// 4 -> 2 values, a DPP exchange across lane bit 3 for 2 -> 1, and three DPP
// adds (half-row mirror, quad swaps) finish the 8-lane groups.  Every lane
// returns the wave total of value halving_dim(lane).
__device__ __forceinline__ int halving_dim(int lane) {
  return ((lane >> 3) & 1) + 2 * ((lane >> 4) & 1) + 4 * ((lane >> 5) & 1);
}
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl,
                                                               0xF, 0xF, false));
}
__device__ __forceinline__ float wave_sum8_halving(const float (&o)[8]) {
  float s4[4], s2[2];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, o[e]),
                                                    __builtin_bit_cast(uint32_t, o[4 + e]), false, false);
    s4[e] = __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
  }
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, s4[e]),
                                                    __builtin_bit_cast(uint32_t, s4[2 + e]), false, false);
    s2[e] = __builtin_bit_cast(float, (uint32_t)r[0]) + __builtin_bit_cast(float, (uint32_t)r[1]);
  }
  const bool hi = (__lane_id() >> 3) & 1;
  float v = (hi ? s2[1] : s2[0]) + row_ror<8>(hi ? s2[0] : s2[1]);
  v += dpp_f<0x141>(v);  // row_half_mirror: lane i <- lane 7 - i of its 8
  v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
  return v;
}

// ---------------------------------------------------------------- finish
// grid = 256 items (query head h, dims 8c..8c+7), block = 64 (one wave).
// Workgroups are handed to the 8 XCDs round-robin (XCD = blockIdx.x mod 8),
// so item b takes h = 4 (b mod 8) + (b div 64) and c = (b div 8) mod 8: the
// 8 items of a head -- and the 4 heads of one kv head -- share an XCD and
// read that head's partials and tail rows through one L2.  Lane s holds FP8
// partials s and s + 64; lane t attends tail key committed + t.
__global__ __launch_bounds__(64) void k_decode_finish(DecodeArgs a) {
  const int j = blockIdx.x >> 3;
  const int h = (blockIdx.x & 7) * 4 + (j >> 3), c = j & 7, kvh = h / GQA;
  const int l = threadIdx.x;
  const int ntail = a.qpos + 1 - a.committed;  // 0..64
  const uint16_t* qrow = a.q + (size_t)h * D;
  const uint16_t* knew = a.knew ? a.knew + (size_t)kvh * D : nullptr;
  // ---- every load first: partials, then the tail row of this lane.  Loads
  // go out unconditionally (partials beyond nwg and tail rows beyond the
  // tail read a valid partial / row, and their values are replaced), so no
  // register is set up or merged on a branch.
  const float* ph = a.part + (size_t)h * a.nwg * kPart;
  float pm[2], pl[2];
  f32x4 po[2][2];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const int s = l + 64 * u;
    const float* pp = ph + (size_t)(s < a.nwg ? s : 0) * kPart;
    const f32x2 ml = *(const f32x2*)pp;
    pm[u] = s < a.nwg ? ml[0] : -1e30f;
    pl[u] = s < a.nwg ? ml[1] : 0.f;
    po[u][0] = *(const f32x4*)(pp + 4 + 8 * c);
    po[u][1] = *(const f32x4*)(pp + 8 + 8 * c);
  }
  const bool live = l < ntail;
  // the fresh token completes the group: commit it in this launch
  const bool commit = a.knew && ntail == G;
  const int trow = live ? l : 0;  // (tail row 0 exists whatever the tail length)
  const bool fresh = a.knew && l == ntail - 1;
  const uint16_t* kp = fresh ? knew : a.ktail + ((size_t)trow * NKV + kvh) * D;
  const uint16_t* vp = fresh ? a.vnew + kvh * D : a.vtail + ((size_t)trow * NKV + kvh) * D;
  u32x4 kq[8], qq[8], vrow[8];
#pragma unroll
  for (int cc = 0; cc < 8; cc++) {
    kq[cc] = *(const u32x4*)(kp + 8 * cc);
    qq[cc] = *(const u32x4*)(qrow + 8 * cc);
  }
  // (this lane's 8 V dims on their own: indexing the full row below with
  // the runtime c would put it in scratch memory)
  const u32x4 vv = *(const u32x4*)(vp + 8 * c);
  if (commit) {
#pragma unroll
    for (int cc = 0; cc < 8; cc++) vrow[cc] = *(const u32x4*)(vp + 8 * cc);
  }
  // the fresh token joins the tail, written once per kv head
  if (a.knew && c == 0 && h % GQA == 0 && l < 16) {
    const int row = ntail - 1, cc = l & 7;
    uint16_t* dst = (l < 8 ? a.ktail : a.vtail) + ((size_t)row * NKV + kvh) * D + cc * 8;
    const uint16_t* src = (l < 8 ? knew : a.vnew + kvh * D) + cc * 8;
    *(u32x4*)dst = *(const u32x4*)src;
  }
  // ---- tail scores (log2 units) and this lane's V values (dims 8c..8c+7)
  float x = -1e30f, vf[8];
  if (!commit) {
    // (pairs taken with shufflevector: a bit_cast of one 32-bit element into
    // the dot product's f16x2 operand compiled to the same source registers
    // for all four elements of a 16-byte chunk)
    float sacc = 0.f;
#pragma unroll
    for (int cc = 0; cc < 8; cc++) {
      const f16x8 q8 = __builtin_bit_cast(f16x8, qq[cc]), k8 = __builtin_bit_cast(f16x8, kq[cc]);
      sacc = __builtin_amdgcn_fdot2(__builtin_shufflevector(q8, q8, 0, 1), __builtin_shufflevector(k8, k8, 0, 1), sacc, false);
      sacc = __builtin_amdgcn_fdot2(__builtin_shufflevector(q8, q8, 2, 3), __builtin_shufflevector(k8, k8, 2, 3), sacc, false);
      sacc = __builtin_amdgcn_fdot2(__builtin_shufflevector(q8, q8, 4, 5), __builtin_shufflevector(k8, k8, 4, 5), sacc, false);
      sacc = __builtin_amdgcn_fdot2(__builtin_shufflevector(q8, q8, 6, 7), __builtin_shufflevector(k8, k8, 6, 7), sacc, false);
    }
    x = live ? sacc * (a.scale * kLog2e) : -1e30f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      vf[2 * i] = h2f((uint16_t)vv[i]);
      vf[2 * i + 1] = h2f((uint16_t)(vv[i] >> 16));
    }
  } else {
    // The fresh token fills the group: it is committed (kv_commit_group,
    // engine.cu:202-228) and, as in the reference, the group is attended in
    // its FP8 form.  Every wave of the kv head quantises what it needs; the
    // wave (c 0, first query head) writes the bytes and the scales.
    float kf[64], vfl[64];
#pragma unroll
    for (int cc = 0; cc < 8; cc++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        kf[8 * cc + 2 * i] = h2f((uint16_t)kq[cc][i]);
        kf[8 * cc + 2 * i + 1] = h2f((uint16_t)(kq[cc][i] >> 16));
        vfl[8 * cc + 2 * i] = h2f((uint16_t)vrow[cc][i]);
        vfl[8 * cc + 2 * i + 1] = h2f((uint16_t)(vrow[cc][i] >> 16));
      }
    float ak = 0.f, av = 0.f;
#pragma unroll
    for (int d = 0; d < D; d++) {
      ak = __builtin_fmaxf(ak, __builtin_fabsf(kf[d]));
      av = __builtin_fmaxf(av, __builtin_fabsf(vfl[d]));
    }
    const float sck = quant_scale(wave_max_fast(ak)), scv = quant_scale(wave_max_fast(av));
    const uint16_t skh = f2h(sck), svh = f2h(scv);
    const float kdq = h2f(skh), vdq = h2f(svh);
    const bool writer = c == 0 && h % GQA == 0;
    const size_t row = ((size_t)(a.committed + l) * NKV + kvh) * D;
    float sacc = 0.f;
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const uint32_t kb = e4m3x4(kf[4 * j] / sck, kf[4 * j + 1] / sck, kf[4 * j + 2] / sck,
                                 kf[4 * j + 3] / sck);
      sacc = __builtin_fmaf(h2f((uint16_t)(qq[j >> 1][(j & 1) * 2] & 0xFFFF)),
                            e4m3_to_f32<0>(kb) * kdq, sacc);
      sacc = __builtin_fmaf(h2f((uint16_t)(qq[j >> 1][(j & 1) * 2] >> 16)),
                            e4m3_to_f32<1>(kb) * kdq, sacc);
      sacc = __builtin_fmaf(h2f((uint16_t)(qq[j >> 1][(j & 1) * 2 + 1] & 0xFFFF)),
                            e4m3_to_f32<2>(kb) * kdq, sacc);
      sacc = __builtin_fmaf(h2f((uint16_t)(qq[j >> 1][(j & 1) * 2 + 1] >> 16)),
                            e4m3_to_f32<3>(kb) * kdq, sacc);
      if (writer) *(uint32_t*)(a.kc8 + row + 4 * j) = kb;
    }
    x = sacc * (a.scale * kLog2e);
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const uint32_t vb = e4m3x4(h2f((uint16_t)vv[2 * j]) / scv, h2f((uint16_t)(vv[2 * j] >> 16)) / scv,
                                 h2f((uint16_t)vv[2 * j + 1]) / scv,
                                 h2f((uint16_t)(vv[2 * j + 1] >> 16)) / scv);
      vf[4 * j] = e4m3_to_f32<0>(vb) * vdq;
      vf[4 * j + 1] = e4m3_to_f32<1>(vb) * vdq;
      vf[4 * j + 2] = e4m3_to_f32<2>(vb) * vdq;
      vf[4 * j + 3] = e4m3_to_f32<3>(vb) * vdq;
    }
    if (writer) {
#pragma unroll
      for (int j = 0; j < 16; j++)
        *(uint32_t*)(a.vc8 + row + 4 * j) =
            e4m3x4(vfl[4 * j] / scv, vfl[4 * j + 1] / scv, vfl[4 * j + 2] / scv, vfl[4 * j + 3] / scv);
      if (l == 0) {
        a.ksc[(a.committed / G) * NKV + kvh] = skh;
        a.vsc[(a.committed / G) * NKV + kvh] = svh;
      }
    }
  }
  // ---- one softmax over tail keys and partials
  const float M = wave_max_fast(__builtin_fmaxf(x, __builtin_fmaxf(pm[0], pm[1])));
  const float pt = live ? __builtin_amdgcn_exp2f(x - M) : 0.f;
  float L = pt, o[8];
#pragma unroll
  for (int e = 0; e < 8; e++) o[e] = pt * vf[e];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    const float wgt = pl[u] > 0.f ? __builtin_amdgcn_exp2f(pm[u] - M) : 0.f;
    L = __builtin_fmaf(pl[u], wgt, L);
#pragma unroll
    for (int e = 0; e < 4; e++) {
      o[e] = __builtin_fmaf(po[u][0][e], wgt, o[e]);
      o[4 + e] = __builtin_fmaf(po[u][1][e], wgt, o[4 + e]);
    }
  }
  L = wave_sum_fast(L);
  // the 8 dims summed by recursive halving: lanes of each 8-lane group end
  // with dim e(l), one store per group
  const float oe = wave_sum8_halving(o);
  if ((l & 7) == 0) a.out[h * D + 8 * c + halving_dim(l)] = f2h(oe * (1.f / L));
}

}  // namespace cia

using namespace cia;

// workgroups per half: about one pair per wave, at most one workgroup per CU
// pair
static int dec_nwg(int npairs) {
  static int cap = 0;
  if (cap == 0) {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        cus >= 2)
      cap = cus / 2 < kMaxWgPerHalf ? cus / 2 : kMaxWgPerHalf;
    else
      cap = kMaxWgPerHalf;
  }
  int nwg = (npairs + kDecWaves - 1) / kDecWaves;
  if (nwg < 1) nwg = 1;
  return nwg > cap ? cap : nwg;
}

extern "C" int64_t cia_decode_workspace_bytes(int max_tokens) {
  if (max_tokens < 0) return 0;
  // partials, then the prepared q / fresh k rows of a step with the QK
  // producers inside
  return (int64_t)NH * kMaxWgPerHalf * kPart * (int64_t)sizeof(float) +
         (int64_t)(NH + NKV) * D * (int64_t)sizeof(uint16_t);
}

// Flash-decoding with the library's split and, when knew/vnew are given, the
// tail write of the fresh token fused in.  Internal entry shared by
// cia_attn_decode and the layer driver; mid_event (may be NULL) is recorded
// between the two launches, for per-kernel timing.
// prep (may be NULL): a QkPrep when q and knew arrive raw.
extern "C" __attribute__((visibility("hidden"))) int cia_decode_mfma(
    const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8, const uint16_t* ksc,
    const uint16_t* vsc, uint16_t* ktail, uint16_t* vtail, const uint16_t* knew,
    const uint16_t* vnew, int committed, int qpos, float scale, uint16_t* out, void* ws,
    int64_t ws_bytes, void* stream, void* mid_event, const void* prep) {
  const int npairs = committed / 32;
  const int nwg = dec_nwg(npairs);
  if ((int64_t)NH * nwg * kPart * (int64_t)sizeof(float) > ws_bytes) return CIA_ERR_ARG;
  DecodeArgs da{q, (uint8_t*)kc8, (uint8_t*)vc8, (uint16_t*)ksc, (uint16_t*)vsc, ktail, vtail, knew, vnew, committed, qpos, scale,
                (float*)ws, npairs, nwg, out, QkPrep{}, nullptr};
  if (prep) {
    // the prepared q and fresh k rows follow the partials
    constexpr int64_t kRowsB = (int64_t)(NH + NKV) * D * sizeof(uint16_t);
    const int64_t off = (int64_t)NH * nwg * kPart * (int64_t)sizeof(float);
    if (off + kRowsB > ws_bytes) return CIA_ERR_ARG;
    da.prep = *(const QkPrep*)prep;
    da.prepq = (uint16_t*)((char*)ws + off);
  }
  hipStream_t s = (hipStream_t)stream;
  if (da.prep.qw)
    hipLaunchKernelGGL(k_decode_attend<true>, dim3(nwg, 2), dim3(64 * kDecWaves), 0, s, da);
  else
    hipLaunchKernelGGL(k_decode_attend<false>, dim3(nwg, 2), dim3(64 * kDecWaves), 0, s, da);
  int st = launch_status();
  if (st) return st;
  if (mid_event) {
    const hipError_t e = hipEventRecord((hipEvent_t)mid_event, s);
    if (e != hipSuccess) {
      set_hip_error(e);
      return CIA_ERR_HIP;
    }
  }
  if (da.prep.qw) {
    // the finish reads the rows the attend prepared
    da.q = da.prepq;
    if (da.knew) da.knew = da.prepq + NH * D;
  }
  hipLaunchKernelGGL(k_decode_finish, dim3(kItems), dim3(64), 0, s, da);
  return launch_status();
}
