// decode_tok.hip -- flash-decoding of a run of consecutive tokens through
// up to 8 attention layers each, in ONE launch: per layer the reference
// runs attn_decode_split -> attn_decode_combine (engine.cu:846-852) after
// the fresh token's tail write and, when the token fills the group, its
// commit (engine.cu:190-228, 830-845).  The layers of one step share their
// context length, so one grid serves them all and layer l + 1's FP8 K and V
// stream into LDS while layer l's partials merge across the chip.  The
// tokens of a run up to the one that fills the group keep the same FP8
// groups, so the run's steps (token, layer) go in order through the same
// grid, and the last layer of token t hands over to layer 0 of token t + 1
// as one layer to the next.
//
// Work split.  As in the one-layer decode (decode_kv.hip): workgroup =
// (kv head g, key range r), 8R workgroups (one per CU, all resident), the
// committed groups of a kv head spread over its 8R FP8 waves in whole
// groups, two per unit; the extra groups past 16 per workgroup one each to
// wave 8 of ranges 1..ne; the fp16 tail on waves 8-11 of range 0 (one query
// head each), with the fresh token's tail write and the group commit on the
// step whose token fills the group.  The per-wave arithmetic (S^T on the
// matrix cores, online softmax in log2 units, P V through transposed LDS
// reads; the tail's scores and commit) is the one-layer kernel's, so every
// layer's output is bit-identical to a launch of that kernel.
//
// Across layers.  An FP8 wave's key groups are the same in every layer.
// After the S^T of its last unit of layer l it sends the first unit of
// layer l + 1's scales and K into the LDS it has just read, and once the
// workgroup's part of layer l's merge chain is done (barrier B3) that unit's
// V: the next layer's bytes stream while the rest of layer l (softmax, P V,
// merges, the wait below) runs, and the chain's memory operations are not
// queued behind the V.  Layer l + 1's scores start
// only when layer l's output is complete, as in the engine, where the next
// layer's q is computed from it: wave 12 (control) waits until all 32 final
// merges of layer l have stored their output rows and counted themselves in
// layer l's done counter, and only then reads layer l + 1's q rows (and
// fresh k / v), prepares them (RMSNorm + RoPE with the producers) into LDS,
// and opens the layer with a workgroup barrier.  The wait is bounded: after
// kSpinMax polls it records a fault in the workspace (read by
// cia_decode_fault) and goes on, so no launch can hang.
//
// Merge.  Waves 9-12 take query heads 0-3 (lane = dim): each merges its
// head's 8 or 9 wave partials from LDS, stores the workgroup's partial row
// (agent-coherent), waits for the acknowledgement and takes a ticket on its
// (layer, kv head, head) counter; the last of the R to arrive resets the
// counter, fetches the R rows with coherent loads, writes the output row and
// counts it in the layer's done counter.  No wave that sends DMAs ever waits
// for a store's acknowledgement (vmcnt counts loads and stores in order, so
// such a wait would also wait for the next layer's stream).  The counters
// are zero between launches: the tickets reset themselves, and the final
// merge that completes the last layer resets the done counters.
#include <cmath>
#include <type_traits>

#include "decode_wave.h"
#include "qk_prep.h"

namespace cia {

constexpr int kTokWaves = 13;                 // 8 FP8, tail / extra, 3 tail / merge, control
constexpr int kTokThreads = 64 * kTokWaves;
constexpr int kMergeW0 = kFpWaves + 1;        // waves 9..12 merge query heads 0..3
constexpr int kCtlW = kTokWaves - 1;          // wave 12: control (and head 3's merge)
constexpr uint32_t kDoneTarget = NKV * GQA;   // final merges of one layer
constexpr int kSpinMax = 1 << 16;             // polls of a go word before giving up

// LDS arena (one object, as in the one-layer kernel)
constexpr int tK = 0;                                       // [8 waves][kHalfB]
constexpr int tV = tK + kFpWaves * kHalfB;                  // [8 waves][kHalfB]
constexpr int tScale = tV + kFpWaves * kHalfB;              // [8 waves][2 slots][K, V][kScaleB]
constexpr int tQ = tScale + kFpWaves * 4 * kScaleB;         // fp16 q rows [4][64] + 64 zeros
constexpr int tKn = tQ + (GQA * D + 64) * 2;                // fp16 fresh k row [64]
constexpr int tVn = tKn + D * 2;                            // fp16 fresh v row [64]
constexpr int tO = tVn + D * 2;                             // f32 [9 partials][4][64]
constexpr int tML = tO + (kFpWaves + 1) * GQA * D * 4;      // f32x2 [9][4]
constexpr int tX = (tML + (kFpWaves + 1) * GQA * 8 + 127) / 128 * 128;  // extra wave: K, V tile
constexpr int tXS = tX + 2 * kTileB;                        // extra wave: [2 slots][K, V][kScaleB]
constexpr int tSC = tXS + 4 * kScaleB;                     // f32 [2][64]: RoPE sin, cos per lane
constexpr int tINV = tSC + 2 * D * 4;                       // f32 [64]: RoPE inverse frequency per lane
constexpr int tBytes = tINV + D * 4;
static_assert(tBytes <= 160 * 1024, "LDS");

// Timeline build (-DCIA_TIMELINE, `make TIMELINE=1`): each wave keeps up to
// 64 s_memrealtime stamps (100 MHz, low 32 bits), one per lane of a register
// (a per-lane select, so the counted memory operations and their exact
// waits are unchanged), and stores them once at its end into
// tl_buf[workgroup][wave][64]; cia_timeline_read copies them out.  Stamp k
// of layer li is lane 8 li + k (FP8 waves: 0 opened, 1 first unit's K
// landed, 2 its V landed, 3 units done, 4 partials in LDS, 5 the next
// layer's K sent, 6 the next layer's V sent; merge waves:
// 0 opened, 1 partials in LDS, 2 own partial acknowledged, 3 ticket,
// 4 final rows fetched, 5 output counted; control: 6 wait begun, 7 q rows
// loaded; tail waves of range 0: 6 tail rows landed, 7 tail done); lane 63:
// the wave's start.
#ifdef CIA_TIMELINE
constexpr int kTlMaxWg = 8 * kMaxRanges;
__device__ uint32_t tl_buf[kTlMaxWg * kTokWaves * 64];
#define TL_STAMP(k) (tl = l == (k) ? (uint32_t)__builtin_amdgcn_s_memrealtime() : tl)
#else
#define TL_STAMP(k) ((void)0)
#endif

struct TokLayer {
  const uint16_t* q;     // [32][64], raw when the producers run here
  uint8_t* kc8;          // written only when the fresh token completes a group
  uint8_t* vc8;
  uint16_t* ksc;
  uint16_t* vsc;
  uint16_t* ktail;
  uint16_t* vtail;
  const uint16_t* knew;  // the fresh token [8][64] (key qpos)
  const uint16_t* vnew;
  uint16_t* out;         // [32][64]
  const uint16_t* qw;    // producers' norm weights [64] (kPrep)
  const uint16_t* kw;
};

struct TokArgs {
  TokLayer L[kTokMaxLayers];
  int nl, committed, qpos;
  int ntok;        // tokens (decode steps) in this launch: qpos, qpos + 1, ...
  int qs, kvs;     // token t's q / out rows at L[li].q + t qs, its k / v at + t kvs
  float scale, eps;
  float* part;     // [8][kMaxRanges][4][kPartRow]
  uint32_t* tick;  // [layer][8][4], kCntStride apart
  uint32_t* done;  // [layer], kCntStride apart
  uint32_t* err;   // fault word
  uint32_t* go;    // [workgroup] layers opened for it, kTokGoStride apart
  int ng, R, ne;
  int rp[4], up[5], nep[4];  // unequal ranges per head pair (rp[0] = 0: R, ne for all)
  RopeTable rt;
};

// grid = 8R, block = kTokThreads.  kPrep: q and the fresh k arrive raw and
// the QK producers (engine.cu:799-801) run here.
template <bool kPrep, bool kXPre>
__global__ __launch_bounds__(kTokThreads) void k_decode_tok(TokArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[tBytes];
  uint16_t* sq = (uint16_t*)(lds + tQ);
  uint16_t* skn = (uint16_t*)(lds + tKn);
  uint16_t* svn = (uint16_t*)(lds + tVn);
  float* sO = (float*)(lds + tO);    // [p][i][d] at (p * 4 + i) * 64 + d
  f32x2* sml = (f32x2*)(lds + tML);  // [p][i] at p * 4 + i

  // ---- the workgroup's (kv head, range), as in the one-layer decode
  const int bx = blockIdx.x, xcd = bx & 7, yy = bx >> 3;
  int g, r, R = a.R, ne = a.ne;
  if (a.R == 1) {
    g = xcd;
    r = yy;
  } else if (a.rp[0] > 0) {
    const int U = xcd * (a.R >> 1) + (yy >> 1);
    const int p = U >= a.up[2] ? (U >= a.up[3] ? 3 : 2) : (U >= a.up[1] ? 1 : 0);
    g = 2 * p + (yy & 1);
    r = U - a.up[p];
    R = a.rp[p];
    ne = a.nep[p];
  } else {
    g = 2 * (xcd & 3) + (yy & 1);
    r = (xcd >> 2) * (a.R >> 1) + (yy >> 1);
  }
  const int tid = threadIdx.x, l = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
#ifdef CIA_TIMELINE
  uint32_t tl = 0;
  TL_STAMP(63);
#endif
  const bool xw = w == kFpWaves && r != 0 && r <= ne;      // the extra FP8 wave
  const bool tailw = r == 0 && w >= kFpWaves && w < kFpWaves + GQA;
  if (w == kFpWaves && !xw && !tailw) return;               // (nothing for wave 8 here)
  const bool fp8w = w < kFpWaves || xw;
  const int np = r <= ne ? kFpWaves + 1 : kFpWaves;         // wave partials in LDS
  const float qscale = a.scale * kLog2e;
  const int nl = a.nl, qpos = a.qpos, committed = a.committed;
  // steps: token tok's layer li is step tok * nl + li
  const int ntok = a.ntok, ns = ntok * nl;
  // the step each wave is at (its role loop sets them): token, tail keys
  // of the token (the fresh one last) and step
  int tok = 0, tt = qpos + 1 - committed, step = 0;

  // ---- control wave: the RoPE rotation of lane l at a token's position
  // (the same for every layer of the token) into LDS for the waves that
  // prepare rows, and the zero row of the block-diagonal Q^T (both read
  // after B1 of layer 0).  The first token's here; each later token's by
  // the control loop once the token before has passed B3, from the inverse
  // frequencies kept in LDS.
  float* ssc = (float*)(lds + tSC);
  float* sinv = (float*)(lds + tINV);
  auto rope_rows = [&](int pos) __attribute__((always_inline)) {
    float sn, cs;
    rope_sincos_f(sinv[l], pos, sn, cs);
    ssc[l] = sn;
    ssc[D + l] = cs;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // (written before the barrier the readers pass)
  };
  if (w == kCtlW) {
    if constexpr (kPrep) {
      float invf = 0.f;
#pragma unroll
      for (int k = 0; k < D / 2; k++) {
        const float fk = __builtin_bit_cast(
            float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, a.rt.invf[k])));
        invf = (l & 31) == k ? fk : invf;
      }
      sinv[l] = invf;
      rope_rows(qpos);
    }
    sq[GQA * D + l] = 0;
  }

  // ---- FP8 wave state, kept across layers
  const int n = l & 15, c = l >> 4;  // MFMA column / k-group of this lane
  int g0 = 0, g1 = 0;
  {
    const int om = r * kFpWaves + w, nwv = R * kFpWaves, ngm = a.ng - ne;
    if (xw) {
      g0 = ngm + r - 1;
      g1 = g0 + 1;
    } else {
      g0 = (int)(((unsigned)om * (unsigned)ngm) / (unsigned)nwv);
      g1 = (int)(((unsigned)(om + 1) * (unsigned)ngm) / (unsigned)nwv);
    }
  }
  // (w & 7: the compiler then sees that a wave's DMA targets stay inside
  // the tile and scale regions.)  The extra wave has one tile each of K and
  // V: its second tile (always masked) is fetched into, and read from, the
  // first (tile stride ts = 0).
  uint8_t* kw = xw ? lds + tX : lds + tK + (w & 7) * kHalfB;
  uint8_t* vw = xw ? lds + tX + kTileB : lds + tV + (w & 7) * kHalfB;
  uint8_t* sw = xw ? lds + tXS : lds + tScale + (w & 7) * 4 * kScaleB;
  const int ts = xw ? 0 : kTileB;
  const uint32_t nsc = (uint32_t)a.ng * (NKV * 2);  // scale resources end at the last group
  //   K or V: lane l fetches key (l >> 2) of a 16-key block, chunk l & 3
  const uint32_t loff = (uint32_t)((l >> 2) * (NKV * D) + g * D + 16 * (l & 3));
  //   group scales of kv head g, groups s - sh (even lanes) and s - sh + 1
  //   (odd lanes); sh = 1 when s is the last committed group
  const uint32_t soff = (uint32_t)(((l & 1) * NKV + g) * 2);
  auto scale_shift = [&](int u) { return u + 1 >= a.ng && u > 0 ? 1 : 0; };
  auto issue_scales = [&](int li, int u, uint8_t* slot) {
    const uint32_t so = (uint32_t)(u - scale_shift(u)) * (NKV * 2);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.L[li].ksc, nsc), (lds_void_t*)slot, 2, soff,
                                             so, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.L[li].vsc, nsc),
                                             (lds_void_t*)(slot + kScaleB), 2, soff, so, 0, 0);
  };
  // a unit's K or V: 8 DMAs (the second group past the range refetches the first)
  auto issue = [&](const uint8_t* base, int u, uint8_t* dst) {
    const __amdgpu_buffer_rsrc_t rc = buf_rsrc(base);
#pragma unroll
    for (int t = 0; t < 2; t++) {
      const int grp = u + t < g1 ? u + t : u;
#pragma unroll
      for (int j = 0; j < 4; j++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rc, (lds_void_t*)(dst + t * ts + j * kBlkB), 16, loff,
            (uint32_t)grp * (G * NKV * D) + (uint32_t)j * (16 * NKV * D), 0, 0);
    }
  };
  // per-lane LDS offsets: K reads, V transposed reads
  const int krd = (n & 3) * kBlkB + 64 * ((n >> 2) + 4 * c);
  int vrd[4];
  {
    const int k = n >> 1, h = n & 1;
    const int base = (k >> 2) * ts + (k & 3) * kBlkB + 64 * c + 8 * h;
#pragma unroll
    for (int mu = 0; mu < 4; mu++) vrd[mu] = base + 256 * ((c + mu) & 3);
  }
  f16x8 qop[8];
  float mx = -1e30f, lsum = 0.f;
  f32x4 O[4];
  int slot = 0;
  bool vpre = false;
  const f16x2 one2 = f16x2{(_Float16)1.0f, (_Float16)1.0f};
  using T_ = std::integral_constant<bool, true>;
  using F_ = std::integral_constant<bool, false>;

  // One unit of layer li (slot = the scale slot holding its scales): wait
  // for its scales and K, send its V unless it went out already, S^T, then
  // (kMore) the next unit's scales and K (unit un of layer lin) once this
  // unit's K is read; softmax; wait for V; P V.  No load sits under a
  // branch, so every wait is exact.
  auto unit = [&](int li, int u, int lin, int un, auto more_tag, auto vpre_tag) {
    constexpr bool kMore = decltype(more_tag)::value;
    constexpr bool kVPre = decltype(vpre_tag)::value;
    const bool t1ok = u + 1 < g1;
    if constexpr (kVPre) {
      __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8): all but this unit's V
    } else {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      __builtin_amdgcn_sched_barrier(0);
      issue(a.L[li].vc8, u, vw);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (u == g0) TL_STAMP(8 * li + 1);
    const uint32_t* scl = (const uint32_t*)(sw + slot * 2 * kScaleB);
    const int sh = scale_shift(u);
    const float ks0 = h2f((uint16_t)scl[sh]) * qscale, ks1 = h2f((uint16_t)scl[1]) * qscale;
    const _Float16 vs0 = __builtin_bit_cast(_Float16, (uint16_t)scl[kScaleB / 4 + sh]);
    const _Float16 vs1 = __builtin_bit_cast(_Float16, (uint16_t)scl[kScaleB / 4 + 1]);
    f32x4 S[2];
#pragma unroll
    for (int t = 0; t < 2; t++) {
      S[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int m2 = 0; m2 < 4; m2++) {
        const u32x4 kk = *(const u32x4*)(kw + krd + t * ts + 16 * m2);
        S[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cvt8(kk[0], kk[1]), qop[2 * m2], S[t], 0, 0, 0);
        S[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(cvt8(kk[2], kk[3]), qop[2 * m2 + 1], S[t], 0, 0, 0);
      }
    }
    if constexpr (kMore) {
      // this unit's K (and the other scale slot) fully read
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_sched_barrier(0);
      issue_scales(lin, un, sw + (slot ^ 1) * 2 * kScaleB);
      issue(a.L[lin].kc8, un, kw);
      __builtin_amdgcn_sched_barrier(0);
      if (lin != li) TL_STAMP(8 * li + 5);
    }
    // ---- online softmax over the unit's 128 keys (4 per lane and tile)
    float rmx = -1e30f;
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        S[t][v] *= t ? ks1 : ks0;
        if (t == 1 && !t1ok) S[t][v] = -1e30f;
        rmx = __builtin_fmaxf(rmx, S[t][v]);
      }
    rmx = head_max(rmx);
    const float mnew = __builtin_fmaxf(mx, rmx);
    const float corr = __builtin_amdgcn_exp2f(mx - mnew);
    mx = mnew;
    f16x8 P;
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
      for (int v = 0; v < 4; v++) P[4 * t + v] = (_Float16)__builtin_amdgcn_exp2f(S[t][v] - mnew);
    float rs = 0.f;
#pragma unroll
    for (int e = 0; e < 4; e++) rs = __builtin_amdgcn_fdot2(f16x2{P[2 * e], P[2 * e + 1]}, one2, rs, false);
    rs = head_sum(rs);
    lsum = __builtin_fmaf(lsum, corr, rs);
#pragma unroll
    for (int v = 0; v < 4; v++) {
      P[v] *= vs0;
      P[4 + v] *= vs1;
    }
    float oc[4];
#pragma unroll
    for (int v = 0; v < 4; v++)
      oc[v] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, corr), v));
    // ---- O = O corr + (P sv) V
    if constexpr (kMore) __builtin_amdgcn_s_waitcnt(0x0F7A);  // vmcnt(10): next scales + K in flight
    else __builtin_amdgcn_s_waitcnt(0x0F70);                  // vmcnt(0)
    if (u == g0) TL_STAMP(8 * li + 2);
    f32x4 T[4];
#pragma unroll
    for (int d = 0; d < 4; d++) T[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    // (the V^T reads of two products in flight: 54.9-55.0 -> 54.7-54.9 us
    // per token against one product's reads at a time, A/B on one box)
    unit_pv(T, P, vw, vrd, n, c);
    if constexpr (kMore) {
      // this unit's V fully read: the caller sends the next unit's V
      __builtin_amdgcn_s_waitcnt(0xC07F);
    }
#pragma unroll
    for (int d = 0; d < 4; d++)
#pragma unroll
      for (int v = 0; v < 4; v++) O[d][v] = __builtin_fmaf(O[d][v], oc[v], T[d][v]);
  };

  // the first unit of layer 0: scales and K
  if (kXPre && fp8w) {
    __builtin_amdgcn_sched_barrier(0);
    issue_scales(0, g0, sw);
    issue(a.L[0].kc8, g0, kw);
    issue(a.L[0].vc8, g0, vw);
    __builtin_amdgcn_sched_barrier(0);
    vpre = true;
  }

  // control wave: wait for the step before, then the step's q rows (and
  // fresh token) into LDS; li: the step's layer (the timestamp build's)
  auto control_wait = [&]([[maybe_unused]] int li) __attribute__((always_inline)) {
    // step - 1 complete (every output row stored): this workgroup's go word
    // reaches step (written by the count that completed that step); read
    // on the scalar path, so the polls do not queue behind the V DMAs the
    // FP8 waves sent at B3 (56.3-56.5 -> 54.9-55.1 us per token at 32 768
    // keys x 6 layers against the vector poll, A/B on one box)
    uint32_t* gw = a.go + (size_t)blockIdx.x * kTokGoStride;
    TL_STAMP(8 * li + 6);
    int it = 0;
    for (;;) {
      const uint32_t v = scalar_poll(gw);
      if (v >= (uint32_t)step) break;
      if (++it > kSpinMax) {
        if (l == 0) __hip_atomic_fetch_or(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
    // the last step's word is written no more: back to zero for the next launch
    if (step == ns - 1 && l == 0) __hip_atomic_store(gw, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  // layer li's q rows i0..i1-1 of the kv head (and, with `fresh` on range
  // 0, the fresh token) into LDS, prepared when the producers run here
  auto open_rows = [&](int li, int i0, int i1, bool fresh) __attribute__((always_inline)) {
    const TokLayer& Ly = a.L[li];
    uint16_t qr[GQA];
#pragma unroll
    for (int i = 0; i < GQA; i++)
      if (i >= i0 && i < i1) qr[i] = Ly.q[(size_t)tok * a.qs + (g * GQA + i) * D + l];
    uint16_t kr = 0, vr = 0, qwv = 0, kwv = 0;
    if (fresh && r == 0) {
      kr = Ly.knew[(size_t)tok * a.kvs + g * D + l];
      vr = Ly.vnew[(size_t)tok * a.kvs + g * D + l];
    }
    if constexpr (kPrep) {
      qwv = Ly.qw[l];
      if (fresh && r == 0) kwv = Ly.kw[l];
    }
#ifdef CIA_TIMELINE
    __builtin_amdgcn_s_waitcnt(0x0F70);  // (the loads landed: the stamp after them)
    if (w == kCtlW) TL_STAMP(8 * li + 7);
#endif
    float sn = 0.f, cs = 1.f;
    if constexpr (kPrep) {
      sn = ssc[l];
      cs = ssc[D + l];
    }
#pragma unroll
    for (int i = 0; i < GQA; i++) {
      if (i < i0 || i >= i1) continue;
      if constexpr (kPrep)
        sq[i * D + l] = qk_norm_rope_sc(h2f(qr[i]), h2f(qwv), l, sn, cs, a.eps);
      else
        sq[i * D + l] = qr[i];
    }
    if (fresh && r == 0) {
      if constexpr (kPrep)
        skn[l] = qk_norm_rope_sc(h2f(kr), h2f(kwv), l, sn, cs, a.eps);
      else
        skn[l] = kr;
      svn[l] = vr;
    }
  };
  // FP8 waves: layer li's units (the next layer's first unit sent on the way)
  auto fp8_layer = [&](int li) __attribute__((always_inline)) {
    // ============================================== FP8 waves: layer li
    {
      const int qoff = ((n >> 2) == c ? (n & 3) * D : GQA * D) * 2;
#pragma unroll
      for (int m = 0; m < 8; m++) qop[m] = *(const f16x8*)((const uint8_t*)sq + qoff + 16 * m);
    }
    mx = -1e30f;
    lsum = 0.f;
#pragma unroll
    for (int d = 0; d < 4; d++) O[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (!kXPre) {
      // the layer's first unit once the layer is open
      __builtin_amdgcn_sched_barrier(0);
      issue_scales(li, g0, sw + slot * 2 * kScaleB);
      issue(a.L[li].kc8, g0, kw);
      __builtin_amdgcn_sched_barrier(0);
      vpre = false;
    }
    // the next unit: this layer's, or the next step's first (layer li + 1,
    // or layer 0 of the next token; the same groups, no commit between)
    const int nli = li + 1 == nl ? 0 : li + 1;
    for (int u = g0;; u += 2) {
      const bool lastu = u + 2 >= g1;
      const int lin = lastu ? nli : li, un = lastu ? g0 : u + 2;
      if ((!lastu || step + 1 < ns) && (kXPre || !lastu)) {
        if (vpre) unit(li, u, lin, un, T_{}, T_{});
        else unit(li, u, lin, un, T_{}, F_{});
        // the next unit's V, once this unit's P V has read the buffer (the
        // next layer's: after B3, issued by the caller)
        if (!lastu) issue(a.L[lin].vc8, un, vw);
        vpre = true;
      } else {
        if (vpre) unit(li, u, lin, un, F_{}, T_{});
        else unit(li, u, lin, un, F_{}, F_{});
        vpre = false;
      }
      slot ^= 1;
      if (lastu) break;
    }
    TL_STAMP(8 * li + 3);
    // the four key blocks of each (head, dim) summed: lane l holds head
    // l >> 4, dim 16 delta + (l & 15)
    const int pw = xw ? kFpWaves : w;
#pragma unroll
    for (int d = 0; d < 4; d++)
      sO[(pw * GQA + (l >> 4)) * D + 16 * d + (l & 15)] = col4_sum4(O[d][0], O[d][1], O[d][2], O[d][3]);
    if (l < GQA) sml[pw * GQA + l] = f32x2{mx, lsum};
  };
  // tail waves (range 0): layer li's fp16 tail, fresh token and commit.
  // tail_load runs before B1: the old rows of the kv head's tail into
  // registers, K and V in one batch, so their round trip runs under the wait
  // for the layer's q; the fresh row comes from LDS after B1.  On the step
  // that commits the group the V rows load after the scores (the K
  // quantisation needs the registers).
  u32x4 tkq[8];
  uint32_t tvr[G / 2];
  auto tail_load = [&](int li, auto commit_tag) __attribute__((always_inline)) {
    tail_k_load(a.L[li].ktail, g, tt - 1, tkq);
    if constexpr (!decltype(commit_tag)::value) tail_v_load(a.L[li].vtail, g, tt - 1, tvr);
  };
  auto tail_layer = [&](int li, auto commit_tag) __attribute__((always_inline)) {
    constexpr bool commit = decltype(commit_tag)::value;
    const TokLayer& Ly = a.L[li];
    const int i = w - kFpWaves;  // query head 4g + i
#ifdef CIA_TIMELINE
    __builtin_amdgcn_s_waitcnt(0x0F70);  // (the rows landed: the stamp after them)
    TL_STAMP(8 * li + 6);
#endif
    if (i == 0) {
      // the fresh token into its tail row (engine.cu:190-198)
      Ly.ktail[((size_t)(tt - 1) * NKV + g) * D + l] = skn[l];
      Ly.vtail[((size_t)(tt - 1) * NKV + g) * D + l] = svn[l];
    }
    // ---- scores: lane = key (the fresh row from LDS); q from LDS as used
    const bool live = l < tt;
    const uint16_t* qrow = sq + i * D;
    u32x4 kq[8];
#pragma unroll
    for (int cc = 0; cc < 8; cc++) kq[cc] = tkq[cc];
    if (l == tt - 1) {
#pragma unroll
      for (int cc = 0; cc < 8; cc++) kq[cc] = *(const u32x4*)(skn + 8 * cc);
    }
    float x;
    if constexpr (!commit) {
      float sacc = 0.f;
#pragma unroll
      for (int cc = 0; cc < 8; cc++) {
        const f16x8 q8 = *(const f16x8*)(qrow + 8 * cc), k8 = __builtin_bit_cast(f16x8, kq[cc]);
        sacc = __builtin_amdgcn_fdot2(__builtin_shufflevector(q8, q8, 0, 1), __builtin_shufflevector(k8, k8, 0, 1), sacc, false);
        sacc = __builtin_amdgcn_fdot2(__builtin_shufflevector(q8, q8, 2, 3), __builtin_shufflevector(k8, k8, 2, 3), sacc, false);
        sacc = __builtin_amdgcn_fdot2(__builtin_shufflevector(q8, q8, 4, 5), __builtin_shufflevector(k8, k8, 4, 5), sacc, false);
        sacc = __builtin_amdgcn_fdot2(__builtin_shufflevector(q8, q8, 6, 7), __builtin_shufflevector(k8, k8, 6, 7), sacc, false);
      }
      x = sacc * qscale;
    } else {
      // The fresh token fills the group: kv_commit_group (engine.cu:202-228)
      // of kv head g, and the group is attended in its FP8 form.  Lane l
      // quantises key l (dims 4j..4j+3 of its row are words 2(j & 1) and
      // 2(j & 1) + 1 of chunk j / 2); wave 8 writes the bytes and the scale.
      float ak = 0.f;
#pragma unroll
      for (int cc = 0; cc < 8; cc++)
#pragma unroll
        for (int e = 0; e < 4; e++)
          ak = __builtin_fmaxf(ak, __builtin_fmaxf(__builtin_fabsf(h2f((uint16_t)kq[cc][e])),
                                                   __builtin_fabsf(h2f((uint16_t)(kq[cc][e] >> 16)))));
      const float sck = quant_scale(wave_max_fast(ak));
      const uint16_t skh = f2h(sck);
      const float kdq = h2f(skh);
      uint8_t* krow8 = Ly.kc8 + ((size_t)(committed + l) * NKV + g) * D;
      // x / sck by quant_div, the reciprocal taken once
      const float rk = 1.0f / sck, sk = quant_div_s(sck);
      float sacc = 0.f;
#pragma unroll
      for (int j = 0; j < 16; j++) {
        const u32x4 src = kq[j >> 1];
        const int e0 = (j & 1) * 2;
        const uint32_t kb = e4m3x4(quant_div(h2f((uint16_t)src[e0]), sk, rk),
                                   quant_div(h2f((uint16_t)(src[e0] >> 16)), sk, rk),
                                   quant_div(h2f((uint16_t)src[e0 + 1]), sk, rk),
                                   quant_div(h2f((uint16_t)(src[e0 + 1] >> 16)), sk, rk));
        const f16x8 q8 = *(const f16x8*)(qrow + 8 * (j >> 1));
        const int o4 = (j & 1) * 4;
        sacc = __builtin_fmaf((float)q8[o4 + 0], e4m3_to_f32<0>(kb) * kdq, sacc);
        sacc = __builtin_fmaf((float)q8[o4 + 1], e4m3_to_f32<1>(kb) * kdq, sacc);
        sacc = __builtin_fmaf((float)q8[o4 + 2], e4m3_to_f32<2>(kb) * kdq, sacc);
        sacc = __builtin_fmaf((float)q8[o4 + 3], e4m3_to_f32<3>(kb) * kdq, sacc);
        if (i == 0) *(uint32_t*)(krow8 + 4 * j) = kb;
      }
      if (i == 0 && l == 0) Ly.ksc[(committed / G) * NKV + g] = skh;
      x = sacc * qscale;
    }
    x = live ? x : -1e30f;
    const float M = wave_max_fast(x);
    const float p = live ? __builtin_amdgcn_exp2f(sub_rn(x, M)) : 0.f;
    const float L = wave_sum_fast(p);
    // ---- P V (the fresh V row from LDS)
    const uint32_t fv = *(const uint32_t*)(svn + 2 * (l & 31));
    f32x2 o;
    if constexpr (!commit) {
      o = tail_pv(tvr, p, tt - 1, fv);
    } else {
      // the whole group (tt == 64): V quantised with its group scale; lane =
      // dim, the rows held two per register (row 2k low, 2k + 1 high), the
      // fresh row 63 from LDS
      uint32_t vp[G / 2];
#pragma unroll
      for (int k = 0; k < G / 2; k++) {
        const uint32_t lo = Ly.vtail[((size_t)(2 * k) * NKV + g) * D + l];
        const uint32_t hi = 2 * k + 1 < G - 1 ? (uint32_t)Ly.vtail[((size_t)(2 * k + 1) * NKV + g) * D + l]
                                              : (uint32_t)svn[l];
        vp[k] = lo | (hi << 16);
      }
      float av = 0.f;
#pragma unroll
      for (int k = 0; k < G / 2; k++)
        av = __builtin_fmaxf(av, __builtin_fmaxf(__builtin_fabsf(h2f((uint16_t)vp[k])),
                                                 __builtin_fabsf(h2f((uint16_t)(vp[k] >> 16)))));
      const float scv = quant_scale(wave_max_fast(av));
      const uint16_t svh = f2h(scv);
      const float vdq = h2f(svh);
      const float rv = 1.0f / scv, sv = quant_div_s(scv);
      // P V in the order of tail_pv: even rows, odd rows, then their sum
      float oe = 0.f, oo = 0.f;
#pragma unroll
      for (int k = 0; k < G; k++) {
        const float vk = h2f((uint16_t)(vp[k >> 1] >> (16 * (k & 1))));
        const uint32_t vb = e4m3x2(quant_div(vk, sv, rv), 0.f) & 0xFFu;
        if (i == 0) Ly.vc8[((size_t)(committed + k) * NKV + g) * D + l] = (uint8_t)vb;
        const float pk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), k));
        if (k & 1) oo = __builtin_fmaf(pk, e4m3_to_f32<0>(vb) * vdq, oo);
        else oe = __builtin_fmaf(pk, e4m3_to_f32<0>(vb) * vdq, oe);
      }
      if (i == 0 && l == 0) Ly.vsc[(committed / G) * NKV + g] = svh;
      o = f32x2{oe + oo, 0.f};
    }
    if constexpr (!commit) {
      if (l < 32) *(f32x2*)(sO + (kFpWaves * GQA + i) * D + 2 * l) = o;
    } else {
      sO[(kFpWaves * GQA + i) * D + l] = o[0];
    }
    if (l == 0) sml[kFpWaves * GQA + i] = f32x2{M, L};
    TL_STAMP(8 * li + 7);
  };
  // merge waves: head i of layer li, the final merge where this workgroup is the last
  // merge waves: head i of layer li.  merge_publish: the workgroup's partial
  // of the head from LDS; with R = 1 it is the output (stored and counted);
  // else it is stored for the final merge and a ticket taken: true when this
  // workgroup holds the head's last partial (then merge_finish runs here).
  auto count_done = [&](int li) __attribute__((always_inline)) {
    // the output row stored: counted in layer li's done counter, which
    // counts on through the launch's tokens (token tok's layer li is
    // complete at (tok + 1) kDoneTarget; no reset between two uses, so none
    // to order before the go words).  The count that completes the step
    // sets every workgroup's go word to step + 1 (but after the last), and
    // on the last token it resets the counter for the next launch.
    stores_acked();
    uint32_t old = 0;
    if (l == 0)
      old = __hip_atomic_fetch_add(a.done + li * kCntStride, 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    old = (uint32_t)__builtin_amdgcn_readfirstlane((int)old);
    if (old == (uint32_t)(tok + 1) * kDoneTarget - 1) {
      if (l == 0 && tok == ntok - 1)
        __hip_atomic_store(a.done + li * kCntStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (step + 1 < ns) {
        // (agent-coherent stores: the relaxed agent-scope atomic store's form)
        const __amdgpu_buffer_rsrc_t rg = buf_rsrc(a.go);
        for (int x = l; x < (int)gridDim.x; x += 64)
          __builtin_amdgcn_raw_buffer_store_b32((uint32_t)(step + 1), rg, x * (kTokGoStride * 4), 0, kCoherent);
      }
    }
#ifdef CIA_TIMELINE
    __builtin_amdgcn_s_waitcnt(0x0F70);
    TL_STAMP(8 * li + 5);
#endif
  };
  auto merge_publish = [&](int li) __attribute__((always_inline)) -> bool {
    const TokLayer& Ly = a.L[li];
    const int i = w - kMergeW0, d = l, h = g * GQA + i;
    // the workgroup's partial of (head i, dim d) (every read first)
    f32x2 ml[kFpWaves + 1];
    float ov[kFpWaves + 1];
#pragma unroll
    for (int p = 0; p <= kFpWaves; p++) {
      const int pp = p < np ? p : 0;
      ml[p] = sml[pp * GQA + i];
      ov[p] = sO[(pp * GQA + i) * D + d];
    }
    float M = -1e30f;
#pragma unroll
    for (int p = 0; p <= kFpWaves; p++) M = p < np ? __builtin_fmaxf(M, ml[p][0]) : M;
    float L = 0.f, Oa = 0.f;
#pragma unroll
    for (int p = 0; p <= kFpWaves; p++) {
      const float wt = p < np ? __builtin_amdgcn_exp2f(ml[p][0] - M) : 0.f;
      L = __builtin_fmaf(ml[p][1], wt, L);
      Oa = __builtin_fmaf(ov[p], wt, Oa);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // (the LDS reads done before the next layer's writes)
    bool last = false;
    if (R == 1) {
      __builtin_amdgcn_raw_buffer_store_b16(f2h(Oa * (1.0f / L)), buf_rsrc(Ly.out + (size_t)tok * a.qs), d * 2, h * D * 2,
                                            kCoherent);
      count_done(li);
    } else {
      // the row (agent-coherent stores: the relaxed agent-scope atomic
      // store's form), its base in the scalar offset
      const __amdgpu_buffer_rsrc_t rp = buf_rsrc(a.part);
      const int rb = ((g * kMaxRanges + r) * GQA + i) * kPartRow * 4;
      __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, Oa), rp, (4 + d) * 4, rb, kCoherent);
      if (d == 0) {
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, M), rp, 0, rb, kCoherent);
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, L), rp, 4, rb, kCoherent);
      }
      stores_acked();
      TL_STAMP(8 * li + 2);
      uint32_t* tk = a.tick + ((li * NKV + g) * GQA + i) * kCntStride;
      uint32_t ticket = 0;
      if (d == 0) ticket = __hip_atomic_fetch_add(tk, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      ticket = (uint32_t)__builtin_amdgcn_readfirstlane((int)ticket);
      TL_STAMP(8 * li + 3);
      last = ticket == (uint32_t)(R - 1);
    }
    return last;
  };
  // ---- the last of the R partials of (kv head g, head i): every row
  // stored.  The ticket goes back to zero for the next launch.
  auto merge_finish = [&](int li) __attribute__((always_inline)) {
    const TokLayer& Ly = a.L[li];
    const int i = w - kMergeW0, d = l, h = g * GQA + i;
    uint32_t* tk = a.tick + ((li * NKV + g) * GQA + i) * kCntStride;
    if (d == 0) __hip_atomic_store(tk, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // (the resource ends at the R partials: reads past them return zero)
    const __amdgpu_buffer_rsrc_t rs =
        buf_rsrc(a.part + (size_t)g * kMaxRanges * kPartF, (uint32_t)R * (GQA * kPartRow * 4));
    const __amdgpu_buffer_rsrc_t ro = buf_rsrc(Ly.out + (size_t)tok * a.qs);
    // lane p weighs partial p, then lane d sums dim d (the row reads go
    // out together; the weights come from lane p).  NP: 32 partials, or
    // kMaxRanges for the unequal ranges; the terms past R weigh 0.
    auto finish = [&](auto np_tag) {
      constexpr int NP = decltype(np_tag)::value;
      // (per-lane offsets: lane p's row, dim d; the head and the row of
      // the dim reads go in the scalar offset)
      const int ho = i * kPartRow * 4;
      const int po = l * (GQA * kPartRow * 4);
      const float mp = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, po, ho, kCoherent));
      const float lp = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, po, ho + 4, kCoherent));
      const int vo = (4 + d) * 4;
      float pv[NP];
#pragma unroll
      for (int p = 0; p < NP; p++)
        pv[p] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                              rs, vo, ho + p * (GQA * kPartRow * 4), kCoherent));
      const bool ok = l < R && lp > 0.f;
      const float Mf = wave_max_fast(ok ? mp : -1e30f);
      const float wt = ok ? __builtin_amdgcn_exp2f(mp - Mf) : 0.f;
      const float Lf = wave_sum_fast(ok ? lp * wt : 0.f);
      float Of = 0.f;
#pragma unroll
      for (int p = 0; p < NP; p++)
        Of = __builtin_fmaf(pv[p], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wt), p)), Of);
      TL_STAMP(8 * li + 4);
      __builtin_amdgcn_raw_buffer_store_b16(f2h(Of * (1.0f / Lf)), ro, d * 2, h * D * 2, kCoherent);
    };
    if (R <= 32)
      finish(std::integral_constant<int, 32>{});
    else
      finish(std::integral_constant<int, kMaxRanges>{});
    count_done(li);
  };
  // Each role runs its own loop over the layers (so that no role's registers
  // stay live through another's code); every wave passes B1, B2 and B3 of
  // each layer in order (and B0 with the producers).
  auto b1 = [&]() {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): LDS stores done (DMAs still in flight)
    __builtin_amdgcn_s_barrier();        // B1: layer li's q rows and fresh token in LDS
  };
  auto b2 = [&]() {
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();        // B2: every wave partial of layer li in LDS
  };
  // B3: the workgroup's part of layer li's merge chain is done (its partials
  // published and ticketed; where it held a final merge, the output stored
  // and counted).  Only then do the FP8 waves send the next layer's V: the
  // compute unit's memory requests are served in order, so the chain's
  // stores, atomics and loads would otherwise queue behind 64 KiB of V.
  auto b3 = [&]() { __builtin_amdgcn_s_barrier(); };
  // the merge waves' part of layer li after B2
  auto merge_part = [&](int li) __attribute__((always_inline)) {
    if (merge_publish(li)) merge_finish(li);
  };
  // With the producers the four merge waves prepare one q row each (wave 9
  // also the fresh token) between B0 (the control wave's wait ended) and B1;
  // without them the control wave copies the rows itself.
  auto b0 = [&]() {
    if constexpr (kPrep) __builtin_amdgcn_s_barrier();  // B0: layer li may open
  };
  auto prep_part = [&](int li) __attribute__((always_inline)) {
    if constexpr (kPrep) {
      b0();
      if (w >= kMergeW0) open_rows(li, w - kMergeW0, w - kMergeW0 + 1, w == kMergeW0);
    }
  };
  // Each role's loop runs the steps in order: token tok = st / nl, layer
  // li = st % nl (a run of tokens without a commit between them; only the
  // last token may commit).
  if (fp8w) {
    for (int st = 0; st < ns; st++) {
      tok = st / nl;
      const int li = st - tok * nl;
      step = st;
      b0();
      b1();
      TL_STAMP(8 * li);
      fp8_layer(li);
      b2();
      TL_STAMP(8 * li + 4);
      b3();
      if (kXPre && st + 1 < ns) {
        __builtin_amdgcn_sched_barrier(0);
        issue(a.L[li + 1 == nl ? 0 : li + 1].vc8, g0, vw);
        __builtin_amdgcn_sched_barrier(0);
        TL_STAMP(8 * li + 6);
      }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // (nothing left in flight)
  } else if (w == kCtlW) {
    for (int st = 0; st < ns; st++) {
      tok = st / nl;
      const int li = st - tok * nl;
      step = st;
      if (st > 0) control_wait(li);
      if constexpr (kPrep) {
        // a new token: its rotation (every wave has passed B3 of the token
        // before, so that token's reads are done; B0 orders the writes
        // before the next reads)
        if (li == 0 && st > 0) rope_rows(qpos + tok);
        prep_part(li);
      }
      else
        open_rows(li, 0, GQA, true);
      b1();
      TL_STAMP(8 * li);
      b2();
      TL_STAMP(8 * li + 1);
      merge_part(li);
      b3();
    }
  } else if (tailw) {
    // (one loop for the token that commits the group, one for the others:
    // their registers never meet)
    auto tail_loop = [&](auto commit_tag) __attribute__((always_inline)) {
      for (int li = 0; li < nl; li++) {
        step = tok * nl + li;
        tail_load(li, commit_tag);
        prep_part(li);
        b1();
        TL_STAMP(8 * li);
        tail_layer(li, commit_tag);
        b2();
        TL_STAMP(8 * li + 1);
        if (w >= kMergeW0) merge_part(li);
        // (wave 8 wrote the fresh row: stored before B3 when a next token
        // follows in this launch, so that its tail loads, after B3, read it)
        if (w == kFpWaves && tok + 1 < ntok) __builtin_amdgcn_s_waitcnt(0x0F70);
        b3();
      }
    };
    // (only the last token may fill the group)
    for (tok = 0; tok < ntok; tok++) {
      tt = qpos + tok + 1 - committed;
      if (tt == G) break;
      tail_loop(F_{});
    }
    if (tok < ntok) tail_loop(T_{});
  } else {
    for (int st = 0; st < ns; st++) {
      tok = st / nl;
      const int li = st - tok * nl;
      step = st;
      prep_part(li);
      b1();
      TL_STAMP(8 * li);
      b2();
      TL_STAMP(8 * li + 1);
      merge_part(li);
      b3();
    }
  }
#ifdef CIA_TIMELINE
  tl_buf[((size_t)blockIdx.x * kTokWaves + w) * 64 + l] = tl;
#endif
}

}  // namespace cia

using namespace cia;

// kXPre: the next layer's first unit streams while a layer merges (its K
// after the last S^T, its V after B3; measured 70.0 against 71.9 us/token
// without, 32 768 keys x 6 layers, when the V went out after P V)
constexpr bool kTokXPre = true;

// The layers of one decode step in one launch when they qualify: every
// layer on the group-64 cache with the library's split (nsplit 0), the
// fresh token landing in its tail, the same committed count, the producers
// on all layers or none (one eps and theta), and at least one group per FP8
// wave.  Returns 1 when cia_decode_tok can run them.
extern "C" __attribute__((visibility("hidden"))) int cia_decode_tok_fits(const cia_layer* L,
                                                                          int nl, int past) {
  if (nl < 1 || nl > kTokMaxLayers) return 0;
  const int committed = L[0].committed;
  for (int j = 0; j < nl; j++) {
    const cia_layer& y = L[j];
    if (y.budget > 0 || y.nsplit != 0 || y.committed != committed) return 0;
    if (!y.kc8 || !y.vc8 || !y.ksc || !y.vsc || !y.ktail || !y.vtail) return 0;
    const int slot = past - y.committed;
    if (slot < 0 || slot >= G || past >= y.maxT) return 0;
    if (slot == G - 1 && y.committed + G > y.maxT) return 0;
    if ((y.qw == nullptr) != (L[0].qw == nullptr)) return 0;
    if (y.qw && (!y.kw || y.eps != L[0].eps || y.theta != L[0].theta)) return 0;
    if (!aligned(y.kc8, 16) || !aligned(y.vc8, 16) || !aligned(y.ksc, 2) || !aligned(y.vsc, 2) ||
        !aligned(y.ktail, 16) || !aligned(y.vtail, 16))
      return 0;
  }
  if (!L[0].ws_decode) return 0;
  const int ng = committed / G, R = dec_ranges(ng);
  if (R > 1 && device_cus() < NKV * R) return 0;
  const int ne = R > 1 ? std::min(std::max(ng - 16 * R, 0), R - 1) : 0;
  int rp[4], up[5], nep[4];
  pair_ranges(ng, R, slow_pair(L[0].kc8, L[0].vc8), rp, up, nep);
  if (rp[0] > 0) {
    for (int p = 0; p < 4; p++)
      if (ng - nep[p] < kFpWaves * rp[p]) return 0;
  } else if (ng - ne < kFpWaves * R) {
    return 0;
  }
  // the layers' other buffers must agree on the slow pair (one geometry)
  for (int j = 1; j < nl; j++)
    if (slow_pair(L[j].kc8, L[j].vc8) != slow_pair(L[0].kc8, L[0].vc8)) return 0;
  // one workgroup per compute unit must fit (LDS, registers)
  static int occ[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!occ[dev]) {
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_decode_tok<false, kTokXPre>, kTokThreads, 0) !=
            hipSuccess ||
        nb < 1)
      occ[dev] = -1;
    else
      occ[dev] = 1;
  }
  return occ[dev] > 0;
}

// ntok decode steps of nl layers (cia_decode_tok_fits true at past) in one
// launch, positions past .. past + ntok - 1: token t's q / out rows of layer
// j at q + t qs + j * 2048 / out + t qs + j * 2048, its fresh k / v at
// k + t kvs + j * 512, v + t kvs + j * 512 (the decode loop's [step][layer]
// rows).  Token t + 1's layer 0 is scored after token t's last layer's
// output is stored, as layer j + 1 after layer j.  Only the last token may
// fill the group (the caller splits its runs there: the groups of the FP8
// waves stay the same).  With the producers the control wave writes each
// token's rotation before the token's first layer opens.  The workspace is
// layer 0's ws_decode.
extern "C" __attribute__((visibility("hidden"))) int cia_decode_tok(
    const cia_layer* L, int nl, const uint16_t* q, const uint16_t* k, const uint16_t* v,
    uint16_t* out, int past, float scale, int ntok, int64_t qs, int64_t kvs, void* stream) {
  if (!q || !k || !v || !out) return CIA_ERR_NULL;
  if (ntok < 1 || ntok > G) return CIA_ERR_ARG;
  if (!aligned(q, 2) || !aligned(k, 2) || !aligned(v, 2) || !aligned(out, 2)) return CIA_ERR_ALIGN;
  const int committed = L[0].committed, ng = committed / G, R = dec_ranges(ng);
  if (ntok > 1) {
    // the run ends at the step that fills the group, inside every layer
    if (past - committed + ntok > G || qs < 0 || kvs < 0 || qs > INT32_MAX / G ||
        kvs > INT32_MAX / G)
      return CIA_ERR_ARG;
    for (int j = 0; j < nl; j++)
      if (past + ntok > L[j].maxT) return CIA_ERR_ARG;
  }
  TokArgs ta{};
  for (int j = 0; j < nl; j++) {
    TokLayer& t = ta.L[j];
    t.q = q + (size_t)j * NH * D;
    t.kc8 = L[j].kc8;
    t.vc8 = L[j].vc8;
    t.ksc = L[j].ksc;
    t.vsc = L[j].vsc;
    t.ktail = L[j].ktail;
    t.vtail = L[j].vtail;
    t.knew = k + (size_t)j * NKV * D;
    t.vnew = v + (size_t)j * NKV * D;
    t.out = out + (size_t)j * NH * D;
    t.qw = L[j].qw;
    t.kw = L[j].kw;
  }
  ta.nl = nl;
  ta.committed = committed;
  ta.qpos = past;
  ta.ntok = ntok;
  ta.qs = (int)qs;
  ta.kvs = (int)kvs;
  ta.scale = scale;
  ta.eps = L[0].eps;
  char* ws = (char*)L[0].ws_decode;
  ta.part = (float*)ws;
  ta.tick = (uint32_t*)(ws + kTokTickOff);
  ta.done = (uint32_t*)(ws + kTokDoneOff);
  ta.err = (uint32_t*)(ws + kTokErrOff);
  ta.go = (uint32_t*)(ws + kTokGoOff);
  ta.ng = ng;
  ta.R = R;
  ta.ne = R > 1 ? std::min(std::max(ng - 16 * R, 0), R - 1) : 0;
  pair_ranges(ng, R, slow_pair(L[0].kc8, L[0].vc8), ta.rp, ta.up, ta.nep);
  const bool prep = L[0].qw != nullptr;
  if (prep) {
    for (int d = 0; d < D / 2; d++)
      ta.rt.invf[d] = (float)std::pow((double)L[0].theta, -(2.0 * d) / D);
  }
  hipStream_t s = (hipStream_t)stream;
  if (prep)
    hipLaunchKernelGGL((k_decode_tok<true, kTokXPre>), dim3(NKV * R), dim3(kTokThreads), 0, s, ta);
  else
    hipLaunchKernelGGL((k_decode_tok<false, kTokXPre>), dim3(NKV * R), dim3(kTokThreads), 0, s, ta);
  return launch_status();
}

#ifdef CIA_TIMELINE
// the timeline build's stamps: [workgroup][wave][64] uint32 of the last
// one-launch decode (see tl_buf); bytes >= 8 * kMaxRanges * 13 * 64 * 4
extern "C" int cia_timeline_read(void* dst, int64_t bytes) {
  if (!dst || bytes < (int64_t)sizeof(tl_buf)) return CIA_ERR_ARG;
  const hipError_t e = hipMemcpyFromSymbol(dst, HIP_SYMBOL(tl_buf), sizeof(tl_buf), 0,
                                           hipMemcpyDeviceToHost);
  if (e != hipSuccess) {
    set_hip_error(e);
    return CIA_ERR_HIP;
  }
  return CIA_OK;
}
#endif

extern "C" int cia_decode_fault(const void* ws, int64_t ws_bytes, int* fault) {
  CIA_REQUIRE(ws && fault, CIA_ERR_NULL);
  CIA_REQUIRE(ws_bytes >= kWsBytes, CIA_ERR_ARG);
  uint32_t f = 0;
  const hipError_t e = hipMemcpy(&f, (const char*)ws + kTokErrOff, sizeof(f), hipMemcpyDeviceToHost);
  if (e != hipSuccess) {
    set_hip_error(e);
    return CIA_ERR_HIP;
  }
  *fault = (int)f;
  return CIA_OK;
}
