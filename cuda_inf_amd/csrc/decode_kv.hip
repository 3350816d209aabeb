// decode_kv.hip -- flash-decoding of one query over the group-64 FP8 cache on
// gfx950 matrix cores, in one launch (replaces the launch pair
// attn_decode_split -> attn_decode_combine, engine.cu:386-480, with the
// library's own split; the fresh token's tail write, engine.cu:190-198, and
// the group commit on the step that fills the group, engine.cu:202-228,
// ride along).
//
// Work split.  Workgroup = (kv head g, key range r); 8R workgroups, R ranges
// per kv head on average (R = 1, or even and at most 32).  Workgroups go to
// the 8 XCDs round-robin (XCD = blockIdx mod 8), and the numbering puts kv
// heads 2j and 2j + 1 of the same range on one XCD: a kv head's 64 bytes are
// half of a 128-byte line, and when the two halves are fetched by different
// XCDs every line crosses the fabric twice (measured: a plain read of the
// same bytes at half the rate).  On long streams the head pair whose bytes
// sit at 384..511 of each 512-byte block (a quarter of the cache that
// streams about a third slower) gets more ranges than the other three pairs
// (41 against 29 at R = 32), so that its workgroups end with the others'.
//
// FP8 waves (8 per workgroup).  The committed groups of kv head g are
// spread evenly over the 8R waves of the kv head (whole 64-key groups), and
// a wave takes its groups two at a time (a unit: 8 KiB of K, 8 KiB of V).
// A unit reaches the wave's LDS by DMA (global_load_lds_dwordx4, no staging registers): 16
// keys x 64 bytes per instruction, lane i's 16 bytes at base + 16 i, blocks
// of 16 keys padded to 1040 bytes.
//   S^T = K Q^T on v_mfma_f32_16x16x32_f16 with the four k-groups of the
//     operands holding four different key blocks (block-diagonal Q^T), so
//     the 16 output columns are (key block b, query head i) and every
//     column is real.  A = K: lane (c, r) holds key
//     16 (r & 3) + (r >> 2) + 4c of the tile, 8 dims, read as 16 bytes per
//     two products and converted fp8 -> fp16 exactly.  Output lane (c, n)
//     with n = 4b + i holds keys 16v + 4b + c (v = 0..3) of head i.
//   Online softmax in registers (scale and K group scale folded, log2
//     units), reduced over the 16 lanes of a head.
//   O = P V with P as the A operand as it stands: in product mu the
//     k-group c of V holds key block (c + mu) & 3 and a lane's P is used
//     only when its block is that one.  V comes from LDS through
//     ds_read_b64_tr_b8 (8 keys of one dim per lane).  The V group scale is
//     folded into P.  Output rows are (key block, head), summed over the
//     blocks at the end.
//   LDS reads of both operands are per-lane base + immediate and
//   bank-conflict-free (K: 8 lanes of a b128 read hit 8 distinct 16-byte
//   slots of a 128-byte bank cycle; V: the 16 lanes of a tr_b8 block hit 16
//   distinct 8-byte slots).
// Tail waves (4, only in the workgroup of range 0).  Wave i takes query head
//   4g + i over the fp16 tail (keys committed..qpos): lane = key for the
//   scores, lane = dim for P V.  With a fresh token it writes the token into
//   the tail, and on the step whose token fills the group it quantises the
//   group (bytes and scales bit-exact with kv_commit_group) and attends it
//   in its FP8 form, as the reference does after its commit.
// Merge.  Each workgroup merges its waves in LDS into one partial (m, l,
//   o[64]) per query head.  With R > 1 it stores the partial with
//   agent-coherent stores, waits until they have reached the agent, and
//   takes a ticket from kv head g's arrival counter (one device-scope atomic
//   per workgroup).  The workgroup that draws the last ticket resets the
//   counter, fetches the R partials in one batch of coherent loads and
//   writes the output.  Measured on this part, against this order:
//   - epoch-tagged 64-bit partial words stored with no wait, polled by one
//     merging workgroup (a word per writer, then the whole set) or by the
//     first R/2 workgroups (a slice of outputs each): coherent loads of words
//     whose stores are still in flight took 2-3 us, and the kernel lost
//     1-2 us per layer against this order;
//   - release / acquire fences at agent scope (buffer_wbl2 / buffer_inv): about
//     10 us each;
//   - a device-scope atomic round trip: about 0.25 us idle, 0.4-0.5 us under
//     the stream; the acknowledgement of agent-coherent stores about 0.6 us.
#include <algorithm>
#include <mutex>
#include <type_traits>
#include <utility>

#include "attn_range.h"
#include "decode_wave.h"
#include "qk_prep.h"

namespace cia {

constexpr int kTailWaves = GQA;            // tail waves (workgroup of range 0)
constexpr int kDecThreads = 64 * (kFpWaves + kTailWaves);
// LDS arena (one object: with several, the compiler tracks the LDS DMA
// conservatively and turns the exact waits below into waits for everything)
constexpr int kLdsK = 0;                                  // [8 waves][kHalfB]
constexpr int kLdsV = kLdsK + kFpWaves * kHalfB;          // [8 waves][kHalfB]
constexpr int kLdsScale = kLdsV + kFpWaves * kHalfB;      // [8 waves][2 slots][K, V][kScaleB]
constexpr int kLdsQ = kLdsScale + kFpWaves * 4 * kScaleB; // fp16 q rows [4][64] + 128 zero bytes
constexpr int kLdsKn = kLdsQ + (GQA * D + 64) * 2;        // fp16 fresh k row [64]
constexpr int kLdsO = kLdsKn + D * 2;                     // f32 [9 partials][4][64]
constexpr int kLdsML = kLdsO + (kFpWaves + 1) * GQA * D * 4;  // f32x2 [9][4]
constexpr int kLdsTicket = kLdsML + (kFpWaves + 1) * GQA * 8;  // the workgroup's ticket
// the extra wave's one group: K tile, V tile, then its K and V scales
constexpr int kLdsX = (kLdsTicket + 16 + 127) / 128 * 128;
constexpr int kLdsXS = kLdsX + 2 * kTileB;
constexpr int kLdsBytes = kLdsXS + 2 * kScaleB;
static_assert(kLdsBytes <= 160 * 1024, "LDS");
// the split entry's workspace: two share slots per (kv head, range), then the counters
constexpr int64_t kSplitWsBytes = 2 * kPartBytes + (int64_t)NKV * kCntStride * sizeof(uint32_t);

// The drop-in split entry's shares meet in this file-scope device array
// (two share slots per (kv head, range), then the arrival counters) unless
// the caller passes a workspace: cia_attn_decode_split allocates nothing.
// The kernels address it from device code.  The counters are zero at load,
// cleared again by a fill kernel on the first call on a device, and every
// complete call leaves them at zero; calls that overlap on one GPU race.
static __device__ __align__(256) uint8_t split_scratch[kSplitWsBytes];


struct DecArgs {
  const uint16_t* q;     // [32][64], raw when prep.qw is set
  uint8_t* kc8;          // written only when the fresh token completes a group
  uint8_t* vc8;
  uint16_t* ksc;
  uint16_t* vsc;
  uint16_t* ktail;
  uint16_t* vtail;
  const uint16_t* knew;  // fresh token [8][64] (key qpos, raw with prep), or null
  const uint16_t* vnew;
  int committed, qpos;
  float scale;
  float* part;           // [8][kMaxRanges][4][kPartRow] partials
  uint32_t* cnt;         // [8] arrival counters, kCntStride apart; zero between calls
  uint16_t* out;         // [32][64]
  int ng;                // committed groups
  int R;                 // workgroups per kv head
  int ne;                // extra groups: the last ne groups, one each to wave 8
                         // of workgroups 1..ne
  // decode mode, unequal ranges: kv heads 2p and 2p + 1 have rp[p]
  // workgroups each (extra groups nep[p]); up = prefix sums of rp.  rp[0] = 0:
  // R and ne for every head.
  int rp[4], up[5], nep[4];
  QkPrep prep;
  // split mode (the reference's attn_decode_split partials, committed keys only)
  float* pm;             // [32][nsplit] max score (natural units), -1e30 when empty
  float* pl;             // [32][nsplit] sum of exp(s - m)
  float* po;             // [32][nsplit][64] sum of exp(s - m) v
  int nsplit, chunk, total;
  int sub;               // workgroups per split (> 1: each takes a share of one
                         // split and the last to arrive merges the shares,
                         // through part and cnt[g * kCntStride + split]);
                         // -1: range mode (the decode's ranges, rp / up)
};

// ---------------------------------------------------------------- kernel
// grid = 8R, block = kDecThreads.  kPrep: q (and the fresh k) arrive raw and
// the QK producers (engine.cu:799-801) run here.
// kSplit: the committed keys of the reference's splits (attn_decode_split,
// engine.cu:396-465; split s covers keys [s chunk, (s + 1) chunk) of the
// qpos + 1): workgroup r of kv head g takes splits [r nsplit / R,
// (r + 1) nsplit / R); its FP8 waves share a split's groups when it has at
// most 8 splits, else take whole splits, and each finished split (or share)
// is written as (m, l, o) -- straight to pm / pl / po when the workgroup has
// 8 splits or more (one wave per split), else through LDS and its merge.
// With sub > 1 workgroups per split (fewer splits than ranges), workgroup r
// takes share r % sub of split r / sub; the shares meet in part and the last
// workgroup to arrive writes the split.  kRange (fewer splits than ranges,
// each split at least as long as a range): the workgroups take the
// decode's key ranges (rp / up), each touching at most two splits, and a
// split's shares (one per range touching it) meet in part, the last range
// to arrive writing the split.  Keys outside a segment's range are
// masked.  The tail keys (fp16 rows) of the splits a workgroup writes are
// taken by its tail waves and folded in by the split's writer.
template <bool kPrep, bool kSplit, bool kRange = false>
__global__ __launch_bounds__(kDecThreads) void k_decode(DecArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBytes];
  uint16_t* sq = (uint16_t*)(lds + kLdsQ);
  uint16_t* skn = (uint16_t*)(lds + kLdsKn);
  float* sO = (float*)(lds + kLdsO);    // [p][i][d] at (p * 4 + i) * 64 + d
  f32x2* sml = (f32x2*)(lds + kLdsML);  // [p][i] at p * 4 + i

  const int bx = blockIdx.x, xcd = bx & 7, yy = bx >> 3;
  int g, r, R = a.R, ne = a.ne;
  if (a.R == 1 || (kSplit && (a.R & 1))) {
    g = xcd;
    r = yy;
  } else if ((!kSplit || kRange) && a.rp[0] > 0) {
    // pair units: workgroups 16j + x and 16j + 8 + x (one XCD) take kv heads
    // 2p and 2p + 1 over the same range; XCD x holds units R/2 x .. R/2 x +
    // R/2 - 1 of the 4R, which go to the pairs in order, rp[p] each
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
  // Wave 8: a tail wave in range 0; in ranges 1..ne the extra wave, which
  // takes one group (an FP8 wave with a one-group buffer in the LDS the
  // others leave free).  The rest return.
  const bool xw = !kSplit && w == kFpWaves && r != 0 && r <= ne;
  if (!kSplit && w >= kFpWaves && r != 0 && !xw) return;
  const float qscale = a.scale * kLog2e;
  // split mode: this workgroup's splits [s0, s0 + ns)
  int s0 = 0, ns = 0, sj = 0;
  if constexpr (kSplit) {
    if constexpr (kRange) {
      // range mode: the splits of the workgroup's committed groups [ga, gb),
      // and for the last range a split of tail keys only, if there is one
      const int ga = (int)(((unsigned)r * (unsigned)a.ng) / (unsigned)R);
      const int gb = (int)(((unsigned)(r + 1) * (unsigned)a.ng) / (unsigned)R);
      s0 = ga * G / a.chunk;
      int shi = (gb * G - 1) / a.chunk;
      if (r == R - 1) shi = max(shi, (a.total - 1) / a.chunk);
      ns = shi - s0 + 1;
    } else if (a.sub > 1) {
      s0 = r / a.sub;
      sj = r - s0 * a.sub;
      ns = 1;
    } else {
      s0 = (int)(((unsigned)r * (unsigned)a.nsplit) / (unsigned)a.R);
      ns = (int)(((unsigned)(r + 1) * (unsigned)a.nsplit) / (unsigned)a.R) - s0;
    }
  }
  // split mode: the splits [tlo, thi] with tail keys (committed..qpos) that
  // this workgroup writes (at most two: splits have 128 keys or more, the
  // tail at most 64); its tail waves take those keys
  int tlo = 1, thi = 0;
  if constexpr (kSplit) {
    if (a.committed < a.total) {
      tlo = max(a.committed / a.chunk, s0);
      thi = min(min((a.total - 1) / a.chunk, s0 + ns - 1), tlo + 1);
    }
    if (w >= kFpWaves && (tlo > thi || w >= kFpWaves + kTailWaves)) return;
  }

  // ================================================================ FP8 waves
  if (w < kFpWaves || xw) {
    const int n = l & 15, c = l >> 4;  // MFMA column / k-group of this lane
    const int om = r * kFpWaves + w, nwv = R * kFpWaves, ngm = a.ng - ne;
    // this wave's committed groups [g0, g1), taken two at a time from g0 (a
    // unit: groups s and s + 1; the second masked when s + 1 == g1); the
    // extra wave's: group ngm + r - 1
    int g0, g1;
    if (xw) {
      g0 = ngm + r - 1;
      g1 = g0 + 1;
    } else {
      g0 = (int)(((unsigned)om * (unsigned)ngm) / (unsigned)nwv);
      g1 = (int)(((unsigned)(om + 1) * (unsigned)ngm) / (unsigned)nwv);
    }
    // split mode: this wave's splits [sa, sb); with part_k > 1 it holds share
    // part_i of its one split's groups (the split's waves are those w with
    // w ns / 8 equal)
    int sa = 0, sb = 0, part_i = 0, part_k = 1;
    // range mode: the wave's keys in split s0 ([wa0, wa1)) and s0 + 1 ([wb0, wb1))
    int wa0 = 0, wa1 = 0, wb0 = 0, wb1 = 0;
    if constexpr (kSplit) {
      if constexpr (kRange) {
        // the workgroup's committed groups [ga, gb) as units per split
        // segment (pairs from the segment's first group; a group holding the
        // split boundary is in both segments), dealt to the 8 waves in order
        const int ga = (int)(((unsigned)r * (unsigned)a.ng) / (unsigned)R);
        const int gb = (int)(((unsigned)(r + 1) * (unsigned)a.ng) / (unsigned)R);
        const int bnd = (s0 + 1) * a.chunk;           // first key of split s0 + 1
        const int gA1 = min(gb, (bnd + G - 1) / G);   // segment A: groups [ga, gA1)
        const int gB0 = bnd / G;                      // segment B: groups [gB0, gb)
        const int uA = (gA1 - ga + 1) >> 1, uB = gB0 < gb ? (gb - gB0 + 1) >> 1 : 0;
        const int U = uA + uB, u0 = w * U / kFpWaves, u1 = (w + 1) * U / kFpWaves;
        wa0 = wa1 = wb0 = wb1 = 0;
        if (u0 < min(u1, uA)) {
          wa0 = (ga + 2 * u0) * G;
          wa1 = min(ga + 2 * min(u1, uA), gA1) * G;
        }
        if (max(u0, uA) < u1) {
          wb0 = (gB0 + 2 * (max(u0, uA) - uA)) * G;
          wb1 = min(gB0 + 2 * (u1 - uA), gb) * G;
        }
        sa = wa0 < wa1 ? s0 : s0 + 1;
        sb = wb0 < wb1 ? s0 + 2 : s0 + 1;
        if (sa >= sb) sa = sb = s0;
      } else if (ns <= kFpWaves) {
        const int j = (w * ns) / kFpWaves;
        const int fw = (j * kFpWaves + ns - 1) / ns, lw = ((j + 1) * kFpWaves + ns - 1) / ns;
        sa = s0 + j;
        sb = sa + 1;
        part_k = lw - fw;
        part_i = w - fw;
        if (a.sub > 1) {  // share sj of the split's sub * 8 wave shares
          part_k = kFpWaves * a.sub;
          part_i = sj * kFpWaves + w;
        }
      } else {
        sa = s0 + (w * ns) / kFpWaves;
        sb = s0 + ((w + 1) * ns) / kFpWaves;
      }
    }
    // the committed keys [ka, kb) of split s that this wave takes (empty: ka == kb)
    auto seg_keys = [&](int s, int& ka, int& kb) {
      const int a0 = s * a.chunk;
      const int b0 = min(min(a0 + a.chunk, a.total), a.committed);
      ka = kb = 0;
      if (a0 >= b0) return;
      if (part_k > 1) {
        const int G0 = a0 / G, ngr = (b0 + G - 1) / G - G0;
        const int q0 = G0 + part_i * ngr / part_k, q1 = G0 + (part_i + 1) * ngr / part_k;
        ka = max(a0, q0 * G);
        kb = min(b0, q1 * G);
        if (ka >= kb) ka = kb = 0;
      } else if constexpr (kRange) {
        ka = max(a0, s > s0 ? wb0 : wa0);
        kb = min(b0, s > s0 ? wb1 : wa1);
        if (ka >= kb) ka = kb = 0;
      } else {
        ka = a0;
        kb = b0;
      }
    };
    // (w & 7: the compiler then sees that a wave's DMA targets stay inside
    // the tile and scale regions, and does not make reads of the q rows wait
    // for them.)  The extra wave has one tile each of K and V: its second
    // tile (always masked) is read from the first (tile stride ts = 0).
    uint8_t* kw = xw ? lds + kLdsX : lds + kLdsK + (w & 7) * kHalfB;
    uint8_t* vw = xw ? lds + kLdsX + kTileB : lds + kLdsV + (w & 7) * kHalfB;
    uint8_t* sw = xw ? lds + kLdsXS : lds + kLdsScale + (w & 7) * 4 * kScaleB;
    const int ts = xw ? 0 : kTileB;
    // Waves 0-3 fetch the raw q row of head 4g + w (and the norm weights)
    // by DMA into a staging area (the partial area, unused until the merge)
    // ahead of their stream, and normalise / copy it into the q rows while
    // the stream is in flight.  (Nothing loaded into registers is used after
    // a wave's DMA has started: vmcnt counts in order, so such a use would
    // wait for the whole unit.)
    uint8_t* qstage = lds + kLdsO + (w & 3) * 1024;
    if (w < GQA) {
      // 8 lanes x 16 bytes; the resource covers just the row, so lanes 8..63
      // read nothing (and write zeros into the rest of the staging slot)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.q + (size_t)(g * GQA + w) * D, 2 * D),
                                               (lds_void_t*)qstage, 16, 16 * l, 0, 0, 0);
      if constexpr (kPrep)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(buf_rsrc(a.prep.qw, 2 * D),
                                                 (lds_void_t*)(qstage + 4096), 16, 16 * l, 0, 0, 0);
    }
    // A unit's data by DMA through buffer resources: each lane's VGPR
    // operand is a fixed offset and the unit's position goes in the scalar
    // offset (the compiler waits on a DMA before overwriting a VGPR the DMA
    // used, so per-unit VGPR addresses would cost a full wait).  With no
    // committed group the resources have no records: the fetch reads nothing.
    const uint32_t nrec = a.ng > 0 ? 0x7fffffffu : 0u;
    const __amdgpu_buffer_rsrc_t rk = buf_rsrc(a.kc8, nrec), rv = buf_rsrc(a.vc8, nrec);
    //   (the scale resources end at the last committed group)
    const uint32_t nsc = (uint32_t)a.ng * (NKV * 2);
    const __amdgpu_buffer_rsrc_t rks = buf_rsrc(a.ksc, nsc), rvs = buf_rsrc(a.vsc, nsc);
    //   K or V: lane l fetches key (l >> 2) of a 16-key block, chunk l & 3
    const uint32_t loff = (uint32_t)((l >> 2) * (NKV * D) + g * D + 16 * (l & 3));
    //   group scales of kv head g, groups s - sh (even lanes) and s - sh + 1
    //   (odd lanes): dwords 0, 1 of the slot (K) and of slot + 256 (V).  sh = 1
    //   when s is the last committed group (s + 1 has no scale), so group s
    //   is in dword sh.
    const uint32_t soff = (uint32_t)(((l & 1) * NKV + g) * 2);
    auto scale_shift = [&](int u) { return u + 1 >= a.ng && u > 0 ? 1 : 0; };
    auto issue_scales = [&](int u, uint8_t* slot) {
      const uint32_t so = (uint32_t)(u - scale_shift(u)) * (NKV * 2);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rks, (lds_void_t*)slot, 2, soff, so, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rvs, (lds_void_t*)(slot + kScaleB), 2, soff, so, 0, 0);
    };
    // (gend: the end of the unit's group range; a second group past it is
    // not the range's: its slot gets the first group again)
    auto issue = [&](int u, int gend, __amdgpu_buffer_rsrc_t rc, uint8_t* dst) {
#pragma unroll
      for (int t = 0; t < 2; t++) {
        if (t == 1 && xw) break;  // (its one group)
        const int grp = u + t < gend ? u + t : u;  // past the range: refetch
#pragma unroll
        for (int j = 0; j < 4; j++)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rc, (lds_void_t*)(dst + t * kTileB + j * kBlkB), 16, loff,
              (uint32_t)grp * (G * NKV * D) + (uint32_t)j * (16 * NKV * D), 0, 0);
      }
    };
    // (a wave without units fetches unit 0 and ignores it)
    int uf = g0 < g1 ? g0 : 0, ufe = g1;
    if constexpr (kSplit) {
      uf = 0;
      ufe = 1;
      for (int s2 = sa; s2 < sb; s2++) {
        int ka2, kb2;
        seg_keys(s2, ka2, kb2);
        if (ka2 < kb2) {
          uf = ka2 / G;
          ufe = (kb2 + G - 1) / G;
          break;
        }
      }
    }
    // Each wave fetches a unit's V only once the unit's K has landed (its K
    // DMAs then hold no more slots, so the V DMAs rarely wait to issue), and
    // multiplies K while V streams in: the workgroup's K lands first and
    // only P V follows the last bytes.
    __builtin_amdgcn_sched_barrier(0);
    issue_scales(uf, sw);
    issue(uf, ufe, rk, kw);
    if (xw) issue(uf, ufe, rv, vw);  // (its one group: K and V at once)
    __builtin_amdgcn_sched_barrier(0);
    if (w < GQA) {
      // the q row landed once at most the unit's 10 scale and K DMAs remain
      __builtin_amdgcn_s_waitcnt(0x0F7A);  // vmcnt(10)
      const uint16_t raw = ((const uint16_t*)qstage)[l];
      if constexpr (kPrep) {
        // RoPE frequency of lane l (the table is in the kernel arguments,
        // read as scalars and selected per lane)
        // (readfirstlane keeps the compiler from turning the selects back
        // into a per-lane load)
        float invf = 0.f;
#pragma unroll
        for (int k = 0; k < D / 2; k++) {
          const float fk = __builtin_bit_cast(
              float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, a.prep.rt.invf[k])));
          invf = (l & 31) == k ? fk : invf;
        }
        float sn, cs;
        rope_sincos_f(invf, a.qpos, sn, cs);
        const uint16_t wq = ((const uint16_t*)(qstage + 4096))[l];
        sq[w * D + l] = qk_norm_rope_sc(h2f(raw), h2f(wq), l, sn, cs, a.prep.eps);
      } else {
        sq[w * D + l] = raw;
      }
      if (w == 0) sq[GQA * D + l] = 0;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): LDS stores done (DMA still in flight)
    __builtin_amdgcn_s_barrier();        // B1: q rows in LDS
    // range mode: the wave's partial of its first split (sml / sO) starts
    // empty (l = 0; the merge skips empty partials), the second's is marked
    // after the stream (f1: written)
    bool f1 = false;
    if constexpr (kSplit)
      if (kRange && l < GQA) sml[w * GQA + l] = f32x2{-1e30f, 0.f};
    // B operand of S^T: lane (c, n = 4b + i) holds head i's dims when b == c
    f16x8 qop[8];
    {
      const int qoff = ((n >> 2) == c ? (n & 3) * D : GQA * D) * 2;
#pragma unroll
      for (int m = 0; m < 8; m++)
        qop[m] = *(const f16x8*)((const uint8_t*)sq + qoff + 16 * m);
    }
    // per-lane LDS offsets: K reads (key 16 (n & 3) + (n >> 2) + 4c), V
    // transposed reads (lane 2k + h of a 16-lane block: key
    // 64 (k >> 2) + 16 (k & 3) + 4 beta + c, dims 8h..8h+7 of the chunk)
    const int krd = (n & 3) * kBlkB + 64 * ((n >> 2) + 4 * c);
    int vrd[4];
    {
      const int k = n >> 1, h = n & 1;
      const int base = (k >> 2) * ts + (k & 3) * kBlkB + 64 * c + 8 * h;
#pragma unroll
      for (int mu = 0; mu < 4; mu++) vrd[mu] = base + 256 * ((c + mu) & 3);
    }
    float mx = -1e30f, lsum = 0.f;  // head n & 3, replicated over its 16 lanes
    f32x4 O[4];                     // [dims 16 delta + n][rows (block c, head v)]
#pragma unroll
    for (int d = 0; d < 4; d++) O[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    const f16x2 one2 = f16x2{(_Float16)1.0f, (_Float16)1.0f};
    // One unit (slot = which scale slot holds its scales): wait for its
    // scales and K, fetch its V, S^T, then (kMore) the next unit's scales and
    // K once this unit's K is read; softmax; wait for V; P V.  No load sits
    // under a branch, so every wait is exact.
    // the unit's group range end (ge), key range (split mode: [ka, kb)) and
    // the next unit (un, its range end une) -- set before each call
    int ge = g1, ka = 0, kb = 0, un = 0, une = g1;
    const int koff = 4 * (n >> 2) + c;  // key of output element v: 16 v + koff of the tile
    // kVPre: the unit's V went out already (after the previous unit's P V,
    // as its last 8 DMAs): wait for the scales and K only
    auto unit = [&](int u, int slot, auto more_tag, auto vpre_tag) {
      constexpr bool kMore = decltype(more_tag)::value;
      constexpr bool kVPre = decltype(vpre_tag)::value;
      const bool t1ok = u + 1 < ge;
      // ---- S^T = K Q^T once the scales and K landed; V goes out now
      if constexpr (kVPre) {
        __builtin_amdgcn_s_waitcnt(0x0F78);  // vmcnt(8): all but this unit's V
      } else {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        __builtin_amdgcn_sched_barrier(0);
        if (!xw) issue(u, ge, rv, vw);
      }
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t* scl = (const uint32_t*)(sw + slot * 2 * kScaleB);
      const int sh = scale_shift(u);  // (then group u + 1 is masked)
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
        // this unit's K (and the other scale slot) fully read: the next
        // unit's may overwrite them
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_sched_barrier(0);
        issue_scales(un, sw + (slot ^ 1) * 2 * kScaleB);
        issue(un, une, rk, kw);
        __builtin_amdgcn_sched_barrier(0);
      }
      // ---- online softmax over the unit's 128 keys (4 per lane and tile)
      float rmx = -1e30f;
#pragma unroll
      for (int t = 0; t < 2; t++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
          S[t][v] *= t ? ks1 : ks0;
          if (t == 1 && !t1ok) S[t][v] = -1e30f;
          if constexpr (kSplit) {
            const int key = (u + t) * G + 16 * v + koff;
            if (key < ka || key >= kb) S[t][v] = -1e30f;
          }
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
      // corrections of the four heads (lanes 0..3 are heads 0..3)
      float oc[4];
#pragma unroll
      for (int v = 0; v < 4; v++)
        oc[v] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, corr), v));
      // ---- O = O corr + (P sv) V
      if constexpr (kMore) __builtin_amdgcn_s_waitcnt(0x0F7A);  // vmcnt(10): next scales + K in flight
      else __builtin_amdgcn_s_waitcnt(0x0F70);                  // vmcnt(0)
      f32x4 T[4];
#pragma unroll
      for (int d = 0; d < 4; d++) T[d] = f32x4{0.f, 0.f, 0.f, 0.f};
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
    int slot = 0;
    if constexpr (!kSplit) {
      using T_ = std::integral_constant<bool, true>;
      using F_ = std::integral_constant<bool, false>;
      int u = g0;
      if (u + 2 < g1) {
        // the first unit, then each next one with its V sent once the
        // previous unit's P V has read the V buffer
        un = u + 2;
        unit(u, slot, T_{}, F_{});
        issue(un, g1, rv, vw);
        for (u += 2, slot ^= 1; u + 2 < g1; u += 2, slot ^= 1) {
          un = u + 2;
          unit(u, slot, T_{}, T_{});
          issue(un, g1, rv, vw);
        }
        unit(u, slot, F_{}, T_{});
      } else if (u < g1) {
        unit(u, slot, F_{}, F_{});
      }
    } else {
      // a finished split (or share): its (m, l, o) per head, then a fresh state
      auto flush = [&](int sp) {
        // the four key blocks summed: lane l holds head hl = l >> 4, dim
        // 16 d + dl of Oc[d]
        const int hl = l >> 4, dl = l & 15;
        float Oc[4];
#pragma unroll
        for (int d = 0; d < 4; d++) Oc[d] = col4_sum4(O[d][0], O[d][1], O[d][2], O[d][3]);
        if (kRange && sp > s0) {
          // range mode, the wave's second split (always its last): its
          // partial into the wave's own K tile, free once the stream is done
          float* x = (float*)(lds + kLdsK + (w & 7) * kHalfB);
#pragma unroll
          for (int d = 0; d < 4; d++) x[hl * kPartRow + 4 + 16 * d + dl] = Oc[d];
          if (l < GQA) {
            x[l * kPartRow] = mx;
            x[l * kPartRow + 1] = lsum;
          }
          f1 = true;
        } else if (ns >= kFpWaves) {  // (then every split has one wave; else all go through the merge)
#pragma unroll
          for (int d = 0; d < 4; d++) a.po[((size_t)(g * GQA + hl) * a.nsplit + sp) * D + 16 * d + dl] = Oc[d];
          if (l < GQA) {
            a.pm[(g * GQA + l) * a.nsplit + sp] = lsum > 0.f ? mx * kLn2 : -1e30f;
            a.pl[(g * GQA + l) * a.nsplit + sp] = lsum;
          }
        } else {
#pragma unroll
          for (int d = 0; d < 4; d++) sO[(w * GQA + hl) * D + 16 * d + dl] = Oc[d];
          if (l < GQA) sml[w * GQA + l] = f32x2{mx, lsum};
        }
        mx = -1e30f;
        lsum = 0.f;
#pragma unroll
        for (int d = 0; d < 4; d++) O[d] = f32x4{0.f, 0.f, 0.f, 0.f};
      };
      int sp = sa;
      bool vpre = false;  // the current unit's V already sent
      if (sp < sb) seg_keys(sp, ka, kb);
      ge = (kb + G - 1) / G;
      int u = ka < kb ? ka / G : -1;
      while (sp < sb) {
        if (u >= 0) {
          // the next unit: in this split, else the first of a later split with keys
          un = -1;
          if (u + 2 < ge) {
            un = u + 2;
            une = ge;
          } else {
            for (int s2 = sp + 1; s2 < sb; s2++) {
              int ka2, kb2;
              seg_keys(s2, ka2, kb2);
              if (ka2 < kb2) {
                un = ka2 / G;
                une = (kb2 + G - 1) / G;
                break;
              }
            }
          }
          using T_ = std::integral_constant<bool, true>;
          using F_ = std::integral_constant<bool, false>;
          if (un >= 0) {
            if (vpre) unit(u, slot, T_{}, T_{});
            else unit(u, slot, T_{}, F_{});
          } else {
            if (vpre) unit(u, slot, F_{}, T_{});
            else unit(u, slot, F_{}, F_{});
          }
          slot ^= 1;
          if (u + 2 < ge) {
            // the next unit's V, once this unit's P V has read the buffer
            issue(un, une, rv, vw);
            vpre = true;
            u += 2;
            continue;
          }
        }
        flush(sp);
        if (++sp >= sb) break;
        seg_keys(sp, ka, kb);
        ge = (kb + G - 1) / G;
        u = ka < kb ? ka / G : -1;
        // the next split's first unit's V (after the flush's stores, so that
        // V stays the last 8 DMAs the unit start may leave outstanding)
        vpre = false;
        if (u >= 0 && un >= 0) {
          issue(un, une, rv, vw);
          vpre = true;
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // (a wave without units: its fetch done)
    if constexpr (kSplit) {
      if (kRange && !f1 && l < GQA) {
        float* x = (float*)(lds + kLdsK + (w & 7) * kHalfB);
        x[l * kPartRow] = -1e30f;
        x[l * kPartRow + 1] = 0.f;
      }
    }
    if constexpr (!kSplit) {
      // ---- the four key blocks of each (head, dim) summed: lane l holds
      // head l >> 4, dim 16 delta + (l & 15)
#pragma unroll
      for (int d = 0; d < 4; d++)
        sO[(w * GQA + (l >> 4)) * D + 16 * d + (l & 15)] = col4_sum4(O[d][0], O[d][1], O[d][2], O[d][3]);
      if (l < GQA) sml[w * GQA + l] = f32x2{mx, lsum};
    }
  } else if constexpr (kSplit) {
    // ================================================ split mode: tail waves
    // wave i = query head 4g + i takes the tail keys of each split in
    // [tlo, thi]: an (m, l, o) partial in log2 units, as the FP8 waves', in
    // the extra wave's LDS buffer (unused here) for the split's writer.
    // Scores lane = tail key (fp32 fma chain from the fp16 rows), o lane = dim.
    const int i = w - kFpWaves, h = g * GQA + i;
    const int tt = a.total - a.committed;
    float* sT = (float*)(lds + kLdsX);  // [2][4][kPartRow]
    // B1 first: the FP8 waves' streams wait on it, and nothing here is needed there
    __builtin_amdgcn_s_barrier();  // B1 (the FP8 waves'; nothing to wait for here)
    // V rows of the tail (lane = dim): every load out before any is used, so
    // they take one round trip.  All 64 rows of the tail buffer are read (one
    // base, constant row offsets); rows past the tail are dropped below.
    uint16_t vr[G];
    const uint16_t* vt = a.vtail + (size_t)g * D + l;
#pragma unroll
    for (int k = 0; k < G; k++) vr[k] = vt[(size_t)k * NKV * D];
    float sc = -1e30f;
    if (l < tt) {
      const uint16_t* kp = a.ktail + ((size_t)l * NKV + g) * D;
      const uint16_t* qp = a.q + (size_t)h * D;
      float acc = 0.f;
#pragma unroll
      for (int d = 0; d < D; d += 8) {
        const u32x4 kk = *(const u32x4*)(kp + d), qq = *(const u32x4*)(qp + d);
#pragma unroll
        for (int e = 0; e < 4; e++) {
          acc = __builtin_fmaf(h2f((uint16_t)qq[e]), h2f((uint16_t)kk[e]), acc);
          acc = __builtin_fmaf(h2f((uint16_t)(qq[e] >> 16)), h2f((uint16_t)(kk[e] >> 16)), acc);
        }
      }
      sc = acc * qscale;
    }
    float vv[G];
#pragma unroll
    for (int k = 0; k < G; k++) vv[k] = k < tt ? h2f(vr[k]) : 0.f;
    for (int sp = tlo; sp <= thi; sp++) {
      // the split's tail keys, as tail rows [k0, k1)
      const int k0 = max(a.committed, sp * a.chunk) - a.committed;
      const int k1 = min(a.total, (sp + 1) * a.chunk) - a.committed;
      const bool in = l >= k0 && l < k1;
      const float mt = wave_max_fast(in ? sc : -1e30f);
      const float p = in ? __builtin_amdgcn_exp2f(sc - mt) : 0.f;
      const float lt = wave_sum_fast(p);
      float ot = 0.f;
#pragma unroll
      for (int k = 0; k < G; k++) {
        const float pk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), k));
        ot = __builtin_fmaf(pk, vv[k], ot);  // (p is 0 outside [k0, k1), vv 0 past the tail)
      }
      float* row = sT + ((sp - tlo) * GQA + i) * kPartRow;
      row[4 + l] = ot;
      if (l == 0) {
        row[0] = mt;
        row[1] = lt;
      }
    }
  } else if constexpr (!kSplit) {
    // ============================================================ tail waves
    const int i = w - kFpWaves;  // query head 4g + i
    const int tt = a.qpos + 1 - a.committed;  // tail keys (the fresh token last)
    const bool fresh = a.knew != nullptr;
    const bool commit = fresh && tt == G;
    const int nold = fresh ? tt - 1 : tt;  // rows already in the tail buffer
    // (the step that commits the group and the others in separate code:
    // their registers never meet)
    auto tail_wave = [&](auto commit_tag) __attribute__((always_inline)) {
      constexpr bool kCommit = decltype(commit_tag)::value;
      // the old rows in one batch (tail_k_load / tail_v_load: rows from
      // nold on read as zero), before B1; on the committing step the V rows
      // load after the scores (the K quantisation needs the registers)
      u32x4 kq[8], qq[8];
      uint32_t vr[G / 2];
      tail_k_load(a.ktail, g, nold, kq);
      if constexpr (!kCommit) tail_v_load(a.vtail, g, nold, vr);
      const uint32_t fv = fresh ? *(const uint32_t*)(a.vnew + g * D + 2 * (l & 31)) : 0u;
      if (fresh && i == 0) {
        // the fresh token: k prepared when raw, kept in LDS for the scores and
        // written into its tail row with v (engine.cu:190-198)
        const uint16_t kraw = a.knew[g * D + l];
        uint16_t kv;
        if constexpr (kPrep)
          kv = qk_norm_rope_lane(h2f(kraw), h2f(a.prep.kw[l]), l, a.qpos, a.prep.eps, a.prep.rt);
        else
          kv = kraw;
        skn[l] = kv;
        a.ktail[((size_t)(tt - 1) * NKV + g) * D + l] = kv;
        a.vtail[((size_t)(tt - 1) * NKV + g) * D + l] = a.vnew[g * D + l];
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_s_barrier();  // B1: q rows and the fresh k in LDS
      // ---- scores: lane = key
      const bool live = l < tt;
#pragma unroll
      for (int cc = 0; cc < 8; cc++) qq[cc] = *(const u32x4*)(sq + i * D + 8 * cc);
      if (fresh && l == tt - 1) {
#pragma unroll
        for (int cc = 0; cc < 8; cc++) kq[cc] = *(const u32x4*)(skn + 8 * cc);
      }
      float x;
      if constexpr (!kCommit) {
        float sacc = 0.f;
#pragma unroll
        for (int cc = 0; cc < 8; cc++) {
          const f16x8 q8 = __builtin_bit_cast(f16x8, qq[cc]), k8 = __builtin_bit_cast(f16x8, kq[cc]);
          sacc = __builtin_amdgcn_fdot2(__builtin_shufflevector(q8, q8, 0, 1), __builtin_shufflevector(k8, k8, 0, 1), sacc, false);
          sacc = __builtin_amdgcn_fdot2(__builtin_shufflevector(q8, q8, 2, 3), __builtin_shufflevector(k8, k8, 2, 3), sacc, false);
          sacc = __builtin_amdgcn_fdot2(__builtin_shufflevector(q8, q8, 4, 5), __builtin_shufflevector(k8, k8, 4, 5), sacc, false);
          sacc = __builtin_amdgcn_fdot2(__builtin_shufflevector(q8, q8, 6, 7), __builtin_shufflevector(k8, k8, 6, 7), sacc, false);
        }
        x = sacc * qscale;
      } else {
        // The fresh token fills the group: kv_commit_group (engine.cu:202-228)
        // of kv head g, and the group is attended in its FP8 form.  Lane l
        // quantises key l; wave 0 writes the bytes and the scale.
        float kf[D];
#pragma unroll
        for (int cc = 0; cc < 8; cc++)
#pragma unroll
          for (int e = 0; e < 4; e++) {
            kf[8 * cc + 2 * e] = h2f((uint16_t)kq[cc][e]);
            kf[8 * cc + 2 * e + 1] = h2f((uint16_t)(kq[cc][e] >> 16));
          }
        float ak = 0.f;
#pragma unroll
        for (int d = 0; d < D; d++) ak = __builtin_fmaxf(ak, __builtin_fabsf(kf[d]));
        const float sck = quant_scale(wave_max_fast(ak));
        const uint16_t skh = f2h(sck);
        const float kdq = h2f(skh);
        uint8_t* krow8 = a.kc8 + ((size_t)(a.committed + l) * NKV + g) * D;
        float sacc = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j++) {
          const uint32_t kb = e4m3x4(kf[4 * j] / sck, kf[4 * j + 1] / sck, kf[4 * j + 2] / sck,
                                     kf[4 * j + 3] / sck);
          const f16x8 q8 = __builtin_bit_cast(f16x8, qq[j >> 1]);
          const int o4 = (j & 1) * 4;
          sacc = __builtin_fmaf((float)q8[o4 + 0], e4m3_to_f32<0>(kb) * kdq, sacc);
          sacc = __builtin_fmaf((float)q8[o4 + 1], e4m3_to_f32<1>(kb) * kdq, sacc);
          sacc = __builtin_fmaf((float)q8[o4 + 2], e4m3_to_f32<2>(kb) * kdq, sacc);
          sacc = __builtin_fmaf((float)q8[o4 + 3], e4m3_to_f32<3>(kb) * kdq, sacc);
          if (i == 0) *(uint32_t*)(krow8 + 4 * j) = kb;
        }
        if (i == 0 && l == 0) a.ksc[(a.committed / G) * NKV + g] = skh;
        x = sacc * qscale;
      }
      x = live ? x : -1e30f;
      const float M = wave_max_fast(x);
      const float p = live ? __builtin_amdgcn_exp2f(sub_rn(x, M)) : 0.f;
      const float L = wave_sum_fast(p);
      // ---- P V (tail_pv: rows summed per parity, then even + odd)
      if constexpr (!kCommit) {
        const f32x2 o = tail_pv(vr, p, fresh ? tt - 1 : -1, fv);
        if (l < 32) *(f32x2*)(sO + (kFpWaves * GQA + i) * D + 2 * l) = o;
      } else {
        // the whole group (tt == 64): V quantised with its group scale;
        // lane = dim, row 63 the fresh one; P V in tail_pv's order
        float vv[G];
#pragma unroll
        for (int k = 0; k < G; k++) {
          const uint16_t* vp = k == G - 1 ? a.vnew + g * D : a.vtail + ((size_t)k * NKV + g) * D;
          vv[k] = h2f(vp[l]);
        }
        float av = 0.f;
#pragma unroll
        for (int k = 0; k < G; k++) av = __builtin_fmaxf(av, __builtin_fabsf(vv[k]));
        const float scv = quant_scale(wave_max_fast(av));
        const uint16_t svh = f2h(scv);
        const float vdq = h2f(svh);
        float oe = 0.f, oo = 0.f;
#pragma unroll
        for (int k = 0; k < G; k++) {
          const uint32_t vb = e4m3x2(vv[k] / scv, 0.f) & 0xFFu;
          if (i == 0) a.vc8[((size_t)(a.committed + k) * NKV + g) * D + l] = (uint8_t)vb;
          const float pk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, p), k));
          if (k & 1) oo = __builtin_fmaf(pk, e4m3_to_f32<0>(vb) * vdq, oo);
          else oe = __builtin_fmaf(pk, e4m3_to_f32<0>(vb) * vdq, oe);
        }
        if (i == 0 && l == 0) a.vsc[(a.committed / G) * NKV + g] = svh;
        sO[(kFpWaves * GQA + i) * D + l] = oe + oo;
      }
      if (l == 0) sml[kFpWaves * GQA + i] = f32x2{M, L};
    };
    using T_ = std::integral_constant<bool, true>;
    using F_ = std::integral_constant<bool, false>;
    if (commit)
      tail_wave(T_{});
    else
      tail_wave(F_{});
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();  // B2: every wave's partial in LDS

  // ================================================================ merge
  if (w >= kFpWaves) return;  // (tail waves: their partial is in LDS)
  if constexpr (kSplit) {
    // the shares' workspace: the caller's, else the library's device array
    float* const part = a.part ? a.part : (float*)split_scratch;
    uint32_t* const cnt = a.part ? a.cnt : (uint32_t*)(split_scratch + 2 * kPartBytes);
    // the tail waves' partial of split sp (head i, dim d) folded into a
    // split's (M, L, O) in log2 units
    auto fold_tail = [&](int sp, int i, int d, float& M, float& L, float& O) {
      const float* row = (const float*)(lds + kLdsX) + ((sp - tlo) * GQA + i) * kPartRow;
      const float mt = row[0], lt = row[1], ot = row[4 + d];
      const float Mn = __builtin_fmaxf(M, mt);
      const float w0 = L > 0.f ? __builtin_amdgcn_exp2f(M - Mn) : 0.f;
      const float w1 = __builtin_amdgcn_exp2f(mt - Mn);
      L = __builtin_fmaf(L, w0, lt * w1);
      O = __builtin_fmaf(O, w0, ot * w1);
      M = Mn;
    };
    if constexpr (kRange) {
      // ---- range mode.  Threads jg = tid / 256 (head i, dim d) take the
      // workgroup's splits s0 + jg and s0 + jg + 2 (the last range's split of
      // tail keys only).  A split's writers are the ranges owning its first
      // and last committed group (a split of tail keys only: the last range).
      const int jg = tid >> 8, i = (tid >> 6) & 3, d = tid & 63, h = g * GQA + i;
      auto owner = [&](int x) {  // the range holding committed group x
        return (int)(((unsigned)(x + 1) * (unsigned)R + (unsigned)a.ng - 1) / (unsigned)a.ng) - 1;
      };
      auto writers = [&](int sp, int& rl, int& rh) {
        const int k0 = sp * a.chunk, k1 = min(min(k0 + a.chunk, a.total), a.committed);
        if (k0 >= k1) {
          rl = rh = R - 1;
          return;
        }
        rl = owner(k0 / G);
        rh = owner((k1 - 1) / G);
      };
      auto write_split = [&](int sp, float M, float L, float O) {
        const size_t pi = (size_t)h * a.nsplit + sp;
        a.po[pi * D + d] = O;
        if (d == 0) {
          a.pm[pi] = L > 0.f ? M * kLn2 : -1e30f;
          a.pl[pi] = L;
        }
      };
      for (int j = jg; j < ns; j += 2) {
        const int sp = s0 + j;
        // the workgroup's share: its waves' partials in wave order (slot 0 in
        // sml / sO, slot 1 in each wave's K tile; a split of tail keys only
        // has none)
        float M = -1e30f, L = 0.f, O = 0.f;
        if (j < 2) {
          for (int p = 0; p < kFpWaves; p++) {
            float mp, lp, op;
            if (j == 0) {
              mp = sml[p * GQA + i][0];
              lp = sml[p * GQA + i][1];
              op = sO[(p * GQA + i) * D + d];
            } else {
              const float* x = (const float*)(lds + kLdsK + p * kHalfB) + i * kPartRow;
              mp = x[0];
              lp = x[1];
              op = x[4 + d];
            }
            if (lp > 0.f) {
              const float Mn = __builtin_fmaxf(M, mp);
              const float c0 = L > 0.f ? __builtin_amdgcn_exp2f(M - Mn) : 0.f;
              const float c1 = __builtin_amdgcn_exp2f(mp - Mn);
              L = __builtin_fmaf(L, c0, lp * c1);
              O = __builtin_fmaf(O, c0, op * c1);
              M = Mn;
            }
          }
        }
        int rl, rh;
        writers(sp, rl, rh);
        if (rl == rh) {  // this workgroup's alone
          if (sp >= tlo && sp <= thi) fold_tail(sp, i, d, M, L, O);
          write_split(sp, M, L, O);
        } else {
          float* row = part + ((size_t)(g * 2 * kMaxRanges + 2 * r + j) * GQA + i) * kPartRow;
          __hip_atomic_store(row + 4 + d, O, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (d == 0) {
            __hip_atomic_store(row, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(row + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
      stores_acked();  // the shares have reached the agent
      __builtin_amdgcn_s_barrier();        // the workgroup's shares stored
      // a ticket per shared split: lane 0 of waves 0 and 1 (splits s0, s0 + 1)
      uint32_t* sticket = (uint32_t*)(lds + kLdsTicket);
      if (w < 2 && l == 0 && w < ns) {
        int rl, rh;
        writers(s0 + w, rl, rh);
        if (rl != rh)
          sticket[w] = __hip_atomic_fetch_add(cnt + g * kCntStride + s0 + w, 1u, __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT);
      }
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_s_barrier();
      if (jg < ns) {
        const int j = jg, sp = s0 + j;
        int rl, rh;
        writers(sp, rl, rh);
        if (rl == rh || sticket[j] != (uint32_t)(rh - rl)) return;
        // ---- the last share of split sp to arrive: every share stored.  The
        // counter goes back to zero for the next call.  Shares in range order.
        if (i == 0 && d == 0)
          __hip_atomic_store(cnt + g * kCntStride + sp, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const __amdgpu_buffer_rsrc_t rs = buf_rsrc(part + (size_t)g * 2 * kMaxRanges * GQA * kPartRow);
        float M = -1e30f, L = 0.f, O = 0.f;
        for (int p0 = rl; p0 <= rh; p0 += 8) {
          float mp[8], lp[8], op[8];
#pragma unroll
          for (int k = 0; k < 8; k++) {
            const int rr = p0 + k <= rh ? p0 + k : p0;
            const int ga = (int)(((unsigned)rr * (unsigned)a.ng) / (unsigned)R);
            const int slot = 2 * rr + (sp - ga * G / a.chunk);
            const int o = (slot * GQA + i) * kPartRow;
            mp[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, o * 4, 0, kCoherent));
            lp[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (o + 1) * 4, 0, kCoherent));
            op[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (o + 4 + d) * 4, 0, kCoherent));
          }
#pragma unroll
          for (int k = 0; k < 8; k++) {
            if (p0 + k <= rh && lp[k] > 0.f) {
              const float Mn = __builtin_fmaxf(M, mp[k]);
              const float c0 = L > 0.f ? __builtin_amdgcn_exp2f(M - Mn) : 0.f;
              const float c1 = __builtin_amdgcn_exp2f(mp[k] - Mn);
              L = __builtin_fmaf(L, c0, lp[k] * c1);
              O = __builtin_fmaf(O, c0, op[k] * c1);
              M = Mn;
            }
          }
        }
        if (sp >= tlo && sp <= thi) fold_tail(sp, i, d, M, L, O);
        write_split(sp, M, L, O);
      }
      return;
    }
    if (ns >= kFpWaves) {
      // the FP8 waves wrote their splits straight out (before B2): waves
      // 0-3 (head i = w, lane = dim) fold the tail into the tail splits
      if (tlo > thi || tid >= GQA * D) return;
      const int i = tid >> 6, d = tid & 63, h = g * GQA + i;
      for (int sp = tlo; sp <= thi; sp++) {
        const size_t pi = (size_t)h * a.nsplit + sp;
        const float m0 = __hip_atomic_load(a.pm + pi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float l0 = __hip_atomic_load(a.pl + pi, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const float o0 = __hip_atomic_load(a.po + pi * D + d, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        float M = l0 > 0.f ? m0 * kLog2e : -1e30f, L = l0, O = o0;
        fold_tail(sp, i, d, M, L, O);
        a.po[pi * D + d] = O;
        if (d == 0) {
          a.pm[pi] = L > 0.f ? M * kLn2 : -1e30f;
          a.pl[pi] = L;
        }
      }
      return;
    }
    // splits shared by several waves (at most 7 splits here): merge the
    // shares of each, head i = tid / 64, dim d
    if (ns < kFpWaves && tid < GQA * D) {
      const int i = tid >> 6, d = tid & 63, h = g * GQA + i;
      for (int j = 0; j < ns; j++) {
        const int fw = (j * kFpWaves + ns - 1) / ns, lw = ((j + 1) * kFpWaves + ns - 1) / ns;
        float M = -1e30f;
        for (int p = fw; p < lw; p++) M = __builtin_fmaxf(M, sml[p * GQA + i][0]);
        float L = 0.f, Oacc = 0.f;
        for (int p = fw; p < lw; p++) {
          const float wt = __builtin_amdgcn_exp2f(sml[p * GQA + i][0] - M);
          L = __builtin_fmaf(sml[p * GQA + i][1], wt, L);
          Oacc = __builtin_fmaf(sO[(p * GQA + i) * D + d], wt, Oacc);
        }
        const int sp = s0 + j;
        if (a.sub <= 1 && sp >= tlo && sp <= thi) fold_tail(sp, i, d, M, L, Oacc);
        if (a.sub > 1) {
          // this workgroup's share of the split, for the last to arrive
          float* row = part + ((size_t)(g * kMaxRanges + r) * GQA + i) * kPartRow;
          __hip_atomic_store(row + 4 + d, Oacc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          if (d == 0) {
            __hip_atomic_store(row, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(row + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          stores_acked();
          continue;
        }
        a.po[((size_t)h * a.nsplit + sp) * D + d] = Oacc;
        if (d == 0) {
          a.pm[h * a.nsplit + sp] = L > 0.f ? M * kLn2 : -1e30f;
          a.pl[h * a.nsplit + sp] = L;
        }
      }
    }
    if (a.sub <= 1) return;
    __builtin_amdgcn_s_barrier();  // the workgroup's share stored
    uint32_t* ctr = cnt + g * kCntStride + s0;
    uint32_t* sticket = (uint32_t*)(lds + kLdsTicket);
    if (tid == 0) *sticket = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    if (*sticket != (uint32_t)(a.sub - 1)) return;
    // ---- the last share of split s0 to arrive: every share stored.  The
    // counter goes back to zero for the next call.
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid < GQA * D) {
      const int i = tid >> 6, d = tid & 63, h = g * GQA + i;
      const __amdgpu_buffer_rsrc_t rs =
          buf_rsrc(part + (size_t)(g * kMaxRanges + s0 * a.sub) * GQA * kPartRow);
      // shares 8 at a time (the loads of a batch go out together)
      float M = -1e30f, L = 0.f, O = 0.f;
      for (int p0 = 0; p0 < a.sub; p0 += 8) {
        float mp[8], lp[8], op[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
          const int o = ((p0 + k < a.sub ? p0 + k : p0) * GQA + i) * kPartRow;
          mp[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, o * 4, 0, kCoherent));
          lp[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (o + 1) * 4, 0, kCoherent));
          op[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, (o + 4 + d) * 4, 0, kCoherent));
        }
        float Mb = M;
#pragma unroll
        for (int k = 0; k < 8; k++) Mb = p0 + k < a.sub ? __builtin_fmaxf(Mb, mp[k]) : Mb;
        const float c = __builtin_amdgcn_exp2f(M - Mb);
        L *= c;
        O *= c;
#pragma unroll
        for (int k = 0; k < 8; k++) {
          const float wt = p0 + k < a.sub ? __builtin_amdgcn_exp2f(mp[k] - Mb) : 0.f;
          L = __builtin_fmaf(lp[k], wt, L);
          O = __builtin_fmaf(op[k], wt, O);
        }
        M = Mb;
      }
      if (s0 >= tlo && s0 <= thi) fold_tail(s0, i, d, M, L, O);
      a.po[((size_t)h * a.nsplit + s0) * D + d] = O;
      if (d == 0) {
        a.pm[h * a.nsplit + s0] = L > 0.f ? M * kLn2 : -1e30f;
        a.pl[h * a.nsplit + s0] = L;
      }
    }
    return;
  }
  float* pg = a.part + (size_t)g * kMaxRanges * kPartF;  // kv head g's partials
  if (tid < GQA * D) {
    // the workgroup's partial of (head 4g + i, dim d)
    const int i = tid >> 6, d = tid & 63;
    const int np = r == 0 || r <= ne ? kFpWaves + 1 : kFpWaves;
    // (every read first, then the arithmetic: the reads go out together)
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
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int p = 0; p <= kFpWaves; p++) {
      const float wt = p < np ? __builtin_amdgcn_exp2f(ml[p][0] - M) : 0.f;
      L = __builtin_fmaf(ml[p][1], wt, L);
      O = __builtin_fmaf(ov[p], wt, O);
    }
    if (R == 1) {
      a.out[(size_t)(g * GQA + i) * D + d] = f2h(O * (1.0f / L));
    } else {
      float* row = pg + (size_t)(r * GQA + i) * kPartRow;
      __hip_atomic_store(row + 4 + d, O, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (d == 0) {
        __hip_atomic_store(row, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(row + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      stores_acked();
    }
  }
  if (R == 1) return;
  __builtin_amdgcn_s_barrier();  // B3: the workgroup's partial stored
  uint32_t* ctr = a.cnt + g * kCntStride;
  uint32_t* sticket = (uint32_t*)(lds + kLdsTicket);
  if (tid == 0) *sticket = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();  // B4
  if (*sticket != (uint32_t)(R - 1)) return;
  // ---- the last workgroup of kv head g to arrive: every partial stored.
  // The counter goes back to zero for the next call.
  if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float* sp = (float*)(lds + kLdsK);  // [R][4][kPartRow] (the K tiles are free)
  {
    // the R partials, 16 bytes per load, one batch per thread
    constexpr int kPer = (kMaxRanges * kPartF / 4 + 64 * kFpWaves - 1) / (64 * kFpWaves);
    const int nvec = R * (kPartF / 4);
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(pg);
    u32x4 v[kPer];
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      const int e = tid + 64 * kFpWaves * k;
      v[k] = __builtin_amdgcn_raw_buffer_load_b128(rs, (e < nvec ? e : 0) * 16, 0, kCoherent);
    }
#pragma unroll
    for (int k = 0; k < kPer; k++) {
      const int e = tid + 64 * kFpWaves * k;
      if (e < nvec) *(u32x4*)(sp + 4 * e) = v[k];
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();  // B5
  if (tid < GQA * D) {
    // wave i = query head 4g + i: lane p weighs partial p, then lane d sums
    // dim d (the row reads go out together; the weights come from lane p)
    // (NP: 32 partials, or kMaxRanges for the unequal ranges; the terms past
    // R weigh 0 and leave the sum's bits as they are)
    const int i = w, lane = l;
    auto finish = [&](auto np_tag) {
      constexpr int NP = decltype(np_tag)::value;
      const f32x2 mlp = *(const f32x2*)(sp + (size_t)((lane < R ? lane : 0) * GQA + i) * kPartRow);
      float ov[NP];
#pragma unroll
      for (int p = 0; p < NP; p++) ov[p] = sp[((p < R ? p : 0) * GQA + i) * kPartRow + 4 + lane];
      const bool ok = lane < R && mlp[1] > 0.f;
      const float M = wave_max_fast(ok ? mlp[0] : -1e30f);
      const float wt = ok ? __builtin_amdgcn_exp2f(mlp[0] - M) : 0.f;
      const float L = wave_sum_fast(ok ? mlp[1] * wt : 0.f);
      float O = 0.f;
#pragma unroll
      for (int p = 0; p < NP; p++)
        O = __builtin_fmaf(ov[p], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wt), p)), O);
      a.out[(size_t)(g * GQA + i) * D + lane] = f2h(O * (1.0f / L));
    };
    if (R <= 32)
      finish(std::integral_constant<int, 32>{});
    else
      finish(std::integral_constant<int, kMaxRanges>{});
  }
}

}  // namespace cia

using namespace cia;

extern "C" int64_t cia_decode_workspace_bytes(int max_tokens) {
  return max_tokens < 0 ? 0 : kWsBytes;
}

// Flash-decoding with the library's split and, when knew/vnew are given, the
// fresh token's tail write (and the group commit on the step it fills the
// group) fused in.  Internal entry shared by cia_attn_decode and the layer
// driver; mid_event (may be NULL) is recorded after the launch.  prep (may
// be NULL): a QkPrep when q and knew arrive raw.
extern "C" __attribute__((visibility("hidden"))) int cia_decode_mfma(
    const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8, const uint16_t* ksc,
    const uint16_t* vsc, uint16_t* ktail, uint16_t* vtail, const uint16_t* knew,
    const uint16_t* vnew, int committed, int qpos, float scale, uint16_t* out, void* ws,
    int64_t ws_bytes, void* stream, void* mid_event, const void* prep) {
  if (ws_bytes < kWsBytes) return CIA_ERR_ARG;
  if (committed % G || committed > qpos + 1 || qpos + 1 - committed > G) return CIA_ERR_STATE;
  if (knew && (!vnew || qpos + 1 - committed < 1)) return CIA_ERR_ARG;
  const int ng = committed / G, R = dec_ranges(ng);
  // groups past 16 per workgroup go one each to the extra waves
  const int ne = R > 1 ? std::min(std::max(ng - 16 * R, 0), R - 1) : 0;
  DecArgs da{q, (uint8_t*)kc8, (uint8_t*)vc8, (uint16_t*)ksc, (uint16_t*)vsc, ktail, vtail,
             knew, vnew, committed, qpos, scale, (float*)ws,
             (uint32_t*)((char*)ws + kPartBytes), out, ng, R, ne, {}, {}, {}, QkPrep{}};
  pair_ranges(ng, R, slow_pair(kc8, vc8), da.rp, da.up, da.nep);
  if (prep) da.prep = *(const QkPrep*)prep;
  hipStream_t s = (hipStream_t)stream;
  if (da.prep.qw)
    hipLaunchKernelGGL((k_decode<true, false>), dim3(NKV * R), dim3(kDecThreads), 0, s, da);
  else
    hipLaunchKernelGGL((k_decode<false, false>), dim3(NKV * R), dim3(kDecThreads), 0, s, da);
  int st = launch_status();
  if (st) return st;
  if (mid_event) {
    const hipError_t e = hipEventRecord((hipEvent_t)mid_event, s);
    if (e != hipSuccess) {
      set_hip_error(e);
      return CIA_ERR_HIP;
    }
  }
  return CIA_OK;
}

// ---------------------------------------------------------------- no allocation
// cia_attn_decode's workspace as a file-scope device array: the entry below
// allocates nothing.  Its arrival counters are zero at load; every complete
// call leaves them at zero, and the first call on a device clears them once
// more with a fill kernel.  Calls on one device share the array: calls that
// overlap (different streams, or host threads) race.
static __device__ __align__(256) uint8_t scratch[kWsBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices];  // this device's address of `scratch`

__global__ void k_zero_u32(uint32_t* p, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = 0u;
}

// the current device's copy of `scratch` (set up on its first call)
int scratch_for_device(void** out, hipStream_t s) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_hip_error(e);
    return CIA_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxDevices) return CIA_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      set_hip_error(e);
      return CIA_ERR_HIP;
    }
    hipLaunchKernelGGL(k_zero_u32, dim3(1), dim3(256), 0, s,
                       (uint32_t*)((char*)p + kPartBytes), NKV * kCntStride);
    const int st = launch_status();
    if (st) return st;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return CIA_OK;
}

// split_scratch's counters cleared by a fill kernel (no memset node, so the
// call stays capturable) on the first call on a device.  A first call made
// under stream capture records the fill into the graph (each replay clears
// the counters before its split launch, harmlessly) and leaves the device
// unmarked, so the next eager call clears them too.
__global__ void k_zero_split_counters() {
  uint32_t* c = (uint32_t*)(split_scratch + 2 * kPartBytes);
  for (int i = threadIdx.x; i < NKV * kCntStride; i += blockDim.x) c[i] = 0u;
}

std::mutex g_split_mu;
bool g_split_ready[kMaxDevices];

int split_scratch_prepare(hipStream_t s) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_hip_error(e);
    return CIA_ERR_HIP;
  }
  if (dev < 0 || dev >= kMaxDevices) return CIA_ERR_ARG;
  std::lock_guard<std::mutex> lock(g_split_mu);
  if (g_split_ready[dev]) return CIA_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(s, &cs);
  if (e != hipSuccess) {
    set_hip_error(e);
    return CIA_ERR_HIP;
  }
  hipLaunchKernelGGL(k_zero_split_counters, dim3(1), dim3(256), 0, s);
  const int st = launch_status();
  if (st) return st;
  if (cs == hipStreamCaptureStatusNone) g_split_ready[dev] = true;
  return CIA_OK;
}

}  // namespace

extern "C" int cia_attn_decode_noalloc(const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8,
                                       const uint16_t* ksc, const uint16_t* vsc,
                                       const uint16_t* ktail, const uint16_t* vtail, int committed,
                                       int qpos, float scale, uint16_t* out, void* stream) {
  CIA_REQUIRE(q && kc8 && vc8 && ksc && vsc && ktail && vtail && out, CIA_ERR_NULL);
  CIA_REQUIRE(committed >= 0 && committed % G == 0 && qpos >= 0, CIA_ERR_ARG);
  CIA_REQUIRE(aligned(q, 16) && aligned(kc8, 16) && aligned(vc8, 16) && aligned(ktail, 16) &&
                  aligned(vtail, 16) && aligned(ksc, 2) && aligned(vsc, 2) && aligned(out, 2),
              CIA_ERR_ALIGN);
  CIA_REQUIRE(committed <= qpos + 1 && qpos - committed < G, CIA_ERR_STATE);
  // the workspace this context needs must fit the array (it does for every
  // context: the partials are sized for the largest split)
  CIA_REQUIRE(cia_decode_workspace_bytes(qpos + 1) <= (int64_t)sizeof(scratch), CIA_ERR_ARG);
  void* ws = nullptr;
  const int st = scratch_for_device(&ws, (hipStream_t)stream);
  if (st) return st;
  return cia_decode_mfma(q, kc8, vc8, ksc, vsc, (uint16_t*)ktail, (uint16_t*)vtail, nullptr,
                         nullptr, committed, qpos, scale, out, ws, kWsBytes, stream, nullptr,
                         nullptr);
}

extern "C" int64_t cia_split_workspace_bytes(int nsplit) {
  return nsplit < 1 ? 0 : kSplitWsBytes;
}

// The reference's split partials on the matrix cores, one launch of
// k_decode<false, true> (the tail keys folded in by the split's writer).
// Fewer splits than ranges are each spread over several workgroups, which
// meet in ws (the caller's workspace of kSplitWsBytes, counters zeroed
// before its first use) or, when ws is NULL, in split_scratch.  Internal
// entry of cia_attn_decode_split(_ws) for nsplit <= kSplitMfmaMax
// (arguments checked there).
extern "C" __attribute__((visibility("hidden"))) int cia_split_mfma(
    const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8, const uint16_t* ksc,
    const uint16_t* vsc, const uint16_t* ktail, const uint16_t* vtail, int committed, int qpos,
    float scale, float* pm, float* pl, float* po, int nsplit, void* ws, void* stream) {
  const int total = qpos + 1, chunk = (total + nsplit - 1) / nsplit;
  // workgroups per kv head: up to one per 8 CUs; fewer splits than that
  // are each spread over sub workgroups
  int cap = kMaxRanges;
  const int cus = device_cus();
  if (cus > 0 && cus / NKV < cap) cap = cus / NKV > 0 ? cus / NKV : 1;
  int sub = nsplit < cap ? cap / nsplit : 1;
  int R = nsplit < cap ? nsplit * sub : cap;
  // Range mode, for fewer splits than workgroups when a split is at least
  // as long as a workgroup's key range: the workgroups take the decode's
  // key ranges of each kv head (unequal per head pair on long streams), a
  // range touching at most two splits; a split's shares meet in part and
  // the last workgroup to arrive writes it.
  const int ng = committed / G;
  DecArgs da{};
  if (nsplit < cap && !(cap & 1) && ng >= cap) {
    pair_ranges(ng, cap, slow_pair(kc8, vc8), da.rp, da.up, da.nep);
    int rmin = cap;
    if (da.rp[0] > 0)
      for (int p = 0; p < 4; p++) rmin = std::min(rmin, da.rp[p]);
    if ((int64_t)((ng + rmin - 1) / rmin) * G <= chunk) {
      sub = -1;
      R = cap;
      for (int p = 0; p < 4; p++) da.nep[p] = 0;
    } else {
      da.rp[0] = 0;
    }
  }
  if ((sub > 1 || sub < 0) && !ws) {
    const int st = split_scratch_prepare((hipStream_t)stream);
    if (st) return st;
  }
  da.q = q;
  da.kc8 = (uint8_t*)kc8;
  da.vc8 = (uint8_t*)vc8;
  da.ksc = (uint16_t*)ksc;
  da.vsc = (uint16_t*)vsc;
  da.ktail = (uint16_t*)ktail;
  da.vtail = (uint16_t*)vtail;
  da.committed = committed;
  da.qpos = qpos;
  da.scale = scale;
  da.ng = committed / G;
  da.R = R;
  da.pm = pm;
  da.pl = pl;
  da.po = po;
  da.nsplit = nsplit;
  da.chunk = chunk;
  da.total = total;
  da.sub = sub;
  da.part = (float*)ws;
  da.cnt = ws ? (uint32_t*)((char*)ws + 2 * kPartBytes) : nullptr;
  hipStream_t s = (hipStream_t)stream;
  if (sub < 0)
    hipLaunchKernelGGL((k_decode<false, true, true>), dim3(NKV * R), dim3(kDecThreads), 0, s, da);
  else
    hipLaunchKernelGGL((k_decode<false, true>), dim3(NKV * R), dim3(kDecThreads), 0, s, da);
  return launch_status();
}
