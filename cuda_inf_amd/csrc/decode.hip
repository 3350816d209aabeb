// decode.hip -- flash-decoding over the group-64 FP8 cache on gfx950
// (engine.cu:386-480) and the entry points of the fused causal prefill
// (engine.cu:236-308, kernel in prefill_mfma.hip) and of the matrix-core
// decode (decode_kv.hip).
//
// The reference launches one block per (query head, split) and so reads
// every K/V byte four times (once per query head of a GQA group).  Here a
// workgroup owns (kv head, split) and serves all four query heads from one
// read of each key row.  Split ranges are the reference's
// ceil((qpos+1)/nsplit) so the partials keep its [h*nsplit+split] meaning.
#include "attn_range.h"

namespace cia {

__device__ __forceinline__ void split_range(int total, int nsplit, int sp, int* a, int* b) {
  const int chunk = (total + nsplit - 1) / nsplit;
  const int ks = sp * chunk;
  *a = ks;
  *b = total < ks + chunk ? total : ks + chunk;
}

// grid = (8 kv heads, nsplit), block = 256
__global__ __launch_bounds__(256) void k_decode_split(const uint16_t* __restrict__ q,
                                                      Group64Cache c, int qpos, float scale,
                                                      float* __restrict__ pm,
                                                      float* __restrict__ pl,
                                                      float* __restrict__ po, int nsplit) {
  __shared__ float lds[kRangeLds];
  __shared__ float sM[4], sL[4], sO[4 * D];
  const int kvh = blockIdx.x, sp = blockIdx.y;
  int a, b;
  split_range(qpos + 1, nsplit, sp, &a, &b);
  attend_range(q, c, kvh, scale, a, b, lds, sM, sL, sO);
  const int j = threadIdx.x >> 6, d = threadIdx.x & 63;
  const int pi = (kvh * GQA + j) * nsplit + sp;
  po[(size_t)pi * D + d] = sO[j * D + d];
  if (d == 0) {
    pm[pi] = sM[j];
    pl[pi] = sL[j];
  }
}

// engine.cu:467-480 with runtime nsplit: the same merge (global max over the
// splits' m, splits with l <= 0 skipped, exp weights), spread over 4 blocks
// per query head (16 dims each) of 1024 threads: thread (group j, lane e)
// takes splits j, j + 64, ... of dim 16 (blockIdx.y) + e, the first four
// loaded before anything waits on them; the 4 groups of a wave are added
// with permlane swaps, then the 16 waves' sums in LDS.  grid = (32 heads, 4).
constexpr int kCombThreads = 1024;
constexpr int kCombDims = 16;
constexpr int kCombGroups = kCombThreads / kCombDims;
constexpr int kCombPre = 4;  // splits per thread held in registers

__global__ __launch_bounds__(kCombThreads) void k_decode_combine(const float* __restrict__ pm,
                                                                 const float* __restrict__ pl,
                                                                 const float* __restrict__ po,
                                                                 uint16_t* __restrict__ out,
                                                                 int nsplit) {
  constexpr int kWaves = kCombThreads / 64;
  __shared__ float sred[kWaves];
  __shared__ float sacc[kWaves][kCombDims];
  __shared__ float sl[kWaves];
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int e = tid % kCombDims, j = tid / kCombDims, d = blockIdx.y * kCombDims + e;
  const float* hm = pm + (size_t)h * nsplit;
  const float* hl = pl + (size_t)h * nsplit;
  const float* ho = po + (size_t)h * nsplit * D;
  float mv[kCombPre], lv[kCombPre], ov[kCombPre];
#pragma unroll
  for (int k = 0; k < kCombPre; k++) {
    const int s = j + kCombGroups * k;
    const int sc = s < nsplit ? s : 0;
    mv[k] = s < nsplit ? hm[sc] : -1e30f;
    lv[k] = s < nsplit ? hl[sc] : 0.f;
    ov[k] = s < nsplit ? ho[(size_t)sc * D + d] : 0.f;
  }
  float gm = -1e30f;
#pragma unroll
  for (int k = 0; k < kCombPre; k++) gm = __builtin_fmaxf(gm, mv[k]);
  for (int s = j + kCombGroups * kCombPre; s < nsplit; s += kCombGroups)
    gm = __builtin_fmaxf(gm, hm[s]);
  gm = wave_max_fast(gm);
  if (lane == 0) sred[wv] = gm;
  __syncthreads();
  gm = sred[0];
#pragma unroll
  for (int k = 1; k < kWaves; k++) gm = __builtin_fmaxf(gm, sred[k]);
  float l = 0.f, acc = 0.f;
#pragma unroll
  for (int k = 0; k < kCombPre; k++) {
    if (lv[k] > 0.f) {
      const float w = fast_exp(mv[k] - gm);
      l = __builtin_fmaf(lv[k], w, l);
      acc = __builtin_fmaf(ov[k], w, acc);
    }
  }
#pragma unroll 4
  for (int s = j + kCombGroups * kCombPre; s < nsplit; s += kCombGroups) {
    const float ls = hl[s];
    if (ls <= 0.f) continue;
    const float w = fast_exp(hm[s] - gm);
    l = __builtin_fmaf(ls, w, l);
    acc = __builtin_fmaf(ho[(size_t)s * D + d], w, acc);
  }
  // lanes e, e + 16, e + 32, e + 48 of a wave hold its 4 groups of dim e
  acc = col4_sum(acc);
  l = col4_sum(l);
  if (lane < kCombDims) {
    sacc[wv][lane] = acc;
    if (lane == 0) sl[wv] = l;
  }
  __syncthreads();
  if (tid < kCombDims) {
    float L = 0.f, A = 0.f;
#pragma unroll
    for (int k = 0; k < kWaves; k++) {
      L += sl[k];
      A += sacc[k][tid];
    }
    out[h * D + blockIdx.y * kCombDims + tid] = f2h(A / L);
  }
}

// The same merge for up to kCombSmall splits: one wave per query head.
// Lane s loads split s's m and l, lane d dim d of every split's o (all loads
// out before any is used); the global max and the weights are per-lane work
// over the splits, and each split's weight reaches the dims by readlane.
// grid = 32 heads, block = 64.
constexpr int kCombSmall = 32;
__global__ __launch_bounds__(64) void k_decode_combine_small(const float* __restrict__ pm,
                                                             const float* __restrict__ pl,
                                                             const float* __restrict__ po,
                                                             uint16_t* __restrict__ out,
                                                             int nsplit) {
  const int h = blockIdx.x, lane = threadIdx.x;
  const int ls = lane < nsplit ? lane : 0;
  const float m = pm[(size_t)h * nsplit + ls], lv = pl[(size_t)h * nsplit + ls];
  const float* ho = po + (size_t)h * nsplit * D + lane;
  float ov[kCombSmall];
#pragma unroll
  for (int s = 0; s < kCombSmall; s++) ov[s] = ho[(size_t)(s < nsplit ? s : 0) * D];
  const bool ok = lane < nsplit && lv > 0.f;  // (splits with l <= 0 are skipped)
  const float M = wave_max_fast(ok ? m : -1e30f);
  const float w = ok ? fast_exp(m - M) : 0.f;
  const float L = wave_sum_fast(ok ? lv * w : 0.f);
  float acc = 0.f;
#pragma unroll
  for (int s = 0; s < kCombSmall; s++)
    acc = __builtin_fmaf(ov[s], __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), s)), acc);
  out[h * D + lane] = f2h(acc / L);
}

}  // namespace cia

using namespace cia;

// The matrix-core split runs for up to 512 splits per head of at least 128
// keys each.  Smaller splits take the fp32 kernel above: the matrix cores
// round the softmax numerators to fp16, and a split's own output o / l over
// a handful of keys (with outlier values) would carry that rounding unaveraged.
constexpr int kSplitMfmaMax = 512;
constexpr int kSplitMfmaMinKeys = 128;
extern "C" __attribute__((visibility("hidden"))) int cia_split_mfma(
    const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8, const uint16_t* ksc,
    const uint16_t* vsc, const uint16_t* ktail, const uint16_t* vtail, int committed, int qpos,
    float scale, float* pm, float* pl, float* po, int nsplit, void* ws, void* stream);
extern "C" int64_t cia_split_workspace_bytes(int nsplit);

static int check_cache(const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8,
                       const uint16_t* ksc, const uint16_t* vsc, const uint16_t* ktail,
                       const uint16_t* vtail, int committed) {
  CIA_REQUIRE(q && kc8 && vc8 && ksc && vsc && ktail && vtail, CIA_ERR_NULL);
  CIA_REQUIRE(committed >= 0 && committed % G == 0, CIA_ERR_ARG);
  CIA_REQUIRE(aligned(q, 16) && aligned(kc8, 16) && aligned(vc8, 16) && aligned(ktail, 16) &&
                  aligned(vtail, 16) && aligned(ksc, 2) && aligned(vsc, 2),
              CIA_ERR_ALIGN);
  return CIA_OK;
}

// cia_attn_decode_split with ws (the caller's workspace, or NULL for the
// library's device array)
static int decode_split(const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8,
                        const uint16_t* ksc, const uint16_t* vsc, const uint16_t* ktail,
                        const uint16_t* vtail, int committed, int qpos, float scale, float* pm,
                        float* pl, float* po, int nsplit, void* ws, void* stream) {
  int st = check_cache(q, kc8, vc8, ksc, vsc, ktail, vtail, committed);
  if (st) return st;
  CIA_REQUIRE(pm && pl && po, CIA_ERR_NULL);
  CIA_REQUIRE(qpos >= 0 && nsplit >= 1 && nsplit <= CIA_NSPLIT_MAX, CIA_ERR_ARG);
  CIA_REQUIRE(qpos - committed < G, CIA_ERR_STATE);  // the tail holds at most 64 keys
  if (nsplit <= kSplitMfmaMax && (qpos + nsplit) / nsplit >= kSplitMfmaMinKeys)
    return cia_split_mfma(q, kc8, vc8, ksc, vsc, ktail, vtail, committed, qpos, scale, pm, pl, po,
                          nsplit, ws, stream);
  Group64Cache c{kc8, vc8, ksc, vsc, ktail, vtail, committed};
  hipLaunchKernelGGL(k_decode_split, dim3(NKV, nsplit), dim3(256), 0, (hipStream_t)stream, q, c,
                     qpos, scale, pm, pl, po, nsplit);
  return launch_status();
}

extern "C" int cia_attn_decode_split(const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8,
                                     const uint16_t* ksc, const uint16_t* vsc,
                                     const uint16_t* ktail, const uint16_t* vtail, int committed,
                                     int qpos, float scale, float* pm, float* pl, float* po,
                                     int nsplit, void* stream) {
  return decode_split(q, kc8, vc8, ksc, vsc, ktail, vtail, committed, qpos, scale, pm, pl, po,
                      nsplit, nullptr, stream);
}

extern "C" int cia_attn_decode_split_ws(const uint16_t* q, const uint8_t* kc8,
                                        const uint8_t* vc8, const uint16_t* ksc,
                                        const uint16_t* vsc, const uint16_t* ktail,
                                        const uint16_t* vtail, int committed, int qpos,
                                        float scale, float* pm, float* pl, float* po, int nsplit,
                                        void* ws, int64_t ws_bytes, void* stream) {
  CIA_REQUIRE(ws, CIA_ERR_NULL);
  CIA_REQUIRE(nsplit >= 1 && ws_bytes >= cia_split_workspace_bytes(nsplit), CIA_ERR_ARG);
  CIA_REQUIRE(aligned(ws, 16), CIA_ERR_ALIGN);
  return decode_split(q, kc8, vc8, ksc, vsc, ktail, vtail, committed, qpos, scale, pm, pl, po,
                      nsplit, ws, stream);
}

extern "C" int cia_attn_decode_combine(const float* pm, const float* pl, const float* po,
                                       uint16_t* out, int nsplit, void* stream) {
  CIA_REQUIRE(pm && pl && po && out, CIA_ERR_NULL);
  CIA_REQUIRE(nsplit >= 1 && nsplit <= CIA_NSPLIT_MAX, CIA_ERR_ARG);
  if (nsplit <= kCombSmall)
    hipLaunchKernelGGL(k_decode_combine_small, dim3(NH), dim3(64), 0, (hipStream_t)stream, pm, pl,
                       po, out, nsplit);
  else
    hipLaunchKernelGGL(k_decode_combine, dim3(NH, D / kCombDims), dim3(kCombThreads), 0,
                       (hipStream_t)stream, pm, pl, po, out, nsplit);
  return launch_status();
}

extern "C" __attribute__((visibility("hidden"))) int cia_decode_mfma(
    const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8, const uint16_t* ksc,
    const uint16_t* vsc, uint16_t* ktail, uint16_t* vtail, const uint16_t* knew,
    const uint16_t* vnew, int committed, int qpos, float scale, uint16_t* out, void* ws,
    int64_t ws_bytes, void* stream, void* mid_event, const void* prep);

extern "C" int cia_attn_decode(const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8,
                               const uint16_t* ksc, const uint16_t* vsc, const uint16_t* ktail,
                               const uint16_t* vtail, int committed, int qpos, float scale,
                               uint16_t* out, void* ws, int64_t ws_bytes, void* stream) {
  int st = check_cache(q, kc8, vc8, ksc, vsc, ktail, vtail, committed);
  if (st) return st;
  CIA_REQUIRE(out && ws, CIA_ERR_NULL);
  CIA_REQUIRE(aligned(ws, 16) && aligned(out, 2), CIA_ERR_ALIGN);
  CIA_REQUIRE(qpos >= 0 && ws_bytes >= 0, CIA_ERR_ARG);
  CIA_REQUIRE(committed <= qpos + 1 && qpos - committed < G, CIA_ERR_STATE);
  return cia_decode_mfma(q, kc8, vc8, ksc, vsc, (uint16_t*)ktail, (uint16_t*)vtail, nullptr,
                         nullptr, committed, qpos, scale, out, ws, ws_bytes, stream, nullptr,
                         nullptr);
}

// attn_sum support lives in mass.hip
extern "C" __attribute__((visibility("hidden"))) int cia_mass_group64(const uint16_t* q, const uint8_t* kc8, const uint16_t* ksc,
                                const uint16_t* ktail, int committed, float* attn_sum, int S,
                                int past, float scale, void* ws, void* stream);

extern "C" __attribute__((visibility("hidden"))) int cia_prefill_mfma(
    const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8, const uint16_t* ksc,
    const uint16_t* vsc, const uint16_t* ktail, const uint16_t* vtail, int committed,
    uint16_t* out, int S, int past, float scale, void* stream);

extern "C" int cia_attention_fused(const uint16_t* q, const uint8_t* kc8, const uint8_t* vc8,
                                   const uint16_t* ksc, const uint16_t* vsc,
                                   const uint16_t* ktail, const uint16_t* vtail, int committed,
                                   uint16_t* out, float* attn_sum, int S, int past, float scale,
                                   void* ws, int64_t ws_bytes, void* stream) {
  CIA_REQUIRE(S >= 0 && past >= 0 && ws_bytes >= 0, CIA_ERR_ARG);
  if (S == 0) return CIA_OK;
  int st = check_cache(q, kc8, vc8, ksc, vsc, ktail, vtail, committed);
  if (st) return st;
  CIA_REQUIRE(out, CIA_ERR_NULL);
  CIA_REQUIRE(aligned(out, 2), CIA_ERR_ALIGN);
  CIA_REQUIRE(past + S - 1 - committed < G, CIA_ERR_STATE);
  CIA_REQUIRE(scale >= 0.0f && scale < __builtin_inff(), CIA_ERR_ARG);
  if (attn_sum) {
    CIA_REQUIRE(ws, CIA_ERR_NULL);
    CIA_REQUIRE(aligned(attn_sum, 4) && aligned(ws, 16), CIA_ERR_ALIGN);
    CIA_REQUIRE(ws_bytes >= cia_mass_workspace_bytes(S), CIA_ERR_ARG);
  }
  st = cia_prefill_mfma(q, kc8, vc8, ksc, vsc, ktail, vtail, committed, out, S, past, scale,
                        stream);
  if (st || !attn_sum) return st;
  return cia_mass_group64(q, kc8, ksc, ktail, committed, attn_sum, S, past, scale, ws, stream);
}
