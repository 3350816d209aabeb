// kv_cache.hip -- the FP8 E4M3 KV writers of the cuda_inf attention path on
// gfx950: tail append and group-64 commit (engine.cu:184-228), and the H2O
// per-token slot quantiser (engine.cu:317-333), with the H2O slot choice
// (engine.cu:808-823) run on the device in front of it.  The writers are
// bit-exact: amax is an order-free max, the scale is amax/448 + 1e-12 with
// an IEEE division, the bytes are encoded from x / scale (fp32) and the
// stored scale is fp16(scale).
#include "h2o_place.h"
#include <algorithm>

#include "common.h"

namespace cia {

// ---------------------------------------------------------------- tail
// One thread per 16-byte chunk (8 fp16) of K and of V.
__global__ __launch_bounds__(256) void k_write_tail(const u32x4* __restrict__ k,
                                                    const u32x4* __restrict__ v,
                                                    u32x4* __restrict__ ktail,
                                                    u32x4* __restrict__ vtail,
                                                    int slot, int nchunks) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nchunks) return;
  size_t dst = (size_t)slot * (NKV * D / 8) + i;
  ktail[dst] = k[i];
  vtail[dst] = v[i];
}

// ---------------------------------------------------------------- commit
// One group for kv head h, 256 threads: thread t owns token t/4, dims
// 16*(t%4) .. +15, for K and for V.  Token row r of the group comes from the
// tail when r < slot, else from source token src0 + r - slot (the tail rows
// the reference would have copied it into hold the same fp16 values).
__device__ __forceinline__ void commit_group_rows(const uint16_t* __restrict__ ktail,
                                                  const uint16_t* __restrict__ vtail,
                                                  const uint16_t* __restrict__ ksrc,
                                                  const uint16_t* __restrict__ vsrc, int slot,
                                                  int src0, uint8_t* __restrict__ kc8,
                                                  uint8_t* __restrict__ vc8,
                                                  uint16_t* __restrict__ ksc,
                                                  uint16_t* __restrict__ vsc, int dst_tok_base,
                                                  int grp, int h, int t) {
  const int tok = t >> 2, c = (t & 3) * 16;
  const bool from_tail = tok < slot;
  const size_t row = from_tail ? (size_t)tok : (size_t)(src0 + tok - slot);
  const size_t src = (row * NKV + h) * D + c;
  const uint16_t* kp = (from_tail ? ktail : ksrc) + src;
  const uint16_t* vp = (from_tail ? vtail : vsrc) + src;
  u32x4 kr[2], vr[2];
  kr[0] = *(const u32x4*)kp;
  kr[1] = *(const u32x4*)(kp + 8);
  vr[0] = *(const u32x4*)vp;
  vr[1] = *(const u32x4*)(vp + 8);
  float kf[16], vf[16];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    uint32_t kw = kr[i >> 3][(i & 7) >> 1], vw = vr[i >> 3][(i & 7) >> 1];
    kf[i] = h2f((uint16_t)(kw >> (16 * (i & 1))));
    vf[i] = h2f((uint16_t)(vw >> (16 * (i & 1))));
  }
  float mk = 0.f, mv = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    mk = __builtin_fmaxf(mk, __builtin_fabsf(kf[i]));
    mv = __builtin_fmaxf(mv, __builtin_fabsf(vf[i]));
  }
  mk = wave_max_fast(mk);
  mv = wave_max_fast(mv);
  __shared__ float red[2][4];
  const int w = t >> 6;
  if ((t & 63) == 0) { red[0][w] = mk; red[1][w] = mv; }
  __syncthreads();
  mk = __builtin_fmaxf(__builtin_fmaxf(red[0][0], red[0][1]), __builtin_fmaxf(red[0][2], red[0][3]));
  mv = __builtin_fmaxf(__builtin_fmaxf(red[1][0], red[1][1]), __builtin_fmaxf(red[1][2], red[1][3]));
  const float sck = quant_scale(mk), scv = quant_scale(mv);
  if (t == 0) {
    ksc[grp * NKV + h] = f2h(sck);
    vsc[grp * NKV + h] = f2h(scv);
  }
  // x / scale by quant_div, the reciprocals taken once
  const float rk = 1.0f / sck, sk = quant_div_s(sck), rv = 1.0f / scv, sv = quant_div_s(scv);
  u32x4 kb, vb;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    kb[j] = e4m3x4(quant_div(kf[4 * j], sk, rk), quant_div(kf[4 * j + 1], sk, rk),
                   quant_div(kf[4 * j + 2], sk, rk), quant_div(kf[4 * j + 3], sk, rk));
    vb[j] = e4m3x4(quant_div(vf[4 * j], sv, rv), quant_div(vf[4 * j + 1], sv, rv),
                   quant_div(vf[4 * j + 2], sv, rv), quant_div(vf[4 * j + 3], sv, rv));
  }
  const size_t dst = ((size_t)(dst_tok_base + tok) * NKV + h) * D + c;
  *(u32x4*)(kc8 + dst) = kb;
  *(u32x4*)(vc8 + dst) = vb;
}

// grid = 8 kv heads, block = 256: the group held in the tail
__global__ __launch_bounds__(256) void k_commit_group(const uint16_t* __restrict__ ktail,
                                                      const uint16_t* __restrict__ vtail,
                                                      uint8_t* __restrict__ kc8,
                                                      uint8_t* __restrict__ vc8,
                                                      uint16_t* __restrict__ ksc,
                                                      uint16_t* __restrict__ vsc,
                                                      int dst_tok_base, int grp) {
  commit_group_rows(ktail, vtail, nullptr, nullptr, G, 0, kc8, vc8, ksc, vsc, dst_tok_base, grp,
                    blockIdx.x, threadIdx.x);
}

// ---------------------------------------------------------------- batched append
// The placement loop of engine.cu:830-845 for S tokens arriving at tail
// slot slot0, in two launches instead of two per group.  With cnt0 =
// min(S, 64 - slot0): if slot0 + cnt0 = 64, group 0 is tail rows 0..slot0-1
// plus source tokens 0..cnt0-1, and groups 1..nfull are source tokens
// cnt0 + 64 (g-1) + r; the remaining cnt_last tokens stay in the tail.
struct AppendShape {
  int slot0, S, cnt0, commit0, nfull, s_last, cnt_last;
};

__host__ __device__ inline AppendShape append_shape(int slot0, int S) {
  AppendShape a;
  a.slot0 = slot0;
  a.S = S;
  a.cnt0 = S < G - slot0 ? S : G - slot0;
  a.commit0 = slot0 + a.cnt0 == G;
  a.nfull = a.commit0 ? (S - a.cnt0) / G : 0;
  a.s_last = a.commit0 ? a.cnt0 + G * a.nfull : S;
  a.cnt_last = S - a.s_last;
  return a;
}

// The source token of tail row r after the append (the reference leaves
// row r holding the token the last op that wrote row r put there), or -1
// when the append does not write row r.
__device__ __forceinline__ int append_tail_src(int r, const AppendShape& sh) {
  if (!sh.commit0) return r >= sh.slot0 && r < sh.slot0 + sh.S ? r - sh.slot0 : -1;
  if (r < sh.cnt_last) return sh.s_last + r;
  if (sh.nfull > 0) return sh.cnt0 + G * (sh.nfull - 1) + r;
  return r >= sh.slot0 ? r - sh.slot0 : -1;
}

// grid = (1 + nfull, 8 kv heads), block = 256.  Workgroup (0, h) also
// writes kv head h's tail rows, after its own reads of the old ones (the
// only reads of the tail in the launch), so no second launch is needed.
__global__ __launch_bounds__(256) void k_append_commit(uint16_t* __restrict__ ktail,
                                                       uint16_t* __restrict__ vtail,
                                                       const uint16_t* __restrict__ k,
                                                       const uint16_t* __restrict__ v,
                                                       uint8_t* __restrict__ kc8,
                                                       uint8_t* __restrict__ vc8,
                                                       uint16_t* __restrict__ ksc,
                                                       uint16_t* __restrict__ vsc, AppendShape sh,
                                                       int committed) {
  const int g = blockIdx.x;
  const int slot = g == 0 ? sh.slot0 : 0;
  const int src0 = g == 0 ? 0 : sh.cnt0 + G * (g - 1);
  commit_group_rows(ktail, vtail, k, v, slot, src0, kc8, vc8, ksc, vsc, committed + G * g,
                    committed / G + g, blockIdx.y, threadIdx.x);
  // (every thread's tail reads finished before the barrier inside)
  if (g == 0) {
    const int r = threadIdx.x >> 2, c = (threadIdx.x & 3) * 16, h = blockIdx.y;
    const int src = append_tail_src(r, sh);
    if (src >= 0) {
      const size_t o = ((size_t)r * NKV + h) * D + c, i = ((size_t)src * NKV + h) * D + c;
      const u32x4 k0 = *(const u32x4*)(k + i), k1 = *(const u32x4*)(k + i + 8);
      const u32x4 v0 = *(const u32x4*)(v + i), v1 = *(const u32x4*)(v + i + 8);
      *(u32x4*)(ktail + o) = k0;
      *(u32x4*)(ktail + o + 8) = k1;
      *(u32x4*)(vtail + o) = v0;
      *(u32x4*)(vtail + o + 8) = v1;
    }
  }
}

// The tail as the reference leaves it: row r holds the token the last op
// that wrote row r put there.  grid = 64 rows, block = 64: lane -> (kv head
// lane / 8, 16-byte chunk lane % 8) of K and of V.
__global__ __launch_bounds__(64) void k_append_tail(uint16_t* __restrict__ ktail,
                                                    uint16_t* __restrict__ vtail,
                                                    const uint16_t* __restrict__ k,
                                                    const uint16_t* __restrict__ v,
                                                    AppendShape sh) {
  const int r = blockIdx.x;
  const int src = append_tail_src(r, sh);
  if (src < 0) return;
  const size_t o = (size_t)threadIdx.x * 8;  // element offset inside the row (8 heads x 64)
  *(u32x4*)(ktail + (size_t)r * NKV * D + o) = *(const u32x4*)(k + (size_t)src * NKV * D + o);
  *(u32x4*)(vtail + (size_t)r * NKV * D + o) = *(const u32x4*)(v + (size_t)src * NKV * D + o);
}

// ---------------------------------------------------------------- H2O quant
// Token j, kv head h of k/v into slot `slot` of the H2O buffer; one wave,
// lane d owns dimension d.  A slot < 0 (no slot could be chosen) writes
// nothing.  Called with wave-uniform arguments.
__device__ __forceinline__ void quant_write_row(const uint16_t* __restrict__ k,
                                                const uint16_t* __restrict__ v,
                                                uint8_t* __restrict__ kf, uint8_t* __restrict__ vf,
                                                uint16_t* __restrict__ ks,
                                                uint16_t* __restrict__ vs, int j, int h, int slot,
                                                int d) {
  if (slot < 0) return;
  const size_t src = ((size_t)j * NKV + h) * D + d;
  const float kv = h2f(k[src]), vv = h2f(v[src]);
  const float mk = wave_max_fast(__builtin_fabsf(kv)), mv = wave_max_fast(__builtin_fabsf(vv));
  const float sck = quant_scale(mk), scv = quant_scale(mv);
  // pack 4 neighbouring lanes' bytes into one dword store
  uint32_t kb = e4m3x2(quant_div(kv, quant_div_s(sck), 1.0f / sck), 0.f) & 0xFFu;
  uint32_t vb = e4m3x2(quant_div(vv, quant_div_s(scv), 1.0f / scv), 0.f) & 0xFFu;
  uint32_t kw = kb << (8 * (d & 3)), vw = vb << (8 * (d & 3));
  kw |= __shfl_xor(kw, 1);
  vw |= __shfl_xor(vw, 1);
  kw |= __shfl_xor(kw, 2);
  vw |= __shfl_xor(vw, 2);
  const size_t dst = ((size_t)slot * NKV + h) * D;
  if ((d & 3) == 0) {
    *(uint32_t*)(kf + dst + d) = kw;
    *(uint32_t*)(vf + dst + d) = vw;
  }
  if (d == 0) {
    ks[slot * NKV + h] = f2h(sck);
    vs[slot * NKV + h] = f2h(scv);
  }
}

// grid = S * 8 (token, kv head), block = 64: lane d.  With slot_pos, token j
// writes only if slot_pos[slot] == past + j, i.e. no later token of the
// batch took the same slot (the last write of the per-token order wins).
__global__ __launch_bounds__(64) void k_quant_write(const uint16_t* __restrict__ k,
                                                    const uint16_t* __restrict__ v,
                                                    uint8_t* __restrict__ kf,
                                                    uint8_t* __restrict__ vf,
                                                    uint16_t* __restrict__ ks,
                                                    uint16_t* __restrict__ vs,
                                                    const int32_t* __restrict__ dst_slots,
                                                    const int32_t* __restrict__ slot_pos,
                                                    int past) {
  const int jh = blockIdx.x, j = jh / NKV, h = jh % NKV;
  const int slot = dst_slots[j];
  if (slot_pos && slot >= 0 && slot_pos[slot] != past + j) return;
  quant_write_row(k, v, kf, vf, ks, vs, j, h, slot, threadIdx.x);
}

// ---------------------------------------------------------------- H2O placement
// The slot choice of engine.cu:808-823 on the device.  One block of
// kPlaceThreads threads; thread i owns slots t with t % kPlaceThreads == i
// and is the only thread that reads or writes attn[t] and slotpos[t], so
// every value it reads is its own last write (no cross-thread visibility
// is needed).  Token j < nfill takes slot n_live + j.  Each later token
// takes the minimum (attn, slot) over slots with attn < 1e30 and
// slotpos <= pos - W, else over all slots with attn < 1e30: the first
// strict minimum of the reference's ascending scan, since -0 and +0 compare
// equal there and are given one key here, and NaN never passes < 1e30.
// A chosen slot is marked 1e30 until the end of the batch, then cleared
// to 0 (the reference marks its host copy and clears the device value).
// A slot filled earlier in the same batch can be chosen again; its filling
// token is then not written (its bytes would be overwritten in the
// reference's per-token order).  Up to kPlaceFuse tokens are also
// quantised into their slots here.
constexpr int kPlaceThreads = 1024;
constexpr int kPlaceFuse = 16;

__global__ __launch_bounds__(kPlaceThreads) void k_h2o_place(
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, uint8_t* __restrict__ kf,
    uint8_t* __restrict__ vf, uint16_t* __restrict__ ks, uint16_t* __restrict__ vs,
    float* __restrict__ attn, int32_t* __restrict__ slotpos, int32_t* __restrict__ dst,
    int n_live, int C, int W, int S, int past, int fuse) {
  constexpr int kWaves = kPlaceThreads / 64;
  __shared__ uint64_t red[2][2][kWaves];
  __shared__ int slot_of[kPlaceFuse];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int nfill = min(S, C - n_live);
  for (int t = tid; t < C; t += kPlaceThreads)
    if (t >= n_live && t < n_live + nfill) {
      const int j = t - n_live;
      slotpos[t] = past + j;
      dst[j] = t;
      if (fuse) slot_of[j] = t;
    }
  for (int j = nfill; j < S; j++) {
    const int posj = past + j, lim = posj - W;
    uint64_t kwin = ~0ull, kall = ~0ull;
    for (int t = tid; t < C; t += kPlaceThreads) {
      const float a = attn[t];
      if (a < kPicked) {
        const uint64_t key = place_key(a, t);
        kall = min_u64(kall, key);
        if (slotpos[t] <= lim) kwin = min_u64(kwin, key);
      }
    }
    kwin = wave_min_u64(kwin);
    kall = wave_min_u64(kall);
    const int p = j & 1;  // alternate buffers: one barrier per token
    if (lane == 0) {
      red[p][0][wave] = kwin;
      red[p][1][wave] = kall;
    }
    __syncthreads();
    kwin = red[p][0][0];
    kall = red[p][1][0];
#pragma unroll
    for (int w = 1; w < kWaves; w++) {
      kwin = min_u64(kwin, red[p][0][w]);
      kall = min_u64(kall, red[p][1][w]);
    }
    const uint64_t kb = kwin != ~0ull ? kwin : kall;
    const int best = kb != ~0ull ? (int)(uint32_t)kb : -1;
    if (best >= 0 && best % kPlaceThreads == tid) {
      attn[best] = kPicked;
      slotpos[best] = posj;
    }
    if (tid == 0) {
      dst[j] = best;
      if (fuse) {
        slot_of[j] = best;
        if (best >= n_live && best < n_live + nfill) slot_of[best - n_live] = -1;
      }
    }
  }
  if (nfill < S)
    for (int t = tid; t < C; t += kPlaceThreads)
      if (attn[t] == kPicked) attn[t] = 0.0f;  // a reused slot starts fresh
  if (!fuse) return;
  __syncthreads();
  for (int jh = wave; jh < S * NKV; jh += kWaves)
    quant_write_row(k, v, kf, vf, ks, vs, jh / NKV, jh % NKV, slot_of[jh / NKV], lane);
}

// ---------------------------------------------------------------- codec check
// 16 consecutive fp32 bit patterns per thread -> 16 bytes
__global__ __launch_bounds__(256) void k_e4m3_range(uint32_t first, int64_t n,
                                                    uint8_t* __restrict__ out) {
  const int64_t i0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
  if (i0 >= n) return;
  if (i0 + 16 <= n) {
    u32x4 r;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float x[4];
#pragma unroll
      for (int e = 0; e < 4; e++)
        x[e] = __builtin_bit_cast(float, first + (uint32_t)(i0 + 4 * j + e));
      r[j] = e4m3x4(x[0], x[1], x[2], x[3]);
    }
    *(u32x4*)(out + i0) = r;
  } else {
    for (int64_t i = i0; i < n; i++)
      out[i] = (uint8_t)e4m3x2(__builtin_bit_cast(float, first + (uint32_t)i), 0.f);
  }
}

}  // namespace cia

using namespace cia;

extern "C" int cia_e4m3_encode_range(uint32_t first_bits, int64_t n, uint8_t* out,
                                     void* stream) {
  CIA_REQUIRE(n >= 0 && n <= ((int64_t)1 << 32), CIA_ERR_ARG);
  if (n == 0) return CIA_OK;
  CIA_REQUIRE(out, CIA_ERR_NULL);
  CIA_REQUIRE(aligned(out, 16), CIA_ERR_ALIGN);
  const int64_t threads = (n + 15) / 16;
  hipLaunchKernelGGL(k_e4m3_range, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, first_bits, n, out);
  return launch_status();
}

extern "C" int cia_kv_write_tail(const uint16_t* k, const uint16_t* v, uint16_t* ktail,
                                 uint16_t* vtail, int slot, int cnt, void* stream) {
  CIA_REQUIRE(slot >= 0 && cnt >= 0 && slot + cnt <= G, CIA_ERR_ARG);
  if (cnt == 0) return CIA_OK;
  CIA_REQUIRE(k && v && ktail && vtail, CIA_ERR_NULL);
  CIA_REQUIRE(aligned(k, 16) && aligned(v, 16) && aligned(ktail, 16) && aligned(vtail, 16),
              CIA_ERR_ALIGN);
  const int nchunks = cnt * NKV * D / 8;
  hipLaunchKernelGGL(k_write_tail, dim3((nchunks + 255) / 256), dim3(256), 0,
                     (hipStream_t)stream, (const u32x4*)k, (const u32x4*)v, (u32x4*)ktail,
                     (u32x4*)vtail, slot, nchunks);
  return launch_status();
}

extern "C" int cia_kv_commit_group(const uint16_t* ktail, const uint16_t* vtail, uint8_t* kc8,
                                   uint8_t* vc8, uint16_t* ksc, uint16_t* vsc, int dst_tok_base,
                                   int grp, void* stream) {
  CIA_REQUIRE(ktail && vtail && kc8 && vc8 && ksc && vsc, CIA_ERR_NULL);
  CIA_REQUIRE(dst_tok_base >= 0 && grp >= 0, CIA_ERR_ARG);
  CIA_REQUIRE(aligned(ktail, 16) && aligned(vtail, 16) && aligned(kc8, 16) && aligned(vc8, 16) &&
                  aligned(ksc, 2) && aligned(vsc, 2),
              CIA_ERR_ALIGN);
  hipLaunchKernelGGL(k_commit_group, dim3(NKV), dim3(256), 0, (hipStream_t)stream, ktail, vtail,
                     kc8, vc8, ksc, vsc, dst_tok_base, grp);
  return launch_status();
}

// S tokens at positions past.. into the group-64 cache whose tail holds
// tokens committed..past-1 (past - committed in [0, 64)); returns the new
// committed count in *committed.  Internal entry of the layer driver.
extern "C" __attribute__((visibility("hidden"))) int cia_kv_append_batched(
    const uint16_t* k, const uint16_t* v, uint16_t* ktail, uint16_t* vtail, uint8_t* kc8,
    uint8_t* vc8, uint16_t* ksc, uint16_t* vsc, int* committed, int S, int past, int maxT,
    void* stream) {
  CIA_REQUIRE(committed && k && v && ktail && vtail && kc8 && vc8 && ksc && vsc, CIA_ERR_NULL);
  CIA_REQUIRE(aligned(k, 16) && aligned(v, 16) && aligned(ktail, 16) && aligned(vtail, 16) &&
                  aligned(kc8, 16) && aligned(vc8, 16) && aligned(ksc, 2) && aligned(vsc, 2),
              CIA_ERR_ALIGN);
  const int c = *committed;
  CIA_REQUIRE(S >= 0 && c >= 0 && c % G == 0, CIA_ERR_ARG);
  CIA_REQUIRE(past >= c && past - c < G, CIA_ERR_STATE);
  if (S == 0) return CIA_OK;
  CIA_REQUIRE(past + S <= maxT, CIA_ERR_ARG);
  const AppendShape sh = append_shape(past - c, S);
  const int ncommit = sh.commit0 ? 1 + sh.nfull : 0;
  hipStream_t s = (hipStream_t)stream;
  // (with a commit, its first workgroup per kv head also writes the tail)
  if (ncommit)
    hipLaunchKernelGGL(k_append_commit, dim3(ncommit, NKV), dim3(256), 0, s, ktail, vtail, k, v,
                       kc8, vc8, ksc, vsc, sh, c);
  else
    hipLaunchKernelGGL(k_append_tail, dim3(G), dim3(64), 0, s, ktail, vtail, k, v, sh);
  const int st = launch_status();
  if (st) return st;
  *committed = c + G * ncommit;
  return CIA_OK;
}

extern "C" int cia_kv_quant_write(const uint16_t* k, const uint16_t* v, uint8_t* kf, uint8_t* vf,
                                  uint16_t* ks, uint16_t* vs, const int32_t* dst_slots, int S,
                                  void* stream) {
  CIA_REQUIRE(S >= 0, CIA_ERR_ARG);
  if (S == 0) return CIA_OK;
  CIA_REQUIRE(k && v && kf && vf && ks && vs && dst_slots, CIA_ERR_NULL);
  CIA_REQUIRE(aligned(kf, 4) && aligned(vf, 4) && aligned(k, 2) && aligned(v, 2), CIA_ERR_ALIGN);
  hipLaunchKernelGGL(k_quant_write, dim3(S * NKV), dim3(64), 0, (hipStream_t)stream, k, v, kf, vf,
                     ks, vs, dst_slots, (const int32_t*)nullptr, 0);
  return launch_status();
}

extern "C" int cia_h2o_place(const uint16_t* k, const uint16_t* v, uint8_t* kf, uint8_t* vf,
                             uint16_t* ks, uint16_t* vs, float* attn_sum, int32_t* slot_pos,
                             int32_t* dst_slots, int* n_live, int C, int W, int S, int past,
                             void* stream) {
  CIA_REQUIRE(n_live, CIA_ERR_NULL);
  CIA_REQUIRE(S >= 0 && past >= 0 && C >= 1 && W >= 0 && *n_live >= 0 && *n_live <= C,
              CIA_ERR_ARG);
  if (S == 0) return CIA_OK;
  CIA_REQUIRE(k && v && kf && vf && ks && vs && attn_sum && slot_pos && dst_slots, CIA_ERR_NULL);
  CIA_REQUIRE(aligned(kf, 4) && aligned(vf, 4) && aligned(k, 2) && aligned(v, 2) &&
                  aligned(attn_sum, 4) && aligned(slot_pos, 4) && aligned(dst_slots, 4),
              CIA_ERR_ALIGN);
  const int nfill = std::min(S, C - *n_live);
  // more evictions than slots: the reference's scan runs out of slots < 1e30
  if (S - nfill > C) return CIA_ERR_NOSLOT;
  const int fuse = S <= kPlaceFuse;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(k_h2o_place, dim3(1), dim3(kPlaceThreads), 0, s, k, v, kf, vf, ks, vs,
                     attn_sum, slot_pos, dst_slots, *n_live, C, W, S, past, fuse);
  int st = launch_status();
  if (st) return st;
  if (!fuse) {
    hipLaunchKernelGGL(k_quant_write, dim3(S * NKV), dim3(64), 0, s, k, v, kf, vf, ks, vs,
                       dst_slots, (const int32_t*)slot_pos, past);
    if ((st = launch_status())) return st;
  }
  *n_live += nfill;
  return CIA_OK;
}
