// kv_cache.hip -- the FP8 E4M3 KV writers of the cuda_inf attention path on
// gfx950: tail append and group-64 commit (engine.cu:184-228), and the H2O
// per-token slot quantiser (engine.cu:317-333).  All three are bit-exact:
// amax is an order-free max, the scale is amax/448 + 1e-12 with an IEEE
// division, the bytes are encoded from x / scale (fp32) and the stored scale
// is fp16(scale).
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
// grid = 8 kv heads, block = 256: thread t owns token t/4, dims
// 16*(t%4) .. +15 of its head, for K and for V.
__global__ __launch_bounds__(256) void k_commit_group(const uint16_t* __restrict__ ktail,
                                                      const uint16_t* __restrict__ vtail,
                                                      uint8_t* __restrict__ kc8,
                                                      uint8_t* __restrict__ vc8,
                                                      uint16_t* __restrict__ ksc,
                                                      uint16_t* __restrict__ vsc,
                                                      int dst_tok_base, int grp) {
  const int h = blockIdx.x, t = threadIdx.x;
  const int tok = t >> 2, c = (t & 3) * 16;
  const size_t src = ((size_t)tok * NKV + h) * D + c;
  u32x4 kr[2], vr[2];
  kr[0] = *(const u32x4*)(ktail + src);
  kr[1] = *(const u32x4*)(ktail + src + 8);
  vr[0] = *(const u32x4*)(vtail + src);
  vr[1] = *(const u32x4*)(vtail + src + 8);
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
  u32x4 kb, vb;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    kb[j] = e4m3x4(kf[4 * j] / sck, kf[4 * j + 1] / sck, kf[4 * j + 2] / sck, kf[4 * j + 3] / sck);
    vb[j] = e4m3x4(vf[4 * j] / scv, vf[4 * j + 1] / scv, vf[4 * j + 2] / scv, vf[4 * j + 3] / scv);
  }
  const size_t dst = ((size_t)(dst_tok_base + tok) * NKV + h) * D + c;
  *(u32x4*)(kc8 + dst) = kb;
  *(u32x4*)(vc8 + dst) = vb;
}

// ---------------------------------------------------------------- H2O quant
// grid = S * 8 (token, kv head), block = 64: lane d.
__global__ __launch_bounds__(64) void k_quant_write(const uint16_t* __restrict__ k,
                                                    const uint16_t* __restrict__ v,
                                                    uint8_t* __restrict__ kf,
                                                    uint8_t* __restrict__ vf,
                                                    uint16_t* __restrict__ ks,
                                                    uint16_t* __restrict__ vs,
                                                    const int32_t* __restrict__ dst_slots) {
  const int jh = blockIdx.x, j = jh / NKV, h = jh % NKV, d = threadIdx.x;
  const size_t src = ((size_t)j * NKV + h) * D + d;
  const float kv = h2f(k[src]), vv = h2f(v[src]);
  const float mk = wave_max_fast(__builtin_fabsf(kv)), mv = wave_max_fast(__builtin_fabsf(vv));
  const float sck = quant_scale(mk), scv = quant_scale(mv);
  const int slot = dst_slots[j];
  // pack 4 neighbouring lanes' bytes into one dword store
  uint32_t kb = e4m3x2(kv / sck, 0.f) & 0xFFu, vb = e4m3x2(vv / scv, 0.f) & 0xFFu;
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

extern "C" int cia_kv_quant_write(const uint16_t* k, const uint16_t* v, uint8_t* kf, uint8_t* vf,
                                  uint16_t* ks, uint16_t* vs, const int32_t* dst_slots, int S,
                                  void* stream) {
  CIA_REQUIRE(S >= 0, CIA_ERR_ARG);
  if (S == 0) return CIA_OK;
  CIA_REQUIRE(k && v && kf && vf && ks && vs && dst_slots, CIA_ERR_NULL);
  CIA_REQUIRE(aligned(kf, 4) && aligned(vf, 4) && aligned(k, 2) && aligned(v, 2), CIA_ERR_ALIGN);
  hipLaunchKernelGGL(k_quant_write, dim3(S * NKV), dim3(64), 0, (hipStream_t)stream, k, v, kf, vf,
                     ks, vs, dst_slots);
  return launch_status();
}
