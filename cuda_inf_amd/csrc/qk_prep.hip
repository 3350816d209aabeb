// qk_prep.hip -- the reference's three QK-producer launches
// (rmsnorm_head on q, rmsnorm_head on k, rope; engine.cu:799-801) as one
// gfx950 launch, with the fixed-order arithmetic of qk_prep.h.
#include <cmath>

#include "qk_prep.h"

namespace cia {

// one wave per (token, head): heads 0..31 are q, 32..39 are k.
// grid = ceil(S * 40 / 4), block = 256
__global__ __launch_bounds__(256) void k_qk_norm_rope(uint16_t* __restrict__ q,
                                                      uint16_t* __restrict__ k,
                                                      const uint16_t* __restrict__ qw,
                                                      const uint16_t* __restrict__ kw,
                                                      const int32_t* __restrict__ pos, int S,
                                                      float eps, RopeTable rt) {
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6), d = threadIdx.x & 63;
  const int i = item / (NH + NKV), hh = item % (NH + NKV);
  if (i >= S) return;  // whole waves
  uint16_t* row = hh < NH ? q + ((size_t)i * NH + hh) * D : k + ((size_t)i * NKV + hh - NH) * D;
  const float w = h2f(hh < NH ? qw[d] : kw[d]);
  row[d] = qk_norm_rope_lane(h2f(row[d]), w, d, pos[i], eps, rt);
}

// The layer driver's form: raw q [S][32][64] and k [S][8][64] read, the
// prepared rows written to oq [S][32][64] and ok [S][8][64], at positions
// pos0 + i.
__global__ __launch_bounds__(256) void k_qk_prep_into(const uint16_t* __restrict__ q,
                                                      const uint16_t* __restrict__ k,
                                                      const uint16_t* __restrict__ qw,
                                                      const uint16_t* __restrict__ kw,
                                                      uint16_t* __restrict__ oq,
                                                      uint16_t* __restrict__ ok, int pos0, int S,
                                                      float eps, RopeTable rt) {
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6), d = threadIdx.x & 63;
  const int i = item / (NH + NKV), hh = item % (NH + NKV);
  if (i >= S) return;
  const size_t r = hh < NH ? (size_t)i * NH + hh : (size_t)i * NKV + hh - NH;
  const float x = h2f(hh < NH ? q[r * D + d] : k[r * D + d]);
  const float w = h2f(hh < NH ? qw[d] : kw[d]);
  (hh < NH ? oq : ok)[r * D + d] = qk_norm_rope_lane(x, w, d, pos0 + i, eps, rt);
}

RopeTable rope_table(float theta);
RopeTable rope_table(float theta) {
  RopeTable t;
  for (int i = 0; i < D / 2; i++) t.invf[i] = (float)std::pow((double)theta, -(2.0 * i) / D);
  return t;
}

}  // namespace cia

using namespace cia;

// Internal entry of the layer driver (see k_qk_prep_into)
extern "C" __attribute__((visibility("hidden"))) int cia_qk_prep_into(
    const uint16_t* q, const uint16_t* k, const uint16_t* qw, const uint16_t* kw, uint16_t* oq,
    uint16_t* ok, int pos0, int S, float eps, float theta, void* stream) {
  const int64_t items = (int64_t)S * (NH + NKV);
  hipLaunchKernelGGL(k_qk_prep_into, dim3((unsigned)((items + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, q, k, qw, kw, oq, ok, pos0, S, eps, rope_table(theta));
  return launch_status();
}

// The decode kernels' prep descriptor for a layer (table cached per theta)
extern "C" __attribute__((visibility("hidden"))) const void* cia_qk_prep_desc(
    const uint16_t* qw, const uint16_t* kw, float eps, float theta) {
  static thread_local QkPrep p{};
  static thread_local float cached = 0.0f;
  if (cached != theta) {
    p.rt = rope_table(theta);
    cached = theta;
  }
  p.qw = qw;
  p.kw = kw;
  p.eps = eps;
  return &p;
}

extern "C" int cia_qk_norm_rope(uint16_t* q, uint16_t* k, const uint16_t* qw, const uint16_t* kw,
                                const int32_t* pos, int S, float eps, float theta, void* stream) {
  CIA_REQUIRE(S >= 0, CIA_ERR_ARG);
  if (S == 0) return CIA_OK;
  CIA_REQUIRE(q && k && qw && kw && pos, CIA_ERR_NULL);
  CIA_REQUIRE(eps >= 0.0f && theta > 0.0f && theta < __builtin_inff(), CIA_ERR_ARG);
  CIA_REQUIRE(aligned(q, 2) && aligned(k, 2) && aligned(qw, 2) && aligned(kw, 2) && aligned(pos, 4),
              CIA_ERR_ALIGN);
  const int64_t items = (int64_t)S * (NH + NKV);
  hipLaunchKernelGGL(k_qk_norm_rope, dim3((unsigned)((items + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, q, k, qw, kw, pos, S, eps, rope_table(theta));
  return launch_status();
}
