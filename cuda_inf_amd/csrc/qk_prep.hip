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

RopeTable rope_table(float theta) {
  RopeTable t;
  for (int i = 0; i < D / 2; i++) t.invf[i] = (float)std::pow((double)theta, -(2.0 * i) / D);
  return t;
}

}  // namespace cia

using namespace cia;

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
