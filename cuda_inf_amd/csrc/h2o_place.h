// h2o_place.h -- the H2O slot rule's ordering helpers (engine.cu:808-823),
// shared by the placement kernel and the single-token attention launch that
// places its token itself.
#pragma once
#include "common.h"

namespace cia {

// a slot chosen earlier in the same batch carries this mass until the end
// of the batch (the reference marks its host copy)
constexpr float kPicked = 1e30f;

// (mass, slot) as one unsigned key: float order for the mass (-0 and +0
// equal, as in the reference's < comparisons), lower slot first on ties
__device__ __forceinline__ uint64_t place_key(float a, int t) {
  uint32_t b = __float_as_uint(a == 0.0f ? 0.0f : a);
  b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);  // float order as unsigned order
  return ((uint64_t)b << 32) | (uint32_t)t;
}

__device__ __forceinline__ uint64_t min_u64(uint64_t a, uint64_t b) { return b < a ? b : a; }

__device__ __forceinline__ uint64_t wave_min_u64(uint64_t x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = min_u64(x, __shfl_xor(x, off));
  return x;
}

}  // namespace cia
