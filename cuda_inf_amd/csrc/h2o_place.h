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

// the partner of lane l in DPP / permlane steps, for the key's two halves
template <int kN>
__device__ __forceinline__ uint64_t row_ror_u64(uint64_t x) {
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)x, 0x120 + kN, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(x >> 32), 0x120 + kN, 0xF, 0xF, false);
  return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// minimum key over the wave, in every lane (a minimum is exact in any
// order): DPP rotations within each 16-lane row, then the row swaps
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t x) {
  x = min_u64(x, row_ror_u64<8>(x));
  x = min_u64(x, row_ror_u64<4>(x));
  x = min_u64(x, row_ror_u64<2>(x));
  x = min_u64(x, row_ror_u64<1>(x));
  const uint32_t lo = (uint32_t)x, hi = (uint32_t)(x >> 32);
  auto r16l = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
  auto r16h = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
  x = min_u64(((uint64_t)(uint32_t)r16h[0] << 32) | (uint32_t)r16l[0],
              ((uint64_t)(uint32_t)r16h[1] << 32) | (uint32_t)r16l[1]);
  const uint32_t lo2 = (uint32_t)x, hi2 = (uint32_t)(x >> 32);
  auto r32l = __builtin_amdgcn_permlane32_swap(lo2, lo2, false, false);
  auto r32h = __builtin_amdgcn_permlane32_swap(hi2, hi2, false, false);
  return min_u64(((uint64_t)(uint32_t)r32h[0] << 32) | (uint32_t)r32l[0],
                 ((uint64_t)(uint32_t)r32h[1] << 32) | (uint32_t)r32l[1]);
}

}  // namespace cia
