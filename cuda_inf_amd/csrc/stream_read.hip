// stream_read.hip -- a plain streaming read of one layer's committed FP8 K
// and V bytes: the measured ceiling that the decode kernel's stream is
// compared against (a measurement utility; no counterpart in the reference).
// 256 workgroups of 512 threads; consecutive lanes read consecutive 16-byte
// chunks (so every 128-byte line is fetched by one wave of one XCD), 8 chunks
// of K and 8 of V in flight per thread per round.
#include "common.h"

namespace cia {

constexpr int kSrThreads = 512;
constexpr int kSrBlocks = 256;

__global__ __launch_bounds__(kSrThreads) void k_stream_read(const u32x4* k, const u32x4* v,
                                                            int64_t n16, uint32_t* sink) {
  const int64_t nthr = (int64_t)gridDim.x * kSrThreads;
  const int64_t t = (int64_t)blockIdx.x * kSrThreads + threadIdx.x;
  uint32_t acc = 0;
  for (int64_t base = 0; base < n16; base += 8 * nthr) {
    u32x4 x[16];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int64_t idx = base + i * nthr + t;
      const bool in = idx < n16;
      x[i] = in ? k[idx] : u32x4{0, 0, 0, 0};
      x[8 + i] = in ? v[idx] : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < 16; i++) acc ^= x[i][0] ^ x[i][1] ^ x[i][2] ^ x[i][3];
  }
  // (keeps the loads; a match is harmless: one word, any writer)
  if (acc == 0x9e3779b9u) sink[0] = acc;
}

}  // namespace cia

using namespace cia;

extern "C" int cia_stream_read(const void* k, const void* v, int64_t bytes, uint32_t* sink,
                               void* stream) {
  if (!k || !v || !sink) return CIA_ERR_NULL;
  if (bytes < 0 || bytes % 16) return CIA_ERR_ARG;
  if (bytes == 0) return CIA_OK;
  hipLaunchKernelGGL(k_stream_read, dim3(kSrBlocks), dim3(kSrThreads), 0, (hipStream_t)stream,
                     (const u32x4*)k, (const u32x4*)v, bytes / 16, sink);
  return launch_status();
}
