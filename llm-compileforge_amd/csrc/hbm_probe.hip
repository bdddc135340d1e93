// HBM read probe (measurement helper, no reference counterpart): each wave
// reads whole chunks at the chunk indices it is given -- the access shape of
// the decode kernel (independent waves, whole multi-KiB runs at random
// offsets) with no arithmetic -- so its rate is the practical read ceiling
// for that shape.
#include "cf_host.hpp"

namespace cf {
namespace {

__global__ __launch_bounds__(256) void read_probe_kernel(const uint4* __restrict__ buf, const int32_t* __restrict__ idx,
                                                         int per_wave, int64_t chunk16, uint32_t* out) {
  const int lane = threadIdx.x & 63;
  const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  uint32_t acc = 0;
  for (int i = 0; i < per_wave; ++i) {
    const uint4* p = buf + (int64_t)idx[w * per_wave + i] * chunk16;
#pragma unroll 4
    for (int64_t s = lane; s < chunk16; s += 64) {
      const uint4 v = p[s];
      acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
  }
  if (acc == 0x9E3779B9u) out[w * 64 + lane] = acc;  // keeps the loads; practically never written
}

}  // namespace
}  // namespace cf

using namespace cf;

extern "C" int32_t cf_hbm_read_probe(const void* buf, int64_t buf_bytes, const int32_t* chunk_ids, int64_t waves,
                                     int64_t chunks_per_wave, int64_t chunk_bytes, uint32_t* sink, void* stream) {
  CF_CHECK(buf && chunk_ids && sink, "NULL argument");
  CF_CHECK(chunk_bytes >= 16 && chunk_bytes % 16 == 0, "chunk_bytes must be a positive multiple of 16");
  CF_CHECK(((uintptr_t)buf & 15) == 0, "buffer must be 16-byte aligned");
  CF_CHECK(waves > 0 && waves % 4 == 0 && waves / 4 < (int64_t)INT32_MAX, "waves must be a positive multiple of 4");
  CF_CHECK(chunks_per_wave > 0 && chunks_per_wave < (int64_t)INT32_MAX, "chunks_per_wave must be positive");
  CF_CHECK(buf_bytes / chunk_bytes <= (int64_t)INT32_MAX, "too many chunks for int32 ids");
  // ids are trusted to lie in [0, buf_bytes / chunk_bytes): the caller builds them
  hipLaunchKernelGGL(read_probe_kernel, dim3((unsigned)(waves / 4)), dim3(256), 0, (hipStream_t)stream,
                     (const uint4*)buf, chunk_ids, (int)chunks_per_wave, chunk_bytes / 16, sink);
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}
