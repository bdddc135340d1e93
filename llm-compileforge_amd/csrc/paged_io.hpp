// Paged-cache row I/O: write new token rows into one paged tensor (K or V,
// any layout and dtype, e4m3fn quantized with per-head scales) and gather
// tables of blocks into dense [R, S, H, D] tensors.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cf {

struct PagedWriteParams {
  const void* x;       // [T, H, D] new rows
  int64_t x_s[3];      // element strides
  const void* slots;   // [T] i32 | i64: block * bs + offset
  int64_t slot_s;
  void* cache;         // [NB, bs, H, D]
  int64_t c_s[4];      // element strides
  const float* scale;  // [H] or [1] (e4m3fn caches), else null
  int64_t sc_s;        // 0 for a single scale
  int64_t T, NB;
  int H, D, bs;
};

struct PagedGatherParams {
  const void* cache;   // [NB, bs, H, D]
  int64_t c_s[4];
  const int32_t* tables;  // [R, Mb] physical block ids; ids outside [0, NB) give zero rows
  int64_t t_sr, t_sm;
  const float* scale;  // e4m3fn caches: [H] or [1] dequant scales
  int64_t sc_s;
  void* out;           // [R, S, H, D]
  int64_t o_s[4];
  int64_t NB;
  int R, Mb, S, H, D, bs;
};

int32_t launch_paged_write(const PagedWriteParams& p, int x_dt, int slot_dt, int cache_dt, hipStream_t stream);
int32_t launch_paged_gather(const PagedGatherParams& p, int cache_dt, int out_dt, hipStream_t stream);
// bytes (a multiple of 16) from a device-visible view of pinned host memory.
int32_t launch_stage_from_host(const void* src_dev_view, void* dst, uint64_t bytes, hipStream_t stream);

}  // namespace cf
