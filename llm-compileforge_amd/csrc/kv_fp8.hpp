// Parameters and launchers of the FP8 KV quantization kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cf {

// A strided view [S0, S1, H, D] (head axis 2); strides in elements.  Rank-3
// tensors [T, H, D] are carried as [1, T, H, D].
struct Rank4 {
  const void* base;
  int64_t size[4];
  int64_t stride[4];
};

struct KvWriteParams {
  Rank4 k_new, v_new;  // [T, H, D]
  const void* slots;
  int64_t slot_stride;
  void* k_cache;
  void* v_cache;
  int64_t kc_s[4], vc_s[4];  // [NB, bs, H, D] byte strides (e4m3: 1 byte per element)
  const float* k_scale;
  const float* v_scale;
  int64_t ks_s, vs_s;
  int64_t T;
  int64_t NB;  // cache blocks; slots outside [0, NB * bs) are skipped
  int H, D, bs;
};

int32_t launch_amax_scale(const Rank4& x, int x_dt, float* scales, int64_t s_stride, hipStream_t stream);
int32_t launch_quantize(const Rank4& x, int x_dt, const float* scales, int64_t s_stride, const Rank4& out,
                        hipStream_t stream);
// K and V with their own per-head scales; one launch when the outputs are
// native-tile (e.g. paired) K and V views of [S0, 16, H, D] pools.
int32_t launch_quantize_kv(const Rank4& k, const Rank4& v, int x_dt, const float* ks, int64_t ks_s, const float* vs,
                           int64_t vs_s, const Rank4& ko, const Rank4& vo, hipStream_t stream);
int32_t launch_dequantize(const Rank4& q, const float* scales, int64_t s_stride, const Rank4& out,
                          hipStream_t stream);
int32_t launch_kv_write_fp8(const KvWriteParams& p, int x_dt, int slot_dt, hipStream_t stream);

}  // namespace cf
