// Parameters shared by the paged-decode kernels and their host launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cf {

// All strides are in elements of the tensor they index.
struct DecodeParams {
  const void* q;
  int64_t q_sb, q_sh;  // q [B, Hq, D], D stride 1
  const void* k;
  const void* v;
  int64_t k_s[4];  // k_cache [NB, bs, Hkv, D]
  int64_t v_s[4];  // v_cache [NB, bs, Hkv, D]
  const int32_t* tables;
  int64_t t_sb, t_sm;  // block_tables [B, Mb]
  const int32_t* seq_lens;
  int64_t sl_s;  // seq_lens [B]
  const int32_t* shared;  // optional [B]: leading tokens sequence b shares with b - 1
  int64_t sh_s;
  const float* k_scale;
  const float* v_scale;
  int64_t ks_s, vs_s;  // 0 when the scale is a single value
  void* out;
  int64_t o_sb, o_sh;  // out [B, Hq, D], D stride 1
  float* ws_o;         // generic path: [B, Hq, max_parts, D] un-normalized partial outputs;
                       // MFMA path: [rows, D] partial rows (see decode_mfma.hip)
  float* ws_ml;        // running max and sum per partial row
  int2* own_desc;      // MFMA path: per (sequence, KV head), the sequence's own run
  int2* pre_desc;      // MFMA path: per (sequence, KV head), its shared-prefix run
  int64_t rec_own;     // MFMA path: first row of the per-(sequence, head) own-run records
  int64_t rec_pre;     // ... and of the shared-prefix records
  float scale;
  int B, Hq, Hkv, G, D, bs, Mb, PT, max_parts;
  int NB;  // cache blocks; a block id outside [0, NB) contributes no tokens
};

// Launchers (return a CF_* status; kernels are enqueued on `stream`).
int32_t launch_decode_generic(const DecodeParams& p, int q_dt, int kv_dt, hipStream_t stream);
int32_t launch_decode_mfma(const DecodeParams& p, int q_dt, int kv_dt, hipStream_t stream);
bool decode_mfma_supported(const DecodeParams& p, int q_dt, int kv_dt);
// Workspace of the MFMA path: two (m, l, o) partial slots per launched wave.
uint64_t decode_mfma_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim);
void decode_mfma_bind_workspace(DecodeParams& p, void* workspace);

int32_t launch_decode_reduce(const DecodeParams& p, int q_dt, hipStream_t stream);
// LDS bytes of one generic-kernel workgroup (G query heads, partition PT).
size_t generic_lds_bytes(int64_t G, int64_t D, int64_t PT, int64_t bs);

}  // namespace cf
