// Parameters of the chunked-prefill kernels (paged attention of query chunks
// against the paged KV cache, causal within the chunk).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cf {

struct PrefillParams {
  const void* q;
  int64_t q_sr, q_sh;  // q [Tq, Hq, D], D stride 1
  void* out;
  int64_t o_sr, o_sh;  // out [Tq, Hq, D], D stride 1
  const void* k;
  const void* v;
  int64_t k_s[4], v_s[4];  // caches [NB, bs, Hkv, D]
  const int32_t* tables;
  int64_t t_sb, t_sm;  // block_tables [N, Mb]
  const int32_t* seq_lens;
  int64_t sl_s;  // seq_lens [N]: cached tokens + chunk tokens
  const int32_t* q_start;
  int64_t qs_s;  // q_start [N + 1]: first q row of each chunk
  const float* k_scale;
  const float* v_scale;
  int64_t ks_s, vs_s;
  float scale;
  int N, Tq, Hq, Hkv, G, D, Mb, NB;
  int RB;         // query rows per work item (128 / G: 128 query columns)
  int max_items;  // bound on work items: (Tq / RB + N) * Hkv
  // workspace
  int4* chunks;  // [N] {first q row, rows, position of the first row, row blocks before it}
  int4* items;   // [max_items] {chunk, row block, KV head, tiles}, longest first
  int* header;   // {items, shared queue counter, items in the per-XCD lists, 8 list counters}
};

// Query rows per work item for GQA group G.
int prefill_rows_per_item(int G);
bool prefill_supported(const PrefillParams& p, int q_dt, int kv_dt);
uint64_t prefill_workspace_bytes(int64_t Tq, int64_t N, int64_t Hq, int64_t Hkv, int64_t D);
void prefill_bind_workspace(PrefillParams& p, void* workspace);
int32_t launch_prefill(PrefillParams& p, int q_dt, int kv_dt, hipStream_t stream);

}  // namespace cf
