// extern "C" entry points of libcf_hip.so (declared in include/cf_hip.h):
// argument validation, dispatch to the kernel launchers, error state and
// the launch-timing hook.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "cf_host.hpp"
#include "decode_params.hpp"
#include "kv_fp8.hpp"
#include "paged_io.hpp"
#include "prefill_params.hpp"

namespace cf {

// ---- error state --------------------------------------------------------
namespace {
thread_local std::string g_error;
}

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
}

const std::string& last_error() { return g_error; }

int32_t view_of(const CfTensor* t, const char* name, int rank, View* v) {
  CF_CHECK(t != nullptr, "%s: descriptor is NULL", name);
  CF_CHECK(t->t.rank == rank, "%s: expected rank %d, got %d", name, rank, t->t.rank);
  const int eb = dtype_bytes(t->dtype);
  CF_CHECK(eb > 0, "%s: unknown dtype code %d", name, t->dtype);
  CF_CHECK(t->t.elem_size == eb, "%s: elem_size %d does not match dtype %s", name, t->t.elem_size,
           dtype_name(t->dtype));
  CF_CHECK(t->t.device == SFA_ROCM, "%s: expected device memory (SFA_ROCM), got device %d", name,
           (int)t->t.device);
  // The union members share their first three fields; sizes/strides follow.
  const SFATensorRaw4& r = t->t.r4;
  const int64_t* sizes = &r.offset + 1;
  const int64_t* strides = sizes + rank;
  CF_CHECK(r.offset >= 0, "%s: negative offset", name);
  v->rank = rank;
  v->dtype = t->dtype;
  v->elem = eb;
  bool empty = false;
  for (int i = 0; i < rank; ++i) {
    v->size[i] = sizes[i];
    v->stride[i] = strides[i];
    CF_CHECK(sizes[i] >= 0, "%s: negative size on dim %d", name, i);
    CF_CHECK(strides[i] >= 0, "%s: negative stride on dim %d", name, i);
    if (sizes[i] == 0) empty = true;
  }
  CF_CHECK(empty || r.aligned != nullptr, "%s: NULL data pointer", name);
  v->base = (char*)r.aligned + r.offset * eb;
  return CF_OK;
}

// ---- launch profiling ---------------------------------------------------
namespace {
struct ProfRecord {
  std::string name;
  hipEvent_t begin, end;
};
std::mutex g_prof_mu;
bool g_prof_on = false;
std::vector<ProfRecord> g_prof_records;
std::vector<hipEvent_t> g_prof_pool;

// Callers hold g_prof_mu.
hipEvent_t take_event() {
  if (!g_prof_pool.empty()) {
    hipEvent_t e = g_prof_pool.back();
    g_prof_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Events armed by a ProfileScope for this thread's next launch.
struct Pending {
  const char* name = nullptr;
  hipEvent_t begin = nullptr, end = nullptr;
};
thread_local Pending g_pending;

// Callers hold g_prof_mu.
void release_pending() {
  if (g_pending.begin) g_prof_pool.push_back(g_pending.begin);
  if (g_pending.end) g_prof_pool.push_back(g_pending.end);
  g_pending = Pending{};
}
}  // namespace

bool profiling_enabled() { return g_prof_on; }

void profile_arm(const char* name) {
  if (!g_prof_on) return;
  std::lock_guard<std::mutex> lock(g_prof_mu);
  release_pending();
  hipEvent_t b = take_event(), e = take_event();
  if (!b || !e) {
    if (b) g_prof_pool.push_back(b);
    if (e) g_prof_pool.push_back(e);
    return;
  }
  g_pending.name = name;
  g_pending.begin = b;
  g_pending.end = e;
}

void profile_disarm() {
  if (!g_pending.begin && !g_pending.end) return;
  std::lock_guard<std::mutex> lock(g_prof_mu);
  release_pending();
}

ArmedEvents profile_take() {
  ArmedEvents ev;
  if (!g_pending.begin) return ev;
  ev.name = g_pending.name;
  ev.begin = g_pending.begin;
  ev.end = g_pending.end;
  g_pending = Pending{};
  return ev;
}

void profile_commit(const ArmedEvents& ev, bool launched) {
  if (!ev.begin) return;
  std::lock_guard<std::mutex> lock(g_prof_mu);
  if (launched) {
    g_prof_records.push_back(ProfRecord{ev.name, ev.begin, ev.end});
  } else {
    g_prof_pool.push_back(ev.begin);
    if (ev.end) g_prof_pool.push_back(ev.end);
  }
}

namespace {
hipStream_t as_stream(void* s) { return (hipStream_t)s; }

// Optional per-head scale vector [H] or [1], f32.
int32_t scale_view(const CfTensor* t, const char* name, int64_t H, const float** ptr, int64_t* stride) {
  View v;
  int32_t rc = view_of(t, name, 1, &v);
  if (rc) return rc;
  CF_CHECK(v.dtype == CF_F32, "%s: expected f32, got %s", name, dtype_name(v.dtype));
  CF_CHECK(v.size[0] == H || v.size[0] == 1, "%s: expected %lld or 1 entries, got %lld", name, (long long)H,
           (long long)v.size[0]);
  *ptr = (const float*)v.base;
  *stride = v.size[0] == 1 ? 0 : v.stride[0];
  return CF_OK;
}

bool is_float_dtype(int dt) { return dt == CF_F32 || dt == CF_F16 || dt == CF_BF16; }

// [T, H, D] or [S0, S1, H, D] -> Rank4 (head axis 2).
Rank4 rank4_of(const View& v) {
  Rank4 r;
  r.base = v.base;
  const int lead = 4 - v.rank;
  for (int i = 0; i < lead; ++i) {
    r.size[i] = 1;
    r.stride[i] = 0;
  }
  for (int i = 0; i < v.rank; ++i) {
    r.size[lead + i] = v.size[i];
    r.stride[lead + i] = v.stride[i];
  }
  return r;
}

int32_t view_of_34(const CfTensor* t, const char* name, View* v) {
  CF_CHECK(t != nullptr, "%s: descriptor is NULL", name);
  CF_CHECK(t->t.rank == 3 || t->t.rank == 4, "%s: expected rank 3 or 4, got %d", name, t->t.rank);
  return view_of(t, name, t->t.rank, v);
}
}  // namespace

int device_cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

// ---- fixed scratch for the no-allocation decode entry point -------------
// Device memory the library owns for callers that cannot allocate: one
// array per device, held from the code object's load until the process
// ends.  Host code never uses the array's name as an address (in host code
// it is only a stand-in); the device address comes from hipGetSymbolAddress
// once per device, with that device current, and is kept per device.
constexpr uint64_t kNoAllocScratchBytes = 64ull << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

// The current device's scratch address (resolved on its first use there).
int32_t noalloc_scratch(void** out) {
  int dev = -1;
  CF_HIP_CHECK(hipGetDevice(&dev));
  CF_CHECK(dev >= 0 && dev < kMaxDevices, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      set_error("hipGetSymbolAddress(scratch) failed on device %d: %s", dev, hipGetErrorString(e));
      return CF_ERR_HIP;
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return CF_OK;
}

}  // namespace cf

using namespace cf;

extern "C" {

int32_t cf_abi_version(void) { return CF_ABI_VERSION; }

int32_t cf_last_error(char* buf, uint64_t len) {
  const std::string& e = last_error();
  if (buf && len > 0) {
    const size_t n = std::min<size_t>(e.size(), (size_t)len - 1);
    std::memcpy(buf, e.data(), n);
    buf[n] = '\0';
  }
  return (int32_t)e.size();
}

static int64_t decode_max_parts(int64_t max_blocks, int32_t bs, int32_t pt) {
  return std::max<int64_t>(1, ceil_div(max_blocks * (int64_t)bs, pt));
}

// Partition length of the generic (VALU) path: the caller's, halved while the
// launch would hold fewer than ~1k workgroups (small batches / few heads)
// and a partition keeps at least max(block_size, 32) tokens, so short
// batches still spread over the GPU; halved further (down to one block)
// while a workgroup's scores would not fit its 64 KiB of LDS (many query
// heads per KV head).  A function of the call's sizes only: the workspace
// query and the launch agree on it.
static int32_t generic_partition(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                 int64_t max_blocks, int32_t bs, int32_t pt) {
  const int64_t floor_tokens = std::max<int64_t>(bs, 32);
  int64_t t = pt;
  while (t / 2 >= floor_tokens && (t / 2) % bs == 0 &&
         batch * num_kv_heads * decode_max_parts(max_blocks, bs, (int32_t)t) < 1024)
    t /= 2;
  const int64_t G = num_kv_heads > 0 ? num_q_heads / num_kv_heads : 1;
  while (t / 2 >= bs && (t / 2) % bs == 0 && generic_lds_bytes(G, head_dim, t, bs) > 64 * 1024) t /= 2;
  return (int32_t)t;
}

// Generic-path layout: [o partials, 256-byte padded] [(m, l)].
static uint64_t generic_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t head_dim, int64_t parts) {
  if (parts <= 1) return 0;
  const uint64_t rows = (uint64_t)batch * num_q_heads * parts;
  const uint64_t o_bytes = rows * head_dim * 4;
  const uint64_t ml_bytes = rows * 2 * 4;
  return ((o_bytes + 255) & ~(uint64_t)255) + ml_bytes;
}

int32_t cf_paged_decode_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                                        int64_t head_dim, int64_t max_blocks_per_seq, int32_t block_size,
                                        int32_t partition_tokens, uint64_t* bytes_out) {
  CF_CHECK(bytes_out != nullptr, "bytes_out is NULL");
  CF_CHECK(batch >= 0 && num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0 && max_blocks_per_seq >= 0,
           "invalid sizes");
  CF_CHECK(num_q_heads % num_kv_heads == 0, "num_heads %lld is not a multiple of num_kv_heads %lld",
           (long long)num_q_heads, (long long)num_kv_heads);
  CF_CHECK(block_size > 0 && partition_tokens > 0 && partition_tokens % block_size == 0,
           "partition_tokens (%d) must be a positive multiple of block_size (%d)", partition_tokens,
           block_size);
  const int32_t gpt = generic_partition(batch, num_q_heads, num_kv_heads, head_dim, max_blocks_per_seq, block_size,
                                        partition_tokens);
  const int64_t parts = decode_max_parts(max_blocks_per_seq, block_size, gpt);
  const uint64_t generic = generic_workspace_bytes(batch, num_q_heads, head_dim, parts);
  const uint64_t mfma =
      block_size == 16 ? decode_mfma_workspace_bytes(batch, num_q_heads, num_kv_heads, head_dim) : 0;
  *bytes_out = generic > mfma ? generic : mfma;
  return CF_OK;
}

int32_t cf_paged_decode(const CfTensor* q, const CfTensor* k_cache, const CfTensor* v_cache,
                        const CfTensor* block_tables, const CfTensor* seq_lens, const CfTensor* k_scale,
                        const CfTensor* v_scale, float scale, int32_t block_size, int32_t partition_tokens,
                        CfTensor* out, void* workspace, uint64_t workspace_bytes, void* stream) {
  return cf_paged_decode_shared(q, k_cache, v_cache, block_tables, seq_lens, nullptr, k_scale, v_scale, scale,
                                block_size, partition_tokens, out, workspace, workspace_bytes, stream);
}

int32_t cf_paged_decode_shared(const CfTensor* q, const CfTensor* k_cache, const CfTensor* v_cache,
                               const CfTensor* block_tables, const CfTensor* seq_lens,
                               const CfTensor* shared_prefix_lens, const CfTensor* k_scale,
                               const CfTensor* v_scale, float scale, int32_t block_size,
                               int32_t partition_tokens, CfTensor* out, void* workspace,
                               uint64_t workspace_bytes, void* stream) {
  View vq, vk, vv, vt, vs, vo;
  int32_t rc;
  if ((rc = view_of(q, "q", 3, &vq))) return rc;
  if ((rc = view_of(k_cache, "k_cache", 4, &vk))) return rc;
  if ((rc = view_of(v_cache, "v_cache", 4, &vv))) return rc;
  if ((rc = view_of(block_tables, "block_tables", 2, &vt))) return rc;
  if ((rc = view_of(seq_lens, "seq_lens", 1, &vs))) return rc;
  if ((rc = view_of(out, "out", 3, &vo))) return rc;

  CF_CHECK(is_float_dtype(vq.dtype), "q: dtype must be f32, f16 or bf16, got %s", dtype_name(vq.dtype));
  CF_CHECK(is_float_dtype(vk.dtype) || vk.dtype == CF_F8E4M3FN,
           "k_cache: dtype must be f32, f16, bf16 or f8e4m3fn, got %s", dtype_name(vk.dtype));
  CF_CHECK(vv.dtype == vk.dtype, "v_cache dtype %s differs from k_cache dtype %s", dtype_name(vv.dtype),
           dtype_name(vk.dtype));
  CF_CHECK(vt.dtype == CF_I32, "block_tables: expected i32, got %s", dtype_name(vt.dtype));
  CF_CHECK(vs.dtype == CF_I32, "seq_lens: expected i32, got %s", dtype_name(vs.dtype));
  CF_CHECK(vo.dtype == vq.dtype, "out dtype %s differs from q dtype %s", dtype_name(vo.dtype),
           dtype_name(vq.dtype));

  const int64_t B = vq.size[0], Hq = vq.size[1], D = vq.size[2];
  const int64_t NB = vk.size[0], bs = vk.size[1], Hkv = vk.size[2];
  for (int i = 0; i < 4; ++i)
    CF_CHECK(vv.size[i] == vk.size[i], "v_cache shape differs from k_cache shape on dim %d", i);
  CF_CHECK(vk.size[3] == D, "k_cache head_dim %lld differs from q head_dim %lld", (long long)vk.size[3],
           (long long)D);
  CF_CHECK(bs == block_size, "k_cache block dim %lld differs from block_size %d", (long long)bs, block_size);
  CF_CHECK(Hq > 0, "q has no heads");
  CF_CHECK(Hkv > 0 && Hq % Hkv == 0, "num_heads %lld is not a multiple of num_kv_heads %lld", (long long)Hq,
           (long long)Hkv);
  CF_CHECK(D > 0 && D <= 512, "head_dim %lld out of range (1..512)", (long long)D);
  CF_CHECK(vt.size[0] == B, "block_tables has %lld rows, batch is %lld", (long long)vt.size[0], (long long)B);
  CF_CHECK(vs.size[0] == B, "seq_lens has %lld entries, batch is %lld", (long long)vs.size[0], (long long)B);
  CF_CHECK(vo.size[0] == B && vo.size[1] == Hq && vo.size[2] == D, "out shape must be [%lld, %lld, %lld]",
           (long long)B, (long long)Hq, (long long)D);
  CF_CHECK(vq.stride[2] == 1 || D == 1, "q: head_dim stride must be 1");
  CF_CHECK(vo.stride[2] == 1 || D == 1, "out: head_dim stride must be 1");
  CF_CHECK(block_size > 0, "block_size must be positive");
  CF_CHECK(partition_tokens > 0 && partition_tokens % block_size == 0,
           "partition_tokens (%d) must be a positive multiple of block_size (%d)", partition_tokens, block_size);
  CF_CHECK(NB < (int64_t)INT32_MAX, "too many cache blocks");
  CF_CHECK(vt.size[1] * (int64_t)bs < (int64_t)INT32_MAX, "block table capacity overflows int32");
  CF_CHECK(std::isfinite(scale), "scale must be finite");

  DecodeParams p{};
  p.q = vq.base;
  p.q_sb = vq.stride[0];
  p.q_sh = vq.stride[1];
  p.k = vk.base;
  p.v = vv.base;
  for (int i = 0; i < 4; ++i) {
    p.k_s[i] = vk.stride[i];
    p.v_s[i] = vv.stride[i];
  }
  p.tables = (const int32_t*)vt.base;
  p.t_sb = vt.stride[0];
  p.t_sm = vt.stride[1];
  p.seq_lens = (const int32_t*)vs.base;
  p.sl_s = vs.stride[0];
  if (shared_prefix_lens != nullptr) {
    View vsh;
    if ((rc = view_of(shared_prefix_lens, "shared_prefix_lens", 1, &vsh))) return rc;
    CF_CHECK(vsh.dtype == CF_I32, "shared_prefix_lens: expected i32, got %s", dtype_name(vsh.dtype));
    CF_CHECK(vsh.size[0] == B, "shared_prefix_lens has %lld entries, batch is %lld", (long long)vsh.size[0],
             (long long)B);
    p.shared = (const int32_t*)vsh.base;
    p.sh_s = vsh.stride[0];
  }
  p.out = vo.base;
  p.o_sb = vo.stride[0];
  p.o_sh = vo.stride[1];
  p.scale = scale;
  p.B = (int)B;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.G = (int)(Hq / Hkv);
  p.D = (int)D;
  p.bs = block_size;
  p.Mb = (int)vt.size[1];
  p.NB = (int)NB;
  p.PT = generic_partition(B, Hq, Hkv, D, vt.size[1], block_size, partition_tokens);
  p.max_parts = (int)decode_max_parts(vt.size[1], block_size, p.PT);

  if (vk.dtype == CF_F8E4M3FN) {
    CF_CHECK(k_scale != nullptr && v_scale != nullptr, "f8e4m3fn caches need k_scale and v_scale");
    if ((rc = scale_view(k_scale, "k_scale", Hkv, &p.k_scale, &p.ks_s))) return rc;
    if ((rc = scale_view(v_scale, "v_scale", Hkv, &p.v_scale, &p.vs_s))) return rc;
  } else {
    CF_CHECK(k_scale == nullptr && v_scale == nullptr, "k_scale/v_scale apply to f8e4m3fn caches only");
  }
  if (B == 0) return CF_OK;

  const bool mfma = decode_mfma_supported(p, vq.dtype, vk.dtype);
  const uint64_t need = mfma ? decode_mfma_workspace_bytes(B, Hq, Hkv, D)
                             : generic_workspace_bytes(B, Hq, D, p.max_parts);
  if (need > 0) {
    if (workspace == nullptr || workspace_bytes < need) {
      set_error("workspace of %llu bytes needed, %llu given", (unsigned long long)need,
                (unsigned long long)workspace_bytes);
      return CF_ERR_WORKSPACE;
    }
    CF_CHECK(((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
    if (mfma) {
      decode_mfma_bind_workspace(p, workspace);
    } else {
      const uint64_t rows = (uint64_t)B * Hq * p.max_parts;
      char* base = (char*)workspace;
      p.ws_o = (float*)base;
      p.ws_ml = (float*)(base + (((rows * D * 4) + 255) & ~(uint64_t)255));
    }
  }

  hipStream_t st = as_stream(stream);
  if (mfma) return launch_decode_mfma(p, vq.dtype, vk.dtype, st);
  rc = launch_decode_generic(p, vq.dtype, vk.dtype, st);
  if (rc) return rc;
  if (p.max_parts > 1) rc = launch_decode_reduce(p, vq.dtype, st);
  return rc;
}

int32_t cf_paged_decode_shared_noalloc(const CfTensor* q, const CfTensor* k_cache, const CfTensor* v_cache,
                                       const CfTensor* block_tables, const CfTensor* seq_lens,
                                       const CfTensor* shared_prefix_lens, const CfTensor* k_scale,
                                       const CfTensor* v_scale, float scale, int32_t block_size,
                                       int32_t partition_tokens, CfTensor* out, void* stream) {
  void* ws = nullptr;
  int32_t rc = noalloc_scratch(&ws);
  if (rc) return rc;
  // The decode kernels rewrite every workspace cell they read in the same
  // call (merge descriptors, partial rows), so nothing needs clearing.
  rc = cf_paged_decode_shared(q, k_cache, v_cache, block_tables, seq_lens, shared_prefix_lens, k_scale, v_scale,
                              scale, block_size, partition_tokens, out, ws, kNoAllocScratchBytes, stream);
  if (rc == CF_ERR_WORKSPACE) {
    const std::string msg = last_error();
    set_error("this call needs more than the library's fixed scratch of %llu bytes per device (%s); use "
              "cf_paged_decode_shared with a workspace",
              (unsigned long long)kNoAllocScratchBytes, msg.c_str());
  }
  return rc;
}

int32_t cf_prefill_chunk_workspace_bytes(int64_t num_q_tokens, int64_t num_chunks, int64_t num_q_heads,
                                         int64_t num_kv_heads, int64_t head_dim, int32_t block_size,
                                         uint64_t* bytes_out) {
  CF_CHECK(bytes_out != nullptr, "bytes_out is NULL");
  CF_CHECK(num_q_tokens >= 0 && num_chunks >= 0 && num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0,
           "invalid sizes");
  CF_CHECK(num_q_heads % num_kv_heads == 0, "num_heads %lld is not a multiple of num_kv_heads %lld",
           (long long)num_q_heads, (long long)num_kv_heads);
  CF_CHECK(block_size == 16, "block_size must be 16, got %d", block_size);
  *bytes_out = prefill_workspace_bytes(num_q_tokens, num_chunks, num_q_heads, num_kv_heads, head_dim);
  return CF_OK;
}

int32_t cf_prefill_chunk_fp8(const CfTensor* q, const CfTensor* k_cache, const CfTensor* v_cache,
                             const CfTensor* block_tables, const CfTensor* seq_lens, const CfTensor* q_start,
                             const CfTensor* k_scale, const CfTensor* v_scale, float scale, int32_t block_size,
                             CfTensor* out, void* workspace, uint64_t workspace_bytes, void* stream) {
  View vq, vk, vv, vt, vs, vqs, vo;
  int32_t rc;
  if ((rc = view_of(q, "q", 3, &vq))) return rc;
  if ((rc = view_of(k_cache, "k_cache", 4, &vk))) return rc;
  if ((rc = view_of(v_cache, "v_cache", 4, &vv))) return rc;
  if ((rc = view_of(block_tables, "block_tables", 2, &vt))) return rc;
  if ((rc = view_of(seq_lens, "seq_lens", 1, &vs))) return rc;
  if ((rc = view_of(q_start, "q_start", 1, &vqs))) return rc;
  if ((rc = view_of(out, "out", 3, &vo))) return rc;

  CF_CHECK(vq.dtype == CF_BF16 || vq.dtype == CF_F16, "q: dtype must be bf16 or f16, got %s", dtype_name(vq.dtype));
  CF_CHECK(vk.dtype == CF_BF16 || vk.dtype == CF_F16 || vk.dtype == CF_F8E4M3FN,
           "k_cache: dtype must be bf16, f16 or f8e4m3fn, got %s", dtype_name(vk.dtype));
  CF_CHECK(vv.dtype == vk.dtype, "v_cache dtype %s differs from k_cache dtype %s", dtype_name(vv.dtype),
           dtype_name(vk.dtype));
  CF_CHECK(vt.dtype == CF_I32, "block_tables: expected i32, got %s", dtype_name(vt.dtype));
  CF_CHECK(vs.dtype == CF_I32, "seq_lens: expected i32, got %s", dtype_name(vs.dtype));
  CF_CHECK(vqs.dtype == CF_I32, "q_start: expected i32, got %s", dtype_name(vqs.dtype));
  CF_CHECK(vo.dtype == vq.dtype, "out: dtype %s differs from q dtype %s", dtype_name(vo.dtype),
           dtype_name(vq.dtype));

  const int64_t Tq = vq.size[0], Hq = vq.size[1], D = vq.size[2];
  const int64_t NB = vk.size[0], bs = vk.size[1], Hkv = vk.size[2];
  const int64_t N = vt.size[0];
  for (int i = 0; i < 4; ++i)
    CF_CHECK(vv.size[i] == vk.size[i], "v_cache shape differs from k_cache shape on dim %d", i);
  CF_CHECK(vk.size[3] == D, "k_cache head_dim %lld differs from q head_dim %lld", (long long)vk.size[3],
           (long long)D);
  CF_CHECK(block_size == 16, "block_size must be 16, got %d", block_size);
  CF_CHECK(bs == block_size, "k_cache block dim %lld differs from block_size %d", (long long)bs, block_size);
  CF_CHECK(Hq > 0, "q has no heads");
  CF_CHECK(Hkv > 0 && Hq % Hkv == 0, "num_heads %lld is not a multiple of num_kv_heads %lld", (long long)Hq,
           (long long)Hkv);
  CF_CHECK(vs.size[0] == N, "seq_lens has %lld entries, block_tables has %lld rows", (long long)vs.size[0],
           (long long)N);
  CF_CHECK(vqs.size[0] == N + 1, "q_start must have %lld entries, got %lld", (long long)(N + 1),
           (long long)vqs.size[0]);
  CF_CHECK(vo.size[0] == Tq && vo.size[1] == Hq && vo.size[2] == D, "out shape must be [%lld, %lld, %lld]",
           (long long)Tq, (long long)Hq, (long long)D);
  CF_CHECK(vq.stride[2] == 1, "q: head_dim stride must be 1");
  CF_CHECK(vo.stride[2] == 1, "out: head_dim stride must be 1");
  CF_CHECK(NB < (int64_t)INT32_MAX, "too many cache blocks");
  CF_CHECK(Tq < (int64_t)INT32_MAX / 2 && N < (int64_t)INT32_MAX / 2, "too many query rows or chunks");
  CF_CHECK(Hkv < 65536, "too many KV heads");
  CF_CHECK(std::isfinite(scale), "scale must be finite");

  PrefillParams p{};
  p.q = vq.base;
  p.q_sr = vq.stride[0];
  p.q_sh = vq.stride[1];
  p.out = vo.base;
  p.o_sr = vo.stride[0];
  p.o_sh = vo.stride[1];
  p.k = vk.base;
  p.v = vv.base;
  for (int i = 0; i < 4; ++i) {
    p.k_s[i] = vk.stride[i];
    p.v_s[i] = vv.stride[i];
  }
  p.tables = (const int32_t*)vt.base;
  p.t_sb = vt.stride[0];
  p.t_sm = vt.stride[1];
  p.seq_lens = (const int32_t*)vs.base;
  p.sl_s = vs.stride[0];
  p.q_start = (const int32_t*)vqs.base;
  p.qs_s = vqs.stride[0];
  p.scale = scale;
  p.N = (int)N;
  p.Tq = (int)Tq;
  p.Hq = (int)Hq;
  p.Hkv = (int)Hkv;
  p.G = (int)(Hq / Hkv);
  p.D = (int)D;
  p.Mb = (int)vt.size[1];
  p.NB = (int)NB;
  if (vk.dtype == CF_F8E4M3FN) {
    CF_CHECK(k_scale != nullptr && v_scale != nullptr, "f8e4m3fn caches need k_scale and v_scale");
    if ((rc = scale_view(k_scale, "k_scale", Hkv, &p.k_scale, &p.ks_s))) return rc;
    if ((rc = scale_view(v_scale, "v_scale", Hkv, &p.v_scale, &p.vs_s))) return rc;
  } else {
    CF_CHECK(k_scale == nullptr && v_scale == nullptr, "k_scale/v_scale apply to f8e4m3fn caches only");
  }
  if (!prefill_supported(p, vq.dtype, vk.dtype)) {
    set_error("prefill: needs bf16 q over bf16/e4m3 caches or f16 q over f16/e4m3 caches, head_dim 64/128, "
              "GQA group 1/2/4/8/16, native or token-major caches with 16-byte aligned blocks, heads and token "
              "rows, and 16-byte aligned q rows");
    return CF_ERR_UNSUPPORTED;
  }
  if (Tq == 0 || N == 0) return CF_OK;
  p.RB = prefill_rows_per_item(p.G);
  CF_CHECK((Tq / p.RB + N) * Hkv < (int64_t)INT32_MAX / 2, "too many prefill work items");
  p.max_items = (int)((Tq / p.RB + N) * Hkv);
  const uint64_t need = prefill_workspace_bytes(Tq, N, Hq, Hkv, D);
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("workspace of %llu bytes needed, %llu given", (unsigned long long)need,
              (unsigned long long)workspace_bytes);
    return CF_ERR_WORKSPACE;
  }
  CF_CHECK(((uintptr_t)workspace & 255) == 0, "workspace must be 256-byte aligned");
  prefill_bind_workspace(p, workspace);
  return launch_prefill(p, vq.dtype, vk.dtype, as_stream(stream));
}

int32_t cf_fp8_amax_scale(const CfTensor* x, CfTensor* scales, void* stream) {
  View vx, vsc;
  int32_t rc;
  if ((rc = view_of_34(x, "x", &vx))) return rc;
  if ((rc = view_of(scales, "scales", 1, &vsc))) return rc;
  CF_CHECK(is_float_dtype(vx.dtype), "x: dtype must be f32, f16 or bf16, got %s", dtype_name(vx.dtype));
  CF_CHECK(vsc.dtype == CF_F32, "scales: expected f32, got %s", dtype_name(vsc.dtype));
  const Rank4 x4 = rank4_of(vx);
  CF_CHECK(vsc.size[0] == x4.size[2], "scales has %lld entries, x has %lld heads", (long long)vsc.size[0],
           (long long)x4.size[2]);
  CF_CHECK(vsc.stride[0] == 1 || vsc.size[0] <= 1, "scales must be contiguous");
  CF_CHECK(x4.size[2] < 65536, "too many heads");
  CF_CHECK(x4.size[0] * x4.size[1] / std::max<int64_t>(1, 4096 / std::max<int64_t>(1, x4.size[3])) < (int64_t)INT32_MAX,
           "x too large");
  if (x4.size[2] == 0) return CF_OK;
  return launch_amax_scale(x4, vx.dtype, (float*)vsc.base, 1, as_stream(stream));
}

int32_t cf_kv_amax_scale(const CfTensor* x, CfTensor* scales_out, void* stream) {
  return cf_fp8_amax_scale(x, scales_out, stream);
}

int32_t cf_fp8_quantize(const CfTensor* x, const CfTensor* scales, CfTensor* out, void* stream) {
  View vx, vo;
  int32_t rc;
  if ((rc = view_of_34(x, "x", &vx))) return rc;
  if ((rc = view_of_34(out, "out", &vo))) return rc;
  CF_CHECK(is_float_dtype(vx.dtype), "x: dtype must be f32, f16 or bf16, got %s", dtype_name(vx.dtype));
  CF_CHECK(vo.dtype == CF_F8E4M3FN, "out: expected f8e4m3fn, got %s", dtype_name(vo.dtype));
  const Rank4 x4 = rank4_of(vx), o4 = rank4_of(vo);
  for (int i = 0; i < 4; ++i) CF_CHECK(o4.size[i] == x4.size[i], "out shape differs from x");
  const float* sp;
  int64_t ss;
  if ((rc = scale_view(scales, "scales", x4.size[2], &sp, &ss))) return rc;
  return launch_quantize(x4, vx.dtype, sp, ss, o4, as_stream(stream));
}

int32_t cf_fp8_quantize_kv(const CfTensor* k, const CfTensor* v, const CfTensor* k_scales, const CfTensor* v_scales,
                           CfTensor* k_out, CfTensor* v_out, void* stream) {
  View vk, vv, vko, vvo;
  int32_t rc;
  if ((rc = view_of_34(k, "k", &vk))) return rc;
  if ((rc = view_of_34(v, "v", &vv))) return rc;
  if ((rc = view_of_34(k_out, "k_out", &vko))) return rc;
  if ((rc = view_of_34(v_out, "v_out", &vvo))) return rc;
  CF_CHECK(is_float_dtype(vk.dtype), "k: dtype must be f32, f16 or bf16, got %s", dtype_name(vk.dtype));
  CF_CHECK(vv.dtype == vk.dtype, "v: dtype %s differs from k's %s", dtype_name(vv.dtype), dtype_name(vk.dtype));
  CF_CHECK(vko.dtype == CF_F8E4M3FN && vvo.dtype == CF_F8E4M3FN, "k_out, v_out: expected f8e4m3fn");
  const Rank4 k4 = rank4_of(vk), v4 = rank4_of(vv), ko4 = rank4_of(vko), vo4 = rank4_of(vvo);
  for (int i = 0; i < 4; ++i) {
    CF_CHECK(v4.size[i] == k4.size[i], "v shape differs from k");
    CF_CHECK(ko4.size[i] == k4.size[i] && vo4.size[i] == k4.size[i], "output shapes differ from k");
  }
  const float *ksp, *vsp;
  int64_t kss, vss;
  if ((rc = scale_view(k_scales, "k_scales", k4.size[2], &ksp, &kss))) return rc;
  if ((rc = scale_view(v_scales, "v_scales", k4.size[2], &vsp, &vss))) return rc;
  return launch_quantize_kv(k4, v4, vk.dtype, ksp, kss, vsp, vss, ko4, vo4, as_stream(stream));
}

int32_t cf_fp8_dequantize(const CfTensor* q, const CfTensor* scales, CfTensor* out, void* stream) {
  View vq, vo;
  int32_t rc;
  if ((rc = view_of_34(q, "q", &vq))) return rc;
  if ((rc = view_of_34(out, "out", &vo))) return rc;
  CF_CHECK(vq.dtype == CF_F8E4M3FN, "q: expected f8e4m3fn, got %s", dtype_name(vq.dtype));
  CF_CHECK(vo.dtype == CF_F32, "out: expected f32, got %s", dtype_name(vo.dtype));
  const Rank4 q4 = rank4_of(vq), o4 = rank4_of(vo);
  for (int i = 0; i < 4; ++i) CF_CHECK(o4.size[i] == q4.size[i], "out shape differs from q");
  const float* sp;
  int64_t ss;
  if ((rc = scale_view(scales, "scales", q4.size[2], &sp, &ss))) return rc;
  return launch_dequantize(q4, sp, ss, o4, as_stream(stream));
}

int32_t cf_kv_write_fp8(const CfTensor* k_new, const CfTensor* v_new, const CfTensor* slot_mapping,
                        CfTensor* k_cache, CfTensor* v_cache, const CfTensor* k_scale, const CfTensor* v_scale,
                        void* stream) {
  View vk, vv, vsl, vkc, vvc;
  int32_t rc;
  if ((rc = view_of(k_new, "k_new", 3, &vk))) return rc;
  if ((rc = view_of(v_new, "v_new", 3, &vv))) return rc;
  if ((rc = view_of(slot_mapping, "slot_mapping", 1, &vsl))) return rc;
  if ((rc = view_of(k_cache, "k_cache", 4, &vkc))) return rc;
  if ((rc = view_of(v_cache, "v_cache", 4, &vvc))) return rc;
  CF_CHECK(is_float_dtype(vk.dtype), "k_new: dtype must be f32, f16 or bf16, got %s", dtype_name(vk.dtype));
  CF_CHECK(vv.dtype == vk.dtype, "v_new dtype differs from k_new dtype");
  CF_CHECK(vsl.dtype == CF_I32 || vsl.dtype == CF_I64, "slot_mapping: expected i32 or i64, got %s",
           dtype_name(vsl.dtype));
  CF_CHECK(vkc.dtype == CF_F8E4M3FN && vvc.dtype == CF_F8E4M3FN, "caches must be f8e4m3fn");
  for (int i = 0; i < 3; ++i) CF_CHECK(vv.size[i] == vk.size[i], "v_new shape differs from k_new on dim %d", i);
  for (int i = 0; i < 4; ++i) CF_CHECK(vvc.size[i] == vkc.size[i], "v_cache shape differs from k_cache on dim %d", i);
  const int64_t T = vk.size[0], H = vk.size[1], D = vk.size[2];
  CF_CHECK(vsl.size[0] == T, "slot_mapping has %lld entries, %lld tokens given", (long long)vsl.size[0],
           (long long)T);
  CF_CHECK(vkc.size[2] == H && vkc.size[3] == D, "cache [NB, bs, %lld, %lld] does not match new rows [T, %lld, %lld]",
           (long long)vkc.size[2], (long long)vkc.size[3], (long long)H, (long long)D);
  CF_CHECK(vkc.size[1] > 0, "cache block size must be positive");
  CF_CHECK(T < (int64_t)INT32_MAX && H * D < (int64_t)INT32_MAX, "too many rows");
  KvWriteParams p{};
  if ((rc = scale_view(k_scale, "k_scale", H, &p.k_scale, &p.ks_s))) return rc;
  if ((rc = scale_view(v_scale, "v_scale", H, &p.v_scale, &p.vs_s))) return rc;
  p.k_new = rank4_of(vk);
  p.v_new = rank4_of(vv);
  p.slots = vsl.base;
  p.slot_stride = vsl.stride[0];
  p.k_cache = vkc.base;
  p.v_cache = vvc.base;
  for (int i = 0; i < 4; ++i) {
    p.kc_s[i] = vkc.stride[i];
    p.vc_s[i] = vvc.stride[i];
  }
  p.T = T;
  p.H = (int)H;
  p.D = (int)D;
  p.bs = (int)vkc.size[1];
  p.NB = vkc.size[0];
  return launch_kv_write_fp8(p, vk.dtype, vsl.dtype, as_stream(stream));
}

int32_t cf_paged_write(const CfTensor* x_new, const CfTensor* slot_mapping, CfTensor* cache, const CfTensor* scale,
                       void* stream) {
  View vx, vsl, vc;
  int32_t rc;
  if ((rc = view_of(x_new, "x_new", 3, &vx))) return rc;
  if ((rc = view_of(slot_mapping, "slot_mapping", 1, &vsl))) return rc;
  if ((rc = view_of(cache, "cache", 4, &vc))) return rc;
  CF_CHECK(is_float_dtype(vx.dtype), "x_new: dtype must be f32, f16 or bf16, got %s", dtype_name(vx.dtype));
  CF_CHECK(vsl.dtype == CF_I32 || vsl.dtype == CF_I64, "slot_mapping: expected i32 or i64, got %s",
           dtype_name(vsl.dtype));
  CF_CHECK(is_float_dtype(vc.dtype) || vc.dtype == CF_F8E4M3FN,
           "cache: dtype must be f32, f16, bf16 or f8e4m3fn, got %s", dtype_name(vc.dtype));
  const int64_t T = vx.size[0], H = vx.size[1], D = vx.size[2];
  CF_CHECK(vsl.size[0] == T, "slot_mapping has %lld entries, %lld rows given", (long long)vsl.size[0], (long long)T);
  CF_CHECK(vc.size[2] == H && vc.size[3] == D, "cache [NB, bs, %lld, %lld] does not match rows [T, %lld, %lld]",
           (long long)vc.size[2], (long long)vc.size[3], (long long)H, (long long)D);
  CF_CHECK(vc.size[1] > 0, "cache block size must be positive");
  CF_CHECK(H < 65536 && D < 65536 && vc.size[1] < 65536, "cache dims too large");
  PagedWriteParams p{};
  if (vc.dtype == CF_F8E4M3FN) {
    CF_CHECK(scale != nullptr, "f8e4m3fn caches need a scale");
    if ((rc = scale_view(scale, "scale", H, &p.scale, &p.sc_s))) return rc;
  } else {
    CF_CHECK(scale == nullptr, "scale applies to f8e4m3fn caches only");
  }
  p.x = vx.base;
  for (int i = 0; i < 3; ++i) p.x_s[i] = vx.stride[i];
  p.slots = vsl.base;
  p.slot_s = vsl.stride[0];
  p.cache = vc.base;
  for (int i = 0; i < 4; ++i) p.c_s[i] = vc.stride[i];
  p.T = T;
  p.NB = vc.size[0];
  p.H = (int)H;
  p.D = (int)D;
  p.bs = (int)vc.size[1];
  return launch_paged_write(p, vx.dtype, vsl.dtype, vc.dtype, as_stream(stream));
}

int32_t cf_paged_gather(const CfTensor* cache, const CfTensor* block_tables, const CfTensor* scale, CfTensor* out,
                        void* stream) {
  View vc, vt, vo;
  int32_t rc;
  if ((rc = view_of(cache, "cache", 4, &vc))) return rc;
  if ((rc = view_of(block_tables, "block_tables", 2, &vt))) return rc;
  if ((rc = view_of(out, "out", 4, &vo))) return rc;
  CF_CHECK(is_float_dtype(vc.dtype) || vc.dtype == CF_F8E4M3FN,
           "cache: dtype must be f32, f16, bf16 or f8e4m3fn, got %s", dtype_name(vc.dtype));
  CF_CHECK(vt.dtype == CF_I32, "block_tables: expected i32, got %s", dtype_name(vt.dtype));
  CF_CHECK(is_float_dtype(vo.dtype), "out: dtype must be f32, f16 or bf16, got %s", dtype_name(vo.dtype));
  const int64_t R = vt.size[0];
  CF_CHECK(vo.size[0] == R && vo.size[2] == vc.size[2] && vo.size[3] == vc.size[3],
           "out must be [%lld, S, %lld, %lld]", (long long)R, (long long)vc.size[2], (long long)vc.size[3]);
  CF_CHECK(vc.size[1] > 0, "cache block size must be positive");
  CF_CHECK(R < (int64_t)INT32_MAX && vo.size[1] < (int64_t)INT32_MAX && vt.size[1] < (int64_t)INT32_MAX &&
               vc.size[2] < 65536 && vc.size[3] < 65536 && vc.size[1] < 65536,
           "gather dims too large");
  PagedGatherParams p{};
  if (vc.dtype == CF_F8E4M3FN) {
    CF_CHECK(scale != nullptr, "f8e4m3fn caches need a scale");
    if ((rc = scale_view(scale, "scale", vc.size[2], &p.scale, &p.sc_s))) return rc;
  } else {
    CF_CHECK(scale == nullptr, "scale applies to f8e4m3fn caches only");
  }
  p.cache = vc.base;
  for (int i = 0; i < 4; ++i) {
    p.c_s[i] = vc.stride[i];
    p.o_s[i] = vo.stride[i];
  }
  p.tables = (const int32_t*)vt.base;
  p.t_sr = vt.stride[0];
  p.t_sm = vt.stride[1];
  p.out = vo.base;
  p.NB = vc.size[0];
  p.R = (int)R;
  p.Mb = (int)vt.size[1];
  p.S = (int)vo.size[1];
  p.H = (int)vc.size[2];
  p.D = (int)vc.size[3];
  p.bs = (int)vc.size[1];
  return launch_paged_gather(p, vc.dtype, vo.dtype, as_stream(stream));
}

int32_t cf_stage_from_host(const void* host_src, void* dev_dst, uint64_t bytes, void* stream) {
  CF_CHECK(host_src != nullptr && dev_dst != nullptr, "NULL pointer");
  CF_CHECK(bytes % 16 == 0, "bytes (%llu) must be a multiple of 16", (unsigned long long)bytes);
  CF_CHECK(((uintptr_t)host_src & 15) == 0 && ((uintptr_t)dev_dst & 15) == 0, "pointers must be 16-byte aligned");
  if (bytes == 0) return CF_OK;
  // The device's view of the host buffer; fails unless the memory is pinned
  // and mapped (hipHostMalloc), so nothing else is ever dereferenced.
  // A refused query also sets HIP's per-thread last error, which the caller's
  // next runtime check (torch's, after its next launch) would report as its
  // own failure: read it back here so the refusal stays this call's.
  void* view = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&view, const_cast<void*>(host_src), 0);
  if (e != hipSuccess || view == nullptr) {
    (void)hipGetLastError();
    set_error("host_src is not mapped pinned host memory (hipHostGetDevicePointer: %s)", hipGetErrorString(e));
    return CF_ERR_INVALID;
  }
  hipPointerAttribute_t attr;
  const hipError_t ea = hipPointerGetAttributes(&attr, dev_dst);
  if (ea != hipSuccess || attr.type != hipMemoryTypeDevice) {
    (void)hipGetLastError();
    set_error("dev_dst is not device memory (hipPointerGetAttributes: %s)", hipGetErrorString(ea));
    return CF_ERR_INVALID;
  }
  return launch_stage_from_host(view, dev_dst, bytes, as_stream(stream));
}

int32_t cf_profile_enable(int32_t on) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  g_prof_on = on != 0;
  return CF_OK;
}

int32_t cf_profile_reset(void) {
  std::lock_guard<std::mutex> lock(g_prof_mu);
  for (auto& r : g_prof_records) {
    (void)hipEventSynchronize(r.end);
    g_prof_pool.push_back(r.begin);
    g_prof_pool.push_back(r.end);
  }
  g_prof_records.clear();
  return CF_OK;
}

int32_t cf_profile_query(const char* prefix, double* total_ms, int64_t* launches) {
  CF_CHECK(prefix != nullptr && total_ms != nullptr && launches != nullptr, "NULL argument");
  std::lock_guard<std::mutex> lock(g_prof_mu);
  double sum = 0.0;
  int64_t n = 0;
  const size_t plen = std::strlen(prefix);
  for (auto& r : g_prof_records) {
    if (r.name.compare(0, plen, prefix) != 0) continue;
    CF_HIP_CHECK(hipEventSynchronize(r.end));
    float ms = 0.0f;
    CF_HIP_CHECK(hipEventElapsedTime(&ms, r.begin, r.end));
    sum += ms;
    ++n;
  }
  *total_ms = sum;
  *launches = n;
  return CF_OK;
}

int32_t cf_profile_reserve(int64_t events) {
  CF_CHECK(events >= 0 && events <= (1 << 20), "cf_profile_reserve: %lld events out of range", (long long)events);
  std::lock_guard<std::mutex> lock(g_prof_mu);
  while ((int64_t)g_prof_pool.size() < events) {
    hipEvent_t e = nullptr;
    CF_HIP_CHECK(hipEventCreate(&e));
    g_prof_pool.push_back(e);
  }
  return CF_OK;
}

int32_t cf_profile_durations(const char* prefix, float* ms, int64_t cap, int64_t* launches) {
  CF_CHECK(prefix != nullptr && launches != nullptr, "NULL argument");
  CF_CHECK(cap >= 0 && (cap == 0 || ms != nullptr), "cf_profile_durations: NULL output for %lld entries",
           (long long)cap);
  std::lock_guard<std::mutex> lock(g_prof_mu);
  int64_t n = 0;
  const size_t plen = std::strlen(prefix);
  for (auto& r : g_prof_records) {
    if (r.name.compare(0, plen, prefix) != 0) continue;
    if (n < cap) {
      CF_HIP_CHECK(hipEventSynchronize(r.end));
      float d = 0.0f;
      CF_HIP_CHECK(hipEventElapsedTime(&d, r.begin, r.end));
      ms[n] = d;
    }
    ++n;
  }
  *launches = n;
  return CF_OK;
}

}  // extern "C"
