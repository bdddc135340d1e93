// Paged-cache row I/O kernels.
//
// paged_write: token i's row goes to slot slots[i] = block * bs + offset of
// a [NB, bs, H, D] cache (the reference's token placement,
// python_runtime/engine/cache_manager.py:139-171 and _kv_cache.py:68-104),
// converted to the cache dtype: e4m3fn codes are e4m3_from_f32(x / scale[h])
// (FP8KVCacheQuantizer's arithmetic, compiler/quantize/fp8_kv_cache.py:89),
// bf16 / fp16 round to nearest even, f32 is exact.  Slots outside
// [0, NB * bs) are skipped.
//
// paged_gather: out[r, s] = the row of token s of table r (block
// tables[r][s / bs], offset s % bs), dequantized (e4m3fn: code * scale[h]);
// a table entry outside [0, NB) gives zeros (the reference gathers a
// request's blocks in table order and leaves positions past its table zero,
// cache_manager.py:173-197).
//
// Both kernels give one thread a piece of 16 channels of one (token, head)
// row when the head dim is a multiple of 16 (a lone channel otherwise),
// and move a piece with 16-byte loads / stores where the row is contiguous
// and aligned, element by element otherwise (e.g. the channel-major V
// layout, token stride 1).
#include "cf_device.hpp"
#include "cf_host.hpp"
#include "paged_io.hpp"

namespace cf {

namespace {

template <int DT>
__device__ __forceinline__ float load_as_f32(const void* base, int64_t i) {
  using E = Elem<DT>;
  return E::load((const typename E::T*)base + i);
}

template <int DT>
__device__ __forceinline__ void store_from_f32(void* base, int64_t i, float v) {
  using E = Elem<DT>;
  E::store((typename E::T*)base + i, v);
}

// Loads n (<= 16) elements of one row as f32: 16-byte vectors when `vec`
// (then n == 16 and the address is 16-byte aligned), strided otherwise.
template <int DT>
__device__ __forceinline__ void load_row(const void* base, int64_t off, int64_t stride, int n, bool vec, float* f) {
  if (vec) {
    constexpr int EB = sizeof(typename Elem<DT>::T);
    const uint4* s = (const uint4*)((const char*)base + off * EB);
#pragma unroll
    for (int q = 0; q < 16 * EB / 16; ++q) {
      const uint4 u = s[q];
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (EB == 4) {
          f[4 * q + j] = u2f(w[j]);
        } else if constexpr (EB == 2) {
          f[8 * q + 2 * j] = Elem<DT>::load((const typename Elem<DT>::T*)&w[j]);
          f[8 * q + 2 * j + 1] = Elem<DT>::load((const typename Elem<DT>::T*)&w[j] + 1);
        } else {
#pragma unroll
          for (int b = 0; b < 4; ++b) f[16 * q + 4 * j + b] = Elem<DT>::load((const typename Elem<DT>::T*)&w[j] + b);
        }
      }
    }
  } else {
    for (int e = 0; e < n; ++e) f[e] = load_as_f32<DT>(base, off + e * stride);
  }
}

// Stores n (<= 16) values of one row converted to DT (e4m3fn: divided by
// `div` first); vector stores when `vec`.
template <int DT>
__device__ __forceinline__ void store_row(void* base, int64_t off, int64_t stride, int n, bool vec, const float* f,
                                          float div) {
  using E = Elem<DT>;
  using T = typename E::T;
  if (vec) {
    constexpr int EB = sizeof(T);
    T tmp[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      if constexpr (DT == kE4M3) tmp[e] = e4m3_from_f32(f[e] / div);
      else E::store(&tmp[e], f[e]);
    }
    uint4* d = (uint4*)((char*)base + off * EB);
#pragma unroll
    for (int q = 0; q < 16 * EB / 16; ++q) d[q] = ((const uint4*)tmp)[q];
  } else {
    for (int e = 0; e < n; ++e) {
      T* dst = (T*)base + off + e * stride;
      if constexpr (DT == kE4M3) *dst = e4m3_from_f32(f[e] / div);
      else E::store(dst, f[e]);
    }
  }
}

template <int XT, int ST, int CT>
__global__ __launch_bounds__(256) void paged_write_kernel(PagedWriteParams p, int pw, bool xvec, bool cvec) {
  const int np = p.D / pw;
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= p.T * p.H * np) return;
  const int c = (int)(u % np), h = (int)((u / np) % p.H);
  const int64_t i = u / ((int64_t)np * p.H);
  const int64_t sl = ST == kI64 ? ((const int64_t*)p.slots)[i * p.slot_s]
                                : (int64_t)((const int32_t*)p.slots)[i * p.slot_s];
  if (sl < 0 || sl >= p.NB * p.bs) return;
  const int64_t blk = sl / p.bs, off = sl % p.bs;
  float f[16];
  load_row<XT>(p.x, i * p.x_s[0] + h * p.x_s[1] + (int64_t)c * pw * p.x_s[2], p.x_s[2], pw, xvec, f);
  const float div = CT == kE4M3 ? p.scale[h * p.sc_s] : 1.0f;
  store_row<CT>(p.cache, blk * p.c_s[0] + off * p.c_s[1] + h * p.c_s[2] + (int64_t)c * pw * p.c_s[3], p.c_s[3], pw,
                cvec, f, div);
}

template <int CT, int OT>
__global__ __launch_bounds__(256) void paged_gather_kernel(PagedGatherParams p, int pw, bool cvec, bool ovec) {
  const int np = p.D / pw;
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= (int64_t)p.R * p.S * p.H * np) return;
  const int c = (int)(u % np), h = (int)((u / np) % p.H);
  const int64_t rs = u / ((int64_t)np * p.H);
  const int s = (int)(rs % p.S), r = (int)(rs / p.S);
  const int jb = s / p.bs;
  int64_t blk = -1;
  if (jb < p.Mb) {
    const int id = p.tables[(int64_t)r * p.t_sr + (int64_t)jb * p.t_sm];
    if (id >= 0 && id < p.NB) blk = id;
  }
  float f[16];
  if (blk >= 0) {
    load_row<CT>(p.cache, blk * p.c_s[0] + (int64_t)(s % p.bs) * p.c_s[1] + h * p.c_s[2] + (int64_t)c * pw * p.c_s[3],
                 p.c_s[3], pw, cvec, f);
    if constexpr (CT == kE4M3) {
      const float sc = p.scale[h * p.sc_s];
      for (int e = 0; e < pw; ++e) f[e] *= sc;
    }
  } else {
    for (int e = 0; e < pw; ++e) f[e] = 0.0f;
  }
  store_row<OT>(p.out, (int64_t)r * p.o_s[0] + (int64_t)s * p.o_s[1] + h * p.o_s[2] + (int64_t)c * pw * p.o_s[3],
                p.o_s[3], pw, ovec, f, 1.0f);
}

int dt_bytes(int dt) { return dt == kF32 ? 4 : (dt == kE4M3 ? 1 : 2); }

// A row piece of 16 elements at element offsets base + k * (row strides)
// moves as 16-byte vectors when the innermost stride is 1 and every row
// start is 16-byte aligned.
bool rows_aligned(const void* base, const int64_t* strides, int n_outer, int64_t inner, int eb) {
  if (inner != 1 || ((uintptr_t)base & 15)) return false;
  for (int i = 0; i < n_outer; ++i)
    if ((strides[i] * eb) % 16 != 0) return false;
  return true;
}

int64_t grid_of(int64_t threads) { return (threads + 255) / 256; }

}  // namespace

int32_t launch_paged_write(const PagedWriteParams& p, int x_dt, int slot_dt, int cache_dt, hipStream_t stream) {
  if (p.T == 0 || p.H == 0 || p.D == 0) return CF_OK;
  const int pw = p.D % 16 == 0 ? 16 : 1;
  const bool xvec = pw == 16 && rows_aligned(p.x, p.x_s, 2, p.x_s[2], dt_bytes(x_dt));
  const bool cvec = pw == 16 && rows_aligned(p.cache, p.c_s, 3, p.c_s[3], dt_bytes(cache_dt));
  const int64_t threads = p.T * p.H * (p.D / pw);
  CF_CHECK(grid_of(threads) < (int64_t)INT32_MAX, "paged write too large");
  const dim3 grid((unsigned)grid_of(threads));
  ProfileScope prof("cf_paged_write", stream);
#define CF_PW(XT, ST, CT) \
  CF_LAUNCH((paged_write_kernel<XT, ST, CT>), grid, dim3(256), 0, stream, p, pw, xvec, cvec)
#define CF_PW_C(XT, ST)                                                              \
  switch (cache_dt) {                                                                \
    case kF32: CF_PW(XT, ST, kF32); break;                                           \
    case kF16: CF_PW(XT, ST, kF16); break;                                           \
    case kBF16: CF_PW(XT, ST, kBF16); break;                                         \
    case kE4M3: CF_PW(XT, ST, kE4M3); break;                                         \
    default: set_error("paged write: unsupported cache dtype %d", cache_dt); return CF_ERR_UNSUPPORTED; \
  }
#define CF_PW_X(ST)                                                                  \
  switch (x_dt) {                                                                    \
    case kF32: CF_PW_C(kF32, ST); break;                                             \
    case kF16: CF_PW_C(kF16, ST); break;                                             \
    case kBF16: CF_PW_C(kBF16, ST); break;                                           \
    default: set_error("paged write: unsupported row dtype %d", x_dt); return CF_ERR_UNSUPPORTED; \
  }
  if (slot_dt == kI64) {
    CF_PW_X(kI64);
  } else {
    CF_PW_X(kI32);
  }
#undef CF_PW_X
#undef CF_PW_C
#undef CF_PW
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

int32_t launch_paged_gather(const PagedGatherParams& p, int cache_dt, int out_dt, hipStream_t stream) {
  if (p.R == 0 || p.S == 0 || p.H == 0 || p.D == 0) return CF_OK;
  const int pw = p.D % 16 == 0 ? 16 : 1;
  const bool cvec = pw == 16 && rows_aligned(p.cache, p.c_s, 3, p.c_s[3], dt_bytes(cache_dt));
  const bool ovec = pw == 16 && rows_aligned(p.out, p.o_s, 3, p.o_s[3], dt_bytes(out_dt));
  const int64_t threads = (int64_t)p.R * p.S * p.H * (p.D / pw);
  CF_CHECK(grid_of(threads) < (int64_t)INT32_MAX, "paged gather too large");
  const dim3 grid((unsigned)grid_of(threads));
  ProfileScope prof("cf_paged_gather", stream);
#define CF_PG(CT, OT) \
  CF_LAUNCH((paged_gather_kernel<CT, OT>), grid, dim3(256), 0, stream, p, pw, cvec, ovec)
#define CF_PG_O(CT)                                                                  \
  switch (out_dt) {                                                                  \
    case kF32: CF_PG(CT, kF32); break;                                               \
    case kF16: CF_PG(CT, kF16); break;                                               \
    case kBF16: CF_PG(CT, kBF16); break;                                             \
    default: set_error("paged gather: unsupported output dtype %d", out_dt); return CF_ERR_UNSUPPORTED; \
  }
  switch (cache_dt) {
    case kF32: CF_PG_O(kF32); break;
    case kF16: CF_PG_O(kF16); break;
    case kBF16: CF_PG_O(kBF16); break;
    case kE4M3: CF_PG_O(kE4M3); break;
    default: set_error("paged gather: unsupported cache dtype %d", cache_dt); return CF_ERR_UNSUPPORTED;
  }
#undef CF_PG_O
#undef CF_PG
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

// ---- upload of host-packed tables --------------------------------------------
// Copies n 16-byte words from device-visible pinned host memory into device
// memory: the upload rides the compute queue with the kernels that read it,
// so back-to-back calls hand nothing between the copy engine and the
// compute queue.  Host memory is read once: plain vector loads.
__global__ __launch_bounds__(256) void stage_from_host_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                              int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) dst[i] = src[i];
}

int32_t launch_stage_from_host(const void* src_dev_view, void* dst, uint64_t bytes, hipStream_t stream) {
  const int64_t n = (int64_t)(bytes / 16);
  if (n == 0) return CF_OK;
  const int64_t blocks = std::min<int64_t>(ceil_div(n, 256), 64);
  ProfileScope prof("cf_stage_from_host", stream);
  CF_LAUNCH(stage_from_host_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, (const uint4*)src_dev_view,
            (uint4*)dst, n);
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

}  // namespace cf
