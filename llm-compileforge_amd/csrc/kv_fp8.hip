// FP8 (OCP e4m3fn) KV quantization kernels.
//
// Arithmetic follows FP8KVCacheQuantizer (reference
// compiler/quantize/fp8_kv_cache.py:66-105), applied per KV head:
//   amax  = max |x|                                  (:81)
//   scale = 1.0 if amax == 0 else max(amax / 448, 1e-12)   (:82-86)
//   code  = e4m3fn(f32(x) / scale)                   (:89)
//   deq   = f32(code) * scale                        (:105)
// The division is IEEE correctly rounded (the library is built without
// fast-math and with correctly-rounded fp32 division), so codes and scales
// are bit-identical to the CPU path.
#include "cf_device.hpp"
#include "cf_host.hpp"
#include "kv_fp8.hpp"

#include <algorithm>

namespace cf {

namespace {

// ---- amax -> scale ------------------------------------------------------

__global__ void zero_u32_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// One workgroup per (row chunk, head).  |x| is compared as unsigned bits:
// for non-negative floats (and NaN, whose bits exceed +inf) integer order is
// float order, so atomicMax on the bits gives amax and propagates NaN like
// torch's max.
template <int XT>
__global__ __launch_bounds__(256) void amax_kernel(Rank4 x, uint32_t* amax_bits, int rows_per_block) {
  const int h = blockIdx.y;
  const int64_t nrows = x.size[0] * x.size[1];
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < nrows ? r0 + rows_per_block : nrows;
  using XE = Elem<XT>;
  const typename XE::T* base = (const typename XE::T*)x.base;
  uint32_t m = 0;
  const int64_t D = x.size[3];
  const int64_t n = (r1 - r0) * D;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const int64_t r = r0 + i / D, d = i % D;
    const int64_t a = r / x.size[1], t = r % x.size[1];
    const float v = XE::load(base + a * x.stride[0] + t * x.stride[1] + h * x.stride[2] + d * x.stride[3]);
    const uint32_t u = f2u(v) & 0x7FFFFFFFu;
    m = m > u ? m : u;
  }
  m = wave_umax(m);
  if ((threadIdx.x & 63) == 0 && m != 0u) atomicMax(amax_bits + h, m);
}

__global__ void scale_from_amax_kernel(uint32_t* scale_bits, int64_t stride, int H) {
  const int h = blockIdx.x * blockDim.x + threadIdx.x;
  if (h >= H) return;
  uint32_t* slot = scale_bits + h * stride;
  const float amax = u2f(*slot);
  float s;
  if (amax == 0.0f) {
    s = 1.0f;
  } else {
    s = amax / 448.0f;
    // torch.clamp(min=1e-12): NaN stays NaN, values below the bound are raised.
    if (s < 1e-12f) s = 1e-12f;
  }
  *slot = f2u(s);
}

// ---- quantize / dequantize ----------------------------------------------

// Flat index -> (a, t, h, d) of a [S0, S1, H, D] view.
__device__ __forceinline__ int64_t offset4(const Rank4& v, int64_t i) {
  const int64_t D = v.size[3], H = v.size[2], S1 = v.size[1];
  const int64_t d = i % D;
  i /= D;
  const int64_t h = i % H;
  i /= H;
  const int64_t t = i % S1;
  const int64_t a = i / S1;
  return a * v.stride[0] + t * v.stride[1] + h * v.stride[2] + d * v.stride[3];
}

__device__ __forceinline__ int64_t head_of(const Rank4& v, int64_t i) { return (i / v.size[3]) % v.size[2]; }

template <int XT>
__global__ __launch_bounds__(256) void quantize_kernel(Rank4 x, const float* scales, int64_t s_stride, Rank4 out) {
  const int64_t n = x.size[0] * x.size[1] * x.size[2] * x.size[3];
  using XE = Elem<XT>;
  const typename XE::T* xb = (const typename XE::T*)x.base;
  uint8_t* ob = (uint8_t*)out.base;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float v = XE::load(xb + offset4(x, i));
    ob[offset4(out, i)] = e4m3_from_f32(v / scales[head_of(x, i) * s_stride]);
  }
}

__global__ __launch_bounds__(256) void dequantize_kernel(Rank4 q, const float* scales, int64_t s_stride, Rank4 out) {
  const int64_t n = q.size[0] * q.size[1] * q.size[2] * q.size[3];
  const uint8_t* qb = (const uint8_t*)q.base;
  float* ob = (float*)out.base;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    ob[offset4(out, i)] = f32_from_e4m3(qb[offset4(q, i)]) * scales[head_of(q, i) * s_stride];
  }
}

// ---- paged KV write -------------------------------------------------------

// One workgroup per new token; threads cover (kv head, d) for K then V.
template <int XT, int ST>
__global__ __launch_bounds__(256) void kv_write_kernel(KvWriteParams p) {
  const int64_t i = blockIdx.x;
  int64_t slot;
  if (ST == kI64) slot = ((const int64_t*)p.slots)[i * p.slot_stride];
  else slot = ((const int32_t*)p.slots)[i * p.slot_stride];
  if (slot < 0 || slot >= p.NB * p.bs) return;
  const int64_t blk = slot / p.bs, off = slot % p.bs;
  using XE = Elem<XT>;
  const int n = p.H * p.D;
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    const int h = j / p.D, d = j % p.D;
    const float kv = XE::load((const typename XE::T*)p.k_new.base + i * p.k_new.stride[1] +
                              h * p.k_new.stride[2] + d * p.k_new.stride[3]);
    const float vv = XE::load((const typename XE::T*)p.v_new.base + i * p.v_new.stride[1] +
                              h * p.v_new.stride[2] + d * p.v_new.stride[3]);
    uint8_t* kd = (uint8_t*)p.k_cache + blk * p.kc_s[0] + off * p.kc_s[1] + h * p.kc_s[2] + d * p.kc_s[3];
    uint8_t* vd = (uint8_t*)p.v_cache + blk * p.vc_s[0] + off * p.vc_s[1] + h * p.vc_s[2] + d * p.vc_s[3];
    *kd = e4m3_from_f32(kv / p.k_scale[h * p.ks_s]);
    *vd = e4m3_from_f32(vv / p.v_scale[h * p.vs_s]);
  }
}

// Streaming (non-temporal) 16-byte accesses for data touched once.
typedef unsigned nt_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 stream_load16(const void* p) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load((const nt_u32x4*)p));
}
__device__ __forceinline__ void stream_store16(void* p, uint4 v) {
  __builtin_nontemporal_store(__builtin_bit_cast(nt_u32x4, v), (nt_u32x4*)p);
}

// The 16 elements held in EB 16-byte registers (as load16 reads them) as floats.
template <int XT>
__device__ __forceinline__ void unpack16(const uint4* u, float* f) {
  if constexpr (XT == kF32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[4 * i] = u2f(u[i].x);
      f[4 * i + 1] = u2f(u[i].y);
      f[4 * i + 2] = u2f(u[i].z);
      f[4 * i + 3] = u2f(u[i].w);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint32_t w[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (XT == kBF16) {
          f[8 * i + 2 * j] = f32_from_bf16_bits(w[j] & 0xFFFFu);
          f[8 * i + 2 * j + 1] = f32_from_bf16_bits(w[j] >> 16);
        } else {
          f[8 * i + 2 * j] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] & 0xFFFFu));
          f[8 * i + 2 * j + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[j] >> 16));
        }
      }
    }
  }
}

__device__ __forceinline__ uint4 pack16(const uint32_t* b) {
  uint4 r;
  r.x = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
  r.y = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
  r.z = b[8] | (b[9] << 8) | (b[10] << 16) | (b[11] << 24);
  r.w = b[12] | (b[13] << 8) | (b[14] << 16) | (b[15] << 24);
  return r;
}

// Paged write into the native layout (block size 16: K tile [bs][D] token
// rows, V tile [D][bs] channel rows).  One thread per (new token, head,
// 16-channel piece): 16 K values quantized into one 16-byte store of the
// token's K row, 16 V values into one byte of each of 16 V channel rows.
// Codes are the same e4m3_from_f32(x / scale) as kv_write_kernel.
template <int XT, int ST>
__device__ __forceinline__ int64_t slot_at(const KvWriteParams& p, int64_t i) {
  return ST == kI64 ? ((const int64_t*)p.slots)[i * p.slot_stride]
                    : (int64_t)((const int32_t*)p.slots)[i * p.slot_stride];
}

// Workgroups [0, k_blocks): K, one thread per (new row, head, 16-channel
// piece): a 16-byte load, 16 conversions, one 16-byte store of the token's
// K row piece.  Workgroups after that: V, one per (group of 16 new rows,
// 256 channels of the H * D); each thread owns one (head, channel).  V is
// channel-major in a block (16 tokens of a channel are 16 contiguous
// bytes), so the rows are split into runs of consecutive slots inside one
// block: a run starting in the group is written by this workgroup (it may
// extend past the group), a full block row as one 16-byte store, a partial
// run as byte stores.  Run boundaries depend only on the slots, so every
// thread of the workgroup writes the same runs.
//
// The kernel is bound by latency and instruction issue (a few microseconds
// for a step's rows), not by bytes: loads of the new rows do not wait for
// the slots, index math is 32-bit, and the per-row work of the V path is
// vector code (one scalar unit serves the CU's four SIMDs).
template <int XT, int ST>
__global__ __launch_bounds__(256) void kv_write_native_kernel(KvWriteParams p, uint32_t k_blocks, uint32_t v_chunks) {
  using XE = Elem<XT>;
  using T = typename XE::T;
  constexpr int EB = sizeof(T);
  const int64_t cap = p.NB * 16;
  if (blockIdx.x < k_blocks) {
    const uint32_t nch = (uint32_t)p.D / 16u, per_row = nch * (uint32_t)p.H;
    const uint32_t u = blockIdx.x * 256u + threadIdx.x;
    if (u >= (uint32_t)p.T * per_row) return;  // the host keeps T * H * D / 16 below 2^31
    const uint32_t i = u / per_row, rem = u - i * per_row;
    const uint32_t h = rem / nch, c = rem - h * nch;
    const uint4* src = (const uint4*)((const uint8_t*)p.k_new.base +
                                      ((int64_t)i * p.k_new.stride[1] + (int64_t)h * p.k_new.stride[2] + c * 16) * EB);
    uint4 raw[EB];
#pragma unroll
    for (int j = 0; j < EB; ++j) raw[j] = src[j];
    const int64_t sl = slot_at<XT, ST>(p, i);
#pragma unroll
    for (int j = 0; j < EB; ++j) asm volatile("" ::"v"(raw[j].x), "v"(raw[j].y), "v"(raw[j].z), "v"(raw[j].w));
    if (sl < 0 || sl >= cap) return;
    float f[16];
    unpack16<XT>(raw, f);
    const Fp8Quant qk(p.k_scale[h * p.ks_s]);
    *(uint4*)((uint8_t*)p.k_cache + (sl >> 4) * p.kc_s[0] + (int64_t)h * p.kc_s[2] + (sl & 15) * p.D + c * 16) =
        qk.pack16(f);
    return;
  }
  const uint32_t vb = blockIdx.x - k_blocks;
  const uint32_t g = vb / v_chunks;
  const int hd = (int)(vb - g * v_chunks) * 256 + (int)threadIdx.x;
  const bool mine = hd < p.H * p.D;
  const int h = mine ? hd / p.D : 0, d = mine ? hd % p.D : 0;
  // lane l holds the slot of row g * 16 - 1 + l (-1 outside [0, T)): the
  // row before the group, the group's 16 rows and the 15 after them (a run
  // starting in the group ends within 16 rows)
  const int lane = (int)(threadIdx.x & 63);
  const int64_t r = (int64_t)g * 16 - 1 + lane;
  const int64_t sl = r >= 0 && r < p.T ? slot_at<XT, ST>(p, r) : -1;
  // rows g*16 .. g*16+30 of this thread's channel (clamped to the last row),
  // loaded while the slots are in flight: a uniform row base + the thread's
  // 32-bit (head, channel) offset (the host checks it fits)
  const int last = (int)(p.T - 1 - (int64_t)g * 16 < 30 ? p.T - 1 - (int64_t)g * 16 : 30);
  const uint8_t* gbase = (const uint8_t*)p.v_new.base + (int64_t)g * 16 * p.v_new.stride[1] * EB;
  const uint32_t rs = (uint32_t)(p.v_new.stride[1] * EB);
  const uint32_t voff = (uint32_t)(((int64_t)h * p.v_new.stride[2] + d) * EB);
  T raw[31];
#pragma unroll
  for (int e = 0; e < 31; ++e) raw[e] = *(const T*)(gbase + (voff + (uint32_t)(e < last ? e : last) * rs));
  const bool valid = sl >= 0 && sl < cap;
  const int64_t up = __shfl_up(sl, 1, 64);
  // cont: this row takes the slot after the previous row's, in the same block
  const bool cont = valid && lane > 0 && sl == up + 1 && (sl & 15) != 0;
  const uint32_t vm = (uint32_t)__ballot(valid), cm = (uint32_t)__ballot(cont);
  // Lane 1 + e <-> row e of the group.  Runs start at valid rows that do not
  // continue the previous one; the group owns the valid rows 0..15 from its
  // first run start on, and rows 16..30 that continue its last run.
  const uint32_t starts = vm & ~cm & 0x1FFFEu;
  if (!mine || starts == 0u) return;
  const int e0 = __builtin_ctz(starts) - 1;     // first owned row, 0..15
  const int ext = __builtin_ctz(~(cm >> 17));  // <= 15: runs stop at a block end
  const uint32_t own = ((vm & 0x1FFFEu & ~((2u << e0) - 1u)) >> 1) | (((1u << ext) - 1u) << 16);
  // each row's destination (block row base + token offset), per lane
  const int64_t dst = valid ? (sl >> 4) * p.vc_s[0] + (sl & 15) : 0;
  const uint32_t chan = (uint32_t)((int64_t)h * p.vc_s[2] + d * 16);
  uint8_t* vcache = (uint8_t*)p.v_cache;
  auto dst_of = [&](int e) {  // row e's destination (uniform)
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)(uint64_t)dst, e + 1);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)dst >> 32), e + 1);
    return (int64_t)(((uint64_t)hi << 32) | lo);
  };
  const Fp8Quant qv(p.v_scale[h * p.vs_s]);
  const uint32_t ow = own >> e0;
  if (ow <= 0xFFFFu) {
    // the owned rows lie in e0 .. e0+15: one window of 16 values, quantized
    // together
    float win[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      if (e0 == k) {
#pragma unroll
        for (int j = 0; j < 16; ++j) win[j] = XE::load(&raw[k + j]);
      }
    }
    const uint4 c4 = qv.pack16(win);
    if (ow == 0xFFFFu && ((cm >> (e0 + 2)) & 0x7FFFu) == 0x7FFFu) {
      // a run of 16 rows fills one block's channel row (its start is at
      // token 0 of the block)
      *(uint4*)(vcache + dst_of(e0) + chan) = c4;
      return;
    }
    const uint32_t cw[4] = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if ((ow >> j) & 1u) vcache[dst_of(e0 + j) + chan] = (uint8_t)(cw[j >> 2] >> (8 * (j & 3)));
    return;
  }
  // owned rows spread over more than 16 (a short run, then a run reaching
  // past the group): byte by byte
#pragma unroll
  for (int e = 0; e < 31; ++e)
    if ((own >> e) & 1u) vcache[dst_of(e) + chan] = qv(XE::load(&raw[e]));
}

// Whether kv_write_native_kernel applies: native cache layout with block
// size 16, 16-byte aligned K rows and V channel rows, and new K/V rows whose
// 16-channel pieces are 16-byte aligned.
bool kv_write_native_ok(const KvWriteParams& p, int x_dt) {
  const int eb = x_dt == kF32 ? 4 : 2;
  if (p.bs != 16 || p.D % 16 != 0) return false;
  if (p.kc_s[3] != 1 || p.kc_s[1] != p.D || p.vc_s[1] != 1 || p.vc_s[3] != 16) return false;
  if ((p.kc_s[0] | p.kc_s[2] | p.vc_s[0] | p.vc_s[2]) & 15) return false;
  if (((uintptr_t)p.k_cache | (uintptr_t)p.v_cache) & 15) return false;
  for (const Rank4* x : {&p.k_new, &p.v_new}) {
    if (x->stride[3] != 1 || ((uintptr_t)x->base & 15)) return false;
    if (((x->stride[1] * eb) | (x->stride[2] * eb)) & 15) return false;
  }
  // 32-bit index math and offsets: K pieces, a V row's (head, channel)
  // offset plus 30 row strides, a V channel row's offset in a block
  if (p.T * p.H * (p.D / 16) >= (int64_t)INT32_MAX) return false;
  if (p.v_new.stride[1] < 0 || p.v_new.stride[2] < 0 || p.vc_s[2] < 0) return false;
  if (((int64_t)(p.H - 1) * p.v_new.stride[2] + p.D + 30 * p.v_new.stride[1]) * eb >= (int64_t)UINT32_MAX) return false;
  if ((int64_t)(p.H - 1) * p.vc_s[2] + (int64_t)p.D * 16 >= (int64_t)UINT32_MAX) return false;
  return true;
}

// ---- row-piece kernels (head_dim a multiple of 16) ------------------------
// A row is the D elements of one (a, t, h) of a [S0, S1, H, D] view; a piece
// is 16 consecutive elements of a row.  Pieces load and store as 16-byte
// vectors where the view's rows are contiguous and 16-byte aligned, element
// by element otherwise (e.g. the channel-major V layout).

__device__ __forceinline__ int64_t row_offset(const Rank4& v, int64_t a_t, int h) {
  const int64_t t = a_t % v.size[1], a = a_t / v.size[1];
  return a * v.stride[0] + t * v.stride[1] + (int64_t)h * v.stride[2];
}

template <int XT>
__device__ __forceinline__ void load_piece(const Rank4& x, int64_t off, bool vec, float* f) {
  using XE = Elem<XT>;
  const typename XE::T* src = (const typename XE::T*)x.base + off;
  if (vec) {
    load16<XT>(src, f);
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) f[e] = XE::load(src + e * x.stride[3]);
  }
}

// One workgroup per (run of rows_per_block rows, head): max |x| over its
// pieces, one atomic per workgroup.
template <int XT>
__global__ __launch_bounds__(256) void amax_rows_kernel(Rank4 x, uint32_t* amax_bits, int rows_per_block, bool vec) {
  const int h = blockIdx.y;
  const int64_t rows = x.size[0] * x.size[1];
  const int np = (int)(x.size[3] / 16);
  const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
  const int64_t n = (rows - r0 < rows_per_block ? rows - r0 : rows_per_block) * np;
  uint32_t m = 0;
  for (int64_t i = threadIdx.x; i < n; i += 256) {
    const int64_t r = r0 + i / np;
    const int c = (int)(i % np);
    float f[16];
    load_piece<XT>(x, row_offset(x, r, h) + (int64_t)c * 16 * x.stride[3], vec, f);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t u = f2u(f[e]) & 0x7FFFFFFFu;
      m = m > u ? m : u;
    }
  }
  m = wave_umax(m);
  __shared__ uint32_t wm[4];
  if ((threadIdx.x & 63) == 0) wm[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    m = wm[0];
    for (int w = 1; w < 4; ++w) m = m > wm[w] ? m : wm[w];
    if (m != 0u) atomicMax(amax_bits + h, m);
  }
}

// One thread per piece: e4m3fn(x / scales[h]).
template <int XT>
__global__ __launch_bounds__(256) void quantize_rows_kernel(Rank4 x, const float* scales, int64_t s_stride, Rank4 out,
                                                            bool xvec, bool ovec) {
  const int H = (int)x.size[2];
  const int np = (int)(x.size[3] / 16);
  const int64_t n = x.size[0] * x.size[1] * H * np;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int c = (int)(i % np);
    const int h = (int)((i / np) % H);
    const int64_t r = i / ((int64_t)np * H);
    float f[16];
    load_piece<XT>(x, row_offset(x, r, h) + (int64_t)c * 16 * x.stride[3], xvec, f);
    const Fp8Quant qz(scales[h * s_stride]);
    uint32_t b[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) b[e] = qz(f[e]);
    uint8_t* dst = (uint8_t*)out.base + row_offset(out, r, h) + (int64_t)c * 16 * out.stride[3];
    if (ovec) {
      *(uint4*)dst = pack16(b);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) dst[e * out.stride[3]] = (uint8_t)b[e];
    }
  }
}

// One thread per piece: f32(code) * scales[h].
__global__ __launch_bounds__(256) void dequantize_rows_kernel(Rank4 q, const float* scales, int64_t s_stride, Rank4 out,
                                                              bool qvec, bool ovec) {
  const int H = (int)q.size[2];
  const int np = (int)(q.size[3] / 16);
  const int64_t n = q.size[0] * q.size[1] * H * np;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    const int c = (int)(i % np);
    const int h = (int)((i / np) % H);
    const int64_t r = i / ((int64_t)np * H);
    const uint8_t* src = (const uint8_t*)q.base + row_offset(q, r, h) + (int64_t)c * 16 * q.stride[3];
    uint32_t b[16];
    if (qvec) {
      const uint4 u = *(const uint4*)src;
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 16; ++e) b[e] = (w[e >> 2] >> (8 * (e & 3))) & 0xFFu;
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) b[e] = src[e * q.stride[3]];
    }
    const float sc = scales[h * s_stride];
    float* dst = (float*)out.base + row_offset(out, r, h) + (int64_t)c * 16 * out.stride[3];
    if (ovec) {
#pragma unroll
      for (int e = 0; e < 16; e += 4)
        *(float4*)(dst + e) = make_float4(f32_from_e4m3(b[e]) * sc, f32_from_e4m3(b[e + 1]) * sc,
                                          f32_from_e4m3(b[e + 2]) * sc, f32_from_e4m3(b[e + 3]) * sc);
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) dst[e * out.stride[3]] = f32_from_e4m3(b[e]) * sc;
    }
  }
}

// Whether rows of v (element size eb) load/store as aligned 16-byte pieces.
bool rows_vectorizable(const Rank4& v, int eb) {
  if (v.stride[3] != 1 || ((uintptr_t)v.base & 15)) return false;
  for (int i = 0; i < 3; ++i)
    if (v.size[i] > 1 && (v.stride[i] * eb) % 16 != 0) return false;
  return true;
}

// ---- span kernels (32-bit indexing) ---------------------------------------
// For views whose rows are uniformly strided ([S0, S1] folds into one row
// axis) and whose 16-element pieces are contiguous and 16-byte aligned.
// Piece k of a launch is (row k / P, head (k % P) / np, piece (k % P) % np)
// with np = D / 16 and P = H * np, so consecutive threads read consecutive
// pieces of a row; the host checks that rows * P fits in 31 bits.
struct SpanView {
  const char* base;    // bytes
  int64_t row_stride;  // bytes
  int64_t head_stride; // bytes
  int rows, H, np, P;
};

constexpr int kSpanMaxHeads = 1024;  // per-head maxima a workgroup keeps in LDS

// amax over a span: each workgroup takes a contiguous range of rows, keeps
// one running max per head in LDS (a thread flushes its register max when
// its piece moves to another head), then raises the global per-head bits
// with atomicMax only where its max exceeds the value already there -- so
// after the first few workgroups almost none of them issue the atomic, and
// the launch can be wide without the workgroups queueing on H addresses.
template <int XT>
__global__ __launch_bounds__(256) void amax_span_kernel(SpanView v, uint32_t* amax_bits, int rows_per_wg, int q256,
                                                        int r256) {
  constexpr int EB = sizeof(typename Elem<XT>::T);
  __shared__ uint32_t hmax[kSpanMaxHeads];
  for (int h = threadIdx.x; h < v.H; h += 256) hmax[h] = 0u;
  __syncthreads();
  const int r_begin = blockIdx.x * rows_per_wg;
  const int r_end = min(r_begin + rows_per_wg, v.rows);
  const int n = (r_end - r_begin) * v.P;
  int row = r_begin + (int)threadIdx.x / v.P, rem = (int)threadIdx.x % v.P;
  int cur = -1;
  uint32_t m = 0u;
  for (int k = threadIdx.x; k < n; k += 256) {
    const int h = rem / v.np, c = rem - h * v.np;
    float f[16];
    load16<XT>(v.base + row * v.row_stride + h * v.head_stride + c * 16 * EB, f);
    if (h != cur) {
      if (cur >= 0 && m != 0u) atomicMax(&hmax[cur], m);
      cur = h;
      m = 0u;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t u = f2u(f[e]) & 0x7FFFFFFFu;
      m = m > u ? m : u;
    }
    row += q256;
    rem += r256;
    if (rem >= v.P) {
      rem -= v.P;
      ++row;
    }
  }
  if (cur >= 0 && m != 0u) atomicMax(&hmax[cur], m);
  __syncthreads();
  for (int h = threadIdx.x; h < v.H; h += 256) {
    const uint32_t mine = hmax[h];
    if (mine != 0u && mine > __hip_atomic_load(amax_bits + h, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
      atomicMax(amax_bits + h, mine);
  }
}

// One thread per piece of a span: 16 elements in, one 16-byte store out
// into an output whose rows are contiguous 16-byte-aligned runs (e.g. the
// native / paired K tile rows); output row r sits at (r / o_s1) * o_s0 +
// (r % o_s1) * o_s1stride.  Loads and stores are non-temporal: every byte
// is touched once.  (A fixed grid striding over the pieces with the next
// piece's loads in flight measured slower: 515 vs 414 us at the
// Llama-3-8B pool size.)
template <int XT>
__global__ __launch_bounds__(256) void quantize_span_kernel(SpanView x, const float* scales, int64_t s_stride,
                                                            char* out, int o_s1, int64_t o_s0, int64_t o_s1stride,
                                                            int64_t o_head, int n) {
  constexpr int EB = sizeof(typename Elem<XT>::T);
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k >= n) return;
  const int row = k / x.P, rem = k - row * x.P;
  const int h = rem / x.np, c = rem - h * x.np;
  const char* src = x.base + row * x.row_stride + h * x.head_stride + c * 16 * EB;
  uint4 raw[EB];
#pragma unroll
  for (int i = 0; i < EB; ++i) raw[i] = stream_load16(src + 16 * i);
  float f[16];
  unpack16<XT>(raw, f);
  const Fp8Quant qz(scales[h * s_stride]);
  const int a = row / o_s1, t = row - a * o_s1;
  stream_store16(out + a * o_s0 + t * o_s1stride + h * o_head + c * 16, qz.pack16(f));
}

// Channel-major outputs with 16 tokens per block (the native / paired V
// tile: the 16 tokens of one channel are 16 contiguous bytes).  One thread
// per (block, head, channel): the channel's 16 tokens are read from the
// token-major source (consecutive threads read consecutive channels, so
// every load instruction is one contiguous run), converted and written as
// one 16-byte store -- the transpose happens in registers.
template <int XT>
__global__ __launch_bounds__(256) void quantize_transpose16_kernel(Rank4 x, const float* scales, int64_t s_stride,
                                                                   char* out, int64_t o_blk, int64_t o_head,
                                                                   int64_t o_chan, int n) {
  using XE = Elem<XT>;
  using T = typename XE::T;
  const int k = blockIdx.x * 256 + threadIdx.x;
  if (k >= n) return;
  const int D = (int)x.size[3], H = (int)x.size[2];
  const int d = k % D;
  const int hk = k / D;
  const int h = hk % H;
  const int a = hk / H;
  const T* src = (const T*)x.base + a * x.stride[0] + h * x.stride[2] + (int64_t)d * x.stride[3];
  float f[16];
#pragma unroll
  for (int t = 0; t < 16; ++t) f[t] = XE::load(src + t * x.stride[1]);
  const Fp8Quant qz(scales[h * s_stride]);
  stream_store16(out + a * o_blk + h * o_head + (int64_t)d * o_chan, qz.pack16(f));
}

// K and V of [S0, 16, H, D] pools into native-tile outputs in one launch:
// K tiles [16 tokens][D] (row stride D bytes) and V tiles [D][16 tokens] at
// the same block and head strides -- in particular the paired layout, where
// the two tiles of a (block, head) sit side by side.  One workgroup per block
// writes every K and V tile of the block: K in pieces of 16 channels taken in
// tile order (head, token, piece), so each wave writes 1 KiB of a tile; V as
// 16-token channel rows, the transpose done in registers.  Writing both
// halves of every pair from one workgroup keeps the write stream whole
// (a K-only pass writes half of every 4 KiB pair: 4.9 vs 5.8 TB/s measured
// on the part).  Per-head scales and reciprocals come from LDS.
template <int XT>
__global__ __launch_bounds__(256) void quantize_kv_tiles_kernel(Rank4 k, Rank4 v, const float* ks, int64_t ks_s,
                                                                const float* vs, int64_t vs_s, char* k_out,
                                                                char* v_out, int64_t o_blk, int64_t o_head) {
  using XE = Elem<XT>;
  using T = typename XE::T;
  constexpr int EB = sizeof(T);
  __shared__ float sc[4][kSpanMaxHeads];  // K scale, K reciprocal, V scale, V reciprocal
  const int H = (int)k.size[2], D = (int)k.size[3];
  for (int h = threadIdx.x; h < H; h += 256) {
    const float a = ks[h * ks_s], b = vs[h * vs_s];
    sc[0][h] = a;
    sc[1][h] = 1.0f / a;
    sc[2][h] = b;
    sc[3][h] = 1.0f / b;
  }
  __syncthreads();
  const int64_t blk = blockIdx.x;
  const int np = D >> 4;         // 16-channel pieces per K row
  const int nk = 16 * H * np;    // K pieces of the block
  const T* kb = (const T*)k.base + blk * k.stride[0];
  char* kob = k_out + blk * o_blk;
  for (int q = threadIdx.x; q < nk; q += 256) {
    const int c = q % np, t = (q / np) & 15, h = q / (16 * np);
    const char* src = (const char*)(kb + t * k.stride[1] + h * k.stride[2] + c * 16);
    uint4 raw[EB];
#pragma unroll
    for (int i = 0; i < EB; ++i) raw[i] = stream_load16(src + 16 * i);
    float f[16];
    unpack16<XT>(raw, f);
    const Fp8Quant qz(sc[0][h], sc[1][h]);
    stream_store16(kob + h * o_head + t * D + c * 16, qz.pack16(f));
  }
  const int nv = H * D;
  const T* vb = (const T*)v.base + blk * v.stride[0];
  char* vob = v_out + blk * o_blk;
  for (int ch = threadIdx.x; ch < nv; ch += 256) {
    const int h = ch / D, d = ch - h * D;
    const T* src = vb + h * v.stride[2] + (int64_t)d * v.stride[3];
    float f[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) f[t] = XE::load(src + t * v.stride[1]);
    const Fp8Quant qz(sc[2][h], sc[3][h]);
    stream_store16(vob + h * o_head + d * 16, qz.pack16(f));
  }
}

// A SpanView of v (element size eb) when its rows fold into one uniformly
// strided axis, its pieces are contiguous and 16-byte aligned and the launch
// indexes fit in 31 bits.
bool span_of(const Rank4& v, int eb, SpanView* s) {
  if (v.size[3] % 16 != 0 || v.size[3] == 0 || v.stride[3] != 1 || ((uintptr_t)v.base & 15)) return false;
  const int64_t rows = v.size[0] * v.size[1];
  int64_t rs = v.stride[1];
  if (v.size[1] == 1) rs = v.stride[0];
  else if (v.size[0] > 1 && v.stride[0] != v.size[1] * v.stride[1]) return false;
  if (((rs * eb) & 15) || ((v.stride[2] * eb) & 15)) return false;
  if (v.size[2] > kSpanMaxHeads) return false;
  const int64_t np = v.size[3] / 16, P = v.size[2] * np;
  if (rows <= 0 || P <= 0 || rows * P >= (int64_t)INT32_MAX - 256) return false;
  s->base = (const char*)v.base;
  s->row_stride = rs * eb;
  s->head_stride = v.stride[2] * eb;
  s->rows = (int)rows;
  s->H = (int)v.size[2];
  s->np = (int)np;
  s->P = (int)P;
  return true;
}

int grid_for(int64_t n) {
  int64_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  return (int)(g < 1 ? 1 : g);
}

}  // namespace

int32_t launch_amax_scale(const Rank4& x, int x_dt, float* scales, int64_t s_stride, hipStream_t stream) {
  const int H = (int)x.size[2];
  // The (contiguous) scale vector doubles as the amax accumulator: its fp32
  // slots hold amax bits until the finalize step turns them into scales.
  uint32_t* acc = (uint32_t*)scales;
  {
    ProfileScope prof("cf_fp8_zero", stream);
    CF_LAUNCH(zero_u32_kernel, dim3((H + 255) / 256), dim3(256), 0, stream, acc, H);
  }
  CF_HIP_CHECK(hipGetLastError());
  const int64_t T = x.size[0] * x.size[1];
  SpanView sv;
  if (T > 0 && span_of(x, x_dt == kF32 ? 4 : 2, &sv)) {
    // ~16 KB of source per workgroup, at most 8 workgroups per CU's worth
    const int eb = x_dt == kF32 ? 4 : 2;
    const int64_t row_bytes = (int64_t)sv.P * 16 * eb;
    int64_t wgs = std::max<int64_t>(1, (int64_t)sv.rows * row_bytes / (16 * 1024));
    wgs = std::min<int64_t>(wgs, 8 * (int64_t)device_cu_count());
    const int rows_per_wg = (int)ceil_div(sv.rows, wgs);
    wgs = ceil_div(sv.rows, rows_per_wg);
    const int q256 = 256 / sv.P, r256 = 256 % sv.P;
    ProfileScope prof("cf_fp8_amax", stream);
    switch (x_dt) {
      case kF32: CF_LAUNCH((amax_span_kernel<kF32>), dim3((unsigned)wgs), dim3(256), 0, stream, sv, acc, rows_per_wg, q256, r256); break;
      case kF16: CF_LAUNCH((amax_span_kernel<kF16>), dim3((unsigned)wgs), dim3(256), 0, stream, sv, acc, rows_per_wg, q256, r256); break;
      case kBF16: CF_LAUNCH((amax_span_kernel<kBF16>), dim3((unsigned)wgs), dim3(256), 0, stream, sv, acc, rows_per_wg, q256, r256); break;
      default: set_error("amax: unsupported dtype %d", x_dt); return CF_ERR_UNSUPPORTED;
    }
    CF_HIP_CHECK(hipGetLastError());
  } else if (T > 0 && x.size[3] > 0 && x.size[3] % 16 == 0) {
    // rows of 16-element pieces: ~16 KB per workgroup
    const int rows = (int)std::max<int64_t>(1, 8192 / x.size[3]);
    const dim3 grid((unsigned)ceil_div(T, rows), H);
    const bool vec = rows_vectorizable(x, x_dt == kF32 ? 4 : 2);
    ProfileScope prof("cf_fp8_amax", stream);
    switch (x_dt) {
      case kF32: CF_LAUNCH((amax_rows_kernel<kF32>), grid, dim3(256), 0, stream, x, acc, rows, vec); break;
      case kF16: CF_LAUNCH((amax_rows_kernel<kF16>), grid, dim3(256), 0, stream, x, acc, rows, vec); break;
      case kBF16: CF_LAUNCH((amax_rows_kernel<kBF16>), grid, dim3(256), 0, stream, x, acc, rows, vec); break;
      default: set_error("amax: unsupported dtype %d", x_dt); return CF_ERR_UNSUPPORTED;
    }
    CF_HIP_CHECK(hipGetLastError());
  } else if (T > 0 && x.size[3] > 0) {
    const int rows = (int)std::max<int64_t>(1, 4096 / std::max<int64_t>(1, x.size[3]));
    const dim3 grid((unsigned)ceil_div(T, rows), H);
    ProfileScope prof("cf_fp8_amax", stream);
    switch (x_dt) {
      case kF32: CF_LAUNCH((amax_kernel<kF32>), grid, dim3(256), 0, stream, x, acc, rows); break;
      case kF16: CF_LAUNCH((amax_kernel<kF16>), grid, dim3(256), 0, stream, x, acc, rows); break;
      case kBF16: CF_LAUNCH((amax_kernel<kBF16>), grid, dim3(256), 0, stream, x, acc, rows); break;
      default: set_error("amax: unsupported dtype %d", x_dt); return CF_ERR_UNSUPPORTED;
    }
    CF_HIP_CHECK(hipGetLastError());
  }
  {
    ProfileScope prof("cf_fp8_scale", stream);
    CF_LAUNCH(scale_from_amax_kernel, dim3((H + 255) / 256), dim3(256), 0, stream, acc, s_stride, H);
  }
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

int32_t launch_quantize(const Rank4& x, int x_dt, const float* scales, int64_t s_stride, const Rank4& out,
                        hipStream_t stream) {
  const int64_t n = x.size[0] * x.size[1] * x.size[2] * x.size[3];
  if (n == 0) return CF_OK;
  ProfileScope prof("cf_fp8_quantize", stream);
  const int xeb = x_dt == kF32 ? 4 : 2;
  SpanView sv;
  // token-major output rows (contiguous 16-byte pieces): one thread per piece
  if (span_of(x, xeb, &sv) && rows_vectorizable(out, 1) && out.size[1] < (int64_t)INT32_MAX &&
      n / 16 < (int64_t)INT32_MAX - 256) {
    const int np = (int)(n / 16);
    const int os1 = (int)std::max<int64_t>(out.size[1], 1);
    const dim3 grid((unsigned)ceil_div(np, 256));
    char* ob = (char*)out.base;
#define CF_QS(XT) \
  CF_LAUNCH((quantize_span_kernel<XT>), grid, dim3(256), 0, stream, sv, scales, s_stride, ob, os1, out.stride[0], \
            out.stride[1], out.stride[2], np)
    switch (x_dt) {
      case kF32: CF_QS(kF32); break;
      case kF16: CF_QS(kF16); break;
      case kBF16: CF_QS(kBF16); break;
      default: set_error("quantize: unsupported dtype %d", x_dt); return CF_ERR_UNSUPPORTED;
    }
#undef CF_QS
    CF_HIP_CHECK(hipGetLastError());
    return CF_OK;
  }
  // channel-major 16-token output blocks (the native / paired V tile)
  if (out.size[1] == 16 && out.stride[1] == 1 && out.stride[3] % 16 == 0 && ((uintptr_t)out.base & 15) == 0 &&
      (out.size[0] <= 1 || out.stride[0] % 16 == 0) && (out.size[2] <= 1 || out.stride[2] % 16 == 0) &&
      n / 16 < (int64_t)INT32_MAX - 256) {
    const int nt = (int)(n / 16);
    const dim3 grid((unsigned)ceil_div(nt, 256));
    char* ob = (char*)out.base;
    switch (x_dt) {
      case kF32: CF_LAUNCH((quantize_transpose16_kernel<kF32>), grid, dim3(256), 0, stream, x, scales, s_stride, ob, out.stride[0], out.stride[2], out.stride[3], nt); break;
      case kF16: CF_LAUNCH((quantize_transpose16_kernel<kF16>), grid, dim3(256), 0, stream, x, scales, s_stride, ob, out.stride[0], out.stride[2], out.stride[3], nt); break;
      case kBF16: CF_LAUNCH((quantize_transpose16_kernel<kBF16>), grid, dim3(256), 0, stream, x, scales, s_stride, ob, out.stride[0], out.stride[2], out.stride[3], nt); break;
      default: set_error("quantize: unsupported dtype %d", x_dt); return CF_ERR_UNSUPPORTED;
    }
    CF_HIP_CHECK(hipGetLastError());
    return CF_OK;
  }
  if (x.size[3] % 16 == 0) {
    const dim3 grid(grid_for(n / 16));
    const bool xv = rows_vectorizable(x, x_dt == kF32 ? 4 : 2), ov = rows_vectorizable(out, 1);
    switch (x_dt) {
      case kF32: CF_LAUNCH((quantize_rows_kernel<kF32>), grid, dim3(256), 0, stream, x, scales, s_stride, out, xv, ov); break;
      case kF16: CF_LAUNCH((quantize_rows_kernel<kF16>), grid, dim3(256), 0, stream, x, scales, s_stride, out, xv, ov); break;
      case kBF16: CF_LAUNCH((quantize_rows_kernel<kBF16>), grid, dim3(256), 0, stream, x, scales, s_stride, out, xv, ov); break;
      default: set_error("quantize: unsupported dtype %d", x_dt); return CF_ERR_UNSUPPORTED;
    }
    CF_HIP_CHECK(hipGetLastError());
    return CF_OK;
  }
  const dim3 grid(grid_for(n));
  switch (x_dt) {
    case kF32: CF_LAUNCH((quantize_kernel<kF32>), grid, dim3(256), 0, stream, x, scales, s_stride, out); break;
    case kF16: CF_LAUNCH((quantize_kernel<kF16>), grid, dim3(256), 0, stream, x, scales, s_stride, out); break;
    case kBF16: CF_LAUNCH((quantize_kernel<kBF16>), grid, dim3(256), 0, stream, x, scales, s_stride, out); break;
    default: set_error("quantize: unsupported dtype %d", x_dt); return CF_ERR_UNSUPPORTED;
  }
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

static bool quantize_kv_tiles_ok(const Rank4& k, const Rank4& v, int x_dt, const Rank4& ko, const Rank4& vo) {
  const int eb = x_dt == kF32 ? 4 : 2;
  for (int i = 0; i < 4; ++i)
    if (k.size[i] != v.size[i] || ko.size[i] != k.size[i] || vo.size[i] != k.size[i]) return false;
  const int64_t H = k.size[2], D = k.size[3];
  if (k.size[0] < 1 || k.size[1] != 16 || H < 1 || H > kSpanMaxHeads || D < 16 || D % 16 != 0) return false;
  if (k.size[0] > INT32_MAX || 16 * H * D > INT32_MAX) return false;
  // K pieces: 16 contiguous elements, 16-byte aligned
  if (k.stride[3] != 1 || ((uintptr_t)k.base & 15)) return false;
  for (int i = 0; i < 3; ++i)
    if ((k.stride[i] * eb) % 16 != 0) return false;
  // outputs: K rows of D bytes, V channel rows of 16 bytes, shared block / head strides
  if (ko.stride[3] != 1 || ko.stride[1] != D || vo.stride[1] != 1 || vo.stride[3] != 16) return false;
  if (ko.stride[0] != vo.stride[0] || ko.stride[2] != vo.stride[2]) return false;
  if (((uintptr_t)ko.base & 15) || ((uintptr_t)vo.base & 15) || ko.stride[0] % 16 || ko.stride[2] % 16) return false;
  return true;
}

int32_t launch_quantize_kv(const Rank4& k, const Rank4& v, int x_dt, const float* ks, int64_t ks_s, const float* vs,
                           int64_t vs_s, const Rank4& ko, const Rank4& vo, hipStream_t stream) {
  if (k.size[0] * k.size[1] * k.size[2] * k.size[3] == 0) return CF_OK;
  if (quantize_kv_tiles_ok(k, v, x_dt, ko, vo)) {
    ProfileScope prof("cf_kv_quantize_fp8", stream);
    const dim3 grid((unsigned)k.size[0]);
    char* kb = (char*)ko.base;
    char* vb = (char*)vo.base;
    switch (x_dt) {
      case kF32: CF_LAUNCH((quantize_kv_tiles_kernel<kF32>), grid, dim3(256), 0, stream, k, v, ks, ks_s, vs, vs_s, kb, vb, ko.stride[0], ko.stride[2]); break;
      case kF16: CF_LAUNCH((quantize_kv_tiles_kernel<kF16>), grid, dim3(256), 0, stream, k, v, ks, ks_s, vs, vs_s, kb, vb, ko.stride[0], ko.stride[2]); break;
      case kBF16: CF_LAUNCH((quantize_kv_tiles_kernel<kBF16>), grid, dim3(256), 0, stream, k, v, ks, ks_s, vs, vs_s, kb, vb, ko.stride[0], ko.stride[2]); break;
      default: set_error("quantize_kv: unsupported dtype %d", x_dt); return CF_ERR_UNSUPPORTED;
    }
    CF_HIP_CHECK(hipGetLastError());
    return CF_OK;
  }
  int32_t rc = launch_quantize(k, x_dt, ks, ks_s, ko, stream);
  if (rc != CF_OK) return rc;
  return launch_quantize(v, x_dt, vs, vs_s, vo, stream);
}

int32_t launch_dequantize(const Rank4& q, const float* scales, int64_t s_stride, const Rank4& out,
                          hipStream_t stream) {
  const int64_t n = q.size[0] * q.size[1] * q.size[2] * q.size[3];
  if (n == 0) return CF_OK;
  ProfileScope prof("cf_fp8_dequantize", stream);
  if (q.size[3] % 16 == 0) {
    CF_LAUNCH(dequantize_rows_kernel, dim3(grid_for(n / 16)), dim3(256), 0, stream, q, scales, s_stride, out,
                       rows_vectorizable(q, 1), rows_vectorizable(out, 4));
    CF_HIP_CHECK(hipGetLastError());
    return CF_OK;
  }
  CF_LAUNCH(dequantize_kernel, dim3(grid_for(n)), dim3(256), 0, stream, q, scales, s_stride, out);
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

int32_t launch_kv_write_fp8(const KvWriteParams& p, int x_dt, int slot_dt, hipStream_t stream) {
  if (p.T == 0) return CF_OK;
  if (kv_write_native_ok(p, x_dt)) {
    const uint32_t k_blocks = (uint32_t)ceil_div(p.T * p.H * (p.D / 16), 256);
    const uint32_t v_chunks = (uint32_t)ceil_div((int64_t)p.H * p.D, 256);
    const int64_t blocks = k_blocks + ceil_div(p.T, 16) * v_chunks;
    CF_CHECK(blocks < (int64_t)INT32_MAX, "kv_write: too many rows");
    const dim3 grid((unsigned)blocks);
    ProfileScope prof("cf_kv_write_fp8", stream);
#define CF_KVN(XT, ST) \
  CF_LAUNCH((kv_write_native_kernel<XT, ST>), grid, dim3(256), 0, stream, p, k_blocks, v_chunks)
    switch (x_dt * 8 + (slot_dt == kI64 ? 1 : 0)) {
      case kF32 * 8: CF_KVN(kF32, kI32); break;
      case kF32 * 8 + 1: CF_KVN(kF32, kI64); break;
      case kF16 * 8: CF_KVN(kF16, kI32); break;
      case kF16 * 8 + 1: CF_KVN(kF16, kI64); break;
      case kBF16 * 8: CF_KVN(kBF16, kI32); break;
      case kBF16 * 8 + 1: CF_KVN(kBF16, kI64); break;
      default: set_error("kv_write: unsupported dtype %d", x_dt); return CF_ERR_UNSUPPORTED;
    }
#undef CF_KVN
    CF_HIP_CHECK(hipGetLastError());
    return CF_OK;
  }
  const dim3 grid((unsigned)p.T);
  const int threads = p.H * p.D >= 256 ? 256 : 64 * (int)ceil_div(p.H * p.D, 64);
  ProfileScope prof("cf_kv_write_fp8", stream);
#define CF_KVW(XT, ST) CF_LAUNCH((kv_write_kernel<XT, ST>), grid, dim3(threads), 0, stream, p)
  if (slot_dt == kI64) {
    switch (x_dt) {
      case kF32: CF_KVW(kF32, kI64); break;
      case kF16: CF_KVW(kF16, kI64); break;
      case kBF16: CF_KVW(kBF16, kI64); break;
      default: set_error("kv_write: unsupported dtype %d", x_dt); return CF_ERR_UNSUPPORTED;
    }
  } else {
    switch (x_dt) {
      case kF32: CF_KVW(kF32, kI32); break;
      case kF16: CF_KVW(kF16, kI32); break;
      case kBF16: CF_KVW(kBF16, kI32); break;
      default: set_error("kv_write: unsupported dtype %d", x_dt); return CF_ERR_UNSUPPORTED;
    }
  }
#undef CF_KVW
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

}  // namespace cf
