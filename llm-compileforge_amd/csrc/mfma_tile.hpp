// MFMA tile helpers shared by the paged decode and chunked-prefill kernels
// (gfx950, v_mfma_f32_16x16x32_{bf16,f16}).
//
// A tile is 32 tokens (two 16-token blocks) of one KV head in the native
// layout (K tile [bs][D], V tile [D][bs]).  Lane l (i = l % 16, q = l / 16)
// of a wave loads:
//   K rows of tokens 8*(i/4)%16 + i%4 and that + 4 (A operands of the two
//   S^T = K Q^T chains), channels [q*D/4, (q+1)*D/4);
//   V channel 16t + i, tokens 8q..8q+7 (B operand of O^T = V^T P^T).
// With that assignment the QK output of lane (i, q) holds the scores of
// column i for tokens 8q..8q+7, which is exactly the P^T operand the P.V
// product needs from the same lane: no cross-lane shuffles between the two.
#pragma once

#include <type_traits>

#include "cf_device.hpp"

namespace cf {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

// KV data is read once per call: non-temporal (streaming) loads.
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
template <class T>
__device__ __forceinline__ T stream_load(const void* ptr);
template <>
__device__ __forceinline__ uint4 stream_load<uint4>(const void* ptr) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load((const u32x4_t*)ptr));
}
template <>
__device__ __forceinline__ uint2 stream_load<uint2>(const void* ptr) {
  return __builtin_bit_cast(uint2, __builtin_nontemporal_load((const u32x2_t*)ptr));
}
__device__ __forceinline__ bf16x8_t as_bf16x8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }

// 8 e4m3 codes (two dwords, byte order = element order) -> 8 bf16.
__device__ __forceinline__ bf16x8_t e4m3x8_to_bf16(uint32_t lo, uint32_t hi) {
  uint4 r;
  r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false));
  r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true));
  r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false));
  r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true));
  return as_bf16x8(r);
}

template <int KT>
struct KvTraits;
template <>
struct KvTraits<kE4M3> {
  static constexpr int kBytes = 1;
};
template <>
struct KvTraits<kBF16> {
  static constexpr int kBytes = 2;
};
template <>
struct KvTraits<kF16> {
  static constexpr int kBytes = 2;
};

// Raw per-lane registers of one 32-token tile.  VTOK: V stored token-major
// (the reference's [NB, bs, Hkv, D] order): the tile's 32 V rows are loaded
// as 16-byte row pieces and transposed through LDS before the P.V product.
template <int KT, int D, bool VTOK = false>
struct TileRegs {
  static constexpr int KB = KvTraits<KT>::kBytes;
  static constexpr int KCHUNK = D / 4 * KB / 16;  // uint4 per K row slice
  static constexpr int NV = D / 16;
  uint4 k1[KCHUNK];  // K row slice of token 8*(i/4) + i%4
  uint4 k2[KCHUNK];  // ... and of that token + 4
  // channel-major V: 8 tokens of one channel per PV MFMA (8 bytes e4m3,
  // 16 bytes bf16); token-major V: 16-byte pieces of the 32 x D tile
  using VT = typename std::conditional<KB == 1, uint2, uint4>::type;
  static constexpr int NVR = VTOK ? 32 * D * KB / (64 * 16) : NV;
  using VR = typename std::conditional<VTOK, uint4, VT>::type;
  VR v[NVR];
};

// Loads one 32-token tile (blocks blkA, blkB of KV head h).  K: token rows
// of D elements with unit channel stride, token stride kv.k_tok (D in the
// native / paired layouts, Hkv * D token-major).  V: the native tile
// [D][bs] (channel rows) or, VTOK, token rows at stride kv.v_tok.
// Invalid blocks (id -1) read block 0 instead; their tokens are masked.
struct KvCacheView {
  const uint8_t* k;
  const uint8_t* v;
  int64_t k_blk, k_head, v_blk, v_head;
  int64_t k_tok, v_tok;  // token strides (elements)
};

template <int KT, int D, bool VTOK = false>
__device__ __forceinline__ void load_tile(TileRegs<KT, D, VTOK>& r, const KvCacheView& kv, int blkA, int blkB, int li,
                                          int lq, int h, int lane) {
  constexpr int KB = KvTraits<KT>::kBytes;
  using R = TileRegs<KT, D, VTOK>;
  const int64_t a = blkA < 0 ? 0 : blkA, bb = blkB < 0 ? 0 : blkB;
  const uint8_t* kA = kv.k + (a * kv.k_blk + (int64_t)h * kv.k_head) * KB;
  const uint8_t* kB = kv.k + (bb * kv.k_blk + (int64_t)h * kv.k_head) * KB;
  const uint8_t* vA = kv.v + (a * kv.v_blk + (int64_t)h * kv.v_head) * KB;
  const uint8_t* vB = kv.v + (bb * kv.v_blk + (int64_t)h * kv.v_head) * KB;
  // K: lane (li, lq) reads token koff = 8*(li/4)%16 + li%4 (+4) of block A
  // (li < 8) or B, channels [lq*D/4, (lq+1)*D/4).
  const int koff = (8 * (li >> 2) + (li & 3)) & 15;
  const int64_t ktok = VTOK ? kv.k_tok : D;
  const uint8_t* k1 = (li < 8 ? kA : kB) + (koff * ktok + lq * (D / 4)) * KB;
#pragma unroll
  for (int c = 0; c < R::KCHUNK; ++c) {
    r.k1[c] = stream_load<uint4>(k1 + 16 * c);
    r.k2[c] = stream_load<uint4>(k1 + 4 * ktok * KB + 16 * c);
  }
  if constexpr (VTOK) {
    // row piece i of lane l: token row l / LPR + RPI * i, bytes (l % LPR) * 16
    constexpr int LPR = D * KB / 16, RPI = 64 / LPR;
#pragma unroll
    for (int i = 0; i < R::NVR; ++i) {
      const int row = lane / LPR + RPI * i;
      r.v[i] = stream_load<uint4>((row < 16 ? vA : vB) + ((row & 15) * kv.v_tok) * KB + (lane % LPR) * 16);
    }
  } else {
    // V: lane (li, lq) reads channel 16t + li, tokens 8*(lq%2)..+7 of block A
    // (lq < 2) or B.
    const uint8_t* vp = (lq < 2 ? vA : vB) + (li * 16 + (lq & 1) * 8) * KB;
#pragma unroll
    for (int t = 0; t < R::NV; ++t) r.v[t] = stream_load<typename R::VT>(vp + t * 256 * KB);
  }
}

// Token-major V: the wave's LDS staging area holds the tile's 32 token rows
// of D elements (KB bytes each) at vtok_row_stride bytes apart -- the row
// pieces exactly as loaded -- and the transposing LDS reads return the
// channel-major operand the native layout loads straight from HBM.
//  e4m3 (ds_read_b64_tr_b8): within each group of 16 lanes, lane L receives
//   byte L % 8 of the 8-byte words supplied by lanes 2j + L / 8 (j = 0..7).
//   Lane (li, lq) of PV step t points lanes 2j + b at token 8 lq + j,
//   channels 16 t + 8 b .. + 7, and receives channel 16 t + li of tokens
//   8 lq .. 8 lq + 7.
//  16-bit (ds_read_b64_tr_b16): lane L receives element L % 4 of the 8-byte
//   words (4 elements) supplied by lanes 4j + L / 4 (j = 0..3).  Two reads per
//   operand: for tokens 8 lq + 4 h .. + 3, lane (li, lq) points at token
//   8 lq + 4 h + li / 4, channels 16 t + 4 (li % 4) .. + 3, and receives
//   channel 16 t + li of those four tokens.  Token row q is staged at row
//   vtok_slot(q): the four rows one read takes are then every other row.
// The row stride's 16-byte pad spreads the rows a group reads over the banks
// (a 16-bit row then starts 4 banks after the previous one, so rows two
// apart -- the 32-byte pieces one 16-bit read takes -- are 8 banks apart).
template <int D, int KB = 1>
constexpr int vtok_row_stride() {
  return D * KB + 16;
}
template <int D, int KB = 1>
constexpr int vtok_stage_bytes() {
  return 32 * vtok_row_stride<D, KB>();
}

// Staging row of 16-bit token row q: rows 8 k + 0..3 go to the even rows
// of 8 k .. 8 k + 7, rows 8 k + 4..7 to the odd ones.
__device__ __forceinline__ int vtok_slot(int q) { return (q & ~7) | ((q & 3) << 1) | ((q >> 2) & 1); }

template <int D, int KB = 1>
__device__ __forceinline__ void vtok_stage(uint8_t* stage, const uint4* v, int lane) {
  constexpr int LPR = D * KB / 16, RPI = 64 / LPR, NVR = 32 * D * KB / (64 * 16);
#pragma unroll
  for (int i = 0; i < NVR; ++i) {
    const int q = lane / LPR + RPI * i;
    *(uint4*)(stage + (KB == 2 ? vtok_slot(q) : q) * vtok_row_stride<D, KB>() + (lane % LPR) * 16) = v[i];
  }
}

typedef int v2i32_t __attribute__((ext_vector_type(2)));

template <int D>
__device__ __forceinline__ uint2 vtok_operand(const uint8_t* stage, int t, int li, int lq) {
  const uint8_t* src = stage + (8 * lq + (li >> 1)) * vtok_row_stride<D>() + 16 * t + 8 * (li & 1);
  const v2i32_t r = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
      (__attribute__((address_space(3))) v2i32_t*)((__attribute__((address_space(3))) const uint8_t*)src));
  return make_uint2((uint32_t)r.x, (uint32_t)r.y);
}

typedef short v4i16_t __attribute__((ext_vector_type(4)));

// 16-bit V: channel 16 t + li of tokens 8 lq .. 8 lq + 7 (8 elements), rows
// at vtok_slot.
template <int D>
__device__ __forceinline__ uint4 vtok_operand16(const uint8_t* stage, int t, int li, int lq) {
  constexpr int RS = vtok_row_stride<D, 2>();
  const uint8_t* src = stage + (8 * lq + 2 * (li >> 2)) * RS + 32 * t + 8 * (li & 3);
  const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16_t*)((__attribute__((address_space(3))) const uint8_t*)src));
  const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16_t*)((__attribute__((address_space(3))) const uint8_t*)(src + RS)));
  const uint2 a = __builtin_bit_cast(uint2, lo), b = __builtin_bit_cast(uint2, hi);
  return make_uint4(a.x, a.y, b.x, b.y);
}

// Keeps the first `nbytes` bytes of an 8-byte register pair, zeroing the rest.
__device__ __forceinline__ uint2 keep_bytes(uint2 v, int nbytes) {
  const uint64_t x = ((uint64_t)v.y << 32) | v.x;
  const uint64_t m = nbytes >= 8 ? ~0ull : (nbytes <= 0 ? 0ull : ((1ull << (8 * nbytes)) - 1));
  const uint64_t y = x & m;
  return make_uint2((uint32_t)y, (uint32_t)(y >> 32));
}

// Zeroes the V elements of this lane's tokens >= n_valid (of its 8): cache
// slots past a sequence's end may hold any bit pattern, NaN codes included,
// and 0 * NaN would poison the sum.
__device__ __forceinline__ uint2 mask_tokens(uint2 v, int n_valid) { return keep_bytes(v, n_valid); }
__device__ __forceinline__ uint4 mask_tokens(uint4 v, int n_valid) {
  const uint2 lo = keep_bytes(make_uint2(v.x, v.y), n_valid * 2);
  const uint2 hi = keep_bytes(make_uint2(v.z, v.w), n_valid * 2 - 8);
  return make_uint4(lo.x, lo.y, hi.x, hi.y);
}

template <int KT>
__device__ __forceinline__ bf16x8_t k_operand(const uint4* raw, int c) {
  if constexpr (KT == kE4M3) {
    const uint4 u = raw[c >> 1];
    return (c & 1) ? e4m3x8_to_bf16(u.z, u.w) : e4m3x8_to_bf16(u.x, u.y);
  } else {
    return as_bf16x8(raw[c]);
  }
}

// 8 e4m3 codes -> 8 fp16 (exact: e4m3 values lie inside fp16's range and
// precision).
__device__ __forceinline__ f16x8_t e4m3x8_to_f16(uint32_t lo, uint32_t hi) {
  uint4 r;
  r.x = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, false));
  r.y = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(lo, 1.0f, true));
  r.z = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, false));
  r.w = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(hi, 1.0f, true));
  return __builtin_bit_cast(f16x8_t, r);
}



// Query-typed MFMA operands: bf16 queries multiply bf16 K (bf16 caches, or
// e4m3 converted exactly); fp16 queries multiply fp16 K (fp16 caches, or
// e4m3 converted exactly).
template <int QT>
using QOp = typename std::conditional<QT == kF16, f16x8_t, bf16x8_t>::type;

template <int QT>
__device__ __forceinline__ QOp<QT> as_qop(uint4 u) {
  return __builtin_bit_cast(QOp<QT>, u);
}

template <int QT, int KT>
__device__ __forceinline__ QOp<QT> k_operand_q(const uint4* raw, int c) {
  if constexpr (QT == kF16) {
    if constexpr (KT == kE4M3) {
      const uint4 u = raw[c >> 1];
      return (c & 1) ? e4m3x8_to_f16(u.z, u.w) : e4m3x8_to_f16(u.x, u.y);
    } else {
      return __builtin_bit_cast(f16x8_t, raw[c]);
    }
  } else {
    return k_operand<KT>(raw, c);
  }
}

__device__ __forceinline__ f32x4_t mfma16(bf16x8_t a, bf16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4_t mfma16(f16x8_t a, f16x8_t b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// fp32 -> the output's 16-bit code (round to nearest even).
template <int QT>
__device__ __forceinline__ uint16_t out_bits(float x) {
  if constexpr (QT == kF16) return __builtin_bit_cast(uint16_t, (_Float16)x);
  else return bf16_bits_from_f32(x);
}

__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  return v;
}

__device__ __forceinline__ int wave_incl_max(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(v, o, 64);
    if (lane >= o) v = max(v, u);
  }
  return v;
}

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

}  // namespace
}  // namespace cf
