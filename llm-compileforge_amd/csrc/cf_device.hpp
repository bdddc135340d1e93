// Device-side scalar helpers shared by the cf_hip kernels (gfx950).
//
// Number formats:
//   - OCP FP8 E4M3 "fn" (bias 7, no infinities, S.1111.111 is NaN, max 448).
//     Encoding follows the OCP 8-bit floating point specification (v1.0)
//     with round-to-nearest-even, and matches torch's float8_e4m3fn cast,
//     which the reference uses (compiler/quantize/fp8_kv_cache.py:89):
//     magnitudes >= 480 (and the round-up band (464, 480)) give the NaN code
//     0x7F, not a saturated 448.
//   - bfloat16 with round-to-nearest-even and quiet-NaN 0x7FC0, as torch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cf {

__device__ __forceinline__ uint32_t f2u(float f) { return __float_as_uint(f); }
__device__ __forceinline__ float u2f(uint32_t u) { return __uint_as_float(u); }

// fp32 -> OCP e4m3fn code, round-to-nearest-even.
__device__ __forceinline__ uint8_t e4m3_from_f32(float f) {
  const uint32_t bits = f2u(f);
  const uint32_t sign = bits & 0x80000000u;
  const uint32_t mag = bits ^ sign;
  uint32_t code;
  if (mag >= 0x43F00000u) {
    // |f| >= 480, +-inf and NaN all map to the NaN code.
    code = 0x7Fu;
  } else if (mag < 0x3C800000u) {
    // |f| < 2^-6: subnormal range, quantum 2^-9.  |f| * 512 is exact
    // (power-of-two scaling of a value far from overflow); rint is RNE.
    code = (uint32_t)__builtin_rintf(u2f(mag) * 512.0f);
  } else {
    // Normal range: keep 3 mantissa bits with RNE on the 20 dropped bits,
    // then rebias the exponent from 127 to 7 (120 << 3 in code units).
    // A carry out of the mantissa correctly bumps the exponent; values in
    // (464, 480) round up into the NaN code 0x7F, as the format requires.
    const uint32_t rounded = mag + 0x7FFFFu + ((mag >> 20) & 1u);
    code = (rounded >> 20) - (120u << 3);
  }
  return (uint8_t)(code | (sign >> 24));
}

// e4m3fn(x / scale) with x / scale correctly rounded in fp32 (the
// reference's `(x.float() / scale).to(float8_e4m3fn)`), fast:
//
// 1. The quotient is computed as x * (1 / scale) wherever that provably
//    gives the same code.  q' = fl(x * fl(1/s)) is within 1.5 ulp of the
//    correctly rounded x / s, so both encode to the same code unless they
//    can straddle an RNE decision point.  In the normal range those are the
//    midpoints between codes, whose 20 dropped mantissa bits are exactly
//    0x80000 (no midpoint lies near a binade edge); a q' within 8 ulp of one
//    is recomputed with the IEEE division.  So are the subnormal range
//    (|q'| < 2^-6, where the decision points sit elsewhere in the bits; a
//    small share of real data, handled off the common path), NaNs, and
//    every element when the scale is not a positive normal number with a
//    normal reciprocal.
// 2. The encode uses gfx950's v_cvt_pk_fp8_f32 (RNE, OCP e4m3), which
//    matches the format-defined encoder (e4m3_from_f32 above) on all 2^32
//    fp32 inputs except NaNs of positive sign, which it encodes as 0xFF
//    instead of 0x7F -- those never reach it (step 1 sends them to
//    e4m3_from_f32).  The library's exhaustive device tests pin both.
struct Fp8Quant {
  float s, r;
  bool fast;
  __device__ __forceinline__ explicit Fp8Quant(float scale) : Fp8Quant(scale, 1.0f / scale) {}
  // `recip` must be fl(1 / scale) (computed once per head by the caller).
  __device__ __forceinline__ Fp8Quant(float scale, float recip) : s(scale), r(recip) {
    const uint32_t es = (f2u(scale) >> 23) & 0x1FFu;  // sign + exponent
    const uint32_t er = (f2u(r) >> 23) & 0x1FFu;
    fast = es != 0u && es < 0xFFu && er != 0u && er < 0xFFu;
  }
  // Whether q' = x * r may encode differently from x / s (see above).
  static __device__ __forceinline__ bool needs_division(float q) {
    const uint32_t mag = f2u(q) & 0x7FFFFFFFu;
    return (mag - 0x3C800000u) > (0x7F800000u - 0x3C800000u) || ((mag & 0xFFFFFu) - 0x7FFF8u) < 16u;
  }
  __device__ __forceinline__ uint8_t operator()(float x) const {
    const float q = x * r;
    if (__builtin_expect(!fast || needs_division(q), 0)) return e4m3_from_f32(x / s);
    return (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(q, q, 0, false) & 0xFF);
  }
  // 16 values -> 16 codes, element e in byte e % 4 of word e / 4.
  __device__ __forceinline__ uint4 pack16(const float* f) const {
    uint32_t w[4];
    uint32_t redo = 0u;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float q[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        q[j] = f[4 * g + j] * r;
        redo |= (uint32_t)needs_division(q[j]) << (4 * g + j);
      }
      int v = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
      v = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], v, true);
      w[g] = (uint32_t)v;
    }
    if (!fast) redo = 0xFFFFu;
    if (__builtin_expect(redo != 0u, 0)) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        if ((redo >> e) & 1u) {
          const uint32_t c = e4m3_from_f32(f[e] / s);
          const int sh = 8 * (e & 3);
          w[e >> 2] = (w[e >> 2] & ~(0xFFu << sh)) | (c << sh);
        }
      }
    }
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};

// OCP e4m3fn code -> fp32 (exact).
__device__ __forceinline__ float f32_from_e4m3(uint32_t c) {
  const uint32_t sign = (c & 0x80u) << 24;
  const uint32_t e = (c >> 3) & 0xFu;
  const uint32_t m = c & 0x7u;
  uint32_t mag;
  if (e == 0) {
    // m * 2^-9, exact in fp32.
    mag = f2u((float)m * 0.001953125f);
  } else if (e == 15 && m == 7) {
    mag = 0x7FC00000u;
  } else {
    mag = ((e + 120u) << 23) | (m << 20);
  }
  return u2f(sign | mag);
}

// bf16 <-> fp32
__device__ __forceinline__ float f32_from_bf16_bits(uint32_t h) { return u2f(h << 16); }

__device__ __forceinline__ uint16_t bf16_bits_from_f32(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Element access by dtype code (CfDtype numbering).
enum : int { kF32 = 0, kF16 = 1, kBF16 = 2, kI64 = 3, kI32 = 4, kE4M3 = 7 };

template <int DT> struct Elem;
template <> struct Elem<kF32> {
  using T = float;
  static __device__ __forceinline__ float load(const T* p) { return *p; }
  static __device__ __forceinline__ void store(T* p, float v) { *p = v; }
};
template <> struct Elem<kF16> {
  using T = _Float16;
  static __device__ __forceinline__ float load(const T* p) { return (float)*p; }
  static __device__ __forceinline__ void store(T* p, float v) { *p = (_Float16)v; }
};
template <> struct Elem<kBF16> {
  using T = uint16_t;
  static __device__ __forceinline__ float load(const T* p) { return f32_from_bf16_bits(*p); }
  static __device__ __forceinline__ void store(T* p, float v) { *p = bf16_bits_from_f32(v); }
};
template <> struct Elem<kE4M3> {
  using T = uint8_t;
  static __device__ __forceinline__ float load(const T* p) { return f32_from_e4m3(*p); }
  static __device__ __forceinline__ void store(T* p, float v) { *p = e4m3_from_f32(v); }
};

// 16 consecutive elements of dtype code XT (16-byte aligned) as floats.
template <int XT>
__device__ __forceinline__ void load16(const void* src, float* f) {
  const uint4* s = (const uint4*)src;
  if constexpr (XT == kF32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint4 u = s[i];
      f[4 * i] = u2f(u.x);
      f[4 * i + 1] = u2f(u.y);
      f[4 * i + 2] = u2f(u.z);
      f[4 * i + 3] = u2f(u.w);
    }
  } else if constexpr (XT == kE4M3) {
    const uint4 u = s[0];
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 16; ++j) f[j] = f32_from_e4m3((w[j >> 2] >> (8 * (j & 3))) & 0xFFu);
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint4 u = s[i];
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
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

// Wavefront (64-lane) reductions.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ uint32_t wave_umax(uint32_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t w = (uint32_t)__shfl_xor((int)v, o, 64);
    v = v > w ? v : w;
  }
  return v;
}

}  // namespace cf
