// MFMA paged-decode kernel for bf16 and OCP e4m3fn KV caches (gfx950).
//
// Same semantics as the generic kernel (reference kernels/paged_attention.py
// :21-73): softmax(q.k * scale) . v over a sequence's first
// min(seq_len, Mb*bs) tokens, query head h reading KV head h / G.
//
// Shape of the work
//   One workgroup of NW waves per (partition, KV head, sequence).  A
//   partition is PT tokens (a multiple of 32); each wave takes 32-token
//   tiles (two 16-token blocks) round-robin.  The G query heads that share
//   the KV head are the 16 columns of the MFMA tiles (zero-padded when
//   G < 16), so every K/V byte is read once per workgroup.
//
// Per 32-token tile (v_mfma_f32_16x16x32_bf16, lane l: i = l % 16,
// q = l / 16; an A operand row and a B operand column are indexed by i,
// output rows by 4q + v):
//   S^T = K Q^T   two MFMA chains (rows = tokens), D/32 MFMAs each.  Lane
//                 (i, q) feeds the K row of token 8*(i/4) + i%4 (+4 for the
//                 second chain), channels [q*D/4, (q+1)*D/4); the chains'
//                 outputs land so that lane (i, q) holds the scores of head
//                 i for the 8 consecutive tokens 8q..8q+7.
//   online softmax per head (lane-local, plus a max across the 4 q groups).
//   O^T += V^T P^T  D/16 MFMAs; lane (i, q) feeds channel 16t + i of V for
//                 tokens 8q..8q+7 -- 8 consecutive tokens of one channel,
//                 which the native V layout ([NB, Hkv, D, bs]) stores
//                 contiguously -- and its own 8 probabilities as P^T.  The
//                 output holds O[head i][16t + 4q + v], so the softmax
//                 rescale stays lane-local.
// e4m3 codes convert to bf16 exactly (v_cvt_scalef32_pk_bf16_fp8 with scale
// 1.0); the per-KV-head dequant scales factor out of both products.
// Workgroups combine their waves through LDS and write either the final
// output (one partition) or (m, l, o) partials for decode_reduce.
#include <type_traits>

#include "cf_device.hpp"
#include "cf_host.hpp"
#include "decode_params.hpp"

namespace cf {

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

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

// Raw per-lane registers of one 32-token tile.
template <int KT, int D>
struct TileRegs {
  static constexpr int KB = KvTraits<KT>::kBytes;
  static constexpr int KCHUNK = D / 4 * KB / 16;  // uint4 per K row slice
  static constexpr int NV = D / 16;
  uint4 k1[KCHUNK];  // K row slice of token 8*(i/4) + i%4
  uint4 k2[KCHUNK];  // ... and of that token + 4
  // V: 8 tokens of one channel per PV MFMA (8 bytes e4m3, 16 bytes bf16)
  using VT = typename std::conditional<KB == 1, uint2, uint4>::type;
  VT v[NV];
};

template <int KT, int D>
__device__ __forceinline__ void load_tile(TileRegs<KT, D>& r, const DecodeParams& p, const uint8_t* kbase,
                                          const uint8_t* vbase, int blkA, int blkB, int li, int lq, int h) {
  constexpr int KB = KvTraits<KT>::kBytes;
  using R = TileRegs<KT, D>;
  const int tok1 = 8 * (li >> 2) + (li & 3);  // 0..27 within the tile; tok2 = tok1 + 4
  // Invalid blocks (id -1) read block 0 instead; their tokens are masked.
  const int kblk = max(tok1 < 16 ? blkA : blkB, 0);
  const int koff = tok1 & 15;
  const uint8_t* k1 = kbase + ((int64_t)kblk * p.k_s[0] + (int64_t)koff * p.k_s[1] + (int64_t)h * p.k_s[2] +
                               (int64_t)lq * (D / 4)) * KB;
  const uint8_t* k2 = k1 + (int64_t)4 * p.k_s[1] * KB;
#pragma unroll
  for (int c = 0; c < R::KCHUNK; ++c) {
    r.k1[c] = *(const uint4*)(k1 + 16 * c);
    r.k2[c] = *(const uint4*)(k2 + 16 * c);
  }
  const int vblk = max(lq < 2 ? blkA : blkB, 0);
  const uint8_t* vp = vbase + ((int64_t)vblk * p.v_s[0] + (int64_t)(lq & 1) * 8 + (int64_t)h * p.v_s[2] +
                               (int64_t)li * p.v_s[3]) * KB;
  const int64_t vstep = (int64_t)16 * p.v_s[3] * KB;
#pragma unroll
  for (int t = 0; t < R::NV; ++t) r.v[t] = *(const typename R::VT*)(vp + t * vstep);
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

__device__ __forceinline__ bf16x8_t v_operand(uint2 raw) { return e4m3x8_to_bf16(raw.x, raw.y); }
__device__ __forceinline__ bf16x8_t v_operand(uint4 raw) { return as_bf16x8(raw); }

template <int KT, int D, int NW, bool DIRECT>
__global__ __launch_bounds__(NW * 64) void decode_mfma_kernel(DecodeParams p) {
  constexpr int NC = D / 32;  // QK MFMAs per 16-token chain
  constexpr int NV = D / 16;  // PV MFMAs per tile
  extern __shared__ float smem[];
  const int part = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lq = lane >> 4;
  const int G = p.G;

  int ctx = p.seq_lens[(int64_t)b * p.sl_s];
  ctx = min(ctx, p.Mb * 16);
  const int start = part * p.PT;
  if (start >= ctx) {
    if (DIRECT && ctx <= 0) {
      for (int i = tid; i < G * D; i += NW * 64) {
        const int g = i / D, d = i % D;
        Elem<kBF16>::store((uint16_t*)p.out + (int64_t)b * p.o_sb + (int64_t)(h * G + g) * p.o_sh + d, 0.0f);
      }
    }
    return;
  }
  const int count = min(p.PT, ctx - start);
  const int nblk = (count + 15) >> 4;
  const int ntiles = (count + 31) >> 5;

  int* sblk = (int*)smem;                            // [PT / 16], padded to 4
  float* sm = smem + ((p.PT / 16 + 3) & ~3);         // [NW][16]
  float* sl = sm + NW * 16;                          // [NW][16]
  float* so = sl + NW * 16;                          // [NW][G][D]
  const int blk0 = start >> 4;
  for (int i = tid; i < nblk; i += NW * 64) {
    const int id = p.tables[(int64_t)b * p.t_sb + (int64_t)(blk0 + i) * p.t_sm];
    sblk[i] = (id >= 0 && id < p.NB) ? id : -1;
  }

  // Q^T operand: column i = query head h*G + i, channels [lq*D/4, (lq+1)*D/4).
  bf16x8_t qop[NC];
  if (li < G) {
    const uint16_t* qrow = (const uint16_t*)p.q + (int64_t)b * p.q_sb + (int64_t)(h * G + li) * p.q_sh + lq * (D / 4);
#pragma unroll
    for (int c = 0; c < NC; ++c) qop[c] = as_bf16x8(*(const uint4*)(qrow + 8 * c));
  } else {
#pragma unroll
    for (int c = 0; c < NC; ++c) qop[c] = as_bf16x8(make_uint4(0, 0, 0, 0));
  }
  __syncthreads();

  const float ks = p.k_scale ? p.k_scale[h * p.ks_s] : 1.0f;
  const float vs = p.v_scale ? p.v_scale[h * p.vs_s] : 1.0f;
  const float qk_scale = p.scale * ks * kLog2e;  // scores in log2 units
  const uint8_t* kbase = (const uint8_t*)p.k;
  const uint8_t* vbase = (const uint8_t*)p.v;

  float m = -INFINITY;  // running max of head li (same in all 4 q groups)
  float l = 0.0f;       // this lane's share of the running sum
  f32x4_t o[NV];
#pragma unroll
  for (int t = 0; t < NV; ++t) o[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  TileRegs<KT, D> cur, nxt;
  int tile = wave;
  if (tile < ntiles) {
    const int j = 2 * tile;
    load_tile<KT, D>(cur, p, kbase, vbase, sblk[j], j + 1 < nblk ? sblk[j + 1] : -1, li, lq, h);
  }
  for (; tile < ntiles; tile += NW) {
    const int ntile = tile + NW;
    if (ntile < ntiles) {
      const int j = 2 * ntile;
      load_tile<KT, D>(nxt, p, kbase, vbase, sblk[j], j + 1 < nblk ? sblk[j + 1] : -1, li, lq, h);
    }
    const int t0 = tile * 32;
    // ---- S^T = K Q^T -------------------------------------------------
    f32x4_t s1 = {0.0f, 0.0f, 0.0f, 0.0f}, s2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k_operand<KT>(cur.k1, c), qop[c], s1, 0, 0, 0);
      s2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k_operand<KT>(cur.k2, c), qop[c], s2, 0, 0, 0);
    }
    // lane (li, lq): s1[v] -> token 8lq + v, s2[v] -> token 8lq + 4 + v, head li
    const int nvalid = count - t0 - 8 * lq;  // valid tokens among this lane's 8
    const int blkmine = sblk[2 * tile + (lq >> 1)];
    const bool lane_blk_ok = (2 * tile + (lq >> 1) < nblk) && blkmine >= 0;
    float s[8];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      s[v] = (lane_blk_ok && v < nvalid) ? s1[v] * qk_scale : -INFINITY;
      s[4 + v] = (lane_blk_ok && 4 + v < nvalid) ? s2[v] * qk_scale : -INFINITY;
    }
    float mt = s[0];
#pragma unroll
    for (int v = 1; v < 8; ++v) mt = fmaxf(mt, s[v]);
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mnew = fmaxf(m, mt);
    const bool live = mnew != -INFINITY;
    const float alpha = live ? __builtin_amdgcn_exp2f(m - mnew) : 1.0f;
    float pr[8];
    float psum = 0.0f;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      pr[v] = live ? __builtin_amdgcn_exp2f(s[v] - mnew) : 0.0f;
      psum += pr[v];
    }
    l = l * alpha + psum;
    m = mnew;
    bf16x8_t pop;
#pragma unroll
    for (int v = 0; v < 8; ++v) pop[v] = (__bf16)pr[v];
    // ---- O^T += V^T P^T ------------------------------------------------
    const bool partial = t0 + 32 > count || !lane_blk_ok;
    const int nv_mask = lane_blk_ok ? nvalid : 0;
#pragma unroll
    for (int t = 0; t < NV; ++t) {
      auto raw = partial ? mask_tokens(cur.v[t], nv_mask) : cur.v[t];
      o[t] = o[t] * alpha;
      o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(v_operand(raw), pop, o[t], 0, 0, 0);
    }
    if (ntile < ntiles) cur = nxt;
  }

  // ---- combine the waves ------------------------------------------------
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (lq == 0 && li < G) {
    sm[wave * 16 + li] = m;
    sl[wave * 16 + li] = l;
  }
  if (li < G) {
#pragma unroll
    for (int t = 0; t < NV; ++t) {
      float* dst = so + ((size_t)wave * G + li) * D + 16 * t + 4 * lq;
      *(float4*)dst = make_float4(o[t][0], o[t][1], o[t][2], o[t][3]);
    }
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += NW * 64) {
    const int g = i / D, d = i % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, sm[w * 16 + g]);
    float L = 0.0f, acc = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        const float mw = sm[w * 16 + g];
        if (mw == -INFINITY) continue;
        const float e = __builtin_amdgcn_exp2f(mw - M);
        L += sl[w * 16 + g] * e;
        acc += so[((size_t)w * G + g) * D + d] * e;
      }
    }
    acc *= vs;
    const int hq = h * G + g;
    if (DIRECT) {
      Elem<kBF16>::store((uint16_t*)p.out + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh + d,
                         L > 0.0f ? acc / L : 0.0f);
    } else {
      const int64_t row = ((int64_t)b * p.Hq + hq) * p.max_parts + part;
      p.ws_o[row * D + d] = acc;
      if (d == 0) {
        // partials carry natural-log maxima, like the generic kernel's
        p.ws_ml[row * 2] = M == -INFINITY ? -INFINITY : M * (1.0f / kLog2e);
        p.ws_ml[row * 2 + 1] = L;
      }
    }
  }
}

constexpr int kWaves = 4;

size_t lds_bytes(const DecodeParams& p) {
  return ((size_t)((p.PT / 16 + 3) & ~3) + 2 * kWaves * 16 + (size_t)kWaves * p.G * p.D) * 4;
}

template <int KT, int D>
int32_t launch_t(const DecodeParams& p, hipStream_t stream) {
  const dim3 grid(p.max_parts, p.Hkv, p.B);
  const size_t lds = lds_bytes(p);
  ProfileScope prof("cf_decode_mfma", stream);
  if (p.max_parts == 1)
    hipLaunchKernelGGL((decode_mfma_kernel<KT, D, kWaves, true>), grid, dim3(kWaves * 64), lds, stream, p);
  else
    hipLaunchKernelGGL((decode_mfma_kernel<KT, D, kWaves, false>), grid, dim3(kWaves * 64), lds, stream, p);
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

bool decode_mfma_supported(const DecodeParams& p, int q_dt, int kv_dt) {
  if (q_dt != kBF16) return false;
  if (kv_dt != kBF16 && kv_dt != kE4M3) return false;
  if (p.bs != 16 || (p.D != 64 && p.D != 128) || p.G > 16 || p.PT % 32 != 0) return false;
  if (p.NB < 1) return false;  // invalid block ids are redirected to block 0 (then masked)
  if (lds_bytes(p) > 64 * 1024) return false;
  const int kb = kv_dt == kE4M3 ? 1 : 2;
  // K: channel stride 1, rows 16-byte aligned.
  if (p.k_s[3] != 1) return false;
  for (int i = 0; i < 3; ++i)
    if ((p.k_s[i] * kb) % 16 != 0) return false;
  // V: token stride 1 (channel-major blocks), runs of 8 tokens aligned.
  if (p.v_s[1] != 1) return false;
  if ((p.v_s[0] * kb) % 16 != 0 || (p.v_s[2] * kb) % 16 != 0 || (p.v_s[3] * kb) % 16 != 0) return false;
  if (!aligned16(p.k) || !aligned16(p.v)) return false;
  // q rows: 16-byte aligned slices.
  if (!aligned16(p.q) || (p.q_sb * 2) % 16 != 0 || (p.q_sh * 2) % 16 != 0) return false;
  return true;
}

int32_t launch_decode_mfma(const DecodeParams& p, int q_dt, int kv_dt, hipStream_t stream) {
  (void)q_dt;
  if (kv_dt == kE4M3) {
    if (p.D == 128) return launch_t<kE4M3, 128>(p, stream);
    if (p.D == 64) return launch_t<kE4M3, 64>(p, stream);
  } else {
    if (p.D == 128) return launch_t<kBF16, 128>(p, stream);
    if (p.D == 64) return launch_t<kBF16, 64>(p, stream);
  }
  set_error("MFMA decode: unsupported head_dim %d", p.D);
  return CF_ERR_UNSUPPORTED;
}

}  // namespace cf
