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
#include "cf_device.hpp"
#include "cf_host.hpp"
#include "decode_params.hpp"
#include "mfma_tile.hpp"

namespace cf {

namespace {

// ---------------------------------------------------------------------------
// Work split: the "tile stream".
//
// Tiles are 32-token pieces of one sequence for one KV head, ordered
// (KV head, sequence, tile).  With Tb = sum_b ceil(len_b / 32) tiles per head
// and T = Hkv * Tb in all, wave w of the Wtot launched waves takes the
// contiguous range [w * chunk, min((w + 1) * chunk, T)), chunk = ceil(T /
// Wtot): every wave gets the same number of tiles whatever the length mix,
// and no workgroup is launched for nothing.  Inside its range a wave keeps
// one online-softmax state per (sequence, KV head) run; a run that covers a
// whole sequence is normalized and written to the output, a run that
// covers part of one (it starts or ends at the wave's range boundary) is
// written as an (m, l, o) partial into the wave's slot 0 (first run) or 1
// (last run); decode_merge_kernel then combines the partials of every split
// (sequence, KV head).  (Merging inside this kernel, by the last wave to
// finish a split sequence, needs an agent-scope release per partial; on
// gfx950 that is an L2 writeback per flush and cost more than the separate
// launch.)
// ---------------------------------------------------------------------------

// Read-only inputs the tile walk indexes with wave-uniform addresses.  Passed
// as separate __restrict__ kernel arguments so the compiler may read them
// through the scalar cache (s_load, counted by lgkmcnt) instead of vector
// loads, whose vmcnt waits would also wait for the K/V prefetch.
struct Index {
  const int32_t* __restrict__ tables;
  const int32_t* __restrict__ lens;
  const float* __restrict__ kscale;
  const float* __restrict__ vscale;
};

__device__ __forceinline__ int eff_len(const DecodeParams& p, const Index& ix, int b) {
  const int ctx = ix.lens[(int64_t)b * p.sl_s];
  const int cap = p.Mb * 16;
  return ctx < 0 ? 0 : (ctx < cap ? ctx : cap);
}

__device__ __forceinline__ int ntiles_of(const DecodeParams& p, const Index& ix, int b) {
  return (eff_len(p, ix, b) + 31) >> 5;
}




// Tiles per KV head (sum over sequences).
__device__ int tiles_per_head(const DecodeParams& p, const Index& ix, int lane) {
  int tb = 0;
  for (int base = 0; base < p.B; base += 64) {
    const int b = base + lane;
    tb += wave_sum_i(b < p.B ? ntiles_of(p, ix, b) : 0);
  }
  return uniform(tb);
}

// Sequence b holding tile r (0 <= r < Tb) of a head and the tiles before it.
__device__ void locate(const DecodeParams& p, const Index& ix, int r, int lane, int* b_out, int* before_out) {
  int running = 0;
  for (int base = 0; base < p.B; base += 64) {
    const int b = base + lane;
    const int n = b < p.B ? ntiles_of(p, ix, b) : 0;
    const int incl = wave_incl_scan(n, lane) + running;
    const unsigned long long hit = __ballot(incl > r);
    if (hit) {
      const int idx = __ffsll((long long)hit) - 1;
      *b_out = uniform(base + idx);
      *before_out = uniform(__shfl(incl - n, idx, 64));
      return;
    }
    running = uniform(__shfl(incl, 63, 64));
  }
  *b_out = p.B;
  *before_out = running;
}

struct Coord {
  int h, b, j;  // KV head, sequence, tile within the sequence
  int len;      // effective length of sequence b
  int nt;       // tiles of sequence b
  int blkA, blkB;  // physical blocks of the tile (-1: none / invalid)
};

__device__ __forceinline__ int checked_block(const DecodeParams& p, const Index& ix, int b, int jb) {
  const int id = ix.tables[(int64_t)b * p.t_sb + (int64_t)jb * p.t_sm];
  return (id >= 0 && id < p.NB) ? id : -1;
}

__device__ __forceinline__ void fetch_ids(const DecodeParams& p, const Index& ix, Coord& c) {
  const int nblk = (c.len + 15) >> 4;
  c.blkA = checked_block(p, ix, c.b, 2 * c.j);
  c.blkB = 2 * c.j + 1 < nblk ? checked_block(p, ix, c.b, 2 * c.j + 1) : -1;
}

// Next tile in stream order (the caller knows one exists).
__device__ __forceinline__ Coord advance(const DecodeParams& p, const Index& ix, Coord c) {
  if (c.j + 1 < c.nt) {
    c.j += 1;
  } else {
    c.j = 0;
    do {
      c.b += 1;
      if (c.b == p.B) {
        c.b = 0;
        c.h += 1;
      }
      c.len = eff_len(p, ix, c.b);
      c.nt = (c.len + 31) >> 5;
    } while (c.nt == 0);
  }
  fetch_ids(p, ix, c);
  return c;
}

template <int D>
__device__ __forceinline__ void load_q(bf16x8_t* qop, const DecodeParams& p, int b, int h, int li, int lq) {
  constexpr int NC = D / 32;
  if (li < p.G) {
    const uint16_t* qrow =
        (const uint16_t*)p.q + (int64_t)b * p.q_sb + (int64_t)(h * p.G + li) * p.q_sh + lq * (D / 4);
#pragma unroll
    for (int c = 0; c < NC; ++c) qop[c] = as_bf16x8(*(const uint4*)(qrow + 8 * c));
  } else {
#pragma unroll
    for (int c = 0; c < NC; ++c) qop[c] = as_bf16x8(make_uint4(0, 0, 0, 0));
  }
}

template <int KT, int D>
__global__ __launch_bounds__(256) void decode_stream_kernel(DecodeParams p, const int32_t* __restrict__ tables,
                                                            const int32_t* __restrict__ lens,
                                                            const float* __restrict__ kscale,
                                                            const float* __restrict__ vscale) {
  const Index ix{tables, lens, kscale, vscale};
  constexpr int NC = D / 32;
  constexpr int NV = D / 16;
  const int lane = threadIdx.x & 63;
  const int li = lane & 15, lq = lane >> 4;
  const int w = uniform(blockIdx.x * 4 + (threadIdx.x >> 6));
  const int Wtot = gridDim.x * 4;
  const int G = p.G;

  // Sequences with no tokens get zero rows (no tile of theirs is ever
  // visited); wave w takes sequences w, w + Wtot, ...
  for (int bz = w; bz < p.B; bz += Wtot) {
    if (eff_len(p, ix, bz) == 0) {
      uint16_t* orow = (uint16_t*)p.out + (int64_t)bz * p.o_sb;
      for (int e = lane; e < p.Hq * D; e += 64) orow[(int64_t)(e / D) * p.o_sh + e % D] = 0;
      for (int hh = lane; hh < p.Hkv; hh += 64) p.merge_desc[(int64_t)bz * p.Hkv + hh] = make_int2(0, 0);
    }
  }
  const int Tb = tiles_per_head(p, ix, lane);
  const int64_t T = (int64_t)p.Hkv * Tb;
  if (T == 0) return;
  const int64_t chunk = (T + Wtot - 1) / Wtot;
  int64_t tau = (int64_t)w * chunk;
  if (tau >= T) return;
  const int64_t tau_end = tau + chunk < T ? tau + chunk : T;

  Coord c0;
  c0.h = uniform((int)(tau / Tb));
  {
    int b, before;
    locate(p, ix, (int)(tau % Tb), lane, &b, &before);
    c0.b = b;
    c0.j = uniform((int)(tau % Tb) - before);
  }
  c0.len = eff_len(p, ix, c0.b);
  c0.nt = (c0.len + 31) >> 5;
  fetch_ids(p, ix, c0);
  Coord c1 = c0;
  bool has1 = tau + 1 < tau_end;
  if (has1) c1 = advance(p, ix, c0);

  const KvCacheView kv{(const uint8_t*)p.k, (const uint8_t*)p.v, p.k_s[0], p.k_s[2], p.v_s[0], p.v_s[2]};
  TileRegs<KT, D> r0, r1;
  load_tile<KT, D>(r0, kv, c0.blkA, c0.blkB, li, lq, c0.h);

  bf16x8_t qop[NC];
  load_q<D>(qop, p, c0.b, c0.h, li, lq);
  float m = -INFINITY, l = 0.0f;
  f32x4_t o[NV];
#pragma unroll
  for (int t = 0; t < NV; ++t) o[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  int run_j0 = c0.j;
  bool first_run = true;

  for (;;) {
    // Always issue the next tile's loads (the last iteration reloads its
    // own tile) so every path has the same number of loads in flight and
    // the compiler's vmcnt waits stay exact.
    load_tile<KT, D>(r1, kv, c1.blkA, c1.blkB, li, lq, c1.h);
    const bool has2 = has1 && tau + 2 < tau_end;
    Coord c2 = c1;
    if (has2) c2 = advance(p, ix, c1);

    // ---- S^T = K Q^T ---------------------------------------------------
    const float ks = ix.kscale ? ix.kscale[c0.h * p.ks_s] : 1.0f;
    const float qk_scale = p.scale * ks * kLog2e;  // scores in log2 units
    f32x4_t s1 = {0.0f, 0.0f, 0.0f, 0.0f}, s2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k_operand<KT>(r0.k1, c), qop[c], s1, 0, 0, 0);
      s2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k_operand<KT>(r0.k2, c), qop[c], s2, 0, 0, 0);
    }
    // lane (li, lq): s1[v] -> token 8lq + v, s2[v] -> token 8lq + 4 + v, head li
    float sc[8];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      sc[v] = s1[v] * qk_scale;
      sc[4 + v] = s2[v] * qk_scale;
    }
    // Tiles at a sequence's end or with an invalid block are the only ones
    // with masked tokens (a wave-uniform condition).
    const bool partial = c0.len - 32 * c0.j < 32 || c0.blkA < 0 || c0.blkB < 0;
    int nvalid = 8;
    if (partial) {
      const bool blk_ok = (lq < 2 ? c0.blkA : c0.blkB) >= 0;
      nvalid = blk_ok ? c0.len - 32 * c0.j - 8 * lq : 0;
#pragma unroll
      for (int v = 0; v < 8; ++v)
        if (v >= nvalid) sc[v] = -INFINITY;
#pragma unroll
      for (int t = 0; t < NV; ++t) r0.v[t] = mask_tokens(r0.v[t], nvalid);
    }
    float mt = sc[0];
#pragma unroll
    for (int v = 1; v < 8; ++v) mt = fmaxf(mt, sc[v]);
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    // Lazy rescaling: the running max moves only when a score exceeds it by
    // more than 8 (log2 units), so p = 2^(s - m) <= 256 -- exact enough in
    // fp16/bf16 operands and fp32 sums -- and the O rescale is skipped on
    // almost every tile.
    if (__any(mt > m + 8.0f)) {
      const float mnew = mt > m + 8.0f ? mt : m;
      const float alpha = mnew == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m - mnew);
      l *= alpha;
#pragma unroll
      for (int t = 0; t < NV; ++t) o[t] = o[t] * alpha;
      m = mnew;
    }
    float pr[8];
    float psum = 0.0f;
    const bool live = m != -INFINITY;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      pr[v] = live ? __builtin_amdgcn_exp2f(sc[v] - m) : 0.0f;
      psum += pr[v];
    }
    l += psum;

    // ---- O^T += V^T P^T --------------------------------------------------
    if constexpr (KT == kE4M3) {
      // e4m3 V converts exactly to fp16; P in fp16 (p <= 256) keeps 11 bits.
      f16x8_t pop;
#pragma unroll
      for (int v = 0; v < 8; ++v) pop[v] = (_Float16)pr[v];
#pragma unroll
      for (int t = 0; t < NV; ++t)
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(e4m3x8_to_f16(r0.v[t].x, r0.v[t].y), pop, o[t], 0, 0, 0);
    } else {
      // bf16 V: P = P_hi + P_lo in bf16 (two MFMAs) keeps ~16 bits.
      bf16x8_t pop, plo;
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const __bf16 hi = (__bf16)pr[v];
        pop[v] = hi;
        plo[v] = (__bf16)(pr[v] - (float)hi);
      }
#pragma unroll
      for (int t = 0; t < NV; ++t) {
        const bf16x8_t vop = as_bf16x8(r0.v[t]);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop, o[t], 0, 0, 0);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, plo, o[t], 0, 0, 0);
      }
    }

    // ---- end of a (sequence, head) run ------------------------------------
    const bool run_ends = !has1 || c1.b != c0.b || c1.h != c0.h;
    if (run_ends) {
      float lt = l + __shfl_xor(l, 16, 64);
      lt += __shfl_xor(lt, 32, 64);
      const float vs = ix.vscale ? ix.vscale[c0.h * p.vs_s] : 1.0f;
      const bool complete = run_j0 == 0 && c0.j == c0.nt - 1;
      if (run_j0 == 0 && lane == 0) {
        // The wave holding a sequence's first tile tells the merge kernel
        // what to do: nothing (complete here) or which slots to combine.
        int2 desc = make_int2(0, 0);
        if (!complete) {
          const int64_t s_tile = tau - c0.j;
          const int w1 = (int)(s_tile / chunk);
          const int w2 = (int)((s_tile + c0.nt - 1) / chunk);
          desc = make_int2(w1 * 2 + ((int64_t)w1 * chunk < s_tile ? 1 : 0), w2 - w1 + 1);
        }
        p.merge_desc[(int64_t)c0.b * p.Hkv + c0.h] = desc;
      }
      if (li < G) {
        if (complete) {
          const float inv = lt > 0.0f ? vs / lt : 0.0f;
          uint16_t* orow = (uint16_t*)p.out + (int64_t)c0.b * p.o_sb + (int64_t)(c0.h * G + li) * p.o_sh + 4 * lq;
#pragma unroll
          for (int t = 0; t < NV; ++t) {
            uint2 packed;
            packed.x = (uint32_t)bf16_bits_from_f32(o[t][0] * inv) | ((uint32_t)bf16_bits_from_f32(o[t][1] * inv) << 16);
            packed.y = (uint32_t)bf16_bits_from_f32(o[t][2] * inv) | ((uint32_t)bf16_bits_from_f32(o[t][3] * inv) << 16);
            *(uint2*)(orow + 16 * t) = packed;
          }
        } else {
          const int64_t slot = (int64_t)w * 2 + (first_run ? 0 : 1);
          float* os = p.ws_o + (slot * G + li) * D + 4 * lq;
#pragma unroll
          for (int t = 0; t < NV; ++t)
            *(float4*)(os + 16 * t) = make_float4(o[t][0] * vs, o[t][1] * vs, o[t][2] * vs, o[t][3] * vs);
          if (lq == 0) {
            p.ws_ml[(slot * G + li) * 2] = m == -INFINITY ? -INFINITY : m * (1.0f / kLog2e);
            p.ws_ml[(slot * G + li) * 2 + 1] = lt;
          }
        }
      }
      first_run = false;
    }
    if (!has1) break;

    c0 = c1;
    c1 = c2;
    has1 = has2;
    r0 = r1;
    ++tau;
    if (run_ends) {
      load_q<D>(qop, p, c0.b, c0.h, li, lq);
      m = -INFINITY;
      l = 0.0f;
#pragma unroll
      for (int t = 0; t < NV; ++t) o[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      run_j0 = c0.j;
    }
  }
}

// Combines the (m, l, o) partials of each (sequence b, KV head h) whose
// tiles were split between waves w1..w2 and writes the normalized rows;
// sequences processed whole by one wave were written by the decode kernel.
// One wave per (h, b).  Wave w1 holds the run in slot 2*w1 + 1 if the run
// was not its first, else 2*w1; later waves in their slot 0.
template <int D, int G>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecodeParams p, const int32_t* __restrict__ lens, int Wtot) {
  constexpr int E = G * D / 64;  // output elements per lane
  __shared__ float wgt[64][G];
  __shared__ float inv_l[G];
  const int h = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x;
  const int2 desc = p.merge_desc[(int64_t)b * p.Hkv + h];
  const int nslots = desc.y;
  if (nslots == 0) return;  // written whole by the decode kernel (or empty)
  const int slot_first = desc.x;
  const int w1 = slot_first >> 1;
  (void)lens;
  (void)Wtot;
  float acc[E];
#pragma unroll
  for (int i = 0; i < E; ++i) acc[i] = 0.0f;
  float Mg[G], Lg[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    Mg[g] = -INFINITY;
    Lg[g] = 0.0f;
  }
  // Slots are taken 64 at a time; the running max per head rescales what
  // earlier rounds accumulated (lane-local sums, merged at the end).
  for (int k0 = 0; k0 < nslots; k0 += 64) {
    const int kn = min(64, nslots - k0);
    const int k = k0 + lane;
    const int slot = k == 0 ? slot_first : 2 * (w1 + k);
    float m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[g] = -INFINITY;
      l[g] = 0.0f;
      if (lane < kn) {
        const float2 ml = *(const float2*)(p.ws_ml + ((int64_t)slot * G + g) * 2);
        m[g] = ml.x;
        l[g] = ml.y;
      }
    }
    float scale_old[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float mnew = fmaxf(Mg[g], wave_max(m[g]));
      scale_old[g] = (mnew == -INFINITY || Mg[g] == -INFINITY) ? (Mg[g] == -INFINITY ? 0.0f : 1.0f)
                                                                 : __expf(Mg[g] - mnew);
      const float wk = (m[g] == -INFINITY) ? 0.0f : __expf(m[g] - mnew);
      Lg[g] = Lg[g] * scale_old[g] + wave_sum(l[g] * wk);
      Mg[g] = mnew;
      if (lane < kn) wgt[lane][g] = wk;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < E; ++i) acc[i] *= scale_old[(lane + 64 * i) / D];
    for (int kk = 0; kk < kn; ++kk) {
      const int sk = (k0 + kk) == 0 ? slot_first : 2 * (w1 + k0 + kk);
      const float* o = p.ws_o + (int64_t)sk * G * D;
#pragma unroll
      for (int i = 0; i < E; ++i) {
        const int idx = lane + 64 * i;
        acc[i] += wgt[kk][idx / D] * o[idx];
      }
    }
    __syncthreads();
  }
  if (lane < G) {
    float lg = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g)
      if (g == lane) lg = Lg[g];
    inv_l[lane] = lg > 0.0f ? 1.0f / lg : 0.0f;
  }
  __syncthreads();
  uint16_t* out = (uint16_t*)p.out + (int64_t)b * p.o_sb;
#pragma unroll
  for (int i = 0; i < E; ++i) {
    const int idx = lane + 64 * i;
    const int g = idx / D, d = idx % D;
    out[(int64_t)(h * G + g) * p.o_sh + d] = bf16_bits_from_f32(acc[i] * inv_l[g]);
  }
}

int cu_count() {
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

// Resident 4-wave workgroups per CU.  One per CU (one wave per SIMD) reads
// the randomly placed KV blocks faster on MI355X than two or three: more
// concurrent streams of 2 KiB chunks cost more than the latency they hide
// (measured: 115.6 us vs 121.1 us vs 125.4 us for 1/2/3 per CU on the
// Llama-3-8B shape).  kMaxStreamBlocksPerCU bounds workspace sizes.
constexpr int kStreamBlocksPerCU = 1;
constexpr int kMaxStreamBlocksPerCU = 4;

template <int KT, int D>
int blocks_per_cu() {
  static int cached = 0;
  if (cached == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_stream_kernel<KT, D>, 256, 0) != hipSuccess || n < 1)
      n = 1;
    cached = n < kStreamBlocksPerCU ? n : kStreamBlocksPerCU;
  }
  return cached;
}

template <int KT, int D>
int32_t launch_stream_t(const DecodeParams& p0, hipStream_t stream) {
  DecodeParams p = p0;
  const int blocks = cu_count() * blocks_per_cu<KT, D>();
  {
    ProfileScope prof("cf_decode_mfma", stream);
    hipLaunchKernelGGL((decode_stream_kernel<KT, D>), dim3(blocks), dim3(256), 0, stream, p, p.tables, p.seq_lens,
                       p.k_scale, p.v_scale);
  }
  CF_HIP_CHECK(hipGetLastError());
  {
    const dim3 grid(p.Hkv, p.B);
    const int Wtot = blocks * 4;
    ProfileScope prof("cf_decode_merge", stream);
    switch (p.G) {
      case 1: hipLaunchKernelGGL((decode_merge_kernel<D, 1>), grid, dim3(64), 0, stream, p, p.seq_lens, Wtot); break;
      case 2: hipLaunchKernelGGL((decode_merge_kernel<D, 2>), grid, dim3(64), 0, stream, p, p.seq_lens, Wtot); break;
      case 4: hipLaunchKernelGGL((decode_merge_kernel<D, 4>), grid, dim3(64), 0, stream, p, p.seq_lens, Wtot); break;
      case 8: hipLaunchKernelGGL((decode_merge_kernel<D, 8>), grid, dim3(64), 0, stream, p, p.seq_lens, Wtot); break;
      case 16: hipLaunchKernelGGL((decode_merge_kernel<D, 16>), grid, dim3(64), 0, stream, p, p.seq_lens, Wtot); break;
      default: set_error("MFMA decode: unsupported GQA group %d", p.G); return CF_ERR_UNSUPPORTED;
    }
  }
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

// Workspace layout: [o partials: 2 slots per wave x G x D f32, 256-byte
// padded] [(m, l): 2 slots per wave x G x 2 f32, padded] [merge descriptors:
// one int2 per (sequence, KV head)].
namespace {
uint64_t stream_waves() { return (uint64_t)cu_count() * kMaxStreamBlocksPerCU * 4; }
uint64_t pad256(uint64_t x) { return (x + 255) & ~(uint64_t)255; }
uint64_t stream_o_bytes(int64_t G, int64_t D) { return pad256(stream_waves() * 2 * G * D * 4); }
uint64_t stream_ml_bytes(int64_t G) { return pad256(stream_waves() * 2 * G * 2 * 4); }
}  // namespace

uint64_t decode_mfma_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim) {
  const int64_t G = num_kv_heads > 0 ? num_q_heads / num_kv_heads : num_q_heads;
  return stream_o_bytes(G, head_dim) + stream_ml_bytes(G) + (uint64_t)batch * num_kv_heads * 8;
}

void decode_mfma_bind_workspace(DecodeParams& p, void* workspace) {
  p.ws_o = (float*)workspace;
  p.ws_ml = (float*)((char*)workspace + stream_o_bytes(p.G, p.D));
  p.merge_desc = (int2*)((char*)workspace + stream_o_bytes(p.G, p.D) + stream_ml_bytes(p.G));
}

bool decode_mfma_supported(const DecodeParams& p, int q_dt, int kv_dt) {
  if (q_dt != kBF16) return false;
  if (kv_dt != kBF16 && kv_dt != kE4M3) return false;
  if (p.bs != 16 || (p.D != 64 && p.D != 128)) return false;
  if (p.G != 1 && p.G != 2 && p.G != 4 && p.G != 8 && p.G != 16) return false;
  if (p.NB < 1) return false;  // invalid block ids are redirected to block 0 (then masked)
  const int kb = kv_dt == kE4M3 ? 1 : 2;
  // Native layout: K tile [bs][D] (token stride D, channel stride 1), V tile
  // [D][bs] (token stride 1, channel stride bs); block/head strides free.
  if (p.k_s[3] != 1 || p.k_s[1] != p.D || p.v_s[1] != 1 || p.v_s[3] != 16) return false;
  for (int i = 0; i < 3; ++i)
    if ((p.k_s[i] * kb) % 16 != 0) return false;
  // V: token stride 1 (channel-major blocks), runs of 8 tokens aligned.
  if (p.v_s[1] != 1) return false;
  if ((p.v_s[0] * kb) % 16 != 0 || (p.v_s[2] * kb) % 16 != 0 || (p.v_s[3] * kb) % 16 != 0) return false;
  if (!aligned16(p.k) || !aligned16(p.v)) return false;
  // q rows: 16-byte aligned slices; out rows: 8-byte aligned groups of 4.
  if (!aligned16(p.q) || (p.q_sb * 2) % 16 != 0 || (p.q_sh * 2) % 16 != 0) return false;
  if (((uintptr_t)p.out & 7) != 0 || (p.o_sb * 2) % 8 != 0 || (p.o_sh * 2) % 8 != 0) return false;
  return true;
}

int32_t launch_decode_mfma(const DecodeParams& p, int q_dt, int kv_dt, hipStream_t stream) {
  (void)q_dt;
  if (kv_dt == kE4M3) {
    if (p.D == 128) return launch_stream_t<kE4M3, 128>(p, stream);
    if (p.D == 64) return launch_stream_t<kE4M3, 64>(p, stream);
  } else {
    if (p.D == 128) return launch_stream_t<kBF16, 128>(p, stream);
    if (p.D == 64) return launch_stream_t<kBF16, 64>(p, stream);
  }
  set_error("MFMA decode: unsupported head_dim %d", p.D);
  return CF_ERR_UNSUPPORTED;
}

}  // namespace cf
