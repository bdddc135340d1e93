// Chunked prefill over the paged KV cache (bf16 / e4m3fn, native layout).
//
// A chunk of L new query rows whose sequence now holds S tokens (its own
// K/V already written to the cache) puts row i at position S - L + i; the
// row attends to cache positions [0, S - L + i] (causal inside the chunk,
// everything before it).  This is the reference's decode semantics
// (kernels/paged_attention.py:21-73) applied per row with the length cut
// to the row's position, the rule the reference's chunked prefill
// (runtime/src/engine/scheduler.rs:178-226) implies.
//
// Shape of the work.  The 16 columns of an MFMA tile hold query columns
// (row, query head): 16/G rows x the G query heads of one KV head.  A wave
// carries NCT = 4 such column tiles (a "query block" of QB = 64/G rows), so
// every 32-token K/V tile it loads and converts feeds 4 x 16 MFMAs.  Each
// (query block, KV head) is one run over the tiles up to its last row's
// position; runs are laid out in a tile stream (KV head, query block, tile)
// and split evenly over the resident waves exactly like the decode kernel
// (decode_mfma.hip), with (m, l, o) partials for runs split between waves,
// merged by prefill_merge_kernel.
#include "cf_device.hpp"
#include "cf_host.hpp"
#include "mfma_tile.hpp"
#include "prefill_params.hpp"

namespace cf {

namespace {

constexpr int kNCT = 4;  // column tiles per wave

// ---- plan: one wave lists the query blocks and their tile offsets ---------
// Chunks are taken in order and made disjoint: chunk n covers q rows
// [max(q_start[n], end of chunk n-1), max(q_start[n+1], that)), clamped to
// [0, Tq).  Its rows sit at positions seq_lens[n] - L + i.
__device__ __forceinline__ int block_kvlen(int pos0, int qb, int QB, int rows, int cap) {
  return max(0, min(pos0 + qb * QB + rows, cap));
}

__global__ __launch_bounds__(64) void prefill_plan_kernel(PrefillParams p) {
  const int lane = threadIdx.x;
  const int cap = p.Mb * 16;
  int vbase = 0, tbase = 0, rend = 0;
  for (int n0 = 0; n0 < p.N; n0 += 64) {
    const int n = n0 + lane;
    int a = 0, b = 0, S = 0;
    if (n < p.N) {
      a = min(max(p.q_start[(int64_t)n * p.qs_s], 0), p.Tq);
      b = min(max(p.q_start[(int64_t)(n + 1) * p.qs_s], 0), p.Tq);
      S = p.seq_lens[(int64_t)n * p.sl_s];
    }
    const int row1 = max(wave_incl_max(max(a, b), lane), rend);
    int prev_end = __shfl_up(row1, 1, 64);
    if (lane == 0) prev_end = rend;
    const int row0 = n < p.N ? max(a, prev_end) : row1;
    const int L = n < p.N ? row1 - row0 : 0;
    const int pos0 = S - L;
    const int nqb = (L + p.QB - 1) / p.QB;
    int ctiles = 0;
    for (int qb = 0; qb < nqb; ++qb) {
      const int rows = min(p.QB, L - qb * p.QB);
      ctiles += (block_kvlen(pos0, qb, p.QB, rows, cap) + 31) >> 5;
    }
    const int incl_v = wave_incl_scan(nqb, lane);
    const int incl_t = wave_incl_scan(ctiles, lane);
    int run = tbase + incl_t - ctiles;
    for (int qb = 0; qb < nqb; ++qb) {
      const int v = vbase + incl_v - nqb + qb;
      const int rows = min(p.QB, L - qb * p.QB);
      const int kvlen = block_kvlen(pos0, qb, p.QB, rows, cap);
      if (v < p.max_v) {
        p.vseq[v] = make_int4(n, row0 + qb * p.QB, rows, pos0 + qb * p.QB);
        p.vtiles[v] = run;
        // query blocks that read nothing get zero rows from the merge kernel
        if (kvlen == 0)
          for (int h = 0; h < p.Hkv; ++h) p.merge_desc[(int64_t)v * p.Hkv + h] = make_int2(-1, 0);
      }
      run += (kvlen + 31) >> 5;
    }
    vbase += __shfl(incl_v, 63, 64);
    tbase += __shfl(incl_t, 63, 64);
    rend = __shfl(row1, 63, 64);
  }
  if (lane == 0) {
    // max_v bounds the block count of disjoint chunks; the check is a guard
    const bool fits = vbase <= p.max_v;
    if (fits) p.vtiles[vbase] = tbase;
    p.header[0] = fits ? vbase : 0;
    p.header[1] = fits ? tbase : 0;
  }
}

struct PIndex {
  const int32_t* __restrict__ tables;
  const int4* __restrict__ vseq;
  const int* __restrict__ vtiles;
  const float* __restrict__ kscale;
  const float* __restrict__ vscale;
};

struct PCoord {
  int h, v, j;
  int n, row0, rows, pos0;  // query block: chunk, first row, rows, position of the first row
  int kvlen, nt;            // cache tokens the block reads, and their tiles
  int blkA, blkB;
};

__device__ __forceinline__ void set_block(const PrefillParams& p, const PIndex& ix, PCoord& c) {
  const int4 e = ix.vseq[c.v];
  c.n = e.x;
  c.row0 = e.y;
  c.rows = e.z;
  c.pos0 = e.w;
  c.kvlen = block_kvlen(c.pos0, 0, 0, c.rows, p.Mb * 16);
  c.nt = (c.kvlen + 31) >> 5;
}

__device__ __forceinline__ int checked_block(const PrefillParams& p, const PIndex& ix, int n, int jb) {
  const int id = ix.tables[(int64_t)n * p.t_sb + (int64_t)jb * p.t_sm];
  return (id >= 0 && id < p.NB) ? id : -1;
}

__device__ __forceinline__ void fetch_ids(const PrefillParams& p, const PIndex& ix, PCoord& c) {
  const int nblk = (c.kvlen + 15) >> 4;
  c.blkA = checked_block(p, ix, c.n, 2 * c.j);
  c.blkB = 2 * c.j + 1 < nblk ? checked_block(p, ix, c.n, 2 * c.j + 1) : -1;
}

__device__ __forceinline__ PCoord advance(const PrefillParams& p, const PIndex& ix, PCoord c, int nv) {
  if (c.j + 1 < c.nt) {
    c.j += 1;
  } else {
    c.j = 0;
    do {
      c.v += 1;
      if (c.v == nv) {
        c.v = 0;
        c.h += 1;
      }
      set_block(p, ix, c);
    } while (c.nt == 0);
  }
  fetch_ids(p, ix, c);
  return c;
}

// Query block v holding tile r (0 <= r < Tb) of a head: largest v with
// vtiles[v] <= r (binary search, wave-uniform).
__device__ __forceinline__ int find_block(const PIndex& ix, int nv, int r) {
  int lo = 0, hi = nv - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (ix.vtiles[mid] <= r) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

template <int D, int G>
__device__ __forceinline__ void load_q_block(bf16x8_t (*qop)[D / 32], const PrefillParams& p, const PCoord& c,
                                             int li, int lq) {
  constexpr int NC = D / 32;
  constexpr int RPT = 16 / G;  // rows per column tile
#pragma unroll
  for (int ct = 0; ct < kNCT; ++ct) {
    const int t = ct * RPT + li / G;
    if (t < c.rows) {
      const uint16_t* qrow = (const uint16_t*)p.q + (int64_t)(c.row0 + t) * p.q_sr +
                             (int64_t)(c.h * G + li % G) * p.q_sh + lq * (D / 4);
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) qop[ct][cc] = as_bf16x8(*(const uint4*)(qrow + 8 * cc));
    } else {
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) qop[ct][cc] = as_bf16x8(make_uint4(0, 0, 0, 0));
    }
  }
}

template <int D>
struct PRun {
  float m[kNCT], l[kNCT];
  f32x4_t o[kNCT][D / 16];
  int j0;
  __device__ __forceinline__ void reset(int j) {
#pragma unroll
    for (int ct = 0; ct < kNCT; ++ct) {
      m[ct] = -INFINITY;
      l[ct] = 0.0f;
#pragma unroll
      for (int t = 0; t < D / 16; ++t) o[ct][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }
    j0 = j;
  }
};

template <int KT, int D, int G>
__device__ __forceinline__ void prefill_tile(PRun<D>& st, TileRegs<KT, D>& r, const PCoord& c,
                                             const bf16x8_t (*qop)[D / 32], float qk_scale, int li, int lq) {
  constexpr int NC = D / 32;
  constexpr int NV = D / 16;
  constexpr int RPT = 16 / G;
  // tokens past the block's cache length may hold any bits: zero their V
  const bool edge = c.kvlen - 32 * c.j < 32 || c.blkA < 0 || c.blkB < 0;
  const bool blk_ok = (lq < 2 ? c.blkA : c.blkB) >= 0;
  const int nvalid = blk_ok ? c.kvlen - 32 * c.j - 8 * lq : 0;  // valid of this lane's 8 tokens
  if (edge) {
#pragma unroll
    for (int t = 0; t < NV; ++t) r.v[t] = mask_tokens(r.v[t], nvalid);
  }
  // operands converted once for all column tiles
  bf16x8_t k1[NC], k2[NC];
#pragma unroll
  for (int cc = 0; cc < NC; ++cc) {
    k1[cc] = k_operand<KT>(r.k1, cc);
    k2[cc] = k_operand<KT>(r.k2, cc);
  }
  using VOp = typename std::conditional<KT == kE4M3, f16x8_t, bf16x8_t>::type;
  VOp vop[NV];
#pragma unroll
  for (int t = 0; t < NV; ++t) {
    if constexpr (KT == kE4M3) vop[t] = e4m3x8_to_f16(r.v[t].x, r.v[t].y);
    else vop[t] = as_bf16x8(r.v[t]);
  }
  const int kp0 = 32 * c.j + 8 * lq;  // cache position of this lane's first token
#pragma unroll
  for (int ct = 0; ct < kNCT; ++ct) {
    f32x4_t s1 = {0.0f, 0.0f, 0.0f, 0.0f}, s2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1[cc], qop[ct][cc], s1, 0, 0, 0);
      s2 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k2[cc], qop[ct][cc], s2, 0, 0, 0);
    }
    float sc[8];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      sc[v] = s1[v] * qk_scale;
      sc[4 + v] = s2[v] * qk_scale;
    }
    // causal: column li's row sits at position qpos; only tiles reaching
    // past the column tile's first row (or the cache end) need masks
    const int qmin = c.pos0 + ct * RPT;
    if (edge || 32 * c.j + 31 > qmin) {
      const int qpos = qmin + li / G;
#pragma unroll
      for (int v = 0; v < 8; ++v)
        if (v >= nvalid || kp0 + v > qpos) sc[v] = -INFINITY;
    }
    float mt = sc[0];
#pragma unroll
    for (int v = 1; v < 8; ++v) mt = fmaxf(mt, sc[v]);
    mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    if (__any(mt > st.m[ct] + 8.0f)) {
      const float mnew = mt > st.m[ct] + 8.0f ? mt : st.m[ct];
      const float alpha = mnew == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(st.m[ct] - mnew);
      st.l[ct] *= alpha;
#pragma unroll
      for (int t = 0; t < NV; ++t) st.o[ct][t] = st.o[ct][t] * alpha;
      st.m[ct] = mnew;
    }
    float pr[8];
    float psum = 0.0f;
    const bool live = st.m[ct] != -INFINITY;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      pr[v] = live ? __builtin_amdgcn_exp2f(sc[v] - st.m[ct]) : 0.0f;
      psum += pr[v];
    }
    st.l[ct] += psum;
    if constexpr (KT == kE4M3) {
      f16x8_t pop;
#pragma unroll
      for (int v = 0; v < 8; ++v) pop[v] = (_Float16)pr[v];
#pragma unroll
      for (int t = 0; t < NV; ++t)
        st.o[ct][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop[t], pop, st.o[ct][t], 0, 0, 0);
    } else {
      bf16x8_t pop, plo;
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const __bf16 hi = (__bf16)pr[v];
        pop[v] = hi;
        plo[v] = (__bf16)(pr[v] - (float)hi);
      }
#pragma unroll
      for (int t = 0; t < NV; ++t) {
        st.o[ct][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop[t], pop, st.o[ct][t], 0, 0, 0);
        st.o[ct][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop[t], plo, st.o[ct][t], 0, 0, 0);
      }
    }
  }
}

template <int D, int G>
__device__ __forceinline__ void prefill_flush(const PrefillParams& p, const PIndex& ix, const PRun<D>& st,
                                              const PCoord& c, int64_t tau, int64_t chunk, int w, bool first_run,
                                              int lane) {
  constexpr int NV = D / 16;
  constexpr int RPT = 16 / G;
  const int li = lane & 15, lq = lane >> 4;
  const float vs = ix.vscale ? ix.vscale[c.h * p.vs_s] : 1.0f;
  const bool complete = st.j0 == 0 && c.j == c.nt - 1;
  if (st.j0 == 0 && lane == 0) {
    int2 desc = make_int2(0, 0);
    if (!complete) {
      const int64_t s_tile = tau - c.j;
      const int w1 = (int)(s_tile / chunk);
      const int w2 = (int)((s_tile + c.nt - 1) / chunk);
      desc = make_int2(w1 * 2 + ((int64_t)w1 * chunk < s_tile ? 1 : 0), w2 - w1 + 1);
    }
    p.merge_desc[(int64_t)c.v * p.Hkv + c.h] = desc;
  }
  const int64_t slot = (int64_t)w * 2 + (first_run ? 0 : 1);
#pragma unroll
  for (int ct = 0; ct < kNCT; ++ct) {
    float lt = st.l[ct] + __shfl_xor(st.l[ct], 16, 64);
    lt += __shfl_xor(lt, 32, 64);
    const int t = ct * RPT + li / G;
    if (complete) {
      if (t < c.rows) {
        const float inv = lt > 0.0f ? vs / lt : 0.0f;
        uint16_t* orow = (uint16_t*)p.out + (int64_t)(c.row0 + t) * p.o_sr + (int64_t)(c.h * G + li % G) * p.o_sh +
                         4 * lq;
#pragma unroll
        for (int tt = 0; tt < NV; ++tt) {
          uint2 packed;
          packed.x = (uint32_t)bf16_bits_from_f32(st.o[ct][tt][0] * inv) |
                     ((uint32_t)bf16_bits_from_f32(st.o[ct][tt][1] * inv) << 16);
          packed.y = (uint32_t)bf16_bits_from_f32(st.o[ct][tt][2] * inv) |
                     ((uint32_t)bf16_bits_from_f32(st.o[ct][tt][3] * inv) << 16);
          *(uint2*)(orow + 16 * tt) = packed;
        }
      }
    } else {
      const int col = ct * 16 + li;
      float* os = p.ws_o + (slot * (16 * kNCT) + col) * D + 4 * lq;
#pragma unroll
      for (int tt = 0; tt < NV; ++tt)
        *(float4*)(os + 16 * tt) = make_float4(st.o[ct][tt][0] * vs, st.o[ct][tt][1] * vs, st.o[ct][tt][2] * vs,
                                               st.o[ct][tt][3] * vs);
      if (lq == 0) {
        p.ws_ml[(slot * (16 * kNCT) + col) * 2] = st.m[ct] == -INFINITY ? -INFINITY : st.m[ct] * (1.0f / kLog2e);
        p.ws_ml[(slot * (16 * kNCT) + col) * 2 + 1] = lt;
      }
    }
  }
}

template <int KT, int D, int G>
__global__ __launch_bounds__(256) void prefill_stream_kernel(PrefillParams p, const int32_t* __restrict__ tables,
                                                             const int4* __restrict__ vseq,
                                                             const int* __restrict__ vtiles,
                                                             const int* __restrict__ header,
                                                             const float* __restrict__ kscale,
                                                             const float* __restrict__ vscale) {
  constexpr int NC = D / 32;
  const PIndex ix{tables, vseq, vtiles, kscale, vscale};
  const int lane = threadIdx.x & 63;
  const int li = lane & 15, lq = lane >> 4;
  const int w = uniform(blockIdx.x * 4 + (threadIdx.x >> 6));
  const int Wtot = gridDim.x * 4;
  const int nv = header[0];
  const int Tb = header[1];
  const int64_t T = (int64_t)p.Hkv * Tb;
  if (T == 0 || nv == 0) return;
  const int64_t chunk = (T + Wtot - 1) / Wtot;
  int64_t tau = (int64_t)w * chunk;
  if (tau >= T) return;
  const int64_t tau_end = tau + chunk < T ? tau + chunk : T;

  PCoord c0;
  c0.h = (int)(tau / Tb);
  {
    const int r = (int)(tau % Tb);
    c0.v = find_block(ix, nv, r);
    c0.j = r - ix.vtiles[c0.v];
  }
  set_block(p, ix, c0);
  fetch_ids(p, ix, c0);
  bool has1 = tau + 1 < tau_end;
  PCoord c1 = has1 ? advance(p, ix, c0, nv) : c0;

  const KvCacheView kv{(const uint8_t*)p.k, (const uint8_t*)p.v, p.k_s[0], p.k_s[2], p.v_s[0], p.v_s[2]};
  TileRegs<KT, D> r0, r1;
  load_tile<KT, D>(r0, kv, c0.blkA, c0.blkB, li, lq, c0.h);
  bf16x8_t qop[kNCT][NC];
  load_q_block<D, G>(qop, p, c0, li, lq);
  float qk_scale = p.scale * (ix.kscale ? ix.kscale[c0.h * p.ks_s] : 1.0f) * kLog2e;
  PRun<D> st;
  st.reset(c0.j);
  bool first_run = true;
  for (;;) {
    load_tile<KT, D>(r1, kv, c1.blkA, c1.blkB, li, lq, c1.h);
    const bool has2 = has1 && tau + 2 < tau_end;
    PCoord c2 = has2 ? advance(p, ix, c1, nv) : c1;
    prefill_tile<KT, D, G>(st, r0, c0, qop, qk_scale, li, lq);
    const bool run_ends = !has1 || c1.v != c0.v || c1.h != c0.h;
    if (run_ends) {
      prefill_flush<D, G>(p, ix, st, c0, tau, chunk, w, first_run, lane);
      first_run = false;
    }
    if (!has1) break;
    c0 = c1;
    c1 = c2;
    has1 = has2;
    r0 = r1;
    ++tau;
    if (run_ends) {
      load_q_block<D, G>(qop, p, c0, li, lq);
      qk_scale = p.scale * (ix.kscale ? ix.kscale[c0.h * p.ks_s] : 1.0f) * kLog2e;
      st.reset(c0.j);
    }
  }
}

// Combines the partials of query blocks split between waves.  One workgroup
// of 256 threads per (KV head, query block).
template <int D, int G>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillParams p, const int* __restrict__ header) {
  constexpr int COLS = 16 * kNCT;
  constexpr int RPT = 16 / G;
  const int v = blockIdx.x, h = blockIdx.y;
  if (v >= header[0]) return;
  const int2 desc = p.merge_desc[(int64_t)v * p.Hkv + h];
  const int nslots = desc.y;
  const int slot_first = desc.x;
  if (nslots == 0 && slot_first >= 0) return;  // written by the stream kernel
  const int w1 = slot_first >> 1;
  const int4 e = p.vseq[v];
  const int row0 = e.y, rows = e.z;
  for (int idx = threadIdx.x; idx < COLS * D; idx += blockDim.x) {
    const int col = idx / D, d = idx % D;
    const int ct = col / 16, li = col % 16;
    const int t = ct * RPT + li / G;
    if (t >= rows) continue;
    float M = -INFINITY;
    for (int k = 0; k < nslots; ++k) {
      const int slot = k == 0 ? slot_first : 2 * (w1 + k);
      M = fmaxf(M, p.ws_ml[((int64_t)slot * COLS + col) * 2]);
    }
    float L = 0.0f, acc = 0.0f;
    if (M != -INFINITY) {
      for (int k = 0; k < nslots; ++k) {
        const int slot = k == 0 ? slot_first : 2 * (w1 + k);
        const float m = p.ws_ml[((int64_t)slot * COLS + col) * 2];
        if (m == -INFINITY) continue;
        const float f = __expf(m - M);
        L += p.ws_ml[((int64_t)slot * COLS + col) * 2 + 1] * f;
        acc += p.ws_o[((int64_t)slot * COLS + col) * D + d] * f;
      }
    }
    uint16_t* orow = (uint16_t*)p.out + (int64_t)(row0 + t) * p.o_sr + (int64_t)(h * G + li % G) * p.o_sh;
    orow[d] = bf16_bits_from_f32(L > 0.0f ? acc / L : 0.0f);
  }
}

int prefill_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  return n;
}

constexpr int kPrefillBlocksPerCU = 1;  // 4-wave workgroups resident per CU

uint64_t pad256(uint64_t x) { return (x + 255) & ~(uint64_t)255; }
uint64_t prefill_waves() { return (uint64_t)prefill_cus() * kPrefillBlocksPerCU * 4; }

template <int KT, int D, int G>
int32_t launch_t(PrefillParams& p, hipStream_t stream) {
  {
    ProfileScope prof("cf_prefill_plan", stream);
    hipLaunchKernelGGL(prefill_plan_kernel, dim3(1), dim3(64), 0, stream, p);
  }
  CF_HIP_CHECK(hipGetLastError());
  const int blocks = prefill_cus() * kPrefillBlocksPerCU;
  {
    ProfileScope prof("cf_prefill_mfma", stream);
    hipLaunchKernelGGL((prefill_stream_kernel<KT, D, G>), dim3(blocks), dim3(256), 0, stream, p, p.tables,
                       (const int4*)p.vseq, (const int*)p.vtiles, (const int*)p.header, p.k_scale, p.v_scale);
  }
  CF_HIP_CHECK(hipGetLastError());
  {
    ProfileScope prof("cf_prefill_merge", stream);
    hipLaunchKernelGGL((prefill_merge_kernel<D, G>), dim3(p.max_v, p.Hkv), dim3(256), 0, stream, p,
                       (const int*)p.header);
  }
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

template <int KT, int D>
int32_t launch_g(PrefillParams& p, hipStream_t stream) {
  switch (p.G) {
    case 1: return launch_t<KT, D, 1>(p, stream);
    case 2: return launch_t<KT, D, 2>(p, stream);
    case 4: return launch_t<KT, D, 4>(p, stream);
    case 8: return launch_t<KT, D, 8>(p, stream);
    case 16: return launch_t<KT, D, 16>(p, stream);
  }
  set_error("prefill: unsupported GQA group %d", p.G);
  return CF_ERR_UNSUPPORTED;
}

}  // namespace

bool prefill_supported(const PrefillParams& p, int q_dt, int kv_dt) {
  if (q_dt != kBF16) return false;
  if (kv_dt != kBF16 && kv_dt != kE4M3) return false;
  if (p.D != 64 && p.D != 128) return false;
  if (p.G != 1 && p.G != 2 && p.G != 4 && p.G != 8 && p.G != 16) return false;
  if (p.NB < 1) return false;
  const int kb = kv_dt == kE4M3 ? 1 : 2;
  if (p.k_s[3] != 1 || p.k_s[1] != p.D || p.v_s[1] != 1 || p.v_s[3] != 16) return false;
  if ((p.k_s[0] * kb) % 16 || (p.k_s[2] * kb) % 16 || (p.v_s[0] * kb) % 16 || (p.v_s[2] * kb) % 16) return false;
  if (((uintptr_t)p.k & 15) || ((uintptr_t)p.v & 15)) return false;
  if (((uintptr_t)p.q & 15) || (p.q_sr * 2) % 16 || (p.q_sh * 2) % 16) return false;
  if (((uintptr_t)p.out & 7) || (p.o_sr * 2) % 8 || (p.o_sh * 2) % 8) return false;
  return true;
}

// Workspace: [vseq int4 x max_v][vtiles int x (max_v + 1)][header 2 int]
//            [o: 2 slots per wave x 16*NCT x D f32][(m, l)][merge descs int2 x max_v x Hkv]
uint64_t prefill_workspace_bytes(int64_t Tq, int64_t N, int64_t Hq, int64_t Hkv, int64_t D) {
  const int64_t G = Hkv > 0 ? Hq / Hkv : 1;
  const int64_t QB = G > 0 ? kNCT * 16 / G : 1;
  const uint64_t max_v = (uint64_t)(Tq / QB + N + 1);
  const uint64_t slots = prefill_waves() * 2;
  return pad256(max_v * 16) + pad256((max_v + 1) * 4) + 256 + pad256(slots * 16 * kNCT * D * 4) +
         pad256(slots * 16 * kNCT * 2 * 4) + pad256(max_v * Hkv * 8);
}

void prefill_bind_workspace(PrefillParams& p, void* workspace) {
  const uint64_t max_v = (uint64_t)p.max_v;
  const uint64_t slots = prefill_waves() * 2;
  char* w = (char*)workspace;
  p.vseq = (int4*)w;
  w += pad256(max_v * 16);
  p.vtiles = (int*)w;
  w += pad256((max_v + 1) * 4);
  p.header = (int*)w;
  w += 256;
  p.ws_o = (float*)w;
  w += pad256(slots * 16 * kNCT * p.D * 4);
  p.ws_ml = (float*)w;
  w += pad256(slots * 16 * kNCT * 2 * 4);
  p.merge_desc = (int2*)w;
}

int prefill_query_block(int G) { return kNCT * 16 / G; }

int32_t launch_prefill(PrefillParams& p, int kv_dt, hipStream_t stream) {
  if (kv_dt == kE4M3) {
    if (p.D == 128) return launch_g<kE4M3, 128>(p, stream);
    if (p.D == 64) return launch_g<kE4M3, 64>(p, stream);
  } else {
    if (p.D == 128) return launch_g<kBF16, 128>(p, stream);
    if (p.D == 64) return launch_g<kBF16, 64>(p, stream);
  }
  set_error("prefill: unsupported head_dim %d", p.D);
  return CF_ERR_UNSUPPORTED;
}

}  // namespace cf
