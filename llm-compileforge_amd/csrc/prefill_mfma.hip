// Chunked prefill over the paged KV cache (bf16 queries over bf16 / e4m3fn caches, fp16 queries over
// fp16 / e4m3fn caches; native, paired or token-major).
//
// A chunk of L new query rows whose sequence now holds S tokens (its own
// K/V already written to the cache) puts row i at position S - L + i; the
// row attends to cache positions [0, S - L + i] (causal inside the chunk,
// everything before it), read through the chunk's block table up to
// Mb * 16 tokens.  This is the reference's decode semantics
// (kernels/paged_attention.py:21-73) applied per row with the length cut
// to the row's position, the rule the reference's chunked prefill
// (runtime/src/engine/scheduler.rs:178-226) implies.
//
// Shape of the work.  A work item is (chunk n, KV head h, row block rb):
// RB = 128 / G query rows of chunk n times the G query heads of h, i.e.
// 128 query columns (column c: row c / G, head c % G).  One workgroup of
// four waves takes an item; wave w owns columns [32 w, 32 w + 32) as two
// 16-column tiles of v_mfma_f32_16x16x32_{bf16,f16}.  The item's K/V are
// walked in 32-token tiles (two 16-token blocks).  Each tile is read from
// HBM / L2 once per workgroup, converted (e4m3 K -> bf16, e4m3 V -> fp16,
// both exact) and written to LDS in MFMA operand order: an LDS entry is the
// 16 bytes one lane feeds one MFMA, entries of one MFMA are consecutive, so
// every operand read is a conflict-free ds_read_b128.  Two LDS buffers and
// one register stage: in step j the registers holding tile j + 1 go to the
// free buffer and tile j + 2 starts loading into them, while tile j is
// computed from the other buffer.  Each staging wave reads one block, so
// its load addresses are a scalar block base plus a per-lane offset; the
// row pair index runs fastest, so 8 consecutive threads write 8
// consecutive LDS entries (no bank conflicts).
//
// Per tile and column tile the math is the decode kernel's (decode_mfma.hip):
// S^T = K Q^T as two 16-token MFMA chains, online softmax in log2 units
// with lazy rescaling, O^T += V^T P^T; the K-row order inside the tile
// makes each lane's scores exactly the P^T operand it feeds.  The softmax
// keeps cross-lane work off the common path: the rescale test is lane-local
// (a column's max across its 4 lanes is taken only when some lane passes
// the threshold), and the row sums come out of the MFMA pipe as one more
// PV product against an all-ones V channel instead of per-score adds.
//
// A wave issues in order, one instruction per four cycles at most, so its
// MFMAs overlap VALU work only when the two are interleaved in its own
// instruction stream.  Each step is laid out in phases that give every
// batch of MFMAs independent VALU work (sched_group_barrier pins the
// interleave): column tile 0's QK^T beside the staging conversion, column
// tile 1's QK^T beside column tile 0's max, one lazy-rescale branch for
// both column tiles, then both P.V products beside the exponentials.
//
// Items come from a list the plan kernel sorts longest first (counting
// sort on the tile count), so the persistent workgroups finish together
// without splitting an item: there are no partials and no merge pass.
// The longest items, up to 75 % of the tiles, form eight per-XCD lists
// (list x: sorted positions x, x + 8, ...; with Hkv a multiple of 8 these
// are the items of heads x, x + 8, ..., so all row blocks of a (chunk, KV
// head) read its K/V through one XCD's L2); a workgroup takes from its
// XCD's list, then from one shared queue over the remaining, shorter
// items.  The shared tail keeps the XCDs finishing together: they do not
// run equally fast (on the measured part the odd XCDs took ~6 % longer per
// tile), which fully static per-XCD lists turned into a 10 % longer launch.
#include <type_traits>

#include "cf_device.hpp"
#include "cf_host.hpp"
#include "mfma_tile.hpp"
#include "prefill_params.hpp"

namespace cf {

namespace {

constexpr int kCols = 128;        // query columns per work item
constexpr int kPlanThreads = 1024;
constexpr int kCostBins = 2048;   // tile counts at or above share the last bin
constexpr int kXcds = 8;          // workgroup g runs on XCD g % 8, each with its own L2
constexpr int kAffinePct = 75;    // share of the tiles taken from per-XCD lists

__device__ __forceinline__ float wave_incl_scanf(float v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float u = __shfl_up(v, o, 64);
    if (lane >= o) v += u;
  }
  return v;
}

__device__ __forceinline__ int item_kvlen(int pos0, int rb, int RB, int L, int cap) {
  const int rows = min(RB, L - rb * RB);
  return max(0, min(pos0 + rb * RB + rows, cap));
}

// ---- plan: chunk rows, work items, longest-first order -------------------
// Chunks are taken in order and made disjoint: chunk n covers q rows
// [max(q_start[n], end of chunk n-1), max(q_start[n+1], that)), clamped to
// [0, Tq).  Its rows sit at positions seq_lens[n] - L + i.
__global__ __launch_bounds__(kPlanThreads) void prefill_plan_kernel(PrefillParams p) {
  __shared__ int hist[kCostBins];
  __shared__ int wave_tot[kPlanThreads / 64];
  __shared__ float wave_tiles[kPlanThreads / 64];
  __shared__ int s_aff;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cap = p.Mb * 16;
  if (wave == 0) {
    // chunk rows, and in .w the row blocks of the chunks before this one
    int rend = 0, nrb_run = 0;
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
      const int nrb = (L + p.RB - 1) / p.RB;
      const int incl = wave_incl_scan(nrb, lane) + nrb_run;
      if (n < p.N) p.chunks[n] = make_int4(row0, L, S - L, incl - nrb);
      rend = __shfl(row1, 63, 64);
      nrb_run = __shfl(incl, 63, 64);
    }
    if (lane == 0) wave_tot[0] = nrb_run;
  }
  for (int i = tid; i < kCostBins; i += kPlanThreads) hist[i] = 0;
  if (tid == 0) s_aff = 0x7fffffff;
  __syncthreads();
  const int nblocks = wave_tot[0];  // row blocks of all chunks
  __syncthreads();
  // Row block f (flattened over chunks): its chunk by binary search on .w;
  // items (f, h) for every KV head.  Bin kCostBins-1-tiles puts the longest
  // items first.
  for (int f = tid; f < nblocks; f += kPlanThreads) {
    int lo = 0, hi = p.N - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (p.chunks[mid].w <= f) lo = mid;
      else hi = mid - 1;
    }
    const int4 c = p.chunks[lo];
    const int tiles = (item_kvlen(c.z, f - c.w, p.RB, c.y, cap) + 31) >> 5;
    atomicAdd(&hist[kCostBins - 1 - min(tiles, kCostBins - 1)], p.Hkv);
  }
  __syncthreads();
  // Exclusive scans of the bins (two per thread): the items, and the
  // tiles in them (bin b: kCostBins - 1 - b tiles per item; in float, as
  // only the split point below depends on it).  The longest items, up to
  // the first bin that reaches kAffinePct of all tiles, go to the per-XCD
  // lists.
  const int h0 = hist[2 * tid], h1 = hist[2 * tid + 1];
  const float t0 = (float)h0 * (float)(kCostBins - 1 - 2 * tid), t1 = (float)h1 * (float)(kCostBins - 2 - 2 * tid);
  const int incl = wave_incl_scan(h0 + h1, lane);
  const float tincl = wave_incl_scanf(t0 + t1, lane);
  if (lane == 63) {
    wave_tot[wave] = incl;
    wave_tiles[wave] = tincl;
  }
  __syncthreads();
  int base = 0;
  float tbase = 0.0f, tall = 0.0f;
#pragma unroll
  for (int w = 0; w < kPlanThreads / 64; ++w) {
    if (w < wave) {
      base += wave_tot[w];
      tbase += wave_tiles[w];
    }
    tall += wave_tiles[w];
  }
  const int excl = base + incl - (h0 + h1);
  const int total = base + incl;  // inclusive through this thread's bins
  const float target = tall * (kAffinePct / 100.0f);
  if (h0 > 0 && tbase + tincl - t1 >= target) atomicMin(&s_aff, excl + h0);
  if (h1 > 0 && tbase + tincl >= target) atomicMin(&s_aff, excl + h0 + h1);
  __syncthreads();
  hist[2 * tid] = excl;
  hist[2 * tid + 1] = excl + h0;
  __syncthreads();
  for (int f = tid; f < nblocks; f += kPlanThreads) {
    int lo = 0, hi = p.N - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (p.chunks[mid].w <= f) lo = mid;
      else hi = mid - 1;
    }
    const int4 c = p.chunks[lo];
    const int rb = f - c.w;
    const int tiles = (item_kvlen(c.z, rb, p.RB, c.y, cap) + 31) >> 5;
    const int at = atomicAdd(&hist[kCostBins - 1 - min(tiles, kCostBins - 1)], p.Hkv);
    for (int h = 0; h < p.Hkv; ++h)
      if (at + h < p.max_items) p.items[at + h] = make_int4(lo, rb, h, tiles);
  }
  if (tid == kPlanThreads - 1) {
    const int n_items = min(total, p.max_items);  // the last thread's inclusive sum: all items
    p.header[0] = n_items;
    p.header[1] = 0;                               // shared queue counter
    p.header[2] = min(s_aff, n_items) & ~(kXcds - 1);  // items in the per-XCD lists
  }
  if (tid < kXcds) p.header[3 + tid] = 0;  // per-XCD list counters
}

// ---- the work-item kernel ---------------------------------------------------

template <int KT, int D>
struct Geo {
  static constexpr int KB = KvTraits<KT>::kBytes;
  static constexpr int NC = D / 32;             // QK MFMA steps per chain
  static constexpr int NV = D / 16;             // PV MFMAs per column tile
  static constexpr int KENT = 2 * NC * 64;      // K operand entries (16 B) per tile
  static constexpr int VENT = NV * 64;          // V operand entries per tile
  static constexpr int KUPL = D / 4 * KB / 16;  // 16-byte K loads per (chain, lane)
  static constexpr int KU = 2 * 64 * KUPL;      // K loads per tile
  static constexpr int VPER = KB;               // 16-byte loads per channel row of a block (16 tokens)
  static constexpr int VU = 2 * D * VPER;       // V loads per tile
  static constexpr int KPT = (KU + 255) / 256;  // per thread
  static constexpr int VPT = (VU + 255) / 256;
  // Token-major V (the reference's [NB, bs, Hkv, D] layout): a 16-byte load
  // is VCH channels of one token; the tile is staged as 32 rows of 16-bit
  // values, RS bytes apart at rows vtok_slot (no bank conflicts on the reads), and
  // read back transposed into the operand order.
  static constexpr int VCH = 16 / KB;                  // channels per load
  static constexpr int VCPR = D / VCH;                 // loads per token row
  static constexpr int VRS = vtok_row_stride<D, 2>();  // LDS bytes per staged row
  static constexpr int VENT_TOK = (32 * VRS + 15) / 16;
};

struct TileIds {
  int a, b;  // physical blocks (block 0 stands in for an invalid id)
  int ok;    // bit 0: a valid, bit 1: b valid
};

// Table entries -> ids; anything outside [0, NB) (including the -1 that
// stands for a block past the item) is invalid.
__device__ __forceinline__ TileIds tile_resolve(int ia, int ib, int NB) {
  const bool va = (unsigned)ia < (unsigned)NB, vb = (unsigned)ib < (unsigned)NB;
  TileIds t;
  t.a = va ? ia : 0;
  t.b = vb ? ib : 0;
  t.ok = (va ? 1 : 0) | (vb ? 2 : 0);
  return t;
}

// Block ids of tile j from the item's table row (`trow`, stride t_sm).
__device__ __forceinline__ TileIds tile_ids(const PrefillParams& p, const int32_t* __restrict__ trow, int j,
                                            int kvlen) {
  const int nblk = (kvlen + 15) >> 4;
  const int ia = trow[(int64_t)(2 * j) * p.t_sm];
  const int ib = 2 * j + 1 < nblk ? trow[(int64_t)(2 * j + 1) * p.t_sm] : -1;
  return tile_resolve(ia, ib, p.NB);
}

// K piece u of a tile: 16 bytes of one token row.  X = block of the tile
// (each wave's pieces come from one block, so its load addresses are one
// scalar base plus a per-lane offset), s = chain, cp = 16-byte part of the
// lane's D / 4 channels, (li, lq) = the lane it feeds.  The row pair index
// runs fastest, so 8 consecutive threads write 8 consecutive LDS entries.
struct KPiece {
  int X, s, cp, li, lq, row;
};

template <int KT, int D>
__device__ __forceinline__ KPiece k_piece(int u) {
  using Gm = Geo<KT, D>;
  constexpr int PB = 64 * Gm::KUPL;  // pieces per block
  KPiece q;
  q.X = u / PB;
  const int idx = u % PB;
  const int l8 = idx & 7;
  q.lq = (idx >> 3) & 3;
  const int sc = idx >> 5;  // s * KUPL + cp
  q.cp = sc % Gm::KUPL;
  q.s = sc / Gm::KUPL;
  q.li = l8 + 8 * q.X;
  q.row = (l8 & 3) + 8 * (l8 >> 2) + 4 * q.s;
  return q;
}

// Global loads of one K/V tile into registers (16 bytes each).  K rows are
// token rows of k_s[1] elements' stride (head_dim in the native layout);
// V is the native tile (VTOK false: channel rows of 16 tokens) or
// token-major (a load is one token's VCH channels).
template <int KT, int D, bool VTOK>
__device__ __forceinline__ void stage_load(uint4* kr, uint4* vr, const PrefillParams& p, const TileIds& t, int h,
                                           int tid) {
  using Gm = Geo<KT, D>;
  const uint8_t* kbase = (const uint8_t*)p.k;
  const uint8_t* vbase = (const uint8_t*)p.v;
#pragma unroll
  for (int i = 0; i < Gm::KPT; ++i) {
    const int u = tid + 256 * i;
    if (Gm::KU % 256 == 0 || u < Gm::KU) {
      const KPiece q = k_piece<KT, D>(u);
      const int blk = uniform(q.X) ? t.b : t.a;
      const uint8_t* b = kbase + ((int64_t)blk * p.k_s[0] + (int64_t)h * p.k_s[2]) * Gm::KB;
      const uint32_t off = (uint32_t)((q.row * p.k_s[1] + q.lq * (D / 4)) * Gm::KB + q.cp * 16);
      kr[i] = *(const uint4*)(b + off);
    }
  }
#pragma unroll
  for (int i = 0; i < Gm::VPT; ++i) {
    const int u = tid + 256 * i;
    if (Gm::VU % 256 == 0 || u < Gm::VU) {
      if constexpr (VTOK) {
        // 16 bytes of token r of block X: channels VCH c .. VCH c + VCH - 1
        const int X = u / (16 * Gm::VCPR), r = (u / Gm::VCPR) % 16, c = u % Gm::VCPR;
        const int blk = uniform(X) ? t.b : t.a;
        const uint8_t* b = vbase + ((int64_t)blk * p.v_s[0] + (int64_t)h * p.v_s[2]) * Gm::KB;
        const uint32_t off = (uint32_t)(r * p.v_s[1] * Gm::KB + c * 16);
        vr[i] = *(const uint4*)(b + off);
      } else {
        // 16 bytes of channel d of block X: all 16 tokens (e4m3) or half of them (bf16)
        const int X = u / (D * Gm::VPER), rem = u % (D * Gm::VPER);
        const int d = rem / Gm::VPER, part = rem % Gm::VPER;
        const int blk = uniform(X) ? t.b : t.a;
        const uint8_t* b = vbase + ((int64_t)blk * p.v_s[0] + (int64_t)h * p.v_s[2]) * Gm::KB;
        const uint32_t off = (uint32_t)(d * 16 * Gm::KB + part * 16);
        vr[i] = *(const uint4*)(b + off);
      }
    }
  }
}

// All ones when token r of block X (of a tile whose blocks' validity bits
// are `ok`) is below `valid`, tile-relative, and its block is valid; else 0.
__device__ __forceinline__ uint32_t vtok_keep_mask(int ok, int X, int r, int valid) {
  const uint32_t blk_ok = (uint32_t)(ok >> X) & 1u;
  const uint32_t in_len = (uint32_t)(16 * X + r < valid);
  return 0u - (blk_ok & in_len);
}

// Converts the staged registers and writes them in operand order: K entry
// (chain s, step c, lane) = the 8 channels lane (li, lq) feeds step c of
// chain s; V entry (step t, lane) = channel 16 t + li, tokens 8 lq .. 8 lq + 7.
// V tokens at or past `valid` (tile-relative) or in an invalid block become
// zero (cache slots there may hold any bits, NaN codes included).
// FULL: the caller knows every token of the tile is valid.
template <int QT, int KT, int D, bool VTOK, bool FULL = false>
__device__ __forceinline__ void stage_write(uint4* lds, const uint4* kr, const uint4* vr, const TileIds& t,
                                            int valid, int tid) {
  using Gm = Geo<KT, D>;
#pragma unroll
  for (int i = 0; i < Gm::KPT; ++i) {
    const int u = tid + 256 * i;
    if (Gm::KU % 256 == 0 || u < Gm::KU) {
      const KPiece q = k_piece<KT, D>(u);
      const int s = q.s, cp = q.cp, lane = q.li + 16 * q.lq;
      if constexpr (KT == kE4M3 && QT == kF16) {
        // e4m3 K converts exactly to the fp16 operands fp16 queries multiply
        lds[(s * Gm::NC + 2 * cp) * 64 + lane] = __builtin_bit_cast(uint4, e4m3x8_to_f16(kr[i].x, kr[i].y));
        lds[(s * Gm::NC + 2 * cp + 1) * 64 + lane] = __builtin_bit_cast(uint4, e4m3x8_to_f16(kr[i].z, kr[i].w));
      } else if constexpr (KT == kE4M3) {
        lds[(s * Gm::NC + 2 * cp) * 64 + lane] = __builtin_bit_cast(uint4, e4m3x8_to_bf16(kr[i].x, kr[i].y));
        lds[(s * Gm::NC + 2 * cp + 1) * 64 + lane] = __builtin_bit_cast(uint4, e4m3x8_to_bf16(kr[i].z, kr[i].w));
      } else {
        lds[(s * Gm::NC + cp) * 64 + lane] = kr[i];
      }
    }
  }
  uint4* vl = lds + Gm::KENT;
  // Tiles whose 32 tokens are all valid (all but an item's last tile) skip
  // the masking (a wave-uniform branch).
  const bool full = FULL || (valid >= 32 && t.ok == 3);
  if constexpr (VTOK) {
    // token row 16 X + r of the staged tile, 16-bit, at row vtok_slot of
    // it (the order vtok_operand16 reads); a token past `valid`
    // or in an invalid block is written as zeros.  The keep mask is formed
    // arithmetically: written as a short-circuit select, the ROCm 7.2
    // compiler dropped the keep lanes' copy of the loaded value (bf16,
    // head_dim 64) and wrote zeros.
    uint8_t* rows = (uint8_t*)vl;
#pragma unroll
    for (int i = 0; i < Gm::VPT; ++i) {
      const int u = tid + 256 * i;
      if (Gm::VU % 256 == 0 || u < Gm::VU) {
        const int X = u / (16 * Gm::VCPR), r = (u / Gm::VCPR) % 16, c = u % Gm::VCPR;
        const uint32_t km = full ? ~0u : vtok_keep_mask(t.ok, X, r, valid);
        const uint4 v = make_uint4(vr[i].x & km, vr[i].y & km, vr[i].z & km, vr[i].w & km);
        uint8_t* row = rows + vtok_slot(16 * X + r) * Gm::VRS;
        if constexpr (KT == kE4M3) {
          *(uint4*)(row + 32 * c) = __builtin_bit_cast(uint4, e4m3x8_to_f16(v.x, v.y));
          *(uint4*)(row + 32 * c + 16) = __builtin_bit_cast(uint4, e4m3x8_to_f16(v.z, v.w));
        } else {
          *(uint4*)(row + 16 * c) = v;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < Gm::VPT; ++i) {
    const int u = tid + 256 * i;
    if (Gm::VU % 256 == 0 || u < Gm::VU) {
      const int X = u / (D * Gm::VPER), rem = u % (D * Gm::VPER);
      const int d = rem / Gm::VPER, part = rem % Gm::VPER;
      const bool ok = (t.ok >> X) & 1;
      const int li = d & 15, tt = d >> 4;
      if (full) {
        if constexpr (KT == kE4M3) {
          vl[tt * 64 + 32 * X + li] = __builtin_bit_cast(uint4, e4m3x8_to_f16(vr[i].x, vr[i].y));
          vl[tt * 64 + 32 * X + 16 + li] = __builtin_bit_cast(uint4, e4m3x8_to_f16(vr[i].z, vr[i].w));
        } else {
          vl[tt * 64 + 32 * X + 16 * part + li] = vr[i];
        }
      } else if constexpr (KT == kE4M3) {
        const int n0 = ok ? valid - 16 * X : 0;  // valid tokens among this load's 16
        const uint2 lo = keep_bytes(make_uint2(vr[i].x, vr[i].y), n0);
        const uint2 hi = keep_bytes(make_uint2(vr[i].z, vr[i].w), n0 - 8);
        vl[tt * 64 + 32 * X + li] = __builtin_bit_cast(uint4, e4m3x8_to_f16(lo.x, lo.y));
        vl[tt * 64 + 32 * X + 16 + li] = __builtin_bit_cast(uint4, e4m3x8_to_f16(hi.x, hi.y));
      } else {
        const int n0 = ok ? valid - 16 * X - 8 * part : 0;
        vl[tt * 64 + 32 * X + 16 * part + li] = mask_tokens(vr[i], n0);
      }
    }
  }
}

// Zeroes, in the staged registers, the V tokens at or past `valid`
// (tile-relative) or in an invalid block, so that the tile can then be
// written without masking.
template <int KT, int D, bool VTOK>
__device__ __forceinline__ void mask_staged_v(uint4* vr, const TileIds& t, int valid, int tid) {
  using Gm = Geo<KT, D>;
  if constexpr (VTOK) {
#pragma unroll
    for (int i = 0; i < Gm::VPT; ++i) {
      const int u = tid + 256 * i;
      if (Gm::VU % 256 == 0 || u < Gm::VU) {
        const int X = u / (16 * Gm::VCPR), r = (u / Gm::VCPR) % 16;
        const uint32_t km = vtok_keep_mask(t.ok, X, r, valid);
        vr[i] = make_uint4(vr[i].x & km, vr[i].y & km, vr[i].z & km, vr[i].w & km);
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < Gm::VPT; ++i) {
    const int u = tid + 256 * i;
    if (Gm::VU % 256 == 0 || u < Gm::VU) {
      const int X = u / (D * Gm::VPER), rem = u % (D * Gm::VPER);
      const int part = rem % Gm::VPER;
      const bool ok = (t.ok >> X) & 1;
      if constexpr (KT == kE4M3) {
        const int n0 = ok ? valid - 16 * X : 0;
        const uint2 lo = keep_bytes(make_uint2(vr[i].x, vr[i].y), n0);
        const uint2 hi = keep_bytes(make_uint2(vr[i].z, vr[i].w), n0 - 8);
        vr[i] = make_uint4(lo.x, lo.y, hi.x, hi.y);
      } else {
        vr[i] = mask_tokens(vr[i], ok ? valid - 16 * X - 8 * part : 0);
      }
    }
  }
}

template <int QT, int KT, int D, int G, bool VTOK>
__global__ __launch_bounds__(256, 2) void prefill_item_kernel(PrefillParams p, const int32_t* __restrict__ tables,
                                                              const int4* __restrict__ items,
                                                              const int4* __restrict__ chunks, int* header,
                                                              const float* __restrict__ kscale,
                                                              const float* __restrict__ vscale) {
  using Gm = Geo<KT, D>;
  constexpr int NC = Gm::NC, NV = Gm::NV;
  constexpr int RB = kCols / G;
  __shared__ uint4 lds[2][Gm::KENT + (VTOK ? Gm::VENT_TOK : Gm::VENT)];
  __shared__ int s_item;
  const int xcd = blockIdx.x % kXcds;
  bool own_list = true;  // (thread 0) this XCD's list still has items
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int li = lane & 15, lq = lane >> 4;
  // list x is drained by the workgroups with blockIdx.x % 8 == x (wherever
  // they run), so a grid of fewer than 8 takes every item from the queue
  const int n_items = header[0], n_aff = gridDim.x >= kXcds ? header[2] : 0;
  const int cap = p.Mb * 16;
  // Beside the memory-bound decode kernel (a mixed step's two streams), a
  // SIMD holds one wave of each; the prefill's, on the step's critical path,
  // issues first.  Among the prefill's own waves the priorities are equal.
  __builtin_amdgcn_s_setprio(2);

  for (;;) {
    if (tid == 0) {
      int it = n_items;
      if (own_list) {
        const int pos = kXcds * atomicAdd(&header[3 + xcd], 1) + xcd;
        if (pos < n_aff) it = pos;
        else own_list = false;
      }
      if (!own_list) {
        const int pos = n_aff + atomicAdd(&header[1], 1);
        it = pos < n_items ? pos : n_items;
      }
      s_item = it;
    }
    __syncthreads();
    const int it = uniform(s_item);
    __syncthreads();
    if (it >= n_items) break;
    const int4 item = items[it];
    const int n = uniform(item.x), rb = uniform(item.y), h = uniform(item.z), nt = uniform(item.w);
    const int4 ch = chunks[n];
    const int row0 = uniform(ch.x + rb * RB);
    const int rows = uniform(min(RB, ch.y - rb * RB));
    const int pos0 = uniform(ch.z + rb * RB);
    const int kvlen = uniform(max(0, min(pos0 + rows, cap)));

    // This wave's columns: tile k, column li -> item column 32 wave + 16 k + li.
    QOp<QT> qop[2][NC];
    int lim[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int col = 32 * wave + 16 * k + li;
      const int r = col / G, g = col % G;
      const bool used = r < rows;
      lim[k] = used ? max(0, min(pos0 + r + 1, cap)) : 0;
      const int rr = used ? r : 0;
      const uint16_t* qrow = (const uint16_t*)p.q + (int64_t)(row0 + rr) * p.q_sr +
                             (int64_t)(h * G + g) * p.q_sh + lq * (D / 4);
#pragma unroll
      for (int c = 0; c < NC; ++c) qop[k][c] = as_qop<QT>(*(const uint4*)(qrow + 8 * c));
    }
    // tokens every column of this wave may see
    int lmin = min(lim[0], lim[1]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) lmin = min(lmin, __shfl_xor(lmin, o, 64));
    lmin = uniform(lmin);
    const int lmin_t = lmin >> 5;  // tiles before the first one some column of the wave cannot see whole
    float qk_scale = p.scale * (kscale ? kscale[h * p.ks_s] : 1.0f) * kLog2e;
    if (qk_scale < 0.0f) {
      // the softmax takes its max on raw scores: keep the scale positive by
      // negating q instead (exact: a sign bit flip in bf16 or fp16)
      qk_scale = -qk_scale;
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          uint4 u = __builtin_bit_cast(uint4, qop[k][c]);
          u.x ^= 0x80008000u;
          u.y ^= 0x80008000u;
          u.z ^= 0x80008000u;
          u.w ^= 0x80008000u;
          qop[k][c] = as_qop<QT>(u);
        }
    }
    // A zero scale makes every score 0 (uniform weights over the visible
    // tokens); the smallest normal scale gives the same weights (products
    // ~1e-34, exp2 of which is 1.0f) and keeps -inf * scale = -inf for the
    // masked ones.
    if (qk_scale == 0.0f) qk_scale = 1.17549435e-38f;

    float m[2] = {-INFINITY, -INFINITY};
    f32x4_t o[2][NV];
    // Row sums come from the PV MFMAs: an extra V tile whose channel 0 is all
    // ones gives O[column][0] = sum of P (lane (li, lq = 0), element 0).
    f32x4_t ol[2] = {f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int t = 0; t < NV; ++t) o[k][t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    // K/V registers of the tile in flight and the block ids of tiles j ..
    // j + 3.  At the start of step j, tile j + 1 goes from the registers to
    // the free LDS buffer and tile j + 2 starts loading into the same
    // registers, while tile j is computed from the other buffer.  Past the
    // item's last tile the ids repeat the last valid ones: the extra load
    // reads real blocks and is never used.
    uint4 kr[Gm::KPT], vr[Gm::VPT];
    const int32_t* trow = tables + (int64_t)n * p.t_sb;
    const int nblk = (kvlen + 15) >> 4, nfull = kvlen >> 5;
    const int64_t tsm = p.t_sm;
    const int32_t* tp = trow + 6 * tsm;  // table entry of tile 3's first block, advanced every step
    TileIds id0 = tile_ids(p, trow, 0, kvlen);
    TileIds id1 = nt > 1 ? tile_ids(p, trow, 1, kvlen) : id0;
    TileIds id2 = nt > 2 ? tile_ids(p, trow, 2, kvlen) : id1;
    if (nt > 0) {
      stage_load<KT, D, VTOK>(kr, vr, p, id0, h, tid);
      stage_write<QT, KT, D, VTOK>(lds[0], kr, vr, id0, kvlen, tid);
    }
    if (nt > 1) stage_load<KT, D, VTOK>(kr, vr, p, id1, h, tid);
    __syncthreads();

    // P in fp16 against fp16 V operands (e4m3 V converts exactly; fp16 V as
    // is); against bf16 V as bf16 hi + lo
    using POp = typename std::conditional<KT == kBF16, bf16x8_t, f16x8_t>::type;
    using KOp = QOp<QT>;

    // The tile's math per column tile k, in pieces the step below orders so
    // that each batch of MFMAs has independent VALU work beside it.
    // Scores: lane (li, lq) holds s1[v] -> token tok0 + v, s2[v] -> token
    // tok0 + 4 + v.
    auto qk = [&](auto kc, const KOp* a1, const KOp* a2, f32x4_t& s1, f32x4_t& s2) {
      constexpr int k = decltype(kc)::value;
      s1 = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      s2 = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        s1 = mfma16(a1[c], qop[k][c], s1);
        s2 = mfma16(a2[c], qop[k][c], s2);
      }
    };
    // Scores column tile k may not see (edge tiles only) become -inf, in
    // place.
    auto mask = [&](auto kc, f32x4_t& s1, f32x4_t& s2, int ok, int tok0) {
      constexpr int k = decltype(kc)::value;
      const bool blk_ok = (ok >> (lq >> 1)) & 1;  // lanes lq 0-1 read block a, 2-3 block b
      const int nvalid = blk_ok ? lim[k] - tok0 : 0;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (v >= nvalid) s1[v] = -INFINITY;
        if (v + 4 >= nvalid) s2[v] = -INFINITY;
      }
    };
    // The lane's max of column tile k's scaled scores (qk_scale > 0: the
    // max of the scaled scores, in log2 units).  NaN-propagating maximum
    // (three-input v_maximum3 on gfx950, no canonicalizing of the MFMA
    // results): it equals fmaxf whenever no score is NaN, and a NaN score
    // makes the column's output NaN either way.
    auto lane_max = [&](const f32x4_t& s1, const f32x4_t& s2) {
      const float m1 = __builtin_elementwise_maximum(__builtin_elementwise_maximum(s1[0], s1[1]),
                                                     __builtin_elementwise_maximum(s1[2], s1[3]));
      const float m2 = __builtin_elementwise_maximum(__builtin_elementwise_maximum(s2[0], s2[1]),
                                                     __builtin_elementwise_maximum(s2[2], s2[3]));
      return __builtin_elementwise_maximum(m1, m2) * qk_scale;
    };
    // The lazy rescale of column tile k: the running max moves only when a
    // score passes it by more than 8, so p <= 256.  The caller's lane-local
    // test decides; the column max (across the 4 lanes of a column) is taken
    // only then.
    auto rescale = [&](auto kc, float mt) {
      constexpr int k = decltype(kc)::value;
      mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
      const float mnew = mt > m[k] + 8.0f ? mt : m[k];
      const float alpha = mnew == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[k] - mnew);
      ol[k] = ol[k] * alpha;
#pragma unroll
      for (int t = 0; t < NV; ++t) o[k][t] = o[k][t] * alpha;
      m[k] = mnew;
    };
    // A column with nothing visible yet keeps m = -inf; its scores are all
    // -inf, so any finite reference gives p = 0.
    auto mref_of = [&](auto kc) {
      constexpr int k = decltype(kc)::value;
      return m[k] == -INFINITY ? 0.0f : m[k];
    };
    auto probs = [&](const f32x4_t& s1, const f32x4_t& s2, float mref, POp& pk, POp& pl) {
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const float sv = v < 4 ? s1[v] : s2[v - 4];
        const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sv, qk_scale, -mref));
        if constexpr (KT != kBF16) {
          pk[v] = (_Float16)pv;
        } else {
          const __bf16 hi = (__bf16)pv;
          pk[v] = hi;
          pl[v] = (__bf16)(pv - (float)hi);
        }
      }
    };
    // O^T += V^T P^T for column tile k; the row sums come out of the same
    // pipe as O[column][0] against a V tile whose channel 0 is all ones.
    auto pv = [&](auto kc, const uint4* vraw, const POp& pk, const POp& pl) {
      constexpr int k = decltype(kc)::value;
      if constexpr (KT != kBF16) {
        const _Float16 one = li == 0 ? (_Float16)1.0f : (_Float16)0.0f;
        const f16x8_t ones = {one, one, one, one, one, one, one, one};
        ol[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, pk, ol[k], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < NV; ++t)
          o[k][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, vraw[t]), pk, o[k][t], 0, 0, 0);
      } else {
        const __bf16 one = li == 0 ? (__bf16)1.0f : (__bf16)0.0f;
        const bf16x8_t ones = {one, one, one, one, one, one, one, one};
        ol[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pk, ol[k], 0, 0, 0);
        ol[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pl, ol[k], 0, 0, 0);
#pragma unroll
        for (int t = 0; t < NV; ++t) {
          const bf16x8_t vop = as_bf16x8(vraw[t]);
          o[k][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pk, o[k][t], 0, 0, 0);
          o[k][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pl, o[k][t], 0, 0, 0);
        }
      }
    };
    // MFMAs of one column tile's P.V (or QK^T) product per batch below.
    constexpr int kPvMfma = KT != kBF16 ? NV + 1 : 2 * NV + 2;
    constexpr int kQkMfma = 2 * NC;

    // One step: the next tile's registers go to the other LDS buffer and
    // the tile after it starts loading into them (interleaved with the
    // first QK^T products), then tile j's math from buffer P.  The
    // registers hold a whole valid tile here (mask_staged_v has zeroed what
    // may not be read); on an item's last step they go to a buffer no one
    // reads.  A wave whose columns see nothing of tile j still runs its
    // math: every score is masked, so it adds exact zeros.
    auto step = [&](auto par, int j) {
      constexpr int P = decltype(par)::value;
      const int valid_next = kvlen - 32 * (j + 1);
      if (!(j + 2 <= nfull && id1.ok == 3)) mask_staged_v<KT, D, VTOK>(vr, id1, valid_next, tid);
      // table entries of tile j + 3, read now and resolved after the math
      int raw_a = -1, raw_b = -1;
      if (j + 3 < nt) {
        raw_a = tp[0];
        if (2 * (j + 3) + 1 < nblk) raw_b = tp[tsm];
      }
      tp += 2 * tsm;
      const uint4* kl = lds[P];
      const uint4* vl = kl + Gm::KENT;
      KOp a1[NC], a2[NC];
      uint4 vraw[NV];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        a1[c] = as_qop<QT>(kl[c * 64 + lane]);
        a2[c] = as_qop<QT>(kl[(NC + c) * 64 + lane]);
      }
      const bool edge = j >= lmin_t || id0.ok != 3;
      const int tok0 = 32 * j + 8 * lq;
      constexpr auto K0 = std::integral_constant<int, 0>{};
      constexpr auto K1 = std::integral_constant<int, 1>{};
      f32x4_t s1a, s2a, s1b, s2b;
      POp pa, pla, pb, plb;
      // QK^T of column tile 0 beside the next tile's conversion into LDS
      qk(K0, a1, a2, s1a, s2a);
      stage_write<QT, KT, D, VTOK, true>(lds[1 - P], kr, vr, id1, valid_next, tid);
      stage_load<KT, D, VTOK>(kr, vr, p, id2, h, tid);
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * NC, 0);
#pragma unroll
      for (int i = 0; i < kQkMfma; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
        __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x020, Gm::KPT + Gm::VPT, 0);
      if (edge) mask(K0, s1a, s2a, id0.ok, tok0);
      // QK^T of column tile 1 beside column tile 0's max; the V operands
      // are read from LDS meanwhile (not earlier: fewer registers live
      // across the QK^T products)
      qk(K1, a1, a2, s1b, s2b);
#pragma unroll
      for (int t = 0; t < NV; ++t)
        vraw[t] = VTOK ? vtok_operand16<D>((const uint8_t*)vl, t, li, lq) : vl[t * 64 + lane];
      const float mta = lane_max(s1a, s2a);
      // keeps the max here, beside the MFMAs, instead of sunk past the
      // next branch to its use
      asm volatile("" ::"v"(mta));
#pragma unroll
      for (int i = 0; i < kQkMfma; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x100, (VTOK ? 2 : 1) * NV / kQkMfma > 0 ? (VTOK ? 2 : 1) * NV / kQkMfma : 1, 1);
        __builtin_amdgcn_sched_group_barrier(0x002, 1, 1);
      }
      if (edge) mask(K1, s1b, s2b, id0.ok, tok0);
      const float mtb = lane_max(s1b, s2b);
      const bool up_a = mta > m[0] + 8.0f, up_b = mtb > m[1] + 8.0f;
      if (__any(up_a || up_b)) {
        rescale(K0, mta);
        rescale(K1, mtb);
      }
      // exponentials of column tile 0, then its P.V beside the exponentials
      // of column tile 1, then column tile 1's P.V
      probs(s1a, s2a, mref_of(K0), pa, pla);
      pv(K0, vraw, pa, pla);
      probs(s1b, s2b, mref_of(K1), pb, plb);
      pv(K1, vraw, pb, plb);
      __builtin_amdgcn_sched_group_barrier(0x002, 20, 2);
#pragma unroll
      for (int i = 0; i < 2 * kPvMfma; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 2);
        __builtin_amdgcn_sched_group_barrier(0x002, 1, 2);
      }
      const TileIds id3 = j + 3 < nt ? tile_resolve(raw_a, raw_b, p.NB) : id2;
      __syncthreads();
      id0 = id1;
      id1 = id2;
      id2 = id3;
    };
    for (int j = 0; j < nt; j += 2) {
      step(std::integral_constant<int, 0>{}, j);
      if (j + 1 < nt) step(std::integral_constant<int, 1>{}, j + 1);
    }

    // ---- normalized output --------------------------------------------------
    const float vs = vscale ? vscale[h * p.vs_s] : 1.0f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float lt = __shfl(ol[k][0], li, 64);  // lane (li, 0) holds column li's sum
      const int col = 32 * wave + 16 * k + li;
      const int r = col / G, g = col % G;
      if (r < rows) {
        const float inv = lt > 0.0f ? vs / lt : 0.0f;
        uint16_t* orow = (uint16_t*)p.out + (int64_t)(row0 + r) * p.o_sr + (int64_t)(h * G + g) * p.o_sh + 4 * lq;
#pragma unroll
        for (int t = 0; t < NV; ++t) {
          uint2 packed;
          packed.x = (uint32_t)out_bits<QT>(o[k][t][0] * inv) | ((uint32_t)out_bits<QT>(o[k][t][1] * inv) << 16);
          packed.y = (uint32_t)out_bits<QT>(o[k][t][2] * inv) | ((uint32_t)out_bits<QT>(o[k][t][3] * inv) << 16);
          *(uint2*)(orow + 16 * t) = packed;
        }
      }
    }
  }
}

int prefill_cus() {
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 256;
  return n;
}

constexpr int kItemBlocksPerCU = 2;  // resident workgroups per CU (8 waves)

template <int QT, int KT, int D, int G, bool VTOK>
int32_t launch_t(PrefillParams& p, hipStream_t stream) {
  static int per_cu = 0;
  if (per_cu == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, prefill_item_kernel<QT, KT, D, G, VTOK>, 256, 0) !=
            hipSuccess ||
        n < 1)
      n = 1;
    per_cu = n < kItemBlocksPerCU ? n : kItemBlocksPerCU;
  }
  {
    ProfileScope prof("cf_prefill_plan", stream);
    CF_LAUNCH(prefill_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, p);
  }
  CF_HIP_CHECK(hipGetLastError());
  {
    ProfileScope prof("cf_prefill_mfma", stream);
    CF_LAUNCH((prefill_item_kernel<QT, KT, D, G, VTOK>), dim3(prefill_cus() * per_cu), dim3(256), 0, stream, p,
                       p.tables, (const int4*)p.items, (const int4*)p.chunks, p.header, p.k_scale, p.v_scale);
  }
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

template <int QT, int KT, int D, bool VTOK>
int32_t launch_v(PrefillParams& p, hipStream_t stream) {
  switch (p.G) {
    case 1: return launch_t<QT, KT, D, 1, VTOK>(p, stream);
    case 2: return launch_t<QT, KT, D, 2, VTOK>(p, stream);
    case 4: return launch_t<QT, KT, D, 4, VTOK>(p, stream);
    case 8: return launch_t<QT, KT, D, 8, VTOK>(p, stream);
    case 16: return launch_t<QT, KT, D, 16, VTOK>(p, stream);
  }
  set_error("prefill: unsupported GQA group %d", p.G);
  return CF_ERR_UNSUPPORTED;
}

// V in token rows (token stride != 1) or the native channel rows
template <int QT, int KT, int D>
int32_t launch_g(PrefillParams& p, hipStream_t stream) {
  return p.v_s[1] != 1 ? launch_v<QT, KT, D, true>(p, stream) : launch_v<QT, KT, D, false>(p, stream);
}

template <int QT, int KT>
int32_t launch_d(PrefillParams& p, hipStream_t stream) {
  if (p.D == 128) return launch_g<QT, KT, 128>(p, stream);
  if (p.D == 64) return launch_g<QT, KT, 64>(p, stream);
  set_error("prefill: unsupported head_dim %d", p.D);
  return CF_ERR_UNSUPPORTED;
}

uint64_t pad256(uint64_t x) { return (x + 255) & ~(uint64_t)255; }

}  // namespace

bool prefill_supported(const PrefillParams& p, int q_dt, int kv_dt) {
  // bf16 queries over bf16 or e4m3 caches; fp16 queries over fp16 or e4m3
  if (q_dt == kBF16) {
    if (kv_dt != kBF16 && kv_dt != kE4M3) return false;
  } else if (q_dt == kF16) {
    if (kv_dt != kF16 && kv_dt != kE4M3) return false;
  } else {
    return false;
  }
  if (p.D != 64 && p.D != 128) return false;
  if (p.G != 1 && p.G != 2 && p.G != 4 && p.G != 8 && p.G != 16) return false;
  if (p.NB < 1) return false;
  const int kb = kv_dt == kE4M3 ? 1 : 2;
  // native (K token rows of head_dim, V channel rows of 16 tokens) or
  // token-major (the reference's layout: both caches in token rows)
  const bool native = p.k_s[3] == 1 && p.k_s[1] == p.D && p.v_s[1] == 1 && p.v_s[3] == 16;
  const bool token_major = p.k_s[3] == 1 && p.v_s[3] == 1 && p.v_s[1] != 1 && (p.k_s[1] * kb) % 16 == 0 &&
                           (p.v_s[1] * kb) % 16 == 0;
  if (!native && !token_major) return false;
  // in-block offsets (15 token rows plus a row) are 32-bit in the kernel
  const int64_t max_off = 16 * (p.k_s[1] > p.v_s[1] ? p.k_s[1] : p.v_s[1]) * kb + (int64_t)p.D * 16 * kb;
  if (p.k_s[1] < 0 || p.v_s[1] < 0 || max_off >= ((int64_t)1 << 32)) return false;
  if ((p.k_s[0] * kb) % 16 || (p.k_s[2] * kb) % 16 || (p.v_s[0] * kb) % 16 || (p.v_s[2] * kb) % 16) return false;
  if (((uintptr_t)p.k & 15) || ((uintptr_t)p.v & 15)) return false;
  if (((uintptr_t)p.q & 15) || (p.q_sr * 2) % 16 || (p.q_sh * 2) % 16) return false;
  if (((uintptr_t)p.out & 7) || (p.o_sr * 2) % 8 || (p.o_sh * 2) % 8) return false;
  return true;
}

int prefill_rows_per_item(int G) { return kCols / G; }

// Workspace: [chunks int4 x N][items int4 x max_items][header 11 int]
uint64_t prefill_workspace_bytes(int64_t Tq, int64_t N, int64_t Hq, int64_t Hkv, int64_t D) {
  (void)D;
  const int64_t G = Hkv > 0 ? Hq / Hkv : 1;
  const int64_t RB = G > 0 ? kCols / G : 1;
  const uint64_t max_items = (uint64_t)(Tq / RB + N) * (uint64_t)Hkv;
  return pad256((uint64_t)N * 16) + pad256(max_items * 16) + 256;
}

void prefill_bind_workspace(PrefillParams& p, void* workspace) {
  char* w = (char*)workspace;
  p.chunks = (int4*)w;
  w += pad256((uint64_t)p.N * 16);
  p.items = (int4*)w;
  w += pad256((uint64_t)p.max_items * 16);
  p.header = (int*)w;
}

int32_t launch_prefill(PrefillParams& p, int q_dt, int kv_dt, hipStream_t stream) {
  if (q_dt == kF16) return kv_dt == kE4M3 ? launch_d<kF16, kE4M3>(p, stream) : launch_d<kF16, kF16>(p, stream);
  return kv_dt == kE4M3 ? launch_d<kBF16, kE4M3>(p, stream) : launch_d<kBF16, kBF16>(p, stream);
}

}  // namespace cf
