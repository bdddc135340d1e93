// MFMA paged-decode kernel for bf16 and OCP e4m3fn KV caches (gfx950).
//
// Same semantics as the generic kernel (reference kernels/paged_attention.py
// :21-73): softmax(q.k * scale) . v over a sequence's first
// min(seq_len, Mb*bs) tokens, query head h reading KV head h / G.
//
// Per 32-token tile (v_mfma_f32_16x16x32_bf16, lane l: i = l % 16,
// q = l / 16; an A operand row and a B operand column are indexed by i,
// output rows by 4q + v):
//   S^T = K Q^T   two MFMA chains (rows = tokens), D/32 MFMAs each.  Lane
//                 (i, q) feeds the K row of token 8*(i/4) + i%4 (+4 for the
//                 second chain), channels [q*D/4, (q+1)*D/4); the chains'
//                 outputs land so that lane (i, q) holds the scores of
//                 column i for the 8 consecutive tokens 8q..8q+7.
//   online softmax per column (lane-local, plus a max across the 4 q groups).
//   O^T += V^T P^T  D/16 MFMAs; lane (i, q) feeds channel 16t + i of V for
//                 tokens 8q..8q+7 -- 8 consecutive tokens of one channel,
//                 which the native V layout ([NB, Hkv, D, bs]) stores
//                 contiguously -- and its own 8 probabilities as P^T.  The
//                 output holds O[column i][16t + 4q + v], so the softmax
//                 rescale stays lane-local.
// The 16 MFMA columns are query heads: the G query heads of the tile's KV
// head (zero-padded when G < 16), so each K/V byte is read once for all of
// them.  e4m3 codes convert to bf16 exactly (v_cvt_scalef32_pk_bf16_fp8,
// scale 1.0); the per-KV-head dequant scales factor out of both products.
//
// Shared prefixes (radix-cache blocks).  When the caller states, per
// sequence, how many leading tokens it shares with the previous sequence
// (same physical blocks), consecutive sequences that share at least
// kMinShareTiles whole tiles form groups of up to 16/G members.  The
// group's common tiles are read once, in a "prefix run" whose 16 columns
// are the members' query heads (member m, head g -> column m*G + g); each
// member then reads only its own remaining tiles.  A member's output is the
// merge of its prefix partial and its own-run partial.
#include "cf_device.hpp"
#include "cf_host.hpp"
#include "decode_params.hpp"
#include "mfma_tile.hpp"

namespace cf {

namespace {

// ---------------------------------------------------------------------------
// Work split: the "tile stream".
//
// Within a KV head, runs are laid out sequence by sequence: a group
// leader's prefix run (its group's shared tiles), then each sequence's own
// run (its tiles after the shared prefix, all of them outside a group).
// The stream is (KV head, run, tile), each run preceded by kRunPad empty
// slots (planned launches); with Tb slots per head and T = Hkv * Tb in all,
// wave w of the Wtot launched waves takes the slots [w * chunk,
// min((w + 1) * chunk, T)), chunk = ceil(T / Wtot): every wave gets the
// same amount of work (tiles plus run changes) whatever the length mix, and
// no workgroup is launched for nothing.  Inside its range a wave keeps
// one online-softmax state per run.  A run the wave holds whole is written
// out: normalized to the output (a sequence outside any group), or as an
// (m, l, o) record (a group member's own run, a prefix run).  A run split
// between waves leaves an (m, l, o) partial in each wave's slot 0 (its
// first run) or 1 (its last run).  decode_merge_kernel combines what each
// (sequence, KV head) left.  (Merging inside this kernel, by the last wave
// to finish a split sequence, needs an agent-scope release per partial; on
// gfx950 that is an L2 writeback per flush and cost more than the separate
// launch.)
//
// Partial rows (ws_o [rows][D] f32, ws_ml [rows][2]): wave slot s holds
// rows [16 s, 16 s + 16), one per MFMA column; own-run records start at row
// rec_own, G rows per (sequence, KV head); prefix records at rec_pre, G rows
// per (member sequence, KV head).
// ---------------------------------------------------------------------------

constexpr int kPlanMaxB = 2048;    // batches up to this size keep a per-sequence plan in LDS
// Stream slots a run's start costs in planned launches.  Ending one run and
// starting the next (flush, new table rows, new q columns) takes about as
// long as one to two tiles (per-wave timings on the Llama-3-8B shape: 1.2 us
// a tile, 1.6 us a run), so each run is preceded by kRunPad empty slots and
// waves split the padded stream evenly: a wave whose range crosses several
// run boundaries gets correspondingly fewer tiles.  2 measured faster than
// 1 or 3.
constexpr int kRunPad = 2;
constexpr int kMinShareTiles = 2;  // shortest shared prefix (32-token tiles) given a group run
constexpr int kSlotCols = 16;      // columns of one partial slot (the MFMA width)
constexpr int kOwn = 0, kPrefix = 1;

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

// ---- per-sequence plan (LDS), built by wave 0 of every workgroup ----------
struct Plan {
  int len[kPlanMaxB];       // effective length
  int j0[kPlanMaxB];        // first tile of the sequence's own run
  int pre[kPlanMaxB];       // group leaders: prefix tiles | members << 24; others 0
  int psum[kPlanMaxB + 1];  // first stream tile (within a KV head) of the sequence's runs
};

// LDS bytes of the plan, rounded up so what follows it is 16-byte aligned.
constexpr size_t kPlanLdsBytes = (sizeof(Plan) + 15) & ~(size_t)15;

// Pass 1: lengths; j0 <- tiles shared with the previous sequence;
// psum <- first member of the sequence's group.  A sequence sharing fewer
// than kMinShareTiles tiles with its predecessor starts a group; groups are
// cut every 16/G members.
__device__ void plan_pass1(const DecodeParams& p, const Index& ix, const int32_t* shared, Plan* pl, int lane) {
  const int SG = kSlotCols / p.G;
  int carry_full = 0, carry_hs = 0;
  for (int base = 0; base < p.B; base += 64) {
    const int b = base + lane;
    const int len = b < p.B ? eff_len(p, ix, b) : 0;
    const int full = len >> 5;
    int fprev = __shfl_up(full, 1, 64);
    if (lane == 0) fprev = carry_full;
    int lcpt = 0;
    if (shared != nullptr && SG > 1 && b > 0 && b < p.B) {
      const int sh = shared[(int64_t)b * p.sh_s];
      lcpt = min(max(sh, 0) >> 5, min(full, fprev));
    }
    const bool hard = lcpt < kMinShareTiles;  // always true for b = 0
    const int hs = max(wave_incl_max(hard ? b : -1, lane), carry_hs);
    if (b < p.B) {
      pl->len[b] = len;
      pl->j0[b] = lcpt;
      pl->psum[b] = hs + SG * ((b - hs) / SG);
    }
    carry_full = __shfl(full, 63, 64);
    carry_hs = __shfl(hs, 63, 64);
  }
}

// Pass 2: each group leader records its members and the tiles all of them
// share (the minimum over the chain of neighbour shares).
__device__ void plan_pass2(const DecodeParams& p, Plan* pl, int lane) {
  const int SG = kSlotCols / p.G;
  for (int base = 0; base < p.B; base += 64) {
    const int b = base + lane;
    if (b < p.B) {
      int pre = 0;
      if (pl->psum[b] == b) {
        int n = 1, P = 1 << 23;
        for (int k = 1; k < SG && b + k < p.B && pl->psum[b + k] == b; ++k) {
          ++n;
          P = min(P, pl->j0[b + k]);
        }
        if (n > 1) pre = P | (n << 24);
      }
      pl->pre[b] = pre;
    }
  }
}

// Pass 3: j0 <- the group's shared tiles; psum <- exclusive scan of the
// stream slots of each sequence's runs (prefix run for leaders + own run),
// kRunPad + tiles per run.
__device__ void plan_pass3(const DecodeParams& p, Plan* pl, int lane) {
  int carry = 0;
  for (int base = 0; base < p.B; base += 64) {
    const int b = base + lane;
    int rt = 0, j0 = 0;
    if (b < p.B) {
      const int lead = pl->psum[b];
      j0 = pl->pre[lead] & 0xFFFFFF;
      const int own = ((pl->len[b] + 31) >> 5) - j0;
      rt = (lead == b && j0 > 0 ? kRunPad + j0 : 0) + (own > 0 ? kRunPad + own : 0);
    }
    const int incl = wave_incl_scan(rt, lane) + carry;
    if (b < p.B) {
      pl->j0[b] = j0;
      pl->psum[b] = incl - rt;
    }
    carry = __shfl(incl, 63, 64);
  }
  if (lane == 0) pl->psum[p.B] = carry;
}

// Largest b with psum[b] <= r (64-ary search; psum[0] = 0 <= r): the
// sequence whose runs hold stream slot r.
__device__ int plan_find(const Plan* pl, int B, int r, int lane) {
  int lo = 0, n = B;
  while (n > 1) {
    const int step = (n + 63) >> 6;
    const int off = lane * step;
    const bool ok = off < n && pl->psum[lo + off] <= r;
    const unsigned long long m = __ballot(ok);
    const int idx = 63 - __clzll((long long)m);
    lo = uniform(lo + idx * step);
    n = uniform(min(step, n - idx * step));
  }
  return lo;
}

// ---- without a plan (batches above kPlanMaxB): no groups -------------------
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

// Per-sequence lookups, from the LDS plan or (PL = false) from seq_lens.
template <bool PL>
struct Seqs {
  const int32_t* __restrict__ lens;
  int64_t sl_s;
  int cap;  // table capacity in tokens
  const Plan* pl;
  __device__ __forceinline__ int len(int b) const {
    if constexpr (PL) {
      return uniform(pl->len[b]);
    } else {
      const int ctx = lens[(int64_t)b * sl_s];
      return ctx < 0 ? 0 : (ctx < cap ? ctx : cap);
    }
  }
  __device__ __forceinline__ int j0(int b) const {
    if constexpr (PL) return uniform(pl->j0[b]);
    else return 0;
  }
  __device__ __forceinline__ int pre(int b) const {
    if constexpr (PL) return uniform(pl->pre[b]);
    else return 0;
  }
  // stream slots of sequence b's runs (0: it has none)
  __device__ __forceinline__ int run_slots(int b) const {
    if constexpr (PL) return uniform(pl->psum[b + 1] - pl->psum[b]);
    else return (len(b) + 31) >> 5;
  }
};

struct Coord {
  int h, b, j;      // KV head, sequence (a prefix run: the group's leader), tile within the sequence
  int kind;         // kOwn or kPrefix
  int first, last;  // the run's tiles [first, last)
  int len;          // effective length of sequence b
  int ncols;        // MFMA columns in use: G, or members * G for a prefix run
  int blkA, blkB;   // physical blocks of the tile (-1: none / invalid)
  int64_t v;        // the tile's stream slot
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

__device__ __forceinline__ void own_run(Coord& c, int j0, int G) {
  c.kind = kOwn;
  c.first = j0;
  c.last = (c.len + 31) >> 5;
  c.ncols = G;
  c.j = j0;
}

// First run of sequence b (the caller knows it has one).
template <bool PL>
__device__ __forceinline__ void enter_seq(const Seqs<PL>& s, Coord& c, int b, int G) {
  c.b = b;
  c.len = s.len(b);
  const int pre = s.pre(b);
  if (pre & 0xFFFFFF) {
    c.kind = kPrefix;
    c.first = 0;
    c.last = pre & 0xFFFFFF;
    c.ncols = (pre >> 24) * G;
    c.j = 0;
  } else {
    own_run(c, s.j0(b), G);
  }
}

// Stream slot of the tile after c (the next run's first tile when c ends
// its run).
template <bool PL>
__device__ __forceinline__ int64_t next_slot(const Coord& c) {
  constexpr int pad = PL ? kRunPad : 0;
  return c.v + 1 + (c.j + 1 < c.last ? 0 : pad);
}

// Next tile in stream order (the caller knows one exists).
template <bool PL>
__device__ __forceinline__ Coord advance(const DecodeParams& p, const Index& ix, const Seqs<PL>& s, Coord c) {
  c.v = next_slot<PL>(c);
  if (c.j + 1 < c.last) {
    c.j += 1;
  } else if (c.kind == kPrefix && c.last < ((c.len + 31) >> 5)) {
    own_run(c, c.last, p.G);  // the leader's own tiles follow its group's prefix
  } else {
    int b = c.b;
    do {
      b += 1;
      if (b == p.B) {
        b = 0;
        c.h += 1;
      }
    } while (s.run_slots(b) == 0);
    enter_seq(s, c, b, p.G);
  }
  fetch_ids(p, ix, c);
  return c;
}

// Q operand terms per channel: fp32 queries are split exactly into three
// bf16 terms (hi + mid + lo, 8 significant bits each), 16-bit queries are
// their own single term.
template <int QT>
constexpr int q_terms() {
  return QT == kF32 ? 3 : 1;
}

// Q operand columns: column i < ncols is query head (i % G) of KV head h for
// sequence b + i / G; the rest are zero.  Term s of channel chunk cc is
// qop[s * D / 32 + cc].
template <int QT, int D>
__device__ __forceinline__ void load_q(QOp<QT>* qop, const DecodeParams& p, const Coord& c, int li, int lq) {
  constexpr int NC = D / 32;
  if constexpr (QT == kF32) {
    // x - hi and (x - hi) - mid are exact in fp32, so hi + mid + lo == x
    // (bf16 has fp32's exponent range).  Unused columns read column 0's row
    // and keep zeros (no divergent branch around the operand registers).
    const bool used = li < c.ncols;
    const int m = used ? li / p.G : 0, g = used ? li - m * p.G : 0;
    const float* qrow = (const float*)p.q + (int64_t)(c.b + m) * p.q_sb + (int64_t)(c.h * p.G + g) * p.q_sh +
                        lq * (D / 4);
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      const float4 a = *(const float4*)(qrow + 8 * cc), b = *(const float4*)(qrow + 8 * cc + 4);
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      bf16x8_t hi, mid, lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xv = used ? x[e] : 0.0f;
        const __bf16 h = (__bf16)xv;
        const float r = xv - (float)h;
        const __bf16 md = (__bf16)r;
        hi[e] = h;
        mid[e] = md;
        lo[e] = (__bf16)(r - (float)md);
      }
      qop[cc] = hi;
      qop[NC + cc] = mid;
      qop[2 * NC + cc] = lo;
    }
    return;
  }
  if (li < c.ncols) {
    const int m = li / p.G, g = li - m * p.G;
    const uint16_t* qrow = (const uint16_t*)p.q + (int64_t)(c.b + m) * p.q_sb + (int64_t)(c.h * p.G + g) * p.q_sh +
                           lq * (D / 4);
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) qop[cc] = as_qop<QT>(*(const uint4*)(qrow + 8 * cc));
  } else {
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) qop[cc] = as_qop<QT>(make_uint4(0, 0, 0, 0));
  }
}

// Outputs: bf16 / fp16 codes for 16-bit queries, fp32 for fp32 queries.
template <int QT>
__device__ __forceinline__ void store_out1(void* out, int64_t off, float v) {
  if constexpr (QT == kF32) ((float*)out)[off] = v;
  else ((uint16_t*)out)[off] = out_bits<QT>(v);
}

// Four consecutive outputs (8-byte aligned codes, 16-byte aligned fp32).
template <int QT>
__device__ __forceinline__ void store_out4(void* out, int64_t off, float a, float b, float c, float d) {
  if constexpr (QT == kF32) {
    *(float4*)((float*)out + off) = make_float4(a, b, c, d);
  } else {
    uint2 packed;
    packed.x = (uint32_t)out_bits<QT>(a) | ((uint32_t)out_bits<QT>(b) << 16);
    packed.y = (uint32_t)out_bits<QT>(c) | ((uint32_t)out_bits<QT>(d) << 16);
    *(uint2*)((uint16_t*)out + off) = packed;
  }
}

// Writes out a finished run (normalized output, record or wave-slot
// partial) and, from the wave holding the run's first tile, the merge
// descriptors of the sequences it covers.
template <int QT, bool PL, int D>
__device__ __forceinline__ void flush_run(const DecodeParams& p, const Index& ix, const Plan* pl, const Coord& c,
                                          const f32x4_t* o, float m, float l, int run_j0, bool first_run,
                                          int64_t chunk, int w, int lane) {
  constexpr int pad = PL ? kRunPad : 0;
  constexpr int NV = D / 16;
  const int li = lane & 15, lq = lane >> 4;
  const int G = p.G;
  float lt = l + __shfl_xor(l, 16, 64);
  lt += __shfl_xor(lt, 32, 64);
  const float vs = ix.vscale ? ix.vscale[c.h * p.vs_s] : 1.0f;
  const bool holds_first = run_j0 == c.first;
  const bool complete = holds_first && c.j == c.last - 1;
  const bool direct = complete && c.kind == kOwn && c.first == 0;  // a whole sequence outside any group
  const int64_t bh = (int64_t)c.b * p.Hkv + c.h;
  if (holds_first) {
    int2 d = make_int2(0, 0);
    if (!complete) {
      // the run's tiles, stream slots [s_tile, s_tile + len), span waves
      // w1..w2; w1 holds it in slot 1 when its range also holds the
      // previous run's last tile (slot s_tile - pad - 1), else in slot 0
      const int64_t s_tile = c.v - (c.j - c.first);
      const int64_t w1 = s_tile / chunk;
      const int64_t w2 = (s_tile + (c.last - c.first) - 1) / chunk;
      d = make_int2((int)((w1 * 2 + (s_tile - pad - 1 >= w1 * chunk ? 1 : 0)) * kSlotCols), (int)(w2 - w1 + 1));
    }
    if (c.kind == kOwn) {
      if (lane == 0) {
        if (complete && !direct) d = make_int2((int)(p.rec_own + bh * G), -1);
        p.own_desc[bh] = d;
        if (c.first == 0) p.pre_desc[bh] = make_int2(0, 0);
      }
    } else if (lane < c.ncols / G) {
      const int64_t bm = (int64_t)(c.b + lane) * p.Hkv + c.h;
      p.pre_desc[bm] = complete ? make_int2((int)(p.rec_pre + bm * G), -1) : make_int2(d.x + lane * G, d.y);
      // a member whose tokens all lie in the shared prefix has no own run
      if constexpr (PL) {
        if (((pl->len[c.b + lane] + 31) >> 5) == c.last) p.own_desc[bm] = make_int2(0, 0);
      }
    }
  }
  if (li >= c.ncols) return;
  if (direct) {
    const float inv = lt > 0.0f ? vs / lt : 0.0f;
    const int64_t orow = (int64_t)c.b * p.o_sb + (int64_t)(c.h * G + li) * p.o_sh + 4 * lq;
#pragma unroll
    for (int t = 0; t < NV; ++t)
      store_out4<QT>(p.out, orow + 16 * t, o[t][0] * inv, o[t][1] * inv, o[t][2] * inv, o[t][3] * inv);
    return;
  }
  int64_t row;
  if (!complete) {
    row = ((int64_t)w * 2 + (first_run ? 0 : 1)) * kSlotCols + li;
  } else if (c.kind == kOwn) {
    row = p.rec_own + bh * G + li;
  } else {
    const int mm = li / G;
    row = p.rec_pre + ((int64_t)(c.b + mm) * p.Hkv + c.h) * G + (li - mm * G);
  }
  float* os = p.ws_o + row * D + 4 * lq;
#pragma unroll
  for (int t = 0; t < NV; ++t)
    *(float4*)(os + 16 * t) = make_float4(o[t][0] * vs, o[t][1] * vs, o[t][2] * vs, o[t][3] * vs);
  if (lq == 0) {
    p.ws_ml[row * 2] = m == -INFINITY ? -INFINITY : m * (1.0f / kLog2e);
    p.ws_ml[row * 2 + 1] = lt;
  }
}

// The stream range a launched wave takes (its "stream wave").  The stream
// is head-major, so the ranges w, w + Wtot/Hkv, ... cover the same sequence
// positions of the Hkv heads, i.e. the same blocks.  Workgroups are dealt
// to the 8 XCDs round-robin (workgroup g on XCD g % 8), each with its own
// L2, so the permutation gives the Hkv heads of one range to waves of the
// same XCD, consecutive in the workgroup order: the heads of a block are
// then read at about the same time from one XCD (adjacent 4 KiB tiles in
// the paired layout; the 128-byte head slices of each token row in the
// token-major layout).  A bijection on [0, Wtot) when the workgroups split
// evenly over the XCDs and Hkv divides each XCD's waves, the identity
// otherwise; it changes which wave does what, never the result.
__device__ __forceinline__ int stream_wave(int w, int Wtot, int Hkv) {
  constexpr int kXcds = 8;
  if (Hkv <= 1 || Wtot % (4 * kXcds) != 0 || (Wtot / kXcds) % Hkv != 0) return w;
  const int g = w >> 2, i = w & 3;
  const int x = g % kXcds, lw = (g / kXcds) * 4 + i;  // XCD, wave index within it
  const int k = x * (Wtot / kXcds / Hkv) + lw / Hkv;     // range among the Wtot / Hkv per head
  return (lw % Hkv) * (Wtot / Hkv) + k;
}

template <int QT, int KT, int D, bool PL, bool VTOK>
__global__ __launch_bounds__(256) void decode_stream_kernel(DecodeParams p, const int32_t* __restrict__ tables,
                                                            const int32_t* __restrict__ lens,
                                                            const float* __restrict__ kscale,
                                                            const float* __restrict__ vscale,
                                                            const int32_t* __restrict__ shared) {
  extern __shared__ int dyn_lds[];
  Plan* pl = reinterpret_cast<Plan*>(dyn_lds);
  const Index ix{tables, lens, kscale, vscale};
  const Seqs<PL> seqs{lens, p.sl_s, p.Mb * 16, pl};
  constexpr int NC = D / 32;
  constexpr int NV = D / 16;
  const int lane = threadIdx.x & 63;
  const int li = lane & 15, lq = lane >> 4;
  const int wave = uniform(threadIdx.x >> 6);
  const int Wtot = gridDim.x * 4;
  const int w = uniform(stream_wave(blockIdx.x * 4 + wave, Wtot, p.Hkv));

  if constexpr (PL) {
    if (wave == 0) plan_pass1(p, ix, shared, pl, lane);
    __syncthreads();
    if (wave == 0) plan_pass2(p, pl, lane);
    __syncthreads();
    if (wave == 0) plan_pass3(p, pl, lane);
    __syncthreads();
  }

  // Sequences with no tokens get zero rows (no tile of theirs is ever
  // visited); wave w takes sequences w, w + Wtot, ...
  for (int bz = w; bz < p.B; bz += Wtot) {
    if (eff_len(p, ix, bz) == 0) {
      const int64_t orow = (int64_t)bz * p.o_sb;
      for (int e = lane; e < p.Hq * D; e += 64) store_out1<QT>(p.out, orow + (int64_t)(e / D) * p.o_sh + e % D, 0.0f);
      for (int hh = lane; hh < p.Hkv; hh += 64) {
        p.own_desc[(int64_t)bz * p.Hkv + hh] = make_int2(0, 0);
        p.pre_desc[(int64_t)bz * p.Hkv + hh] = make_int2(0, 0);
      }
    }
  }
  int Tb;
  if constexpr (PL) Tb = uniform(pl->psum[p.B]);
  else Tb = tiles_per_head(p, ix, lane);
  const int64_t T = (int64_t)p.Hkv * Tb;
  if (T == 0) return;
  const int64_t chunk = (T + Wtot - 1) / Wtot;
  const int64_t v0 = (int64_t)w * chunk;  // this wave's stream slots [v0, v_end)
  if (v0 >= T) return;
  const int64_t v_end = v0 + chunk < T ? v0 + chunk : T;

  Coord c0;
  c0.h = uniform((int)(v0 / Tb));
  {
    const int r = uniform((int)(v0 % Tb));
    if constexpr (PL) {
      // slot r: a run's padding (start at that run's first tile) or a tile
      const int b = plan_find(pl, p.B, r, lane);
      int o = r - uniform(pl->psum[b]);
      int vrun = uniform(pl->psum[b]);
      enter_seq(seqs, c0, b, p.G);
      if (c0.kind == kPrefix && o >= kRunPad + c0.last) {
        o -= kRunPad + c0.last;
        vrun += kRunPad + c0.last;
        own_run(c0, c0.last, p.G);
      }
      c0.j = c0.first + (o > kRunPad ? o - kRunPad : 0);
      c0.v = (int64_t)c0.h * Tb + vrun + kRunPad + (c0.j - c0.first);
    } else {
      int b, before;
      locate(p, ix, r, lane, &b, &before);
      enter_seq(seqs, c0, b, p.G);
      c0.j = r - before;
      c0.v = v0;
    }
  }
  if (c0.v >= v_end) return;  // the range holds padding only
  fetch_ids(p, ix, c0);
  Coord c1 = c0;
  bool has1 = next_slot<PL>(c0) < v_end;
  if (has1) c1 = advance(p, ix, seqs, c0);

  const KvCacheView kv{(const uint8_t*)p.k, (const uint8_t*)p.v, p.k_s[0], p.k_s[2], p.v_s[0], p.v_s[2],
                       p.k_s[1], p.v_s[1]};
  // token-major V: this wave's LDS staging rows, after the plan
  uint8_t* vstage = (uint8_t*)dyn_lds + (PL ? kPlanLdsBytes : 0) + wave * vtok_stage_bytes<D, KvTraits<KT>::kBytes>();
  (void)vstage;
  TileRegs<KT, D, VTOK> r0, r1;
  load_tile<KT, D, VTOK>(r0, kv, c0.blkA, c0.blkB, li, lq, c0.h, lane);

  constexpr int QS = q_terms<QT>();
  QOp<QT> qop[QS * NC];
  load_q<QT, D>(qop, p, c0, li, lq);
  float m = -INFINITY, l = 0.0f;
  f32x4_t o[NV];
#pragma unroll
  for (int t = 0; t < NV; ++t) o[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  int run_j0 = c0.j;
  bool first_run = true;

  // the next run's q columns, loaded a tile ahead (fp32 queries load theirs
  // when the run starts: three terms a tile ahead would not fit the registers)
  QOp<QT> qnext[QT == kF32 ? 1 : NC];
  for (;;) {
    // A run ends with this tile: the next run's q loads go out now, ahead
    // of the next tile's K/V, so they have landed when that tile computes
    // (a load issued after the flush would stall it a full round trip).
    const bool run_ends = !has1 || c1.b != c0.b || c1.h != c0.h || c1.kind != c0.kind;
    if constexpr (QT != kF32) {
      if (has1 && run_ends) load_q<QT, D>(qnext, p, c1, li, lq);
    }
    // Always issue the next tile's loads (the last iteration reloads its
    // own tile) so every path has the same number of loads in flight and
    // the compiler's vmcnt waits stay exact.
    load_tile<KT, D, VTOK>(r1, kv, c1.blkA, c1.blkB, li, lq, c1.h, lane);
    const bool has2 = has1 && next_slot<PL>(c1) < v_end;
    Coord c2 = c1;
    if (has2) c2 = advance(p, ix, seqs, c1);

    // ---- S^T = K Q^T ---------------------------------------------------
    const float ks = ix.kscale ? ix.kscale[c0.h * p.ks_s] : 1.0f;
    const float qk_scale = p.scale * ks * kLog2e;  // scores in log2 units
    f32x4_t s1 = {0.0f, 0.0f, 0.0f, 0.0f}, s2 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if constexpr (QS == 3) {
        // smallest term first
        const QOp<QT> ka = k_operand_q<QT, KT>(r0.k1, c), kb = k_operand_q<QT, KT>(r0.k2, c);
        s1 = mfma16(ka, qop[2 * NC + c], s1);
        s2 = mfma16(kb, qop[2 * NC + c], s2);
        s1 = mfma16(ka, qop[NC + c], s1);
        s2 = mfma16(kb, qop[NC + c], s2);
        s1 = mfma16(ka, qop[c], s1);
        s2 = mfma16(kb, qop[c], s2);
      } else {
        s1 = mfma16(k_operand_q<QT, KT>(r0.k1, c), qop[c], s1);
        s2 = mfma16(k_operand_q<QT, KT>(r0.k2, c), qop[c], s2);
      }
    }
    // lane (li, lq): s1[v] -> token 8lq + v, s2[v] -> token 8lq + 4 + v, column li
    float sc[8];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      sc[v] = s1[v] * qk_scale;
      sc[4 + v] = s2[v] * qk_scale;
    }
    // Tiles at a sequence's end or with an invalid block are the only ones
    // with masked tokens (a wave-uniform condition).
    const bool partial = c0.len - 32 * c0.j < 32 || c0.blkA < 0 || c0.blkB < 0;
    // V operands of the P.V product: loaded channel-major, or (VTOK) staged
    // in LDS and read back transposed
    using VT = typename TileRegs<KT, D, VTOK>::VT;
    VT vraw[NV];
    if constexpr (VTOK) {
      constexpr int KB = KvTraits<KT>::kBytes;
      // the previous tile's transposed reads are done before its rows are overwritten
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      vtok_stage<D, KB>(vstage, r0.v, lane);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int t = 0; t < NV; ++t) {
        if constexpr (KB == 1) vraw[t] = vtok_operand<D>(vstage, t, li, lq);
        else vraw[t] = vtok_operand16<D>(vstage, t, li, lq);
      }
    } else {
#pragma unroll
      for (int t = 0; t < NV; ++t) vraw[t] = r0.v[t];
    }
    int nvalid = 8;
    if (partial) {
      const bool blk_ok = (lq < 2 ? c0.blkA : c0.blkB) >= 0;
      nvalid = blk_ok ? c0.len - 32 * c0.j - 8 * lq : 0;
#pragma unroll
      for (int v = 0; v < 8; ++v)
        if (v >= nvalid) sc[v] = -INFINITY;
#pragma unroll
      for (int t = 0; t < NV; ++t) vraw[t] = mask_tokens(vraw[t], nvalid);
    }
    float mt = sc[0];
#pragma unroll
    for (int v = 1; v < 8; ++v) mt = fmaxf(mt, sc[v]);
    // Lazy rescaling: the running max moves only when a score exceeds it by
    // more than 8 (log2 units), so p = 2^(s - m) <= 256 -- exact enough in
    // fp16/bf16 operands and fp32 sums -- and the O rescale is skipped on
    // almost every tile.
    if (__any(mt > m + 8.0f)) {
      // the lane-local test decides; the column max (across the 4 lanes of
      // a column) is taken only then
      mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
      mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
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
    if constexpr (KT == kE4M3 || KT == kF16) {
      // e4m3 V converts exactly to fp16 (fp16 V is used as is); P in fp16
      // (p <= 256) keeps 11 bits -- 22 as P_hi + P_lo for fp32 queries.
      f16x8_t pop;
#pragma unroll
      for (int v = 0; v < 8; ++v) pop[v] = (_Float16)pr[v];
      if constexpr (QT == kF32) {
        f16x8_t plo;
#pragma unroll
        for (int v = 0; v < 8; ++v) plo[v] = (_Float16)(pr[v] - (float)pop[v]);
#pragma unroll
        for (int t = 0; t < NV; ++t) {
          const f16x8_t vop = e4m3x8_to_f16(vraw[t].x, vraw[t].y);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, plo, o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop, o[t], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int t = 0; t < NV; ++t) {
          f16x8_t vop;
          if constexpr (KT == kE4M3) vop = e4m3x8_to_f16(vraw[t].x, vraw[t].y);
          else vop = __builtin_bit_cast(f16x8_t, vraw[t]);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vop, pop, o[t], 0, 0, 0);
        }
      }
    } else {
      // bf16 V: P = P_hi + P_lo in bf16 (two MFMAs) keeps ~16 bits; fp32
      // queries add a third term (24 bits).
      bf16x8_t pop, plo;
#pragma unroll
      for (int v = 0; v < 8; ++v) {
        const __bf16 hi = (__bf16)pr[v];
        pop[v] = hi;
        plo[v] = (__bf16)(pr[v] - (float)hi);
      }
      if constexpr (QT == kF32) {
        bf16x8_t pl2;
#pragma unroll
        for (int v = 0; v < 8; ++v) pl2[v] = (__bf16)((pr[v] - (float)pop[v]) - (float)plo[v]);
#pragma unroll
        for (int t = 0; t < NV; ++t) {
          const bf16x8_t vop = as_bf16x8(vraw[t]);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pl2, o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, plo, o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop, o[t], 0, 0, 0);
        }
      } else {
#pragma unroll
        for (int t = 0; t < NV; ++t) {
          const bf16x8_t vop = as_bf16x8(vraw[t]);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, pop, o[t], 0, 0, 0);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vop, plo, o[t], 0, 0, 0);
        }
      }
    }

    // ---- end of a run -----------------------------------------------------
    if (run_ends) {
      flush_run<QT, PL, D>(p, ix, pl, c0, o, m, l, run_j0, first_run, chunk, w, lane);
      first_run = false;
    }
    if (!has1) break;

    c0 = c1;
    c1 = c2;
    has1 = has2;
    r0 = r1;
    if (run_ends) {
      if constexpr (QT == kF32) {
        load_q<QT, D>(qop, p, c0, li, lq);
      } else {
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) qop[cc] = qnext[cc];
      }
      m = -INFINITY;
      l = 0.0f;
#pragma unroll
      for (int t = 0; t < NV; ++t) o[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      run_j0 = c0.j;
    }
  }
}

// Row of the k-th partial a merge descriptor names: {row, -1} is one
// record; {row, n} is n wave-slot rows, the first at `row` (slot * 16 +
// column), then slot 0 of each following wave at the same column.
__device__ __forceinline__ int64_t part_row(int2 d, int k) {
  if (d.y < 0 || k == 0) return d.x;
  const int w1 = (d.x / kSlotCols) >> 1;
  const int col = d.x % kSlotCols;
  return (int64_t)(2 * (w1 + k)) * kSlotCols + col;
}

// Combines the (m, l, o) partials of each (sequence b, KV head h) that the
// decode kernel did not write whole: its own run's and its group's prefix
// run's, each a record or the wave slots of a split run.  NSL workgroups per
// (h, b), each owning 1/NSL of the G x D output (more workgroups for small
// grids); one wave of the first does the work when the partials fit its
// registers, all four waves of each otherwise.  Partial rows hold the G
// heads of h in consecutive rows.
template <int QT, int D, int G, int NSL>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeParams p) {
  constexpr int E = G * D / 64;  // output elements per lane
  constexpr int kWaves = 4;
  const int h = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = uniform((int)threadIdx.x >> 6);
  const int2 dn = p.own_desc[(int64_t)b * p.Hkv + h];
  const int2 dp = p.pre_desc[(int64_t)b * p.Hkv + h];
  const int nown = dn.y < 0 ? 1 : dn.y;
  const int npre = dp.y < 0 ? 1 : dp.y;
  const int nsrc = nown + npre;
  if (nsrc == 0) return;  // written whole by the decode kernel (or empty)
  constexpr int KMAX = 64 / E;  // partials the register path holds
  if (nsrc <= KMAX) {
    if (wave != 0 || blockIdx.z != 0) return;
    // Few partials (the usual case): every load is issued at once -- each
    // lane's slice of every partial row and every (m, l) -- so the merge
    // costs one round trip after the descriptors.
    float ov[KMAX][E], mk[KMAX][G], lk[KMAX][G];
#pragma unroll
    for (int k = 0; k < KMAX; ++k) {
      if (k < nsrc) {
        const int64_t row = k < nown ? part_row(dn, k) : part_row(dp, k - nown);
        const float* o = p.ws_o + row * D;
#pragma unroll
        for (int i = 0; i < E; ++i) ov[k][i] = o[lane + 64 * i];
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float2 ml = *(const float2*)(p.ws_ml + (row + g) * 2);
          mk[k][g] = ml.x;
          lk[k][g] = ml.y;
        }
      }
    }
    float Mg[G], Lg[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      Mg[g] = -INFINITY;
#pragma unroll
      for (int k = 0; k < KMAX; ++k)
        if (k < nsrc) Mg[g] = fmaxf(Mg[g], mk[k][g]);
      Lg[g] = 0.0f;
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        if (k < nsrc) {
          const float w = mk[k][g] == -INFINITY ? 0.0f : __expf(mk[k][g] - Mg[g]);
          mk[k][g] = w;  // now the weight
          Lg[g] += w * lk[k][g];
        }
      }
    }
    const int64_t out = (int64_t)b * p.o_sb;
#pragma unroll
    for (int i = 0; i < E; ++i) {
      const int idx = lane + 64 * i;
      const int g = idx / D, d = idx % D;
      float a = 0.0f;
      float lg = 0.0f;
#pragma unroll
      for (int gg = 0; gg < G; ++gg)
        if (gg == g) lg = Lg[gg];
#pragma unroll
      for (int k = 0; k < KMAX; ++k) {
        if (k < nsrc) {
          float w = 0.0f;
#pragma unroll
          for (int gg = 0; gg < G; ++gg)
            if (gg == g) w = mk[k][gg];
          a += w * ov[k][i];
        }
      }
      store_out1<QT>(p.out, out + (int64_t)(h * G + g) * p.o_sh + d, lg > 0.0f ? a / lg : 0.0f);
    }
    return;
  }
  // Many partials (a sequence split over hundreds of waves), in chunks of
  // up to 256: the chunk's (m, l) pairs and row indices are staged in LDS;
  // wave w reduces heads w, w + 4, ... (max, weights, weighted sum of l)
  // and keeps their running (M, L); then each thread accumulates one
  // 16-byte slice of the G x D output over every NP-th partial of the
  // chunk, a batch of loads in flight at a time, and the NP phases are
  // summed through LDS at the end.
  constexpr int kChunk = 256;
  constexpr int NF4 = G * D / 4 / NSL;            // 16-byte slices of the output in this workgroup
  static_assert(G * D / 4 % NSL == 0, "output slices split evenly");
  constexpr int FPT = NF4 > 256 ? NF4 / 256 : 1;  // slices per thread
  constexpr int NP = NF4 >= 256 ? 1 : 256 / NF4;  // partial phases
  constexpr int U = FPT == 1 ? 16 : 8;            // partials per batch of loads
  __shared__ float sm[G][kChunk];                 // m, then the partial's weight
  __shared__ float sl[G][kChunk];
  __shared__ int srow[kChunk];
  __shared__ float run_m[G], run_l[G], run_sc[G];
  __shared__ float4 red[NP > 1 ? NP - 1 : 1][NP > 1 ? NF4 : 1];
  const int tid = (int)threadIdx.x;
  const int ph = FPT == 1 ? tid / NF4 : 0;
  int fs[FPT], gs[FPT];
#pragma unroll
  for (int j = 0; j < FPT; ++j) {
    fs[j] = (int)blockIdx.z * NF4 + (FPT == 1 ? tid % NF4 : tid + 256 * j);
    gs[j] = 4 * fs[j] / D;
  }
  if (tid < G) {
    run_m[tid] = -INFINITY;
    run_l[tid] = 0.0f;
  }
  float4 acc[FPT];
#pragma unroll
  for (int j = 0; j < FPT; ++j) acc[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int c0 = 0; c0 < nsrc; c0 += kChunk) {
    const int n = min(kChunk, nsrc - c0);
    if (tid < n) {
      const int k = c0 + tid;
      const int row = (int)(k < nown ? part_row(dn, k) : part_row(dp, k - nown));
      srow[tid] = row;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float2 ml = *(const float2*)(p.ws_ml + ((int64_t)row + g) * 2);
        sm[g][tid] = ml.x;
        sl[g][tid] = ml.y;
      }
    }
    __syncthreads();
    for (int g = wave; g < G; g += kWaves) {
      float mx = -INFINITY;
      for (int k = lane; k < n; k += 64) mx = fmaxf(mx, sm[g][k]);
      mx = wave_max(mx);
      const float mold = run_m[g];
      const float mnew = fmaxf(mold, mx);
      float ls = 0.0f;
      for (int k = lane; k < n; k += 64) {
        const float mk = sm[g][k];
        const float w = mk == -INFINITY ? 0.0f : __expf(mk - mnew);
        sm[g][k] = w;
        ls += w * sl[g][k];
      }
      ls = wave_sum(ls);
      if (lane == 0) {
        const float sc = mold == -INFINITY ? 0.0f : __expf(mold - mnew);
        run_sc[g] = sc;
        run_l[g] = run_l[g] * sc + ls;
        run_m[g] = mnew;
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < FPT; ++j) {
      const float sc = run_sc[gs[j]];
      acc[j].x *= sc;
      acc[j].y *= sc;
      acc[j].z *= sc;
      acc[j].w *= sc;
    }
    for (int kb = ph; kb < n; kb += NP * U) {
      float4 ov[U][FPT];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int k = kb + u * NP;
        if (k < n) {
          const float4* o = (const float4*)(p.ws_o + (int64_t)srow[k] * D);
#pragma unroll
          for (int j = 0; j < FPT; ++j) ov[u][j] = o[fs[j]];
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int k = kb + u * NP;
        if (k < n) {
#pragma unroll
          for (int j = 0; j < FPT; ++j) {
            const float w = sm[gs[j]][k];
            acc[j].x += w * ov[u][j].x;
            acc[j].y += w * ov[u][j].y;
            acc[j].z += w * ov[u][j].z;
            acc[j].w += w * ov[u][j].w;
          }
        }
      }
    }
    __syncthreads();  // the next chunk restages sm, sl, srow
  }
  if constexpr (NP > 1) {
    if (ph > 0) red[ph - 1][fs[0] % NF4] = acc[0];
    __syncthreads();
    if (ph > 0) return;
#pragma unroll
    for (int q = 0; q < NP - 1; ++q) {
      const float4 r = red[q][fs[0] % NF4];
      acc[0].x += r.x;
      acc[0].y += r.y;
      acc[0].z += r.z;
      acc[0].w += r.w;
    }
  }
  const int64_t out = (int64_t)b * p.o_sb;
#pragma unroll
  for (int j = 0; j < FPT; ++j) {
    const int g = gs[j], d = 4 * fs[j] % D;
    const float lg = run_l[g];
    auto nrm = [&](float a) { return lg > 0.0f ? a / lg : 0.0f; };
    store_out4<QT>(p.out, out + (int64_t)(h * G + g) * p.o_sh + d, nrm(acc[j].x), nrm(acc[j].y), nrm(acc[j].z),
                   nrm(acc[j].w));
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
// Llama-3-8B shape).  The workspace holds slots for this many waves.
constexpr int kStreamBlocksPerCU = 1;
// Merge grids of fewer (sequence, KV head) pairs than this split each
// output over 4 workgroups.
constexpr int kMergeSplitBelow = 256;

template <int KT, int D, bool PL, bool VTOK>
constexpr size_t stream_lds_bytes() {
  return (PL ? kPlanLdsBytes : 0) + (VTOK ? 4 * (size_t)vtok_stage_bytes<D, KvTraits<KT>::kBytes>() : 0);
}

template <int QT, int KT, int D, bool PL, bool VTOK>
int blocks_per_cu() {
  static int cached = 0;
  if (cached == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, decode_stream_kernel<QT, KT, D, PL, VTOK>, 256,
                                                     stream_lds_bytes<KT, D, PL, VTOK>()) != hipSuccess ||
        n < 1)
      n = 1;
    cached = n < kStreamBlocksPerCU ? n : kStreamBlocksPerCU;
  }
  return cached;
}

template <int QT, int KT, int D, bool PL, bool VTOK>
int32_t launch_stream_t(const DecodeParams& p, hipStream_t stream) {
  const int blocks = cu_count() * blocks_per_cu<QT, KT, D, PL, VTOK>();
  ProfileScope prof("cf_decode_mfma", stream);
  CF_LAUNCH((decode_stream_kernel<QT, KT, D, PL, VTOK>), dim3(blocks), dim3(256), (stream_lds_bytes<KT, D, PL, VTOK>()),
            stream, p, p.tables, p.seq_lens, p.k_scale, p.v_scale, PL ? p.shared : nullptr);
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

// Whether V is token-major (the reference's [NB, bs, Hkv, D] order, unit
// channel stride) rather than the native channel-major tile.
bool v_token_major(const DecodeParams& p) { return p.v_s[3] == 1 && p.v_s[1] != 1; }

template <int QT, int KT, int D, bool VTOK>
int32_t launch_pl(const DecodeParams& p, hipStream_t stream) {
  return p.B <= kPlanMaxB ? launch_stream_t<QT, KT, D, true, VTOK>(p, stream)
                          : launch_stream_t<QT, KT, D, false, VTOK>(p, stream);
}

template <int QT, int KT, int D>
int32_t launch_t(const DecodeParams& p, hipStream_t stream) {
  int32_t rc;
  rc = v_token_major(p) ? launch_pl<QT, KT, D, true>(p, stream) : launch_pl<QT, KT, D, false>(p, stream);
  if (rc) return rc;
  // Small grids (few sequences x KV heads) split each output over 4
  // workgroups, so that long sequences' many partials are read by more CUs.
  const bool split = (int64_t)p.B * p.Hkv < kMergeSplitBelow;
  const dim3 grid(p.Hkv, p.B, split ? 4 : 1);
  ProfileScope prof("cf_decode_merge", stream);
#define CF_MERGE(G)                                                                         \
  if (split) CF_LAUNCH((decode_merge_kernel<QT, D, G, 4>), grid, dim3(256), 0, stream, p); \
  else CF_LAUNCH((decode_merge_kernel<QT, D, G, 1>), grid, dim3(256), 0, stream, p);
  switch (p.G) {
    case 1: CF_MERGE(1) break;
    case 2: CF_MERGE(2) break;
    case 4: CF_MERGE(4) break;
    case 8: CF_MERGE(8) break;
    case 16: CF_MERGE(16) break;
    default: set_error("MFMA decode: unsupported GQA group %d", p.G); return CF_ERR_UNSUPPORTED;
  }
#undef CF_MERGE
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

// Workspace layout: [partial rows: o, D f32 each, 256-byte padded]
// [(m, l) per row, padded] [own-run descriptors: int2 per (sequence, KV
// head), padded] [prefix descriptors, same].  Rows: 2 slots x 16 columns per
// wave, then G own-run and G prefix records per (sequence, KV head).
uint64_t stream_waves() { return (uint64_t)cu_count() * kStreamBlocksPerCU * 4; }
uint64_t pad256(uint64_t x) { return (x + 255) & ~(uint64_t)255; }
uint64_t slot_rows() { return stream_waves() * 2 * kSlotCols; }
uint64_t total_rows(int64_t batch, int64_t num_q_heads) { return slot_rows() + 2 * (uint64_t)batch * num_q_heads; }

}  // namespace

uint64_t decode_mfma_workspace_bytes(int64_t batch, int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim) {
  const uint64_t rows = total_rows(batch, num_q_heads);
  const uint64_t desc = pad256((uint64_t)batch * num_kv_heads * 8);
  return pad256(rows * head_dim * 4) + pad256(rows * 2 * 4) + 2 * desc;
}

void decode_mfma_bind_workspace(DecodeParams& p, void* workspace) {
  const uint64_t rows = total_rows(p.B, p.Hq);
  const uint64_t desc = pad256((uint64_t)p.B * p.Hkv * 8);
  char* w = (char*)workspace;
  p.ws_o = (float*)w;
  w += pad256(rows * p.D * 4);
  p.ws_ml = (float*)w;
  w += pad256(rows * 2 * 4);
  p.own_desc = (int2*)w;
  w += desc;
  p.pre_desc = (int2*)w;
  p.rec_own = (int64_t)slot_rows();
  p.rec_pre = p.rec_own + (int64_t)p.B * p.Hq;
}

bool decode_mfma_supported(const DecodeParams& p, int q_dt, int kv_dt) {
  // bf16 or fp32 queries over bf16 or e4m3 caches; fp16 queries over fp16
  // or e4m3
  if (q_dt == kBF16 || q_dt == kF32) {
    if (kv_dt != kBF16 && kv_dt != kE4M3) return false;
  } else if (q_dt == kF16) {
    if (kv_dt != kF16 && kv_dt != kE4M3) return false;
  } else {
    return false;
  }
  if (p.bs != 16 || (p.D != 64 && p.D != 128)) return false;
  if (p.G != 1 && p.G != 2 && p.G != 4 && p.G != 8 && p.G != 16) return false;
  if (p.NB < 1) return false;  // invalid block ids are redirected to block 0 (then masked)
  // partial-row indices and descriptors are int32
  if ((uint64_t)total_rows(p.B, p.Hq) >= (uint64_t)INT32_MAX / 2) return false;
  const int kb = kv_dt == kE4M3 ? 1 : 2;
  // K: token rows with unit channel stride, 16-byte aligned (token stride D
  // in the native / paired layouts, any multiple of 16 bytes token-major).
  // V: the native tile [D][bs] (token stride 1, channel stride bs), or
  // token-major rows (channel stride 1) -- block/head strides free.
  if (p.k_s[3] != 1) return false;
  for (int i = 0; i < 3; ++i)
    if ((p.k_s[i] * kb) % 16 != 0) return false;
  const bool v_native = p.v_s[1] == 1 && p.v_s[3] == 16;
  const bool v_tok = p.v_s[3] == 1 && p.v_s[1] != 1 && (p.v_s[1] * kb) % 16 == 0;
  if (!v_native && !v_tok) return false;
  // native V rides with the native K tile (token stride D)
  if (v_native && p.k_s[1] != p.D) return false;
  if ((p.v_s[0] * kb) % 16 != 0 || (p.v_s[2] * kb) % 16 != 0) return false;
  if (v_native && (p.v_s[3] * kb) % 16 != 0) return false;
  if (!aligned16(p.k) || !aligned16(p.v)) return false;
  // q rows: 16-byte aligned slices; out rows: aligned groups of 4 (8 bytes
  // of 16-bit codes, 16 bytes of fp32).
  const int qb = q_dt == kF32 ? 4 : 2, oal = q_dt == kF32 ? 16 : 8;
  if (!aligned16(p.q) || (p.q_sb * qb) % 16 != 0 || (p.q_sh * qb) % 16 != 0) return false;
  if (((uintptr_t)p.out & (oal - 1)) != 0 || (p.o_sb * qb) % oal != 0 || (p.o_sh * qb) % oal != 0) return false;
  return true;
}

template <int QT, int KT>
int32_t launch_d(const DecodeParams& p, hipStream_t stream) {
  if (p.D == 128) return launch_t<QT, KT, 128>(p, stream);
  if (p.D == 64) return launch_t<QT, KT, 64>(p, stream);
  set_error("MFMA decode: unsupported head_dim %d", p.D);
  return CF_ERR_UNSUPPORTED;
}

int32_t launch_decode_mfma(const DecodeParams& p, int q_dt, int kv_dt, hipStream_t stream) {
  if (q_dt == kF16) return kv_dt == kE4M3 ? launch_d<kF16, kE4M3>(p, stream) : launch_d<kF16, kF16>(p, stream);
  if (q_dt == kF32) return kv_dt == kE4M3 ? launch_d<kF32, kE4M3>(p, stream) : launch_d<kF32, kBF16>(p, stream);
  return kv_dt == kE4M3 ? launch_d<kBF16, kE4M3>(p, stream) : launch_d<kBF16, kBF16>(p, stream);
}

}  // namespace cf
