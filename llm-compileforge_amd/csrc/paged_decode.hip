// Paged decode attention: generic VALU kernel (any dtype, any block size,
// any strides) and the log-sum-exp partition reduce.
//
// Semantics follow the reference CPU path (kernels/paged_attention.py:21-73):
// sequence b attends non-causally to its first min(seq_len, Mb*bs) cached
// tokens, gathered in block-table order; query head h reads KV head h / G
// (repeat_interleave, :57-60); softmax(q.k * scale) . v in fp32.
//
// Work split: one workgroup per (partition, kv head, sequence).  A
// partition is PT consecutive tokens.  With more than one partition per
// sequence the workgroup writes (m, l, o) partials, merged by
// decode_reduce; with a single partition it writes the output directly.
// Scores: 16 lanes per token, each taking every 16th channel (consecutive
// lanes read consecutive channels of a K row), summed across the 16 lanes.
// P.V: the G * D outputs are spread over the 256 threads and, when there are
// fewer outputs than threads, the partition's tokens are split between
// thread groups whose sums meet in LDS.
#include "cf_device.hpp"
#include "cf_host.hpp"
#include "decode_params.hpp"

namespace cf {

namespace {

constexpr int kGenericThreads = 256;

__device__ __forceinline__ int effective_len(const DecodeParams& p, int b) {
  int ctx = p.seq_lens[(int64_t)b * p.sl_s];
  const int cap = p.Mb * p.bs;
  ctx = ctx < cap ? ctx : cap;
  return ctx > 0 ? ctx : 0;
}

template <int QT, int KT, bool DIRECT>
__global__ __launch_bounds__(kGenericThreads) void decode_generic_kernel(DecodeParams p) {
  extern __shared__ float smem[];
  const int part = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int G = p.G, D = p.D, bs = p.bs, PT = p.PT;
  const int ctx = effective_len(p, b);
  const int start = part * PT;

  using OutE = Elem<QT>;
  if (start >= ctx) {
    if (DIRECT && ctx == 0) {
      for (int i = tid; i < G * D; i += kGenericThreads) {
        const int g = i / D, d = i % D;
        OutE::store((typename OutE::T*)p.out + (int64_t)b * p.o_sb + (int64_t)(h * G + g) * p.o_sh + d, 0.0f);
      }
    }
    return;
  }
  const int count = min(PT, ctx - start);

  float* sq = smem;                           // [G][D]
  float* sc = sq + G * D;                     // [G][PT]
  int* sblk = (int*)(sc + G * PT);            // [PT / bs]
  float* sml = (float*)(sblk + ((PT / bs + 1) & ~1));  // [G][2]
  float* sacc = sml + 2 * G;                  // [256] P.V partial sums

  using QE = Elem<QT>;
  using KE = Elem<KT>;
  const typename QE::T* qb = (const typename QE::T*)p.q + (int64_t)b * p.q_sb;
  for (int i = tid; i < G * D; i += kGenericThreads) {
    const int g = i / D, d = i % D;
    sq[i] = QE::load(qb + (int64_t)(h * G + g) * p.q_sh + d);
  }
  const int nblk = (count + bs - 1) / bs;
  const int blk0 = start / bs;
  for (int i = tid; i < nblk; i += kGenericThreads)
    sblk[i] = p.tables[(int64_t)b * p.t_sb + (int64_t)(blk0 + i) * p.t_sm];
  __syncthreads();

  const float ks = p.k_scale ? p.k_scale[h * p.ks_s] : 1.0f;
  const float vs = p.v_scale ? p.v_scale[h * p.vs_s] : 1.0f;
  const float qk_scale = p.scale * ks;

  // scores: token i on the 16 lanes of slot i % 16, channels sub, sub + 16, ...
  constexpr int kChunk = 8;  // channels per lane held in registers at once
  const typename KE::T* kbase = (const typename KE::T*)p.k;
  const int sub = tid & 15, slot = tid >> 4;
  for (int i0 = 0; i0 < count; i0 += kGenericThreads / 16) {
    const int i = i0 + slot;
    const bool tok_ok = i < count;
    const int tok = start + i;
    const int64_t blk = tok_ok ? sblk[i / bs] : -1;
    const bool blk_ok = (uint64_t)blk < (uint64_t)p.NB;
    const typename KE::T* krow =
        kbase + (blk_ok ? blk : 0) * p.k_s[0] + (int64_t)(tok % bs) * p.k_s[1] + (int64_t)h * p.k_s[2];
    for (int d0 = 0; d0 < D; d0 += 16 * kChunk) {
      // every load issued before any is used: out-of-range channels read
      // channel 0 of the row (or of block 0) and are zeroed afterwards; a
      // cache without blocks (possibly a null pointer) is not read at all
      float kv[kChunk];
      if (p.NB > 0) {
#pragma unroll
        for (int c = 0; c < kChunk; ++c) {
          const int d = d0 + sub + 16 * c;
          kv[c] = KE::load(krow + (int64_t)(d < D ? d : 0) * p.k_s[3]);
        }
      }
#pragma unroll
      for (int c = 0; c < kChunk; ++c)
        if (!blk_ok || d0 + sub + 16 * c >= D) kv[c] = 0.0f;
      for (int g = 0; g < G; ++g) {
        const float* qg = sq + g * D;
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < kChunk; ++c) {
          const int d = d0 + sub + 16 * c;
          if (d < D) acc = fmaf(qg[d], kv[c], acc);
        }
        // sum over the token's 16 lanes (aligned groups of 16)
        acc += __shfl_xor(acc, 8, 64);
        acc += __shfl_xor(acc, 4, 64);
        acc += __shfl_xor(acc, 2, 64);
        acc += __shfl_xor(acc, 1, 64);
        if (sub == 0 && tok_ok) {
          const float prev = d0 == 0 ? 0.0f : sc[g * PT + i];
          sc[g * PT + i] = prev + acc;
        }
      }
    }
    if (sub == 0 && tok_ok)
      for (int g = 0; g < G; ++g) sc[g * PT + i] = blk_ok ? sc[g * PT + i] * qk_scale : -INFINITY;
  }
  __syncthreads();

  // softmax statistics per query head: one wave per head
  const int wave = tid / 64, lane = tid % 64;
  for (int g = wave; g < G; g += kGenericThreads / 64) {
    float m = -INFINITY;
    for (int i = lane; i < count; i += 64) m = fmaxf(m, sc[g * PT + i]);
    m = wave_max(m);
    float l = 0.0f;
    for (int i = lane; i < count; i += 64) {
      const float e = m == -INFINITY ? 0.0f : expf(sc[g * PT + i] - m);
      sc[g * PT + i] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) {
      sml[2 * g] = m;
      sml[2 * g + 1] = l;
    }
  }
  __syncthreads();

  // p . v: output (g, d) = sum over tokens; with GD < 256 outputs the tokens
  // are dealt round-robin to ng = 256 / GD thread groups.  Channel rows of
  // 16 tokens (the native V tile at block size 16) go by whole blocks
  // instead, the block's 16 values of the thread's channel in one vector
  // load.
  const typename KE::T* vbase = (const typename KE::T*)p.v;
  const int GD = G * D;
  const int ng = GD < kGenericThreads ? kGenericThreads / GD : 1;
  constexpr int64_t kEs = sizeof(typename KE::T);
  const bool vtile = bs == 16 && p.v_s[1] == 1 && ((uintptr_t)p.v & 15) == 0 &&
                     ((p.v_s[0] * kEs) & 15) == 0 && ((p.v_s[2] * kEs) & 15) == 0 && ((p.v_s[3] * kEs) & 15) == 0;
  for (int o0 = 0; o0 < GD; o0 += kGenericThreads) {
    const int grp = ng > 1 ? tid / GD : 0;
    const int o = ng > 1 ? tid % GD : o0 + tid;
    const bool active = grp < ng && o < GD;
    const int g = active ? o / D : 0, d = active ? o % D : 0;
    float acc = 0.0f;
    if (active && vtile) {
      for (int bi = grp; bi < nblk; bi += ng) {
        const int64_t blk = sblk[bi];
        if ((uint64_t)blk >= (uint64_t)p.NB) continue;
        float v16[16];
        load16<KT>(vbase + blk * p.v_s[0] + (int64_t)h * p.v_s[2] + (int64_t)d * p.v_s[3], v16);
        const int t0 = bi * 16;
#pragma unroll
        for (int e = 0; e < 16; ++e)
          if (t0 + e < count) acc = fmaf(sc[g * PT + t0 + e], v16[e], acc);
      }
    } else if (active) {
      // kU tokens per step, their loads issued together (an invalid block
      // reads block 0 and gets weight 0; a cache without blocks is not read)
      constexpr int kU = 8;
      for (int t0 = grp; p.NB > 0 && t0 < count; t0 += kU * ng) {
        float vv[kU], ww[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
          const int t = t0 + u * ng;
          const int tt = t < count ? t : grp;
          const int64_t blk = sblk[tt / bs];
          const bool ok = t < count && (uint64_t)blk < (uint64_t)p.NB;
          const typename KE::T* vrow = vbase + (ok ? blk : 0) * p.v_s[0] + (int64_t)((start + tt) % bs) * p.v_s[1] +
                                       (int64_t)h * p.v_s[2];
          vv[u] = KE::load(vrow + (int64_t)d * p.v_s[3]);
          ww[u] = ok ? sc[g * PT + tt] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) acc = fmaf(ww[u], vv[u], acc);
      }
    }
    if (ng > 1) {
      sacc[tid] = acc;
      __syncthreads();
      if (tid >= GD) break;  // GD < 256: one pass, the first GD threads finish it
      acc = 0.0f;
      for (int k = 0; k < ng; ++k) acc += sacc[k * GD + tid];
    } else if (!active) {
      continue;
    }
    acc *= vs;
    const int hq = h * G + g;
    if (DIRECT) {
      const float l = sml[2 * g + 1];
      OutE::store((typename OutE::T*)p.out + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh + d,
                  l > 0.0f ? acc / l : 0.0f);
    } else {
      const int64_t row = ((int64_t)b * p.Hq + hq) * p.max_parts + part;
      p.ws_o[row * D + d] = acc;
      if (d == 0) {
        p.ws_ml[row * 2] = sml[2 * g];
        p.ws_ml[row * 2 + 1] = sml[2 * g + 1];
      }
    }
  }
}

// Merges the partition partials of one (sequence, query head):
// O = sum_i exp(m_i - M) o_i / sum_i exp(m_i - M) l_i with M = max_i m_i.
// 256 threads: (m, l) are read lane-parallel and reduced across the block;
// the weighted sum takes the partitions in 256 / D interleaved groups (all
// their loads independent), whose sums meet in LDS.
template <int OT>
__global__ __launch_bounds__(256) void decode_reduce_kernel(DecodeParams p) {
  __shared__ float red[8];
  __shared__ float part_acc[256];
  const int hq = blockIdx.x, b = blockIdx.y;
  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  const int ctx = effective_len(p, b);
  const int nparts = (ctx + p.PT - 1) / p.PT;
  using OutE = Elem<OT>;
  typename OutE::T* o = (typename OutE::T*)p.out + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh;
  const int64_t row0 = ((int64_t)b * p.Hq + hq) * p.max_parts;
  const float* ml = p.ws_ml + row0 * 2;
  const float* po = p.ws_o + row0 * p.D;
  if (nparts == 0) {
    for (int d = tid; d < p.D; d += 256) OutE::store(o + d, 0.0f);
    return;
  }
  float mloc = -INFINITY;
  for (int i = tid; i < nparts; i += 256) mloc = fmaxf(mloc, ml[i * 2]);
  mloc = wave_max(mloc);
  if (lane == 0) red[wave] = mloc;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  // A partition whose blocks were all invalid has m = -inf and l = 0.
  float lloc = 0.0f;
  for (int i = tid; i < nparts; i += 256) {
    const float m = ml[i * 2];
    if (m != -INFINITY) lloc += ml[i * 2 + 1] * expf(m - M);
  }
  lloc = wave_sum(lloc);
  if (lane == 0) red[4 + wave] = lloc;
  __syncthreads();
  const float L = (red[4] + red[5]) + (red[6] + red[7]);
  const float inv = L > 0.0f ? 1.0f / L : 0.0f;
  if (p.D > 128) {
    for (int d = tid; d < p.D; d += 256) {
      float acc = 0.0f;
      for (int i = 0; i < nparts; ++i) {
        const float m = ml[i * 2];
        if (m != -INFINITY) acc = fmaf(expf(m - M), po[(int64_t)i * p.D + d], acc);
      }
      OutE::store(o + d, acc * inv);
    }
    return;
  }
  const int ng = 256 / p.D;
  const int grp = tid / p.D, d = tid % p.D;
  float acc = 0.0f;
  if (grp < ng) {
#pragma unroll 4
    for (int i = grp; i < nparts; i += ng) {
      const float m = ml[i * 2];
      const float w = m != -INFINITY ? expf(m - M) : 0.0f;
      acc = fmaf(w, po[(int64_t)i * p.D + d], acc);
    }
  }
  part_acc[tid] = acc;
  __syncthreads();
  if (tid < p.D) {
    float s = 0.0f;
    for (int g = 0; g < ng; ++g) s += part_acc[g * p.D + tid];
    OutE::store(o + tid, s * inv);
  }
}

template <int QT, int KT>
int32_t launch_generic_t(const DecodeParams& p, hipStream_t stream) {
  const dim3 grid(p.max_parts, p.Hkv, p.B);
  const size_t lds = generic_lds_bytes(p.G, p.D, p.PT, p.bs);
  if (lds > 64 * 1024) {
    set_error("generic decode needs %zu bytes of LDS (G=%d, D=%d, partition=%d); use a smaller partition",
              lds, p.G, p.D, p.PT);
    return CF_ERR_UNSUPPORTED;
  }
  if (p.max_parts == 1) {
    ProfileScope prof("cf_decode_generic", stream);
    CF_LAUNCH((decode_generic_kernel<QT, KT, true>), grid, dim3(kGenericThreads), lds, stream, p);
  } else {
    ProfileScope prof("cf_decode_generic", stream);
    CF_LAUNCH((decode_generic_kernel<QT, KT, false>), grid, dim3(kGenericThreads), lds, stream, p);
  }
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

template <int QT>
int32_t launch_generic_q(const DecodeParams& p, int kv_dt, hipStream_t stream) {
  switch (kv_dt) {
    case kF32: return launch_generic_t<QT, kF32>(p, stream);
    case kF16: return launch_generic_t<QT, kF16>(p, stream);
    case kBF16: return launch_generic_t<QT, kBF16>(p, stream);
    case kE4M3: return launch_generic_t<QT, kE4M3>(p, stream);
  }
  set_error("unsupported KV dtype %d", kv_dt);
  return CF_ERR_UNSUPPORTED;
}

}  // namespace

int32_t launch_decode_generic(const DecodeParams& p, int q_dt, int kv_dt, hipStream_t stream) {
  switch (q_dt) {
    case kF32: return launch_generic_q<kF32>(p, kv_dt, stream);
    case kF16: return launch_generic_q<kF16>(p, kv_dt, stream);
    case kBF16: return launch_generic_q<kBF16>(p, kv_dt, stream);
  }
  set_error("unsupported q dtype %d", q_dt);
  return CF_ERR_UNSUPPORTED;
}

size_t generic_lds_bytes(int64_t G, int64_t D, int64_t PT, int64_t bs) {
  // q [G][D], scores [G][PT], block ids [PT / bs] (even), (m, l) [G][2], P.V sums [256]
  return (size_t)(G * D + G * PT + ((PT / bs + 1) & ~1) + 2 * G + kGenericThreads) * 4;
}

int32_t launch_decode_reduce(const DecodeParams& p, int q_dt, hipStream_t stream) {
  const dim3 grid(p.Hq, p.B);
  const int threads = 256;
  ProfileScope prof("cf_decode_reduce", stream);
  switch (q_dt) {
    case kF32: CF_LAUNCH((decode_reduce_kernel<kF32>), grid, dim3(threads), 0, stream, p); break;
    case kF16: CF_LAUNCH((decode_reduce_kernel<kF16>), grid, dim3(threads), 0, stream, p); break;
    case kBF16: CF_LAUNCH((decode_reduce_kernel<kBF16>), grid, dim3(threads), 0, stream, p); break;
    default: set_error("unsupported output dtype %d", q_dt); return CF_ERR_UNSUPPORTED;
  }
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

}  // namespace cf
