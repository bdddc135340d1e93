/*
 * cf_hip.h -- C ABI of libcf_hip.so: paged decode attention over a paged
 * KV cache (bf16 / fp32 / OCP FP8 e4m3) and FP8 KV quantization on MI355X
 * (gfx950).
 *
 * Conventions (all entry points):
 *   - Return 0 on success and a negative CF_ERR_* code on failure; the
 *     message is kept per thread and read with cf_last_error().  Nothing is
 *     thrown across the ABI.
 *   - Tensors are CfTensor: an SFATensor (include/sfa.h, layout of the
 *     reference include/sfa.h:54-99) plus a dtype code.  Strides are in
 *     elements.  Device memory carries device = SFA_ROCM.
 *   - The caller owns every buffer, including outputs and workspace.  The
 *     library never frees caller memory and allocates nothing on these
 *     paths.
 *   - Work is enqueued on `stream` (a hipStream_t; NULL = the legacy
 *     default stream) and the calls return without synchronizing.
 *     Calls are reentrant.
 *   - Everything a kernel assumes about shapes, dtypes, strides and ranges
 *     that can be checked on the host is checked before any launch.
 */
#ifndef CF_HIP_H
#define CF_HIP_H

#include <stdint.h>

#include "sfa.h"

#ifdef __cplusplus
extern "C" {
#endif

#define CF_ABI_VERSION 1

/* dtype codes: 0..6 follow the reference's SfaConstant.dtype_code numbering
 * (reference include/sfa_abi.proto:86); 7 is added for OCP FP8 e4m3fn. */
typedef enum {
    CF_F32 = 0,
    CF_F16 = 1,
    CF_BF16 = 2,
    CF_I64 = 3,
    CF_I32 = 4,
    CF_I8 = 5,
    CF_U8 = 6,
    CF_F8E4M3FN = 7,
} CfDtype;

typedef struct {
    SFATensor t;
    int32_t dtype; /* CfDtype */
    int32_t reserved;
} CfTensor;

enum {
    CF_OK = 0,
    CF_ERR_INVALID = -1,     /* bad argument: shape, dtype, stride, range  */
    CF_ERR_HIP = -2,         /* a HIP runtime call failed                  */
    CF_ERR_WORKSPACE = -3,   /* workspace missing or too small             */
    CF_ERR_UNSUPPORTED = -4, /* valid request this build does not handle   */
    CF_ERR_OUT_OF_BLOCKS = -5, /* block pool exhausted                     */
    CF_ERR_NOT_FOUND = -6,   /* unknown request id                         */
};

/* ABI version of the loaded library (compare with CF_ABI_VERSION).
 * Counterpart of the reference's SFA_VERSION (compiler/sfa_abi.py:32-33). */
int32_t cf_abi_version(void);

/* Copies the calling thread's last error message into buf (NUL-terminated,
 * truncated to len) and returns the full message length. */
int32_t cf_last_error(char* buf, uint64_t len);

/* Workspace needed by cf_paged_decode (on the current device) for a batch
 * whose block tables hold at most max_blocks_per_seq entries.  Replaces no
 * reference function: the reference decode (kernels/paged_attention.py
 * :21-73) gathers into temporaries; this path splits long contexts across
 * waves and merges (m, l, o) partials instead. */
int32_t cf_paged_decode_workspace_bytes(int64_t batch, int64_t num_q_heads,
                                        int64_t num_kv_heads,
                                        int64_t head_dim,
                                        int64_t max_blocks_per_seq,
                                        int32_t block_size,
                                        int32_t partition_tokens,
                                        uint64_t* bytes_out);

/* Paged decode attention, one query token per sequence.
 * Replaces paged_attention / _paged_attention_cpu
 * (reference kernels/paged_attention.py:200-227, :21-73).
 *
 *   q            [B, Hq, D]            f32 | f16 | bf16, D stride 1
 *   k_cache      [NB, bs, Hkv, D]      f32 | f16 | bf16 | e4m3fn, any strides
 *   v_cache      [NB, bs, Hkv, D]      same dtype as k_cache, any strides
 *   block_tables [B, Mb]               i32, physical block ids
 *   seq_lens     [B]                   i32
 *   k_scale,     [Hkv] or [1]          f32 dequant scales (e4m3fn caches
 *   v_scale                            only; NULL otherwise)
 *   scale        softmax scale (the reference default 1/sqrt(D) is applied
 *                by the caller)
 *   out          [B, Hq, D]            dtype of q
 *
 * Sequence b attends to its first min(seq_lens[b], Mb*bs) tokens, read
 * through block_tables[b]; query head h uses KV head h / (Hq/Hkv).
 * Sequences of length 0 produce zeros.  A block id outside [0, NB)
 * contributes no tokens (the dict-based Python API rejects such tables
 * before the call, as the reference's indexing would).
 *
 * With bf16 q, bf16/e4m3fn caches, bs = 16, head_dim 64 or 128, G <= 16,
 * K rows with unit channel stride and V stored channel-major inside a
 * block (token stride 1: the layout cf_hip.layout calls "native"), one
 * MFMA kernel balances 32-token tiles evenly over all waves of the GPU and
 * a merge kernel combines the sequences split between waves;
 * partition_tokens is unused there.  Other inputs run a generic kernel that
 * splits sequences into partition_tokens partitions (multiple of bs)
 * merged by a log-sum-exp reduce.
 *
 * workspace: cf_paged_decode_workspace_bytes() bytes, 256-byte aligned;
 * calls that share a workspace must not overlap. */
int32_t cf_paged_decode(const CfTensor* q, const CfTensor* k_cache,
                        const CfTensor* v_cache, const CfTensor* block_tables,
                        const CfTensor* seq_lens, const CfTensor* k_scale,
                        const CfTensor* v_scale, float scale,
                        int32_t block_size, int32_t partition_tokens,
                        CfTensor* out, void* workspace,
                        uint64_t workspace_bytes, void* stream);

/* cf_paged_decode with a statement of which sequences share cached
 * prefix blocks (the radix cache's shared prefixes, reference
 * runtime/src/cache/radix.rs:50-177 and block.rs share_prefix:273-306).
 *
 *   shared_prefix_lens  [B] i32, or NULL (then this is cf_paged_decode):
 *       the first shared_prefix_lens[b] tokens of sequence b are stored in
 *       the same physical blocks, in the same table positions, as those of
 *       sequence b - 1 (entry 0 is ignored; values are clipped to both
 *       sequences' lengths; 0 = nothing shared).
 *
 * Results are those of cf_paged_decode on the same tables (up to the
 * rounding of a different summation order).  The MFMA path reads a shared
 * run of whole 32-token tiles once for up to 16/G consecutive sharing
 * sequences instead of once per sequence; other paths ignore the hint.
 * The statement is trusted: a claimed share the tables do not have makes
 * the sharers read the first sharer's blocks (block ids stay range-checked,
 * so no access leaves the cache).  Batches above 2048 sequences ignore it. */
int32_t cf_paged_decode_shared(const CfTensor* q, const CfTensor* k_cache,
                               const CfTensor* v_cache,
                               const CfTensor* block_tables,
                               const CfTensor* seq_lens,
                               const CfTensor* shared_prefix_lens,
                               const CfTensor* k_scale, const CfTensor* v_scale,
                               float scale, int32_t block_size,
                               int32_t partition_tokens, CfTensor* out,
                               void* workspace, uint64_t workspace_bytes,
                               void* stream);

/* No counterpart in the reference.  For callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops or harnesses
 * that forbid hipMalloc): cf_paged_decode_shared with the workspace taken
 * from a fixed scratch array inside the library instead of a caller
 * buffer -- 64 MiB (67,108,864 bytes) per device, held by every GPU the
 * library runs on until the process ends.  Same arguments, results and
 * errors as cf_paged_decode_shared minus the workspace; the caller still
 * passes every input and the output.  A call whose workspace need
 * (cf_paged_decode_workspace_bytes) exceeds the scratch returns
 * CF_ERR_WORKSPACE with the need in the message (the Llama-3-70B shape at
 * batch 128 needs about 26 MB).  Allocates nothing: no hipMalloc, no
 * hipFree.  All calls on one device share its scratch and leave their
 * contents there, so calls that overlap on one device -- on two streams,
 * or from two threads without ordering -- race. */
int32_t cf_paged_decode_shared_noalloc(const CfTensor* q, const CfTensor* k_cache,
                                       const CfTensor* v_cache,
                                       const CfTensor* block_tables,
                                       const CfTensor* seq_lens,
                                       const CfTensor* shared_prefix_lens,
                                       const CfTensor* k_scale,
                                       const CfTensor* v_scale, float scale,
                                       int32_t block_size,
                                       int32_t partition_tokens, CfTensor* out,
                                       void* stream);

/* Workspace needed by cf_prefill_chunk_fp8 (on the current device) for
 * num_q_tokens query rows in num_chunks chunks.  Grows with the query
 * rows (one small record per query block), not with the cached context. */
int32_t cf_prefill_chunk_workspace_bytes(int64_t num_q_tokens, int64_t num_chunks,
                                         int64_t num_q_heads, int64_t num_kv_heads,
                                         int64_t head_dim, int32_t block_size,
                                         uint64_t* bytes_out);

/* Chunked-prefill attention over the paged cache: the chunk step of the
 * reference's scheduler (runtime/src/engine/scheduler.rs:178-226), whose
 * attention the reference states only as the per-row decode of
 * kernels/paged_attention.py:21-73 with the length cut to the row, and
 * dense causal attention (kernels/flash_attention.py:179-202) when nothing
 * is cached.  The chunk's own K/V are in the cache already
 * (cf_kv_write_fp8).
 *
 *   q            [Tq, Hq, D]           bf16 | f16, D stride 1, rows of all
 *                                      chunks
 *   k_cache,     [NB, 16, Hkv, D]      bf16 | f16 | e4m3fn (bf16 q: bf16 or
 *   v_cache                            e4m3fn; f16 q: f16 or e4m3fn), native
 *                                      or paired tiles, or the reference's
 *                                      token-major rows (16-byte aligned)
 *   block_tables [N, Mb]               i32, one row per chunk's sequence
 *   seq_lens     [N]                   i32, tokens of the sequence including
 *                                      the chunk
 *   q_start      [N + 1]               i32, chunk n owns q rows
 *                                      [q_start[n], q_start[n+1])
 *   k_scale, v_scale                   as cf_paged_decode
 *   out          [Tq, Hq, D]           q's dtype
 *
 * Chunk n has L = q_start[n+1] - q_start[n] rows; row i sits at position
 * seq_lens[n] - L + i and attends to cache positions [0, that] (causal:
 * bottom-right aligned), read through block_tables[n] up to Mb*16 tokens.
 * Chunks are taken in order and made disjoint (a chunk starting before the
 * previous one ends starts where it ends).  Rows at negative positions get
 * zeros; rows outside every chunk are not written.  block_size must be 16.
 * Unsupported dtypes/layouts return CF_ERR_UNSUPPORTED (no generic path).
 * workspace: cf_prefill_chunk_workspace_bytes() bytes, 256-byte aligned. */
int32_t cf_prefill_chunk_fp8(const CfTensor* q, const CfTensor* k_cache,
                             const CfTensor* v_cache, const CfTensor* block_tables,
                             const CfTensor* seq_lens, const CfTensor* q_start,
                             const CfTensor* k_scale, const CfTensor* v_scale,
                             float scale, int32_t block_size, CfTensor* out,
                             void* workspace, uint64_t workspace_bytes, void* stream);

/* Per-head FP8 scale: scales[h] = amax/448 over x[:, h, :], clamped below
 * at 1e-12, and 1.0 where amax == 0.  This is
 * FP8KVCacheQuantizer.quantize_block's scale rule (reference
 * compiler/quantize/fp8_kv_cache.py:81-86) applied per KV head.
 *   x       [T, H, Dx] or [S0, S1, H, Dx]  f32 | f16 | bf16
 *   scales  [H]         f32 (output, contiguous) */
int32_t cf_fp8_amax_scale(const CfTensor* x, CfTensor* scales, void* stream);

/* The same per-KV-head scale computation under the name the K/V-cache
 * callers use (quantize_block's scale rule, reference
 * compiler/quantize/fp8_kv_cache.py:81-86, per KV head):
 * scales_out[h] = amax(|x[..., h, :]|) / 448, >= 1e-12, 1.0 for an
 * all-zero head.  Arguments as cf_fp8_amax_scale. */
int32_t cf_kv_amax_scale(const CfTensor* x, CfTensor* scales_out, void* stream);

/* out[t,h,d] = e4m3fn(f32(x[t,h,d]) / scales[h]) with IEEE division and
 * round-to-nearest-even, |v| >= 480 -> NaN code (torch's float8_e4m3fn
 * conversion).  Reference compiler/quantize/fp8_kv_cache.py:89.
 *   x [T,H,Dx] or [S0,S1,H,Dx] f32|f16|bf16; scales [H] or [1] f32;
 *   out: e4m3fn, same shape (any strides) */
int32_t cf_fp8_quantize(const CfTensor* x, const CfTensor* scales,
                        CfTensor* out, void* stream);

/* k_out = e4m3fn(k / k_scales[h]) and v_out = e4m3fn(v / v_scales[h]) in
 * one call: the reference's FP8KVCacheQuantizer.quantize_kv (independent K
 * and V scales, compiler/quantize/fp8_kv_cache.py:107-122) quantizing
 * straight into cache storage.
 *   k, v [S0,S1,H,Dx] (or [T,H,Dx]) f32|f16|bf16, same dtype and shape;
 *   k_scales, v_scales [H] or [1] f32; k_out, v_out e4m3fn, same shape.
 * Codes equal cf_fp8_quantize's for each tensor.  When k, v are [S0,16,H,D]
 * pools with 16-byte rows and the outputs are native-tile K / V views (K
 * rows D bytes apart, V 16-token channel rows, shared block and head strides:
 * the native and paired cache layouts) both are written by one launch, a
 * workgroup per block writing every (block, head) pair whole; otherwise it
 * runs cf_fp8_quantize on each. */
int32_t cf_fp8_quantize_kv(const CfTensor* k, const CfTensor* v,
                           const CfTensor* k_scales, const CfTensor* v_scales,
                           CfTensor* k_out, CfTensor* v_out, void* stream);

/* out[t,h,d] = f32(q[t,h,d]) * scales[h].
 * Reference compiler/quantize/fp8_kv_cache.py:95-105.
 *   q [T,H,Dx] or [S0,S1,H,Dx] e4m3fn; scales [H] or [1] f32;
 *   out: f32, same shape */
int32_t cf_fp8_dequantize(const CfTensor* q, const CfTensor* scales,
                          CfTensor* out, void* stream);

/* Writes new K/V rows into a paged e4m3fn cache, quantizing with the given
 * per-head scales: token i goes to block slot_mapping[i] / bs, offset
 * slot_mapping[i] % bs (reference token placement:
 * python_runtime/engine/cache_manager.py:139-171, _kv_cache.py:68-104);
 * slots < 0 or >= NB * bs are skipped.
 *   k_new, v_new  [T, Hkv, D]       f32 | f16 | bf16
 *   slot_mapping  [T]               i32 | i64
 *   k_cache,      [NB, bs, Hkv, D]  e4m3fn, any strides
 *   v_cache
 *   k_scale,      [Hkv] or [1]      f32
 *   v_scale
 * Slots must be distinct: rows that repeat a slot race, and which one lands
 * is not defined (the reference's sequential loop keeps the last; the
 * engine's CacheManager drops the earlier repeats before it calls here).
 * The caller must not target a block that other sequences share. */
int32_t cf_kv_write_fp8(const CfTensor* k_new, const CfTensor* v_new,
                        const CfTensor* slot_mapping, CfTensor* k_cache,
                        CfTensor* v_cache, const CfTensor* k_scale,
                        const CfTensor* v_scale, void* stream);

/* Writes new rows into one paged tensor (a K or a V cache, any layout):
 * row i goes to block slot_mapping[i] / bs, offset slot_mapping[i] % bs
 * (reference CacheManager.write_paged placement,
 * python_runtime/engine/cache_manager.py:139-171; _kv_cache.py:68-104),
 * converted to the cache dtype (e4m3fn: e4m3fn(f32(x) / scale[h]), the
 * FP8KVCacheQuantizer arithmetic; bf16/f16: round to nearest even).
 * Slots < 0 or >= NB * bs are skipped.
 *   x_new         [T, H, D]        f32 | f16 | bf16
 *   slot_mapping  [T]              i32 | i64
 *   cache         [NB, bs, H, D]   f32 | f16 | bf16 | e4m3fn, any strides
 *   scale         [H] or [1] f32   (e4m3fn caches; NULL otherwise)
 * Slots must be distinct (repeats race; CacheManager keeps the last of
 * each before calling).
 * The caller must not target a slot that another sequence still reads. */
int32_t cf_paged_write(const CfTensor* x_new, const CfTensor* slot_mapping,
                       CfTensor* cache, const CfTensor* scale, void* stream);

/* Gathers the first S tokens of each block table into a dense tensor:
 * out[r, s] = row s % bs of block block_tables[r][s / bs], dequantized
 * (e4m3fn: code * scale[h]) and converted to out's dtype; a table entry
 * outside [0, NB) gives zero rows (pad short tables with -1).  Replaces
 * CacheManager.read_paged / _gather_kv_flat
 * (reference python_runtime/engine/cache_manager.py:173-197,
 * _kv_cache.py:106-132).
 *   cache         [NB, bs, H, D]   f32 | f16 | bf16 | e4m3fn, any strides
 *   block_tables  [R, Mb]          i32
 *   scale         [H] or [1] f32   (e4m3fn caches; NULL otherwise)
 *   out           [R, S, H, D]     f32 | f16 | bf16, any strides */
int32_t cf_paged_gather(const CfTensor* cache, const CfTensor* block_tables,
                        const CfTensor* scale, CfTensor* out, void* stream);

/* Uploads `bytes` (a multiple of 16; both pointers 16-byte aligned) from
 * pinned, mapped host memory (hipHostMalloc, torch pin_memory) to device
 * memory with a kernel on `stream`, so the upload is ordered with the
 * stream's kernels on the compute queue (no copy-engine hand-off between
 * back-to-back calls).  Fails with CF_ERR_INVALID if host_src is not mapped
 * pinned memory or dev_dst is not device memory.  No reference counterpart:
 * the upload of the tables the dict-based paged_attention packs on the host
 * (reference kernels/paged_attention.py:200-227 takes host dicts). */
int32_t cf_stage_from_host(const void* host_src, void* dev_dst, uint64_t bytes, void* stream);

/* ---- Paged block pool (host) ---------------------------------------------
 * Replaces the reference's BlockManager (runtime/src/cache/block.rs:78-352;
 * Python binding PyBlockManager, runtime/src/lib.rs:82-168): reference-
 * counted physical blocks and per-request tables, same allocation order
 * (free list = stack initialised 0..n-1, taken from and returned to its
 * end), same error cases.  Handles are not thread-safe.  List outputs go to
 * caller buffers of `cap` entries; *n_out receives the full count (pass a
 * NULL buffer to query it).  Errors: CF_ERR_OUT_OF_BLOCKS (pool exhausted;
 * also a duplicate id in cf_bp_allocate, as the reference reports it),
 * CF_ERR_NOT_FOUND (unknown request), CF_ERR_INVALID. */
int32_t cf_bp_create(int64_t num_blocks, int64_t block_size, void** out);
int32_t cf_bp_destroy(void* pool);
int32_t cf_bp_num_free(void* pool, int64_t* out);
int32_t cf_bp_ref_count(void* pool, int64_t block_id, int64_t* out);
/* BlockManager::allocate (block.rs:145-173). */
int32_t cf_bp_allocate(void* pool, const char* request_id, int64_t num_tokens,
                       int32_t* out, int64_t cap, int64_t* n_out);
/* BlockManager::free (block.rs:177-196); also releases the request's device row. */
int32_t cf_bp_free(void* pool, const char* request_id);
/* BlockManager::free_block (block.rs:199-210). */
int32_t cf_bp_free_block(void* pool, int64_t block_id);
/* BlockManager::increment_ref_count (block.rs:321-325). */
int32_t cf_bp_increment_ref_count(void* pool, int64_t block_id);
/* BlockManager::assign_cached_blocks (block.rs:214-231). */
int32_t cf_bp_assign_cached_blocks(void* pool, const char* request_id,
                                   const int32_t* block_ids, int64_t n);
/* BlockManager::ensure_blocks (block.rs:235-266). */
int32_t cf_bp_ensure_blocks(void* pool, const char* request_id, int64_t target_tokens);
/* BlockManager::share_prefix (block.rs:271-303). */
int32_t cf_bp_share_prefix(void* pool, const char* src_request_id, const char* dst_request_id,
                           int64_t prefix_len, int32_t* out, int64_t cap, int64_t* n_out);
/* BlockManager::get_blocks (block.rs:307-312). */
int32_t cf_bp_get_blocks(void* pool, const char* request_id, int32_t* out, int64_t cap,
                         int64_t* n_out);
/* No reference counterpart (the reference writes into shared blocks, the
 * hazard of a shared partial block).  For each request i, makes the blocks
 * holding positions [start[i], start[i] + count[i]) its own: the table grows
 * to cover them, then each touched block with reference count > 1 is
 * replaced by a fresh block and (old, new) is appended to copies
 * ([copies_cap][2]) for cf_copy_blocks.  slots (sum of count) receives each
 * token's block * block_size + offset.  All-or-nothing on exhaustion. */
int32_t cf_bp_prepare_writes(void* pool, int64_t n_requests, const char* const* request_ids,
                             const int64_t* start, const int64_t* count, int64_t* slots,
                             int32_t* copies, int64_t copies_cap, int64_t* n_copies);
/* Sets a request's token count (its device row length). */
int32_t cf_bp_set_len(void* pool, const char* request_id, int64_t tokens);
/* Device-resident tables (no reference counterpart; the reference builds
 * tables on the host every step).  cf_bp_bind_rows sizes the device table
 * [rows, cols] (initialised to -1 by the caller) and lengths [rows];
 * cf_bp_table_deltas lists the cells that changed since its last call as
 * [n][4] = {row, col, value, 0} (col = -1: the row's length), assigning a
 * row to each new request and zeroing freed requests' lengths;
 * cf_block_tables_apply scatters them on the device. */
int32_t cf_bp_bind_rows(void* pool, int32_t rows, int32_t cols);
int32_t cf_bp_row_of(void* pool, const char* request_id, int32_t* row);
int32_t cf_bp_table_deltas(void* pool, int32_t* deltas, int64_t cap, int64_t* n_out);
/* Per device row: leading tokens it shares (same physical blocks) with the
 * row before, capped by both lengths -- the decode kernel's shared-prefix
 * statement (cf_paged_decode_shared). */
int32_t cf_bp_shared_prefix_lens(void* pool, int32_t* out, int64_t rows);
int32_t cf_block_tables_apply(CfTensor* table, CfTensor* lens, const CfTensor* deltas,
                              void* stream);
/* Copies whole blocks of a paged cache viewed as [NB, E] (a block's E
 * elements contiguous, E stride 1): block pairs[i][1] <- pairs[i][0], for
 * copy-on-write.  A destination must not be another pair's source. */
int32_t cf_copy_blocks(CfTensor* cache, const CfTensor* pairs, void* stream);

/* Kernel timing hook for benchmarks (no reference counterpart).  While
 * enabled, every kernel this library launches carries a pair of HIP events
 * that hipExtLaunchKernel records at the kernel's start and end on the
 * launch stream; a launch the runtime rejects leaves no record.  Stamping
 * is not free: each stamped launch adds host work and a completion signal,
 * so a stamped pass runs a few us per launch slower than an unstamped one
 * and is no step timing.  Events come from a pool; cf_profile_reserve
 * creates them ahead of a measured pass (an event created inside it costs
 * host time, lets the GPU idle between launches and lengthens the kernels
 * that follow an idle gap).  cf_profile_query synchronizes on the recorded
 * events and returns the summed duration (ms) and launch count of kernels
 * whose name starts with `prefix`; cf_profile_durations writes up to `cap`
 * of those durations (ms, launch order) and their total count. */
int32_t cf_profile_enable(int32_t on);
int32_t cf_profile_reset(void);
int32_t cf_profile_reserve(int64_t events);
int32_t cf_profile_query(const char* prefix, double* total_ms,
                         int64_t* launches);
int32_t cf_profile_durations(const char* prefix, float* ms, int64_t cap,
                             int64_t* launches);

#ifdef __cplusplus
}
#endif

#endif /* CF_HIP_H */
