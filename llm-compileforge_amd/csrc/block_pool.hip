// Paged KV block pool: reference-counted physical blocks, per-request block
// tables, copy-on-write of shared blocks at write time, and a device-resident
// int32 block table kept current by small delta scatters.
//
// Pool semantics follow the reference's BlockManager
// (runtime/src/cache/block.rs:78-352, exposed to Python as PyBlockManager,
// runtime/src/lib.rs:82-168), including its allocation order: the free list
// is a stack initialised to 0..n-1 and blocks are taken from its end and
// returned to its end.  Added here:
//
//  * prepare_writes: before new tokens are written, make every block the
//    write touches exclusively owned.  A block whose reference count is
//    above one (a prefix shared with another request or held by the radix
//    cache, possibly a partial last block) is replaced in the writer's table
//    by a fresh block, and the pair (old, new) is returned for a device copy
//    of the old block's rows.  Returns each new token's slot (block * bs +
//    offset) for the write kernel.
//  * Device rows: each request gets a row of a device table [rows, cols]
//    and of a length vector [rows]; table_deltas lists the (row, col, value)
//    cells that changed since the last call (col = -1: the row's length) for
//    cf_block_tables_apply to scatter, instead of re-uploading every table
//    each step.
//  * shared_prefix_lens over the rows, the statement the decode kernel takes
//    (leading tokens a row shares, same physical blocks, with the row before).
#include <algorithm>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "cf_host.hpp"

namespace cf {

namespace {

constexpr int32_t kClean = INT32_MAX;

struct Req {
  std::vector<int32_t> table;
  int64_t len = 0;                // tokens (prepare_writes / set_len): the device row length
  int32_t row = -1;               // device row, -1 before its first delta
  int32_t dirty_from = kClean;    // lowest table index changed since the last deltas
  bool len_dirty = false;
  bool queued = false;            // in Pool::dirty
  uint64_t stamp = 0;             // duplicate check in prepare_writes
};

struct Pool {
  int64_t num_blocks = 0, block_size = 0;
  std::vector<int64_t> rc;          // reference count per block
  std::vector<int32_t> free_list;   // stack: back() is allocated next
  std::unordered_map<std::string, std::unique_ptr<Req>> reqs;
  uint64_t stamp = 0;
  // device rows
  int32_t rows = 0, cols = 0;
  std::vector<int32_t> free_rows;                  // stack, back() first
  std::vector<std::vector<int32_t>> mirror;        // per row: the device table cells written so far
  std::vector<int64_t> mirror_len;                 // per row: the device length
  std::vector<Req*> dirty;                         // requests with changes not yet in a delta
  std::vector<int32_t> released_rows;              // rows of freed requests, length to zero

  int64_t free_count() const { return (int64_t)free_list.size(); }
  int64_t ceil_blocks(int64_t tokens) const { return (tokens + block_size - 1) / block_size; }

  int32_t pop_block() {
    const int32_t b = free_list.back();
    free_list.pop_back();
    rc[b] += 1;
    return b;
  }

  Req* find(const char* id) {
    auto it = reqs.find(id);
    return it == reqs.end() ? nullptr : it->second.get();
  }

  Req* get_or_make(const char* id) {
    auto& r = reqs[id];
    if (!r) r.reset(new Req());
    return r.get();
  }

  void touch(Req* r, int32_t from, bool len_changed) {
    if (rows == 0) return;
    r->dirty_from = std::min(r->dirty_from, from);
    r->len_dirty |= len_changed;
    if (!r->queued) {
      r->queued = true;
      dirty.push_back(r);
    }
  }
};

Pool* pool_of(void* h) { return static_cast<Pool*>(h); }

int32_t out_of_blocks(const Pool* p, int64_t needed) {
  set_error("OutOfMemory: need %lld blocks but only %lld free (total pool: %lld)", (long long)needed,
            (long long)p->free_count(), (long long)p->num_blocks);
  return CF_ERR_OUT_OF_BLOCKS;
}

int32_t copy_ids(const std::vector<int32_t>& ids, int32_t* out, int64_t cap, int64_t* n_out) {
  if (n_out) *n_out = (int64_t)ids.size();
  if (out == nullptr) return CF_OK;
  CF_CHECK((int64_t)ids.size() <= cap, "output holds %lld ids, %lld needed", (long long)cap,
           (long long)ids.size());
  std::memcpy(out, ids.data(), ids.size() * sizeof(int32_t));
  return CF_OK;
}

}  // namespace

// ---- device kernels ----------------------------------------------------------

namespace {

__global__ __launch_bounds__(256) void table_apply_kernel(int32_t* table, int64_t t_sr, int64_t t_sc, int32_t* lens,
                                                          int64_t l_s, const int32_t* deltas, int64_t d_sr,
                                                          int64_t d_sc, int64_t n, int64_t R, int64_t C) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int32_t* d = deltas + i * d_sr;
  const int64_t row = d[0], col = d[d_sc], val = d[2 * d_sc];
  if (row < 0 || row >= R) return;
  if (col < 0) {
    lens[row * l_s] = (int32_t)val;
  } else if (col < C) {
    table[row * t_sr + col * t_sc] = (int32_t)val;
  }
}

// One workgroup copies one 16-byte-aligned piece of a block per pair.
__global__ __launch_bounds__(256) void copy_blocks_kernel(char* base, int64_t block_stride, int64_t block_bytes,
                                                          const int32_t* pairs, int64_t p_sr, int64_t p_sc,
                                                          int64_t NB, bool vec) {
  const int64_t pr = blockIdx.y;
  const int64_t src = pairs[pr * p_sr], dst = pairs[pr * p_sr + p_sc];
  if (src < 0 || src >= NB || dst < 0 || dst >= NB || src == dst) return;
  const char* s = base + src * block_stride;
  char* d = base + dst * block_stride;
  if (vec) {
    const int64_t n16 = block_bytes / 16;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
      ((uint4*)d)[i] = ((const uint4*)s)[i];
  } else {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < block_bytes; i += (int64_t)gridDim.x * 256)
      d[i] = s[i];
  }
}

}  // namespace

}  // namespace cf

using namespace cf;

extern "C" {

int32_t cf_bp_create(int64_t num_blocks, int64_t block_size, void** out) {
  CF_CHECK(out != nullptr, "out is NULL");
  *out = nullptr;
  CF_CHECK(num_blocks > 0, "num_blocks must be positive");
  CF_CHECK(block_size > 0, "block_size must be positive");
  CF_CHECK(num_blocks <= (int64_t)INT32_MAX, "num_blocks must fit int32");
  Pool* p = new Pool();
  p->num_blocks = num_blocks;
  p->block_size = block_size;
  p->rc.assign(num_blocks, 0);
  p->free_list.resize(num_blocks);
  for (int64_t i = 0; i < num_blocks; ++i) p->free_list[i] = (int32_t)i;
  *out = p;
  return CF_OK;
}

int32_t cf_bp_destroy(void* h) {
  delete pool_of(h);
  return CF_OK;
}

int32_t cf_bp_num_free(void* h, int64_t* out) {
  CF_CHECK(h && out, "NULL argument");
  *out = pool_of(h)->free_count();
  return CF_OK;
}

int32_t cf_bp_ref_count(void* h, int64_t block_id, int64_t* out) {
  CF_CHECK(h && out, "NULL argument");
  Pool* p = pool_of(h);
  *out = (block_id >= 0 && block_id < p->num_blocks) ? p->rc[block_id] : 0;
  return CF_OK;
}

int32_t cf_bp_allocate(void* h, const char* rid, int64_t num_tokens, int32_t* out, int64_t cap, int64_t* n_out) {
  CF_CHECK(h && rid, "NULL argument");
  CF_CHECK(num_tokens >= 0, "num_tokens must be non-negative");
  Pool* p = pool_of(h);
  if (p->find(rid)) return out_of_blocks(p, 0);  // the reference reports a duplicate id this way
  const int64_t needed = p->ceil_blocks(num_tokens);
  if (needed > p->free_count()) return out_of_blocks(p, needed);
  CF_CHECK(out == nullptr || needed <= cap, "output holds %lld ids, %lld needed", (long long)cap,
           (long long)needed);
  Req* r = p->get_or_make(rid);
  r->table.reserve(needed);
  for (int64_t i = 0; i < needed; ++i) r->table.push_back(p->pop_block());
  p->touch(r, 0, false);
  return copy_ids(r->table, out, cap, n_out);
}

int32_t cf_bp_free(void* h, const char* rid) {
  CF_CHECK(h && rid, "NULL argument");
  Pool* p = pool_of(h);
  auto it = p->reqs.find(rid);
  if (it == p->reqs.end()) return CF_OK;
  Req* r = it->second.get();
  for (int32_t bid : r->table) {
    if (bid < 0 || bid >= p->num_blocks) continue;
    const int64_t rc = p->rc[bid] > 0 ? p->rc[bid] - 1 : 0;
    p->rc[bid] = rc;
    if (rc == 0) p->free_list.push_back(bid);
  }
  if (r->row >= 0) {
    p->released_rows.push_back(r->row);
    p->free_rows.push_back(r->row);
  }
  if (r->queued) p->dirty.erase(std::remove(p->dirty.begin(), p->dirty.end(), r), p->dirty.end());
  p->reqs.erase(it);
  return CF_OK;
}

int32_t cf_bp_free_block(void* h, int64_t bid) {
  CF_CHECK(h, "NULL argument");
  Pool* p = pool_of(h);
  if (bid < 0 || bid >= p->num_blocks) return CF_OK;
  const int64_t rc = p->rc[bid] > 0 ? p->rc[bid] - 1 : 0;
  p->rc[bid] = rc;
  if (rc == 0) p->free_list.push_back((int32_t)bid);
  return CF_OK;
}

int32_t cf_bp_increment_ref_count(void* h, int64_t bid) {
  CF_CHECK(h, "NULL argument");
  Pool* p = pool_of(h);
  if (bid >= 0 && bid < p->num_blocks) p->rc[bid] += 1;
  return CF_OK;
}

int32_t cf_bp_assign_cached_blocks(void* h, const char* rid, const int32_t* ids, int64_t n) {
  CF_CHECK(h && rid && (ids || n == 0), "NULL argument");
  Pool* p = pool_of(h);
  for (int64_t i = 0; i < n; ++i)
    if (ids[i] >= 0 && ids[i] < p->num_blocks) p->rc[ids[i]] += 1;
  Req* r = p->get_or_make(rid);
  r->table.insert(r->table.begin(), ids, ids + n);
  p->touch(r, 0, false);
  return CF_OK;
}

int32_t cf_bp_ensure_blocks(void* h, const char* rid, int64_t target_tokens) {
  CF_CHECK(h && rid, "NULL argument");
  CF_CHECK(target_tokens >= 0, "target_tokens must be non-negative");
  Pool* p = pool_of(h);
  Req* r0 = p->find(rid);
  const int64_t existing = r0 ? (int64_t)r0->table.size() * p->block_size : 0;
  if (existing >= target_tokens) return CF_OK;
  const int64_t extra = p->ceil_blocks(target_tokens - existing);
  if (extra > p->free_count()) return out_of_blocks(p, extra);
  Req* r = p->get_or_make(rid);
  const int32_t from = (int32_t)r->table.size();
  for (int64_t i = 0; i < extra; ++i) r->table.push_back(p->pop_block());
  p->touch(r, from, false);
  return CF_OK;
}

int32_t cf_bp_share_prefix(void* h, const char* src, const char* dst, int64_t prefix_len, int32_t* out, int64_t cap,
                           int64_t* n_out) {
  CF_CHECK(h && src && dst, "NULL argument");
  Pool* p = pool_of(h);
  Req* s = p->find(src);
  if (!s) {
    set_error("Source request '%s' not found", src);
    return CF_ERR_NOT_FOUND;
  }
  CF_CHECK(!p->find(dst), "Destination request '%s' already has blocks", dst);
  CF_CHECK(prefix_len >= 0, "prefix_len must be non-negative");
  const int64_t nb = p->ceil_blocks(prefix_len);
  CF_CHECK(nb <= (int64_t)s->table.size(),
           "Source has %lld blocks, cannot share %lld (prefix_len=%lld, block_size=%lld)",
           (long long)s->table.size(), (long long)nb, (long long)prefix_len, (long long)p->block_size);
  CF_CHECK(out == nullptr || nb <= cap, "output holds %lld ids, %lld needed", (long long)cap, (long long)nb);
  std::vector<int32_t> shared(s->table.begin(), s->table.begin() + nb);
  for (int32_t bid : shared) p->rc[bid] += 1;
  Req* d = p->get_or_make(dst);
  d->table = shared;
  p->touch(d, 0, false);
  return copy_ids(shared, out, cap, n_out);
}

int32_t cf_bp_get_blocks(void* h, const char* rid, int32_t* out, int64_t cap, int64_t* n_out) {
  CF_CHECK(h && rid, "NULL argument");
  Pool* p = pool_of(h);
  Req* r = p->find(rid);
  if (!r) {
    set_error("Unknown request_id: %s", rid);
    return CF_ERR_NOT_FOUND;
  }
  return copy_ids(r->table, out, cap, n_out);
}

// Makes the blocks holding positions [start[i], start[i] + count[i]) of each
// request exclusively its own and returns the tokens' slots.  Per request,
// in order: the table grows to cover the write (blocks taken from the free
// list), then every touched block with a reference count above one is
// replaced, lowest position first, by a fresh block; (old, new) goes to
// `copies`.  All-or-nothing: if the free list cannot cover every request,
// nothing changes.  slots: sum(count) entries, request by request.
int32_t cf_bp_prepare_writes(void* h, int64_t n_req, const char* const* rids, const int64_t* start,
                             const int64_t* count, int64_t* slots, int32_t* copies, int64_t copies_cap,
                             int64_t* n_copies) {
  CF_CHECK(h && (n_req == 0 || (rids && start && count)), "NULL argument");
  Pool* p = pool_of(h);
  const int64_t bs = p->block_size;
  std::vector<Req*> rq(n_req, nullptr);
  // pass 1: blocks needed (growth + copy-on-write), nothing changed yet
  int64_t need = 0, ncopy = 0, nslots = 0;
  const uint64_t stamp = ++p->stamp;
  for (int64_t i = 0; i < n_req; ++i) {
    CF_CHECK(rids[i] != nullptr, "request id %lld is NULL", (long long)i);
    CF_CHECK(start[i] >= 0 && count[i] >= 0, "request %s: start and count must be non-negative", rids[i]);
    Req* r = p->find(rids[i]);
    if (r) {
      CF_CHECK(r->stamp != stamp, "request %s listed twice", rids[i]);
      r->stamp = stamp;
    }
    rq[i] = r;
    if (count[i] == 0) continue;
    nslots += count[i];
    const int64_t have = r ? (int64_t)r->table.size() : 0;
    const int64_t want = p->ceil_blocks(start[i] + count[i]);
    if (want > have) need += want - have;
    for (int64_t j = start[i] / bs; j < std::min(want, have); ++j) {
      const int32_t bid = r->table[j];
      if (bid >= 0 && bid < p->num_blocks && p->rc[bid] > 1) {
        ++need;
        ++ncopy;
      }
    }
  }
  {
    // requests not yet known may appear twice
    std::vector<const char*> fresh;
    for (int64_t i = 0; i < n_req; ++i)
      if (!rq[i]) fresh.push_back(rids[i]);
    std::sort(fresh.begin(), fresh.end(), [](const char* a, const char* b) { return std::strcmp(a, b) < 0; });
    for (size_t i = 1; i < fresh.size(); ++i)
      CF_CHECK(std::strcmp(fresh[i - 1], fresh[i]) != 0, "request %s listed twice", fresh[i]);
  }
  if (need > p->free_count()) return out_of_blocks(p, need);
  CF_CHECK(copies == nullptr || ncopy <= copies_cap, "copies holds %lld pairs, %lld needed",
           (long long)copies_cap, (long long)ncopy);
  CF_CHECK(ncopy == 0 || copies != nullptr, "copy-on-write needed but no copies buffer given");
  CF_CHECK(nslots == 0 || slots != nullptr, "slots is NULL");
  // pass 2: apply
  int64_t c = 0, s = 0;
  for (int64_t i = 0; i < n_req; ++i) {
    if (count[i] == 0) continue;
    Req* r = rq[i] ? rq[i] : p->get_or_make(rids[i]);
    auto& table = r->table;
    const int64_t want = p->ceil_blocks(start[i] + count[i]);
    const int64_t have = (int64_t)table.size();
    int32_t from = kClean;
    if (want > have) from = (int32_t)have;
    for (int64_t j = have; j < want; ++j) table.push_back(p->pop_block());
    for (int64_t j = start[i] / bs; j < have && j < want; ++j) {
      const int32_t old = table[j];
      if (old < 0 || old >= p->num_blocks || p->rc[old] <= 1) continue;
      const int32_t fresh = p->pop_block();
      p->rc[old] -= 1;
      table[j] = fresh;
      copies[2 * c] = old;
      copies[2 * c + 1] = fresh;
      ++c;
      from = std::min(from, (int32_t)j);
    }
    for (int64_t t = 0; t < count[i]; ++t) {
      const int64_t pos = start[i] + t;
      slots[s++] = (int64_t)table[pos / bs] * bs + pos % bs;
    }
    const int64_t end = start[i] + count[i];
    const bool grew = end > r->len;
    if (grew) r->len = end;
    if (from != kClean || grew) p->touch(r, from, grew);
  }
  if (n_copies) *n_copies = c;
  return CF_OK;
}

int32_t cf_bp_set_len(void* h, const char* rid, int64_t tokens) {
  CF_CHECK(h && rid, "NULL argument");
  CF_CHECK(tokens >= 0, "tokens must be non-negative");
  Pool* p = pool_of(h);
  Req* r = p->find(rid);
  if (!r) {
    set_error("Unknown request_id: %s", rid);
    return CF_ERR_NOT_FOUND;
  }
  if (r->len != tokens) {
    r->len = tokens;
    p->touch(r, kClean, true);
  }
  return CF_OK;
}

int32_t cf_bp_bind_rows(void* h, int32_t rows, int32_t cols) {
  CF_CHECK(h, "NULL argument");
  CF_CHECK(rows > 0 && cols > 0, "rows and cols must be positive");
  Pool* p = pool_of(h);
  CF_CHECK(p->rows == 0, "device rows are already bound");
  p->rows = rows;
  p->cols = cols;
  p->mirror.assign(rows, {});
  p->mirror_len.assign(rows, 0);
  p->free_rows.resize(rows);
  for (int32_t r = 0; r < rows; ++r) p->free_rows[r] = rows - 1 - r;  // row 0 first
  for (auto& kv : p->reqs) p->touch(kv.second.get(), 0, true);
  return CF_OK;
}

int32_t cf_bp_row_of(void* h, const char* rid, int32_t* row) {
  CF_CHECK(h && rid && row, "NULL argument");
  Req* r = pool_of(h)->find(rid);
  *row = r ? r->row : -1;
  return CF_OK;
}

// Cells of the device table and lengths that differ from what the device
// holds: deltas [n][4] = {row, col, value, 0}, col = -1 for a length.  A
// request gets a row at its first delta (the lowest free one); a freed
// request's row gets length 0.  *n_out always receives the count; with a
// NULL or too short buffer nothing is consumed (the latter also fails).
// Raises if a table outgrows `cols` or the rows run out.  The device table
// must start filled with -1 and lengths with 0.
int32_t cf_bp_table_deltas(void* h, int32_t* deltas, int64_t cap, int64_t* n_out) {
  CF_CHECK(h && n_out, "NULL argument");
  Pool* p = pool_of(h);
  CF_CHECK(p->rows > 0, "cf_bp_bind_rows first");
  // plan (no change to the pool): rows for new requests, the cells and lengths to send
  std::vector<int32_t> out;
  std::vector<int32_t> zeroed;
  for (int32_t r : p->released_rows)
    if (p->mirror_len[r] != 0) zeroed.push_back(r);
  auto emit = [&](int32_t row, int32_t col, int32_t v) {
    out.push_back(row);
    out.push_back(col);
    out.push_back(v);
    out.push_back(0);
  };
  for (int32_t r : zeroed) emit(r, -1, 0);
  std::vector<int32_t> row_for(p->dirty.size());
  size_t taken = 0;
  for (size_t k = 0; k < p->dirty.size(); ++k) {
    const Req* r = p->dirty[k];
    CF_CHECK((int64_t)r->table.size() <= p->cols, "a request holds %lld blocks, device rows hold %d",
             (long long)r->table.size(), p->cols);
    int32_t row = r->row, from = r->dirty_from;
    if (row < 0) {
      CF_CHECK(taken < p->free_rows.size(), "device rows exhausted (%d rows)", p->rows);
      row = p->free_rows[p->free_rows.size() - 1 - taken++];
      from = 0;
    }
    row_for[k] = row;
    const auto& mir = p->mirror[row];
    const int32_t ncell = std::max((int32_t)r->table.size(), (int32_t)mir.size());
    for (int32_t j = std::min(from, ncell); j < ncell; ++j) {
      const int32_t want = j < (int32_t)r->table.size() ? r->table[j] : -1;
      const int32_t have = j < (int32_t)mir.size() ? mir[j] : -1;
      if (want != have) emit(row, j, want);
    }
    const bool was_zeroed = std::find(zeroed.begin(), zeroed.end(), row) != zeroed.end();
    const int64_t dev_len = was_zeroed ? 0 : p->mirror_len[row];
    if (r->len != dev_len) emit(row, -1, (int32_t)r->len);
  }
  const int64_t n = (int64_t)out.size() / 4;
  *n_out = n;
  if (deltas == nullptr) return CF_OK;  // size query
  CF_CHECK(n <= cap, "deltas holds %lld entries, %lld needed", (long long)cap, (long long)n);
  std::memcpy(deltas, out.data(), out.size() * sizeof(int32_t));
  // commit: the device will hold exactly this
  for (int32_t r : zeroed) p->mirror_len[r] = 0;
  p->released_rows.clear();
  p->free_rows.resize(p->free_rows.size() - taken);
  for (size_t k = 0; k < p->dirty.size(); ++k) {
    Req* r = p->dirty[k];
    const int32_t row = row_for[k];
    const int32_t from = r->row < 0 ? 0 : r->dirty_from;
    r->row = row;
    auto& mir = p->mirror[row];
    if (mir.size() < r->table.size()) mir.resize(r->table.size(), -1);
    for (int32_t j = std::min(from, (int32_t)mir.size()); j < (int32_t)mir.size(); ++j)
      mir[j] = j < (int32_t)r->table.size() ? r->table[j] : -1;
    p->mirror_len[row] = r->len;
    r->dirty_from = kClean;
    r->len_dirty = false;
    r->queued = false;
  }
  p->dirty.clear();
  return CF_OK;
}

// Per device row r (0 .. rows-1): the leading tokens row r holds in the same
// physical blocks as row r - 1, capped by both rows' lengths (0 for row 0
// and for rows without a request), from the host tables.
int32_t cf_bp_shared_prefix_lens(void* h, int32_t* out, int64_t n) {
  CF_CHECK(h && out, "NULL argument");
  Pool* p = pool_of(h);
  CF_CHECK(p->rows > 0 && n == p->rows, "out must hold %d rows", p->rows);
  std::vector<const Req*> at(p->rows, nullptr);
  for (auto& kv : p->reqs)
    if (kv.second->row >= 0) at[kv.second->row] = kv.second.get();
  out[0] = 0;
  for (int32_t r = 1; r < p->rows; ++r) {
    out[r] = 0;
    if (!at[r] || !at[r - 1]) continue;
    const auto& a = at[r - 1]->table;
    const auto& b = at[r]->table;
    size_t j = 0;
    while (j < a.size() && j < b.size() && a[j] == b[j]) ++j;
    out[r] = (int32_t)std::max<int64_t>(0, std::min({(int64_t)j * p->block_size, at[r - 1]->len, at[r]->len}));
  }
  return CF_OK;
}

int32_t cf_block_tables_apply(CfTensor* table, CfTensor* lens, const CfTensor* deltas, void* stream) {
  View vt, vl, vd;
  int32_t rc;
  if ((rc = view_of(table, "table", 2, &vt))) return rc;
  if ((rc = view_of(lens, "lens", 1, &vl))) return rc;
  if ((rc = view_of(deltas, "deltas", 2, &vd))) return rc;
  CF_CHECK(vt.dtype == CF_I32 && vl.dtype == CF_I32 && vd.dtype == CF_I32, "table, lens and deltas must be i32");
  CF_CHECK(vl.size[0] == vt.size[0], "lens must have one entry per table row");
  CF_CHECK(vd.size[1] == 4, "deltas must be [n, 4]");
  const int64_t n = vd.size[0];
  if (n == 0) return CF_OK;
  ProfileScope prof("cf_block_tables_apply", (hipStream_t)stream);
  CF_LAUNCH(table_apply_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     (int32_t*)vt.base, vt.stride[0], vt.stride[1], (int32_t*)vl.base, vl.stride[0],
                     (const int32_t*)vd.base, vd.stride[0], vd.stride[1], n, vt.size[0], vt.size[1]);
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

int32_t cf_copy_blocks(CfTensor* cache, const CfTensor* pairs, void* stream) {
  View vc, vp;
  int32_t rc;
  if ((rc = view_of(cache, "cache", 2, &vc))) return rc;
  if ((rc = view_of(pairs, "pairs", 2, &vp))) return rc;
  CF_CHECK(vp.dtype == CF_I32 && vp.size[1] == 2, "pairs must be i32 [n, 2]");
  CF_CHECK(vc.stride[1] == 1 || vc.size[1] <= 1, "cache: each block's elements must be contiguous ([NB, E], E stride 1)");
  CF_CHECK(vc.stride[0] >= vc.size[1], "cache: blocks overlap");
  const int64_t n = vp.size[0];
  if (n == 0 || vc.size[1] == 0) return CF_OK;
  CF_CHECK(n < 65536, "at most 65535 pairs per call");
  const int64_t eb = vc.elem;
  const int64_t bytes = vc.size[1] * eb, stride = vc.stride[0] * eb;
  const bool vec = ((uintptr_t)vc.base % 16 == 0) && bytes % 16 == 0 && stride % 16 == 0;
  const int64_t per = vec ? bytes / 16 : bytes;
  const unsigned gx = (unsigned)std::min<int64_t>(std::max<int64_t>((per + 255) / 256, 1), 64);
  ProfileScope prof("cf_copy_blocks", (hipStream_t)stream);
  CF_LAUNCH(copy_blocks_kernel, dim3(gx, (unsigned)n), dim3(256), 0, (hipStream_t)stream, vc.base, stride,
                     bytes, (const int32_t*)vp.base, vp.stride[0], vp.stride[1], vc.size[0], vec);
  CF_HIP_CHECK(hipGetLastError());
  return CF_OK;
}

}  // extern "C"
