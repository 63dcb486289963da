// Page accounting of the paged KV arena and the unified pack layout, on the
// host. The packer runs between passes while the previous pass computes, so
// it lives in one C++ call per pack instead of a Python loop per group.
//
// PagePool restates the reference PageArena
// (quail/backends/quail/executor/pages.py:8-275) whose allocation order fixes
// the page ids every block table holds:
//   * the free list is a stack initialised [P-1, ..., 1, 0], so the first
//     allocations take pages 0, 1, 2, ... (pages.py:26);
//   * a key owns the pages it allocates and may borrow the leading pages of
//     a resident key; its table is its borrowed pages, then its own
//     (pages.py:96-98); a page is held once per key whose table names it;
//   * a page goes back on the stack when its last holder releases it, in
//     the order the releasing list names it (pages.py:103-109);
//   * retained keys are evictable, lowest priority first, ties by the order
//     they were retained (pages.py:191-250); the default priority is the
//     key's tokens per page it alone holds.
//
// pack_unified restates the unified causal layout of the reference
// pack_chunk (quail/backends/quail/executor/chunk.py:505-1160: the group
// loop :606-684, the unified pools :913-1054, _PoolBuilder :407-502).
// Each group is [prefix | suffix, suffix, ...]; for the paged causal call a
// group with one suffix whose key's pages cover all its rows is one
// sequence written straight into the key's pages, otherwise the prefix is a
// sequence of its own and each suffix a sequence over the key's full pages
// plus a temporary key's pages, into which the key's partial last page is
// copied first (the tail copy).
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <new>
#include <queue>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "qx_status.h"

namespace {

constexpr int QX_ENOKEY = -2;   // the key is not resident
constexpr int QX_EEXISTS = -3;  // the key is already resident
constexpr int QX_EFULL = -4;    // too few free pages for the pack's temporaries

#define QX_FAIL(code, ...)      \
  do {                          \
    qx::set_error(__VA_ARGS__); \
    return (code);              \
  } while (0)

struct Key {
  std::vector<int32_t> borrowed, owned;
  int64_t tokens = 0;
  uint64_t order = 0;  // allocation order (resident_keys lists keys in it)
  bool pinned = false;
  bool retained = false;
  int64_t alone = 0;     // pages counted in retained_pages while retained
  uint64_t version = 0;  // retention version, 0 when not retained
};

struct Retention {
  double priority;
  uint64_t version;
  int64_t key, alone, tokens;
  bool operator>(const Retention& o) const {
    return priority != o.priority ? priority > o.priority : version > o.version;
  }
};

struct PagePool {
  int64_t num_pages, page;
  std::vector<int32_t> free;  // a stack: back() is the next page handed out
  std::vector<int32_t> holds;
  std::unordered_map<int64_t, Key> keys;
  std::priority_queue<Retention, std::vector<Retention>, std::greater<Retention>> heap;
  int64_t retained_pages = 0;
  uint64_t version = 0;
  uint64_t order = 0;
  int64_t next_temporary = -1;  // temporary keys take negative ids

  int64_t pages_needed(int64_t tokens) const { return (tokens + page - 1) / page; }

  Key* find(int64_t key) {
    auto it = keys.find(key);
    return it == keys.end() ? nullptr : &it->second;
  }

  void take(int64_t n, std::vector<int32_t>& into) {
    for (int64_t i = 0; i < n; ++i) {
      into.push_back(free.back());
      free.pop_back();
    }
  }

  int64_t release(const std::vector<int32_t>& pages) {
    for (int32_t p : pages) holds[p] -= 1;
    int64_t freed = 0;
    for (int32_t p : pages)
      if (holds[p] == 0) {
        free.push_back(p);
        ++freed;
      }
    return freed;
  }

  void forget(Key& k) {
    if (k.retained) retained_pages -= k.alone;
    k.retained = false;
    k.alone = 0;
    k.version = 0;
  }

  // -> pages allocated, or -1 when the free stack is short
  int64_t alloc(int64_t key, int64_t tokens, int64_t capacity, const int32_t* borrowed,
                int64_t n_borrowed) {
    if (n_borrowed > pages_needed(capacity) || n_borrowed * page > tokens) return -2;
    const int64_t need = pages_needed(capacity) - n_borrowed;
    if (need > (int64_t)free.size()) return -1;
    Key k;
    k.borrowed.assign(borrowed, borrowed + n_borrowed);
    take(need, k.owned);
    k.tokens = tokens;
    k.order = ++order;
    for (int32_t p : k.borrowed) holds[p] += 1;
    for (int32_t p : k.owned) holds[p] += 1;
    keys.emplace(key, std::move(k));
    return need;
  }

  int64_t free_key(int64_t key) {
    Key& k = keys.at(key);
    forget(k);
    std::vector<int32_t> all(k.borrowed);
    all.insert(all.end(), k.owned.begin(), k.owned.end());
    keys.erase(key);
    return release(all);
  }

  void retain(int64_t key, bool has_priority, double priority) {
    Key& k = keys.at(key);
    k.pinned = false;
    forget(k);
    int64_t alone = 0;
    for (int32_t p : k.borrowed) alone += holds[p] == 1;
    for (int32_t p : k.owned) alone += holds[p] == 1;
    k.retained = true;
    k.alone = alone;
    retained_pages += alone;
    k.version = ++version;
    if (!has_priority) priority = (double)k.tokens / (double)std::max<int64_t>(1, alone);
    heap.push(Retention{priority, k.version, key, alone, k.tokens});
  }
};

PagePool* pool_of(void* p) { return static_cast<PagePool*>(p); }

// One pack's host arrays (the order of `which` in qx_pack_array).
enum PackArray {
  kIds, kPositions, kFinals, kCuA, kRowsPerAnswer, kSrc, kDst, kTailSrc, kTailDst, kCuQ,
  kUsed, kTable, kSeqPages, kTemporaries, kRowSpans, kSuffixCounts, kFreshKeys, kScalars,
  kNumArrays
};

struct Pack {
  std::vector<int64_t> ids, positions, finals, rows_per_answer, src, dst, tail_src, tail_dst;
  std::vector<int32_t> cu_a, cu_q, used, table;
  std::vector<int64_t> seq_pages, temporaries, row_spans, suffix_counts, fresh_keys;
  // tokens, max_q, max_used, multi-row answers, tail copies present, table width
  std::vector<int64_t> scalars;
};

struct Spec {
  int64_t key, f, start, row0, prefix_end, row1;
  bool fresh;
  int64_t keeps;
  std::vector<int64_t> begins, ends;  // absolute rows of each suffix
};

// a suffix of a document whose last page is partial copies that page's rows
bool remainder_tail_missing(const Spec& s, const std::vector<int32_t>& table, int64_t page) {
  return !s.begins.empty() && s.f % page && s.f / page >= (int64_t)table.size();
}

}  // namespace

extern "C" {

int qx_pages_create(int64_t num_pages, int64_t page_tokens, void** pool) {
  QX_CHECK(pool, "pages_create: null handle");
  QX_CHECK(num_pages >= 0 && num_pages <= INT32_MAX, "pages_create: %lld pages",
           (long long)num_pages);
  QX_CHECK(page_tokens >= 1, "pages_create: page of %lld tokens", (long long)page_tokens);
  PagePool* p = new PagePool();
  p->num_pages = num_pages;
  p->page = page_tokens;
  p->free.resize(num_pages);
  for (int64_t i = 0; i < num_pages; ++i) p->free[i] = (int32_t)(num_pages - 1 - i);
  p->holds.assign(num_pages, 0);
  *pool = p;
  return QX_OK;
}

int qx_pages_destroy(void* pool) {
  delete pool_of(pool);
  return QX_OK;
}

int qx_pages_alloc(void* pool, int64_t key, int64_t tokens, int64_t capacity_tokens,
                   const int32_t* borrowed, int64_t n_borrowed, int64_t* allocated) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p && allocated, "pages_alloc: null pointer");
  if (p->find(key)) QX_FAIL(QX_EEXISTS, "key %lld already resident", (long long)key);
  QX_CHECK(tokens >= 0, "pages_alloc: %lld tokens", (long long)tokens);
  QX_CHECK(capacity_tokens >= tokens, "capacity_tokens must cover logical tokens");
  QX_CHECK(n_borrowed >= 0 && (n_borrowed == 0 || borrowed), "pages_alloc: borrowed pages");
  QX_CHECK(n_borrowed * p->page <= tokens, "a key cannot borrow past its own tokens");
  for (int64_t i = 0; i < n_borrowed; ++i)
    QX_CHECK(borrowed[i] >= 0 && borrowed[i] < p->num_pages && p->holds[borrowed[i]] > 0,
             "pages_alloc: borrowed page %d is not held by a resident key", (int)borrowed[i]);
  *allocated = p->alloc(key, tokens, capacity_tokens, borrowed, n_borrowed);
  return QX_OK;
}

int qx_pages_shared(void* pool, int64_t parent, int64_t shared, int64_t start, int32_t* pages,
                    int64_t cap, int64_t* n) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p && n, "pages_shared: null pointer");
  QX_CHECK(start >= 0 && shared >= start && start % p->page == 0 &&
               (shared - start) % p->page == 0,
           "a borrowed prefix is a whole number of pages");
  Key* k = p->find(parent);
  if (!k) QX_FAIL(QX_ENOKEY, "borrow parent %lld is not resident", (long long)parent);
  QX_CHECK(shared <= k->tokens, "the parent holds fewer tokens than borrowed");
  // a table shorter than the parent's tokens (after drop_leading) yields
  // the pages it has, as a slice of it would
  const int64_t nb = (int64_t)k->borrowed.size(), size = nb + (int64_t)k->owned.size();
  const int64_t lo = std::min(start / p->page, size), hi = std::min(shared / p->page, size);
  QX_CHECK(hi - lo <= cap, "pages_shared: %lld pages, room for %lld", (long long)(hi - lo),
           (long long)cap);
  for (int64_t i = lo; i < hi; ++i) pages[i - lo] = i < nb ? k->borrowed[i] : k->owned[i - nb];
  *n = hi - lo;
  return QX_OK;
}

// table = borrowed pages then owned; info = {tokens, borrowed, owned, pinned,
// retained, allocation order}
int qx_pages_table(void* pool, int64_t key, int32_t* pages, int64_t cap, int64_t* info) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p && info, "pages_table: null pointer");
  Key* k = p->find(key);
  if (!k) QX_FAIL(QX_ENOKEY, "key %lld is not resident", (long long)key);
  const int64_t nb = (int64_t)k->borrowed.size(), no = (int64_t)k->owned.size();
  info[0] = k->tokens;
  info[1] = nb;
  info[2] = no;
  info[3] = k->pinned;
  info[4] = k->retained;
  info[5] = (int64_t)k->order;
  if (pages && cap >= nb + no) {
    std::copy(k->borrowed.begin(), k->borrowed.end(), pages);
    std::copy(k->owned.begin(), k->owned.end(), pages + nb);
  }
  return QX_OK;
}

// stats = {free pages, retained pages, resident tokens, retained tokens,
// resident keys}
int qx_pages_stats(void* pool, int64_t* stats) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p && stats, "pages_stats: null pointer");
  int64_t resident = 0, retained = 0;
  for (auto& kv : p->keys) {
    resident += kv.second.tokens;
    if (kv.second.retained) retained += kv.second.tokens;
  }
  stats[0] = (int64_t)p->free.size();
  stats[1] = p->retained_pages;
  stats[2] = resident;
  stats[3] = retained;
  stats[4] = (int64_t)p->keys.size();
  return QX_OK;
}

// resident keys in allocation order
int qx_pages_keys(void* pool, int64_t* keys, int64_t cap, int64_t* n) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p && n, "pages_keys: null pointer");
  *n = (int64_t)p->keys.size();
  if (!keys || cap < *n) return QX_OK;
  std::vector<std::pair<uint64_t, int64_t>> by_order;
  by_order.reserve(p->keys.size());
  for (auto& kv : p->keys) by_order.emplace_back(kv.second.order, kv.first);
  std::sort(by_order.begin(), by_order.end());
  for (size_t i = 0; i < by_order.size(); ++i) keys[i] = by_order[i].second;
  return QX_OK;
}

int qx_pages_free_key(void* pool, int64_t key, int64_t* freed) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p && freed, "pages_free_key: null pointer");
  if (!p->find(key)) QX_FAIL(QX_ENOKEY, "key %lld is not resident", (long long)key);
  *freed = p->free_key(key);
  return QX_OK;
}

int qx_pages_drop_leading(void* pool, int64_t key, int64_t pages, int64_t* freed) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p && freed, "pages_drop_leading: null pointer");
  Key* k = p->find(key);
  if (!k) QX_FAIL(QX_ENOKEY, "key %lld is not resident", (long long)key);
  QX_CHECK(pages >= 0, "pages_drop_leading: %lld pages", (long long)pages);
  const int64_t take_b = std::min<int64_t>(pages, (int64_t)k->borrowed.size());
  const int64_t take_o = std::min<int64_t>(pages - take_b, (int64_t)k->owned.size());
  std::vector<int32_t> dropped(k->borrowed.begin(), k->borrowed.begin() + take_b);
  dropped.insert(dropped.end(), k->owned.begin(), k->owned.begin() + take_o);
  k->borrowed.erase(k->borrowed.begin(), k->borrowed.begin() + take_b);
  k->owned.erase(k->owned.begin(), k->owned.begin() + take_o);
  *freed = p->release(dropped);
  return QX_OK;
}

int qx_pages_rewind(void* pool, int64_t key, int64_t tokens, int64_t* freed) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p && freed, "pages_rewind: null pointer");
  Key* k = p->find(key);
  if (!k) QX_FAIL(QX_ENOKEY, "key %lld is not resident", (long long)key);
  const int64_t low = (int64_t)k->borrowed.size() * p->page;
  const int64_t high = low + (int64_t)k->owned.size() * p->page;
  QX_CHECK(tokens >= low && tokens <= high, "rewind tokens leave the resident capacity");
  const int64_t keep = p->pages_needed(tokens) - (int64_t)k->borrowed.size();
  std::vector<int32_t> released(k->owned.begin() + keep, k->owned.end());
  k->owned.resize(keep);
  k->tokens = tokens;
  *freed = p->release(released);
  if (k->retained) p->retain(key, false, 0.0);
  return QX_OK;
}

// added = pages added (0 when the capacity is already there), or -1 when the
// free stack is short
int qx_pages_grow(void* pool, int64_t key, int64_t capacity_tokens, int64_t* added) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p && added, "pages_grow: null pointer");
  Key* k = p->find(key);
  if (!k) QX_FAIL(QX_ENOKEY, "key %lld is not resident", (long long)key);
  const int64_t need = p->pages_needed(capacity_tokens) - (int64_t)k->borrowed.size() -
                       (int64_t)k->owned.size();
  if (need <= 0) {
    *added = 0;
    return QX_OK;
  }
  if (need > (int64_t)p->free.size()) {
    *added = -1;
    return QX_OK;
  }
  const size_t first = k->owned.size();
  p->take(need, k->owned);
  for (size_t i = first; i < k->owned.size(); ++i) p->holds[k->owned[i]] += 1;
  *added = need;
  return QX_OK;
}

int qx_pages_set_tokens(void* pool, int64_t key, int64_t tokens) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p, "pages_set_tokens: null pointer");
  Key* k = p->find(key);
  if (!k) QX_FAIL(QX_ENOKEY, "key %lld is not resident", (long long)key);
  k->tokens = tokens;
  return QX_OK;
}

int qx_pages_pin(void* pool, int64_t key) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p, "pages_pin: null pointer");
  Key* k = p->find(key);
  if (!k) QX_FAIL(QX_ENOKEY, "key %lld is not resident", (long long)key);
  p->forget(*k);
  k->pinned = true;
  return QX_OK;
}

int qx_pages_retain(void* pool, int64_t key, int has_priority, double priority) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p, "pages_retain: null pointer");
  if (!p->find(key)) QX_FAIL(QX_ENOKEY, "key %lld is not resident", (long long)key);
  p->retain(key, has_priority != 0, priority);
  return QX_OK;
}

// victim = {found, key, pages it alone held, tokens} of the lowest-priority
// retained key not in `keep`; the key stays resident (the caller frees it)
int qx_pages_pop_victim(void* pool, const int64_t* keep, int64_t n_keep, int64_t* victim) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p && victim && (n_keep == 0 || keep), "pages_pop_victim: null pointer");
  std::unordered_set<int64_t> kept(keep, keep + n_keep);
  std::vector<Retention> passed;
  victim[0] = 0;
  while (!p->heap.empty()) {
    Retention r = p->heap.top();
    p->heap.pop();
    Key* k = p->find(r.key);
    if (!k || !k->retained || k->version != r.version) continue;
    if (kept.count(r.key)) {
      passed.push_back(r);
      continue;
    }
    p->forget(*k);
    victim[0] = 1;
    victim[1] = r.key;
    victim[2] = r.alone;
    victim[3] = r.tokens;
    break;
  }
  for (const Retention& r : passed) p->heap.push(r);
  return QX_OK;
}

// The free stack, bottom first.
int qx_pages_free_list(void* pool, int32_t* pages, int64_t cap, int64_t* n) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p && n, "pages_free_list: null pointer");
  *n = (int64_t)p->free.size();
  if (pages && cap >= *n) std::copy(p->free.begin(), p->free.end(), pages);
  return QX_OK;
}

// groups: 8 int64 per group {key, fresh, f, start, prefix tokens, suffixes,
// suffix tokens kept in the key's pages, every suffix row answers};
// prefix_ids: the fresh groups' prefixes, concatenated; suffix_lens and
// suffix_ids: every group's suffixes, concatenated. On success *pack holds
// the arrays (qx_pack_array) until qx_pack_destroy. On failure every
// temporary key allocated so far is freed and *failed_group names the group.
static int pack_unified(void* pool, const int64_t* groups, int64_t n_groups,
                        const int64_t* prefix_ids, const int64_t* suffix_lens,
                        const int64_t* suffix_ids, void** pack, int64_t* failed_group) {
  PagePool* p = pool_of(pool);
  QX_CHECK(p && pack && failed_group && (n_groups == 0 || groups), "pack_unified: null pointer");
  *pack = nullptr;
  *failed_group = -1;
  Pack* out = new Pack();
  std::vector<Spec> specs;
  specs.reserve(n_groups);
  int64_t n_tok = 0, prefix_at = 0, suffix_at = 0, suffix_id_at = 0;
  bool multi = false;
  out->cu_a.push_back(0);
  for (int64_t g = 0; g < n_groups; ++g) {
    const int64_t* d = groups + 8 * g;
    const int64_t key = d[0], f = d[2], start = d[3], prefix_len = d[4], n = d[5];
    const bool fresh = d[1] != 0, read_all = d[7] != 0;
    if (!p->find(key)) {
      delete out;
      *failed_group = g;
      QX_FAIL(QX_EINVAL, "the paged unified path needs arena pages");
    }
    if (prefix_len < 0 || n < 0) {
      delete out;
      *failed_group = g;
      QX_FAIL(QX_EINVAL, "negative prefix or suffix count");
    }
    const int64_t row0 = n_tok;
    if (fresh) {
      QX_CHECK(prefix_ids || prefix_len == 0, "pack_unified: prefix ids");
      out->ids.insert(out->ids.end(), prefix_ids + prefix_at, prefix_ids + prefix_at + prefix_len);
      for (int64_t i = 0; i < prefix_len; ++i) out->positions.push_back(start + i);
      prefix_at += prefix_len;
      n_tok += prefix_len;
      out->cu_a.push_back((int32_t)n_tok);
    }
    const int64_t prefix_end = n_tok, s_row0 = n_tok;
    Spec s{key, f, start, row0, prefix_end, 0, fresh, d[6], {}, {}};
    int64_t total = 0;
    for (int64_t j = 0; j < n; ++j) {
      const int64_t len = suffix_lens[suffix_at + j];
      s.begins.push_back(s_row0 + total);
      total += len;
      s.ends.push_back(s_row0 + total);
    }
    if (n) {
      out->ids.insert(out->ids.end(), suffix_ids + suffix_id_at, suffix_ids + suffix_id_at + total);
      suffix_id_at += total;
      for (int64_t j = 0; j < n; ++j) {
        const int64_t len = suffix_lens[suffix_at + j];
        for (int64_t i = 0; i < len; ++i) out->positions.push_back(f + i);
        out->cu_a.push_back((int32_t)s.ends[j]);
      }
      if (read_all) {
        for (int64_t r = s_row0; r < s_row0 + total; ++r) out->finals.push_back(r);
        for (int64_t j = 0; j < n; ++j) out->rows_per_answer.push_back(suffix_lens[suffix_at + j]);
        multi = true;
      } else {
        for (int64_t j = 0; j < n; ++j) {
          out->finals.push_back(s.ends[j] - 1);
          out->rows_per_answer.push_back(1);
        }
      }
      n_tok += total;
    }
    suffix_at += n;
    s.row1 = n_tok;
    out->suffix_counts.push_back(n);
    out->row_spans.insert(out->row_spans.end(), {row0, prefix_end, n_tok});
    specs.push_back(std::move(s));
  }

  const int64_t page = p->page;
  std::vector<std::vector<int32_t>> seq_pages;
  std::vector<int64_t> seq_used;
  out->cu_q.push_back(0);
  auto abort_pack = [&](int code, int64_t g) {
    for (int64_t t : out->temporaries) p->free_key(t);
    delete out;
    *failed_group = g;
    return code;
  };
  // pool row of logical row i of a table
  auto row_of = [page](const std::vector<int32_t>& table, int64_t i) {
    return (int64_t)table[i / page] * page + i % page;
  };
  for (int64_t g = 0; g < (int64_t)specs.size(); ++g) {
    const Spec& s = specs[g];
    Key& k = p->keys.at(s.key);
    std::vector<int32_t> table(k.borrowed);
    table.insert(table.end(), k.owned.begin(), k.owned.end());
    const int64_t capacity_rows = (int64_t)table.size() * page;
    const int64_t logical = s.fresh ? s.start : s.f;
    const int64_t count = s.row1 - s.row0;
    int64_t suffix_total = 0;
    for (size_t j = 0; j < s.begins.size(); ++j) suffix_total += s.ends[j] - s.begins[j];
    if (s.fresh) out->fresh_keys.push_back(s.key);
    const bool direct = s.begins.size() == 1 && logical + count <= capacity_rows;
    if (s.keeps && !direct) {
      qx::set_error("keeps suffix KV but its pages hold %lld rows, not %lld",
                    (long long)capacity_rows, (long long)(logical + count));
      return abort_pack(QX_EINVAL, g);
    }
    if (direct) {
      for (int64_t i = 0; i < count; ++i) {
        out->src.push_back(s.row0 + i);
        out->dst.push_back(row_of(table, logical + i));
      }
      seq_pages.push_back(table);
      seq_used.push_back(s.f + suffix_total);
      out->cu_q.push_back((int32_t)(out->cu_q.back() + count));
      continue;
    }
    const int64_t n_prefix = s.prefix_end - s.row0;
    if (s.start + n_prefix > capacity_rows) {
      qx::set_error("a prefix of %lld rows from %lld passes its key's %lld rows",
                    (long long)n_prefix, (long long)s.start, (long long)capacity_rows);
      return abort_pack(QX_EINVAL, g);
    }
    if (remainder_tail_missing(s, table, page)) {
      qx::set_error("the partial page of a %lld-token document is not in its table",
                    (long long)s.f);
      return abort_pack(QX_EINVAL, g);
    }
    if (n_prefix) {
      for (int64_t i = 0; i < n_prefix; ++i) {
        out->src.push_back(s.row0 + i);
        out->dst.push_back(row_of(table, s.start + i));
      }
      const int64_t keep = std::min<int64_t>(p->pages_needed(s.f), (int64_t)table.size());
      seq_pages.emplace_back(table.begin(), table.begin() + keep);
      seq_used.push_back(s.f);
      out->cu_q.push_back((int32_t)(out->cu_q.back() + n_prefix));
    }
    const int64_t remainder = s.f % page;
    const int64_t full = std::min<int64_t>(s.f / page, (int64_t)table.size());
    for (size_t j = 0; j < s.begins.size(); ++j) {
      const int64_t s0 = s.begins[j], s1 = s.ends[j];
      const int64_t temp = p->next_temporary;
      const int64_t got = p->alloc(temp, remainder + (s1 - s0), remainder + (s1 - s0), nullptr, 0);
      if (got < 0) {
        qx::set_error("unified suffix pages exceed the free KV arena (asked %lld rows, free "
                      "pages %lld)", (long long)(remainder + s1 - s0), (long long)p->free.size());
        return abort_pack(QX_EFULL, g);
      }
      p->next_temporary -= 1;
      out->temporaries.push_back(temp);
      const std::vector<int32_t>& tpages = p->keys.at(temp).owned;
      for (int64_t i = 0; i < s1 - s0; ++i) {
        out->src.push_back(s0 + i);
        out->dst.push_back(row_of(tpages, remainder + i));
      }
      if (remainder) {
        const int64_t base = (int64_t)table[s.f / page] * page;
        for (int64_t i = 0; i < remainder; ++i) {
          out->tail_src.push_back(base + i);
          out->tail_dst.push_back(row_of(tpages, i));
        }
      }
      std::vector<int32_t> seq(table.begin(), table.begin() + full);
      seq.insert(seq.end(), tpages.begin(), tpages.end());
      seq_pages.push_back(std::move(seq));
      seq_used.push_back(s.f + (s1 - s0));
      out->cu_q.push_back((int32_t)(out->cu_q.back() + (s1 - s0)));
    }
  }

  size_t width = 1;
  if (!seq_pages.empty()) {
    width = 0;
    for (auto& sp : seq_pages) width = std::max(width, sp.size());
  }
  out->table.assign(seq_pages.size() * width, 0);
  int64_t max_q = 0, max_used = 0;
  for (size_t i = 0; i < seq_pages.size(); ++i) {
    std::copy(seq_pages[i].begin(), seq_pages[i].end(), out->table.begin() + i * width);
    out->seq_pages.push_back((int64_t)seq_pages[i].size());
    out->used.push_back((int32_t)seq_used[i]);
    max_q = std::max<int64_t>(max_q, out->cu_q[i + 1] - out->cu_q[i]);
    max_used = std::max<int64_t>(max_used, seq_used[i]);
  }
  if (!multi) out->rows_per_answer.clear();
  out->scalars = {n_tok, max_q, max_used, multi ? 1 : 0, out->tail_src.empty() ? 0 : 1,
                  (int64_t)width};
  *pack = out;
  return QX_OK;
}

int qx_pack_unified(void* pool, const int64_t* groups, int64_t n_groups,
                    const int64_t* prefix_ids, const int64_t* suffix_lens,
                    const int64_t* suffix_ids, void** pack, int64_t* failed_group) {
  try {
    return pack_unified(pool, groups, n_groups, prefix_ids, suffix_lens, suffix_ids, pack,
                        failed_group);
  } catch (const std::bad_alloc&) {
    qx::set_error("pack_unified: out of host memory");
    return QX_EINVAL;
  }
}

int qx_pack_array(void* pack, int64_t which, const void** data, int64_t* count) {
  Pack* p = static_cast<Pack*>(pack);
  QX_CHECK(p && data && count, "pack_array: null pointer");
  QX_CHECK(which >= 0 && which < kNumArrays, "pack_array: no array %lld", (long long)which);
  auto put64 = [&](const std::vector<int64_t>& v) {
    *data = v.data();
    *count = (int64_t)v.size();
  };
  auto put32 = [&](const std::vector<int32_t>& v) {
    *data = v.data();
    *count = (int64_t)v.size();
  };
  switch (which) {
    case kIds: put64(p->ids); break;
    case kPositions: put64(p->positions); break;
    case kFinals: put64(p->finals); break;
    case kCuA: put32(p->cu_a); break;
    case kRowsPerAnswer: put64(p->rows_per_answer); break;
    case kSrc: put64(p->src); break;
    case kDst: put64(p->dst); break;
    case kTailSrc: put64(p->tail_src); break;
    case kTailDst: put64(p->tail_dst); break;
    case kCuQ: put32(p->cu_q); break;
    case kUsed: put32(p->used); break;
    case kTable: put32(p->table); break;
    case kSeqPages: put64(p->seq_pages); break;
    case kTemporaries: put64(p->temporaries); break;
    case kRowSpans: put64(p->row_spans); break;
    case kSuffixCounts: put64(p->suffix_counts); break;
    case kFreshKeys: put64(p->fresh_keys); break;
    case kScalars: put64(p->scalars); break;
  }
  return QX_OK;
}

int qx_pack_destroy(void* pack) {
  delete static_cast<Pack*>(pack);
  return QX_OK;
}

}  // extern "C"
