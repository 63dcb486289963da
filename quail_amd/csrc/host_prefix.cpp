// Prefix tree over the documents' token sequences, on the host.
//
// Restates the reference planner's PrefixIndex::new and PrefixIndex::tree
// (crates/quail-planner/src/inputs/prefix.rs:33-73), which the Python
// wrapper PrefixTree (quail/common/tokens.py:440-484) exposes:
//   * documents are sorted by their tokens, lexicographically (a proper
//     prefix sorts first), ties kept in input order;
//   * a document shares with its predecessor in that order their common
//     prefix, capped at its own length - 1 (it computes its last token);
//   * tree(page_tokens) rounds each share down to whole pages; a document
//     with a nonzero share borrows from its predecessor or, climbing, from
//     the nearest ancestor that itself borrowed at least as many tokens.
#include <stdint.h>

#include <algorithm>
#include <numeric>
#include <vector>

#include "qx_status.h"

extern "C" int qx_prefix_tree(const int64_t* tokens, const int64_t* offsets, int64_t n,
                              int64_t page_tokens, int64_t* order, int64_t* parent,
                              int64_t* shared) {
  QX_CHECK(n >= 0, "prefix_tree: %lld documents", (long long)n);
  QX_CHECK(page_tokens >= 1, "prefix_tree: page of %lld tokens", (long long)page_tokens);
  if (n == 0) return QX_OK;
  QX_CHECK(offsets && order && parent && shared, "prefix_tree: null pointer");
  QX_CHECK(offsets[0] == 0 && (tokens || offsets[n] == 0), "prefix_tree: tokens");
  for (int64_t i = 0; i < n; ++i)
    QX_CHECK(offsets[i] >= 0 && offsets[i + 1] >= offsets[i], "prefix_tree: offsets not sorted");

  auto first = [&](int64_t i) { return tokens + offsets[i]; };
  auto last = [&](int64_t i) { return tokens + offsets[i + 1]; };

  std::vector<int64_t> idx(n);
  std::iota(idx.begin(), idx.end(), 0);
  std::stable_sort(idx.begin(), idx.end(), [&](int64_t a, int64_t b) {
    return std::lexicographical_compare(first(a), last(a), first(b), last(b));
  });

  std::vector<int64_t> share(n, 0);
  for (int64_t k = 1; k < n; ++k) {
    const int64_t prev = idx[k - 1], cur = idx[k];
    const int64_t len_prev = offsets[prev + 1] - offsets[prev];
    const int64_t len_cur = offsets[cur + 1] - offsets[cur];
    const int64_t m = std::min(len_prev, len_cur);
    const int64_t common = std::mismatch(first(prev), first(prev) + m, first(cur)).first - first(prev);
    const int64_t cap = std::max<int64_t>(len_cur - 1, 0);
    share[cur] = std::min(common, cap) / page_tokens * page_tokens;
  }

  for (int64_t i = 0; i < n; ++i) {
    order[i] = idx[i];
    parent[i] = -1;
    shared[i] = share[i];
  }
  for (int64_t k = 1; k < n; ++k) {
    const int64_t cur = idx[k];
    const int64_t want = share[cur];
    if (want <= 0) continue;
    int64_t owner = idx[k - 1];
    while (parent[owner] >= 0 && share[owner] >= want) owner = parent[owner];
    parent[cur] = owner;
  }
  return QX_OK;
}
