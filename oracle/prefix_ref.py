"""Prefix tree of the reference planner, restated in plain Python.

Test infrastructure (see oracle/__init__.py): the checker of the native
qx_prefix_tree. It restates PrefixIndex::new / PrefixIndex::tree
(crates/quail-planner/src/inputs/prefix.rs:33-73):

  * documents are sorted by their tokens (lexicographic, stable);
  * shared[i] = min(common prefix with the predecessor in that order,
    len(i) - 1): every document computes its own last token;
  * tree(page_tokens) rounds each share down to whole pages and gives each
    document that borrows a parent: its predecessor, or, climbing, the
    nearest ancestor that itself borrowed at least as many tokens.

It is pinned by the planner's own known answers
(crates/quail-planner/tests/prefix.rs:29-76) and by a brute-force
definition over random corpora (tests/test_prefix.py).
"""


def _common_prefix(a, b) -> int:
    n = min(len(a), len(b))
    i = 0
    while i < n and a[i] == b[i]:
        i += 1
    return i


class PrefixIndex:
    """Documents in sorted token order and what each shares with its predecessor."""

    def __init__(self, documents):
        docs = [tuple(int(t) for t in d) for d in documents]
        self.order = sorted(range(len(docs)), key=docs.__getitem__)
        self.shared = [0] * len(docs)
        for prev, cur in zip(self.order, self.order[1:]):
            common = _common_prefix(docs[prev], docs[cur])
            self.shared[cur] = min(common, max(len(docs[cur]) - 1, 0))

    def tree(self, page_tokens: int):
        """(order, parent with None for roots, shared) at page_tokens."""
        shared = [s // page_tokens * page_tokens for s in self.shared]
        parent = [None] * len(shared)
        for prev, cur in zip(self.order, self.order[1:]):
            want = shared[cur]
            if want <= 0:
                continue
            owner = prev
            while parent[owner] is not None and shared[owner] >= want:
                owner = parent[owner]
            parent[cur] = owner
        return list(self.order), parent, shared
