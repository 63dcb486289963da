"""Prefix tree over the documents' token sequences.

Restates the reference planner's PrefixIndex / PrefixTree
(crates/quail-planner/src/inputs/prefix.rs:14-121; Python wrapper
quail/common/tokens.py:440-484):

  * documents are sorted by their tokens (lexicographic, stable);
  * shared[i] = min(common prefix with the predecessor in that order,
    len(i) - 1): every document computes its own last token;
  * tree(page_tokens) rounds each share down to whole pages and gives each
    document that borrows a parent: its predecessor, or, climbing, the
    nearest ancestor that itself borrowed at least as many tokens.
"""

from dataclasses import dataclass


def _common_prefix(a, b) -> int:
    n = min(len(a), len(b))
    i = 0
    while i < n and a[i] == b[i]:
        i += 1
    return i


@dataclass(frozen=True)
class ReaderGroup:
    shared: int
    count: int
    rows: int


@dataclass
class PrefixTree:
    """order: positions in token order (parents before children);
    parent[i]: the document i borrows from, or None; shared[i]: tokens
    borrowed, a multiple of the page size."""

    order: list
    parent: list
    shared: list

    def reader_groups(self, lengths):
        """Borrowers grouped by (parent, shared), in order of first appearance."""
        where = {}
        groups = []
        for index, parent in enumerate(self.parent):
            if parent is None:
                continue
            key = (parent, self.shared[index])
            if key not in where:
                where[key] = len(groups)
                groups.append([self.shared[index], 0, 0])
            g = groups[where[key]]
            g[1] += 1
            g[2] += int(lengths[index]) - self.shared[index]
        return [ReaderGroup(*g) for g in groups]


class PrefixIndex:
    """Documents in sorted token order and what each shares with its predecessor."""

    def __init__(self, documents):
        docs = [tuple(int(t) for t in d) for d in documents]
        self.order = sorted(range(len(docs)), key=docs.__getitem__)
        self.shared = [0] * len(docs)
        for prev, cur in zip(self.order, self.order[1:]):
            common = _common_prefix(docs[prev], docs[cur])
            self.shared[cur] = min(common, max(len(docs[cur]) - 1, 0))

    def tree(self, page_tokens: int) -> PrefixTree:
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
        return PrefixTree(order=list(self.order), parent=parent, shared=shared)
