"""Prefix tree over the documents' token sequences.

The tree itself is computed by qx_prefix_tree (csrc/host_prefix.cpp), which
restates the reference planner's PrefixIndex / PrefixTree
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

import numpy as np

from quail_amd import _lib


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
    """Documents in sorted token order and what each shares with its
    predecessor, computed by the native qx_prefix_tree (host C++).

    documents: token sequences (numpy arrays or lists of ints >= 0)."""

    def __init__(self, documents):
        docs = [np.asarray(d, dtype=np.int64).reshape(-1) for d in documents]
        self._set(docs, [len(d) for d in docs])

    @classmethod
    def from_parts(cls, documents):
        """The index of documents given as lists of token pieces (a prompt's
        prefix and suffixes), joined once into the flat token array."""
        self = cls.__new__(cls)
        pieces, lengths = [], []
        for parts in documents:
            arrays = [np.asarray(p, dtype=np.int64).reshape(-1) for p in parts]
            pieces.extend(arrays)
            lengths.append(sum(len(a) for a in arrays))
        self._set(pieces, lengths)
        return self

    def _set(self, pieces, lengths):
        self._offsets = np.zeros(len(lengths) + 1, dtype=np.int64)
        np.cumsum(np.asarray(lengths, dtype=np.int64), out=self._offsets[1:])
        self._tokens = (np.concatenate(pieces) if pieces else np.zeros(0, dtype=np.int64))
        self._tokens = np.ascontiguousarray(self._tokens, dtype=np.int64)
        self._sorted = None

    def _sorted_shares(self):
        if self._sorted is None:
            order, _, shared = self._native(1)
            self._sorted = (order.tolist(), shared.tolist())
        return self._sorted

    @property
    def order(self):
        """Document positions in sorted token order."""
        return self._sorted_shares()[0]

    @property
    def shared(self):
        """Tokens each document shares with its predecessor in that order."""
        return self._sorted_shares()[1]

    def _native(self, page_tokens):
        n = len(self._offsets) - 1
        order = np.empty(n, dtype=np.int64)
        parent = np.empty(n, dtype=np.int64)
        shared = np.empty(n, dtype=np.int64)
        ptr = lambda a: a.ctypes.data if a.size else None
        _lib.call("qx_prefix_tree", ptr(self._tokens), self._offsets.ctypes.data, n,
                  int(page_tokens), ptr(order), ptr(parent), ptr(shared))
        return order, parent, shared

    def tree(self, page_tokens: int) -> PrefixTree:
        order, parent, shared = self._native(page_tokens)
        return PrefixTree(order=order.tolist(),
                          parent=[None if p < 0 else int(p) for p in parent],
                          shared=shared.tolist())
