"""Prefix tree (the native qx_prefix_tree) against the reference planner's
known answers (crates/quail-planner/tests/prefix.rs:10-76), the oracle's
restatement and a brute-force definition."""

import itertools
import random

import numpy as np
import pytest

from oracle import prefix_ref
from quail_amd import _lib
from quail_amd.prefix import PrefixIndex, ReaderGroup

DOCS = [[1, 2, 3, 4, 5], [1, 2, 3, 4, 9], [1, 2, 3, 4, 5], [], [7, 8], [1, 2]]
LENGTHS = [5, 5, 5, 0, 2, 2]


def test_documents_sort_and_share_all_but_last_token():
    index = PrefixIndex(DOCS)
    assert index.order == [3, 5, 0, 2, 1, 4]
    assert index.shared == [2, 4, 4, 0, 0, 0]


def test_reader_groups_under_one_parent():
    index = PrefixIndex(DOCS)
    tree = index.tree(2)
    assert tree.parent == [5, 0, 0, None, None, None]
    assert tree.reader_groups(LENGTHS) == [ReaderGroup(2, 1, 3), ReaderGroup(4, 2, 2)]
    tree = index.tree(4)
    assert tree.shared == [0, 4, 4, 0, 0, 0]
    assert tree.parent == [None, 0, 0, None, None, None]
    assert tree.reader_groups(LENGTHS) == [ReaderGroup(4, 2, 2)]


def _brute_tree(docs, page):
    """Tree by definition: borrow from the nearest earlier document in sorted
    order whose whole ancestry chain (up to where shares drop) covers it."""
    order = sorted(range(len(docs)), key=lambda i: tuple(docs[i]))
    shared = [0] * len(docs)
    for a, b in zip(order, order[1:]):
        c = len(list(itertools.takewhile(lambda p: p[0] == p[1], zip(docs[a], docs[b]))))
        shared[b] = min(c, max(len(docs[b]) - 1, 0)) // page * page
    parent = [None] * len(docs)
    for a, b in zip(order, order[1:]):
        if shared[b] == 0:
            continue
        owner = a
        chain = [a]
        while parent[owner] is not None and shared[owner] >= shared[b]:
            owner = parent[owner]
            chain.append(owner)
        parent[b] = owner
        # the owner really holds the first shared[b] tokens of b
        assert docs[owner][:shared[b]] == docs[b][:shared[b]]
    return order, parent, shared


def test_random_corpora_match_definition():
    rng = random.Random(7)
    for trial in range(200):
        base = [rng.randrange(4) for _ in range(rng.randrange(0, 12))]
        docs = []
        for _ in range(rng.randrange(1, 12)):
            cut = rng.randrange(0, len(base) + 1)
            docs.append(base[:cut] + [rng.randrange(4) for _ in range(rng.randrange(0, 6))])
        for page in (1, 2, 4):
            tree = PrefixIndex(docs).tree(page)
            order, parent, shared = _brute_tree(docs, page)
            assert tree.order == order
            assert tree.shared == shared
            assert tree.parent == parent
            assert prefix_ref.PrefixIndex(docs).tree(page) == (order, parent, shared)
            # a parent precedes its child in the order
            pos = {d: i for i, d in enumerate(tree.order)}
            for child, p in enumerate(tree.parent):
                if p is not None:
                    assert pos[p] < pos[child]


def test_oracle_matches_the_known_answers():
    index = prefix_ref.PrefixIndex(DOCS)
    assert index.order == [3, 5, 0, 2, 1, 4]
    assert index.shared == [2, 4, 4, 0, 0, 0]
    assert index.tree(2)[1] == [5, 0, 0, None, None, None]


def test_large_corpus_matches_the_oracle():
    """A Qwen3-4B-sized corpus: 512 documents behind one 64-token prefix,
    with some duplicated and nested documents."""
    rng = np.random.default_rng(5)
    prefix = rng.integers(0, 151936, 64)
    docs = [np.concatenate([prefix, rng.integers(0, 151936, int(n))])
            for n in rng.integers(32, 600, 500)]
    docs += [docs[3].copy(), docs[7][:100].copy(), prefix[:40].copy(), np.zeros(0, np.int64)]
    docs += [np.concatenate([docs[9][:200], rng.integers(0, 5, 30)]) for _ in range(8)]
    for page in (1, 16):
        got = PrefixIndex(docs).tree(page)
        want = prefix_ref.PrefixIndex([d.tolist() for d in docs]).tree(page)
        assert (got.order, got.parent, got.shared) == want


def test_native_rejects_bad_offsets():
    tokens = np.arange(6, dtype=np.int64)
    offsets = np.array([0, 4, 2], dtype=np.int64)
    out = [np.empty(2, dtype=np.int64) for _ in range(3)]
    with pytest.raises(_lib.QxError, match="offsets"):
        _lib.call("qx_prefix_tree", tokens.ctypes.data, offsets.ctypes.data, 2, 16,
                  *(o.ctypes.data for o in out))
