"""The tree attention layout (attention_mode="tree"): the reference's known
answers (tests/engine/test_pack_chunk.py:16-51 and the retained-read counts
of :58-100) and the structural read check over seeded corpora with shared
prefixes (each row's call-B keys through its read table, then its call-A
segment, must be exactly its document up to itself)."""

import numpy as np
import pytest

from oracle.packing_ref import PoolModel, check_pack_tree
from quail_amd.arena import KVArena
from quail_amd.chunk import pack_chunk
from quail_amd.prefix import PrefixIndex
from tests.helpers import admit, pack_specs
from tests.test_pack import _corpus


def plain_arena(pages=64, page=16):
    return KVArena(1, pages, page, 1, 8, device="cpu")


def test_many_suffixes_and_a_kept_document():
    # tests/engine/test_pack_chunk.py:16-51
    arena = plain_arena()
    key = ("d", 0)
    arena.activate(key, 4, capacity_tokens=8, base_tokens=4)
    sufs = [[10, 11], [12], [13, 14, 15]]
    chunk = pack_chunk(arena, [dict(key=key, prefix=[1, 2, 3, 4], f=4, suffixes=sufs,
                                    read_all_rows=True)], attention_mode="tree")
    assert chunk.host_ids.tolist() == [1, 2, 3, 4, 10, 11, 12, 13, 14, 15]
    assert chunk.host_positions.tolist() == [0, 1, 2, 3, 4, 5, 4, 4, 5, 6]
    assert chunk.final_indices.tolist() == [4, 5, 6, 7, 8, 9]
    assert chunk.rows_per_answer.tolist() == [2, 1, 3]
    assert chunk.meta["cu_a"].tolist() == [0, 4, 6, 7, 10]
    assert chunk.meta["max_a"] == 4
    assert chunk.layout == [(key, 3)]
    assert chunk.fresh_keys == (key,)
    assert chunk.meta["kv_src"].tolist() == [0, 1, 2, 3]
    # the suffix rows read the document's 4 tokens from its pages
    reads = chunk.meta["reads"]
    assert reads["rows"].tolist() == [4, 5, 6, 7, 8, 9]
    assert reads["used"].tolist() == [4]
    chunk = pack_chunk(arena, [dict(key=key, prefix=None, f=4, suffixes=sufs)],
                       attention_mode="tree")
    assert chunk.host_ids.tolist() == [10, 11, 12, 13, 14, 15]
    assert chunk.final_indices.tolist() == [1, 2, 5]
    assert chunk.rows_per_answer is None
    assert chunk.meta["cu_a"].tolist() == [0, 2, 3, 6]
    reads = chunk.meta["reads"]
    assert reads["rows"].tolist() == [0, 1, 2, 3, 4, 5]
    assert reads["cu_q"].tolist() == [0, 6]
    assert reads["used"].tolist() == [4]
    assert reads["source"].tolist() == [0, 1, 2, 3, 4, 5]
    assert chunk.meta["kv_src"] is None


@pytest.mark.parametrize("shared", [0, 16])
def test_retained_reads_of_a_stacked_then_kept_document(shared):
    # tests/engine/test_pack_chunk.py:58-100 with run = 2: the first pass
    # reads the shared pages of the parent, the second the kept 35 tokens
    arena = plain_arena()
    parent, key = ("d", 0), ("d", 1)
    arena.activate(parent, 32, capacity_tokens=40, base_tokens=32)
    arena.activate(key, 32, capacity_tokens=40, base_tokens=32,
                   borrow=(parent, shared) if shared else None)
    retained = []
    for first in (True, False):
        chunk = pack_chunk(arena, [dict(
            key=key, prefix=list(range(shared, 32)) if first else None,
            f=32 if first else 35, start=shared if first else 0,
            read_key=parent if first and shared else None,
            suffixes=[[91, 92, 93]] if first else [[40, 41]],
            write_suffix_tokens=3 if first else 2, single=True)], attention_mode="tree")
        reads = chunk.meta["reads"]
        retained.append(0 if reads is None else int(reads["used"].sum()))
        if first:
            # the prefix rows, then the 3 kept suffix rows after them
            rows = arena.capacity_rows(key)
            assert chunk.meta["kv_dst"].tolist() == rows[shared:35].tolist()
            # whole document, one causal segment
            assert chunk.meta["cu_a"].tolist() == [0, 32 - shared + 3]
    assert retained == [shared, 35]


def test_unpaged_and_unsupported_groups_are_refused():
    arena = plain_arena()
    with pytest.raises(ValueError, match="needs arena pages"):
        pack_chunk(arena, [dict(key="x", prefix=[1, 2], f=2, start=16, suffixes=[[3]])],
                   attention_mode="tree")
    arena.activate("y", 4)
    with pytest.raises(ValueError, match="canvas"):
        pack_chunk(arena, [dict(key="y", prefix=[1, 2, 3, 4], f=4, suffixes=[[5]],
                                canvas=[1, 2])], attention_mode="tree")


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 7, 11, 100, 200])
def test_tree_packs_read_exactly_their_documents(seed):
    docs = _corpus(seed, 40)
    arena = plain_arena(pages=48)
    tree = PrefixIndex(docs).tree(16)
    adm = admit([d[:-1] for d in docs], [[d[-1:]] for d in docs], arena, 256, tree=tree,
                unified=False)
    pool = PoolModel()
    prompts = {adm.keys[i]: d for i, d in enumerate(docs)}
    checked = packs = stacked = 0
    live = []

    def settle():
        for d, first, end, _ in live.pop(0):
            if adm.report(d, first, end, [0] * (end - first)):
                arena.free_key(adm.keys[d])

    while not adm.done():
        groups = adm.next_chunk(arena.free_pages)
        assert not adm.take_prefills()
        if not groups:
            assert live
            settle()
            continue
        specs = [dict(g, read_key=g["borrow_key"] if g["start"] else None, single=True)
                 for g in pack_specs(adm, groups)]
        stacked += sum(1 for g in specs if g["read_key"] is not None)
        chunk = pack_chunk(arena, specs, attention_mode="tree")
        checked += check_pack_tree(chunk, 16, pool, prompts.__getitem__)
        live.append(groups)
        packs += 1
        if len(live) > 1:
            settle()
    while live:
        settle()
    assert checked == sum(len(d) for d in docs) - adm.borrowed_tokens
    assert packs >= 2 and stacked > 0
    assert arena.free_pages == arena.num_pages


def test_siblings_share_one_stacked_read_of_their_parent():
    prefix = list(range(32))
    docs = [prefix + [100 + i] * (3 + i) for i in range(5)]
    arena = plain_arena()
    tree = PrefixIndex(docs).tree(16)
    adm = admit([d[:-1] for d in docs], [[d[-1:]] for d in docs], arena, 1024, tree=tree,
                unified=False)
    groups = adm.next_chunk(arena.free_pages)
    specs = [dict(g, read_key=g["borrow_key"] if g["start"] else None, single=True)
             for g in pack_specs(adm, groups)]
    chunk = pack_chunk(arena, specs, attention_mode="tree")
    reads = chunk.meta["reads"]
    # the root is one segment with no reads; its four children read the
    # root's 32 tokens in one stacked sequence
    assert reads["used"].tolist() == [32]
    n_root = len(docs[0])
    assert reads["rows"].tolist() == list(range(n_root, len(chunk.host_ids)))
    assert chunk.meta["cu_a"].tolist()[:2] == [0, n_root]
    check_pack_tree(chunk, 16, PoolModel(), {adm.keys[i]: d for i, d in enumerate(docs)}.__getitem__)


# ---- label paths (trie-scored AI.CLASSIFY): call C --------------------------------------

from oracle.labels_ref import (fed_nodes, label_trie, path_contexts, path_reads,  # noqa: E402
                               path_tokens, read_nodes, trie_paths)

LABELS = ((10,), (20, 21, 22), (20, 25, 26, 27, 28), (30, 31, 32), (30, 31, 33))
SPLIT = ((10,), (20, 21), (20, 22), (30, 31, 32), (40,), (40, 41))


def test_label_trie_known_answers():
    # tests/planner/test_classify_cost.py:16, 106-108: LABELS feeds a 4-token
    # suffix and reads 3 of its rows; :138-141: where SPLIT's labels split
    read = read_nodes(LABELS)
    paths = trie_paths(LABELS, read)
    assert len(path_tokens(paths, 7)) == 4 and sum(path_reads(paths, read)) == 3
    assert read == {(), (20,), (30, 31)}
    assert read_nodes(SPLIT) == {(), (20,), (40,)}


@pytest.mark.parametrize("seed", range(8))
def test_trie_paths_hold_every_fed_node_once_and_gather_its_ancestors(seed):
    rng = np.random.default_rng(seed)
    labels = {tuple(rng.integers(1, 5, rng.integers(1, 6)).tolist())
              for _ in range(rng.integers(2, 9))}
    labels = sorted(labels)
    for read in (None, read_nodes(labels)):
        paths = trie_paths(labels, read)
        fed = fed_nodes(set(label_trie(labels)) if read is None else read)
        held = [node for nodes, _, _ in paths for node in nodes]
        assert sorted(held) == sorted(fed) and len(held) == len(set(held))
        where = {}
        for p, (nodes, first, _) in enumerate(paths):
            assert first == len(nodes[0])
            assert all(b[:-1] == a for a, b in zip(nodes, nodes[1:]))
            where.update({node: (p, r) for r, node in enumerate(nodes)})
        for nodes, _, gathers in paths:
            rows = {(c, r) for c, count in gathers for r in range(count)}
            assert rows == {where[nodes[0][:d]] for d in range(len(nodes[0]))}


@pytest.mark.parametrize("labels", [LABELS, SPLIT])
@pytest.mark.parametrize("every_node", [False, True])
def test_label_paths_read_their_document_ancestors_and_path(labels, every_node):
    """Each path row reads the document (call B), the rows above its path's
    first node (call C) and its path up to itself (call A): exactly the
    document, the answer cue and its trie node's tokens."""
    arena = plain_arena()
    doc = list(range(100, 137))          # 37 tokens: the last page is partial
    arena.activate("doc", len(doc))
    pool = PoolModel()
    first = pack_chunk(arena, [dict(key="doc", prefix=doc, f=len(doc), suffixes=[])],
                       attention_mode="tree")
    assert check_pack_tree(first, 16, pool, lambda k: doc) == len(doc)
    read = None if every_node else read_nodes(labels)
    paths = trie_paths(labels, read)
    cue = 7
    tokens = path_tokens(paths, cue)
    mask = path_reads(paths, read)
    group = dict(key="doc", prefix=None, f=len(doc), suffixes=[tokens], read_all_rows=True,
                 paths=paths, read_mask=None if every_node else mask)
    chunk = pack_chunk(arena, [group], attention_mode="tree")
    contexts = path_contexts(paths, cue, doc)
    assert check_pack_tree(chunk, 16, pool, lambda k: doc,
                           lambda k, r: contexts[r]) == len(tokens)
    assert chunk.final_indices.tolist() == [i for i, m in enumerate(mask) if m]
    assert chunk.rows_per_answer.tolist() == ([len(tokens)] if every_node else [sum(mask)])
    nodes = chunk.meta["reads"]["nodes"]
    assert nodes["rows"].tolist() == list(range(len(paths[0][0]), len(tokens)))
    with pytest.raises(ValueError, match="paths pack one suffix"):
        pack_chunk(arena, [dict(group, read_all_rows=False)], attention_mode="tree")
    with pytest.raises(ValueError, match="paths hold"):
        pack_chunk(arena, [dict(group, suffixes=[tokens + [1]], read_mask=None)],
                   attention_mode="tree")


@pytest.mark.parametrize("labels", [LABELS, SPLIT])
@pytest.mark.parametrize("borrow", [0, 32])
def test_label_paths_with_their_document_in_the_same_pack(labels, borrow):
    """A document packed fresh together with its label paths (one group,
    as the stage driver packs it; reference chunk.py:765-786): its rows are
    a causal segment of their own written to its pages, reading a lender's
    first `borrow` tokens from the lender's pages, and each path row reads
    exactly the document, the cue and its trie node's tokens. A read_key
    or `single` on the group does not stack or merge it."""
    arena = plain_arena()
    pool = PoolModel()
    doc = list(range(100, 137))
    prompts = {"doc": doc}
    if borrow:
        parent = doc[:borrow] + [5, 6, 7]
        prompts["parent"] = parent
        arena.activate("parent", len(parent))
        first = pack_chunk(arena, [dict(key="parent", prefix=parent, f=len(parent),
                                        suffixes=[])], attention_mode="tree")
        check_pack_tree(first, 16, pool, prompts.__getitem__)
    arena.activate("doc", len(doc), borrow=("parent", borrow) if borrow else None)
    read = read_nodes(labels)
    paths = trie_paths(labels, read)
    cue = 7
    tokens = path_tokens(paths, cue)
    mask = path_reads(paths, read)
    group = dict(key="doc", prefix=doc[borrow:], f=len(doc), start=borrow, suffixes=[tokens],
                 read_all_rows=True, paths=paths, read_mask=mask, single=True,
                 read_key="parent" if borrow else None)
    chunk = pack_chunk(arena, [group], attention_mode="tree")
    contexts = path_contexts(paths, cue, doc)
    s_row0 = len(doc) - borrow

    def context(key, r):
        return None if r < s_row0 else contexts[r - s_row0]

    assert check_pack_tree(chunk, 16, pool, prompts.__getitem__, context) == s_row0 + len(tokens)
    assert chunk.final_indices.tolist() == [s_row0 + i for i, m in enumerate(mask) if m]
    assert chunk.rows_per_answer.tolist() == [sum(mask)]
    with pytest.raises(ValueError, match="paths pack one suffix"):
        pack_chunk(arena, [dict(group, read_all_rows=False)], attention_mode="tree")


@pytest.mark.parametrize("mode", ["unified", "tree"])
def test_read_rows_and_read_mask_pick_the_answer_rows(mode):
    """read_rows: the last read_rows[j] rows of suffix j answer
    (chunk.py:742-756); read_mask: the marked rows of a group's one suffix
    (:726-741). Rows 0-3 and 12-13 are the two prefixes."""
    arena = plain_arena()
    arena.activate("a", 4)
    arena.activate("b", 2)
    groups = [dict(key="a", prefix=[1, 2, 3, 4], f=4,
                   suffixes=[[10, 11, 12], [13], [14, 15, 16, 17]], read_rows=[2, 1, 3]),
              dict(key="b", prefix=[5, 6], f=2, suffixes=[[20, 21, 22]], read_mask=[1, 0, 1])]
    chunk = pack_chunk(arena, groups, attention_mode=mode)
    assert chunk.final_indices.tolist() == [5, 6, 7, 9, 10, 11, 14, 16]
    assert chunk.rows_per_answer.tolist() == [2, 1, 3, 2]
    if mode == "unified":
        # the last layer's final-row attention follows the answer rows
        fq = chunk.meta["final_query"]
        assert int(fq["cu_q"][-1]) == 8
        for t in chunk.temporary_keys:
            arena.free_key(t)
    with pytest.raises(ValueError, match="read_rows"):
        pack_chunk(arena, [dict(groups[0], read_rows=[4, 1, 1])], attention_mode=mode)
    with pytest.raises(ValueError, match="read_mask"):
        pack_chunk(arena, [dict(groups[1], read_mask=[1, 0])], attention_mode=mode)
    assert arena.free_pages == arena.num_pages - 2   # nothing left behind


def test_unified_refuses_paths_and_canvas():
    arena = plain_arena()
    arena.activate("a", 4)
    with pytest.raises(ValueError, match="tree attention"):
        pack_chunk(arena, [dict(key="a", prefix=[1, 2, 3, 4], f=4, suffixes=[[5]],
                                read_all_rows=True, paths=[([()], 0, [])])])
    with pytest.raises(ValueError, match="canvas"):
        pack_chunk(arena, [dict(key="a", prefix=[1, 2, 3, 4], f=4, suffixes=[[5]],
                                canvas=[1, 2])])
