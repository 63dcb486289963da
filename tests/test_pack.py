"""Pack layout: the reference's known answers and the structural KV-read
oracle over seeded corpora with shared prefixes (the reference drives its
HashModel checker the same way, tests/engine/test_kv_reads.py:27-122)."""

import numpy as np
import pytest

from oracle.packing_ref import PoolModel, check_pack
from quail_amd.arena import KVArena
from quail_amd.chunk import pack_chunk
from quail_amd.prefix import PrefixIndex
from tests.helpers import admit, pack_specs


def plain_arena(pages=64, page=16, layers=1):
    return KVArena(layers, pages, page, 1, 8, device="cpu")


def test_unified_causal_document_and_question_are_one_sequence():
    # tests/engine/test_pack_chunk.py:149-161
    arena = plain_arena()
    key = ("d", 0)
    arena.activate(key, 4, capacity_tokens=8, base_tokens=4)
    chunk = pack_chunk(arena, [dict(key=key, prefix=[1, 2, 3, 4], f=4, suffixes=[[10, 11]])])
    u = chunk.meta["unified"]
    assert u["cu_q_host"] == [0, 6]
    assert u["causal"]
    assert u["used_host"] == [6]
    assert chunk.host_ids.tolist() == [1, 2, 3, 4, 10, 11]
    assert chunk.host_positions.tolist() == [0, 1, 2, 3, 4, 5]
    assert chunk.final_indices.tolist() == [5]
    assert chunk.meta["cu_a"].tolist() == [0, 4, 6]
    assert u["src"].tolist() == [0, 1, 2, 3, 4, 5]
    assert u["dst"].tolist() == [0, 1, 2, 3, 4, 5]     # page 0 is the first allocated
    assert u["table"].tolist() == [[0]]
    assert chunk.fresh_keys == (key,)


def test_many_suffixes_use_temporary_pages_and_tail_copies():
    # a document of 20 tokens (one full page + 4 rows) asked three questions:
    # each question reads the full page plus a temporary page whose first
    # 4 rows are copied from the document's partial page
    arena = plain_arena()
    key = ("d", 0)
    arena.activate(key, 20)
    prompt = list(range(100, 120))
    sufs = [[1, 2], [3], [4, 5, 6]]
    chunk = pack_chunk(arena, [dict(key=key, prefix=prompt, f=20, suffixes=sufs)])
    u = chunk.meta["unified"]
    assert u["cu_q_host"] == [0, 20, 22, 23, 26]
    assert u["used_host"] == [20, 22, 21, 23]
    assert chunk.host_positions.tolist() == list(range(20)) + [20, 21, 20, 20, 21, 22]
    assert chunk.final_indices.tolist() == [21, 22, 25]
    assert len(chunk.temporary_keys) == 3
    assert u["tail_src"].tolist() == [16, 17, 18, 19] * 3
    doc_pages = arena.owned_pages(key)
    for s, temp in enumerate(chunk.temporary_keys):
        assert u["table"][s + 1][0] == doc_pages[0]
        assert u["table"][s + 1][1] == arena.owned_pages(temp)[0]
    pool = PoolModel()
    prompts = {key: prompt}
    # every question row reads the document then its own question
    pool.apply(chunk.host_ids, chunk.host_positions, u)
    from oracle.packing_ref import visible_keys
    reads = visible_keys(u, 16, pool)
    for r, suf in zip([21, 22, 25], sufs):
        want = [(t, p) for p, t in enumerate(prompt + suf)]
        assert reads[r] == want
    for temp in chunk.temporary_keys:
        arena.free_key(temp)
    arena.free_key(key)
    assert arena.free_pages == 64


def _corpus(seed, n, vocab=50, prefix_len=40):
    rng = np.random.default_rng(seed)
    prefix = rng.integers(0, vocab, prefix_len).tolist()
    docs = []
    for _ in range(n):
        # repeated prefixes of varied depth, some duplicates and short docs
        cut = int(rng.integers(0, prefix_len + 1))
        body = rng.integers(0, vocab, int(rng.integers(1, 60))).tolist()
        docs.append(prefix[:cut] + body)
    docs.append(list(docs[0]))                 # an exact duplicate
    return docs


@pytest.mark.parametrize("seed", [0, 1, 2, 3, 4, 5, 7, 11, 100, 101, 200, 201])
def test_packs_read_exactly_their_documents(seed):
    docs = _corpus(seed, 40)
    arena = plain_arena(pages=48)
    prefixes = [d[:-1] for d in docs]
    suffixes = [[d[-1:]] for d in docs]
    tree = PrefixIndex(docs).tree(16)
    adm = admit(prefixes, suffixes, arena, 256, tree=tree)
    pool = PoolModel()
    prompts = {adm.keys[i]: d for i, d in enumerate(docs)}
    checked = 0
    packs = 0
    live = []

    def settle():
        # the loop reads answers one pack late; a finished document's pages go free
        for d, first, end, _ in live.pop(0):
            if adm.report(d, first, end, [0] * (end - first)):
                arena.free_key(adm.keys[d])

    while not adm.done():
        groups = adm.next_chunk(arena.free_pages)
        prefills = adm.take_prefills()
        if not groups and not prefills:
            assert live, "nothing admitted and nothing to free"
            settle()
            continue
        chunk = pack_chunk(arena, pack_specs(adm, groups, prefills))
        checked += check_pack(chunk, 16, pool, prompts.__getitem__)
        for temp in chunk.temporary_keys:
            arena.free_key(temp)
        live.append(groups)
        packs += 1
        if len(live) > 1:
            settle()
    while live:
        settle()
    total = sum(len(d) for d in docs)
    assert checked == total - adm.borrowed_tokens
    assert packs >= 2
    assert arena.free_pages == arena.num_pages
    assert adm.borrowed_tokens > 0


def test_borrowers_read_parent_pages_written_in_the_same_pack():
    prefix = list(range(32))
    docs = [prefix + [100 + i] * (3 + i) for i in range(5)]
    arena = plain_arena()
    tree = PrefixIndex(docs).tree(16)
    adm = admit([d[:-1] for d in docs], [[d[-1:]] for d in docs], arena, 1024, tree=tree)
    groups = adm.next_chunk(arena.free_pages)
    assert len(groups) == 5 and not adm.pending
    specs = pack_specs(adm, groups)
    assert [g["start"] for g in specs] == [0, 32, 32, 32, 32]
    root = specs[0]["key"]
    chunk = pack_chunk(arena, specs)
    u = chunk.meta["unified"]
    root_pages = arena.owned_pages(root)[:2]
    for s in range(1, 5):
        assert u["table"][s][:2].tolist() == root_pages
    check_pack(chunk, 16, PoolModel(), {adm.keys[i]: d for i, d in enumerate(docs)}.__getitem__)
