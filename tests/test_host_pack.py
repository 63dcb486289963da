"""The C++ page accounting and unified packer against their plain-Python
restatements (oracle.pages_ref, oracle.pack_ref), bit for bit, over seeded
random operation sequences and pack layouts: every page id handed out, every
free stack, every block table, scatter map, tail copy and offset array.
The restatements themselves are pinned by the reference's known answers
(tests/test_pages.py, tests/test_pack.py)."""

import random

import numpy as np
import pytest

from oracle.pack_ref import ArenaFullError as RefArenaFull
from oracle.pack_ref import pack_unified_ref
from oracle.pages_ref import RefArena, RefPageArena
from quail_amd.arena import KVArena
from quail_amd.chunk import ArenaFullError, pack_chunk
from quail_amd.pages import PageArena


def _same_state(mine: PageArena, ref: RefPageArena):
    assert mine.free_list() == ref.free
    assert mine.free_pages == ref.free_pages
    assert mine.retained_pages == ref.retained_pages
    assert mine.resident_tokens == ref.resident_tokens
    assert mine.retained_prefix_tokens == ref.retained_prefix_tokens
    assert mine.resident_keys() == list(ref.owned)
    for key in ref.owned:
        assert mine.borrowed_pages(key) == ref.borrowed[key], key
        assert mine.owned_pages(key) == ref.owned[key], key
        assert mine.key_tokens(key) == ref.tokens[key], key
    assert mine.pinned == ref.pinned
    assert mine.retained == ref.retained


def _both(mine, ref, name, *args, **kw):
    """Run one operation on both; they must return the same or raise the same type."""
    try:
        want = getattr(ref, name)(*args, **kw)
    except (KeyError, ValueError) as err:
        with pytest.raises(type(err)):
            getattr(mine, name)(*args, **kw)
        return None
    got = getattr(mine, name)(*args, **kw)
    assert got == want, (name, args, got, want)
    return got


@pytest.mark.parametrize("seed", range(6))
def test_page_pool_matches_the_restatement(seed):
    rng = random.Random(seed)
    page = rng.choice([4, 16])
    mine, ref = PageArena(48, page), RefPageArena(48, page)
    made = 0
    for _ in range(400):
        live = list(ref.owned)
        op = rng.random()
        if op < 0.35 or not live:
            key = f"k{made}"
            made += 1
            tokens = rng.randrange(0, 6 * page)
            cap = tokens + rng.choice([0, 0, rng.randrange(0, 3 * page)])
            borrowed = []
            if live and rng.random() < 0.5:
                parent = rng.choice(live)
                whole = ref.tokens[parent] // page * page
                shared = rng.randrange(0, whole + 1, page) if whole else 0
                shared = min(shared, tokens // page * page)
                borrowed = _both(mine, ref, "shared_pages", parent, shared) or []
            _both(mine, ref, "alloc", key, tokens, cap, borrowed)
        elif op < 0.5:
            _both(mine, ref, "free_key", rng.choice(live))
        elif op < 0.58:
            key = rng.choice(live)
            _both(mine, ref, "rewind", key, rng.randrange(0, 6 * page))
        elif op < 0.66:
            _both(mine, ref, "grow", rng.choice(live), rng.randrange(0, 8 * page))
        elif op < 0.7:
            _both(mine, ref, "drop_leading", rng.choice(live), rng.randrange(0, 3))
        elif op < 0.78:
            _both(mine, ref, "pin", rng.choice(live))
        elif op < 0.9:
            key = rng.choice(live)
            if rng.random() < 0.3:
                prio = float(rng.randrange(0, 5))
                _both(mine, ref, "retain", key, (prio,))
            else:
                _both(mine, ref, "retain", key)
        else:
            keep = frozenset(rng.sample(live, min(len(live), rng.randrange(0, 3))))
            victim = _both(mine, ref, "pop_retained_victim", keep)
            if victim is not None:
                _both(mine, ref, "free_key", victim[0])
        _same_state(mine, ref)


def _arenas(pages, page):
    return KVArena(1, pages, page, 1, 8, device="cpu"), RefArena(pages, page)


def _random_groups(rng, mine, ref, page, docs):
    """Activate `docs` documents (some borrowing an earlier one's prefix) in
    both arenas and return their groups."""
    groups, made = [], []
    for d in range(docs):
        key = ("doc", d, rng.random())
        f = rng.randrange(1, 5 * page)
        start, borrow = 0, None
        if made and rng.random() < 0.4:
            parent, pf = rng.choice(made)
            shared = min(pf - 1, f - 1) // page * page
            if shared > 0:
                start, borrow = shared, (parent, shared)
        n = rng.choice([0, 1, 1, 1, 2, 3])
        sufs = [rng.sample(range(1000), rng.randrange(0, 2 * page)) for _ in range(n)]
        direct_room = n == 1 and rng.random() < 0.6
        cap = f + (len(sufs[0]) if direct_room else 0)
        fresh = rng.random() < 0.8
        got_m = mine.activate(key, f, capacity_tokens=cap, borrow=borrow)
        got_r = ref.activate(key, f, capacity_tokens=cap, borrow=borrow)
        assert got_m == got_r
        if got_r is None:
            continue
        made.append((key, f))
        g = dict(key=key, f=f, start=start, suffixes=sufs,
                 read_all_rows=rng.random() < 0.2)
        if fresh:
            g["prefix"] = rng.sample(range(1000), f - start)
        if direct_room and fresh and rng.random() < 0.5:
            g["write_suffix_tokens"] = len(sufs[0])
        groups.append(g)
    return groups


def _same_pack(chunk, want, mine, ref):
    u, w = chunk.meta["unified"], want["unified"]
    assert np.array_equal(chunk.host_ids, want["ids"])
    assert np.array_equal(chunk.host_positions, want["positions"])
    assert np.array_equal(chunk.final_indices, want["finals"])
    assert np.array_equal(chunk.meta["cu_a"], want["cu_a"])
    assert chunk.tokens == want["tokens"]
    assert chunk.layout == want["layout"]
    assert chunk.row_spans == want["row_spans"]
    assert chunk.fresh_keys == want["fresh_keys"]
    if want["rows_per_answer"] is None:
        assert chunk.rows_per_answer is None
    else:
        assert np.array_equal(chunk.rows_per_answer, want["rows_per_answer"])
    for name in ("src", "dst", "used", "cu_q", "table"):
        assert u[name].dtype == w[name].dtype, name
        assert np.array_equal(u[name], w[name]), name
    for name in ("tail_src", "tail_dst"):
        assert (u[name] is None) == (w[name] is None), name
        if w[name] is not None:
            assert np.array_equal(u[name], w[name]), name
    for name in ("cu_q_host", "used_host", "page_rows", "max_q", "max_used", "causal"):
        assert u[name] == w[name], name
    assert [mine.owned_pages(t) for t in chunk.temporary_keys] == \
        [ref.owned_pages(t) for t in want["temporary_keys"]]


@pytest.mark.parametrize("seed", range(8))
def test_pack_matches_the_restatement(seed):
    rng = random.Random(100 + seed)
    page = rng.choice([4, 16])
    mine, ref = _arenas(rng.choice([40, 400]), page)
    for _ in range(4):
        groups = _random_groups(rng, mine, ref, page, rng.randrange(1, 12))
        try:
            want = pack_unified_ref(ref, groups)
        except (RefArenaFull, ValueError) as err:
            kind = ArenaFullError if isinstance(err, RefArenaFull) else ValueError
            with pytest.raises(kind):
                pack_chunk(mine, groups)
            assert mine.accounting.free_list() == ref.accounting.free
            continue
        chunk = pack_chunk(mine, groups)
        _same_pack(chunk, want, mine, ref)
        for t in chunk.temporary_keys:
            mine.free_key(t)
        for t in want["temporary_keys"]:
            ref.free_key(t)
        assert mine.accounting.free_list() == ref.accounting.free


def test_pack_that_does_not_fit_leaves_no_pages_behind():
    mine, ref = _arenas(4, 16)
    key = ("doc", 0)
    mine.activate(key, 20)
    ref.activate(key, 20)
    groups = [dict(key=key, prefix=list(range(20)), f=20, suffixes=[[1] * 30, [2] * 30])]
    with pytest.raises(RefArenaFull):
        pack_unified_ref(ref, groups)
    free = mine.accounting.free_list()
    with pytest.raises(ArenaFullError):
        pack_chunk(mine, groups)
    assert mine.accounting.free_list() == free == ref.accounting.free


def test_kept_suffix_that_needs_temporaries_is_refused():
    """Keeping suffix KV in the key's pages needs the direct layout; with two
    suffixes both packers refuse the group, and nothing stays allocated."""
    mine, ref = _arenas(16, 16)
    key = ("doc", 0)
    mine.activate(key, 20, capacity_tokens=40)
    ref.activate(key, 20, capacity_tokens=40)
    groups = [dict(key=key, prefix=list(range(20)), f=20, suffixes=[[1, 2], [3]],
                   write_suffix_tokens=2)]
    with pytest.raises(ValueError, match="keeps suffix KV"):
        pack_unified_ref(ref, groups)
    with pytest.raises(ValueError, match="keeps suffix KV"):
        pack_chunk(mine, groups)
    assert mine.accounting.free_list() == ref.accounting.free
