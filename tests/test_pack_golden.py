"""Packs, page tables and unified layouts against the reference's own code.

tests/golden/pack_vectors.npz was written by tests/golden/make_pack_vectors.py
from the reference's JoinAdmission.next_chunk (admission.py:702-866),
KVArena.activate (arena.py:522-563) and pack_chunk(attention_mode="unified")
(chunk.py:505-1160) on the benchmark corpora: the first pack of the
16-document tiny workload and the first three packs of the 512-document
Qwen3-4B-shaped workload (prompt less its last token as the prefix, the last
token as the one question, prefix tree at 16-token pages, an arena large
enough that pages never bind, every answer read before the next pack, no
document released). Here the same inputs go through StageAdmission, KVArena
and pack_chunk, and every array must be equal.
"""

from pathlib import Path

import numpy as np
import pytest

from quail_amd.arena import KVArena
from quail_amd.chunk import pack_chunk
from quail_amd.prefix import PrefixIndex
from quail_amd.workload import make_workload
from tests.helpers import admit, pack_specs

GOLDEN = Path(__file__).resolve().parent / "golden" / "pack_vectors.npz"
PAGE = 16
BIG_ARENA = 20000
PACKS = {"tiny": 1, "qwen3-4b": 3}


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN) as z:
        return {k: z[k] for k in z.files}


def _packs(name):
    wl = make_workload(name, seed=0)
    prompts = [np.asarray(p, dtype=np.int64) for p in wl.prompts]
    tree = PrefixIndex([p.tolist() for p in prompts]).tree(PAGE)
    arena = KVArena(1, BIG_ARENA, PAGE, 1, 2, device="cpu")
    adm = admit([p[:-1] for p in prompts], [[p[-1:]] for p in prompts], arena,
                wl.chunk_budget, tree=tree)
    for _ in range(PACKS[name]):
        groups = adm.next_chunk(arena.free_pages)
        assert not adm.take_prefills()
        docs = [d for d, *_ in groups]
        chunk = pack_chunk(arena, pack_specs(adm, groups))
        yield adm, arena, docs, chunk


def _flat(x):
    return np.asarray(x, dtype=np.int64).reshape(-1)


@pytest.mark.parametrize("name", list(PACKS))
def test_packs_equal_the_reference(golden, name):
    for pack, (adm, arena, docs, chunk) in enumerate(_packs(name)):
        p = f"{name}/{pack}/"
        assert docs == golden[p + "docs"].tolist(), pack
        lenders = [adm.lender.get(d, (-1, 0)) for d in docs]
        assert [lp for lp, _ in lenders] == golden[p + "lenders"].tolist()
        assert [t for _, t in lenders] == golden[p + "lent"].tolist()
        tables = [arena.owned_pages(adm.keys[d]) for d in docs]
        assert [len(t) for t in tables] == golden[p + "table_lens"].tolist()
        assert [x for t in tables for x in t] == golden[p + "tables"].tolist()
        u = chunk.meta["unified"]
        np.testing.assert_array_equal(_flat(chunk.host_ids), golden[p + "input_ids"])
        np.testing.assert_array_equal(_flat(chunk.host_positions), golden[p + "positions"])
        np.testing.assert_array_equal(_flat(chunk.final_indices), golden[p + "final_indices"])
        np.testing.assert_array_equal(_flat(chunk.meta["cu_a"]), golden[p + "cu_a"])
        for field in ("cu_q", "used", "src", "dst", "tail_src", "tail_dst"):
            got = u.get(field)
            got = np.empty(0, np.int64) if got is None else _flat(got)
            np.testing.assert_array_equal(got, golden[p + field], err_msg=f"{p}{field}")
        table = np.asarray(u["table"], dtype=np.int64)
        assert list(table.shape) == golden[p + "table_shape"].tolist()
        np.testing.assert_array_equal(table.reshape(-1), golden[p + "table"])


def test_multi_question_pack_equals_the_reference(golden):
    """Documents asked one to three questions each: every question reads the
    document's full pages plus temporary pages whose first rows are copied
    from its partial last page (the tail copies)."""
    p = "multi/"
    wl = make_workload("tiny", seed=0)
    prompts = [np.asarray(x, dtype=np.int64) for x in wl.prompts]
    lens = golden[p + "question_lens"].tolist()
    flat = golden[p + "questions"].tolist()
    qs, at = [], 0
    for n in lens:
        qs.append(flat[at:at + n])
        at += n
    questions, at = [], 0
    for n in golden[p + "questions_per_doc"].tolist():
        questions.append(qs[at:at + n])
        at += n
    arena = KVArena(1, 4000, PAGE, 1, 2, device="cpu")
    groups = []
    for d, (prompt, same) in enumerate(zip(prompts, golden[p + "lent"].tolist())):
        key = ("doc", d)
        borrow = (("doc", 0), same) if same else None
        assert arena.activate(key, len(prompt), borrow=borrow) is not None
        groups.append(dict(key=key, prefix=prompt[same:], f=len(prompt), start=same,
                           suffixes=questions[d]))
    chunk = pack_chunk(arena, groups)
    u = chunk.meta["unified"]
    assert len(u["tail_src"]) > 0
    np.testing.assert_array_equal(_flat(chunk.host_ids), golden[p + "input_ids"])
    np.testing.assert_array_equal(_flat(chunk.host_positions), golden[p + "positions"])
    np.testing.assert_array_equal(_flat(chunk.final_indices), golden[p + "final_indices"])
    np.testing.assert_array_equal(_flat(chunk.meta["cu_a"]), golden[p + "cu_a"])
    for field in ("cu_q", "used", "src", "dst", "tail_src", "tail_dst"):
        np.testing.assert_array_equal(_flat(u[field]), golden[p + field], err_msg=field)
    table = np.asarray(u["table"], dtype=np.int64)
    assert list(table.shape) == golden[p + "table_shape"].tolist()
    np.testing.assert_array_equal(table.reshape(-1), golden[p + "table"])
