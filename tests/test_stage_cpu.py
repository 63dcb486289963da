"""The stage driver's admission and recovery paths, on the CPU.

StageRun (quail_amd/executor.py) drives admission, packing and the page
accounting exactly as on the GPU; here its pipeline is the oracle's paged
forward (oracle/qwen3_ref.forward_chunk over CPU pools, the same pack
metadata the GPU kernels read), so every answer can be checked against the
document run whole, and the arena's page counts after the stage show that
nothing leaked. Covered (reference behaviour in parentheses):

  * a document longer than one pack is prefilled in pieces
    (admission.py:611-648, 817; stage_executor.py:1176-1189);
  * an arena too small for the stage at once: documents wait for answered
    documents' pages;
  * a pack whose question pages do not fit: answers in flight are read,
    retained KV is evicted, then the part runs as two halves
    (stage_executor.py:1036-1062).
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from oracle import qwen3_ref as ref
from quail_amd import _lib
from quail_amd.admission import OversizedDocumentError, StageAdmission
from quail_amd.arena import KVArena
from quail_amd.executor import StageRun
from quail_amd.model import CONFIGS, build_synthetic
from quail_amd.prefix import PrefixIndex
from tests.helpers import admit, ref_model

CFG = CONFIGS["tiny"]
PAGE = 16


class HostStaging:
    """The pinned upload ring's interface, for a CPU run."""

    def copy(self, name, values, dtype):
        return torch.as_tensor(np.ascontiguousarray(values)).to(dtype)


class OraclePipeline:
    """The pipeline contract (forward_chunk -> final-normed rows) computed by
    the oracle's paged forward over per-layer CPU pools the size of the arena."""

    def __init__(self, model, arena):
        self.m = ref_model(model)
        self.engine = SimpleNamespace(num_q_heads=CFG.heads, num_kv_heads=CFG.kv_heads,
                                      head_dim=CFG.head_dim)
        self.max_chunk_tokens = 1 << 20
        rows = arena.num_pages * PAGE
        self.pools = [(torch.zeros(rows, CFG.kv_heads, CFG.head_dim, dtype=torch.bfloat16),
                       torch.zeros(rows, CFG.kv_heads, CFG.head_dim, dtype=torch.bfloat16))
                      for _ in range(CFG.layers)]
        self.rows_per_pack = []

    def forward_chunk(self, chunk):
        self.rows_per_pack.append(chunk.tokens)
        unified = chunk.host.get("unified", chunk.meta["unified"])
        return ref.forward_chunk(self.m, chunk.host_ids, chunk.host_positions,
                                 np.asarray(chunk.final_indices), unified, self.pools, PAGE)


class MarginReadout:
    """AI.IF margins (yes - no on ids 10, 11) of the final rows, read one pack late."""

    def __init__(self, m):
        self.rows = m.head[[10, 11]]

    def submit(self, normed, rows_per_answer=None):
        return normed

    def result(self, normed):
        yes, no, _, _ = ref.answer(normed, self.rows, [1, 0])
        return (yes - no).double().tolist()


def _model(seed):
    return build_synthetic(CFG, seed=seed, device="cpu", norm_init="random")


def _docs(seed, lengths, shared=32):
    rng = np.random.default_rng(seed)
    prefix = rng.integers(0, CFG.vocab, shared)
    return [np.concatenate([prefix, rng.integers(0, CFG.vocab, n)]).astype(np.int64)
            for n in lengths]


def _run(model, arena, prefixes, suffixes, budget):
    pipe = OraclePipeline(model, arena)
    run = StageRun(pipe, arena, MarginReadout(pipe.m), prefixes, suffixes, budget,
                   staging=HostStaging())
    return run.run(), run, pipe


def _whole(model, prompts):
    m = ref_model(model)
    normed = ref.forward_documents(m, prompts)
    yes, no, _, _ = ref.answer(normed, m.head[[10, 11]], [1, 0])
    return (yes - no).double().numpy()


def test_document_longer_than_a_pack_is_prefilled_in_pieces():
    """Budget 96 rows: the 250- and 130-token documents go in pieces (their
    children wait for the whole prefix, then read its pages); every answer
    equals the document run whole and every page comes back."""
    model = _model(1)
    docs = _docs(1, [40, 250, 20, 130, 8, 60])
    docs[1][200] = 0
    # a child of the long one: it sorts after it, so it reads the long one's pages
    docs.append(np.concatenate([docs[1][:200], [CFG.vocab - 1] * 3]))
    assert PrefixIndex(docs).tree(PAGE).parent[6] == 1
    arena = KVArena(CFG.layers, 64, PAGE, CFG.kv_heads, CFG.head_dim, device="cpu")
    prefixes, suffixes = [d[:-1] for d in docs], [[d[-1:]] for d in docs]
    got, run, pipe = _run(model, arena, prefixes, suffixes, budget=96)
    assert run.stats["prefill_pieces"] >= 3
    assert max(pipe.rows_per_pack) <= 96
    assert run.stats["borrowed_tokens"] >= 192     # the child reads 12 pages of the long one
    want = _whole(model, docs)
    np.testing.assert_allclose(np.array(got), want, atol=0.05)
    assert arena.free_pages == arena.num_pages


def test_admission_pieces_cover_each_prefix_once_in_order():
    """The pieces of a long document tile its prefix: consecutive, no gap,
    none past the pack budget, each filling the room the pack has left;
    its question runs in the pack after its last piece (admission.py:
    611-648, 760-768)."""
    docs = _docs(2, [300, 10])
    arena = KVArena(CFG.layers, 64, PAGE, CFG.kv_heads, CFG.head_dim, device="cpu")
    adm = admit([d[:-1] for d in docs], [[d[-1:]] for d in docs], arena, 100)
    pieces, questions, packs = [], {}, 0
    while not adm.done():
        groups = adm.next_chunk(arena.free_pages)
        prefills = adm.take_prefills()
        assert groups or prefills
        rows = sum(end - start for _, start, end in prefills)
        for d, first, end, carried in groups:
            rows += (adm.flen[d] if carried else 0) + end - first
            questions[d] = (packs, carried)
            adm.report(d, first, end, [True] * (end - first))
        assert rows <= 100
        pieces += [(packs, d, start, end) for d, start, end in prefills]
        packs += 1
    spans = [(start, end) for _, d, start, end in pieces if d == 0]
    assert spans[0][0] == 0 and all(a[1] == b[0] for a, b in zip(spans, spans[1:]))
    assert spans[-1][1] == len(docs[0]) - 1 and len(spans) >= 3
    last_piece = max(i for i, d, _, _ in pieces if d == 0)
    assert questions[0] == (last_piece + 1, False)
    assert questions[1][1]                  # the short one packs whole, with its question


def test_tiny_arena_answers_every_document():
    """20 documents, an arena of 24 pages (the stage needs ~90): admission
    waits for answered documents' pages; every answer equals the document
    run whole and no page leaks."""
    model = _model(3)
    rng = np.random.default_rng(3)
    docs = _docs(3, rng.integers(20, 120, 20).tolist())
    arena = KVArena(CFG.layers, 24, PAGE, CFG.kv_heads, CFG.head_dim, device="cpu")
    prefixes, suffixes = [d[:-1] for d in docs], [[d[-1:]] for d in docs]
    got, run, pipe = _run(model, arena, prefixes, suffixes, budget=512)
    assert run.stats["chunks"] >= 4
    np.testing.assert_allclose(np.array(got), _whole(model, docs), atol=0.05)
    assert arena.free_pages == arena.num_pages


def _two_questions(docs):
    return [d[:-4] for d in docs], [[d[-4:-2], d[-2:]] for d in docs]


def test_full_arena_evicts_retained_kv():
    """Retained KV of an earlier operator fills the arena; documents with two
    questions each need their pages and temporary question pages, which only
    evicting the retained keys provides (arena.py:584-642)."""
    model = _model(4)
    docs = _docs(4, [30, 45, 50], shared=16)
    arena = KVArena(CFG.layers, 24, PAGE, CFG.kv_heads, CFG.head_dim, device="cpu")
    for i in range(4):
        key = ("retained", i)
        assert arena.alloc(key, 4 * PAGE) is not None
        arena.retain(key)
    prefixes, suffixes = _two_questions(docs)
    got, run, _ = _run(model, arena, prefixes, suffixes, budget=512)
    assert run.stats["evictions"] >= 1
    assert arena.evicted_keys == run.stats["evictions"]
    want_a = _whole(model, [np.concatenate([p, s[0]]) for p, s in zip(prefixes, suffixes)])
    # each question follows the prefix directly (its positions restart at f)
    want_b = _whole(model, [np.concatenate([p, s[1]]) for p, s in zip(prefixes, suffixes)])
    np.testing.assert_allclose(np.array([g[0] for g in got]), want_a, atol=0.05)
    np.testing.assert_allclose(np.array([g[1] for g in got]), want_b, atol=0.05)
    assert arena.free_pages == arena.num_pages - arena.retained_pages


class OptimisticRun(StageRun):
    """Admission told `extra` more free pages than the arena has, as when
    another operator takes pages between admission and packing: a pack's
    temporary question pages then do not fit (ArenaFullError)."""

    extra = 0

    def _free_pages(self):
        return self.arena.free_pages + self.extra


def test_full_arena_splits_the_part():
    """A pack of four two-question documents whose question pages exceed
    the free arena, nothing retained to evict: the part runs as two halves
    (stage_executor.py:1036-1062); every answer equals the document run
    whole and no page leaks."""
    model = _model(5)
    docs = _docs(5, [20, 25, 30, 35], shared=0)
    prefixes, suffixes = _two_questions(docs)
    need = sum(-(-len(p) // PAGE) for p in prefixes)
    # five pages past the documents' own: the four documents' question pages
    # (2 + 2 + 2 + 4) do not fit at once, each half does
    arena = KVArena(CFG.layers, need + 5, PAGE, CFG.kv_heads, CFG.head_dim, device="cpu")
    pipe = OraclePipeline(model, arena)
    run = OptimisticRun(pipe, arena, MarginReadout(pipe.m), prefixes, suffixes, 512,
                        staging=HostStaging())
    run.extra = 8
    got = run.run()
    assert run.stats["splits"] >= 1
    for j in range(2):
        want = _whole(model, [np.concatenate([p, s[j]]) for p, s in zip(prefixes, suffixes)])
        np.testing.assert_allclose(np.array([g[j] for g in got]), want, atol=0.05)
    assert arena.free_pages == arena.num_pages


def test_oversized_documents_are_refused_up_front():
    arena = KVArena(CFG.layers, 8, PAGE, CFG.kv_heads, CFG.head_dim, device="cpu")
    docs = _docs(6, [200])
    with pytest.raises(OversizedDocumentError, match="whole arena"):
        StageAdmission([docs[0][:-1]], [[docs[0][-1:]]], arena, 1024)
    with pytest.raises(OversizedDocumentError, match="question exceeds"):
        StageAdmission([docs[0][:10]], [[docs[0][10:200]]], KVArena(
            CFG.layers, 64, PAGE, CFG.kv_heads, CFG.head_dim, device="cpu"), 100)


def test_documents_past_the_attention_key_limit_are_refused_up_front():
    """The paged attention stages at most 2560 page ids (40,960 keys at
    16-token pages, Qwen3's whole context) per sequence: a longer document
    passes the arena and chunked-prefill checks but is refused at
    admission; one at the limit is admitted."""
    limit = _lib.count("qx_paged_attention_max_keys", PAGE)
    assert limit == 2560 * PAGE == 40960
    arena = KVArena(1, 4096, PAGE, CFG.kv_heads, CFG.head_dim, device="cpu")
    rng = np.random.default_rng(0)
    long_doc = rng.integers(0, CFG.vocab, limit + 1)
    with pytest.raises(OversizedDocumentError, match="40960 per sequence"):
        StageAdmission([long_doc[:-1]], [[long_doc[-1:]]], arena, 16384)
    ok = long_doc[:limit]
    StageAdmission([ok[:-1]], [[ok[-1:]]], arena, 16384)
    with pytest.raises(_lib.QxError, match="page of 32 tokens"):
        _lib.count("qx_paged_attention_max_keys", 32)


def test_children_wait_for_a_parent_mid_prefill():
    """A child of a long document is held until the parent's last prefix
    piece is packed, then reads its pages (same pack or later)."""
    docs = _docs(7, [280])
    docs[0][260] = 0
    child = np.concatenate([docs[0][:260], [CFG.vocab - 1] * 3])
    docs = [docs[0], child]
    tree = PrefixIndex(docs).tree(PAGE)
    assert tree.order[0] == 0 and tree.parent[1] == 0
    arena = KVArena(CFG.layers, 64, PAGE, CFG.kv_heads, CFG.head_dim, device="cpu")
    adm = admit([d[:-1] for d in docs], [[d[-1:]] for d in docs], arena, 100, tree=tree)
    parent = tree.order[0]
    child_doc = 1 - parent
    packs = []
    while not adm.done():
        groups = adm.next_chunk(arena.free_pages)
        packs.append((groups, adm.take_prefills()))
        for d, first, end, _ in groups:
            adm.report(d, first, end, [True] * (end - first))
    first_child = next(i for i, (g, _) in enumerate(packs) if any(x[0] == child_doc for x in g))
    last_parent_piece = max(i for i, (_, p) in enumerate(packs) for d, _, _ in p if d == parent)
    assert first_child > last_parent_piece
    assert adm.shared(child_doc) == tree.shared[child_doc] > 0
    assert adm.parent(child_doc) == parent
