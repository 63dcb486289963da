"""Whole stage runs against the reference's driver, pass by pass.

tests/golden/make_pack_vectors.py ran the reference's one-stage driver loop
(StageExecutor.run / _run_part / _run_one, stage_executor.py:1036-1277)
over its own JoinAdmission with chunked prefill, KVArena and pack_chunk on
three stages whose pages bind or whose documents outgrow a pack:

  * pieces: the 16-document tiny corpus, 96-token packs (its longest
    documents are prefilled in pieces) and a 40-page arena;
  * evict: the tiny corpus (seed 1) asked two questions each (temporary
    question pages), 160-token packs and a 36-page arena that retained KV of
    an earlier operator fills in part (evictions);
  * qwen3-4b: the Qwen3-4B AI.IF benchmark with the bench's 3,136-page arena.

It recorded, for every forward pass, its question groups and prefill
pieces, the page table of every key packed, the free pages, and which
documents' answers were read after which pass, with every borrow and every
recovery (evictions, retries, splits). Here StageRun drives the same inputs
through StageAdmission, KVArena and pack_chunk with a pipeline that
computes nothing (CPU only) and a readout that answers True, and every
record must be equal.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from quail_amd.arena import KVArena
from quail_amd.executor import StageRun
from quail_amd.workload import make_workload

GOLDEN = Path(__file__).resolve().parent / "golden" / "pack_vectors.npz"
PAGE = 16
RUNS = {"pieces": ("tiny", 0), "evict": ("tiny", 1), "qwen3-4b": ("qwen3-4b", 0)}


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN) as z:
        return {k: z[k] for k in z.files}


class RecordingPipeline:
    """forward_chunk computes nothing; it records each pass's page tables
    and free pages (temporary question pages counted free, as the
    reference's record was taken after it freed them)."""

    max_chunk_tokens = 1 << 20
    engine = type("E", (), {"num_q_heads": 4, "num_kv_heads": 2, "head_dim": 64})()

    def __init__(self, arena):
        self.arena = arena
        self.run = None
        self.records = []

    def forward_chunk(self, chunk):
        groups, prefills = self.run.passes[-1]
        adm = self.run._adm
        keys = [adm.keys[d] for d, *_ in groups] + [adm.keys[d] for d, _, _ in prefills]
        temp = sum(len(self.arena.owned_pages(k)) for k in chunk.temporary_keys)
        self.records.append(dict(tables=[list(self.arena.owned_pages(k)) for k in keys],
                                 free=self.arena.free_pages + temp, rows=int(chunk.tokens)))
        return None


class TrueReadout:
    def __init__(self):
        self.submitted = 0

    def submit(self, normed, rows_per_answer=None):
        self.submitted += 1
        return self.submitted

    def result(self, handle):
        return [True] * 4096


class RecordingRun(StageRun):
    """StageRun recording which documents finish after which pass."""

    def _report_next(self):
        groups = self._outstanding[0][1]
        before = {d for d, r in enumerate(self._results) if r is not None}
        super()._report_next()
        # in the order the pass's groups settle
        self.reported.extend((len(self.passes), d) for d, *_ in groups
                             if d not in before and self._results[d] is not None)


def _run(golden, name):
    corpus, seed = RUNS[name]
    p = f"stage/{name}/"
    wl = make_workload(corpus, seed=seed)
    prompts = [np.asarray(x, dtype=np.int64) for x in wl.prompts]
    qlens = golden[p + "question_lens"].tolist()
    if qlens == [1]:
        prefixes = [x[:-1] for x in prompts]
        suffixes = [[x[-1:]] for x in prompts]
    else:
        # the reference run asked every document the same questions; their
        # token ids (7..) do not change a pack's layout
        qs = [np.arange(7, 7 + n, dtype=np.int64) + sum(qlens[:i]) for i, n in enumerate(qlens)]
        prefixes = prompts
        suffixes = [list(qs) for _ in prompts]
    arena = KVArena(1, int(golden[p + "pages"][0]), PAGE, 1, 2, device="cpu")
    for i, tokens in enumerate(golden[p + "retained"].tolist()):
        key = ("retained", i)
        assert arena.alloc(key, tokens) is not None
        arena.retain(key, tokens)
    pipe = RecordingPipeline(arena)
    run = RecordingRun(pipe, arena, TrueReadout(), prefixes, suffixes,
                       int(golden[p + "budget"][0]), staging=_HostStaging())
    run.reported = []
    pipe.run = run
    run.run()
    return run, pipe, arena


class _HostStaging:
    """upload()'s staging on the host: tensors stay on the CPU."""

    def copy(self, name, values, dtype):
        return torch.as_tensor(np.ascontiguousarray(values)).to(dtype)


@pytest.mark.parametrize("name", list(RUNS))
def test_stage_run_equals_the_reference_pass_by_pass(golden, name):
    run, pipe, arena = _run(golden, name)
    p = f"stage/{name}/"
    groups = [(i, d, first, end, int(carried))
              for i, (gs, _) in enumerate(run.passes) for d, first, end, carried in gs]
    assert groups == [tuple(x) for x in golden[p + "groups"].tolist()]
    prefills = [(i, *x) for i, (_, ps) in enumerate(run.passes) for x in ps]
    assert prefills == [tuple(x) for x in golden[p + "prefills"].tolist()]
    assert [r["rows"] for r in pipe.records] == golden[p + "rows"].tolist()
    assert [r["free"] for r in pipe.records] == golden[p + "free_pages"].tolist()
    lens = [(i, len(t)) for i, r in enumerate(pipe.records) for t in r["tables"]]
    assert lens == [tuple(x) for x in golden[p + "table_lens"].tolist()]
    flat = [x for r in pipe.records for t in r["tables"] for x in t]
    assert flat == golden[p + "tables"].tolist()
    borrows = sorted((d, par, sh) for d, (par, sh) in run._adm.lender.items())
    assert borrows == [tuple(x) for x in golden[p + "borrows"].tolist()]
    assert run.reported == [tuple(x) for x in golden[p + "reported"].tolist()]
    events = golden[p + "events"]
    kinds = {k: events[events[:, 0] == i] for i, k in enumerate(
        ("evict", "evict_retry", "split", "drop_holds", "reserve_evicted"))}
    assert run.stats["evictions"] == int(kinds["evict"][:, 2].sum()
                                         + kinds["reserve_evicted"][:, 2].sum())
    assert run.stats["evict_retries"] == len(kinds["evict_retry"])
    assert run.stats["splits"] == len(kinds["split"])
    assert run.stats["drop_holds"] == len(kinds["drop_holds"])
    # every page comes back (retained keys the run did not evict stay)
    assert arena.free_pages + arena.retained_pages == arena.num_pages


def test_the_golden_runs_exercise_pieces_binding_pages_and_evictions(golden):
    """The recorded runs hold what they are meant to pin: prefill pieces,
    documents waiting for pages, and evictions of retained KV."""
    assert len(golden["stage/pieces/prefills"]) >= 2
    assert min(golden["stage/pieces/free_pages"]) < 20
    assert golden["stage/evict/events"][:, 2].sum() >= 2
    assert len(golden["stage/qwen3-4b/rows"]) == 11
