"""A stage that needs every recovery path of the driver, on the GPU.

The tiny corpus (16 documents of 48-145 tokens behind a 32-token shared
prefix, the tiny Qwen3 model) asked two questions per document (the last
four prompt tokens, two each: temporary question pages), run through
StageRun and the GPU pipeline with

  * a 96-token pack budget, below the longest documents (145 tokens): those
    are prefilled in pieces and their questions run in the pass after the
    last piece (admission.py:611-648, 760-768);
  * a 20-page arena, 12 of its pages holding retained KV of an earlier
    operator: admission evicts it to reserve documents' pages
    (arena.py:584-642);
  * admission told 8 more free pages than the arena has (another operator
    taking pages between admission and packing): a pack's temporary pages
    then do not fit, retained KV is evicted and the pack retried, and once
    none is left the pack runs as two halves (stage_executor.py:1036-1062).

Every kernel is row-local and a row's attention reads its keys in the same
order wherever they sit in the pool, so each answer must equal bit for bit
the same stage run with room to spare (one pack, a large arena), and both
must match the oracle's documents run whole in float64 at the tiny model's
FP8 bounds (measured in test_gpu_forward.py).
"""

import numpy as np
import pytest
import torch

from oracle import qwen3_ref as ref
from quail_amd.model import CONFIGS, build_synthetic
from quail_amd.workload import make_workload
from tests.helpers import ref_model

pytestmark = pytest.mark.gpu

TOL = 0.05


def _run(model, prefixes, suffixes, num_pages, budget, retained=(), optimism=0):
    from quail_amd import readout as ro
    from quail_amd.arena import KVArena
    from quail_amd.executor import StageRun
    from quail_amd.model import retain_answer_head
    from quail_amd.qwen3 import Qwen3Pipeline

    class OptimisticRun(StageRun):
        def _free_pages(self):
            return self.arena.free_pages + optimism

    cfg = model.config
    arena = KVArena(cfg.layers, num_pages, 16, cfg.kv_heads, cfg.head_dim)
    for i, tokens in enumerate(retained):
        key = ("retained", i)
        assert arena.alloc(key, tokens) is not None
        arena.retain(key, tokens)
    pipe = Qwen3Pipeline(model, arena)
    retain_answer_head(model, [10, 11])
    readout = ro.AsyncMargins(ro.AnswerRows(model, [10], [11]))
    run = OptimisticRun(pipe, arena, readout, prefixes, suffixes, budget)
    results = run.run()
    torch.cuda.synchronize()
    # a document asked one question gets its answer, one asked several the list
    margins = np.array([[a[0] - a[1] for a in (r if isinstance(r, list) else [r])]
                        for r in results], dtype=np.float64)
    assert arena.free_pages + arena.retained_pages == arena.num_pages
    return margins, run, arena


def test_pieces_evictions_and_splits_give_the_same_answers():
    cfg = CONFIGS["tiny"]
    wl = make_workload("tiny", seed=0)
    model = build_synthetic(cfg, seed=0, device="cuda", gen_device="cpu", norm_init="random")
    docs = [np.asarray(p, dtype=np.int64) for p in wl.prompts]
    prefixes = [d[:-4] for d in docs]
    suffixes = [[d[-4:-2], d[-2:]] for d in docs]
    assert max(len(d) for d in docs) > 96
    print("case: tiny corpus seed 0, two questions, 96-token packs, 20-page arena", flush=True)

    got, run, arena = _run(model, prefixes, suffixes, 20, 96, retained=[64] * 3, optimism=8)
    s = run.stats
    print({k: s[k] for k in ("chunks", "prefill_pieces", "evictions", "evict_retries",
                             "splits", "borrowed_tokens")})
    assert s["prefill_pieces"] >= 1 and s["evictions"] >= 1 and s["splits"] >= 1
    assert s["evict_retries"] >= 1
    assert arena.retained_pages == 0 and arena.free_pages == 20

    print("case: the same stage in one pack, 256-page arena", flush=True)
    plain, prun, _ = _run(model, prefixes, suffixes, 256, 2048)
    assert prun.stats["chunks"] == 1 and prun.stats["prefill_pieces"] == 0
    assert np.array_equal(got, plain)

    m = ref_model(model)
    rows = m.head[[10, 11]]
    for j in range(2):
        normed = ref.forward_documents(m, [np.concatenate([p, s[j]])
                                           for p, s in zip(prefixes, suffixes)])
        yes, no, _, _ = ref.answer(normed, rows, [1, 0])
        want = (yes - no).double().numpy()
        d = np.abs(got[:, j] - want)
        print(f"question {j}: max {d.max():.4f} rms {np.sqrt(np.mean(d ** 2)):.4f} "
              f"within {TOL}: {np.mean(d <= TOL):.3f}")
        assert d.max() <= 0.075
        assert np.sum(d > TOL) <= 2
        clear = np.abs(want) > TOL
        assert np.all((got[clear, j] > 0) == (want[clear] > 0))


@pytest.mark.parametrize("length", [36_000, 40_900])
def test_a_document_past_32k_keys_in_pieces_equals_it_whole(length):
    """One document longer than two packs (Qwen3-4B's layer shapes, one
    layer, a 4096-token vocabulary), its 2-token question at positions up
    to 40,901: prefilled in 16,384-row pieces, its last piece's rows and
    question read 2250-2557 pages of its own (past the 2048 of a 32,768-key
    page table), and the answer must equal bit for bit the same document
    packed whole in one 40,960-row pass (every kernel row-local, the keys
    read in the same 64-key tiles either way)."""
    import dataclasses
    cfg = dataclasses.replace(CONFIGS["qwen3-4b"], layers=1, vocab=4096)
    model = build_synthetic(cfg, seed=3, device="cuda", gen_device="cpu", norm_init="random")
    rng = np.random.default_rng(length)
    doc = rng.integers(12, cfg.vocab, length + 2).astype(np.int64)
    prefixes, suffixes = [doc[:-2]], [[doc[-2:]]]
    pages = -(-(length + 2) // 16) + 8
    print(f"case: one {length}-token document, 16384-row pieces, {pages}-page arena", flush=True)
    got, run, _ = _run(model, prefixes, suffixes, pages, 16384)
    assert run.stats["prefill_pieces"] >= 2
    print(f"case: the same document whole, one {length + 2}-row pass", flush=True)
    whole, wrun, _ = _run(model, prefixes, suffixes, pages, 40960)
    assert wrun.stats["chunks"] == 1 and wrun.stats["prefill_pieces"] == 0
    assert np.all(np.isfinite(got))
    assert np.array_equal(got, whole)
