"""The Qwen3-8B and Qwen3-32B-shaped configurations at their real layer shapes.

These models are too large for the oracle at full size, so the checks are
properties that hold at any size (the model is cut to its first two layers;
every layer runs the same kernels at the same shapes):

  * packing invariance: every kernel on the path computes a row from that
    row alone (GEMM rows, norms, quantization, rotary embedding) or from its
    own sequence's keys in a fixed 64-key tiling from key 0 (attention), so a
    document's answer must be bit-identical whether it is packed with the
    others and borrows the shared instruction prefix from its parent, or runs
    alone and computes every row itself;
  * the AI.SCORE value is sigmoid(yes - no) of the AI.IF logits (readout.py
    :331-336 against :44-48), and AI.CLASSIFY returns one logit per label id.

The Qwen3-32B shape also runs the 64/8-head grouping (8 query heads per KV
head, two workgroup groups per KV head in the attention grid).
"""

import dataclasses

import numpy as np
import pytest
import torch

from quail_amd.model import CONFIGS, build_synthetic
from quail_amd.workload import make_workload
from tests.helpers import run_stage

pytestmark = pytest.mark.gpu

LAYERS = 2


def _subset(wl, docs):
    return dataclasses.replace(wl, prompts=[wl.prompts[d] for d in docs])


def _alone(model, wl, kind):
    out = []
    for d in range(wl.documents):
        res, run = run_stage(model, _subset(wl, [d]), kind)
        assert run.stats["borrowed_tokens"] == 0
        out.append(res[0])
    return out


@pytest.mark.parametrize("name,docs", [("qwen3-8b", 6), ("qwen3-32b", 10)])
def test_packed_answers_equal_documents_run_alone(name, docs):
    wl = make_workload(name, seed=3, documents=docs)
    cfg = CONFIGS[wl.model]
    model = build_synthetic(cfg, seed=3, device="cuda", layers=LAYERS)
    kind = "classify" if wl.function == "classify" else "margins"
    packed, run = run_stage(model, wl, kind)
    # the shared instruction prefix (whole pages of it) is borrowed, not recomputed
    shared_pages = wl.prefix_tokens // 16
    assert run.stats["borrowed_tokens"] == (docs - 1) * shared_pages * 16
    alone = _alone(model, wl, kind)
    for d in range(docs):
        a = np.asarray(packed[d], dtype=np.float64)
        b = np.asarray(alone[d], dtype=np.float64)
        assert np.array_equal(a, b), (name, d, a, b)
    if kind == "classify":
        assert all(len(r) == len(wl.label_ids) for r in packed)


def test_q_norm_on_load_is_bit_identical(monkeypatch):
    """The attention normalizing and rotating q as it loads it (the
    qk-norm-rope pass then writes K and V only) gives the same classify
    logits, bit for bit, as the pass writing q too, and runs on every layer
    of every pack (the last layer's final-row attention included)."""
    from quail_amd.engine import Engine

    wl = make_workload("qwen3-8b", seed=6, documents=6)
    model = build_synthetic(CONFIGS[wl.model], seed=6, device="cuda", layers=LAYERS)
    calls = []
    fused = Engine.kv_norm_rope

    def counted(self, *args, **kwargs):
        calls.append(1)
        return fused(self, *args, **kwargs)

    monkeypatch.setattr(Engine, "kv_norm_rope", counted)
    base, _ = run_stage(model, wl, "classify", fuse_q_norm=False)
    assert not calls
    got, run = run_stage(model, wl, "classify", fuse_q_norm=True)
    assert len(calls) == LAYERS * run.stats["chunks"]
    assert len(got) == len(base)
    assert all(np.array_equal(np.asarray(a), np.asarray(b)) for a, b in zip(got, base))


def test_score_is_sigmoid_of_if_margin():
    wl = make_workload("qwen3-32b", seed=4, documents=8)
    model = build_synthetic(CONFIGS[wl.model], seed=4, device="cuda", layers=LAYERS)
    margins, _ = run_stage(model, wl, "margins")
    scores, _ = run_stage(model, wl, "score")
    ym = np.array([y - n for y, n in margins], dtype=np.float64)
    want = 1.0 / (1.0 + np.exp(-ym))
    got = np.asarray(scores, dtype=np.float64).reshape(-1)
    # the score uses fp32 logits, the margins bf16-rounded ones (readout.py:44-48)
    np.testing.assert_allclose(got, want, atol=2e-2)


def test_last_layer_on_final_rows_only_is_bit_identical():
    """The last layer attends, projects and runs its MLP for the final rows
    only (chunk.meta["final_query"]); without that metadata the pipeline
    runs it for every row. The final rows must not change."""
    from quail_amd.arena import KVArena
    from quail_amd.chunk import InputStaging, pack_chunk, upload
    from quail_amd.prefix import PrefixIndex
    from quail_amd.qwen3 import Qwen3Pipeline
    from tests.helpers import admit, pack_specs

    wl = make_workload("qwen3-8b", seed=5, documents=5)
    cfg = CONFIGS[wl.model]
    model = build_synthetic(cfg, seed=5, device="cuda", layers=LAYERS)
    outs = []
    for pruned in (True, False):
        arena = KVArena(LAYERS, 3 * wl.chunk_budget // 16 + 64, 16, cfg.kv_heads, cfg.head_dim)
        prefixes, suffixes = wl.groups_input()
        tree = PrefixIndex(wl.prompts).tree(16)
        adm = admit(prefixes, suffixes, arena, wl.chunk_budget, tree=tree)
        groups = adm.next_chunk(arena.free_pages)
        assert not adm.pending and not adm.take_prefills()
        chunk = pack_chunk(arena, pack_specs(adm, groups))
        upload(chunk, InputStaging())
        if not pruned:
            chunk.meta["final_query"] = None
        outs.append(Qwen3Pipeline(model, arena).forward_chunk(chunk).clone())
    assert outs[0].shape == (wl.documents, cfg.hidden)
    assert torch.equal(outs[0], outs[1])
