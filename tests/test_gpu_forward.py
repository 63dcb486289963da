"""End-to-end parity of the packed prefill pass on the GPU.

The tiny Qwen3 configuration (2 layers, hidden 256, 4/2 heads, D 64,
random-init, 16 documents behind a 32-token shared prefix, one 2048-row
pack) against the oracle (oracle/qwen3_ref.py, itself pinned against torch
and transformers in tests/test_oracle_pins.py). The oracle runs each
document's prompt whole (no pages, no borrowing), so a wrong page table,
scatter map, position or borrowed prefix shows up here.

Two oracle precisions. The reference's torch dequantized path computes its
matmuls and attention in float32 (the torch path on the CPU); the oracle
in float64 is the exact value of the same arithmetic. The float64 oracle is
the checker here.

Why the bar is not asserted per document over many random seeds: FP8
activation quantization makes this network amplify any rounding
difference (one e4m3 code flip moves a value by 1/16, and flips seed more
flips), and random-init margins crowd zero (1% of them within 0.006).
Measured over 512 documents per norm init (32 seeds): the float32 torch
path itself agrees with the exact float64 value on 98.8-99.0% of decisions
(max |d| 0.05, rms 0.011-0.012). This engine against float64: 98.0-98.6%
within 0.05, max 0.064, rms 0.021, 97.7-98.6% of decisions, every decision
whose exact margin is outside +-0.05. The two sources are gfx950's FP8 MFMA,
which rounds inside its dot product (mean relative error 9e-5 against the
exact block sum; bf16 MFMA on the same operands 6e-7), and the attention's
fp16 P; with both contractions replaced by exact ones (everything else the
engine's own kernels) the pass reaches 100% within 0.05 and 99.8% of
decisions, and either one left in alone already reaches rms ~0.02.
test_exact_contractions_meet_the_bar_on_every_document asserts that strictly.
"""

import numpy as np
import pytest
import torch

from oracle import qwen3_ref as ref
from quail_amd.model import CONFIGS, build_synthetic
from quail_amd.workload import make_workload
from tests.helpers import exact_contractions, ref_model, run_stage

pytestmark = pytest.mark.gpu

TOL = 0.05


def _margins(model, wl, **kwargs):
    results, run = run_stage(model, wl, "margins", **kwargs)
    ym = np.array([r[0] - r[1] for r in results], dtype=np.float64)
    return ym, run


def _oracle_margins(model, wl, precision=torch.float64):
    m = ref_model(model)
    ref.set_precision(precision)
    try:
        normed = ref.forward_documents(m, wl.prompts)
        rows = m.head[list(wl.label_ids[:2])]
        yes, no, bits, _ = ref.answer(normed, rows, [1, 0], mode=0)
    finally:
        ref.set_precision(torch.float64)
    return (yes - no).double().numpy(), normed


def _report(name, got, want):
    d = np.abs(got - want)
    agree = np.mean((got > 0) == (want > 0))
    print(f"{name}: n={len(d)} within {TOL}: {np.mean(d <= TOL):.4f} max {d.max():.4f} "
          f"rms {np.sqrt(np.mean(d ** 2)):.4f} decisions agree {agree:.4f}")
    return d, agree


@pytest.mark.parametrize("norm_init", ["ones", "random"])
def test_config1_margins(norm_init):
    """Config 1 (seed 0, one 2048-row pack, 15 documents borrowing the
    32-token prefix) against the float32 oracle (the reference's torch
    path's precision): every margin within 0.05. Against the float64 oracle: at most 0.06 from it, at
    most one document past 0.05 (measured: random norm weights max 0.045,
    all 16 within; norm weights 1 max 0.051, one at 0.051), and the same
    decision on every document whose exact margin is outside +-0.05 (the
    one that differs has |margin| 0.007). A one-ulp change of the bf16
    rotary cache alone moves the exact oracle's margins by up to 0.023 here,
    so a per-document 0.05 bound sits on the noise floor (module doc)."""
    cfg = CONFIGS["tiny"]
    wl = make_workload("tiny", seed=0)
    model = build_synthetic(cfg, seed=0, device="cuda", gen_device="cpu", norm_init=norm_init)
    got, run = _margins(model, wl)
    want, _ = _oracle_margins(model, wl)
    assert run.stats["chunks"] == 1
    assert run.stats["borrowed_tokens"] == 15 * 32      # 2 pages by 15 documents
    d, agree = _report(f"config 1 ({norm_init} norms) vs float64", got, want)
    assert d.max() <= 0.06
    assert np.sum(d > TOL) <= 1
    clear = np.abs(want) > TOL
    assert np.all((got[clear] > 0) == (want[clear] > 0))
    # the reference's torch dequantized path itself computes in float32: the
    # north-star bound holds against it on every document (measured max
    # 0.0498 / 0.0410); the one decision that differs (15 of 16) is a
    # document whose float32 margin is -0.006 / +0.017
    want32, _ = _oracle_margins(model, wl, precision=torch.float32)
    d32, agree32 = _report(f"config 1 ({norm_init} norms) vs float32", got, want32)
    assert np.all(d32 <= TOL)
    clear32 = np.abs(want32) > TOL
    assert np.all((got[clear32] > 0) == (want32[clear32] > 0))
    assert agree32 >= 15 / 16


@pytest.mark.parametrize("norm_init", ["ones", "random"])
def test_tiny_margins_against_exact_math(norm_init):
    """8 seeds x 16 documents against the float64 oracle, at the bounds the
    FP8 noise floor allows (module docstring; measured within 0.969 / 0.984,
    max 0.054 / 0.062, rms 0.021, decisions 0.984): no margin further than
    0.075, rms at most 0.025, >= 96% within 0.05, every decision whose exact
    margin is outside +-0.05 the same, >= 97.5% of all decisions."""
    cfg = CONFIGS["tiny"]
    got_all, want_all = [], []
    for seed in range(8):
        wl = make_workload("tiny", seed=seed)
        model = build_synthetic(cfg, seed=seed, device="cuda", gen_device="cpu",
                                norm_init=norm_init)
        got, _ = _margins(model, wl)
        want, _ = _oracle_margins(model, wl)
        got_all.append(got)
        want_all.append(want)
    got = np.concatenate(got_all)
    want = np.concatenate(want_all)
    d, agree = _report(f"8 seeds ({norm_init} norms) vs float64", got, want)
    assert d.max() <= 0.075
    assert np.sqrt(np.mean(d ** 2)) <= 0.025
    assert np.mean(d <= TOL) >= 0.96
    clear = np.abs(want) > TOL
    assert np.all((got[clear] > 0) == (want[clear] > 0))
    assert agree >= 0.975


@pytest.mark.parametrize("mode", ["unified", "tree"])
def test_bf16_v_arena_the_reference_layout(mode):
    """The reference's KVArena holds V in bf16 (arena.py:111-121): on such an
    arena the engine writes V rows as they are and runs the PV product in
    bf16, as FlashAttention does. 16 seeds x 16 documents against the
    float64 oracle (bf16 probabilities keep 8 bits instead of fp16's 11, so
    the spread is the tree path's): max 0.1, rms <= 0.03, >= 95% within
    0.05, every decision whose exact margin is outside +-0.05 the same,
    >= 97% of all."""
    cfg = CONFIGS["tiny"]
    got_all, want_all = [], []
    for seed in range(16):
        wl = make_workload("tiny", seed=seed)
        model = build_synthetic(cfg, seed=seed, device="cuda", gen_device="cpu",
                                norm_init="ones")
        got, _ = _margins(model, wl, v_dtype=torch.bfloat16, attention_mode=mode)
        want, _ = _oracle_margins(model, wl)
        got_all.append(got)
        want_all.append(want)
    got = np.concatenate(got_all)
    want = np.concatenate(want_all)
    d, agree = _report(f"bf16 V arena ({mode})", got, want)
    assert d.max() <= 0.1
    assert np.sqrt(np.mean(d ** 2)) <= 0.03
    assert np.mean(d <= TOL) >= 0.95
    clear = np.abs(want) > TOL
    assert np.all((got[clear] > 0) == (want[clear] > 0))
    assert agree >= 0.97


@pytest.mark.parametrize("norm_init", ["ones", "random"])
def test_exact_contractions_meet_the_bar_on_every_document(monkeypatch, norm_init):
    """Decomposition: the engine with its two MFMA contractions (the FP8
    GEMMs and the paged attention) replaced by exact float64 ones on the GPU
    and everything else its own (packing, pages, embedding, every norm and
    quantization kernel, qk-norm-rope with the KV page writes, the final
    norm and the answer head) meets the north-star bar against the float64
    oracle on every one of 8 seeds x 16 documents: all margins within 0.05
    and >= 99.5% of decisions (measured 100%, max 0.043). What separates
    the engine from it is the MFMAs' rounding alone."""
    exact_contractions(monkeypatch)
    cfg = CONFIGS["tiny"]
    got_all, want_all = [], []
    for seed in range(8):
        wl = make_workload("tiny", seed=seed)
        model = build_synthetic(cfg, seed=seed, device="cuda", gen_device="cpu",
                                norm_init=norm_init)
        got, _ = _margins(model, wl)
        want, _ = _oracle_margins(model, wl)
        got_all.append(got)
        want_all.append(want)
    got = np.concatenate(got_all)
    want = np.concatenate(want_all)
    d, agree = _report(f"exact contractions ({norm_init} norms)", got, want)
    assert np.all(d <= TOL)
    assert agree >= 0.995


def test_tiny_if_score_and_classify_readouts():
    cfg = CONFIGS["tiny"]
    wl = make_workload("tiny", seed=1)
    model = build_synthetic(cfg, seed=1, device="cuda", gen_device="cpu", norm_init="random")
    m = ref_model(model)
    normed = ref.forward_documents(m, wl.prompts)
    bits, _ = run_stage(model, wl, "if")
    yes, no, want_bits, _ = ref.answer(normed, m.head[[10, 11]], [1, 0], mode=0)
    margin = (yes - no).numpy()
    clear = np.abs(margin) > TOL
    assert np.all(np.array(bits)[clear] == want_bits.numpy()[clear])
    scores, _ = run_stage(model, wl, "score")
    _, _, _, want_score = ref.answer(normed, m.head[[10, 11]], [1, 0], mode=1)
    # sigmoid'(x) <= 1/4, so a 0.05 margin tolerance is 0.0125 on the score
    np.testing.assert_allclose(np.asarray(scores), want_score.numpy(), atol=0.025)
    wl4 = make_workload("tiny", seed=1)
    wl4.label_ids = (10, 11, 12, 13)
    logits, _ = run_stage(model, wl4, "classify")
    want_logits = ref.label_logits(normed, m.head[[10, 11, 12, 13]], mode=0)
    np.testing.assert_allclose(np.stack(logits), want_logits.numpy(), atol=0.05)


@pytest.mark.parametrize("mode", ["unified", "tree"])
@pytest.mark.parametrize("v_dtype", [torch.float16, torch.bfloat16])
def test_kv_write_in_qk_norm_rope_is_bit_identical(monkeypatch, mode, v_dtype):
    """The pipeline with K and V written by the qk-norm-rope pass (into the
    pages, qk_norm_rope_kv; as contiguous K and V rows for the tree
    path, qk_norm_rope_rows) gives the same margins, bit for bit, as with
    the separate qk_norm_rope + kv_scatter, and takes the fused path on
    every layer of every pack."""
    from quail_amd.engine import Engine

    cfg = CONFIGS["tiny"]
    wl = make_workload("tiny", seed=5)
    model = build_synthetic(cfg, seed=5, device="cuda", gen_device="cpu", norm_init="random")
    calls = []
    name = "qk_norm_rope_kv" if mode == "unified" else "qk_norm_rope_rows"
    fused = getattr(Engine, name)

    def counted(self, *args, **kwargs):
        calls.append(1)
        return fused(self, *args, **kwargs)

    monkeypatch.setattr(Engine, name, counted)
    base, _ = run_stage(model, wl, "margins", fuse_kv_write=False, attention_mode=mode,
                        v_dtype=v_dtype)
    assert not calls
    got, run = run_stage(model, wl, "margins", fuse_kv_write=True, attention_mode=mode,
                         v_dtype=v_dtype, fuse_q_norm=False)
    assert len(calls) == cfg.layers * run.stats["chunks"]
    assert len(got) == len(base)
    assert all(np.array_equal(np.asarray(a), np.asarray(b)) for a, b in zip(got, base))


def test_tiny_paged_oracle_agrees_on_the_same_pack():
    """The oracle's paged path over this engine's own pack equals the dense
    per-document oracle (pins pack metadata numerically), and the GPU's
    final rows match it."""
    from quail_amd.arena import KVArena
    from quail_amd.chunk import InputStaging, pack_chunk, upload
    from quail_amd.prefix import PrefixIndex
    from quail_amd.qwen3 import Qwen3Pipeline
    from tests.helpers import admit, pack_specs

    cfg = CONFIGS["tiny"]
    wl = make_workload("tiny", seed=2)
    model = build_synthetic(cfg, seed=2, device="cuda", gen_device="cpu", norm_init="random")
    arena = KVArena(cfg.layers, 256, 16, cfg.kv_heads, cfg.head_dim)
    prefixes, suffixes = wl.groups_input()
    tree = PrefixIndex(wl.prompts).tree(16)
    adm = admit(prefixes, suffixes, arena, wl.chunk_budget, tree=tree)
    groups = adm.next_chunk(arena.free_pages)
    assert not adm.pending and not adm.take_prefills()
    chunk = pack_chunk(arena, pack_specs(adm, groups))
    host_unified = dict(chunk.meta["unified"])
    final = chunk.final_indices.copy()
    upload(chunk, InputStaging())
    normed = Qwen3Pipeline(model, arena).forward_chunk(chunk).float().cpu()
    m = ref_model(model)
    pools = [(torch.zeros(256 * 16, cfg.kv_heads, cfg.head_dim, dtype=torch.bfloat16),
              torch.zeros(256 * 16, cfg.kv_heads, cfg.head_dim, dtype=torch.bfloat16))
             for _ in range(cfg.layers)]
    paged = ref.forward_chunk(m, chunk.host_ids, chunk.host_positions, final, host_unified,
                              pools, 16)
    order = [d for d, *_ in groups]
    dense = ref.forward_documents(m, [wl.prompts[d] for d in order])
    torch.testing.assert_close(paged.float(), dense.float(), rtol=0.02, atol=0.02)
    rel = ((normed - dense.float()).norm() / dense.float().norm()).item()
    assert rel <= 0.06, rel     # the FP8 noise floor of the tiny model (see module doc)


@pytest.mark.parametrize("mode", ["unified", "tree"])
def test_read_rows_answers_equal_those_rows_of_read_all(mode):
    """Several trailing answer rows per suffix (read_rows, chunk.py:742-756):
    the same pack read with read_all_rows gives the same final-normed rows,
    bit for bit (every kernel is row-local; in the unified pack the last
    layer attends for the answer rows only)."""
    from quail_amd.arena import KVArena
    from quail_amd.chunk import InputStaging, pack_chunk, upload
    from quail_amd.qwen3 import Qwen3Pipeline

    cfg = CONFIGS["tiny"]
    model = build_synthetic(cfg, seed=6, device="cuda", gen_device="cpu", norm_init="random")
    docs = make_workload("tiny", seed=6).prompts[:3]
    outs = {}
    for name in ("all", "rows"):
        arena = KVArena(cfg.layers, 256, 16, cfg.kv_heads, cfg.head_dim)
        pipe = Qwen3Pipeline(model, arena)
        groups = []
        for i, d in enumerate(docs):
            d = [int(t) for t in d]
            arena.activate(i, len(d) - 8)
            g = dict(key=i, prefix=d[:-8], f=len(d) - 8, suffixes=[d[-8:-5], d[-5:]])
            g.update(read_all_rows=True) if name == "all" else g.update(read_rows=[2, 3])
            groups.append(g)
        chunk = pack_chunk(arena, groups, attention_mode=mode,
                           attention_heads=(cfg.heads, cfg.kv_heads, cfg.head_dim))
        final = chunk.final_indices.copy()
        upload(chunk, InputStaging())
        outs[name] = (pipe.forward_chunk(chunk).float().cpu(), final.tolist())
    (all_rows, all_final), (got, final) = outs["all"], outs["rows"]
    assert len(final) == 3 * 5 and got.shape[0] == len(final)
    pick = [all_final.index(r) for r in final]
    assert torch.equal(got, all_rows[pick])
