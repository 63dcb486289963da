"""A checkpoint loaded from disk (quail_amd.loader) drives the whole stage:
written in the Hugging Face Qwen3 FP8 layout and loaded back onto the
device, it gives the same AI.IF margins, bit for bit, as the model it was
written from."""

import numpy as np
import torch
import pytest

from quail_amd.loader import load_qwen3_fp8
from quail_amd.model import CONFIGS, build_synthetic
from quail_amd.workload import make_workload
from tests.helpers import run_stage, write_hf_checkpoint

pytestmark = pytest.mark.gpu


def test_loaded_checkpoint_answers_equal_the_written_model(tmp_path):
    wl = make_workload("tiny", seed=7)
    cfg = CONFIGS[wl.model]
    model = build_synthetic(cfg, seed=7, device="cuda", norm_init="random")
    path = write_hf_checkpoint(model, cfg, tmp_path / "ckpt", shards=3)
    loaded = load_qwen3_fp8(path, device="cuda")
    want, _ = run_stage(model, wl, "margins")
    got, _ = run_stage(loaded, wl, "margins")
    assert np.array_equal(np.asarray(got, dtype=np.float64), np.asarray(want, dtype=np.float64))


def test_engine_on_a_checkpoint_written_by_transformers(tmp_path):
    """The stage on a checkpoint written by transformers and huggingface_hub
    (tests/helpers.py: write_transformers_fp8_checkpoint; its loading is
    pinned tensor by tensor against transformers' own reading in
    test_loader.py), against the oracle over the same loaded weights: the
    engine's AI.IF margins within the tiny model's FP8 bounds of the exact
    (float64) margins (max 0.075, rms 0.025), no further from them than 3x
    the float32 torch path is, and the same decision wherever the exact
    margin is outside +-0.05."""
    from oracle import qwen3_ref as ref
    from tests.helpers import ref_model, write_transformers_fp8_checkpoint

    wl = make_workload("tiny", seed=3)
    cfg = CONFIGS[wl.model]
    path = write_transformers_fp8_checkpoint(cfg, tmp_path / "ckpt", seed=3)
    loaded = load_qwen3_fp8(path, device="cuda")
    got, run = run_stage(loaded, wl, "margins")
    got = np.asarray([r[0] - r[1] for r in got], dtype=np.float64)
    assert run.stats["borrowed_tokens"] > 0
    m = ref_model(loaded)
    rows = m.head[list(wl.label_ids[:2])]
    want = {}
    try:
        for prec in (torch.float64, torch.float32):
            ref.set_precision(prec)
            yes, no, _, _ = ref.answer(ref.forward_documents(m, wl.prompts), rows, [1, 0], mode=0)
            want[prec] = (yes - no).double().numpy()
    finally:
        ref.set_precision(torch.float64)
    exact, f32 = want[torch.float64], want[torch.float32]
    d = np.abs(got - exact)
    rms = float(np.sqrt(np.mean(d ** 2)))
    floor = float(np.sqrt(np.mean((f32 - exact) ** 2)))
    print(f"transformers-written checkpoint: margins std {exact.std():.3f}, engine max "
          f"{d.max():.4f} rms {rms:.4f}, float32 path rms {floor:.4f}")
    assert np.isfinite(got).all()
    assert d.max() <= 0.075 and rms <= 0.025
    assert rms <= 3 * max(floor, 1e-3)
    clear = np.abs(exact) > 0.05
    assert np.all((got[clear] > 0) == (exact[clear] > 0))
