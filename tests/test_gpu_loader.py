"""A checkpoint loaded from disk (quail_amd.loader) drives the whole stage:
written in the Hugging Face Qwen3 FP8 layout and loaded back onto the
device, it gives the same AI.IF margins, bit for bit, as the model it was
written from."""

import numpy as np
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
