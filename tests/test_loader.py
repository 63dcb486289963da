"""Local Qwen3 FP8 checkpoints (quail_amd.loader) and the MI355X device spec
(quail_amd.device).

The loader restates what the reference gets from vLLM's loader
(model_loading.py:288-363): q/k/v merged into qkv_proj, gate/up into
gate_up_proj, each with its weight_scale_inv row blocks, the head tied to
the embedding when the config says so. A seeded model written in the
Hugging Face layout (tests/helpers.py: write_hf_checkpoint, split back into
q/k/v and gate/up over two shards) must load back bit for bit.
tests/golden/qwen3-4b-fp8.config.json is the reference's own fixture
(tests/fixtures/qwen3_configs/qwen3-4b-fp8.json, the published
Qwen/Qwen3-4B-FP8 config.json). A checkpoint written by transformers and
huggingface_hub (not by this package) must load to what transformers itself
reads from it.
"""

import dataclasses
import json
from pathlib import Path

import pytest
import torch

from quail_amd.device import MI355X, DeviceSpec, read_device
from quail_amd.loader import config_from_json, load_qwen3_fp8, read_config
from quail_amd.model import CONFIGS, build_synthetic
from tests.helpers import write_hf_checkpoint

GOLDEN = Path(__file__).resolve().parent / "golden"


def _same(a, b):
    if a.dtype == torch.float8_e4m3fn:
        a, b = a.view(torch.uint8), b.view(torch.uint8)
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(a, b)


def test_published_qwen3_4b_fp8_config_is_the_benchmark_model():
    with open(GOLDEN / "qwen3-4b-fp8.config.json") as f:
        cfg = config_from_json(json.load(f), name="qwen3-4b")
    assert cfg == CONFIGS["qwen3-4b"]
    assert cfg.gemm_flops_per_token() == pytest.approx(7.267e9, rel=1e-3)


@pytest.mark.parametrize("tied", [True, False])
def test_checkpoint_round_trip_is_bit_exact(tmp_path, tied):
    cfg = dataclasses.replace(CONFIGS["tiny"], tied_head=tied)
    model = build_synthetic(cfg, seed=4, device="cpu", norm_init="random")
    path = write_hf_checkpoint(model, cfg, tmp_path / "ckpt", shards=2)
    assert read_config(path) == dataclasses.replace(cfg, name="ckpt")
    loaded = load_qwen3_fp8(path, device="cpu")
    assert len(loaded.model.layers) == cfg.layers
    for mine, theirs in zip(loaded.model.layers, model.model.layers):
        for lin in ("qkv_proj", "o_proj"):
            for t in ("weight", "weight_scale_inv"):
                assert _same(getattr(getattr(mine.self_attn, lin), t),
                             getattr(getattr(theirs.self_attn, lin), t)), (lin, t)
        for lin in ("gate_up_proj", "down_proj"):
            for t in ("weight", "weight_scale_inv"):
                assert _same(getattr(getattr(mine.mlp, lin), t),
                             getattr(getattr(theirs.mlp, lin), t)), (lin, t)
        for n in ("q_norm", "k_norm"):
            assert _same(getattr(mine.self_attn, n).weight, getattr(theirs.self_attn, n).weight)
            assert getattr(mine.self_attn, n).variance_epsilon == cfg.eps
        for n in ("input_layernorm", "post_attention_layernorm"):
            assert _same(getattr(mine, n).weight, getattr(theirs, n).weight)
        assert (mine.self_attn.num_heads, mine.self_attn.num_kv_heads,
                mine.self_attn.head_dim) == (cfg.heads, cfg.kv_heads, cfg.head_dim)
        assert _same(mine.self_attn.rotary_emb.cos_sin_cache,
                     theirs.self_attn.rotary_emb.cos_sin_cache)
    assert _same(loaded.model.embed_tokens.weight, model.model.embed_tokens.weight)
    assert _same(loaded.model.norm.weight, model.model.norm.weight)
    assert _same(loaded.lm_head.weight, model.lm_head.weight)
    assert (loaded.lm_head.weight is loaded.model.embed_tokens.weight) == tied


@pytest.mark.parametrize("tied", [True, False])
def test_checkpoint_written_by_transformers(tmp_path, monkeypatch, tied):
    """A checkpoint written by independent code (transformers' Qwen3 names,
    its Fp8Quantize block quantization, huggingface_hub sharding, its
    config.json with rope_parameters and a FineGrainedFP8Config) read by
    the loader, against transformers' own reading of the same files
    (from_pretrained without a GPU dequantizes the FP8 weights, value =
    weight * weight_scale_inv per 128x128 block): every merged projection,
    norm, embedding and head equal, and the oracle's forward over the
    loaded model (FP8 activation quantization off, as transformers has
    none) equal to transformers' forward within the few bf16 ulps of the
    oracle's storage roundings."""
    from transformers import Qwen3ForCausalLM

    from oracle import qwen3_ref as ref
    from oracle.fp8 import dequant_weight
    from quail_amd.workload import make_workload
    from tests.helpers import ref_model, write_transformers_fp8_checkpoint

    cfg = dataclasses.replace(CONFIGS["tiny"], tied_head=tied)
    path = write_transformers_fp8_checkpoint(cfg, tmp_path / "ckpt", seed=3)
    assert len(list(path.glob("*.safetensors"))) > 1
    assert read_config(path) == dataclasses.replace(cfg, name="ckpt")
    loaded = load_qwen3_fp8(path, device="cpu")
    theirs = Qwen3ForCausalLM.from_pretrained(path, dtype=torch.float32).eval()
    theirs.config._attn_implementation = "eager"
    d, hq, hk, inter = cfg.head_dim, cfg.heads, cfg.kv_heads, cfg.intermediate
    dq = lambda lin: dequant_weight(lin.weight, lin.weight_scale_inv)
    for mine, th in zip(loaded.model.layers, theirs.model.layers):
        a, ta = mine.self_attn, th.self_attn
        assert torch.equal(dq(a.qkv_proj), torch.cat([ta.q_proj.weight, ta.k_proj.weight,
                                                      ta.v_proj.weight]))
        assert torch.equal(dq(a.o_proj), ta.o_proj.weight)
        assert torch.equal(dq(mine.mlp.gate_up_proj),
                           torch.cat([th.mlp.gate_proj.weight, th.mlp.up_proj.weight]))
        assert torch.equal(dq(mine.mlp.down_proj), th.mlp.down_proj.weight)
        for n in ("q_norm", "k_norm"):
            assert torch.equal(getattr(a, n).weight.float(), getattr(ta, n).weight)
        for n in ("input_layernorm", "post_attention_layernorm"):
            assert torch.equal(getattr(mine, n).weight.float(), getattr(th, n).weight)
        assert a.qkv_proj.weight.shape == ((hq + 2 * hk) * d, cfg.hidden)
        assert mine.mlp.gate_up_proj.weight.shape == (2 * inter, cfg.hidden)
    assert torch.equal(loaded.model.embed_tokens.weight.float(), theirs.model.embed_tokens.weight)
    assert torch.equal(loaded.model.norm.weight.float(), theirs.model.norm.weight)
    assert torch.equal(loaded.lm_head.weight.float(), theirs.lm_head.weight)
    docs = make_workload("tiny", seed=3).prompts[:4]
    monkeypatch.setattr(ref, "group_quant",
                        lambda y: (y.float(), torch.ones(y.shape[0], y.shape[1] // 128)))
    got = ref.forward_documents(ref_model(loaded), docs).float()
    with torch.no_grad():
        want = torch.stack([theirs.model(input_ids=torch.tensor([list(doc)]))
                            .last_hidden_state[0, -1] for doc in docs])
    rel = (got - want).norm(dim=1) / want.norm(dim=1)
    assert float(rel.max()) <= 0.02, rel
    head = theirs.lm_head.weight.detach()
    lg, lw = got @ head.T, want @ head.T
    assert float((lg - lw).abs().max()) <= 0.02 * float(lw.abs().max()) + 0.01


def test_rope_parameters_are_read_and_checked():
    """transformers 5 writes the rotary base as rope_parameters.rope_theta;
    a rope_type other than default is refused like rope_scaling."""
    with open(GOLDEN / "qwen3-4b-fp8.config.json") as f:
        config = json.load(f)
    theta = config.pop("rope_theta")
    config["rope_parameters"] = {"rope_type": "default", "rope_theta": theta}
    assert config_from_json(config, name="qwen3-4b") == CONFIGS["qwen3-4b"]
    config["rope_parameters"]["rope_type"] = "yarn"
    with pytest.raises(ValueError, match="rope_parameters"):
        config_from_json(config)


def test_keeps_the_first_layers(tmp_path):
    cfg = CONFIGS["tiny"]
    model = build_synthetic(cfg, seed=5, device="cpu")
    path = write_hf_checkpoint(model, cfg, tmp_path / "ckpt", shards=1)
    loaded = load_qwen3_fp8(path, device="cpu", num_layers=1)
    assert len(loaded.model.layers) == 1
    with pytest.raises(ValueError, match="cannot keep"):
        load_qwen3_fp8(path, device="cpu", num_layers=cfg.layers + 1)


def _rewrite_config(path, **changes):
    with open(path / "config.json") as f:
        config = json.load(f)
    config.update(changes)
    with open(path / "config.json", "w") as f:
        json.dump(config, f)


@pytest.mark.parametrize("changes,match", [
    ({"quantization_config": {"quant_method": "fp8", "weight_block_size": [64, 64]}}, "blocks"),
    ({"quantization_config": None}, "FP8"),
    ({"rope_scaling": {"type": "yarn", "factor": 4.0}}, "rope_scaling"),
    ({"model_type": "llama", "architectures": ["LlamaForCausalLM"]}, "Qwen3ForCausalLM"),
    ({"use_sliding_window": True}, "sliding"),
])
def test_rejects_checkpoints_this_engine_does_not_run(tmp_path, changes, match):
    cfg = CONFIGS["tiny"]
    path = write_hf_checkpoint(build_synthetic(cfg, seed=1, device="cpu"), cfg, tmp_path / "c")
    _rewrite_config(path, **changes)
    with pytest.raises(ValueError, match=match):
        load_qwen3_fp8(path, device="cpu")


def test_missing_or_mistyped_tensors_raise(tmp_path):
    from safetensors.torch import load_file, save_file

    cfg = CONFIGS["tiny"]
    path = write_hf_checkpoint(build_synthetic(cfg, seed=2, device="cpu"), cfg, tmp_path / "c",
                               shards=1)
    shard = next(path.glob("*.safetensors"))
    tensors = load_file(str(shard))
    bad = dict(tensors)
    bad["model.layers.0.self_attn.o_proj.weight_scale_inv"] = \
        tensors["model.layers.0.self_attn.o_proj.weight_scale_inv"].to(torch.float16)
    save_file(bad, str(shard))
    with pytest.raises(ValueError, match="o_proj.weight_scale_inv"):
        load_qwen3_fp8(path, device="cpu")
    missing = {k: v for k, v in tensors.items() if "layers.1.mlp.up_proj.weight" not in k}
    save_file(missing, str(shard))
    index = json.loads((path / "model.safetensors.index.json").read_text())
    index["weight_map"] = {k: v for k, v in index["weight_map"].items() if k in missing}
    (path / "model.safetensors.index.json").write_text(json.dumps(index))
    with pytest.raises(KeyError, match="up_proj"):
        load_qwen3_fp8(path, device="cpu")


def test_mi355x_device_spec():
    """The published MI355X figures (288 GB HBM3E at 8 TB/s; dense FP8 5.0,
    bf16 2.5, FP4 10.1 PFLOP/s; vector FP32 157.3 TFLOP/s) in the
    reference's DeviceSpec fields (quail/specs/base.py:404-420)."""
    assert MI355X.name == "mi355x"
    assert MI355X.mem_bytes == 288e9 and MI355X.hbm_bw == 8e12
    assert (MI355X.fp8_flops, MI355X.bf16_flops, MI355X.fp4_flops) == (5.0e15, 2.5e15, 10.1e15)
    assert MI355X.fp32_flops == 157.3e12
    assert MI355X.page_tokens == 16
    reference_fields = {"name", "mem_bytes", "hbm_bw", "fp8_flops", "bf16_flops", "fp32_flops",
                        "usd_per_hour", "price_source", "cuda_name", "modal_gpu", "page_tokens",
                        "mamf_fp8_flops", "mamf_bf16_flops", "fp4_flops"}
    assert {f.name for f in dataclasses.fields(DeviceSpec)} == reference_fields


def test_device_spec_checks(tmp_path):
    good = (Path(__file__).resolve().parent.parent / "quail_amd/devices/mi355x.toml").read_text()
    bad_key = tmp_path / "mi355x.toml"
    bad_key.write_text(good + "\nwarp_size = 64\n")
    with pytest.raises(ValueError, match="unknown keys"):
        read_device(bad_key)
    renamed = tmp_path / "mi350x.toml"
    renamed.write_text(good)
    with pytest.raises(ValueError, match="differs"):
        read_device(renamed)
    zero = tmp_path / "mi355x.toml"
    zero.write_text(good.replace("bf16_flops = 2.5e15", "bf16_flops = 0"))
    with pytest.raises(ValueError, match="bf16_flops"):
        read_device(zero)
