"""Qwen3 FP8 checkpoints from a local directory.

The reference loads a checkpoint through vLLM's model loader
(quail/backends/quail/executor/model_loading.py:288-363), which reads the
Hugging Face `Qwen/Qwen3-*-FP8` files and builds the module surface the
pipeline reads: q/k/v projections merged into `qkv_proj` (rows q|k|v),
gate/up into `gate_up_proj` (rows gate|up), each FP8 linear keeping its
e4m3 `weight` (N, K) and fp32 `weight_scale_inv` (N/128, K/128). This module
reads the same files directly (config.json and the safetensors shards, no
download, no vLLM) and returns the object `quail_amd.model.build_synthetic`
returns, so `Qwen3Pipeline` runs it unchanged.

Only what the Qwen3 FP8 path needs is accepted: `Qwen3ForCausalLM`, FP8
e4m3 weights with 128x128 blocks and dynamic activation scales, no rope
scaling, no sliding window. Anything else raises.
"""

import json
from pathlib import Path
from types import SimpleNamespace

import torch

from quail_amd.model import (BLOCK, Embedding, Qwen3Config, _linear, _norm, rope_cache)

INDEX = "model.safetensors.index.json"


def config_from_json(config: dict, name: str = "checkpoint") -> Qwen3Config:
    """Qwen3Config from a Hugging Face config.json dictionary.

    Raises:
        ValueError: not a Qwen3 FP8 block-quantized checkpoint this engine runs.
    """
    archs = config.get("architectures") or []
    if config.get("model_type") != "qwen3" or "Qwen3ForCausalLM" not in archs:
        raise ValueError(f"{name}: not a Qwen3ForCausalLM checkpoint "
                         f"(model_type={config.get('model_type')!r}, architectures={archs})")
    quant = config.get("quantization_config") or {}
    if (quant.get("quant_method") != "fp8" or quant.get("fmt", "e4m3") != "e4m3"
            or list(quant.get("weight_block_size") or []) != [BLOCK, BLOCK]
            or quant.get("activation_scheme", "dynamic") != "dynamic"):
        raise ValueError(f"{name}: needs FP8 e4m3 weights in {BLOCK}x{BLOCK} blocks with "
                         f"dynamic activation scales, got quantization_config={quant}")
    if config.get("rope_scaling"):
        raise ValueError(f"{name}: rope_scaling {config['rope_scaling']} is not supported")
    # transformers 5 writes the rotary settings as rope_parameters
    # {"rope_type", "rope_theta", ...} instead of a top-level rope_theta
    rope = config.get("rope_parameters") or {}
    if rope.get("rope_type", "default") != "default":
        raise ValueError(f"{name}: rope_parameters {rope} is not supported (only default rope)")
    theta = config.get("rope_theta", rope.get("rope_theta"))
    if config.get("use_sliding_window"):
        raise ValueError(f"{name}: sliding-window attention is not supported")
    if config.get("attention_bias"):
        raise ValueError(f"{name}: attention bias is not supported")
    if config.get("hidden_act", "silu") != "silu":
        raise ValueError(f"{name}: hidden_act {config.get('hidden_act')!r} is not silu")
    heads = int(config["num_attention_heads"])
    hidden = int(config["hidden_size"])
    return Qwen3Config(
        name=name,
        layers=int(config["num_hidden_layers"]),
        hidden=hidden,
        heads=heads,
        kv_heads=int(config.get("num_key_value_heads", heads)),
        head_dim=int(config.get("head_dim") or hidden // heads),
        intermediate=int(config["intermediate_size"]),
        vocab=int(config["vocab_size"]),
        eps=float(config.get("rms_norm_eps", 1e-6)),
        theta=float(10000.0 if theta is None else theta),
        max_positions=int(config.get("max_position_embeddings", 40960)),
        tied_head=bool(config.get("tie_word_embeddings", False)),
    )


def read_config(path) -> Qwen3Config:
    """The Qwen3Config of a checkpoint directory (its config.json)."""
    path = Path(path)
    with open(path / "config.json") as f:
        return config_from_json(json.load(f), name=path.name)


class _Tensors:
    """Tensor names -> safetensors files of a checkpoint directory, opened
    lazily (one safe_open per file), read on the CPU."""

    def __init__(self, path: Path):
        from safetensors import safe_open

        self._open = safe_open
        index = path / INDEX
        if index.exists():
            with open(index) as f:
                weight_map = json.load(f)["weight_map"]
            self.files = {name: path / file for name, file in weight_map.items()}
        else:
            self.files = {}
            shards = sorted(path.glob("*.safetensors"))
            if not shards:
                raise FileNotFoundError(f"{path}: no *.safetensors files")
            for shard in shards:
                with safe_open(str(shard), framework="pt", device="cpu") as f:
                    for name in f.keys():
                        self.files[name] = shard
        self._handles = {}

    def __contains__(self, name):
        return name in self.files

    def get(self, name: str) -> torch.Tensor:
        if name not in self.files:
            raise KeyError(f"checkpoint has no tensor {name!r}")
        file = self.files[name]
        handle = self._handles.get(file)
        if handle is None:
            handle = self._handles[file] = self._open(str(file), framework="pt", device="cpu")
        return handle.get_tensor(name)


def _expect(t: torch.Tensor, name: str, dtype, shape):
    if t.dtype != dtype or tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: expected {dtype} {tuple(shape)}, "
                         f"got {t.dtype} {tuple(t.shape)}")
    return t


def load_qwen3_fp8(path, device="cuda", num_layers: int | None = None):
    """Load a local Qwen3 FP8 checkpoint into the pipeline's module surface.

    Args:
        path: directory holding config.json and model*.safetensors (with
            model.safetensors.index.json when sharded).
        device: where the weights go.
        num_layers: keep only the first layers (model_loading.keep_layers,
            model_loading.py:263-285); every layer's tensors must exist.

    Returns:
        An object with `model.layers[i].self_attn.{qkv_proj, o_proj, q_norm,
        k_norm, rotary_emb, num_heads, num_kv_heads, head_dim}`,
        `mlp.{gate_up_proj, down_proj}`, the two layer norms,
        `model.embed_tokens`, `model.norm`, `lm_head.weight` (the embedding
        when the head is tied) and `config` (a Qwen3Config).
    """
    path = Path(path)
    cfg = read_config(path)
    if num_layers is not None and not 0 < num_layers <= cfg.layers:
        raise ValueError(f"the checkpoint has {cfg.layers} layers; cannot keep {num_layers}")
    tensors = _Tensors(path)
    fp8, bf16, f32 = torch.float8_e4m3fn, torch.bfloat16, torch.float32
    h, d, hq, hk, inter = cfg.hidden, cfg.head_dim, cfg.heads, cfg.kv_heads, cfg.intermediate
    for n in (hq * d, hk * d, h, inter):
        if n % BLOCK:
            raise ValueError(f"{path.name}: width {n} is not a multiple of {BLOCK}")

    def dense(name, n, k):
        w = _expect(tensors.get(f"{name}.weight"), f"{name}.weight", fp8, (n, k))
        s = _expect(tensors.get(f"{name}.weight_scale_inv"), f"{name}.weight_scale_inv", f32,
                    (n // BLOCK, k // BLOCK))
        return w, s

    def merged(parts, k):
        ws, ss = zip(*(dense(name, n, k) for name, n in parts))
        return _linear(torch.cat(ws).to(device), torch.cat(ss).to(device).contiguous())

    def norm(name, n):
        w = _expect(tensors.get(f"{name}.weight"), f"{name}.weight", bf16, (n,))
        return _norm(w.to(device), cfg.eps)

    cos_sin = rope_cache(d, cfg.max_positions, cfg.theta, device=device)
    rotary = SimpleNamespace(cos_sin_cache=cos_sin, head_size=d, base=cfg.theta,
                             is_neox_style=True)
    layers = []
    for i in range(cfg.layers if num_layers is None else num_layers):
        p = f"model.layers.{i}"
        a = f"{p}.self_attn"
        attn = SimpleNamespace(
            qkv_proj=merged(((f"{a}.q_proj", hq * d), (f"{a}.k_proj", hk * d),
                             (f"{a}.v_proj", hk * d)), h),
            o_proj=_linear(*(t.to(device) for t in dense(f"{a}.o_proj", h, hq * d))),
            q_norm=norm(f"{a}.q_norm", d), k_norm=norm(f"{a}.k_norm", d),
            rotary_emb=rotary, num_heads=hq, num_kv_heads=hk, head_dim=d)
        m = f"{p}.mlp"
        mlp = SimpleNamespace(
            gate_up_proj=merged(((f"{m}.gate_proj", inter), (f"{m}.up_proj", inter)), h),
            down_proj=_linear(*(t.to(device) for t in dense(f"{m}.down_proj", h, inter))))
        layers.append(SimpleNamespace(
            self_attn=attn, mlp=mlp,
            input_layernorm=norm(f"{p}.input_layernorm", h),
            post_attention_layernorm=norm(f"{p}.post_attention_layernorm", h)))
    embed = _expect(tensors.get("model.embed_tokens.weight"), "model.embed_tokens.weight",
                    bf16, (cfg.vocab, h)).to(device)
    if cfg.tied_head:
        head = embed
    else:
        head = _expect(tensors.get("lm_head.weight"), "lm_head.weight", bf16,
                       (cfg.vocab, h)).to(device)
    inner = SimpleNamespace(layers=layers, embed_tokens=Embedding(embed),
                            norm=norm("model.norm", h))
    return SimpleNamespace(model=inner, lm_head=SimpleNamespace(weight=head), config=cfg)
