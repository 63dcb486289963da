"""Qwen3 FP8 model objects with the attribute surface the pipeline reads.

Qwen3Pipeline reads vLLM's loaded module (quail/backends/quail/executor/
models/qwen3.py:18-30, 45-68): `model.model.layers[i].self_attn.{qkv_proj,
o_proj, q_norm, k_norm, rotary_emb, num_heads, num_kv_heads, head_dim}`,
`mlp.{gate_up_proj, down_proj}`, `input_layernorm`, `post_attention_layernorm`
(`.weight`, `.variance_epsilon`), `model.model.embed_tokens`, `model.model.norm`.
FP8 linears carry `.weight` e4m3 (N, K) and `.weight_scale_inv` (N/128, K/128)
fp32 (attention.py:471-477); qkv rows are q|k|v and gate_up rows gate|up.

vLLM is not part of this engine, so `build_synthetic` makes that surface
from seeded random weights (N(0, 0.02), each 128x128 block quantized to e4m3
with scale amax/448), and `quail_amd.loader` makes it from a checkpoint.
"""

from dataclasses import dataclass
from types import SimpleNamespace

import torch

FP8_MAX = 448.0
BLOCK = 128


@dataclass(frozen=True)
class Qwen3Config:
    name: str
    layers: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    eps: float = 1e-6
    theta: float = 1e6
    max_positions: int = 40960
    tied_head: bool = True

    @property
    def qkv_out(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    def linear_shapes(self):
        """(K, N) of qkv, o_proj, gate_up, down."""
        return ((self.hidden, self.qkv_out), (self.heads * self.head_dim, self.hidden),
                (self.hidden, 2 * self.intermediate), (self.intermediate, self.hidden))

    def gemm_flops_per_token(self) -> float:
        """2 * linear params, all layers (the reference cost model's GEMM term,
        crates/quail-planner/src/cost/dense_decoder_cost.rs:103-141)."""
        return 2.0 * self.layers * sum(k * n for k, n in self.linear_shapes())

    def attention_flops_per_pair(self) -> float:
        """4 * H * D per (query, key) pair per layer, all layers
        (dense_decoder_cost.rs:78-89)."""
        return 4.0 * self.heads * self.head_dim * self.layers


CONFIGS = {
    # the benchmark models: a 2-layer tiny model for tests, Qwen3-4B, -8B and -32B shapes
    "tiny": Qwen3Config("tiny", 2, 256, 4, 2, 64, 768, 4096, max_positions=4096),
    "qwen3-4b": Qwen3Config("qwen3-4b", 36, 2560, 32, 8, 128, 9728, 151936),
    "qwen3-8b": Qwen3Config("qwen3-8b", 36, 4096, 32, 8, 128, 12288, 151936),
    "qwen3-32b": Qwen3Config("qwen3-32b", 64, 5120, 64, 8, 128, 25600, 151936,
                             tied_head=False),
}


def rope_cache(head_dim: int, max_pos: int, theta: float, device=None) -> torch.Tensor:
    """vLLM RotaryEmbedding.cos_sin_cache: [cos | sin] of pos * theta^(-2i/D),
    computed in fp32 and kept in the model dtype (bf16)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float,
                                             device=device) / head_dim))
    t = torch.arange(max_pos, dtype=torch.float, device=device)
    freqs = torch.outer(t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).to(torch.bfloat16)


def quantize_blocks(w: torch.Tensor):
    """Per 128x128 block: s = amax/448, q = e4m3(clamp(w/s, +-448)).
    Returns (q e4m3 (N, K), weight_scale_inv (N/128, K/128) fp32)."""
    n, k = w.shape
    b = w.float().view(n // BLOCK, BLOCK, k // BLOCK, BLOCK)
    amax = b.abs().amax(dim=(1, 3))
    s = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = (b / s[:, None, :, None]).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.view(n, k), s.contiguous()


class Embedding:
    def __init__(self, weight):
        self.weight = weight

    def __call__(self, ids):
        return self.weight.index_select(0, ids)


def _norm(weight, eps):
    return SimpleNamespace(weight=weight, variance_epsilon=eps)


def _linear(weight, scale):
    return SimpleNamespace(weight=weight, weight_scale_inv=scale)


def build_synthetic(cfg: Qwen3Config, seed: int = 0, device="cuda", gen_device=None,
                    norm_init: str = "ones", layers: int | None = None):
    """Seeded random-init Qwen3 FP8 model with the vLLM attribute surface.

    Weights are drawn on gen_device (default: device) from one generator in
    a fixed order, quantized there, and moved to device, so the same seed and
    gen_device give identical weights on any target. norm_init "ones" is HF's
    initialisation; "random" draws 1 + N(0, 0.1) so tests exercise the norm
    weights.
    """
    gen_device = torch.device(device if gen_device is None else gen_device)
    g = torch.Generator(device=gen_device)
    g.manual_seed(seed)
    bf16 = torch.bfloat16

    def normal(*shape, std=0.02):
        return torch.randn(*shape, generator=g, device=gen_device) * std

    def norm_weight(n):
        if norm_init == "ones":
            return torch.ones(n, dtype=bf16, device=device)
        return (1.0 + normal(n, std=0.1)).to(bf16).to(device)

    def linear(n, k):
        q, s = quantize_blocks(normal(n, k))
        return _linear(q.to(device), s.to(device))

    embed = normal(cfg.vocab, cfg.hidden).to(bf16).to(device)
    cos_sin = rope_cache(cfg.head_dim, cfg.max_positions, cfg.theta, device=device)
    rotary = SimpleNamespace(cos_sin_cache=cos_sin, head_size=cfg.head_dim,
                             base=cfg.theta, is_neox_style=True)
    built = []
    for _ in range(cfg.layers if layers is None else layers):
        attn = SimpleNamespace(
            qkv_proj=linear(cfg.qkv_out, cfg.hidden),
            o_proj=linear(cfg.hidden, cfg.heads * cfg.head_dim),
            q_norm=_norm(norm_weight(cfg.head_dim), cfg.eps),
            k_norm=_norm(norm_weight(cfg.head_dim), cfg.eps),
            rotary_emb=rotary, num_heads=cfg.heads, num_kv_heads=cfg.kv_heads,
            head_dim=cfg.head_dim)
        mlp = SimpleNamespace(gate_up_proj=linear(2 * cfg.intermediate, cfg.hidden),
                              down_proj=linear(cfg.hidden, cfg.intermediate))
        built.append(SimpleNamespace(
            self_attn=attn, mlp=mlp,
            input_layernorm=_norm(norm_weight(cfg.hidden), cfg.eps),
            post_attention_layernorm=_norm(norm_weight(cfg.hidden), cfg.eps)))
    final_norm = _norm(norm_weight(cfg.hidden), cfg.eps)
    if cfg.tied_head:
        head = embed
    else:
        head = normal(cfg.vocab, cfg.hidden).to(bf16).to(device)
    inner = SimpleNamespace(layers=built, embed_tokens=Embedding(embed), norm=final_norm)
    model = SimpleNamespace(model=inner, lm_head=SimpleNamespace(weight=head), config=cfg)
    return model


def retain_answer_head(model, token_ids):
    """Keep the answer rows and the full bf16 head on the model, as
    model_loading.retain_answer_head does (model_loading.py:150-178)."""
    allowed = tuple(sorted(set(token_ids)))
    if not allowed:
        raise ValueError("TRUE/FALSE token ids must not be empty")
    weight = model.lm_head.weight
    idx = torch.tensor(allowed, device=weight.device, dtype=torch.long)
    model.quail_answer_weights = weight.index_select(0, idx).to(torch.bfloat16).contiguous()
    model.quail_answer_token_ids = allowed
    model.quail_full_head = weight.to(torch.bfloat16)


def answer_weights(model, token_ids):
    """The retained rows for a query's answer ids (model_loading.py:255-260)."""
    if tuple(token_ids) != model.quail_answer_token_ids:
        raise ValueError("Query answer token ids differ from the loaded "
                         "model's retained rows")
    return model.quail_answer_weights
