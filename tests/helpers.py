"""Shared test helpers: the oracle's view of a quail_amd model, and runs."""

import torch

from oracle import qwen3_ref as ref


def ref_model(model, device="cpu") -> ref.RefModel:
    """The oracle's copy of a model built by quail_amd.model (on the CPU, or
    on `device` for checks at model sizes the CPU would take too long on)."""
    inner = model.model
    cpu = lambda t: t.detach().to(device)
    layers = []
    for layer in inner.layers:
        a, m = layer.self_attn, layer.mlp
        lin = lambda l: ref.RefLinear(cpu(l.weight), cpu(l.weight_scale_inv))
        layers.append(ref.RefLayer(
            in_norm=cpu(layer.input_layernorm.weight),
            post_norm=cpu(layer.post_attention_layernorm.weight),
            q_norm=cpu(a.q_norm.weight), k_norm=cpu(a.k_norm.weight),
            qkv=lin(a.qkv_proj), o=lin(a.o_proj), gate_up=lin(m.gate_up_proj),
            down=lin(m.down_proj)))
    a0 = inner.layers[0].self_attn
    return ref.RefModel(
        embed=cpu(inner.embed_tokens.weight), norm=cpu(inner.norm.weight), layers=layers,
        cos_sin=cpu(a0.rotary_emb.cos_sin_cache), eps=float(inner.norm.variance_epsilon),
        num_heads=a0.num_heads, num_kv_heads=a0.num_kv_heads, head_dim=a0.head_dim,
        head=cpu(model.lm_head.weight))


def run_stage(model, workload, readout_kind="margins", num_pages=None, use_tree=True,
              attention_mode="unified", fuse_kv_write=None, v_dtype=None, fuse_q_norm=None):
    """Run one stage of the workload through the GPU engine; returns
    (results per document, StageRun). v_dtype: the arena's V page type
    (its default, fp16, when None; bf16 is the reference arena's)."""
    from quail_amd.arena import KVArena
    from quail_amd.executor import StageRun
    from quail_amd.model import retain_answer_head
    from quail_amd.qwen3 import Qwen3Pipeline
    from quail_amd import readout as ro

    cfg = model.config
    if num_pages is None:
        num_pages = 3 * workload.chunk_budget // workload.page_tokens + 64
    arena = KVArena(cfg.layers if len(model.model.layers) == cfg.layers else
                    len(model.model.layers), num_pages, workload.page_tokens,
                    cfg.kv_heads, cfg.head_dim,
                    **({} if v_dtype is None else dict(v_dtype=v_dtype)))
    pipe = Qwen3Pipeline(model, arena)
    if fuse_kv_write is not None:
        pipe.fuse_kv_write = fuse_kv_write
    if fuse_q_norm is not None:
        pipe.fuse_q_norm = fuse_q_norm
    labels = workload.label_ids
    if readout_kind == "classify":
        readout = ro.AsyncLabelLogprobs(model.lm_head.weight, labels, normalize=False)
    else:
        retain_answer_head(model, labels[:2])
        rows = ro.AnswerRows(model, [labels[0]], [labels[1]])
        readout = {"margins": ro.AsyncMargins, "if": ro.AsyncAnswers,
                   "score": ro.AsyncScores}[readout_kind](rows)
    prefixes, suffixes = workload.groups_input()
    run = StageRun(pipe, arena, readout, prefixes, suffixes, workload.chunk_budget,
                   use_tree=use_tree, attention_mode=attention_mode)
    results = run.run()
    torch.cuda.synchronize()
    return results, run


def write_hf_checkpoint(model, cfg, path, shards=2):
    """Write a model with the pipeline's module surface as a Hugging Face
    Qwen3 FP8 checkpoint: q/k/v and gate/up split back into their own
    tensors (with their weight_scale_inv row blocks), tensors spread over
    `shards` safetensors files with a model.safetensors.index.json, and a
    config.json carrying the FP8 quantization_config."""
    import json
    from pathlib import Path

    from safetensors.torch import save_file

    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    d, hq, hk, inter = cfg.head_dim, cfg.heads, cfg.kv_heads, cfg.intermediate
    tensors = {}

    def put(name, t):
        tensors[name] = t.detach().to("cpu").contiguous()

    def split(prefix, linear, parts):
        w, s = linear.weight, linear.weight_scale_inv
        row = 0
        for name, n in parts:
            put(f"{prefix}.{name}.weight", w[row:row + n])
            put(f"{prefix}.{name}.weight_scale_inv", s[row // 128:(row + n) // 128])
            row += n

    for i, layer in enumerate(model.model.layers):
        a, m = f"model.layers.{i}.self_attn", f"model.layers.{i}.mlp"
        attn = layer.self_attn
        split(a, attn.qkv_proj, (("q_proj", hq * d), ("k_proj", hk * d), ("v_proj", hk * d)))
        split(a, attn.o_proj, (("o_proj", cfg.hidden),))
        put(f"{a}.q_norm.weight", attn.q_norm.weight)
        put(f"{a}.k_norm.weight", attn.k_norm.weight)
        split(m, layer.mlp.gate_up_proj, (("gate_proj", inter), ("up_proj", inter)))
        split(m, layer.mlp.down_proj, (("down_proj", cfg.hidden),))
        put(f"model.layers.{i}.input_layernorm.weight", layer.input_layernorm.weight)
        put(f"model.layers.{i}.post_attention_layernorm.weight",
            layer.post_attention_layernorm.weight)
    put("model.embed_tokens.weight", model.model.embed_tokens.weight)
    put("model.norm.weight", model.model.norm.weight)
    if not cfg.tied_head:
        put("lm_head.weight", model.lm_head.weight)
    names = sorted(tensors)
    weight_map = {}
    for k in range(shards):
        file = f"model-{k + 1:05d}-of-{shards:05d}.safetensors"
        part = {n: tensors[n] for n in names[k::shards]}
        save_file(part, str(path / file), metadata={"format": "pt"})
        weight_map.update({n: file for n in part})
    with open(path / "model.safetensors.index.json", "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f)
    config = {
        "architectures": ["Qwen3ForCausalLM"], "model_type": "qwen3",
        "hidden_size": cfg.hidden, "intermediate_size": inter,
        "num_attention_heads": hq, "num_key_value_heads": hk, "head_dim": d,
        "num_hidden_layers": len(model.model.layers), "vocab_size": cfg.vocab,
        "rms_norm_eps": cfg.eps, "rope_theta": cfg.theta, "rope_scaling": None,
        "max_position_embeddings": cfg.max_positions, "hidden_act": "silu",
        "tie_word_embeddings": cfg.tied_head, "torch_dtype": "bfloat16",
        "use_sliding_window": False, "attention_bias": False,
        "quantization_config": {"activation_scheme": "dynamic", "fmt": "e4m3",
                                "quant_method": "fp8", "weight_block_size": [128, 128]},
    }
    with open(path / "config.json", "w") as f:
        json.dump(config, f, indent=1)
    return path


def write_transformers_fp8_checkpoint(cfg, path, seed=0, shard_bytes=400_000):
    """A Qwen3 FP8 checkpoint written by code independent of this package:
    transformers' Qwen3ForCausalLM (its own tensor names and random init,
    norms set to 1 + N(0, 0.1) so that a swapped norm shows), every layer
    projection quantized to e4m3 in 128x128 blocks by transformers'
    Fp8Quantize (the fine-grained FP8 format: `weight` and per-block
    `weight_scale_inv`, the value being weight * scale), the tensors sharded
    by huggingface_hub.save_torch_state_dict (tied head left out, as
    save_pretrained does) and config.json written by transformers with a
    FineGrainedFP8Config. Returns the directory."""
    import types
    from pathlib import Path

    from huggingface_hub import save_torch_state_dict
    from transformers import FineGrainedFP8Config, Qwen3Config, Qwen3ForCausalLM
    from transformers.integrations.finegrained_fp8 import Fp8Quantize

    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    hcfg = Qwen3Config(vocab_size=cfg.vocab, hidden_size=cfg.hidden,
                       intermediate_size=cfg.intermediate, num_hidden_layers=cfg.layers,
                       num_attention_heads=cfg.heads, num_key_value_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, rms_norm_eps=cfg.eps, rope_theta=cfg.theta,
                       tie_word_embeddings=cfg.tied_head,
                       max_position_embeddings=cfg.max_positions)
    torch.manual_seed(seed)
    model = Qwen3ForCausalLM(hcfg)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight"):
                p.copy_(1 + 0.1 * torch.randn_like(p))
    model = model.to(torch.bfloat16)
    qcfg = FineGrainedFP8Config(weight_block_size=(128, 128))
    quantize = Fp8Quantize(types.SimpleNamespace(quantization_config=qcfg))
    state = {}
    for name, t in model.state_dict().items():
        if cfg.tied_head and name == "lm_head.weight":
            continue
        if ".layers." in name and name.endswith("_proj.weight"):
            state.update(quantize._quantize_one(name, t))
        else:
            state[name] = t
    save_torch_state_dict(state, path, max_shard_size=shard_bytes)
    model.config.architectures = ["Qwen3ForCausalLM"]
    model.config.quantization_config = qcfg
    model.config.save_pretrained(path)
    return path


def exact_contractions(monkeypatch):
    """Replace the engine's two MFMA contractions with exact float64 torch
    computations on the GPU, for decomposition tests only: every FP8 GEMM
    (the dequantized operands' matmul, rounded to bf16; gate_up then the
    engine's own SiLU-quant kernel) and the paged attention (exact softmax
    over the pages the block table names, rounded to bf16, then the
    engine's own group quant). Everything else stays the engine's; q goes
    through the engine's qk-norm-rope pass (the attention's q-norm on load
    is an attention kernel's, so the pipeline is kept off it)."""
    from quail_amd.engine import Engine

    def gemm(self, q_input, input_scale, linear, out=None):
        m, k = q_input.shape
        a = (q_input.double().view(m, k // 128, 128) *
             input_scale.double().unsqueeze(-1)).view(m, k)
        w = linear.weight.double()
        s = self.weight_scale(linear).double().repeat_interleave(128, 0).repeat_interleave(128, 1)
        r = (a @ (w * s[:w.shape[0], :w.shape[1]]).T).to(torch.bfloat16)
        if out is None:
            return r
        out.copy_(r)
        return out

    def gate_up(self, q_input, input_scale, linear):
        return self.activation_quant(gemm(self, q_input, input_scale, linear))

    def paged(self, q3, tables, layer, softmax_scale, output, qnorm=None):
        assert qnorm is None, "q reaches the exact attention normalized"
        n, hq, d = q3.shape
        group = hq // self.num_kv_heads
        k_pool, v_pool = self.arena.layer_kv(layer)
        page = self.arena.page_tokens
        cu, used = tables["cu_q"].tolist(), tables["used"].tolist()
        table = tables["table"].tolist()
        causal = bool(tables.get("causal", True))
        scale = d ** -0.5 if softmax_scale is None else softmax_scale
        dev = q3.device
        out = torch.zeros((n, hq, d), dtype=torch.float64, device=dev)
        for s in range(len(used)):
            r0, r1 = cu[s], cu[s + 1]
            q_len, seen = r1 - r0, used[s]
            if q_len == 0:
                continue
            rows = torch.tensor([p * page + j for p in table[s][:-(-seen // page)]
                                 for j in range(page)][:seen], device=dev)
            k = k_pool[rows].double().repeat_interleave(group, dim=1)
            v = v_pool[rows].double().repeat_interleave(group, dim=1)
            scores = torch.einsum("qhd,khd->hqk", q3[r0:r1].double(), k) * scale
            if causal:
                qi = torch.arange(q_len, device=dev)[:, None]
                kj = torch.arange(seen, device=dev)[None, :]
                scores = scores.masked_fill(~(kj < seen - q_len + qi + 1)[None], float("-inf"))
            out[r0:r1] = torch.einsum("hqk,khd->qhd", scores.softmax(-1), v)
        return self.quant(out.to(torch.bfloat16).view(n, hq * d), output=output)

    monkeypatch.setattr(Engine, "gemm", gemm)
    monkeypatch.setattr(Engine, "gate_up_activation_quant", gate_up)
    monkeypatch.setattr(Engine, "_paged", paged)
    monkeypatch.delattr(Engine, "kv_norm_rope")


def admit(prefixes, suffixes, arena, budget, tree=None, unified=True):
    """StageAdmission whose admissions reserve their arena pages as the stage
    driver's do (one question in the document's own pages on the unified
    path, several in temporary pages)."""
    from quail_amd.admission import StageAdmission

    single = all(len(s) == 1 for s in suffixes)
    extra = max(len(s[0]) for s in suffixes) if unified and single else 0
    holder = {}

    def reserve(d, reads, rows):
        adm = holder["adm"]
        parent, shared = (None, 0) if reads is None else reads
        f = len(prefixes[d])
        return arena.reserve(adm.keys[d], f, capacity_tokens=f + extra,
                             borrow=(adm.keys[parent], shared) if shared else None)

    adm = StageAdmission(prefixes, suffixes, arena, budget, tree=tree, extra_tokens=extra,
                         temporary_pages=unified, reserve=reserve)
    holder["adm"] = adm
    return adm


def pack_specs(adm, groups, prefills=()):
    """The pack_chunk groups of one pass's question groups and prefill pieces."""
    return [adm.group_spec(*g) for g in groups] + [adm.piece_spec(*p) for p in prefills]
