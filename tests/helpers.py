"""Shared test helpers: the oracle's view of a quail_amd model, and runs."""

import torch

from oracle import qwen3_ref as ref


def ref_model(model) -> ref.RefModel:
    """The oracle's CPU copy of a model built by quail_amd.model."""
    inner = model.model
    cpu = lambda t: t.detach().to("cpu")
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


def run_stage(model, workload, readout_kind="margins", num_pages=None, use_tree=True):
    """Run one stage of the workload through the GPU engine; returns
    (results per document, StageRun)."""
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
                    cfg.kv_heads, cfg.head_dim)
    pipe = Qwen3Pipeline(model, arena)
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
                   use_tree=use_tree)
    results = run.run()
    torch.cuda.synchronize()
    return results, run
