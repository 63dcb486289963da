"""Qwen3 forward pass over the gfx950 Engine.

The same layer order and contract as the reference pipeline
(quail/backends/quail/executor/models/qwen3.py:15-135 and the ModelPipeline
contract of models/base.py:36-84): input RMSNorm, fused QKV projection,
per-head Q/K RMSNorm with rotary, paged attention, output projection,
post-attention RMSNorm, gate_up projection, SiLU-gated product, down
projection; the final norm runs on `chunk.final_indices` only.

Launches are fused relative to the reference's sequence, with identical
results: the embedding gather with layer 0's norm_quant; the gate_up
projection with the SiLU-gated product and its quant (the bf16 gate_up rows
are never written); the final-row gather with the final fused_add_rms_norm;
the pack's K and V writes with the qk-norm-rope pass (into the arena pages
for a unified pack, as the contiguous rows call A reads for a tree pack).
"""

import torch

from quail_amd.engine import Engine


class Qwen3Pipeline:
    """Forward passes for Qwen3 FP8 checkpoints (see quail_amd.model)."""

    # ModelPipeline contract attributes (models/base.py:58-84)
    warm_tokens = (64, 128, 256, 512, 1024, 2048)
    needs_pages = True
    mask = "causal"
    masks = ("causal",)
    tree_attention = False
    gemm_warmup = True

    def __init__(self, model, arena, *, spec=None, kernels="quail", engine_class=Engine):
        self.layers = model.model.layers
        self.embed = model.model.embed_tokens
        self.final_norm = model.model.norm
        attn = self.layers[0].self_attn
        self.engine = engine_class(
            arena, num_q_heads=attn.num_heads, num_kv_heads=attn.num_kv_heads,
            head_dim=attn.head_dim, rotary=attn.rotary_emb,
            fp8=attn.qkv_proj.weight.dtype.is_floating_point and
            attn.qkv_proj.weight.element_size() == 1, kernels=kernels)
        # element offsets inside the kernels are int64; the reference's
        # 32-bit bound (qwen3.py:31-36) is kept so packs stay comparable
        widest = max(max(layer.self_attn.qkv_proj.weight.shape[0],
                         layer.mlp.gate_up_proj.weight.shape[0]) for layer in self.layers)
        self.max_chunk_tokens = (2**31 - 1) // widest
        self.spec = spec
        # gate_up + SiLU-quant in one launch when the engine has it (an engine
        # class with the reference's primitives only runs them separately)
        self.fuse_swiglu = (hasattr(self.engine, "gate_up_activation_quant") and
                            all(layer.mlp.gate_up_proj.weight.shape[0] % 256 == 0
                                for layer in self.layers))
        # qk-norm-rope writes the pack's K and V straight into the arena pages
        # when the engine has it and the pack's scatter source is its own rows
        self.fuse_kv_write = hasattr(self.engine, "qk_norm_rope_kv")
        # ... and then the attention normalizes and rotates q as it loads it
        # (that pass writes K and V only), at head_dim 128
        self.fuse_q_norm = (hasattr(self.engine, "kv_norm_rope")
                            and self.engine.head_dim == 128)

    def _check_bounds(self, chunk):
        """Token ids index the embedding and positions the rotary cache; the
        kernels gather without bounds checks, so reject bad packs here."""
        ids = getattr(chunk, "host_ids", None)
        if ids is not None and len(ids):
            vocab = self.embed.weight.shape[0]
            if int(ids.min()) < 0 or int(ids.max()) >= vocab:
                raise ValueError(f"token id outside the {vocab}-row embedding")
        pos = getattr(chunk, "host_positions", None)
        if pos is not None and len(pos):
            rows = self.engine.rotary.cos_sin_cache.shape[0]
            if int(pos.min()) < 0 or int(pos.max()) >= rows:
                raise ValueError(f"position outside the {rows}-row rotary cache")

    def linears(self):
        layer = self.layers[0]
        return (layer.self_attn.qkv_proj, layer.self_attn.o_proj,
                layer.mlp.gate_up_proj, layer.mlp.down_proj)

    def before_attention(self, hidden, residual, positions, layer, chunk=None):
        """Normalize and project rows into rotary Q, K, V and the residual.
        With `chunk`, K and V may go straight to its arena pages (then k and
        v are None)."""
        engine = self.engine
        attn = layer.self_attn
        if residual is None:
            residual = hidden
            q_in, q_scale = engine.norm_quant(hidden, layer.input_layernorm)
        else:
            q_in, q_scale = engine.norm_quant(hidden, layer.input_layernorm, residual)
        return self._project_qkv(q_in, q_scale, positions, attn, chunk) + (residual,)

    def _project_qkv(self, q_in, q_scale, positions, attn, chunk=None):
        engine = self.engine
        qkv = engine.gemm(q_in, q_scale, attn.qkv_proj)
        if (chunk is not None and self.fuse_kv_write and chunk.attention_mode == "unified"
                and not chunk.meta.get("kv_written", False)
                and (chunk.meta.get("unified") or {}).get("row_dst") is not None):
            if self.fuse_q_norm:
                return engine.kv_norm_rope(qkv, positions, attn, chunk.meta), None, None
            return engine.qk_norm_rope_kv(qkv, positions, attn, chunk.meta), None, None
        if (chunk is not None and self.fuse_kv_write and chunk.attention_mode == "tree"
                and hasattr(engine, "qk_norm_rope_rows")):
            identity = chunk.meta.get("identity_rows")
            if identity is None or identity.shape[0] != qkv.shape[0]:
                identity = torch.arange(qkv.shape[0], dtype=torch.int64, device=qkv.device)
                chunk.meta["identity_rows"] = identity
            return engine.qk_norm_rope_rows(qkv, positions, attn, identity, chunk.meta)
        q, k = engine.qk_norm_rope(qkv, positions, attn)
        v = qkv[:, (engine.num_q_heads + engine.num_kv_heads) * engine.head_dim:]
        return q, k, v

    def after_attention(self, o_in, o_scale, residual, layer):
        """Project attention rows and apply the residual MLP."""
        engine = self.engine
        hidden = engine.gemm(o_in, o_scale, layer.self_attn.o_proj)
        g_in, g_scale = engine.norm_quant(hidden, layer.post_attention_layernorm, residual)
        if self.fuse_swiglu:
            d_in, d_scale = engine.gate_up_activation_quant(g_in, g_scale, layer.mlp.gate_up_proj)
        else:
            gate_up = engine.gemm(g_in, g_scale, layer.mlp.gate_up_proj)
            d_in, d_scale = engine.activation_quant(gate_up)
        return engine.gemm(d_in, d_scale, layer.mlp.down_proj)

    def forward_chunk(self, chunk):
        """Return the final-normed hidden state of chunk.final_indices."""
        engine = self.engine
        self._check_bounds(chunk)
        chunk.meta["layer"] = 0
        first = self.layers[0]
        q_in, q_scale, residual = engine.embed_norm_quant(
            chunk.input_ids, self.embed.weight, first.input_layernorm)
        hidden = None
        last = len(self.layers) - 1
        final = chunk.final_indices
        for index, layer in enumerate(self.layers):
            if index == 0:
                q, k, v = self._project_qkv(q_in, q_scale, chunk.positions, layer.self_attn,
                                            chunk)
            else:
                q, k, v, residual = self.before_attention(hidden, residual, chunk.positions,
                                                          layer, chunk)
            if index == last and not final.shape[0]:
                # a pass of prefill pieces reads no row: later passes need
                # only the last layer's KV from it
                engine.write_kv_only(q, k, v, chunk)
                return torch.empty((0, self.embed.weight.shape[1]), dtype=torch.bfloat16,
                                   device=q.device)
            if index == last and chunk.meta.get("final_query") is not None:
                # past the last layer's KV only the final rows matter: their
                # attention, o_proj and MLP run alone, bit-identical to what
                # they are in the full pass (every kernel is row-local)
                o_in, o_scale = engine.attention_final(q, k, v, chunk, final)
                residual = residual.index_select(0, final)
                hidden = self.after_attention(o_in, o_scale, residual, layer)
                normed, _ = engine.fused_add_rms_norm(hidden, residual, self.final_norm)
                return normed
            o_in, o_scale = engine.attention(q, k, v, chunk)
            hidden = self.after_attention(o_in, o_scale, residual, layer)
        return engine.final_norm(hidden, residual, final, self.final_norm)
