"""The torch "dequantized path" of the Qwen3 FP8 prefill pass.

Test infrastructure (see oracle/__init__.py). It restates, in plain torch on
the CPU (or on a GPU, as the checker of full-size models: every tensor it
makes follows its inputs' device), the arithmetic of the reference path:

  layer loop and final rows        quail/backends/quail/executor/models/qwen3.py:45-68, 120-135
  norm_quant (layer 0, vLLM)       attention.py:1237-1240 -> rms_norm :539-556 + quant :517-532
  add_rms_norm_quant (Triton)      attention.py:796-829
  FP8 block-scaled GEMM            attention.py:479-490 (DeepGEMM fp8_gemm_nt), here the
                                   matmul of the dequantized operands (ACCUM precision)
  qk_norm_rope (Triton)            attention.py:833-879
  kv_row_scatter / write_kv        attention.py:885-897, 1165-1195
  paged causal varlen attention    attention.py:1477-1573 via FA varlen; restated as the exact
                                   fp32 `_dense_causal_paged` of tests/gpu/test_decode_evaluator.py:12-33
  silu_mul_quant (Triton)          attention.py:771-793
  fused_add_rms_norm (vLLM)        attention.py:558-562
  readouts                         readout.py:44-48 (AnswerRows), :331-336 (AsyncScores),
                                   :188-191 (AsyncLabelLogprobs, normalize=False)
  rotary cache                     vLLM RotaryEmbedding (qwen3.py:29): cat(cos, sin) of
                                   pos * theta^(-2i/D), built in fp32, stored bf16

Activations stay bf16 between kernels exactly where the reference stores
bf16 (residual, GEMM outputs, q/k, attention output); FP8 activation
quantization is kept, so FP8 rounding matches the GPU path.

Pinned: every function here against an independent statement of it
(tests/test_oracle_pins.py: transformers' Qwen3 RMSNorm, rotary embedding
and layer order, torch's scaled-dot-product attention over shuffled pages,
a block-by-block float64 GEMM, the fp8 code table by brute force). Parity
unpinned here (no reference test or vector exists for Qwen3, and the
libraries are absent): the accumulation order of DeepGEMM and
FlashAttention inside a dot product; the oracle computes the exact sums.
"""

from dataclasses import dataclass, field

import torch

from oracle.fp8 import dequant_rows, dequant_weight, group_quant

# Accumulation type of the contractions (GEMMs, attention). float64 makes the
# oracle the exact value of the dequantized math (one rounding, to bf16, at
# each point where the reference stores bf16); the timed CPU baseline uses
# float32, the reference torch path's own type.
ACCUM = torch.float64
# keep each layer's dequantized weights (CPU runs); False dequantizes them at
# every use, for checks on the GPU at model sizes whose fp32 weights would
# not fit
CACHE_WEIGHTS = True


def set_precision(dtype) -> None:
    global ACCUM
    ACCUM = dtype


def set_weight_cache(enabled: bool) -> None:
    global CACHE_WEIGHTS
    CACHE_WEIGHTS = enabled


@dataclass
class RefLinear:
    weight: torch.Tensor        # (N, K) float8_e4m3fn
    scale_inv: torch.Tensor     # (N/128, K/128) fp32

    def dequant(self) -> torch.Tensor:
        if not CACHE_WEIGHTS:
            return dequant_weight(self.weight, self.scale_inv).to(ACCUM)
        cache = self.__dict__.setdefault("_w", {})
        if ACCUM not in cache:
            cache[ACCUM] = dequant_weight(self.weight, self.scale_inv).to(ACCUM)
        return cache[ACCUM]


@dataclass
class RefLayer:
    in_norm: torch.Tensor
    post_norm: torch.Tensor
    q_norm: torch.Tensor
    k_norm: torch.Tensor
    qkv: RefLinear
    o: RefLinear
    gate_up: RefLinear
    down: RefLinear


@dataclass
class RefModel:
    embed: torch.Tensor          # (V, H) bf16, also the tied head
    norm: torch.Tensor           # (H,) bf16
    layers: list
    cos_sin: torch.Tensor        # (max_pos, D) bf16
    eps: float
    num_heads: int
    num_kv_heads: int
    head_dim: int
    head: torch.Tensor = field(default=None)

    def __post_init__(self):
        if self.head is None:
            self.head = self.embed


def rope_cache(head_dim: int, max_pos: int, theta: float) -> torch.Tensor:
    """vLLM RotaryEmbedding's cos_sin_cache, (max_pos, head_dim) bf16."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    t = torch.arange(max_pos, dtype=torch.float)
    freqs = torch.outer(t, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).to(torch.bfloat16)


# ---- kernels ---------------------------------------------------------------

def rms_norm_vllm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """vLLM rms_norm: bf16(bf16(x * rstd) * w) (attention.py:539-556)."""
    xf = x.float()
    rstd = 1.0 / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return ((xf * rstd).to(torch.bfloat16).float() * w.float()).to(torch.bfloat16)


def fused_add_rms_norm(h: torch.Tensor, r: torch.Tensor, w: torch.Tensor, eps: float):
    """vLLM fused_add_rms_norm: z = bf16(h + r); (rms_norm(z), z) (attention.py:558-562)."""
    z = (h.float() + r.float()).to(torch.bfloat16)
    return rms_norm_vllm(z, w, eps), z


def add_rms_norm_quant(x, res, w, eps):
    """Triton add_rms_norm_quant (attention.py:796-829): the sum stays fp32
    for the norm; the residual stores its bf16 rounding."""
    r = x.float() + res.float()
    rstd = 1.0 / torch.sqrt(r.pow(2).mean(-1, keepdim=True) + eps)
    q, s = group_quant(r * rstd * w.float())
    return q, s, r.to(torch.bfloat16)


def norm_quant_first(x, w, eps):
    """Layer 0's Engine.norm_quant without residual (attention.py:1237-1240)."""
    return group_quant(rms_norm_vllm(x, w, eps).float())


def gemm(q, s, lin: RefLinear) -> torch.Tensor:
    """FP8 block-scaled GEMM as the matmul of the dequantized operands, bf16 out."""
    return (dequant_rows(q, s).to(ACCUM) @ lin.dequant().T).to(torch.bfloat16)


def qk_norm_rope(qkv, positions, cos_sin, q_w, k_w, hq, hk, d, eps):
    """Triton qk_norm_rope (attention.py:833-879): per-head RMSNorm with the
    shared (D,) weight, then neox rotation, fp32 math, bf16 out."""
    n = qkv.shape[0]
    half = d // 2
    cs = cos_sin[positions].float()
    cos = cs[:, None, :half]
    sin = cs[:, None, half:]

    def one(x, w):
        x = x.float()
        rstd = 1.0 / torch.sqrt(x.pow(2).mean(-1, keepdim=True) + eps)
        x = x * rstd * w.float()
        a, b = x[..., :half], x[..., half:]
        return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1).to(torch.bfloat16)

    q = one(qkv[:, :hq * d].reshape(n, hq, d), q_w).reshape(n, hq * d)
    k = one(qkv[:, hq * d:(hq + hk) * d].reshape(n, hk, d), k_w).reshape(n, hk * d)
    return q, k


def silu_mul_quant(gate_up):
    """Triton silu_mul_quant (attention.py:771-793)."""
    half = gate_up.shape[1] // 2
    g = gate_up[:, :half].float()
    u = gate_up[:, half:].float()
    return group_quant(g * torch.sigmoid(g) * u)


def paged_attention(q3, k_pool, v_pool, cu_q, used, table, page, causal=True, scale=None):
    """Exact varlen attention through a block table (ACCUM precision), bf16 out.

    Restates `_dense_causal_paged` (tests/gpu/test_decode_evaluator.py:12-33):
    sequence s's query i sees keys [0, used - q_len + i + 1) when causal.
    k_pool, v_pool are (rows, HK, D); pages are `page` rows.
    """
    n, heads, dim = q3.shape
    kv_heads = k_pool.shape[1]
    group = heads // kv_heads
    scale = dim ** -0.5 if scale is None else scale
    dev = q3.device
    out = torch.zeros((n, heads, dim), dtype=ACCUM, device=dev)
    for s in range(len(used)):
        r0, r1 = int(cu_q[s]), int(cu_q[s + 1])
        q_len, seen = r1 - r0, int(used[s])
        if q_len == 0:
            continue
        pages = [int(p) for p in table[s][: -(-seen // page)]]
        rows = torch.tensor([p * page + j for p in pages for j in range(page)],
                            device=k_pool.device)[:seen]
        k = k_pool[rows].to(ACCUM).repeat_interleave(group, dim=1)   # (seen, H, D)
        v = v_pool[rows].to(ACCUM).repeat_interleave(group, dim=1)
        qs = q3[r0:r1].to(ACCUM)                                     # (q_len, H, D)
        scores = torch.einsum("qhd,khd->hqk", qs, k) * scale
        if causal:
            qi = torch.arange(q_len, device=dev)[:, None]
            kj = torch.arange(seen, device=dev)[None, :]
            mask = kj < (seen - q_len + qi + 1)
            scores = scores.masked_fill(~mask[None], float("-inf"))
        w = scores.softmax(-1)
        out[r0:r1] = torch.einsum("hqk,khd->qhd", w, v)
    return out.to(torch.bfloat16)


def varlen_attention(q3, k3, v3, cu):
    """Plain causal varlen attention over packed segments (no pages): the
    unpaged branch of attention_unified (attention.py:1517-1534)."""
    n, heads, dim = q3.shape
    group = heads // k3.shape[1]
    out = torch.zeros((n, heads, dim), dtype=ACCUM, device=q3.device)
    for s in range(len(cu) - 1):
        r0, r1 = int(cu[s]), int(cu[s + 1])
        L = r1 - r0
        k = k3[r0:r1].to(ACCUM).repeat_interleave(group, dim=1)
        v = v3[r0:r1].to(ACCUM).repeat_interleave(group, dim=1)
        scores = torch.einsum("qhd,khd->hqk", q3[r0:r1].to(ACCUM), k) * dim ** -0.5
        mask = torch.tril(torch.ones(L, L, dtype=torch.bool, device=q3.device))
        scores = scores.masked_fill(~mask[None], float("-inf"))
        out[r0:r1] = torch.einsum("hqk,khd->qhd", scores.softmax(-1), v)
    return out.to(torch.bfloat16)


# ---- forward passes ----------------------------------------------------------

def _layer_front(m: RefModel, layer: RefLayer, hidden, residual, positions):
    if residual is None:
        residual = hidden
        q_in, q_s = norm_quant_first(hidden, layer.in_norm, m.eps)
    else:
        q_in, q_s, residual = add_rms_norm_quant(hidden, residual, layer.in_norm, m.eps)
    qkv = gemm(q_in, q_s, layer.qkv)
    hq, hk, d = m.num_heads, m.num_kv_heads, m.head_dim
    q, k = qk_norm_rope(qkv, positions, m.cos_sin, layer.q_norm, layer.k_norm, hq, hk, d, m.eps)
    v = qkv[:, (hq + hk) * d:]
    return q, k, v, residual


def _layer_back(m: RefModel, layer: RefLayer, attn_out, residual):
    o_in, o_s = group_quant(attn_out.float())
    hidden = gemm(o_in, o_s, layer.o)
    g_in, g_s, residual = add_rms_norm_quant(hidden, residual, layer.post_norm, m.eps)
    gate_up = gemm(g_in, g_s, layer.gate_up)
    d_in, d_s = silu_mul_quant(gate_up)
    return gemm(d_in, d_s, layer.down), residual


def forward_chunk(m: RefModel, ids, positions, final_indices, unified, pools, page,
                  layers=None):
    """Qwen3Pipeline.forward_chunk over a packed chunk on the paged path.

    unified: dict with cu_q, used, table, src, dst and optional tail_src /
    tail_dst (host arrays, the meta["unified"] of pack_chunk). pools: per
    layer (k_pool, v_pool) CPU tensors of shape (rows, HK, D), updated in
    place as the reference's write_kv does before its paged read.
    Returns the final-normed bf16 rows (len(final_indices), H).
    """
    hq, hk, d = m.num_heads, m.num_kv_heads, m.head_dim
    ids = torch.as_tensor(ids, dtype=torch.long)
    positions = torch.as_tensor(positions, dtype=torch.long)
    n = ids.shape[0]
    hidden = m.embed[ids]
    residual = None
    src = torch.as_tensor(unified["src"], dtype=torch.long)
    dst = torch.as_tensor(unified["dst"], dtype=torch.long)
    keep = dst >= 0
    src, dst = src[keep], dst[keep]
    tail_src = unified.get("tail_src")
    tail_dst = unified.get("tail_dst")
    run = m.layers if layers is None else m.layers[:layers]
    for index, layer in enumerate(run):
        q, k, v, residual = _layer_front(m, layer, hidden, residual, positions)
        kp, vp = pools[index]
        kp[dst] = k.view(n, hk, d)[src]
        vp[dst] = v.reshape(n, hk, d)[src]
        if tail_src is not None and len(tail_src):
            ts = torch.as_tensor(tail_src, dtype=torch.long)
            td = torch.as_tensor(tail_dst, dtype=torch.long)
            kp[td] = kp[ts].clone()
            vp[td] = vp[ts].clone()
        attn = paged_attention(q.view(n, hq, d), kp, vp, unified["cu_q"], unified["used"],
                               unified["table"], page, causal=unified.get("causal", True))
        hidden, residual = _layer_back(m, layer, attn.view(n, hq * d), residual)
    final = torch.as_tensor(final_indices, dtype=torch.long)
    normed, _ = fused_add_rms_norm(hidden[final], residual[final], m.norm, m.eps)
    return normed


def forward_documents(m: RefModel, documents, layers=None):
    """Each document's whole prompt as its own causal sequence, no pages and
    no borrowing; returns the final-normed bf16 row of each document's last
    token. A correct pack (borrowed prefixes, pages, scatter maps) must give
    the same rows."""
    hq, hk, d = m.num_heads, m.num_kv_heads, m.head_dim
    lengths = [len(doc) for doc in documents]
    dev = m.embed.device
    ids = torch.tensor([int(t) for doc in documents for t in doc], dtype=torch.long, device=dev)
    positions = torch.cat([torch.arange(L, device=dev) for L in lengths])
    cu = [0]
    for L in lengths:
        cu.append(cu[-1] + L)
    n = ids.shape[0]
    hidden = m.embed[ids]
    residual = None
    run = m.layers if layers is None else m.layers[:layers]
    for layer in run:
        q, k, v, residual = _layer_front(m, layer, hidden, residual, positions)
        attn = varlen_attention(q.view(n, hq, d), k.view(n, hk, d), v.reshape(n, hk, d), cu)
        hidden, residual = _layer_back(m, layer, attn.view(n, hq * d), residual)
    final = torch.tensor([c - 1 for c in cu[1:]], dtype=torch.long, device=dev)
    normed, _ = fused_add_rms_norm(hidden[final], residual[final], m.norm, m.eps)
    return normed


# ---- readouts ----------------------------------------------------------------

def label_logits(normed, rows, mode=0):
    """mode 0: bf16 F.linear widened to fp32 (readout.py:44-48, 188-191);
    mode 1: fp32 F.linear of the fp32 operands (readout.py:331-336)."""
    out = (normed.to(ACCUM) @ rows.to(ACCUM).T).float()
    return out.to(torch.bfloat16).float() if mode == 0 else out


def answer(normed, rows, classes, mode=0, temperature=1.0):
    """(yes, no, bits, score) per row; classes[j] is 1 (yes), 0 (no) or -1."""
    logits = label_logits(normed, rows, mode)
    cls = torch.as_tensor(classes)
    yes = logits[:, cls == 1].amax(dim=1)
    no = logits[:, cls == 0].amax(dim=1)
    return yes, no, (yes > no).to(torch.uint8), torch.sigmoid((yes - no) / temperature)
