"""Independent pins of the oracle's floating-point functions (CPU).

Every function of oracle/qwen3_ref.py is checked here against an
implementation that is not this repository's: torch's F.rms_norm and
F.scaled_dot_product_attention, and transformers' Qwen3 modules
(Qwen3RMSNorm, Qwen3RotaryEmbedding, apply_rotary_pos_emb and the whole
Qwen3ForCausalLM). The inputs are chosen so that a plausible mistake fails
a check: rows small enough that eps changes the norm, GQA groups whose
head mapping matters, RoPE at large positions, queries that are a suffix
of their keys, several layers and documents.

Which reference arithmetic each oracle function restates (paths relative
to quail/backends/quail/executor/):
  rms_norm_vllm        attention.py:539-556 (vLLM rms_norm)
  fused_add_rms_norm   attention.py:558-562 (vLLM fused_add_rms_norm)
  add_rms_norm_quant   attention.py:796-829 (Triton)
  qk_norm_rope         attention.py:833-879 (Triton)
  rope_cache           models/qwen3.py:29 (vLLM RotaryEmbedding cos_sin_cache)
  paged/varlen attn    attention.py:1280-1306, 1477-1573 (flash-attn varlen)
  silu_mul_quant       attention.py:771-793 (Triton)
  gemm                 attention.py:479-499 (DeepGEMM fp8_gemm_nt)
  label_logits/answer  readout.py:44-48, 188-191, 331-336
  layer order          models/qwen3.py:45-68, 120-135
"""

import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention.bias import causal_lower_right
from transformers import Qwen3Config
from transformers.models.qwen3 import modeling_qwen3 as hf

from oracle import qwen3_ref as ref
from oracle.fp8 import dequant_weight

BF16 = torch.bfloat16


def _rows(n, h, seed, tiny_rows=0):
    """bf16 rows of assorted magnitudes; the last tiny_rows rows have
    mean(x^2) near eps = 1e-6, where sqrt(ms + eps) and sqrt(ms) + eps part."""
    g = torch.Generator().manual_seed(seed)
    scale = torch.exp(torch.randn(n, 1, generator=g) * 2)
    x = torch.randn(n, h, generator=g) * scale
    if tiny_rows:
        x[-tiny_rows:] = torch.randn(tiny_rows, h, generator=g) * 1e-3
    return x.to(BF16)


def _norm_weight(h, seed):
    g = torch.Generator().manual_seed(seed)
    return (1 + 0.1 * torch.randn(h, generator=g)).to(BF16)


def _ulp_bf16(x):
    """One bf16 unit in the last place of |x| (x bf16)."""
    e = torch.frexp(x.float().abs().clamp_min(2.0 ** -126)).exponent
    return torch.ldexp(torch.ones_like(x, dtype=torch.float32), e - 8)


def _same_or_one_ulp(got, want, identical=0.999):
    assert got.dtype == want.dtype == BF16 and got.shape == want.shape
    same = (got == want).float().mean().item()
    diff = (got.float() - want.float()).abs()
    assert same >= identical, same
    assert bool((diff <= _ulp_bf16(want) * 1.001).all()), diff.max()


# ---- norms -------------------------------------------------------------------


@pytest.mark.parametrize("h", [128, 256, 2560, 5120])
def test_rms_norm_vllm_equals_transformers_qwen3_rmsnorm(h):
    eps = 1e-6
    x = _rows(64, h, seed=h, tiny_rows=8)
    w = _norm_weight(h, seed=h + 1)
    mod = hf.Qwen3RMSNorm(h, eps=eps)
    with torch.no_grad():
        mod.weight.copy_(w)
        mod = mod.to(BF16)
        want = mod(x)
    _same_or_one_ulp(ref.rms_norm_vllm(x, w, eps), want)


def test_rms_norm_vllm_equals_torch_rms_norm():
    """F.rms_norm of the fp32 rows, rounded to bf16, times the bf16 weight."""
    eps = 1e-6
    x = _rows(200, 2560, seed=7, tiny_rows=20)
    w = _norm_weight(2560, seed=8)
    want = (F.rms_norm(x.float(), (2560,), eps=eps).to(BF16).float() * w.float()).to(BF16)
    _same_or_one_ulp(ref.rms_norm_vllm(x, w, eps), want)


def test_fused_add_rms_norm_equals_transformers_residual_then_norm():
    """Qwen3DecoderLayer: residual + hidden in bf16, then the RMSNorm."""
    eps = 1e-6
    h = 2560
    a, b = _rows(96, h, seed=11), _rows(96, h, seed=12)
    w = _norm_weight(h, seed=13)
    mod = hf.Qwen3RMSNorm(h, eps=eps)
    with torch.no_grad():
        mod.weight.copy_(w)
        mod = mod.to(BF16)
        z_want = b + a
        n_want = mod(z_want)
    n_got, z_got = ref.fused_add_rms_norm(a, b, w, eps)
    assert torch.equal(z_got, z_want)
    _same_or_one_ulp(n_got, n_want)


@pytest.mark.parametrize("h", [256, 2560])
def test_add_rms_norm_quant_norms_the_fp32_sum(h):
    """The Triton kernel's fp32 sum normed by torch's F.rms_norm (weight in
    fp32) and quantized gives the same codes; the residual is the bf16 sum."""
    from oracle.fp8 import group_quant
    eps = 1e-6
    x, res = _rows(128, h, seed=21, tiny_rows=8), _rows(128, h, seed=22)
    w = _norm_weight(h, seed=23)
    q, s, r = ref.add_rms_norm_quant(x, res, w, eps)
    total = x.float() + res.float()
    assert torch.equal(r, total.to(BF16))
    want_q, want_s = group_quant(F.rms_norm(total, (h,), weight=w.float(), eps=eps))
    torch.testing.assert_close(s, want_s, rtol=1e-6, atol=0)
    codes_equal = (q.view(torch.uint8) == want_q.view(torch.uint8)).float().mean().item()
    assert codes_equal >= 0.999
    step = (q.float() - want_q.float()).abs()
    assert bool((step <= q.float().abs().clamp_min(2 ** -6) / 8 + 1e-12).all())


def test_norm_quant_first_is_the_transformers_norm_quantized():
    from oracle.fp8 import group_quant
    eps = 1e-6
    x = _rows(64, 2560, seed=31, tiny_rows=4)
    w = _norm_weight(2560, seed=32)
    mod = hf.Qwen3RMSNorm(2560, eps=eps)
    with torch.no_grad():
        mod.weight.copy_(w)
        want = group_quant(mod.to(BF16)(x).float())
    got = ref.norm_quant_first(x, w, eps)
    same = (got[0].view(torch.uint8) == want[0].view(torch.uint8)).float().mean().item()
    assert same >= 0.999


def test_silu_mul_quant_equals_torch_silu():
    """transformers' Qwen3MLP activation (F.silu(gate) * up), quantized."""
    from oracle.fp8 import group_quant
    g = torch.Generator().manual_seed(41)
    gate_up = (torch.randn(64, 2 * 768, generator=g) * 3).to(BF16)
    q, s = ref.silu_mul_quant(gate_up)
    wq, ws = group_quant(F.silu(gate_up[:, :768].float()) * gate_up[:, 768:].float())
    torch.testing.assert_close(s, ws, rtol=1e-6, atol=0)
    assert (q.view(torch.uint8) == wq.view(torch.uint8)).float().mean().item() >= 0.999


def test_gemm_equals_the_blockwise_scaled_sum():
    """C = sum over 128-K blocks of (A_kb W_kb^T) * sA[:, kb] * sW[n / 128, kb]
    (DeepGEMM's definition, attention.py:479-499), summed block by block in
    float64 with the scales applied outside the products, against the
    oracle's dequantize-then-matmul. The (N/128, K/128) scale grid is not
    square, so a transposed scale index fails."""
    from oracle.fp8 import group_quant, quantize_weight_blocks
    g = torch.Generator().manual_seed(43)
    m, n, k = 40, 384, 640
    a_q, a_s = group_quant(torch.randn(m, k, generator=g))
    w = torch.randn(n, k, generator=g) * 0.02
    w[:128, 256:384] *= 40            # a block with a very different scale
    w_q, w_s = quantize_weight_blocks(w)
    got = ref.gemm(a_q, a_s, ref.RefLinear(w_q, w_s))
    acc = torch.zeros(m, n, dtype=torch.float64)
    for kb in range(k // 128):
        cols = slice(kb * 128, (kb + 1) * 128)
        prod = a_q[:, cols].double() @ w_q[:, cols].double().T
        acc += prod * a_s[:, kb:kb + 1].double() * w_s[:, kb].double().repeat_interleave(128)[None]
    want = acc.to(BF16)
    _same_or_one_ulp(got, want, identical=0.999)


def test_readouts_equal_torch_linear_and_softmax():
    """AI.IF / AI.CLASSIFY logits are bf16 F.linear widened to fp32
    (readout.py:44-48, 188-191); AI.SCORE is softmax over (yes, no) taken at
    yes on the fp32 F.linear logits (readout.py:331-336)."""
    g = torch.Generator().manual_seed(47)
    normed = torch.randn(33, 256, generator=g).to(BF16)
    rows = (torch.randn(4, 256, generator=g) * 0.3).to(BF16)
    want0 = F.linear(normed, rows).float()
    _same_or_one_ulp(ref.label_logits(normed, rows, 0).to(BF16), want0.to(BF16))
    torch.testing.assert_close(ref.label_logits(normed, rows, 1),
                               F.linear(normed.float(), rows.float()), rtol=1e-5, atol=1e-5)
    yes, no, bits, score = ref.answer(normed, rows[:2], [1, 0], mode=1)
    logits = F.linear(normed.float(), rows[:2].float())
    torch.testing.assert_close(score, torch.softmax(logits, dim=-1)[:, 0], rtol=1e-5, atol=1e-6)
    assert torch.equal(bits, (logits[:, 0] > logits[:, 1]).to(torch.uint8))
    # several yes / no spellings: the answer is the larger of each class
    yes, no, _, _ = ref.answer(normed, rows, [1, 0, 1, 0], mode=1)
    full = F.linear(normed.float(), rows.float())
    torch.testing.assert_close(yes, torch.maximum(full[:, 0], full[:, 2]))
    torch.testing.assert_close(no, torch.maximum(full[:, 1], full[:, 3]))


# ---- rotary ------------------------------------------------------------------


def _hf_rotary(d, theta, positions):
    cfg = Qwen3Config(head_dim=d, rope_theta=theta, max_position_embeddings=65536,
                      hidden_size=d * 4, num_attention_heads=4, num_key_value_heads=2)
    rot = hf.Qwen3RotaryEmbedding(cfg)
    x = torch.zeros(1, dtype=torch.float32)
    return rot(x, positions[None])        # cos, sin: (1, n, d), [c | c], [s | s]


@pytest.mark.parametrize("d", [64, 128])
def test_rope_cache_equals_transformers_rotary_embedding(d):
    theta = 1e6
    cache = ref.rope_cache(d, 40960, theta)
    pos = torch.tensor([0, 1, 2, 3, 17, 255, 4095, 8191, 16000, 32767, 40959])
    cos, sin = _hf_rotary(d, theta, pos)
    half = d // 2
    # the cache holds bf16 [cos | sin] of the first half of the frequencies
    assert torch.equal(cos[0, :, :half], cos[0, :, half:])
    torch.testing.assert_close(cache[pos, :half].float(), cos[0, :, :half], rtol=0,
                               atol=2 ** -9 + 1e-6)
    torch.testing.assert_close(cache[pos, half:].float(), sin[0, :, :half], rtol=0,
                               atol=2 ** -9 + 1e-6)
    assert torch.equal(cache[pos, :half], cos[0, :, :half].to(BF16))
    assert torch.equal(cache[pos, half:], sin[0, :, :half].to(BF16))


@pytest.mark.parametrize("hq,hk,d", [(4, 2, 64), (32, 8, 128), (64, 8, 128)])
def test_qk_norm_rope_equals_transformers_norm_and_rotation(hq, hk, d):
    """Per-head Qwen3RMSNorm (fp32, the shared (D,) weight), then
    apply_rotary_pos_emb with the same cos/sin, rounded once to bf16: the
    Triton kernel's fp32 pipeline. Also against transformers' own fp32
    cos/sin within their bf16 rounding."""
    eps = 1e-6
    n = 48
    g = torch.Generator().manual_seed(hq * 100 + d)
    qkv = (torch.randn(n, (hq + 2 * hk) * d, generator=g) *
           torch.exp(torch.randn(n, 1, generator=g))).to(BF16)
    positions = torch.randint(0, 32768, (n,), generator=g)
    cache = ref.rope_cache(d, 32768, 1e6)
    q_w, k_w = _norm_weight(d, seed=1), _norm_weight(d, seed=2)
    q_got, k_got = ref.qk_norm_rope(qkv, positions, cache, q_w, k_w, hq, hk, d, eps)

    def hf_path(cos_half, sin_half):
        qn, kn = hf.Qwen3RMSNorm(d, eps=eps), hf.Qwen3RMSNorm(d, eps=eps)
        with torch.no_grad():
            qn.weight.copy_(q_w.float())
            kn.weight.copy_(k_w.float())
            q = qn(qkv[:, :hq * d].float().view(n, hq, d)).transpose(0, 1)[None]
            k = kn(qkv[:, hq * d:(hq + hk) * d].float().view(n, hk, d)).transpose(0, 1)[None]
        cos = torch.cat((cos_half, cos_half), -1)[None]
        sin = torch.cat((sin_half, sin_half), -1)[None]
        qe, ke = hf.apply_rotary_pos_emb(q, k, cos, sin)
        return (qe[0].transpose(0, 1).reshape(n, hq * d).to(BF16),
                ke[0].transpose(0, 1).reshape(n, hk * d).to(BF16))

    half = d // 2
    q_want, k_want = hf_path(cache[positions, :half].float(), cache[positions, half:].float())
    _same_or_one_ulp(q_got, q_want)
    _same_or_one_ulp(k_got, k_want)
    cos, sin = _hf_rotary(d, 1e6, positions)
    q_hf, k_hf = hf_path(cos[0, :, :half], sin[0, :, :half])
    # per-head norms are ~sqrt(D) spread over D values: |x| ~ 1; cos/sin
    # rounded to bf16 move each output by at most ~2 * 2^-9 * |x|
    torch.testing.assert_close(q_got.float(), q_hf.float(), rtol=0.02, atol=0.02)
    torch.testing.assert_close(k_got.float(), k_hf.float(), rtol=0.02, atol=0.02)


# ---- attention ---------------------------------------------------------------


def _sdpa(q, k, v, q_len, kv_len):
    """torch SDPA in float64, GQA by enable_gqa, the queries the last q_len
    positions of kv_len (lower-right causal). q (L, H, D), k/v (S, KH, D)."""
    mask = causal_lower_right(q_len, kv_len)
    out = F.scaled_dot_product_attention(q.double().transpose(0, 1)[None],
                                         k.double().transpose(0, 1)[None],
                                         v.double().transpose(0, 1)[None],
                                         attn_mask=mask, enable_gqa=True)
    return out[0].transpose(0, 1)


@pytest.mark.parametrize("hq,hk,d", [(4, 2, 64), (32, 8, 128), (8, 1, 64)])
def test_varlen_attention_equals_torch_sdpa(hq, hk, d):
    g = torch.Generator().manual_seed(hq + d)
    lengths = [1, 5, 33, 70]
    n = sum(lengths)
    q = torch.randn(n, hq, d, generator=g).to(BF16)
    k = (torch.randn(n, hk, d, generator=g) * 2).to(BF16)
    v = torch.randn(n, hk, d, generator=g).to(BF16)
    cu = [0]
    for L in lengths:
        cu.append(cu[-1] + L)
    got = ref.varlen_attention(q, k, v, cu)
    for s, L in enumerate(lengths):
        r = slice(cu[s], cu[s + 1])
        want = _sdpa(q[r], k[r], v[r], L, L).to(BF16)
        _same_or_one_ulp(got[r], want, identical=0.995)


@pytest.mark.parametrize("hq,hk,d", [(4, 2, 64), (32, 8, 128)])
def test_paged_attention_equals_torch_sdpa_over_gathered_pages(hq, hk, d):
    """Sequences whose queries are the last q_len of `used` keys (borrowed
    prefixes), their K/V scattered over shuffled 16-row pages of a pool; SDPA
    runs on the contiguous rows the test keeps itself."""
    page = 16
    g = torch.Generator().manual_seed(5 * hq + d)
    seqs = [(3, 40), (17, 17), (1, 129), (30, 64), (0, 16)]     # (q_len, used)
    pages_needed = [-(-u // page) for _, u in seqs]
    total_pages = sum(pages_needed) + 7
    perm = torch.randperm(total_pages, generator=g).tolist()
    kpool = torch.randn(total_pages * page, hk, d, generator=g).to(BF16)   # junk elsewhere
    vpool = torch.randn(total_pages * page, hk, d, generator=g).to(BF16)
    width = max(pages_needed)
    table = torch.zeros(len(seqs), width, dtype=torch.int32)
    keys, vals, qs = [], [], []
    cu_q = [0]
    for s, (q_len, used) in enumerate(seqs):
        kk = (torch.randn(used, hk, d, generator=g) * 2).to(BF16)
        vv = torch.randn(used, hk, d, generator=g).to(BF16)
        mine = [perm.pop() for _ in range(pages_needed[s])]
        table[s, :len(mine)] = torch.tensor(mine, dtype=torch.int32)
        for j in range(used):
            kpool[mine[j // page] * page + j % page] = kk[j]
            vpool[mine[j // page] * page + j % page] = vv[j]
        keys.append(kk)
        vals.append(vv)
        qs.append(torch.randn(q_len, hq, d, generator=g).to(BF16))
        cu_q.append(cu_q[-1] + q_len)
    q3 = torch.cat(qs)
    got = ref.paged_attention(q3, kpool, vpool, cu_q, [u for _, u in seqs], table, page)
    for s, (q_len, used) in enumerate(seqs):
        if q_len == 0:
            continue
        want = _sdpa(qs[s], keys[s], vals[s], q_len, used).to(BF16)
        _same_or_one_ulp(got[cu_q[s]:cu_q[s + 1]], want, identical=0.995)


# ---- layer order: the whole model against transformers' Qwen3ForCausalLM -----


def _hf_model(model):
    """transformers' Qwen3ForCausalLM (float32, eager attention) holding the
    dequantized weights of a quail_amd synthetic model."""
    cfg = model.config
    hcfg = Qwen3Config(vocab_size=cfg.vocab, hidden_size=cfg.hidden,
                       intermediate_size=cfg.intermediate, num_hidden_layers=cfg.layers,
                       num_attention_heads=cfg.heads, num_key_value_heads=cfg.kv_heads,
                       head_dim=cfg.head_dim, rms_norm_eps=cfg.eps, rope_theta=cfg.theta,
                       tie_word_embeddings=cfg.tied_head,
                       max_position_embeddings=cfg.max_positions, attention_bias=False)
    hcfg._attn_implementation = "eager"
    m = hf.Qwen3ForCausalLM(hcfg).float().eval()
    d, hq, hk, inter = cfg.head_dim, cfg.heads, cfg.kv_heads, cfg.intermediate
    dq = lambda lin: dequant_weight(lin.weight.cpu(), lin.weight_scale_inv.cpu())
    with torch.no_grad():
        m.model.embed_tokens.weight.copy_(model.model.embed_tokens.weight.float().cpu())
        m.model.norm.weight.copy_(model.model.norm.weight.float().cpu())
        for src, dst in zip(model.model.layers, m.model.layers):
            qkv = dq(src.self_attn.qkv_proj)
            dst.self_attn.q_proj.weight.copy_(qkv[:hq * d])
            dst.self_attn.k_proj.weight.copy_(qkv[hq * d:(hq + hk) * d])
            dst.self_attn.v_proj.weight.copy_(qkv[(hq + hk) * d:])
            dst.self_attn.o_proj.weight.copy_(dq(src.self_attn.o_proj))
            dst.self_attn.q_norm.weight.copy_(src.self_attn.q_norm.weight.float().cpu())
            dst.self_attn.k_norm.weight.copy_(src.self_attn.k_norm.weight.float().cpu())
            gu = dq(src.mlp.gate_up_proj)
            dst.mlp.gate_proj.weight.copy_(gu[:inter])
            dst.mlp.up_proj.weight.copy_(gu[inter:])
            dst.mlp.down_proj.weight.copy_(dq(src.mlp.down_proj))
            dst.input_layernorm.weight.copy_(src.input_layernorm.weight.float().cpu())
            dst.post_attention_layernorm.weight.copy_(
                src.post_attention_layernorm.weight.float().cpu())
    return m


def _no_activation_quant(y):
    """group_quant with the FP8 rounding taken out: the rows themselves, unit scales."""
    y = y.float()
    return y, torch.ones(y.shape[0], y.shape[1] // 128)


@pytest.mark.parametrize("norm_init", ["ones", "random"])
def test_forward_documents_equals_transformers_qwen3(monkeypatch, norm_init):
    """The oracle's layer loop (norm placement, residual adds, the q/k/v and
    gate/up splits, GQA, RoPE, SwiGLU, final norm of each document's last
    row) against transformers' Qwen3ForCausalLM in float32 on the same
    dequantized weights, with the FP8 activation quantization switched off
    in the oracle (transformers has none). What remains is the oracle's
    bf16 roundings at the reference's storage points, a few bf16 ulps."""
    from quail_amd.model import CONFIGS, build_synthetic
    from quail_amd.workload import make_workload
    from tests.helpers import ref_model

    cfg = CONFIGS["tiny"]
    model = build_synthetic(cfg, seed=4, device="cpu", norm_init=norm_init)
    docs = make_workload("tiny", seed=4).prompts[:6]
    monkeypatch.setattr(ref, "group_quant", _no_activation_quant)
    got = ref.forward_documents(ref_model(model), docs).float()
    hfm = _hf_model(model)
    want = []
    with torch.no_grad():
        for doc in docs:
            out = hfm.model(input_ids=torch.tensor([list(doc)]))
            want.append(out.last_hidden_state[0, -1])
    want = torch.stack(want)
    rel = ((got - want).norm(dim=1) / want.norm(dim=1))
    assert float(rel.max()) <= 0.02, rel
    # the readout's logits (tied head) within the same relative bound
    head = hfm.lm_head.weight.detach()
    lg, lw = got @ head[[10, 11]].T, want @ head[[10, 11]].T
    assert float((lg - lw).abs().max()) <= 0.02 * float(lw.abs().max()) + 0.01
