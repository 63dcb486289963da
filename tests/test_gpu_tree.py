"""The tree attention path on the GPU (Engine.attention_tree,
attention.py:1395-1441): its two attention calls with log-sum-exp
(qx_attention_lse) against float32 attention, the fused LSE merge and
o_proj quantization (qx_merge_attn_quant) against a float32 restatement of
the reference's merge_attn_quant (attention.py:902-948), and whole packs
in tree mode against the oracle and against the unified path.

Tolerances: attention outputs are bf16 (one rounding, 2^-8 relative) and
the PV product runs with bf16 probabilities, so outputs are compared at
2e-2 absolute on O(1) values and log-sum-exps at 1e-3. The merge is the
reference's sequence of fp32 operations with its two bf16 roundings; the
kernel fuses a + (b - a) * w into one FMA, which moves a value across a
bf16 rounding boundary now and then, so at least 99.9% of e4m3 codes must
be identical and the rest one code apart. End to end the margins keep the
bounds of the unified path (tests/test_gpu_forward.py).
"""

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from quail_amd import _lib
from quail_amd.model import CONFIGS, build_synthetic
from quail_amd.workload import make_workload
from tests.helpers import run_stage
from tests.test_gpu_forward import TOL, _oracle_margins, _report

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _p(t):
    return None if t is None else t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _ref_attention(q, k, v, scale, causal):
    """float32 attention of one sequence: q (m, HQ, D), k, v (u, HK, D)."""
    m, hq, d = q.shape
    u, hk, _ = k.shape
    g = hq // hk
    kk = k.float().repeat_interleave(g, dim=1)
    vv = v.float().repeat_interleave(g, dim=1)
    s = torch.einsum("mhd,uhd->hmu", q.float(), kk) * scale
    if causal:
        i = torch.arange(m, device=q.device)[:, None]
        j = torch.arange(u, device=q.device)[None, :]
        s = s.masked_fill(j > u - m + i, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)                     # (h, m)
    o = torch.einsum("hmu,uhd->mhd", torch.softmax(s, dim=-1), vv)
    return o, lse


def _lse_call(q, q_ld, q_index, k, v, cu_q, used, table, cu_k, seqs, max_q, max_used, hq, hk, d,
              causal, out, lse):
    _lib.call("qx_attention_lse", _p(q), q_ld, _p(q_index), _p(k), _p(v), _p(cu_q), _p(used),
              _p(table), table.stride(0) if table is not None else 0, _p(cu_k), seqs, max_q,
              max_used, hq, hk, d, float(d ** -0.5), int(causal), _p(out), out.stride(0),
              _p(lse), lse.stride(0), None, 0, int(v.dtype == torch.bfloat16), _stream())


@pytest.mark.parametrize("hq,hk,d", [(32, 8, 128), (4, 2, 64)])
@pytest.mark.parametrize("v_dtype", [torch.bfloat16, torch.float16])
def test_segments_call_matches_float32(hq, hk, d, v_dtype):
    """Call A: causal over contiguous rows in cu_k segments (a zero-length one,
    one shorter than a KV tile, several tiles long)."""
    g = torch.Generator(device=DEV).manual_seed(hq + d)
    lengths = [5, 0, 64, 1, 300, 129, 33]
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    n = int(cu[-1])
    q = torch.randn(n, hq * d, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(n, hk * d, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(n, hk * d, generator=g, device=DEV).to(v_dtype)
    cu_t = torch.tensor(cu, device=DEV)
    used = torch.tensor(lengths, dtype=torch.int32, device=DEV)
    out = torch.full((n, hq * d), float("nan"), dtype=torch.bfloat16, device=DEV)
    lse = torch.full((hq, n), float("nan"), dtype=torch.float32, device=DEV)
    _lse_call(q, q.stride(0), None, k, v, cu_t, used, None, cu_t, len(lengths), max(lengths),
              max(lengths), hq, hk, d, True, out, lse)
    torch.cuda.synchronize()
    for s, length in enumerate(lengths):
        if not length:
            continue
        r0, r1 = int(cu[s]), int(cu[s + 1])
        o, l = _ref_attention(q[r0:r1].view(-1, hq, d), k[r0:r1].view(-1, hk, d),
                              v[r0:r1].view(-1, hk, d), d ** -0.5, True)
        torch.testing.assert_close(out[r0:r1].float().view(-1, hq, d), o, atol=2e-2, rtol=0)
        torch.testing.assert_close(lse[:, r0:r1], l, atol=1e-3, rtol=0)


def test_page_reads_with_row_index_match_float32():
    """Call B: selected query rows (q_index), not causal, keys through block
    tables over 16-row pages (used not a page multiple)."""
    hq, hk, d, page = 32, 8, 128, 16
    g = torch.Generator(device=DEV).manual_seed(7)
    pages = 64
    kp = torch.randn(pages * page, hk * d, generator=g, device=DEV).to(torch.bfloat16)
    vp = torch.randn(pages * page, hk * d, generator=g, device=DEV).to(torch.bfloat16)
    n = 200
    q = torch.randn(n, hq * d, generator=g, device=DEV).to(torch.bfloat16)
    rng = np.random.default_rng(3)
    q_lens = [3, 40, 1, 70]
    used_h = [16, 100, 33, 250]
    rows = rng.choice(n, sum(q_lens), replace=False).astype(np.int64)
    width = max(-(-u // page) for u in used_h)
    table_h = np.zeros((len(q_lens), width), dtype=np.int32)
    for s, u in enumerate(used_h):
        table_h[s, :-(-u // page)] = rng.choice(pages, -(-u // page), replace=False)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    nb = int(cu[-1])
    out = torch.empty(nb, hq * d, dtype=torch.bfloat16, device=DEV)
    lse = torch.empty(hq, nb, dtype=torch.float32, device=DEV)
    table = torch.tensor(table_h, device=DEV)
    _lse_call(q, q.stride(0), torch.tensor(rows, device=DEV), kp, vp, torch.tensor(cu, device=DEV),
              torch.tensor(used_h, dtype=torch.int32, device=DEV), table, None, len(q_lens),
              max(q_lens), max(used_h), hq, hk, d, False, out, lse)
    torch.cuda.synchronize()
    for s in range(len(q_lens)):
        keys = (torch.tensor(table_h[s], device=DEV).long()[:, None] * page
                + torch.arange(page, device=DEV)).reshape(-1)[:used_h[s]]
        sel = torch.tensor(rows[cu[s]:cu[s + 1]], device=DEV)
        o, l = _ref_attention(q[sel].view(-1, hq, d), kp[keys].view(-1, hk, d),
                              vp[keys].view(-1, hk, d), d ** -0.5, False)
        torch.testing.assert_close(out[cu[s]:cu[s + 1]].float().view(-1, hq, d), o, atol=2e-2,
                                   rtol=0)
        torch.testing.assert_close(lse[:, cu[s]:cu[s + 1]], l, atol=1e-3, rtol=0)


def _merge_reference(a, b, la, lb, source):
    """merge_attn_quant (attention.py:902-948) in float32 torch ops."""
    has = source >= 0
    src = source.clamp_min(0).long()
    af = a.float()
    bf = b.float()[src]
    hq = la.shape[0]
    x = lb[:, src] - la                                       # (h, n)
    w = torch.sigmoid(x).to(torch.bfloat16).float().t()      # (n, h)
    n = a.shape[0]
    a3 = af.view(n, hq, -1)
    b3 = bf.view(n, hq, -1)
    merged = (a3 + (b3 - a3) * w[:, :, None]).to(torch.bfloat16).float()
    return torch.where(has[:, None, None], merged, a3).reshape(n, -1)


def test_merge_matches_the_reference_merge():
    hq, d = 32, 128
    g = torch.Generator(device=DEV).manual_seed(11)
    n, nb = 300, 180
    a = torch.randn(n, hq * d, generator=g, device=DEV).to(torch.bfloat16)
    b = torch.randn(nb, hq * d, generator=g, device=DEV).to(torch.bfloat16)
    la = torch.randn(hq, n, generator=g, device=DEV) * 3
    lb = torch.randn(hq, nb, generator=g, device=DEV) * 3
    src = torch.full((n,), -1, dtype=torch.int32, device=DEV)
    pick = torch.randperm(n, generator=g, device=DEV)[:nb]
    src[pick] = torch.arange(nb, dtype=torch.int32, device=DEV)
    q = torch.empty(n, hq * d, dtype=torch.float8_e4m3fn, device=DEV)
    scales = torch.empty(n * hq, dtype=torch.float32, device=DEV)
    _lib.call("qx_merge_attn_quant", _p(a), a.stride(0), _p(b), b.stride(0), _p(la), la.stride(0),
              _p(lb), lb.stride(0), _p(src), n, hq, d, _p(q), q.stride(0), _p(scales), n,
              _stream())
    y = _merge_reference(a, b, la, lb, src)
    want_q, want_s = ofp8.group_quant(y.cpu())
    got_s = scales.view(hq, n).t().cpu()
    codes = q.view(torch.uint8).cpu().numpy().astype(np.int32)
    want_codes = want_q.view(torch.uint8).numpy().astype(np.int32)
    same = codes == want_codes
    assert same.mean() >= 0.999, same.mean()
    # a differing code is an adjacent e4m3 value (same sign byte, code +-1)
    assert np.abs(codes[~same] - want_codes[~same]).max(initial=0) <= 1
    rel = ((got_s - want_s).abs() / want_s).numpy()
    assert (rel == 0).mean() >= 0.99 and rel.max() <= 2 ** -7
    # rows that read nothing resident are quantized a
    keep = (src < 0).cpu().numpy()
    plain_q, _ = ofp8.group_quant(a.float().cpu())
    assert np.array_equal(codes[keep], plain_q.view(torch.uint8).numpy()[keep])


def test_bf16_merge_for_narrow_heads():
    hq, d = 4, 64
    g = torch.Generator(device=DEV).manual_seed(12)
    n = 50
    a = torch.randn(n, hq * d, generator=g, device=DEV).to(torch.bfloat16)
    b = torch.randn(n, hq * d, generator=g, device=DEV).to(torch.bfloat16)
    la = torch.randn(hq, n, generator=g, device=DEV)
    lb = torch.randn(hq, n, generator=g, device=DEV)
    src = torch.arange(n, dtype=torch.int32, device=DEV)
    src[::3] = -1
    out = torch.empty(n, hq * d, dtype=torch.bfloat16, device=DEV)
    _lib.call("qx_merge_attn_quant", _p(a), a.stride(0), _p(b), b.stride(0), _p(la), la.stride(0),
              _p(lb), lb.stride(0), _p(src), n, hq, d, _p(out), out.stride(0), None, 0, _stream())
    want = _merge_reference(a, b, la, lb, src)
    diff = (out.float() - want).abs()
    ulp = want.abs().clamp_min(1e-30) * 2 ** -7
    assert (diff == 0).float().mean() >= 0.999 and bool((diff <= ulp).all())


def test_tiny_tree_pass_on_config1():
    """Config 1 (seed 0, norm weights 1) through the tree path against the
    float64 oracle, at the unified path's config-1 bounds: at most 0.06 from
    it, at most one document past 0.05, every decision whose exact margin is
    outside +-0.05 the same."""
    cfg = CONFIGS["tiny"]
    wl = make_workload("tiny", seed=0)
    model = build_synthetic(cfg, seed=0, device="cuda", gen_device="cpu", norm_init="ones")
    results, run = run_stage(model, wl, "margins", attention_mode="tree")
    tree = np.array([r[0] - r[1] for r in results], dtype=np.float64)
    want, _ = _oracle_margins(model, wl)
    assert run.stats["borrowed_tokens"] == 15 * 32
    d, agree = _report("tree path, config 1 vs float64", tree, want)
    assert d.max() <= 0.06
    assert np.sum(d > TOL) <= 1
    clear = np.abs(want) > TOL
    assert np.all((tree[clear] > 0) == (want[clear] > 0))


def test_tiny_tree_pass_against_exact_math_and_the_unified_pass():
    """8 seeds x 16 documents through the tree path against the float64
    oracle at the FP8 noise floor's bounds. The tree path rounds call A,
    call B, the merge weight and the merge to bf16 (attention.py:902-948)
    on top of what the unified path rounds, so its spread is a little wider
    (measured max 0.088, rms 0.025, 96.9% within 0.05, 99.2% of decisions):
    max 0.1, rms <= 0.03, >= 96% within 0.05, every decision whose exact
    margin is outside +-0.05 the same, >= 97.5% of all; and the tree and
    unified passes within 2 x 0.05 of each other."""
    cfg = CONFIGS["tiny"]
    got_all, want_all, uni_all = [], [], []
    for seed in range(8):
        wl = make_workload("tiny", seed=seed)
        model = build_synthetic(cfg, seed=seed, device="cuda", gen_device="cpu",
                                norm_init="random")
        results, _ = run_stage(model, wl, "margins", attention_mode="tree")
        got_all.append(np.array([r[0] - r[1] for r in results], dtype=np.float64))
        results, _ = run_stage(model, wl, "margins")
        uni_all.append(np.array([r[0] - r[1] for r in results], dtype=np.float64))
        want_all.append(_oracle_margins(model, wl)[0])
    got, want, uni = map(np.concatenate, (got_all, want_all, uni_all))
    d, agree = _report("tree path, 8 seeds vs float64", got, want)
    assert d.max() <= 0.1
    assert np.sqrt(np.mean(d ** 2)) <= 0.03
    assert np.mean(d <= TOL) >= 0.96
    clear = np.abs(want) > TOL
    assert np.all((got[clear] > 0) == (want[clear] > 0))
    assert agree >= 0.975
    assert np.abs(got - uni).max() <= 2 * TOL


def test_qwen3_4b_tree_attention_equals_the_unified_attention():
    """Layer 0 of Qwen3-4B over the first two packs of 40 benchmark documents
    (64-token shared prefix: children read their parent's pages stacked,
    from the same pack and from the one before), packed both ways: every
    row's attention output (bf16, before the o_proj quantization) agrees.
    The tree result rounds call A, call B, the merge weight and the merge to
    bf16 (attention.py:902-948): about 3 * 2^-9 of max(|a|, |b|), so the
    bound is relative to the head's largest value (the o_proj input's FP8
    group): 99.9% of elements within 2^-7 of it and every one within 2^-5
    (measured 6.4e-3 and 1.7e-2; rows with no resident reads are
    bit-identical)."""
    import dataclasses

    from quail_amd.arena import KVArena
    from quail_amd.chunk import InputStaging, pack_chunk, upload
    from quail_amd.prefix import PrefixIndex
    from quail_amd.qwen3 import Qwen3Pipeline
    from tests.helpers import admit, pack_specs

    cfg = dataclasses.replace(CONFIGS["qwen3-4b"], layers=1)
    wl = make_workload("qwen3-4b", seed=0)
    prompts = wl.prompts[:40]
    model = build_synthetic(cfg, seed=0, device="cuda", norm_init="random")
    prefixes = [p[:-1] for p in prompts]
    suffixes = [[p[-1:]] for p in prompts]
    tree = PrefixIndex(prompts).tree(16)
    runs = {}
    for mode in ("unified", "tree"):
        arena = KVArena(1, 2048, 16, cfg.kv_heads, cfg.head_dim)
        pipe = Qwen3Pipeline(model, arena)
        engine = pipe.engine
        adm = admit(prefixes, suffixes, arena, 3000, tree=tree, unified=mode == "unified")
        outs, stacked = [], 0
        for _ in range(2):
            specs = pack_specs(adm, adm.next_chunk(arena.free_pages))
            if mode == "tree":
                specs = [dict(g, read_key=g["borrow_key"] if g["start"] else None, single=True)
                         for g in specs]
                stacked += sum(g["read_key"] is not None for g in specs)
            chunk = pack_chunk(arena, specs, attention_mode=mode,
                               attention_heads=(cfg.heads, cfg.kv_heads, cfg.head_dim))
            upload(chunk, InputStaging())
            layer = pipe.layers[0]
            q_in, q_scale, _ = engine.embed_norm_quant(chunk.input_ids, pipe.embed.weight,
                                                       layer.input_layernorm)
            q, k, v = pipe._project_qkv(q_in, q_scale, chunk.positions, layer.self_attn)
            n = q.shape[0]
            q3 = q.view(n, cfg.heads, cfg.head_dim)
            k3 = k.view(n, cfg.kv_heads, cfg.head_dim)
            v3 = v.view(n, cfg.kv_heads, cfg.head_dim) if v.is_contiguous() else v
            chunk.meta["layer"] = 0
            if mode == "tree":
                outs.append(engine.attention_tree(q3, k3, v3, chunk.meta, quantize=False))
            else:
                engine.write_kv(k3, v3, chunk.meta)
                outs.append(engine.attention_bf16(q3, chunk.meta, 0))
            for t in chunk.temporary_keys:
                arena.free_key(t)
        torch.cuda.synchronize()
        runs[mode] = (outs, stacked)
    assert runs["tree"][1] > 0
    for got, want in zip(runs["tree"][0], runs["unified"][0]):
        n = want.shape[0]
        g3 = got.float().view(n, cfg.heads, cfg.head_dim)
        w3 = want.float().view(n, cfg.heads, cfg.head_dim)
        amax = w3.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
        rel = ((g3 - w3).abs() / amax).flatten()
        qs = torch.quantile(rel[torch.randperm(rel.numel(), device=rel.device)[:1 << 20]],
                            torch.tensor([0.5, 0.9, 0.99, 0.999], device=rel.device))
        print("tree vs unified attention, |diff| / head amax: quantiles 50/90/99/99.9% "
              + " ".join(f"{v:.2e}" for v in qs.tolist()) + f" max {rel.max().item():.2e}")
        assert qs[3].item() <= 2 ** -7 and rel.max().item() <= 2 ** -5


@pytest.mark.parametrize("hq,hk,d,doc_len", [(32, 8, 128, 37), (4, 2, 64, 300)])
@pytest.mark.parametrize("every_node", [False, True])
def test_label_path_rows_attend_to_document_ancestors_and_path(hq, hk, d, doc_len, every_node):
    """Trie-scored AI.CLASSIFY rows (attention.py:1395-1441 with call C,
    :1424-1434, and merge_partial, :407-429): each path row's attention
    output equals float32 attention over the document's keys (from its
    pages), its trie ancestors' rows and itself, taken from the trie alone,
    not from the pack's maps. Same tolerances as the other tree calls."""
    from oracle.labels_ref import path_reads, path_tokens, read_nodes, trie_paths
    from quail_amd.arena import KVArena
    from quail_amd.chunk import InputStaging, pack_chunk, upload
    from quail_amd.engine import Engine

    labels = ((10,), (20, 21, 22), (20, 25, 26, 27, 28), (30, 31, 32), (30, 31, 33))
    g = torch.Generator().manual_seed(doc_len + d)
    arena = KVArena(1, 64, 16, hk, d)
    engine = Engine(arena, num_q_heads=hq, num_kv_heads=hk, head_dim=d,
                    rotary=type("R", (), {"cos_sin_cache": None})())
    heads = (hq, hk, d)
    doc = list(range(100, 100 + doc_len))
    arena.activate("doc", doc_len)

    def rows(n):
        return [(torch.randn(n, h, d, generator=g) * s).to(torch.bfloat16).to(DEV)
                for h, s in ((hq, 1.0), (hk, 1.0), (hk, 2.0))]

    first = pack_chunk(arena, [dict(key="doc", prefix=doc, f=doc_len, suffixes=[])],
                       attention_mode="tree", attention_heads=heads)
    upload(first, InputStaging())
    q1, k1, v1 = rows(doc_len)
    engine.attention_tree(q1, k1, v1, first.meta, quantize=False)
    read = None if every_node else read_nodes(labels)
    paths = trie_paths(labels, read)
    tokens = path_tokens(paths, 7)
    chunk = pack_chunk(arena, [dict(key="doc", prefix=None, f=doc_len, suffixes=[tokens],
                                    read_all_rows=True, paths=paths,
                                    read_mask=None if every_node else path_reads(paths, read))],
                       attention_mode="tree", attention_heads=heads)
    assert chunk.meta["reads"].get("nodes") is not None
    upload(chunk, InputStaging())
    n = len(tokens)
    q2, k2, v2 = rows(n)
    out = engine.attention_tree(q2, k2, v2, chunk.meta, quantize=False)
    torch.cuda.synchronize()
    row_of = {node: i for i, node in enumerate(nd for nodes, _, _ in paths for nd in nodes)}
    scale = d ** -0.5
    for r, node in enumerate(nd for nodes, _, _ in paths for nd in nodes):
        mine = [row_of[node[:depth]] for depth in range(len(node) + 1)]
        k = torch.cat([k1, k2[mine]])
        v = torch.cat([v1, v2[mine]])
        want, _ = _ref_attention(q2[r:r + 1], k, v, scale, causal=False)
        got = out[r].float().view(1, hq, d)
        assert (got - want).abs().max().item() <= 2e-2, f"row {r} node {node}"


def test_merge_partial_matches_the_reference_merge():
    """qx_merge_partial against the reference's merge_partial
    (attention.py:407-429) in float32: merged rows within one bf16 ulp (the
    kernel may fuse the multiply-add), log-sum-exps to 1e-5; a row with no
    call C keys (-inf) keeps its call B result."""
    g = torch.Generator().manual_seed(5)
    nb, nc, hq, d = 50, 20, 4, 128
    out = torch.randn(nb, hq * d, generator=g).to(torch.bfloat16)
    lse = torch.randn(hq, nb, generator=g) * 3
    index = torch.randperm(nb, generator=g)[:nc]
    oc = torch.randn(nc, hq * d, generator=g).to(torch.bfloat16)
    lc = torch.randn(hq, nc, generator=g) * 3
    lc[1, 3] = float("-inf")
    lb = lse[:, index]
    top = torch.maximum(lb, lc)
    wb, wc = (lb - top).exp(), (lc - top).exp()
    total = wb + wc
    merged = (out[index].float().view(nc, hq, d) * (wb / total).T[..., None]
              + oc.float().view(nc, hq, d) * (wc / total).T[..., None])
    want_out = out.clone()
    want_out[index] = merged.to(torch.bfloat16).view(nc, hq * d)
    want_lse = lse.clone()
    want_lse[:, index] = top + total.log()
    o, l_, i_ = out.to(DEV), lse.to(DEV), index.to(DEV)
    c, lcd = oc.to(DEV), lc.to(DEV)
    _lib.call("qx_merge_partial", _p(o), o.stride(0), _p(l_), l_.stride(0), _p(i_), _p(c),
              c.stride(0), _p(lcd), lcd.stride(0), nc, hq, d, _stream())
    torch.cuda.synchronize()
    got = o.float().cpu()
    want = want_out.float()
    diff = (got - want).abs()
    assert bool((diff <= want.abs() * 2 ** -7 + 1e-30).all())
    assert (diff == 0).float().mean() >= 0.99
    torch.testing.assert_close(l_.cpu(), want_lse, rtol=1e-5, atol=1e-5)
    r = int(index[3])
    assert torch.equal(o[r, 1 * d:2 * d].cpu(), out[r, d:2 * d])


@pytest.mark.parametrize("every_node", [False, True])
def test_tiny_label_path_pass_matches_each_label_prefix_run_whole(every_node):
    """The whole pipeline in tree mode over a label-path pack (trie-scored
    AI.CLASSIFY): a document is computed in one pack, then its trie paths in
    the next, reading it from its pages (call B), their ancestors (call C)
    and their own path (call A). Every read row's final-normed hidden state
    equals the oracle's for its document + cue + node tokens run whole as
    one prompt, within the tiny model's FP8 noise floor (relative 0.06, as
    the unified pack's oracle test)."""
    from oracle import qwen3_ref as ref
    from oracle.labels_ref import path_reads, path_tokens, read_nodes, trie_paths
    from quail_amd.arena import KVArena
    from quail_amd.chunk import InputStaging, pack_chunk, upload
    from quail_amd.qwen3 import Qwen3Pipeline
    from tests.helpers import ref_model

    cfg = CONFIGS["tiny"]
    model = build_synthetic(cfg, seed=4, device="cuda", gen_device="cpu", norm_init="random")
    wl = make_workload("tiny", seed=4)
    doc = list(wl.prompts[0][:-1])
    cue = int(wl.prompts[0][-1])
    labels = ((10,), (20, 21, 22), (20, 25, 26, 27, 28), (30, 31, 32), (30, 31, 33))
    arena = KVArena(cfg.layers, 256, 16, cfg.kv_heads, cfg.head_dim)
    pipe = Qwen3Pipeline(model, arena)
    heads = (cfg.heads, cfg.kv_heads, cfg.head_dim)
    arena.activate("doc", len(doc))
    first = pack_chunk(arena, [dict(key="doc", prefix=doc, f=len(doc), suffixes=[[cue]])],
                       attention_mode="tree", attention_heads=heads)
    upload(first, InputStaging())
    pipe.forward_chunk(first)
    read = None if every_node else read_nodes(labels)
    paths = trie_paths(labels, read)
    mask = path_reads(paths, read)
    chunk = pack_chunk(arena, [dict(key="doc", prefix=None, f=len(doc),
                                    suffixes=[path_tokens(paths, cue)], read_all_rows=True,
                                    paths=paths, read_mask=None if every_node else mask)],
                       attention_mode="tree", attention_heads=heads)
    upload(chunk, InputStaging())
    got = pipe.forward_chunk(chunk).float().cpu()
    nodes = [nd for ns, _, _ in paths for nd in ns]
    prompts = [doc + [cue] + list(nd) for nd, m in zip(nodes, mask) if m]
    want = ref.forward_documents(ref_model(model), prompts).float()
    assert got.shape == want.shape
    rel = ((got - want).norm() / want.norm()).item()
    print(f"label-path rows vs each prefix run whole: relative {rel:.4f}")
    assert rel <= 0.06, rel


def test_tiny_trie_scores_from_the_pipeline_match_each_prefix_run_whole():
    """Trie-scored AI.CLASSIFY end to end with this package's label trie
    (quail_amd.labels: read nodes, paths, the suffix tokens, tree_scores):
    the label-path pack through the tree pipeline, its read rows' log-softmax
    over the label tokens, and tree_scores over them, against the same
    scores from the oracle's final rows of each read node's prompt (document
    + cue + node tokens) run whole: every label's log probability within
    0.05 and the same best label."""
    from oracle import qwen3_ref as ref
    from quail_amd import labels as qlabels
    from quail_amd.arena import KVArena
    from quail_amd.chunk import InputStaging, pack_chunk, upload
    from quail_amd.qwen3 import Qwen3Pipeline
    from tests.helpers import ref_model

    cfg = CONFIGS["tiny"]
    model = build_synthetic(cfg, seed=8, device="cuda", gen_device="cpu", norm_init="random")
    wl = make_workload("tiny", seed=8)
    doc = list(wl.prompts[0][:-1])
    cue = int(wl.prompts[0][-1])
    labels = ((10,), (20, 21, 22), (20, 25, 26, 27, 28), (30, 31, 32), (30, 31, 33), (30,))
    arena = KVArena(cfg.layers, 256, 16, cfg.kv_heads, cfg.head_dim)
    pipe = Qwen3Pipeline(model, arena)
    heads = (cfg.heads, cfg.kv_heads, cfg.head_dim)
    arena.activate("doc", len(doc))
    first = pack_chunk(arena, [dict(key="doc", prefix=doc, f=len(doc), suffixes=[[cue]])],
                       attention_mode="tree", attention_heads=heads)
    upload(first, InputStaging())
    pipe.forward_chunk(first)
    read = qlabels.read_nodes(labels)
    paths = qlabels.trie_paths(labels, read)
    mask = qlabels.path_reads(paths, read)
    chunk = pack_chunk(arena, [dict(key="doc", prefix=None, f=len(doc),
                                    suffixes=[qlabels.path_tokens(paths, cue)],
                                    read_all_rows=True, paths=paths, read_mask=mask)],
                       attention_mode="tree", attention_heads=heads)
    upload(chunk, InputStaging())
    got = pipe.forward_chunk(chunk).float().cpu()
    nodes = [nd for ns, _, _ in paths for nd in ns]
    prompts = [doc + [cue] + list(nd) for nd, m in zip(nodes, mask) if m]
    want = ref.forward_documents(ref_model(model), prompts).float()
    targets = sorted({t for ids in labels for t in ids})
    head = model.lm_head.weight.float().cpu()[targets]

    def scores(rows):
        lp = torch.log_softmax(rows @ head.T, dim=-1).double().numpy()
        return qlabels.tree_scores(labels, paths, targets, lp, read)

    s_gpu, s_ref = scores(got), scores(want)
    print("trie scores gpu", np.round(s_gpu, 4), "oracle", np.round(s_ref, 4))
    assert np.all(np.isfinite(s_ref))
    assert np.abs(s_gpu - s_ref).max() <= 0.05
    assert int(np.argmax(s_gpu)) == int(np.argmax(s_ref))


@pytest.mark.parametrize("labels", [((10,), (20, 21, 22), (20, 25, 26, 27, 28), (30, 31, 32),
                                     (30, 31, 33), (30,)), ((11,), (12,), (13,))])
def test_trie_scored_stage_through_the_stage_driver(labels):
    """A trie-scored AI.CLASSIFY stage through StageRun (tree attention,
    label paths on every document, documents that share a prefix borrowing
    its pages) and the AsyncTrieScores readout: each document's label log
    probabilities against tree_scores over the oracle's rows of its read
    nodes' prompts (document + cue + node tokens) run whole, log-softmax
    over the full vocabulary: the same best label, and each label within
    0.05 per term its score sums (its read nodes' log probabilities, and
    the share its label extensions take, each carrying the tiny model's
    FP8 noise). One-token labels read a single row per document."""
    from oracle import qwen3_ref as ref
    from quail_amd import labels as qlabels
    from quail_amd.arena import KVArena
    from quail_amd.executor import StageRun
    from quail_amd.qwen3 import Qwen3Pipeline
    from quail_amd.readout import AsyncTrieScores
    from tests.helpers import ref_model

    cfg = CONFIGS["tiny"]
    model = build_synthetic(cfg, seed=9, device="cuda", gen_device="cpu", norm_init="random")
    wl = make_workload("tiny", seed=9)
    docs = [list(p[:-1]) for p in wl.prompts[:6]]
    cues = [int(p[-1]) for p in wl.prompts[:6]]
    read = qlabels.read_nodes(labels)
    paths = qlabels.trie_paths(labels, read)
    mask = qlabels.path_reads(paths, read)
    arena = KVArena(cfg.layers, 256, 16, cfg.kv_heads, cfg.head_dim)
    pipe = Qwen3Pipeline(model, arena)
    readout = AsyncTrieScores(model.lm_head.weight, labels, paths, read)
    run = StageRun(pipe, arena, readout, docs,
                   [[qlabels.path_tokens(paths, c)] for c in cues], 512,
                   attention_mode="tree", label_paths=(paths, mask))
    got = run.run()
    torch.cuda.synchronize()
    assert run.stats["borrowed_tokens"] > 0
    head = model.lm_head.weight.float().cpu()
    nodes = [nd for ns, _, _ in paths for nd in ns]
    ends = {tuple(ids) for ids in labels}
    terms = np.array([sum(ids[:k] in read for k in range(len(ids)))
                      + any(o != ids and o[:len(ids)] == ids for o in ends)
                      for ids in map(tuple, labels)])
    worst = 0.0
    for d, (doc, cue) in enumerate(zip(docs, cues)):
        prompts = [doc + [cue] + list(nd) for nd, m in zip(nodes, mask) if m]
        rows = ref.forward_documents(ref_model(model), prompts).float()
        lp = torch.log_softmax(rows @ head.T, dim=-1)[:, readout.targets].double().numpy()
        want = qlabels.tree_scores(labels, paths, readout.targets, lp, read)
        diff = np.abs(got[d] - want)
        print(f"document {d}: |diff| per label {np.round(diff, 4)} (terms {terms.tolist()})")
        worst = max(worst, float((diff / terms).max()))
        assert np.all(np.isfinite(want))
        assert int(np.argmax(got[d])) == int(np.argmax(want)), (d, got[d], want)
    print(f"trie-scored stage, {len(docs)} documents: worst |diff| per term {worst:.4f}")
    assert worst <= 0.05
