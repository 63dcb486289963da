"""Each gfx950 kernel against the oracle's restatement of the reference op.

Integer/byte work (scatter, embedding gather) must be bit-exact. Floating
point kernels are compared with tolerances written per test:
  * FP8 outputs: scales within 1e-6 relative and >= 99.9% of e4m3 codes
    identical, the rest one code step away (a 1-ulp fp32 difference can
    move a value across an e4m3 rounding boundary);
  * bf16 outputs: within 1 bf16 ulp (2^-8 relative) of the oracle for
    >= 99.9% of elements, and rtol 1e-2 for all;
  * attention: rtol/atol 2e-2 against exact fp32 brute force, the
    reference's own bound (tests/gpu/test_decode_evaluator.py:175-238).
"""

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import qwen3_ref as ref
from quail_amd import _lib
from quail_amd.engine import Engine, _ptr, _stream

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _engine(hq=4, hk=2, d=64, arena=None, cache=None):
    rotary = type("R", (), {})()
    rotary.cos_sin_cache = cache
    return Engine(arena, num_q_heads=hq, num_kv_heads=hk, head_dim=d, rotary=rotary)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _fp8_close(q_gpu, s_gpu, q_ref, s_ref, min_equal=0.999):
    s_gpu = s_gpu.float().cpu()
    s_ref = s_ref.float().cpu()
    torch.testing.assert_close(s_gpu, s_ref, rtol=1e-6, atol=0)
    a = q_gpu.cpu().view(torch.uint8).numpy().astype(np.int32)
    b = q_ref.cpu().view(torch.uint8).numpy().astype(np.int32)
    equal = (a == b).mean()
    assert equal >= min_equal, f"only {equal:.5f} of e4m3 codes equal"
    # the rest are neighbouring codes (same sign, magnitude code +-1)
    diff = a != b
    if diff.any():
        assert np.all(np.abs((a[diff] & 0x7F) - (b[diff] & 0x7F)) <= 1)


def _bf16_close(x, y, min_ulp1=0.999, rtol=1e-2, atol=None):
    x = x.float().cpu()
    y = y.float().cpu()
    scale = y.abs().max().item() + 1e-30
    atol = 1e-3 * scale if atol is None else atol
    torch.testing.assert_close(x, y, rtol=rtol, atol=atol)
    _, exp = torch.frexp(y)
    ulp = torch.ldexp(torch.ones_like(y), exp - 8)       # one bf16 ulp of y
    close = ((x - y).abs() <= ulp.clamp_min(atol * 1e-2)).float().mean().item()
    assert close >= min_ulp1, f"only {close:.5f} within 1 bf16 ulp"


def test_library_is_native_and_gfx950():
    lib = _lib.load()
    assert lib.qx_device_is_gfx950() == 1
    assert torch.cuda.get_device_properties(0).gcnArchName.startswith("gfx950")


# ---- FP8 block-scaled GEMM ---------------------------------------------------

def _gemm_case(m, n, k, seed, device="cpu"):
    g = _gen(seed)
    a = torch.randn(m, k, generator=g)
    q, s = ofp8.group_quant(a)
    w = torch.randn(n, k, generator=g) * 0.02
    wq, ws = ofp8.quantize_weight_blocks(w)
    return q, s, wq, ws


def _run_gemm(q, s, wq, ws, config=None, monkeypatch=None):
    eng = _engine()
    m, k = q.shape
    scales = torch.empty((k // 128, m), dtype=torch.float32, device=DEV)
    scales.copy_(s.T)
    lin = type("L", (), {})()
    lin.weight = wq.to(DEV)
    lin.weight_scale_inv = ws.to(DEV)
    return eng.gemm(q.to(DEV), scales.permute(1, 0), lin)


@pytest.mark.parametrize("m,n,k", [(1, 256, 128), (100, 512, 256), (257, 768, 384),
                                   (64, 128, 256), (333, 1536, 256)])
def test_gemm_small_shapes_match_dequantized_matmul(m, n, k):
    q, s, wq, ws = _gemm_case(m, n, k, seed=m + n + k)
    out = _run_gemm(q, s, wq, ws)
    want = ref.gemm(q, s, ref.RefLinear(wq, ws))
    _bf16_close(out, want)


# the rescale family: bit-identical to each other
GEMM_CONFIGS = (10, 11, 12, 22)
GEMM_CONFIGS_256 = (10, 11, 22)   # N a multiple of 256 (config 12 needs 320)
PROMOTION_CONFIG = 30             # DeepGEMM's promotion form: its own arithmetic
PROMOTION_WIDE_CONFIG = 31        # the same arithmetic on 256 x 320 tiles


@pytest.mark.parametrize("config", GEMM_CONFIGS + (PROMOTION_CONFIG, PROMOTION_WIDE_CONFIG))
def test_gemm_tile_configs_agree(config, monkeypatch):
    q, s, wq, ws = _gemm_case(300, 1280, 512, seed=9)
    monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(config))
    out = _run_gemm(q, s, wq, ws)
    want = ref.gemm(q, s, ref.RefLinear(wq, ws))
    _bf16_close(out, want)


def test_gemm_configs_are_bit_identical(monkeypatch):
    """Every tile configuration computes each element with the same
    operations in the same order (the engine picks configs by shape, and a
    row's result must not depend on it)."""
    q, s, wq, ws = _gemm_case(700, 1280, 1024, seed=11)
    outs = {}
    for config in GEMM_CONFIGS:
        monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(config))
        outs[config] = _run_gemm(q, s, wq, ws).cpu()
    for config, out in outs.items():
        assert torch.equal(out, outs[10]), config


def test_gemm_persistent_config_with_several_tiles_per_workgroup(monkeypatch):
    """More tiles than CUs (20 x 16 = 320 tiles of 256x256 on a persistent
    grid of 256 workgroups, a partial last row of tiles at M = 5000, an even
    number of 128-K blocks so the cross-tile pipeline runs): config 22 walks
    several tiles per workgroup and equals the one-tile-per-workgroup
    configuration bit for bit, and the oracle to the bf16 tolerance."""
    q, s, wq, ws = _gemm_case(5000, 4096, 512, seed=13)
    outs = {}
    for config in GEMM_CONFIGS_256:
        monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(config))
        outs[config] = _run_gemm(q, s, wq, ws).cpu()
    for config in GEMM_CONFIGS_256:
        assert torch.equal(outs[config], outs[10]), config
    want = ref.gemm(q, s, ref.RefLinear(wq, ws))
    _bf16_close(outs[22], want)
    monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(PROMOTION_CONFIG))
    _bf16_close(_run_gemm(q, s, wq, ws), want)


@pytest.mark.parametrize("m,n,k", [(1, 256, 128), (257, 768, 384), (4000, 2560, 768),
                                   (3000, 5120, 1152), (600, 19456, 640)])
def test_gemm_promotion_kernel_edges(m, n, k, monkeypatch):
    """Config 30 (each 128-K block summed from zero by one 16x16x128 MFMA,
    then total += sA * sW * partial) against the oracle: one row, a partial
    token tile, odd numbers of 128-K blocks (the next tile's first block
    chained across an odd count), several tiles per workgroup."""
    q, s, wq, ws = _gemm_case(m, n, k, seed=m + n + k)
    monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(PROMOTION_CONFIG))
    out = _run_gemm(q, s, wq, ws)
    _bf16_close(out, ref.gemm(q, s, ref.RefLinear(wq, ws)))


@pytest.mark.parametrize("m,n,k", [(1, 1280, 128), (257, 1280, 384), (4000, 2560, 768),
                                   (16294, 2560, 4096), (8192, 2560, 9728), (3000, 5120, 1152),
                                   (600, 10240, 640)])
def test_gemm_wide_promotion_tiles_equal_config_30(m, n, k, monkeypatch):
    """Config 31 (256 x 320 tiles; each wave's 160 weight rows in two
    128-row scale blocks, its tiles promoted with their block's scale) is
    config 30's arithmetic: bit-identical on widths that are multiples of
    both 256 and 320 (one row, a partial token tile, odd numbers of 128-K
    blocks, the Qwen3-4B o_proj and down shapes of a pack and of the GEMM-
    alone record, several tiles per workgroup), and the oracle's result to
    the bf16 tolerance."""
    q, s, wq, ws = _gemm_case(m, n, k, seed=m + n + k)
    outs = {}
    for config in (PROMOTION_CONFIG, PROMOTION_WIDE_CONFIG):
        monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(config))
        outs[config] = _run_gemm(q, s, wq, ws)
    assert torch.equal(outs[PROMOTION_CONFIG], outs[PROMOTION_WIDE_CONFIG])
    if m <= 4000:
        _bf16_close(outs[PROMOTION_WIDE_CONFIG], ref.gemm(q, s, ref.RefLinear(wq, ws)))


@pytest.mark.parametrize("m,n,k", [(16294, 2560, 128), (16294, 2560, 256), (9000, 5120, 384)])
def test_gemm_promotion_tile_boundaries_with_few_blocks(m, n, k, monkeypatch):
    """Both promotion configs with one, two and three 128-K blocks per tile
    and two or more tiles per workgroup: a tile's first block (no fragments
    read ahead), its last (the next tile's first block read to no use, the
    loads rewriting its first rows), and a tile whose first block is also
    its last all meet at tile boundaries. Configs 30 and 31 bit-identical,
    and the first and last 1500 rows (the last token tile partial) the
    oracle's to the bf16 tolerance."""
    q, s, wq, ws = _gemm_case(m, n, k, seed=m + n + k)
    outs = {}
    for config in (PROMOTION_CONFIG, PROMOTION_WIDE_CONFIG):
        monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(config))
        outs[config] = _run_gemm(q, s, wq, ws).cpu()
    assert torch.equal(outs[PROMOTION_CONFIG], outs[PROMOTION_WIDE_CONFIG])
    lin = ref.RefLinear(wq, ws)
    for rows in (slice(0, 1500), slice(m - 1500, m)):
        _bf16_close(outs[PROMOTION_WIDE_CONFIG][rows], ref.gemm(q[rows], s[rows], lin))


@pytest.mark.parametrize("m,n,k", [(1, 640, 256), (300, 640, 512), (700, 1920, 1152)])
def test_gemm_wide_promotion_tiles_at_widths_only_320_divides(m, n, k, monkeypatch):
    """Widths that are multiples of 320 but not of 256 take config 31 (the
    engine's choice) and agree with the oracle to the bf16 tolerance."""
    from quail_amd.engine import gemm_config
    monkeypatch.delenv("QUAIL_GEMM_CONFIG", raising=False)
    assert gemm_config(n, k, m) == PROMOTION_WIDE_CONFIG
    q, s, wq, ws = _gemm_case(m, n, k, seed=m + n + k)
    _bf16_close(_run_gemm(q, s, wq, ws), ref.gemm(q, s, ref.RefLinear(wq, ws)))


def test_gemm_configs_agree_with_zero_weight_blocks(monkeypatch):
    """Weight blocks whose scale is 0 add nothing; configurations skip them
    or run them on zero fragments, and all must agree bit for bit: zero
    blocks at the first and last K block, two in a row, and a whole
    128-row weight block column; with 256 x 320 tiles (config 12) each of
    them falls in a wave whose 160 weight rows straddle two scale blocks."""
    q, s, wq, ws = _gemm_case(520, 1280, 1024, seed=17)
    ws = ws.clone()
    ws[0, 0] = 0.0
    ws[1, 7] = 0.0
    ws[2, 3] = ws[2, 4] = 0.0
    ws[5, :] = 0.0
    outs = {}
    for config in GEMM_CONFIGS:
        monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(config))
        outs[config] = _run_gemm(q, s, wq, ws).cpu()
    for config, out in outs.items():
        assert torch.equal(out, outs[10]), config
    want = ref.gemm(q, s, ref.RefLinear(wq, ws))
    _bf16_close(outs[10], want)
    assert torch.all(outs[10][:, 5 * 128:6 * 128] == 0)
    # the promotion form adds 0 * partial for such blocks (finite operands);
    # its 256 x 320 tiles give the same bits
    monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(PROMOTION_CONFIG))
    out = _run_gemm(q, s, wq, ws).cpu()
    _bf16_close(out, want)
    assert torch.all(out[:, 5 * 128:6 * 128] == 0)
    monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(PROMOTION_WIDE_CONFIG))
    assert torch.equal(_run_gemm(q, s, wq, ws).cpu(), out)


@pytest.mark.parametrize("m,i,k,zero_blocks", [(700, 768, 512, False), (333, 1536, 256, True),
                                               (2000, 9728, 2560, False),
                                               (9000, 1280, 128, False),
                                               (9000, 1280, 256, False)])
@pytest.mark.parametrize("config", ["10", "22", "30"])
def test_gate_up_swiglu_quant_equals_gemm_then_activation_quant(m, i, k, zero_blocks, config,
                                                                 monkeypatch):
    """qx_gemm_fp8_swiglu_quant (gate_up GEMM with the SiLU-quant epilogue)
    against the two launches it replaces, bit for bit, within each
    arithmetic family (10 and 22 against the config-10 GEMM, 30 against the
    config-30 GEMM): a partial token tile, the Qwen3-4B gate_up shape
    (I = 9728, K = 2560) and weight blocks whose scale is 0 in both
    halves."""
    eng = _engine()
    g = _gen(m + i + k)
    a = torch.randn(m, k, generator=g)
    q, s = ofp8.group_quant(a)
    w = torch.randn(2 * i, k, generator=g) * 0.02
    wq, ws = ofp8.quantize_weight_blocks(w)
    if zero_blocks:
        ws[1, 0] = 0.0                 # a gate block
        ws[i // 128 + 2, 1] = 0.0      # an up block
    lin = type("L", (), {})()
    lin.weight = wq.to(DEV)
    lin.weight_scale_inv = ws.to(DEV)
    scales = torch.empty((k // 128, m), dtype=torch.float32, device=DEV)
    scales.copy_(s.T)
    q_in = q.to(DEV)
    sv = scales.permute(1, 0)
    monkeypatch.setenv("QUAIL_GEMM_CONFIG", "30" if config == "30" else "10")
    want_q, want_s = eng.activation_quant(eng.gemm(q_in, sv, lin))
    monkeypatch.setenv("QUAIL_GEMM_CONFIG", config)
    got_q, got_s = eng.gate_up_activation_quant(q_in, sv, lin)
    assert got_q.shape == (m, i) and got_s.shape == (m, i // 128)
    assert torch.equal(got_q.view(torch.uint8), want_q.view(torch.uint8))
    assert torch.equal(got_s, want_s)


@pytest.mark.parametrize("m,n,k", [(16294, 6144, 2560), (16294, 2560, 9728), (4000, 19456, 768),
                                   (4000, 19456, 640)])
def test_gemm_persistent_cross_tile_pipeline_at_pack_shapes(m, n, k, monkeypatch):
    """Config 22 (persistent, the next tile's first block loaded during the
    current tile's last) at a pack's qkv and down shapes and at a ragged M
    with several tiles per workgroup (K = 768: six 128-K blocks): bit-identical
    to config 10. At K = 640 (five blocks, an odd count) config 22 falls back
    to config 10's one-tile-per-workgroup launch, which this case checks."""
    q, s, wq, ws = _gemm_case(m, n, k, seed=m + n + k)
    outs = {}
    for config in (10, 22):
        monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(config))
        outs[config] = _run_gemm(q, s, wq, ws)
    assert torch.equal(outs[10], outs[22])


@pytest.mark.parametrize("m,n,k", [(16294, 2560, 4096), (16294, 2560, 9728), (8192, 2560, 4096),
                                   (3000, 5120, 768), (77, 640, 384), (600, 2560, 640)])
def test_gemm_wide_tiles_at_pack_shapes(m, n, k, monkeypatch):
    """Config 12 (256 x 320 tiles, each wave's 160 weight rows straddling two
    128-row scale blocks) at a 16k-row pack's o_proj and down shapes, the
    GEMM-alone o_proj shape, a ragged M, one partial token tile and an odd
    number of 128-K blocks: bit-identical to config 10 (config 11 where N is
    not a multiple of 256). (The engine takes config 31, the promotion
    form's 256 x 320 tiles, at the first three.)"""
    from quail_amd.engine import gemm_config
    q, s, wq, ws = _gemm_case(m, n, k, seed=m + n + k)
    base = 10 if n % 256 == 0 else 11
    outs = {}
    for config in (base, 12):
        monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(config))
        outs[config] = _run_gemm(q, s, wq, ws)
    assert torch.equal(outs[base], outs[12])
    monkeypatch.delenv("QUAIL_GEMM_CONFIG")
    if m >= 8192:
        assert gemm_config(n, k, m) == PROMOTION_WIDE_CONFIG


@pytest.mark.parametrize("config", [None, PROMOTION_CONFIG, 10])
@pytest.mark.parametrize("k,n", [(2560, 6144), (4096, 2560), (2560, 19456), (9728, 2560)])
def test_gemm_qwen3_4b_shapes_at_8192_tokens(k, n, config, monkeypatch):
    """The GEMM-alone config: M=8192 at the four Qwen3-4B projection shapes,
    activations bf16 N(0, 1) quantized per token per 128 columns, weights
    N(0, 0.02) per 128 x 128 block, against the fp32 matmul of the
    dequantized operands (computed on the GPU in fp32 for time); the
    engine's choice (None) and each family forced."""
    if config is not None:
        monkeypatch.setenv("QUAIL_GEMM_CONFIG", str(config))
    m = 8192
    g = torch.Generator(device=DEV).manual_seed(k + n)
    a = torch.randn(m, k, generator=g, device=DEV).to(torch.bfloat16).float()
    q, s = ofp8.group_quant(a)
    w = torch.randn(n, k, generator=g, device=DEV) * 0.02
    wq, ws = ofp8.quantize_weight_blocks(w)
    out = _run_gemm(q, s, wq, ws)
    want = (ofp8.dequant_rows(q, s) @ ofp8.dequant_weight(wq, ws).T).to(torch.bfloat16)
    _bf16_close(out, want, min_ulp1=0.995)


def test_gemm_rejects_bad_shapes():
    eng = _engine()
    q = torch.zeros((4, 200), dtype=torch.float8_e4m3fn, device=DEV)
    lin = type("L", (), {})()
    lin.weight = torch.zeros((256, 200), dtype=torch.float8_e4m3fn, device=DEV)
    lin.weight_scale_inv = torch.ones((2, 2), device=DEV)
    scales = torch.ones((1, 4), device=DEV).permute(1, 0)
    with pytest.raises(_lib.QxError, match="multiple of 128"):
        eng.gemm(q, scales, lin)
    with pytest.raises(ValueError, match="column-major"):
        eng.gemm(q, torch.ones((4, 2), device=DEV)[:, :1], lin)


# ---- norms and quant ------------------------------------------------------------

@pytest.mark.parametrize("n,h", [(1, 256), (37, 2560), (130, 5120), (5, 4096)])
def test_add_rmsnorm_quant(n, h):
    g = _gen(n + h)
    x = (torch.randn(n, h, generator=g) * 3).to(torch.bfloat16)
    res = (torch.randn(n, h, generator=g) * 2).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(h, generator=g)).to(torch.bfloat16)
    eng = _engine()
    res_d = res.to(DEV).clone()
    norm = type("N", (), {"weight": w.to(DEV), "variance_epsilon": 1e-6})()
    q, s = eng.norm_quant(x.to(DEV), norm, res_d)
    q_ref, s_ref, res_ref = ref.add_rms_norm_quant(x, res, w, 1e-6)
    assert torch.equal(res_d.cpu(), res_ref)
    _fp8_close(q, s, q_ref, s_ref)


@pytest.mark.parametrize("n,h", [(3, 256), (64, 2560)])
def test_rmsnorm_quant_and_embed_fused(n, h):
    g = _gen(7 * n + h)
    x = (torch.randn(n, h, generator=g)).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(h, generator=g)).to(torch.bfloat16)
    norm = type("N", (), {"weight": w.to(DEV), "variance_epsilon": 1e-6})()
    eng = _engine()
    q, s = eng.norm_quant(x.to(DEV), norm)
    q_ref, s_ref = ref.norm_quant_first(x, w, 1e-6)
    _fp8_close(q, s, q_ref, s_ref)
    table = (torch.randn(300, h, generator=g) * 0.02).to(torch.bfloat16)
    ids = torch.randint(0, 300, (n,), generator=g)
    q2, s2, res = eng.embed_norm_quant(ids.to(DEV), table.to(DEV), norm)
    assert torch.equal(res.cpu(), table[ids])
    q2_ref, s2_ref = ref.norm_quant_first(table[ids], w, 1e-6)
    _fp8_close(q2, s2, q2_ref, s2_ref)


def test_fused_add_rms_norm_in_place_and_gathered():
    g = _gen(5)
    n, h = 50, 2560
    hid = torch.randn(n, h, generator=g).to(torch.bfloat16)
    res = torch.randn(n, h, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(h, generator=g)).to(torch.bfloat16)
    norm = type("N", (), {"weight": w.to(DEV), "variance_epsilon": 1e-6})()
    eng = _engine()
    rows = torch.tensor([49, 0, 7, 7, 13])
    out = eng.final_norm(hid.to(DEV), res.to(DEV), rows.to(DEV), norm)
    want, _ = ref.fused_add_rms_norm(hid[rows], res[rows], w, 1e-6)
    _bf16_close(out, want, min_ulp1=0.998)
    hd, rd = hid.to(DEV), res.to(DEV)
    eng.fused_add_rms_norm(hd, rd, norm)
    want_all, z = ref.fused_add_rms_norm(hid, res, w, 1e-6)
    assert torch.equal(rd.cpu(), z)
    _bf16_close(hd, want_all, min_ulp1=0.998)


@pytest.mark.parametrize("n,i", [(3, 768), (40, 9728), (7, 12288)])
def test_silu_mul_quant(n, i):
    g = _gen(n * i)
    gu = (torch.randn(n, 2 * i, generator=g) * 2).to(torch.bfloat16)
    eng = _engine()
    q, s = eng.activation_quant(gu.to(DEV))
    q_ref, s_ref = ref.silu_mul_quant(gu)
    _fp8_close(q, s, q_ref, s_ref, min_equal=0.998)


def test_group_quant_matches_and_zero_group_floor():
    g = _gen(11)
    x = torch.randn(9, 4096, generator=g).to(torch.bfloat16)
    x[3, 256:384] = 0
    eng = _engine()
    q, s = eng.quant(x.to(DEV))
    q_ref, s_ref = ofp8.group_quant(x.float())
    _fp8_close(q, s, q_ref, s_ref, min_equal=1.0)
    assert s[3, 2].item() == np.float32(1e-10) / np.float32(448)


def test_group_scales_equal_the_division_bit_for_bit():
    """The kernels form max(amax, 1e-10) / 448 without a division; over
    groups whose maxima span the bf16 range (2^-30 .. 2^127, and the floor)
    every scale must equal torch's fp32 division exactly, and the codes the
    reference's."""
    g = _gen(13)
    rows = 64
    x = torch.randn(rows, 1024, generator=g)
    exps = torch.linspace(-30, 125, rows * 8).round().view(rows, 8)
    x = (x.view(rows, 8, 128) * torch.exp2(exps)[..., None]).view(rows, 1024)
    x[5, :128] = 0
    x = x.to(torch.bfloat16)
    eng = _engine()
    q, s = eng.quant(x.to(DEV))
    q_ref, s_ref = ofp8.group_quant(x.float())
    assert torch.equal(s.cpu().view(torch.int32), s_ref.view(torch.int32))
    _fp8_close(q, s, q_ref, s_ref, min_equal=1.0)


# ---- qk norm + rope -----------------------------------------------------------------

@pytest.mark.parametrize("hq,hk,d", [(4, 2, 64), (32, 8, 128), (64, 8, 128)])
@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float32])
def test_qk_norm_rope(hq, hk, d, cache_dtype):
    n = 77
    g = _gen(hq * d)
    qkv = torch.randn(n, (hq + 2 * hk) * d, generator=g).to(torch.bfloat16)
    pos = torch.randint(0, 4000, (n,), generator=g)
    pos[0] = 0
    cache = ref.rope_cache(d, 4096, 1e6).to(cache_dtype)
    qw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16)
    attn = type("A", (), {})()
    attn.q_norm = type("N", (), {"weight": qw.to(DEV), "variance_epsilon": 1e-6})()
    attn.k_norm = type("N", (), {"weight": kw.to(DEV), "variance_epsilon": 1e-6})()
    eng = _engine(hq, hk, d, cache=cache.to(DEV))
    q, k = eng.qk_norm_rope(qkv.to(DEV), pos.to(DEV), attn)
    q_ref, k_ref = ref.qk_norm_rope(qkv, pos, cache, qw, kw, hq, hk, d, 1e-6)
    _bf16_close(q, q_ref, min_ulp1=0.998)
    _bf16_close(k, k_ref, min_ulp1=0.998)


V_DTYPES = [torch.bfloat16, torch.float16]


@pytest.mark.parametrize("hq,hk,d", [(4, 2, 64), (32, 8, 128)])
@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("v_dtype", V_DTYPES)
def test_qk_norm_rope_kv_equals_norm_rope_then_scatter(hq, hk, d, cache_dtype, v_dtype):
    """The fused pass writes q, and K / V into pool rows dst[i], bit for bit
    as qk_norm_rope followed by kv_row_scatter(src = 0..n-1); dst < 0 rows
    write nothing. Without q (q_out NULL) it writes the same pages."""
    n, pool_rows = 93, 320
    g = _gen(7 * hq + d)
    qkv = (torch.randn(n, (hq + 2 * hk) * d, generator=g) * 3).to(torch.bfloat16).to(DEV)
    pos = torch.randint(0, 4000, (n,), generator=g).to(DEV)
    cache = ref.rope_cache(d, 4096, 1e6).to(cache_dtype).to(DEV)
    attn = type("A", (), {})()
    attn.q_norm = type("N", (), {"weight": (1 + 0.1 * torch.randn(d, generator=g)).to(
        torch.bfloat16).to(DEV), "variance_epsilon": 1e-6})()
    attn.k_norm = type("N", (), {"weight": (1 + 0.1 * torch.randn(d, generator=g)).to(
        torch.bfloat16).to(DEV), "variance_epsilon": 1e-6})()
    dst = torch.randperm(pool_rows, generator=g)[:n].to(DEV)
    dst[[0, 17, n - 1]] = -1
    pools = []
    for _ in range(3):
        kp = torch.full((pool_rows, hk, d), 7.0, dtype=torch.bfloat16, device=DEV)
        vp = torch.full((pool_rows, hk, d), 7.0, dtype=v_dtype, device=DEV)
        pools.append((kp, vp))
    sep = _engine(hq, hk, d, arena=_Arena(*pools[0], 16), cache=cache)
    q_ref, k = sep.qk_norm_rope(qkv, pos, attn)
    sep.kv_row_scatter(k, qkv[:, (hq + hk) * d:], torch.arange(n, device=DEV), dst, 0)
    fused = _engine(hq, hk, d, arena=_Arena(*pools[1], 16), cache=cache)
    meta = {"layer": 0, "unified": {"row_dst": dst}}
    q = fused.qk_norm_rope_kv(qkv, pos, attn, meta)
    # K and V only (q_out NULL): the K heads and the V copy on their own lanes
    _lib.call("qx_qk_norm_rope_kv", _ptr(qkv), qkv.stride(0), None, 0, _ptr(pools[2][0]),
              _ptr(pools[2][1]), _ptr(dst), None, None, None, _ptr(cache),
              int(cache_dtype == torch.float32), _ptr(pos), _ptr(attn.q_norm.weight),
              _ptr(attn.k_norm.weight), n, hq, hk, d, 1e-6, int(v_dtype == torch.float16),
              _stream())
    torch.cuda.synchronize()
    assert meta["kv_fresh_layer"] == 0
    assert torch.equal(q, q_ref)
    for i in (1, 2):
        assert torch.equal(pools[i][0], pools[0][0])
        assert torch.equal(pools[i][1], pools[0][1])
    assert int((pools[1][0].view(pool_rows, -1) != 7.0).all(1).sum()) == n - 3


@pytest.mark.parametrize("v_dtype", V_DTYPES)
def test_qk_norm_rope_rows_with_pages_equals_norm_rope_then_scatters(v_dtype):
    """The tree path's pass: q, contiguous K and V rows, and the same
    K/V into pool rows row_pool_dst[i] (none when negative), bit for bit as
    qk_norm_rope, then the identity and the page scatters."""
    hq, hk, d, n, pool_rows = 32, 8, 128, 70, 256
    g = _gen(31)
    qkv = (torch.randn(n, (hq + 2 * hk) * d, generator=g) * 3).to(torch.bfloat16).to(DEV)
    pos = torch.randint(0, 4000, (n,), generator=g).to(DEV)
    cache = ref.rope_cache(d, 4096, 1e6).to(torch.bfloat16).to(DEV)
    attn = type("A", (), {})()
    attn.q_norm = type("N", (), {"weight": (1 + 0.1 * torch.randn(d, generator=g)).to(
        torch.bfloat16).to(DEV), "variance_epsilon": 1e-6})()
    attn.k_norm = type("N", (), {"weight": (1 + 0.1 * torch.randn(d, generator=g)).to(
        torch.bfloat16).to(DEV), "variance_epsilon": 1e-6})()
    dst = torch.randperm(pool_rows, generator=g)[:n].to(DEV)
    dst[::3] = -1
    pools = [(torch.zeros(pool_rows, hk, d, dtype=torch.bfloat16, device=DEV),
              torch.zeros(pool_rows, hk, d, dtype=v_dtype, device=DEV)) for _ in range(2)]
    sep = _engine(hq, hk, d, arena=_Arena(*pools[0], 16), cache=cache)
    q_ref, k_ref = sep.qk_norm_rope(qkv, pos, attn)
    v_ref = qkv[:, (hq + hk) * d:].to(v_dtype)
    keep = dst >= 0
    sep.kv_row_scatter(k_ref, qkv[:, (hq + hk) * d:], torch.arange(n, device=DEV)[keep],
                       dst[keep], 0)
    fused = _engine(hq, hk, d, arena=_Arena(*pools[1], 16), cache=cache)
    meta = {"layer": 0, "row_pool_dst": dst}
    q, k, v = fused.qk_norm_rope_rows(qkv, pos, attn, meta=meta)
    torch.cuda.synchronize()
    assert meta["kv_fresh_layer"] == 0
    assert torch.equal(q, q_ref) and torch.equal(k, k_ref) and torch.equal(v, v_ref)
    assert torch.equal(pools[1][0], pools[0][0]) and torch.equal(pools[1][1], pools[0][1])


# ---- KV scatter and paged attention ---------------------------------------------------

class _Arena:
    def __init__(self, kp, vp, page):
        self.kp, self.vp, self.page_tokens = kp, vp, page

    def layer_kv(self, layer):
        return self.kp, self.vp


@pytest.mark.parametrize("v_dtype", V_DTYPES)
def test_kv_scatter_is_bit_exact_and_skips_negative_rows(v_dtype):
    """bf16 V pools take the rows as they are; fp16 V pools take them
    rounded to nearest even (as torch converts) and saturated at +-65504
    (torch would give inf), values below fp16's range flush as torch's do."""
    g = _gen(2)
    n, hk, d = 50, 8, 128
    qkv = torch.randn(n, 48 * 128, generator=g).to(torch.bfloat16).to(DEV)
    k = torch.randn(n, hk * d, generator=g).to(torch.bfloat16).to(DEV)
    v = qkv[:, 40 * 128:]                         # strided v slice of qkv
    kp = torch.zeros(256, hk, d, dtype=torch.bfloat16, device=DEV)
    vp = torch.zeros(256, hk, d, dtype=v_dtype, device=DEV)
    src = torch.arange(n, device=DEV)
    dst = torch.randperm(256, generator=g)[:n].to(DEV)
    dst[5] = -1
    eng = _engine(32, hk, d, arena=_Arena(kp, vp, 16))
    eng.kv_row_scatter(k, v, src, dst, 0)
    ok = dst >= 0
    assert torch.equal(kp[dst[ok]], k.view(n, hk, d)[ok])
    assert torch.equal(vp[dst[ok]], v.reshape(n, hk, d)[ok].to(v_dtype))
    written = torch.zeros(256, dtype=torch.bool, device=DEV)
    written[dst[ok]] = True
    assert torch.all(kp[~written] == 0)
    # values past fp16's range, below it, and of both signs
    big = torch.full((1, hk * d), 3.0e38, dtype=torch.bfloat16, device=DEV)
    big[0, ::2] = 1.0e-30
    big[0, 1::4] = -7.0e4
    eng.kv_row_scatter(big, big, torch.zeros(1, dtype=torch.long, device=DEV),
                       torch.full((1,), 3, dtype=torch.long, device=DEV), 0)
    assert torch.equal(kp[3].reshape(1, -1), big)
    if v_dtype == torch.bfloat16:
        assert torch.equal(vp[3].reshape(1, -1), big)
    else:
        want = big.float().clamp(-65504, 65504).half()
        assert torch.equal(vp[3].reshape(1, -1), want)
        assert bool(torch.isfinite(vp[3]).all())
    # NaN stays NaN in either pool type; +-inf saturates to +-65504 in fp16
    # pools and stays inf in bf16 ones
    odd = torch.ones((1, hk * d), dtype=torch.bfloat16, device=DEV)
    odd[0, 0::3] = float("nan")
    odd[0, 1::3] = float("inf")
    odd[0, 2::6] = float("-inf")
    eng.kv_row_scatter(odd, odd, torch.zeros(1, dtype=torch.long, device=DEV),
                       torch.full((1,), 4, dtype=torch.long, device=DEV), 0)
    got = vp[4].reshape(-1).float().cpu()
    src = odd.reshape(-1).float().cpu()
    nan = torch.isnan(src)
    assert torch.equal(torch.isnan(got), nan)
    if v_dtype == torch.bfloat16:
        assert torch.equal(got[~nan], src[~nan])
    else:
        assert torch.equal(got[~nan], src[~nan].clamp(-65504, 65504))


def _paged_case(seed, hq, hk, d, page, seqs, pool_pages):
    g = _gen(seed)
    rng = np.random.default_rng(seed)
    q_lens = rng.integers(1, 150, seqs)
    q_lens[0] = 1
    extra = rng.integers(0, 100, seqs)
    used = q_lens + extra
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    n = int(cu[-1])
    width = int(max(-(-used // page)))
    perm = rng.permutation(pool_pages)
    table = np.zeros((seqs, width), dtype=np.int32)
    at = 0
    for s in range(seqs):
        need = -(-int(used[s]) // page)
        table[s, :need] = perm[at:at + need]
        at += need
    kp = torch.randn(pool_pages * page, hk, d, generator=g).to(torch.bfloat16)
    vp = torch.randn(pool_pages * page, hk, d, generator=g).to(torch.bfloat16)
    q = torch.randn(n, hq, d, generator=g).to(torch.bfloat16)
    return q, kp, vp, cu, used.astype(np.int32), table


@pytest.mark.parametrize("hq,hk,d", [(4, 2, 64), (32, 8, 128), (64, 8, 128), (8, 8, 128)])
@pytest.mark.parametrize("v_dtype", V_DTYPES)
def test_paged_attention_matches_exact_fp32(hq, hk, d, v_dtype):
    page = 16
    q, kp, vp, cu, used, table = _paged_case(hq + d, hq, hk, d, page, 6, 160)
    want = ref.paged_attention(q, kp, vp, cu, used, table, page)
    # an fp16 V pool holds the bf16 values converted (exact at these magnitudes)
    eng = _engine(hq, hk, d, arena=_Arena(kp.to(DEV), vp.to(v_dtype).to(DEV), page))
    meta = dict(unified=dict(cu_q=torch.tensor(cu, device=DEV),
                             used=torch.tensor(used, device=DEV),
                             table=torch.tensor(table, device=DEV),
                             max_q=int(np.diff(cu).max()), max_used=int(used.max()),
                             causal=True))
    got = eng.attention_bf16(q.to(DEV), meta, 0)
    torch.testing.assert_close(got.float().cpu().view_as(want), want.float(), rtol=2e-2, atol=2e-2)
    if d == 128:
        # the fused o_proj quant equals quantizing the bf16 rows
        meta["layer"] = 0
        meta["unified"]["src"] = torch.empty(0, dtype=torch.long, device=DEV)
        o_q, o_s = eng.attention_unified(q.to(DEV), None, None, meta)
        q_ref, s_ref = ofp8.group_quant(got.float().cpu())
        _fp8_close(o_q, o_s, q_ref, s_ref, min_equal=1.0)


@pytest.mark.parametrize("v_dtype", V_DTYPES)
@pytest.mark.parametrize("q_lens,used", [((33, 64, 100, 7), (4200, 4500, 5003, 8190)),
                                         ((16, 40), (32768 + 113, 40960))])
def test_paged_attention_long_sequences_match_exact_fp32(v_dtype, q_lens, used):
    """Sequences past 4096 keys (more than 64 key tiles), up to Qwen3's whole
    40,960-token context (2560 pages, the most the kernel stages), with
    ragged last pages and query tiles, in a shuffled pool: against exact
    fp32 attention."""
    hq, hk, d, page = 32, 8, 128, 16
    rng = np.random.default_rng(41)
    g = _gen(41)
    q_lens = np.array(q_lens, dtype=np.int64)
    used = np.array(used, dtype=np.int64)
    cu = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    need = -(-used // page)
    pool_pages = int(need.sum()) + 5
    perm = rng.permutation(pool_pages)
    table = np.zeros((len(used), int(need.max())), dtype=np.int32)
    at = 0
    for s_, k_ in enumerate(need):
        table[s_, :k_] = perm[at:at + k_]
        at += int(k_)
    kp = torch.randn(pool_pages * page, hk, d, generator=g).to(torch.bfloat16)
    vp = torch.randn(pool_pages * page, hk, d, generator=g).to(torch.bfloat16)
    q = torch.randn(int(cu[-1]), hq, d, generator=g).to(torch.bfloat16)
    want = ref.paged_attention(q, kp, vp, cu, used.astype(np.int32), table, page)
    eng = _engine(hq, hk, d, arena=_Arena(kp.to(DEV), vp.to(v_dtype).to(DEV), page))
    meta = dict(unified=dict(cu_q=torch.tensor(cu, device=DEV),
                             used=torch.tensor(used.astype(np.int32), device=DEV),
                             table=torch.tensor(table, device=DEV),
                             max_q=int(q_lens.max()), max_used=int(used.max()), causal=True))
    got = eng.attention_bf16(q.to(DEV), meta, 0)
    torch.testing.assert_close(got.float().cpu().view_as(want), want.float(), rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("v_dtype", V_DTYPES)
def test_paged_attention_32_row_workgroups_are_bit_identical(v_dtype):
    """The 4-wave workgroups of 32 query rows (two per CU) that packs of short
    documents take give every row of the 8-wave, 64-row workgroups bit for
    bit: through work lists of either height, with bf16 output and with the
    fused o_proj quant, and exact fp32 attention within the kernel
    tolerance. The tile height comes from qx_paged_attention_tile_rows."""
    from quail_amd import _lib
    from quail_amd.chunk import _work_list

    hq, hk, d, page = 32, 8, 128, 16
    q, kp, vp, cu, used, table = _paged_case(91, hq, hk, d, page, 40, 1200)
    want = ref.paged_attention(q, kp, vp, cu, used, table, page)
    eng = _engine(hq, hk, d, arena=_Arena(kp.to(DEV), vp.to(v_dtype).to(DEV), page))
    host = dict(cu_q=cu, used=used, causal=True)
    assert _work_list(host, (hq, hk, d), choose_rows=True)[2] == 32
    outs = {}
    for rows in (0, 32):
        work, n_work = _work_list(host, (hq, hk, d))[:2] if rows == 0 else \
            _work_list(host, (hq, hk, d), choose_rows=True)[:2]
        tables = dict(cu_q=torch.tensor(cu, device=DEV), used=torch.tensor(used, device=DEV),
                      table=torch.tensor(table, device=DEV), max_q=int(np.diff(cu).max()),
                      max_used=int(used.max()), causal=True,
                      work=torch.tensor(work, device=DEV), n_work=n_work, work_rows=rows)
        q3 = q.to(DEV)
        o_q, o_s = eng._paged(q3, tables, 0, None, None)
        o = torch.empty((q.shape[0], hq * d), dtype=torch.bfloat16, device=DEV)
        _lib.call("qx_paged_attention", _ptr(q3), hq * d, _ptr(eng.arena.kp), _ptr(eng.arena.vp),
                  _ptr(tables["cu_q"]), _ptr(tables["used"]), _ptr(tables["table"]),
                  tables["table"].stride(0), len(used), tables["max_q"], tables["max_used"],
                  hq, hk, d, page, float(d ** -0.5), 1, _ptr(o), None, o.stride(0), None, 0,
                  _ptr(tables["work"]), n_work, rows, int(v_dtype == torch.bfloat16), _stream())
        torch.cuda.synchronize()
        outs[rows] = (o_q.view(torch.uint8).clone(), o_s.clone(), o.clone())
    assert torch.equal(outs[0][0], outs[32][0]) and torch.equal(outs[0][1], outs[32][1])
    assert torch.equal(outs[0][2], outs[32][2])
    torch.testing.assert_close(outs[32][2].float().cpu().view_as(want), want.float(), rtol=2e-2,
                               atol=2e-2)


@pytest.mark.parametrize("cache_dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("v_dtype", V_DTYPES)
def test_attention_with_q_norm_on_load_is_bit_identical(cache_dtype, v_dtype):
    """The K/V-only qk-norm-rope pass plus qx_paged_attention_qnorm on the raw
    qkv rows (q normalized and rotated as the attention loads it) write the
    same pages and give the same e4m3 o_proj input and scales, bit for bit,
    as qk_norm_rope_kv (q written) plus qx_paged_attention; with the 32-row
    and the 64-row workgroups, on a bf16 and an fp32 rotary cache."""
    from quail_amd.chunk import _work_list

    hq, hk, d, page = 32, 8, 128, 16
    _, kp, vp, cu, used, table = _paged_case(57, hq, hk, d, page, 30, 1000)
    n = int(cu[-1])
    g = _gen(58)
    qkv = (torch.randn(n, (hq + 2 * hk) * d, generator=g) * 3).to(torch.bfloat16).to(DEV)
    # each row's key position in its sequence and the pool row it goes to
    pos = np.concatenate([np.arange(u - (cu[s_ + 1] - cu[s_]), u)
                          for s_, u in enumerate(used)]).astype(np.int64)
    seq = np.repeat(np.arange(len(used)), np.diff(cu))
    dst = table[seq, pos // page].astype(np.int64) * page + pos % page
    cache = ref.rope_cache(d, 4096, 1e6).to(cache_dtype).to(DEV)
    attn = type("A", (), {})()
    attn.q_norm = type("N", (), {"weight": (1 + 0.1 * torch.randn(d, generator=g)).to(
        torch.bfloat16).to(DEV), "variance_epsilon": 1e-6})()
    attn.k_norm = type("N", (), {"weight": (1 + 0.1 * torch.randn(d, generator=g)).to(
        torch.bfloat16).to(DEV), "variance_epsilon": 1e-6})()
    host = dict(cu_q=cu, used=used, causal=True)
    for choose in (False, True):
        work, n_work, rows = _work_list(host, (hq, hk, d), choose_rows=choose)
        tables = dict(cu_q=torch.tensor(cu, device=DEV), used=torch.tensor(used, device=DEV),
                      table=torch.tensor(table, device=DEV), max_q=int(np.diff(cu).max()),
                      max_used=int(used.max()), causal=True,
                      work=torch.tensor(work, device=DEV), n_work=n_work, work_rows=rows)
        outs = []
        for fused in (False, True):
            kpool, vpool = kp.clone().to(DEV), vp.to(v_dtype).to(DEV)
            eng = _engine(hq, hk, d, arena=_Arena(kpool, vpool, page), cache=cache)
            meta = {"layer": 0, "unified": {"row_dst": torch.tensor(dst, device=DEV)}}
            p_dev = torch.tensor(pos, device=DEV)
            if fused:
                q = eng.kv_norm_rope(qkv, p_dev, attn, meta)
                qnorm = meta.pop("q_norm_on_load")
            else:
                q = eng.qk_norm_rope_kv(qkv, p_dev, attn, meta)
                qnorm = None
            o_q, o_s = eng._paged(q.view(n, hq, d), tables, 0, None, None, qnorm=qnorm)
            torch.cuda.synchronize()
            outs.append((kpool, vpool, o_q.view(torch.uint8).clone(), o_s.clone()))
        assert rows == (32 if choose else 0)
        for a, b in zip(*outs):
            assert torch.equal(a, b)


def test_answer_head_modes():
    g = _gen(13)
    n, h, t = 33, 2560, 6
    normed = torch.randn(n, h, generator=g).to(torch.bfloat16)
    rows = (torch.randn(t, h, generator=g) * 0.02).to(torch.bfloat16)
    cls = torch.tensor([1, 0, 1, -1, 0, 0], dtype=torch.int32)
    from quail_amd.readout import AnswerRows
    ar = AnswerRows.__new__(AnswerRows)
    ar.weights = rows.to(DEV)
    ar.classes = cls.to(DEV)
    for mode in (0, 1):
        logits = torch.empty(n, t, device=DEV)
        bits = torch.empty(n, dtype=torch.uint8, device=DEV)
        yn = torch.empty(n, 2, device=DEV)
        score = torch.empty(n, device=DEV)
        ar.head(normed.to(DEV), mode=mode, logits=logits, bits=bits, yes_no=yn, score=score)
        want = ref.label_logits(normed, rows, mode)
        if mode == 0:
            _bf16_close(logits, want, min_ulp1=0.99)
        else:
            torch.testing.assert_close(logits.cpu(), want, rtol=1e-4, atol=1e-4)
        yes, no, b, sc = ref.answer(normed, rows, cls.tolist(), mode)
        gy, gn = yn[:, 0].cpu(), yn[:, 1].cpu()
        # the bits are the kernel's own yes > no, and its logits are the
        # oracle's to one bf16 ulp (mode 0) or 1e-4 (mode 1): the decisions
        # agree wherever the oracle's yes-no gap is wider than twice that
        assert torch.equal(bits.cpu(), (gy > gn).to(torch.uint8))
        big = torch.maximum(yes.abs(), no.abs())
        slack = 2 * big * 2 ** -7 if mode == 0 else torch.full_like(big, 2e-4)
        clear = (yes - no).abs() > slack
        assert clear.float().mean() >= 0.9
        assert torch.equal(bits.cpu()[clear], b[clear])
        # sigmoid' <= 1/4: one bf16 ulp of a ~1 logit moves the score < 2e-3
        torch.testing.assert_close(score.cpu(), sc, rtol=0, atol=4e-3 if mode == 0 else 1e-4)
