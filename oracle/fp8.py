"""OCP e4m3fn rounding and the per-token 128-group FP8 quantization.

Test infrastructure (see oracle/__init__.py).

The reference quantizes activations as
    scale = max(amax, 1e-10) / 448;  q = clamp(y / scale, -448, 448) -> e4m3
(Triton kernels, quail/backends/quail/executor/attention.py:780-786, and the
static reference tests/gpu/test_qwen3_5_kernels.py:12-15). e4m3fn rounding is
round-to-nearest-even; `e4m3_table()` and `round_e4m3_bruteforce()` restate
it from the format definition so the torch conversion used here is pinned.
"""

import numpy as np
import torch

FP8_MAX = 448.0
GROUP = 128
SCALE_FLOOR = 1e-10


def e4m3_table() -> np.ndarray:
    """The 256 e4m3fn code points decoded from the format (1-4-3, bias 7).

    Exponent field 0 is subnormal (m/8 * 2^-6); code 0x7f/0xff are NaN;
    there are no infinities.
    """
    out = np.empty(256, dtype=np.float64)
    for code in range(256):
        sign = -1.0 if code & 0x80 else 1.0
        exp = (code >> 3) & 0xF
        man = code & 0x7
        if exp == 0xF and man == 0x7:
            out[code] = np.nan
        elif exp == 0:
            out[code] = sign * (man / 8.0) * 2.0 ** -6
        else:
            out[code] = sign * (1.0 + man / 8.0) * 2.0 ** (exp - 7)
    return out


def round_e4m3_bruteforce(x: np.ndarray) -> np.ndarray:
    """Round finite |x| <= 448 to the nearest e4m3fn value, ties to even code.

    Brute force over the code table; slow, for pinning the fast path.
    """
    table = e4m3_table()
    finite = np.isfinite(table)
    codes = np.nonzero(finite)[0]
    values = table[codes]
    x = np.asarray(x, dtype=np.float64)
    flat = x.reshape(-1)
    out = np.empty_like(flat)
    for i, v in enumerate(flat):
        d = np.abs(values - v)
        best = d.min()
        ties = codes[d == best]
        if len(ties) > 1:
            # the even mantissa (lowest bit 0) wins; +0 over -0 for zero
            even = [c for c in ties if (c & 1) == 0]
            pick = even[0] if even else ties[0]
        else:
            pick = ties[0]
        out[i] = table[pick]
    return out.reshape(x.shape)


def to_e4m3(x: torch.Tensor) -> torch.Tensor:
    """clamp(x, +-448) rounded to e4m3fn (returned as a float8_e4m3fn tensor)."""
    return x.float().clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)


def group_quant(y: torch.Tensor):
    """Per-token 128-group FP8 quantization of fp32 rows.

    Returns (q e4m3 (n, K), scales fp32 (n, K/128)) with
    scale = max(amax, 1e-10)/448 and q = e4m3(clamp(y/scale)) per group
    (attention.py:780-786, vLLM per_token_group_quant_fp8 at :517-532).
    """
    y = y.float()
    n, k = y.shape
    g = y.view(n, k // GROUP, GROUP)
    amax = g.abs().amax(dim=-1)
    scale = amax.clamp_min(SCALE_FLOOR) / FP8_MAX
    q = to_e4m3(g / scale.unsqueeze(-1)).view(n, k)
    return q, scale


def dequant_rows(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """q (n, K) e4m3 with (n, K/128) scales -> fp32 (n, K)."""
    n, k = q.shape
    return (q.float().view(n, k // GROUP, GROUP) * scale.float().unsqueeze(-1)).view(n, k)


def dequant_weight(w: torch.Tensor, scale_inv: torch.Tensor) -> torch.Tensor:
    """W (N, K) e4m3 with (N/128, K/128) weight_scale_inv -> fp32 (N, K)."""
    n, k = w.shape
    s = scale_inv.float().repeat_interleave(GROUP, 0).repeat_interleave(GROUP, 1)
    return w.float() * s[:n, :k]


def quantize_weight_blocks(w: torch.Tensor):
    """The synthetic checkpoint's block quantization: per 128x128 block
    s = amax/448 and q = e4m3(clamp(w/s)); returns (q, weight_scale_inv).
    A block of zeros gets s = 1 (its codes are all zero either way)."""
    n, k = w.shape
    b = w.float().view(n // GROUP, GROUP, k // GROUP, GROUP)
    amax = b.abs().amax(dim=(1, 3))
    s = torch.where(amax > 0, amax / FP8_MAX, torch.ones_like(amax))
    q = to_e4m3(b / s[:, None, :, None]).view(n, k)
    return q, s
