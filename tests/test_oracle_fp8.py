"""Pins the oracle's e4m3fn rounding and group quantization.

The oracle rounds with torch's float8_e4m3fn conversion; these checks tie
that conversion to the format definition (OCP e4m3fn: bias 7, max 448, no
infinities) by brute force over the code table, at every midpoint where a
mistaken rounding mode or saturation would show.
"""

import numpy as np
import torch

from oracle import fp8


def test_code_table_known_values():
    t = fp8.e4m3_table()
    assert t[0x00] == 0.0
    assert t[0x7E] == 448.0            # largest finite
    assert t[0xFE] == -448.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert t[0x08] == 2.0 ** -6        # smallest normal
    assert t[0x01] == 2.0 ** -9        # smallest subnormal
    assert t[0x38] == 1.0
    assert t[0x39] == 1.125
    finite = t[np.isfinite(t)]
    assert len(finite) == 254


def test_torch_conversion_matches_bruteforce_at_midpoints_and_codes():
    t = fp8.e4m3_table()
    pos = np.sort(np.unique(t[np.isfinite(t) & (t >= 0)]))
    mids = (pos[:-1] + pos[1:]) / 2
    # exact code points, midpoints (ties), and points just off the midpoints
    xs = np.concatenate([pos, mids, mids * (1 + 1e-6), mids * (1 - 1e-6)])
    xs = np.concatenate([xs, -xs])
    got = torch.tensor(xs, dtype=torch.float32).to(torch.float8_e4m3fn).float().numpy()
    want = fp8.round_e4m3_bruteforce(xs.astype(np.float32).astype(np.float64))
    np.testing.assert_array_equal(got, want)


def test_ties_round_to_even_mantissa():
    # 1.0625 is halfway between 1.0 (even code 0x38) and 1.125 (odd 0x39)
    assert fp8.to_e4m3(torch.tensor([1.0625])).float().item() == 1.0
    # 1.1875 is halfway between 1.125 (odd) and 1.25 (even 0x3a)
    assert fp8.to_e4m3(torch.tensor([1.1875])).float().item() == 1.25


def test_clamp_saturates_instead_of_nan():
    x = torch.tensor([500.0, -1e6, 448.0, 464.0])
    np.testing.assert_array_equal(fp8.to_e4m3(x).float().numpy(), [448, -448, 448, 448])


def test_group_quant_closed_form():
    g = torch.Generator().manual_seed(3)
    y = torch.randn(5, 384, generator=g) * 7
    y[2, 128:256] = 0.0                       # an all-zero group
    q, s = fp8.group_quant(y)
    amax = y.view(5, 3, 128).abs().amax(-1)
    np.testing.assert_allclose(s.numpy(), np.maximum(amax.numpy(), 1e-10) / 448.0, rtol=0)
    assert s[2, 1].item() == np.float32(1e-10) / np.float32(448.0)
    # the group's largest element maps to +-448 exactly
    big = (q.float().view(5, 3, 128).abs().amax(-1))
    assert torch.all((big == 448.0) | (amax == 0))
    # dequantized error within half an e4m3 step (relative 1/16) of each value
    deq = fp8.dequant_rows(q, s)
    err = (deq - y).abs()
    assert torch.all(err <= y.abs() / 16 + s.repeat_interleave(128, 1) * 2.0 ** -9 + 1e-12)


def test_weight_block_quant_roundtrip():
    g = torch.Generator().manual_seed(4)
    w = torch.randn(256, 384, generator=g) * 0.02
    q, s = fp8.quantize_weight_blocks(w)
    assert s.shape == (2, 3)
    deq = fp8.dequant_weight(q, s)
    rel = ((deq - w).abs() / (w.abs() + 1e-9)).median()
    assert rel < 0.04
    amax = w.view(2, 128, 3, 128).abs().amax(dim=(1, 3))
    torch.testing.assert_close(s, amax / 448.0)
