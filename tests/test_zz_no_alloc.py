"""The allocation-free full-vocabulary readout (qx_vocab_logprobs_noalloc)
against the entry point with a caller workspace (qx_vocab_logprobs), through
the C ABI: the same kernels, so the same bits, on two calls in a row (the
second with fewer rows, after the first left its partials in the shared
array), on the Qwen3 vocabulary; and the size limit is refused."""

import pytest
import torch

from quail_amd import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda"
V, H = 151936, 2560


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _with_workspace(normed, head, targets, out):
    n, t = normed.shape[0], targets.shape[0]
    size = _lib.count("qx_vocab_logprobs_workspace", n, V, t)
    work = torch.empty(size, dtype=torch.uint8, device=DEV)
    _lib.call("qx_vocab_logprobs", normed.data_ptr(), normed.stride(0), head.data_ptr(),
              head.stride(0), targets.data_ptr(), t, out.data_ptr(), out.stride(0), n, V, H,
              work.data_ptr(), size, _stream())


def _no_alloc(normed, head, targets, out):
    n, t = normed.shape[0], targets.shape[0]
    _lib.call("qx_vocab_logprobs_noalloc", normed.data_ptr(), normed.stride(0), head.data_ptr(),
              head.stride(0), targets.data_ptr(), t, out.data_ptr(), out.stride(0), n, V, H,
              _stream())


def test_no_alloc_equals_the_workspace_entry_point_twice():
    g = torch.Generator(device=DEV).manual_seed(5)
    head = (torch.randn(V, H, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    targets = torch.tensor([10, 11, 151935, 0, 77777], dtype=torch.int64, device=DEV)
    limit = _lib.count("qx_vocab_logprobs_noalloc_max_bytes")
    assert limit == 8 << 20
    for n in (300, 37):     # the second call: fewer rows over the first call's leftovers
        assert _lib.count("qx_vocab_logprobs_workspace", n, V, targets.shape[0]) <= limit
        normed = torch.randn(n, H, generator=g, device=DEV).to(torch.bfloat16)
        want = torch.full((n, targets.shape[0]), float("nan"), device=DEV)
        got = torch.full_like(want, float("nan"))
        _with_workspace(normed, head, targets, want)
        _no_alloc(normed, head, targets, got)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(want).all())
        assert torch.equal(got, want)


def test_no_alloc_refuses_more_rows_than_its_array_holds():
    n = 2048        # 1187 head blocks x 2048 rows of partials: 19 MiB
    assert _lib.count("qx_vocab_logprobs_workspace", n, V, 2) > \
        _lib.count("qx_vocab_logprobs_noalloc_max_bytes")
    with pytest.raises(_lib.QxError, match="more than its"):
        _lib.call("qx_vocab_logprobs_noalloc", 16, H, 16, H, 16, 2, 16, 2, n, V, H, None)
