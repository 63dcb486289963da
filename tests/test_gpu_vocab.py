"""Full-vocabulary label log probabilities (qx_vocab_logprobs, the
normalize=True readout of readout.py:143-200) against a float64 restatement:
logits = bf16(normed . head^T) (F.linear's bf16 output), then
logit[target] - logsumexp(logits), with the Qwen3 vocabulary (151,936 rows,
a partial last block of 256) and row counts that use every tile shape.

Tolerance: a logit whose fp32 sum falls next to a bf16 rounding boundary may
round one bf16 step differently from the float64 sum, so each value is within
one bf16 step of its target logit plus 1e-4; nearly all are within 1e-4.
"""

import numpy as np
import pytest
import torch

from quail_amd import _lib
from quail_amd.readout import AsyncLabelLogprobs

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(n, vocab, hidden, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    normed = torch.randn(n, hidden, generator=g, device=DEV).to(torch.bfloat16)
    head = (torch.randn(vocab, hidden, generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    return normed, head


def _want(normed, head, targets):
    logits = (normed.double() @ head.double().T).to(torch.bfloat16).double()
    lse = torch.logsumexp(logits, dim=1, keepdim=True)
    return logits[:, targets] - lse, logits[:, targets]


def _close(got, want, target_logits):
    got, want, tl = got.double().cpu(), want.cpu(), target_logits.cpu()
    # one bf16 step of the target logit: 2^(exponent - 7)
    step = torch.exp2(torch.floor(torch.log2(tl.abs().clamp_min(1e-30))) - 7)
    err = (got - want).abs()
    assert torch.all(err <= step + 1e-4), float((err - step).max())
    assert (err <= 1e-4).double().mean() >= 0.99


@pytest.mark.parametrize("n,vocab,hidden", [(1, 151936, 2560), (37, 151936, 2560),
                                            (100, 151936, 2560), (300, 4096, 256),
                                            (64, 1000, 128)])
def test_vocab_logprobs_match_float64(n, vocab, hidden):
    normed, head = _case(n, vocab, hidden, seed=n + vocab)
    targets = [0, 11, vocab // 2, vocab - 1, 11]
    readout = AsyncLabelLogprobs(head, targets, normalize=True)
    got = readout.logprobs(normed)
    want, tl = _want(normed, head, targets)
    assert got.shape == (n, len(targets))
    _close(got, want, tl)
    # the repeated target reads the same logit
    assert torch.equal(got[:, 1], got[:, 4])


def test_normalized_minus_logits_is_the_row_logsumexp():
    """normalize=True minus normalize=False (the targets' bf16 logits) is one
    number per row, -logsumexp, for every target."""
    normed, head = _case(20, 151936, 2560, seed=3)
    targets = [5, 600, 151935]
    lp = AsyncLabelLogprobs(head, targets, normalize=True).logprobs(normed).double()
    lg = AsyncLabelLogprobs(head, targets, normalize=False).logprobs(normed).double()
    diff = (lp - lg).cpu()
    assert torch.allclose(diff, diff[:, :1].expand_as(diff), atol=1e-4, rtol=0)
    want = -torch.logsumexp((normed.double() @ head.double().T).to(torch.bfloat16).double(),
                            dim=1).cpu()
    assert torch.allclose(diff[:, 0], want, atol=2e-3, rtol=0)


def test_rows_per_answer_fill_nan():
    normed, head = _case(5, 4096, 256, seed=9)
    readout = AsyncLabelLogprobs(head, [1, 2], rows=3, normalize=True)
    values = readout.result(readout.submit(normed, rows_per_answer=[2, 3]))
    assert values.shape == (2, 3, 2)
    flat = readout.logprobs(normed).cpu().numpy()
    assert np.array_equal(values[0, :2], flat[:2]) and np.isnan(values[0, 2]).all()
    assert np.array_equal(values[1], flat[2:])
    with pytest.raises(ValueError, match="rows to read"):
        readout.submit(normed, rows_per_answer=[4, 1])


def test_rejects_bad_arguments():
    normed, head = _case(4, 1000, 128, seed=1)
    with pytest.raises(ValueError, match="outside the vocabulary"):
        AsyncLabelLogprobs(head, [1000], normalize=True)
    t = torch.tensor([1], dtype=torch.long, device=DEV)
    out = torch.empty(4, 1, device=DEV)
    small = torch.empty(8, dtype=torch.uint8, device=DEV)
    with pytest.raises(_lib.QxError, match="workspace"):
        _lib.call("qx_vocab_logprobs", normed.data_ptr(), normed.stride(0), head.data_ptr(),
                  head.stride(0), t.data_ptr(), 1, out.data_ptr(), 1, 4, 1000, 128,
                  small.data_ptr(), 8, torch.cuda.current_stream().cuda_stream)
