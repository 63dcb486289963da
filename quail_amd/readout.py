"""Readouts of the final rows: the last-token answer head.

The reference readouts (quail/backends/quail/executor/readout.py) with the
same contract: `submit(normed) -> handle`, `result(handle) -> values`, the
class attributes `dtype`, `trailing_rows` and `normalize`; results travel
device -> host through reusable pinned buffers and an event, so the host
never stalls the stream. The head itself is one gfx950 kernel
(qx_answer_head) over the retained label rows:

  AnswerRows / AsyncAnswers   AI.IF bits: max TRUE logit > max FALSE logit,
                              bf16 logits (readout.py:22-92)
  AsyncScores                 AI.SCORE: sigmoid((yes - no) / T), fp32 logits
                              (readout.py:314-339)
  AsyncLabelLogprobs          AI.CLASSIFY with one-token labels and
                              normalize=False: bf16 logits -> fp32
                              (readout.py:143-226)
"""

import numpy as np
import torch

from quail_amd import _lib
from quail_amd.model import answer_weights


def _stream():
    return torch.cuda.current_stream().cuda_stream


class AnswerRows:
    """The retained head rows of one query's two answer classes."""

    def __init__(self, model, true_ids, false_ids):
        self.allowed = sorted(set(true_ids) | set(false_ids))
        self.weights = answer_weights(model, tuple(self.allowed))
        true_set, false_set = set(true_ids), set(false_ids)
        cls = [1 if t in true_set else (0 if t in false_set else -1) for t in self.allowed]
        self.classes = torch.tensor(cls, dtype=torch.int32, device=self.weights.device)
        self.true_cols = [i for i, c in enumerate(cls) if c == 1]
        self.false_cols = [i for i, c in enumerate(cls) if c == 0]

    def head(self, normed, *, mode, bits=None, yes_no=None, score=None, logits=None,
             temperature=1.0):
        n, h = normed.shape
        t = self.weights.shape[0]
        _lib.call("qx_answer_head", normed.data_ptr(), normed.stride(0),
                  self.weights.data_ptr(), self.weights.stride(0), t, n, h, mode,
                  self.classes.data_ptr(), float(temperature),
                  None if logits is None else logits.data_ptr(),
                  None if bits is None else bits.data_ptr(),
                  None if yes_no is None else yes_no.data_ptr(),
                  None if score is None else score.data_ptr(), _stream())

    def logits(self, normed):
        """Per row, the best bf16 logit of each class over its spellings."""
        yes_no = torch.empty((normed.shape[0], 2), dtype=torch.float32, device=normed.device)
        self.head(normed, mode=0, yes_no=yes_no)
        return yes_no[:, 0], yes_no[:, 1]

    def __call__(self, normed):
        bits = torch.empty(normed.shape[0], dtype=torch.uint8, device=normed.device)
        self.head(normed, mode=0, bits=bits)
        return bits.int().cpu().tolist()


class _HostReadout:
    trailing_rows = 1
    normalize = False

    def __init__(self):
        self.available = []

    def _copy(self, values):
        host = self.available.pop() if self.available else None
        if host is None or host.shape[0] < values.shape[0] or host.dtype != values.dtype \
                or host.shape[1:] != values.shape[1:]:
            host = torch.empty((max(values.shape[0], 64),) + tuple(values.shape[1:]),
                               dtype=values.dtype, pin_memory=True)
        host[:values.shape[0]].copy_(values, non_blocking=True)
        event = torch.cuda.Event()
        event.record()
        return event, host, values.shape[0]

    def result(self, handle, *, copy=True):
        event, host, count = handle
        event.synchronize()
        values = host[:count].numpy()
        if copy:
            values = values.copy()
        self.available.append(host)
        return values


class AsyncAnswers(_HostReadout):
    """Non-blocking TRUE/FALSE bits for AI.IF."""

    dtype = None

    def __init__(self, rows: AnswerRows):
        super().__init__()
        self.rows = rows

    def submit(self, normed):
        bits = torch.empty(normed.shape[0], dtype=torch.uint8, device=normed.device)
        self.rows.head(normed, mode=0, bits=bits)
        return self._copy(bits)

    def result(self, handle):
        return [int(b) for b in super().result(handle, copy=False).tolist()]


class AsyncMargins(_HostReadout):
    """Non-blocking (yes, no) best logits per row, bf16-valued (AI.IF's margin)."""

    dtype = np.float32

    def __init__(self, rows: AnswerRows):
        super().__init__()
        self.rows = rows

    def submit(self, normed):
        yes_no = torch.empty((normed.shape[0], 2), dtype=torch.float32, device=normed.device)
        self.rows.head(normed, mode=0, yes_no=yes_no)
        return self._copy(yes_no)


class AsyncScores(_HostReadout):
    """Non-blocking yes-against-no sigmoid for AI.SCORE (fp32 logits)."""

    dtype = np.float32

    def __init__(self, rows: AnswerRows, temperature=1.0):
        super().__init__()
        self.rows = rows
        self.temperature = temperature

    def submit(self, normed):
        score = torch.empty(normed.shape[0], dtype=torch.float32, device=normed.device)
        self.rows.head(normed, mode=1, score=score, temperature=self.temperature)
        return self._copy(score)

    def result(self, handle):
        return super().result(handle, copy=False)


class AsyncLabelLogprobs(_HostReadout):
    """Unnormalized logits of one-token labels (AI.CLASSIFY, normalize=False).

    targets are the label token ids in column order; rows of the full head
    are gathered once. normalize=True (full-vocabulary log-softmax) is not
    part of this engine.
    """

    def __init__(self, head, targets, rows=1, normalize=False):
        super().__init__()
        if normalize:
            raise NotImplementedError("full-vocabulary normalized label scores")
        if rows != 1:
            raise NotImplementedError("one row per answer")
        self.targets = list(targets)
        idx = torch.tensor(self.targets, dtype=torch.long, device=head.device)
        self.head_rows = head.index_select(0, idx).to(torch.bfloat16).contiguous()
        self.rows = rows
        self.normalize = normalize
        self.dtype = np.dtype((np.float32, (len(self.targets),)))
        self._none = torch.full((len(self.targets),), -1, dtype=torch.int32, device=head.device)

    def logprobs(self, normed):
        n, h = normed.shape
        t = len(self.targets)
        out = torch.empty((n, t), dtype=torch.float32, device=normed.device)
        _lib.call("qx_answer_head", normed.data_ptr(), normed.stride(0),
                  self.head_rows.data_ptr(), self.head_rows.stride(0), t, n, h, 0, None, 1.0,
                  out.data_ptr(), None, None, None, _stream())
        return out

    def submit(self, normed, rows_per_answer=None):
        if rows_per_answer is not None and any(r != 1 for r in rows_per_answer):
            raise ValueError("this readout holds one row per answer")
        return self._copy(self.logprobs(normed))
