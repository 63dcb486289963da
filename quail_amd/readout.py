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
  AsyncLabelLogprobs          AI.CLASSIFY label scores: normalize=True
                              full-vocabulary log probabilities
                              (qx_vocab_logprobs), normalize=False bf16
                              logits -> fp32 (readout.py:143-226)
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


class _Pending:
    """A submitted copy: the event after it, its pinned buffer, the rows."""

    __slots__ = ("done", "buf", "rows", "kind")

    def __init__(self, done, buf, rows, kind):
        self.done, self.buf, self.rows, self.kind = done, buf, rows, kind


class _HostReadout:
    """Device rows to pinned host buffers without stalling the stream: the
    copy and an event go on the current stream and result() waits on that
    event alone. Idle buffers are pooled per (dtype, row shape) and sized in
    powers of two rows, so a stage allocates pinned memory a few times at
    most."""

    trailing_rows = 1
    normalize = False

    def __init__(self):
        self._idle = {}

    def _copy(self, values):
        kind = (values.dtype, tuple(values.shape[1:]))
        rows = values.shape[0]
        idle = self._idle.setdefault(kind, [])
        fits = [i for i, b in enumerate(idle) if b.shape[0] >= rows]
        if fits:
            buf = idle.pop(fits[0])
        else:
            cap = max(64, 1 << max(rows - 1, 0).bit_length())
            buf = torch.empty((cap,) + kind[1], dtype=kind[0], pin_memory=True)
        buf[:rows].copy_(values, non_blocking=True)
        done = torch.cuda.Event()
        done.record()
        return _Pending(done, buf, rows, kind)

    def result(self, handle, *, copy=True):
        """The handle's rows as numpy; without copy, a view of the pinned
        buffer that the next submit may overwrite."""
        handle.done.synchronize()
        values = handle.buf[:handle.rows].numpy()
        if copy:
            values = values.copy()
        self._idle[handle.kind].append(handle.buf)
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


def answer_rows(rows_per_answer):
    """Each read row's answer and its row within that answer
    (readout.py:95-107)."""
    counts = np.asarray(rows_per_answer, dtype=np.int64)
    starts = np.repeat(np.cumsum(counts) - counts, counts)
    return (np.repeat(np.arange(len(counts)), counts),
            np.arange(int(counts.sum())) - starts)


class AsyncLabelLogprobs(_HostReadout):
    """AI.CLASSIFY label scores (readout.py:143-226).

    normalize=True: each target token's log probability over the full
    vocabulary at temperature 1 (bf16 logits of every head row, as F.linear
    gives them, and their logsumexp in fp32): one qx_vocab_logprobs pass per
    block of rows, which streams the head once per 128 rows and keeps no
    (rows x vocabulary) logits. normalize=False: the targets' rows of the
    head only, unnormalized bf16 logits as fp32 (qx_answer_head).

    rows > 1 holds up to `rows` read rows per answer, unused rows NaN.
    """

    BLOCK_ROWS = 1024

    def __init__(self, head, targets, rows=1, normalize=True):
        super().__init__()
        self.targets = [int(t) for t in targets]
        vocab, hidden = head.shape
        if not 1 <= len(self.targets) <= 16:
            raise ValueError(f"{len(self.targets)} label tokens; 1..16 are supported")
        if any(not 0 <= t < vocab for t in self.targets):
            raise ValueError(f"label token ids outside the vocabulary of {vocab}")
        if rows < 1:
            raise ValueError("rows must be positive")
        self.rows = rows
        self.normalize = normalize
        t = len(self.targets)
        self.dtype = np.dtype((np.float32, (rows, t) if rows > 1 else (t,)))
        idx = torch.tensor(self.targets, dtype=torch.long, device=head.device)
        if normalize:
            self.head = head if head.dtype == torch.bfloat16 else head.to(torch.bfloat16)
            self.head = self.head.contiguous()
            self.target_ids = idx
            self.head_rows = None
        else:
            self.head = None
            self.head_rows = head.index_select(0, idx).to(torch.bfloat16).contiguous()

    def logprobs(self, normed):
        """(rows, targets) fp32 on the device: log probabilities with
        normalize, logits without."""
        n, h = normed.shape
        t = len(self.targets)
        out = torch.empty((n, t), dtype=torch.float32, device=normed.device)
        if n == 0:
            return out
        if not self.normalize:
            _lib.call("qx_answer_head", normed.data_ptr(), normed.stride(0),
                      self.head_rows.data_ptr(), self.head_rows.stride(0), t, n, h, 0, None, 1.0,
                      out.data_ptr(), None, None, None, _stream())
            return out
        vocab = self.head.shape[0]
        if normed.dtype != torch.bfloat16 or normed.stride(1) != 1:
            normed = normed.to(torch.bfloat16).contiguous()
        for start in range(0, n, self.BLOCK_ROWS):
            block = normed[start:start + self.BLOCK_ROWS]
            rows = block.shape[0]
            size = _lib.count("qx_vocab_logprobs_workspace", rows, vocab, t)
            work = torch.empty(size, dtype=torch.uint8, device=normed.device)
            _lib.call("qx_vocab_logprobs", block.data_ptr(), block.stride(0),
                      self.head.data_ptr(), self.head.stride(0), self.target_ids.data_ptr(), t,
                      out[start:].data_ptr(), out.stride(0), rows, vocab, h, work.data_ptr(),
                      size, _stream())
        return out

    def submit(self, normed, rows_per_answer=None):
        values = self.logprobs(normed)
        if self.rows > 1:
            if rows_per_answer is None:
                rows_per_answer = [1] * values.shape[0]
            if max(rows_per_answer) > self.rows:
                raise ValueError(f"a suffix has {max(rows_per_answer)} rows to read; "
                                 f"the readout holds {self.rows}")
            answers = torch.full((len(rows_per_answer), self.rows, values.shape[1]),
                                 float("nan"), dtype=torch.float32, device=values.device)
            answer_index, row_index = (torch.from_numpy(i).to(values.device)
                                       for i in answer_rows(rows_per_answer))
            answers[answer_index, row_index] = values
            values = answers
        elif rows_per_answer is not None and any(r != 1 for r in rows_per_answer):
            raise ValueError("this readout holds one row per answer")
        return self._copy(values)

class AsyncTrieScores:
    """Trie-scored AI.CLASSIFY (the trie_tree rule, label_stages.py:93-99):
    each document's read path rows through AsyncLabelLogprobs (log
    probabilities of the label tokens over the full vocabulary with
    normalize, or raw logits), then quail_amd.labels.tree_scores: one log
    probability per label, in label order.

    Args:
        head: The model's output head, (vocabulary, hidden).
        label_ids: One token id sequence per label.
        paths, read: From quail_amd.labels (trie_paths, read_nodes); read
            None reads every path row.
        targets: The readout's token ids; None takes the labels' tokens.
    """

    def __init__(self, head, label_ids, paths, read=None, targets=None, normalize=True):
        from quail_amd import labels

        self.trie = labels.LabelTrie(label_ids)
        self.paths, self.read = paths, read
        self.targets = (sorted({t for ids in self.trie.labels for t in ids})
                        if targets is None else [int(t) for t in targets])
        self.read_mask = labels.path_reads(paths, read)
        rows = sum(self.read_mask)
        self.logprobs = AsyncLabelLogprobs(head, self.targets, rows=max(rows, 2),
                                           normalize=normalize)
        self.rows = rows

    def submit(self, normed, rows_per_answer=None):
        """normed: the pack's read rows, each answer's `rows` in path order."""
        if rows_per_answer is None:
            if normed.shape[0] % self.rows:
                raise ValueError(f"{normed.shape[0]} rows for answers of {self.rows}")
            rows_per_answer = [self.rows] * (normed.shape[0] // self.rows)
        if any(r != self.rows for r in rows_per_answer):
            raise ValueError(f"each answer reads the {self.rows} path rows")
        return self.logprobs.submit(normed, rows_per_answer=rows_per_answer)

    def result(self, handle):
        values = self.logprobs.result(handle)
        return [self.trie.scores(self.paths, self.targets, v[:self.rows], self.read)
                for v in values]

