"""Admission for one AI.IF / AI.SCORE / AI.CLASSIFY stage over documents.

Decides which documents form each pack, under the pack's token budget and
the arena's free pages, in prefix-tree order (parents before children,
quail/backends/quail/executor/admission.py:424), and whether a document
reads its tree parent's prefix pages instead of recomputing them. This is
the one-stage case of the reference's JoinAdmission.next_chunk
(admission.py:702-866), written around this engine's own state:

  * every document is QUEUED, then ADMITTED once its first rows are packed
    (its pages are activated then), and LENDABLE once all of its prefix is
    packed: a child packed in the same pack after it, or in a later one,
    reads those rows (the layer loop writes a pack's KV before any row of
    it attends);
  * a child reads its parent's first `shared` tokens (prefix-tree sharing,
    a multiple of the page size) when the parent is lendable, still
    resident and holds at least that many tokens; a child whose parent is
    queued or still mid-prefill waits; otherwise it packs its whole prefix;
  * a document longer than one pack is prefilled in pieces (chunked
    prefill, admission.py:611-648, 817; stage_executor.py:1176-1189): its
    pages are activated for the whole document at admission, each later
    pack first continues it with as many prefix tokens as fit (positions
    from where the last piece ended, reading its own pages before that),
    and its question follows in the pack that writes its last prefix token
    when there is room, else in the next;
  * admission stops at the first document short of pages, so documents
    take the arena in tree order; a document short of pack room only waits
    for the next pack.
"""

from collections import deque

import numpy as np

from quail_amd import _lib

QUEUED, ADMITTED, LENDABLE = 0, 1, 2
WAIT = "wait"


class OversizedDocumentError(ValueError):
    """A document that no pack or no arena can hold."""

    def __init__(self, anchor, reason):
        super().__init__(f"document {anchor}: {reason}")
        self.anchor = anchor
        self.reason = reason


class StageAdmission:
    """Packs of one stage over `prefixes` (per document token arrays), each
    document asked `suffixes[d]` (a list of token arrays).

    next_chunk() returns [(document, group)]; a group is the dict
    pack_chunk lays out. A group with no suffixes is a prefill piece: it
    writes prefix rows and reads no answer.
    """

    def __init__(self, prefixes, suffixes, arena, chunk_budget, tree=None, keys=None):
        self.prefixes = [np.asarray(p, dtype=np.int64) for p in prefixes]
        self.suffixes = [[np.asarray(s, dtype=np.int64) for s in sufs] for sufs in suffixes]
        self.arena = arena
        self.chunk_budget = int(chunk_budget)
        n = len(self.prefixes)
        self.keys = list(keys) if keys is not None else [("doc", d) for d in range(n)]
        self.tree_parent = [None] * n if tree is None else list(tree.parent)
        self.tree_shared = [0] * n if tree is None else [int(s) for s in tree.shared]
        self.suffix_rows = [int(sum(len(s) for s in sufs)) for sufs in self.suffixes]
        # the attention kernel's page-table row: longer documents are
        # refused here, not at their first attention launch
        max_keys = _lib.count("qx_paged_attention_max_keys", arena.page_tokens)
        for d in range(n):
            if self.suffix_rows[d] > self.chunk_budget:
                raise OversizedDocumentError(
                    d, f"its {self.suffix_rows[d]} question rows exceed the "
                       f"{self.chunk_budget}-token pack")
            need = arena.pages_needed(len(self.prefixes[d]) + self.suffix_rows[d])
            if need > arena.num_pages:
                raise OversizedDocumentError(
                    d, f"{need} KV pages, more than the {arena.num_pages} of the whole arena")
            keys = len(self.prefixes[d]) + self.suffix_rows[d]
            if keys > max_keys:
                raise OversizedDocumentError(
                    d, f"{keys} tokens, more keys than the paged attention's {max_keys} "
                       f"per sequence")
        self.state = [QUEUED] * n
        # document -> (parent, tokens read from it); documents that read none are absent
        self.lender = {}
        self.borrowed_tokens = 0
        # the children that may still read a document's pages: the arena
        # keeps its pages until each has been admitted
        self.readers_left = [0] * n
        for p in self.tree_parent:
            if p is not None:
                self.readers_left[p] += 1
        self.queue = deque(range(n) if tree is None else tree.order)
        # documents mid-prefill -> the next prefix token to pack (insertion order)
        self.prefilling = {}
        # documents whose first rows are packed (their first group reads the parent)
        self._started = set()
        self.admitted_order = []
        self.pieces = 0

    def done(self) -> bool:
        return not self.queue and not self.prefilling

    # ---- reading a parent's pages ----------------------------------------------

    def _reads_from(self, d):
        """WAIT, None (pack the whole prefix) or (parent, tokens to read)."""
        p = self.tree_parent[d]
        if p is None:
            return None
        if self.state[p] != LENDABLE:
            return WAIT
        tokens = self.tree_shared[d]
        if tokens <= 0 or not self.arena.can_borrow(self.keys[p], tokens):
            return None
        return p, tokens

    def _admit(self, d, reads):
        self.state[d] = ADMITTED
        self.admitted_order.append(d)
        if reads is not None:
            self.lender[d] = reads
            self.borrowed_tokens += reads[1]
        if self.readers_left[d]:
            self.arena.hold(self.keys[d], self.readers_left[d])
        p = self.tree_parent[d]
        if p is not None:
            # admitted either way: the parent's pages need not wait for it
            self.readers_left[p] -= 1
            self.arena.release(self.keys[p])

    # ---- groups -----------------------------------------------------------------

    def _group(self, d, start, end, with_suffixes, first, kept=False):
        """Rows start..end of d's prefix and, optionally, its suffixes; kept:
        no prefix rows (all of them are in its pages already)."""
        f = len(self.prefixes[d])
        g = dict(key=self.keys[d], f=f if with_suffixes else end, start=start,
                 prefix=None if kept else self.prefixes[d][start:end],
                 suffixes=self.suffixes[d] if with_suffixes else [])
        reads = self.lender.get(d)
        g["borrow_key"] = self.keys[reads[0]] if first and reads is not None else None
        return g

    def _continue(self, d, room, groups):
        """The next piece of a document mid-prefill within room; returns the room left."""
        f = len(self.prefixes[d])
        start = self.prefilling[d]
        first = d not in self._started
        self._started.add(d)
        end = min(f, start + room)
        rest = room - (end - start)
        if end == f and self.suffix_rows[d] <= rest:
            # the prefix's last rows and the question in one group
            groups.append((d, self._group(d, start, end, True, first, kept=end == start)))
            del self.prefilling[d]
            self.state[d] = LENDABLE
            return rest - self.suffix_rows[d]
        if end > start:
            groups.append((d, self._group(d, start, end, False, first)))
            self.pieces += 1
        self.prefilling[d] = end
        if end == f:
            # every prefix row is written by this pack: children may read it
            self.state[d] = LENDABLE
        return rest

    def next_chunk(self, room=None):
        """Groups for the next pack, with their arena pages activated.

        Returns a list of (document, group dict). Empty when nothing fits
        (the caller frees pages and retries) or when all are admitted.
        """
        room = self.chunk_budget if room is None else int(room)
        groups = []
        # 1) documents mid-prefill continue first: their pages are held
        for d in list(self.prefilling):
            if room <= 0:
                break
            room = self._continue(d, room, groups)
        # 2) queued documents in tree order
        held = []
        arena = self.arena
        while self.queue and room > 0:
            d = self.queue.popleft()
            f = len(self.prefixes[d])
            most = f + self.suffix_rows[d]  # its rows when it borrows nothing
            if most <= self.chunk_budget and most - max(self.tree_shared[d], 0) > room:
                # too big for the room however much it borrows (and never a
                # long document): held, as the checks below would decide,
                # without asking the arena what it could borrow
                held.append(d)
                continue
            reads = self._reads_from(d)
            if reads == WAIT:
                held.append(d)
                continue
            start = 0 if reads is None else reads[1]
            f = len(self.prefixes[d])
            rows = f - start + self.suffix_rows[d]
            long = rows > self.chunk_budget
            if rows > room and not long:
                held.append(d)          # the next pack has the room
                continue
            lend = None if reads is None else (self.keys[reads[0]], start)
            pages = arena.activate(self.keys[d], f, capacity_tokens=f + self.suffix_rows[d],
                                   borrow=lend)
            if pages is None:
                held.append(d)          # pages come free as answers are read
                break
            self._admit(d, reads)
            if long:
                self.prefilling[d] = start
                room = self._continue(d, room, groups)
                continue
            self.state[d] = LENDABLE
            self._started.add(d)
            groups.append((d, self._group(d, start, f, True, True)))
            room -= rows
        self.queue.extendleft(reversed(held))
        return groups
