"""Admission for one AI.IF / AI.SCORE / AI.CLASSIFY stage over documents.

Decides which documents form each pack, under the pack's token budget and
the arena's free pages, in prefix-tree order, and whether a document reads
its tree parent's prefix pages instead of recomputing them. It takes the
decisions of the reference's JoinAdmission.next_chunk for one stage with
chunked prefill (quail/backends/quail/executor/admission.py:702-866,
611-648), so that pack compositions, prefill pieces and page tables match
the reference's on the same inputs (tests/test_stage_golden.py):

  * a pack is filled in priority order: documents whose prefill has ended
    run their questions first (their pages are already written), then the
    next pieces of documents mid-prefill, then fresh documents in tree
    order;
  * a fresh document is priced at its prefix pages (the tokens past what
    it borrows) plus the largest temporary question cost of the stage,
    and admission stops at the first one the free pages cannot take
    (pages are granted in tree order); one short of pack room waits for
    the next pack;
  * a child borrows its parent's first `shared` tokens (a page multiple)
    when the parent is admitted, its prefix fully written, and the arena
    can serve the borrow; a child whose parent is queued or mid-prefill
    waits; otherwise it packs its whole prefix;
  * a document whose prefix and first question do not fit one pack is
    admitted with its pages reserved whole and writes its prefix in
    pieces that fill the room left in each pack; its questions run in the
    pack after its last piece, and its children wait for that pack;
  * questions are atomic: a document's questions run in as many packs as
    the room and the temporary question pages allow.

The caller reserves a document's pages when it is admitted (`reserve`)
and reports every answered question (`report`); a document whose last
question is answered is finished.
"""

from bisect import bisect_right
from collections import deque
from itertools import accumulate

import numpy as np

from quail_amd import _lib

QUEUED, ACTIVE, DONE = -1, 0, 1
WAIT = "wait"


class OversizedDocumentError(ValueError):
    """A document that no pack or no arena can hold."""

    def __init__(self, anchor, reason):
        super().__init__(f"document {anchor}: {reason}")
        self.anchor = anchor
        self.reason = reason


class StageAdmission:
    """Packs of one stage over `prefixes` (per document token arrays), each
    document asked `suffixes[d]` (a list of token arrays, its questions).

    next_chunk(free_pages) returns groups (document, first question, end
    question, carried): the document's questions first..end-1 and, when
    carried, its prefix rows past what it borrows; take_prefills() the
    pass's prefill pieces (document, start, end). reserve(document,
    borrow, rows) -> bool, when given, allocates a document's pages as it
    is admitted; False keeps it queued and ends the pass's admissions.

    extra_tokens: rows past the prefix a document's own pages cover (the
    one question of the unified path); temporary_pages: whether questions
    take temporary pages (the unified path), priced at admission.
    """

    def __init__(self, prefixes, suffixes, arena, chunk_budget, tree=None, keys=None,
                 extra_tokens=0, temporary_pages=True, reserve=None):
        self.prefixes = [np.asarray(p, dtype=np.int64) for p in prefixes]
        self.suffixes = [[np.asarray(s, dtype=np.int64) for s in sufs] for sufs in suffixes]
        self.arena = arena
        self.chunk_budget = int(chunk_budget)
        self.extra = int(extra_tokens)
        self.temporary_pages = bool(temporary_pages)
        self.reserve = reserve
        n = len(self.prefixes)
        self.keys = list(keys) if keys is not None else [("doc", d) for d in range(n)]
        self.tree_parent = [None] * n if tree is None else list(tree.parent)
        self.tree_shared = [0] * n if tree is None else [int(s) for s in tree.shared]
        page = arena.page_tokens
        self.flen = [len(p) for p in self.prefixes]
        # per document, the questions' cumulative rows and (below) temporary
        # pages, as plain int lists (bisected per pass; built once per stage
        # for every document, so kept out of numpy's per-call cost)
        self.cum = [list(accumulate((len(s) for s in sufs), initial=0)) for sufs in self.suffixes]
        # temporary pages per question: its rows past the document's last
        # partial page (admission.py:54-62)
        self.page_cum = [list(accumulate((-(-(self.flen[d] % page + len(s)) // page)
                                          for s in self.suffixes[d]), initial=0))
                         for d in range(n)]
        # the attention kernel's page-table row: longer documents are
        # refused here, not at their first attention launch
        max_keys = _lib.count("qx_paged_attention_max_keys", page)
        self.page_need = []      # pages of the whole prefix and its extra rows
        self.page_reserve = 0    # the stage's largest temporary question cost
        self.min_fresh = float("inf")
        for d in range(n):
            if not self.suffixes[d]:
                raise OversizedDocumentError(d, "no question")
            longest = max(len(s) for s in self.suffixes[d])
            if longest > self.chunk_budget:
                raise OversizedDocumentError(
                    d, f"its {longest}-token question exceeds the {self.chunk_budget}-token "
                       f"pack")
            need = arena.pages_needed(self.flen[d] + self.extra)
            pc = self.page_cum[d]
            largest = max(b - a for a, b in zip(pc, pc[1:])) if self.temporary_pages else 0
            if need + largest > arena.num_pages:
                raise OversizedDocumentError(
                    d, f"{need + largest} KV pages, more than the {arena.num_pages} of the "
                       f"whole arena")
            keys = self.flen[d] + self.cum[d][-1]
            if keys > max_keys:
                raise OversizedDocumentError(
                    d, f"{keys} tokens, more keys than the paged attention's {max_keys} "
                       f"per sequence")
            self.page_need.append(need)
            self.page_reserve = max(self.page_reserve, largest)
            # the fewest rows it can pack fresh: past a borrow, with its
            # first question; a document longer than a pack fits any room
            least = max(0, self.flen[d] - self.tree_shared[d]) + self.cum[d][1]
            self.min_fresh = min(self.min_fresh, 1 if least > self.chunk_budget else least)
        self.state = [QUEUED] * n
        self.next_q = [0] * n
        self.answers = [[] for _ in range(n)]
        self.in_flight = 0
        self.pending = deque(range(n) if tree is None else tree.order)
        self.ready = deque()       # documents whose prefill ended: questions next
        self.prefill = {}          # document mid-prefill -> its next prefix token
        self.prefilled = []        # documents whose last piece is in this pass
        self.prefills = []         # this pass's pieces (document, start, end)
        self.admitted = set()
        self.writing = set()       # admitted, prefix not fully written yet
        self.lender = {}           # document -> (parent, tokens it reads)
        self.borrowed_tokens = 0
        self.blocked_pages = 0
        self.pieces = 0
        self.admitted_order = []

    def done(self) -> bool:
        return (not self.pending and not self.ready and not self.prefill
                and not self.prefilled and not self.in_flight)

    # ---- borrowing ----------------------------------------------------------------

    def parent(self, d):
        return self.lender.get(d, (None, 0))[0]

    def shared(self, d):
        return self.lender.get(d, (None, 0))[1]

    def borrowers(self):
        """Per document, how many documents the tree has read from it."""
        counts = [0] * len(self.prefixes)
        for p in self.tree_parent:
            if p is not None:
                counts[p] += 1
        return counts

    def _reads_from(self, d, admitted_now):
        """WAIT, None (pack the whole prefix) or (parent, tokens to read).

        A parent admitted in this pack has no pages yet and can always
        serve; one admitted earlier serves while its pages hold the tokens."""
        p = self.tree_parent[d]
        if p is None:
            return None
        if p not in self.admitted or p in self.writing:
            return WAIT
        tokens = self.tree_shared[d]
        key = self.keys[p]
        if ((p not in admitted_now or self.arena.is_resident(key))
                and not self.arena.can_borrow(key, tokens)):
            return None
        return p, tokens

    # ---- pieces and questions ----------------------------------------------------

    def take_prefills(self):
        out, self.prefills = self.prefills, []
        return out

    def _piece(self, d, room):
        """The document's next prefix piece within room; returns the room left."""
        start = self.prefill[d]
        end = min(self.flen[d], start + room)
        self.prefills.append((d, start, end))
        self.pieces += 1
        if end == self.flen[d]:
            del self.prefill[d]
            self.prefilled.append(d)
        else:
            self.prefill[d] = end
        return room - (end - start)

    def _fit(self, d, i, room, page_room):
        """How far from question i fits room rows and page_room temporary
        pages: (end question, rows, pages)."""
        cum = self.cum[d]
        end = bisect_right(cum, cum[i] + room) - 1
        pages = 0
        if self.temporary_pages:
            pc = self.page_cum[d]
            end = min(end, bisect_right(pc, pc[i] + page_room) - 1)
            pages = int(pc[end] - pc[i])
        return end, int(cum[end] - cum[i]), pages

    def _question_pages(self, d, i):
        return int(self.page_cum[d][i + 1] - self.page_cum[d][i]) if self.temporary_pages else 0

    def _launch(self, d, end):
        """A group launched up to question end; True when questions are left."""
        self.next_q[d] = end
        self.in_flight += 1
        return end < len(self.suffixes[d])

    # ---- packs -------------------------------------------------------------------

    def next_chunk(self, free_pages, room=None):
        """Groups for the next pack: [(document, first, end, carried)]."""
        self.blocked_pages = 0
        for d in self.prefilled:
            # its prefix is written: its questions run now, its children may read it
            self.writing.discard(d)
            self.ready.append(d)
        self.prefilled = []
        room = self.chunk_budget if room is None else int(room)
        groups, again, later = [], [], []
        question_pages = 0
        # documents with questions left (their pages are written)
        for _ in range(len(self.ready)):
            if room == 0:
                break
            d = self.ready.popleft()
            i = self.next_q[d]
            if self.cum[d][i + 1] - self.cum[d][i] > room:
                later.append(d)
                continue
            end, rows, pages = self._fit(d, i, room, free_pages)
            if end == i:
                self.blocked_pages = self._question_pages(d, i) - free_pages
                self.ready.appendleft(d)
                break
            free_pages -= pages
            question_pages += pages
            groups.append((d, i, end, False))
            room -= rows
            if self._launch(d, end):
                again.append(d)
        # the next pieces of documents mid-prefill
        for d in list(self.prefill):
            if not room:
                break
            room = self._piece(d, room)
        # fresh documents in tree order
        held, admitted_now = [], set()
        while self.pending and room >= self.min_fresh:
            d = self.pending.popleft()
            reads = self._reads_from(d, admitted_now)
            if reads == WAIT:
                held.append(d)
                continue
            need = (self.page_need[d] if reads is None
                    else self.arena.pages_needed(self.flen[d] - reads[1] + self.extra))
            required = need + max(0, self.page_reserve - question_pages)
            if required > free_pages:
                # pages are granted in tree order: nothing behind it goes first
                self.blocked_pages = required - free_pages
                held.append(d)
                break
            carried = self.flen[d] - (0 if reads is None else reads[1])
            first = int(self.cum[d][1])
            long = carried + first > self.chunk_budget
            if long and not room:
                held.append(d)
                continue
            if carried + first > room and not long:
                held.append(d)      # the next pack has the room
                continue
            if long:
                end = rows = pages = 0
            else:
                end, rows, pages = self._fit(d, 0, room - carried, free_pages - need)
                if end == 0:
                    held.append(d)
                    self.blocked_pages = need + self._question_pages(d, 0) - free_pages
                    break
            if self.reserve is not None and not self.reserve(d, reads,
                                                             self.chunk_budget - room):
                held.append(d)
                break
            question_pages += pages
            free_pages -= need + pages
            self.state[d] = ACTIVE
            admitted_now.add(d)
            self.admitted.add(d)
            self.admitted_order.append(d)
            if reads is not None:
                self.lender[d] = reads
                self.borrowed_tokens += reads[1]
            if long:
                # its prefix goes in pieces; its questions follow them
                self.prefill[d] = self.flen[d] - carried
                self.writing.add(d)
                room = self._piece(d, room)
                continue
            groups.append((d, 0, end, carried > 0))
            room -= carried + rows
            if self._launch(d, end):
                again.append(d)
        self.pending.extendleft(reversed(held))
        self.ready.extendleft(reversed(again))
        self.ready.extendleft(reversed(later))
        return groups

    def report(self, d, first, end, values) -> bool:
        """Answers of questions first..end-1; True when d is finished."""
        if len(self.answers[d]) != first or len(values) != end - first:
            raise AssertionError(f"document {d}: answers {first}:{end} arrived with "
                                 f"{len(self.answers[d])} recorded")
        self.answers[d].extend(values)
        self.in_flight -= 1
        if end == len(self.suffixes[d]):
            self.state[d] = DONE
            return True
        return False

    # ---- pack layout --------------------------------------------------------------

    def group_spec(self, d, first, end, carried):
        """The pack_chunk group of a launched question group."""
        shared = self.shared(d) if carried else 0
        parent = self.parent(d) if carried else None
        return dict(key=self.keys[d], f=self.flen[d], start=shared,
                    prefix=self.prefixes[d][shared:] if carried else None,
                    suffixes=self.suffixes[d][first:end],
                    borrow_key=self.keys[parent] if carried and shared else None)

    def piece_spec(self, d, start, end):
        """The pack_chunk group of a prefill piece: prefix rows start..end-1,
        read after the rows before start (its parent's for a first piece that
        borrows, else its own)."""
        shared = self.shared(d)
        parent = self.parent(d)
        borrow = (self.keys[parent] if start == shared and shared
                  else self.keys[d] if start else None)
        return dict(key=self.keys[d], f=end, start=start, prefix=self.prefixes[d][start:end],
                    suffixes=[], borrow_key=borrow)
