"""Admission for one AI.IF / AI.SCORE / AI.CLASSIFY stage over documents.

Chooses which documents form each pack under the pack's token budget and
the arena's free pages, in prefix-tree order, deciding per document whether
it borrows its parent's prefix pages. This is the single-stage case of the
reference's JoinAdmission.next_chunk (quail/backends/quail/executor/
admission.py:702-866) with its Borrowing rules (:65-157):

  * documents are taken in tree order (parents before children, :424);
  * a document whose parent is not yet admitted waits (Borrowing.decide);
  * an admitted parent that still holds the shared tokens is borrowed
    from, in the same pack or a later one; otherwise the document packs
    whole;
  * a document packs [prefix past the borrowed tokens | its suffixes]; it
    needs pages for prefix + suffix rows less the borrowed pages;
  * admission stops at the first document short of pages (arena order is
    kept) and skips, for this pack only, documents short of pack room.
"""

from collections import deque

import numpy as np


class OversizedDocumentError(ValueError):
    def __init__(self, anchor, reason):
        super().__init__(f"document {anchor}: {reason}")
        self.anchor = anchor
        self.reason = reason


class Borrowing:
    WAIT = "wait"

    def __init__(self, n, tree=None, can_borrow=None):
        self.tree_parent = [None] * n if tree is None else list(tree.parent)
        self.tree_shared = [0] * n if tree is None else list(tree.shared)
        self.tree = tree
        self.can_borrow = can_borrow
        self.admitted = set()
        self.skipped = set()
        self.chosen = {}
        self.borrowed_tokens = 0

    @property
    def order(self):
        return None if self.tree is None else self.tree.order

    def borrowers(self):
        counts = [0] * len(self.tree_parent)
        for p in self.tree_parent:
            if p is not None:
                counts[p] += 1
        return counts

    def decide(self, document, chunk):
        parent = self.tree_parent[document]
        if parent is None or parent in self.skipped:
            return None
        if parent not in self.admitted:
            return self.WAIT
        if self.can_borrow is not None and not self.can_borrow(document, parent, parent in chunk):
            return None
        return parent, self.tree_shared[document]

    def record(self, document, choice):
        self.admitted.add(document)
        if choice is not None:
            self.chosen[document] = choice
            self.borrowed_tokens += choice[1]

    def parent(self, document):
        return self.chosen.get(document, (None, 0))[0]

    def shared(self, document):
        return self.chosen.get(document, (None, 0))[1]


class StageAdmission:
    """Packs of one stage over `prefixes` (per document token arrays) each
    asked `suffixes[d]` (a list of token arrays)."""

    def __init__(self, prefixes, suffixes, arena, chunk_budget, tree=None, keys=None):
        self.prefixes = [np.asarray(p, dtype=np.int64) for p in prefixes]
        self.suffixes = [[np.asarray(s, dtype=np.int64) for s in sufs] for sufs in suffixes]
        self.arena = arena
        self.chunk_budget = chunk_budget
        n = len(self.prefixes)
        self.keys = list(keys) if keys is not None else [("doc", d) for d in range(n)]
        self.borrowing = Borrowing(
            n, tree, can_borrow=lambda d, p, same: arena.can_borrow(self.keys[p],
                                                                    self.borrowing.tree_shared[d]))
        order = tree.order if tree is not None else range(n)
        self.pending = deque(order)
        self.suffix_rows = [int(sum(len(s) for s in sufs)) for sufs in self.suffixes]
        for d in range(n):
            need = len(self.prefixes[d]) + self.suffix_rows[d]
            if need > chunk_budget:
                raise OversizedDocumentError(d, f"{need} rows exceed the {chunk_budget}-token pack")
            if arena.pages_needed(need) > arena.num_pages:
                raise OversizedDocumentError(d, "more pages than the whole arena")
        # parents stay resident until every borrower has been admitted
        self.borrowers_left = self.borrowing.borrowers()
        self.admitted_order = []

    def done(self) -> bool:
        return not self.pending

    def _release_parent(self, d):
        p = self.borrowing.tree_parent[d]
        if p is not None:
            self.borrowers_left[p] -= 1
            self.arena.release(self.keys[p])

    def next_chunk(self, room=None):
        """Groups for the next pack, with their arena pages activated.

        Returns a list of (document, group dict). Empty when nothing fits
        (the caller frees pages and retries) or when all are admitted.
        """
        room = self.chunk_budget if room is None else room
        groups, admitted, held = [], set(), []
        arena = self.arena
        while self.pending:
            d = self.pending.popleft()
            choice = self.borrowing.decide(d, admitted)
            if choice == Borrowing.WAIT:
                held.append(d)
                continue
            shared = 0 if choice is None else choice[1]
            prefix = self.prefixes[d]
            rows = len(prefix) - shared + self.suffix_rows[d]
            if rows > room:
                held.append(d)
                continue
            f = len(prefix)
            borrow = None if choice is None else (self.keys[choice[0]], shared)
            pages = arena.activate(self.keys[d], f, capacity_tokens=f + self.suffix_rows[d],
                                   borrow=borrow)
            if pages is None:
                held.append(d)
                break
            if self.borrowers_left[d]:
                arena.hold(self.keys[d], self.borrowers_left[d])
            self.borrowing.record(d, choice)
            self._release_parent(d)
            admitted.add(d)
            self.admitted_order.append(d)
            room -= rows
            groups.append((d, dict(key=self.keys[d], prefix=prefix[shared:], f=f,
                                   start=shared, suffixes=self.suffixes[d],
                                   borrow_key=None if borrow is None else borrow[0])))
        self.pending.extendleft(reversed(held))
        return groups
