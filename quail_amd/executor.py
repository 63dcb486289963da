"""The GPU loop of one stage: admission -> pack -> forward -> readout.

The reference's StageExecutor.run / _run_part / _run_one
(quail/backends/quail/executor/stage_executor.py:1036-1062, 1115-1277) for
one AI.IF / AI.SCORE / AI.CLASSIFY stage, paged, with finished documents
freed:

  * each pass asks admission for its groups and prefill pieces; while the
    GPU runs the pass, the answers of the pass before it are read (pinned
    buffers and events), so answers arrive one pass late and a document's
    pages are freed as its last answer is read;
  * a document is admitted by reserving its pages (retained KV of earlier
    operators is evicted to make room, never the document's own pages or
    its parent's); a parent with children in the tree is held until each
    child has packed its first rows; when admission reports the free pages
    short, retained KV is evicted before the next pass;
  * a pass whose temporary question pages do not fit evicts retained KV
    and retries, then runs as two halves (the prefill pieces with the
    first);
  * with nothing buildable, the oldest answers are read (their pages come
    free), retained KV is evicted, and as a last resort parents' holds are
    dropped (their queued children pack whole).

Under tree attention a stage may carry label paths (trie-scored
AI.CLASSIFY): each document's one suffix is then the paths' tokens, every
read row goes to the readout, and readout.AsyncTrieScores turns them into
label scores.
"""

import time
from collections import deque

import numpy as np

from quail_amd.admission import StageAdmission
from quail_amd.chunk import ArenaFullError, InputStaging, pack_chunk, upload
from quail_amd.prefix import PrefixIndex


class StageRun:
    def __init__(self, pipeline, arena, readout, prefixes, suffixes, chunk_budget,
                 use_tree=True, staging=None, attention_mode="unified", label_paths=None):
        if label_paths is not None and attention_mode != "tree":
            raise ValueError("label paths run under attention_mode='tree'")
        # (paths, read_mask) of trie-scored AI.CLASSIFY (label_stages.py:93-99):
        # every document's one suffix holds the paths' tokens
        self.label_paths = label_paths
        self.pipeline = pipeline
        self.arena = arena
        self.readout = readout
        self.prefixes = prefixes
        self.suffixes = suffixes
        self.chunk_budget = min(chunk_budget, pipeline.max_chunk_tokens)
        self.use_tree = use_tree
        if attention_mode not in ("unified", "tree"):
            raise ValueError(f"attention_mode {attention_mode!r}")
        self.attention_mode = attention_mode
        self.staging = staging or InputStaging()
        self.stats = dict(chunks=0, fresh_tokens=0, borrowed_tokens=0, pack_s=0.0,
                          admission_s=0.0, prefill_pieces=0, splits=0, evict_retries=0,
                          evictions=0, drop_holds=0)
        # per pass: (groups, prefill pieces) and its rows, in launch order
        self.passes = []
        self.pass_rows = []

    # ---- admission callbacks ----------------------------------------------------------

    def _reserve(self, d, reads, rows):
        """Pages for an admitted document, and the holds its readers need
        (stage_executor.py:584-620)."""
        adm, arena = self._adm, self.arena
        key = adm.keys[d]
        f = adm.flen[d]
        parent, shared = (None, 0) if reads is None else reads
        evicted = arena.evicted_keys
        ok = arena.reserve(key, f, capacity_tokens=f + adm.extra,
                           borrow=(adm.keys[parent], shared) if shared else None)
        self.stats["evictions"] += arena.evicted_keys - evicted
        if not ok:
            return False
        if parent is not None:
            # the parent's pages stay until the document has packed its first rows
            arena.read_state((adm.keys[parent],))
            self._reserved_parents[d] = adm.keys[parent]
        if d not in self._held_parents and self._borrowers[d]:
            self._held_parents.add(d)
            arena.hold(key, self._borrowers[d])
        return True

    def _free_pages(self) -> int:
        """The free pages admission may grant (the arena's free list)."""
        return self.arena.free_pages

    def _evict(self, pages):
        keys = self.arena.evict_retained(pages)
        self.stats["evictions"] += len(keys)
        return keys

    # ---- the loop -----------------------------------------------------------------------

    def run(self):
        """Answers for every document, in document order: a document asked
        one question gets that answer, one asked several the list of them."""
        n = len(self.prefixes)
        t0 = time.perf_counter()
        tree = None
        if self.use_tree:
            tree = PrefixIndex.from_parts(
                [[p, *sufs] for p, sufs in zip(self.prefixes, self.suffixes)]
            ).tree(self.arena.page_tokens)
        unified = self.attention_mode == "unified"
        single = all(len(s) == 1 for s in self.suffixes)
        # a single question lives in the document's own pages on the unified
        # path (stage_executor.py:392-399); several take temporary pages
        extra = max(len(s[0]) for s in self.suffixes) if unified and single and n else 0
        adm = StageAdmission(self.prefixes, self.suffixes, self.arena, self.chunk_budget,
                             tree=tree, extra_tokens=extra, temporary_pages=unified,
                             reserve=self._reserve)
        self._adm = adm
        self._borrowers = adm.borrowers()
        self._held = [adm.keys[d] for d, c in enumerate(self._borrowers) if c]
        self._held_parents, self._reserved_parents = set(), {}
        self._outstanding = deque()
        self._results = [None] * n
        self.stats["admission_s"] += time.perf_counter() - t0
        arena = self.arena
        while not adm.done():
            if len(self._outstanding) > 1:
                self._report_next()
            if adm.blocked_pages:
                self._evict(adm.blocked_pages)
            t = time.perf_counter()
            groups = adm.next_chunk(self._free_pages())
            prefills = adm.take_prefills()
            self.stats["admission_s"] += time.perf_counter() - t
            if not groups and prefills:
                self._run_part([], prefills)
                self._prefilled(prefills)
                continue
            if not groups:
                if adm.done():
                    continue
                if self._outstanding:
                    self._report_next()
                    continue
                if adm.blocked_pages and self._evict(adm.blocked_pages):
                    continue
                if arena.drop_holds(self._held):
                    # parents freed but held for queued children: those pack whole
                    self.stats["drop_holds"] += 1
                    continue
                raise ArenaFullError("no document fits the free KV arena")
            self._run_part(groups, prefills)
            self._prefilled(prefills)
            for d, first, _, carried in groups:
                parent = adm.tree_parent[d]
                if carried and first == 0 and parent is not None:
                    arena.release(adm.keys[parent])    # the child packed its first rows
                if d in self._reserved_parents:
                    arena.done_reading((self._reserved_parents.pop(d),))
        while self._outstanding:
            self._report_next()
        arena.drop_holds(self._held)
        self.stats["borrowed_tokens"] += adm.borrowed_tokens
        self.stats["prefill_pieces"] += adm.pieces
        return self._results

    def _prefilled(self, prefills):
        """A document's first piece has run: its parent's hold for it and its
        read of the parent end (stage_executor.py:1176-1189)."""
        adm = self._adm
        for d, start, _ in prefills:
            if start != adm.shared(d):
                continue
            parent = adm.tree_parent[d]
            if parent is not None:
                self.arena.release(adm.keys[parent])
            if d in self._reserved_parents:
                self.arena.done_reading((self._reserved_parents.pop(d),))

    def _report_next(self):
        """Read the oldest pass's answers; a finished document's pages go free."""
        handle, groups = self._outstanding.popleft()
        values = [] if handle is None else self.readout.result(handle)
        adm = self._adm
        i = 0
        for d, first, end, _ in groups:
            count = end - first
            if adm.report(d, first, end, list(values[i:i + count])):
                answers = adm.answers[d]
                self._results[d] = answers[0] if len(answers) == 1 else list(answers)
                key = adm.keys[d]
                if self.arena.is_resident(key):
                    self.arena.free_key(key)
            i += count

    def _run_part(self, groups, prefills=()):
        """Run one pass, recovering when its temporary pages do not fit
        (stage_executor.py:1036-1062): evict retained KV and retry, then run
        it as two halves (the prefill pieces with the first)."""
        try:
            self._run_one(groups, prefills)
        except ArenaFullError:
            adm = self._adm
            rows = sum((adm.flen[d] if carried else 0) + int(adm.cum[d][end] - adm.cum[d][first])
                       for d, first, end, carried in groups)
            evicted = self._evict(self.arena.pages_needed(rows))
            if evicted:
                self.stats["evict_retries"] += 1
                self._run_part(groups, prefills)
                return
            if len(groups) < 2:
                raise
            self.stats["splits"] += 1
            half = len(groups) // 2
            self._run_part(groups[:half], prefills)
            self._run_part(groups[half:])

    def _run_one(self, groups, prefills):
        adm = self._adm
        specs = ([adm.group_spec(*g) for g in groups]
                 + [adm.piece_spec(*p) for p in prefills])
        chunk = self._pack(specs)
        self.passes.append((list(groups), list(prefills)))
        self.pass_rows.append(int(chunk.tokens))
        self.stats["chunks"] += 1
        self.stats["fresh_tokens"] += chunk.tokens
        try:
            normed = self.pipeline.forward_chunk(chunk)
        finally:
            for key in chunk.temporary_keys:
                self.arena.free_key(key)
        # the earlier passes' answers, while the GPU runs this one
        while self._outstanding:
            self._report_next()
        handle = None
        if groups:
            per_answer = chunk.rows_per_answer
            if per_answer is not None and len(per_answer) and int(np.max(per_answer)) > 1:
                # several read rows per answer (label paths, read_all_rows)
                handle = self.readout.submit(normed,
                                             rows_per_answer=[int(r) for r in per_answer])
            else:
                handle = self.readout.submit(normed)
        self._outstanding.append((handle, list(groups)))

    def _pack(self, specs):
        t = time.perf_counter()
        engine = self.pipeline.engine
        if self.attention_mode == "tree":
            # a borrowing document with one question reads its parent's
            # pages stacked with its siblings (stage_executor.py:772-774)
            # (prefill pieces read no parent this way: they have no suffix)
            specs = [dict(g, read_key=g.get("borrow_key") if g.get("start") and len(g["suffixes"])
                          else None, single=len(g["suffixes"]) == 1) for g in specs]
            if self.label_paths is not None:
                paths, mask = self.label_paths
                specs = [dict(g, paths=paths, read_mask=mask, read_all_rows=True)
                         if len(g["suffixes"]) else g for g in specs]
        chunk = pack_chunk(self.arena, specs, attention_mode=self.attention_mode,
                           attention_heads=(engine.num_q_heads, engine.num_kv_heads,
                                            engine.head_dim))
        upload(chunk, self.staging)
        self.stats["pack_s"] += time.perf_counter() - t
        return chunk
