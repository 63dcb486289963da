"""The GPU loop of one stage: admission -> pack -> forward -> readout.

The reference's StageExecutor.run / _run_one
(quail/backends/quail/executor/stage_executor.py:66-89, 1115-1174,
1191-1344) for one AI.IF / AI.SCORE / AI.CLASSIFY stage: the host packs
pack N+1 while the GPU runs pack N; answers are read one pack late through
pinned buffers and events; temporary pages are freed after each forward
pass (stream order keeps later writers behind it); a document's pages are
freed once its answer is read, or when its last borrower is admitted.
Documents longer than a pack are prefilled in pieces (admission), and a
pack that finds the arena full reads the answers in flight, evicts
retained KV, or runs as two halves. Under tree attention a stage may
carry label paths (trie-scored AI.CLASSIFY): each document's one suffix
is then the paths' tokens, every read row goes to the readout, and
readout.AsyncTrieScores turns them into label scores.
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
                          admission_s=0.0, prefill_pieces=0, splits=0, evict_retries=0)

    def run(self):
        """Answers for every document, in document order."""
        n = len(self.prefixes)
        t0 = time.perf_counter()
        tree = None
        if self.use_tree:
            tree = PrefixIndex.from_parts(
                [[p, *sufs] for p, sufs in zip(self.prefixes, self.suffixes)]
            ).tree(self.arena.page_tokens)
        adm = StageAdmission(self.prefixes, self.suffixes, self.arena, self.chunk_budget,
                             tree=tree)
        self._adm = adm
        self.stats["admission_s"] += time.perf_counter() - t0
        self._results = [None] * n
        self._inflight = deque()

        while not adm.done():
            t = time.perf_counter()
            groups = adm.next_chunk()
            self.stats["admission_s"] += time.perf_counter() - t
            if not groups:
                if self._inflight:
                    self._drain()
                    continue
                raise ArenaFullError("no document fits the free KV arena")
            self._run_part(groups)
        while self._inflight:
            self._drain()
        self.stats["borrowed_tokens"] += adm.borrowed_tokens
        self.stats["prefill_pieces"] += adm.pieces
        return self._results

    def _drain(self):
        """Read the oldest pack's answers and free its answered documents'
        pages. A document asked one question gets that answer; one asked
        several gets the list of them, in question order."""
        handle, docs = self._inflight.popleft()
        values = self.readout.result(handle)
        i = 0
        for d, count in docs:
            self._results[d] = values[i] if count == 1 else list(values[i:i + count])
            i += count
            self.arena.free_key(self._adm.keys[d])

    def _run_part(self, groups):
        """Pack and run groups, recovering from a full arena as the
        reference's _run_part does (stage_executor.py:1036-1062): read the
        answers in flight (their pages come free), then evict retained KV,
        then run the part as two halves (a parent before its readers: the
        groups keep their order)."""
        from quail_amd.chunk import pages_for_questions

        while True:
            try:
                chunk = self._pack(groups)
                break
            except ArenaFullError:
                if self._inflight:
                    self._drain()
                    continue
                need = pages_for_questions(self.arena, [g for _, g in groups])
                if self.arena.evict_retained(need):
                    self.stats["evict_retries"] += 1
                    continue
                if len(groups) < 2:
                    raise
                self.stats["splits"] += 1
                half = len(groups) // 2
                self._run_part(groups[:half])
                self._run_part(groups[half:])
                return
        self.stats["chunks"] += 1
        self.stats["fresh_tokens"] += chunk.tokens
        try:
            normed = self.pipeline.forward_chunk(chunk)
        finally:
            for key in chunk.temporary_keys:
                self.arena.free_key(key)
        # prefill pieces write KV and read no answer
        answered = [(d, len(g["suffixes"])) for d, g in groups if len(g["suffixes"])]
        per_answer = chunk.rows_per_answer
        if per_answer is not None and len(per_answer) and int(np.max(per_answer)) > 1:
            # several read rows per answer (label paths, read_all_rows)
            handle = self.readout.submit(normed, rows_per_answer=[int(r) for r in per_answer])
        else:
            handle = self.readout.submit(normed)
        self._inflight.append((handle, answered))
        if len(self._inflight) > 1:
            self._drain()

    def _pack(self, groups):
        t = time.perf_counter()
        engine = self.pipeline.engine
        specs = [g for _, g in groups]
        if self.attention_mode == "tree":
            # a borrowing document with one question reads its parent's
            # pages stacked with its siblings (stage_executor.py:772-774)
            specs = [dict(g, read_key=g.get("borrow_key") if g.get("start") else None,
                          single=len(g["suffixes"]) == 1) for g in specs]
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
