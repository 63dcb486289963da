"""The GPU loop of one stage: admission -> pack -> forward -> readout.

The reference's StageExecutor.run / _run_one
(quail/backends/quail/executor/stage_executor.py:66-89, 1115-1174,
1191-1344) for one AI.IF / AI.SCORE / AI.CLASSIFY stage: the host packs
pack N+1 while the GPU runs pack N; answers are read one pack late through
pinned buffers and events; temporary pages are freed after each forward
pass (stream order keeps later writers behind it); a document's pages are
freed once its answer is read, or when its last borrower is admitted.
"""

import time
from collections import deque

import numpy as np

from quail_amd.admission import StageAdmission
from quail_amd.chunk import ArenaFullError, InputStaging, pack_chunk, upload
from quail_amd.prefix import PrefixIndex


class StageRun:
    def __init__(self, pipeline, arena, readout, prefixes, suffixes, chunk_budget,
                 use_tree=True, staging=None, attention_mode="unified"):
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
                          admission_s=0.0)

    def run(self):
        """Answers for every document, in document order."""
        n = len(self.prefixes)
        t0 = time.perf_counter()
        tree = None
        if self.use_tree:
            prompts = [np.concatenate([np.asarray(p, dtype=np.int64)] +
                                      [np.asarray(suf, dtype=np.int64).reshape(-1)
                                       for suf in sufs])
                       for p, sufs in zip(self.prefixes, self.suffixes)]
            tree = PrefixIndex(prompts).tree(self.arena.page_tokens)
        adm = StageAdmission(self.prefixes, self.suffixes, self.arena, self.chunk_budget,
                             tree=tree)
        self.stats["admission_s"] += time.perf_counter() - t0
        results = [None] * n
        inflight = deque()

        def drain():
            handle, docs = inflight.popleft()
            values = self.readout.result(handle)
            for i, d in enumerate(docs):
                results[d] = values[i]
                self.arena.free_key(adm.keys[d])

        while not adm.done():
            t = time.perf_counter()
            groups = adm.next_chunk()
            self.stats["admission_s"] += time.perf_counter() - t
            if not groups:
                if inflight:
                    drain()
                    continue
                raise ArenaFullError("no document fits the free KV arena")
            t = time.perf_counter()
            engine = self.pipeline.engine
            specs = [g for _, g in groups]
            if self.attention_mode == "tree":
                # a borrowing document with one question reads its parent's
                # pages stacked with its siblings (stage_executor.py:772-774)
                specs = [dict(g, read_key=g.get("borrow_key") if g.get("start") else None,
                              single=len(g["suffixes"]) == 1) for g in specs]
            chunk = pack_chunk(self.arena, specs, attention_mode=self.attention_mode,
                               attention_heads=(engine.num_q_heads, engine.num_kv_heads,
                                                engine.head_dim))
            upload(chunk, self.staging)
            self.stats["pack_s"] += time.perf_counter() - t
            self.stats["chunks"] += 1
            self.stats["fresh_tokens"] += chunk.tokens
            try:
                normed = self.pipeline.forward_chunk(chunk)
            finally:
                for key in chunk.temporary_keys:
                    self.arena.free_key(key)
            inflight.append((self.readout.submit(normed), [d for d, _ in groups]))
            if len(inflight) > 1:
                drain()
        while inflight:
            drain()
        self.stats["borrowed_tokens"] += adm.borrowing.borrowed_tokens
        return results
