"""Write tests/golden/pack_vectors.npz from the reference's own packing code.

Run in the build container only (it reads the reference sources under
/root/reference; nothing it loads travels anywhere):

    python tests/golden/make_pack_vectors.py

It loads, by file path, the reference's pure-numpy packing modules
(quail/backends/quail/executor/admission.py, pages.py, arena.py, chunk.py,
with attention.py, gdn.py and quail/progress.py they import), with stub
parent packages so that quail/__init__.py (which imports the Rust module,
not built here) never runs, and a stub quail.common.budgets carrying the
one constant gdn.py reads (CHECKPOINT_PASS_QUESTIONS = 1024,
crates/quail-planner/src/cost/budgets.rs:20).

Inputs are the benchmark corpora (quail_amd.workload.make_workload: config
1 "tiny" seed 0 and config 3 "qwen3-4b" seed 0), each document a prefix
(its prompt less the last token) asked one one-token question, and the
prefix tree of the prompts (oracle.prefix_ref, pinned by the planner's own
known answers). The arena is large enough (20,000 pages) that free pages
never bind, so the packs are set by the pack budget and the tree alone.

Outputs, for the first pack of config 1 and the first three of config 3:
  * JoinAdmission.next_chunk's pack composition (admission.py:702-866):
    the documents of each pack in order and, for each, the parent it
    borrows from and how many tokens (Borrowing.chosen);
  * the page table KVArena.activate gives each document
    (arena.py:522-563, pages.py), activated in pack order with its whole
    capacity and its borrow; every answer is reported (admission.py:872)
    before the next pack is composed, and no document is released;
  * pack_chunk(attention_mode="unified")'s layout of each pack
    (chunk.py:505-1160): input ids, positions, final rows, cu_a, and the
    unified pools cu_q, used, table, src, dst, tail_src, tail_dst;
  * the same layout of one pack of documents asked several questions each
    (multi_question_vectors: temporary question pages and tail copies).
"""

import importlib.util
import sys
import types
from pathlib import Path

import numpy as np

REF = Path("/root/reference")
HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
OUT = HERE / "pack_vectors.npz"
BIG_ARENA = 20000
PAGE = 16
PACKS = {"tiny": 1, "qwen3-4b": 3}


def load_reference():
    """The reference packing modules, loaded by file path."""
    packages = {
        "quail": REF / "quail",
        "quail.common": REF / "quail" / "common",
        "quail.backends": REF / "quail" / "backends",
        "quail.backends.quail": REF / "quail" / "backends" / "quail",
        "quail.backends.quail.executor": REF / "quail" / "backends" / "quail" / "executor",
    }
    for name, path in packages.items():
        mod = types.ModuleType(name)
        mod.__path__ = [str(path)]
        sys.modules[name] = mod
    budgets = types.ModuleType("quail.common.budgets")
    budgets.CHECKPOINT_PASS_QUESTIONS = 1024
    sys.modules["quail.common.budgets"] = budgets

    def load(name, path):
        spec = importlib.util.spec_from_file_location(name, path)
        mod = importlib.util.module_from_spec(spec)
        sys.modules[name] = mod
        spec.loader.exec_module(mod)
        return mod

    ex = REF / "quail" / "backends" / "quail" / "executor"
    load("quail.progress", REF / "quail" / "progress.py")
    mods = {}
    for name in ("pages", "attention", "gdn", "arena", "chunk", "admission"):
        mods[name] = load(f"quail.backends.quail.executor.{name}", ex / f"{name}.py")
    return mods


def cpu_staging(chunk_mod):
    """pack_chunk's staging on plain CPU tensors (as the reference's own
    tests/helpers/fakes.py:cpu_staging does)."""
    import torch

    def staged(torch_, data, dtype, pinned=True):
        if isinstance(data, np.ndarray) or torch.is_tensor(data):
            return torch.as_tensor(data, dtype=dtype)
        return torch.tensor(data, dtype=dtype)

    def token_parts(torch_, sequences, total, pinned=True, staging=None):
        ids = [int(t) for seq in sequences for part in chunk_mod._token_parts(seq)
               for t in part]
        assert len(ids) == total
        return torch.tensor(ids, dtype=torch.int64)

    chunk_mod._staged = staged
    chunk_mod._staged_token_parts = token_parts


def arr(x, dtype=np.int64):
    import torch
    if x is None:
        return np.empty(0, dtype=dtype)
    if torch.is_tensor(x):
        x = x.cpu().numpy()
    return np.asarray(x).astype(dtype).reshape(-1)


def vectors(mods, name):
    import torch

    sys.path.insert(0, str(ROOT))
    from oracle.prefix_ref import PrefixIndex
    from quail_amd.workload import make_workload

    wl = make_workload(name, seed=0)
    prompts = [np.asarray(p, dtype=np.int64) for p in wl.prompts]
    prefixes = [p[:-1] for p in prompts]
    suffixes = [p[-1:] for p in prompts]
    order, parents, tree_shared = PrefixIndex([p.tolist() for p in prompts]).tree(PAGE)
    tree = types.SimpleNamespace(order=order, parent=parents, shared=tree_shared)
    keys = [("doc", d) for d in range(len(prompts))]
    arena = mods["arena"].KVArena(num_layers=1, num_pages=BIG_ARENA, page_tokens=PAGE,
                                  num_kv_heads=1, d_head=2, dtype=torch.float32, device="cpu")

    def can_borrow(d, lender, same_chunk):
        # the stage's borrow check (stage_executor.py:99-105) on an arena
        # without a sliding pool: a lender admitted in this pack and not
        # yet allocated can always serve
        if not same_chunk or arena.is_resident(keys[lender]):
            return arena.can_borrow(keys[lender], tree_shared[d])
        return True

    adm = mods["admission"].JoinAdmission(
        [len(p) for p in prefixes], [[1]], wl.chunk_budget, BIG_ARENA, PAGE, tree=tree,
        can_borrow=can_borrow)
    out = {}
    for pack in range(PACKS[name]):
        groups = adm.next_chunk(arena.free_pages)
        assert groups, f"{name}: pack {pack} is empty"
        docs, lenders, lent, specs = [], [], [], []
        for anchor, stage, start, end, carried in groups:
            assert (stage, start, end) == (0, 0, 1) and carried
            parent, shared = adm.borrowing.chosen.get(anchor, (None, 0))
            docs.append(anchor)
            lenders.append(-1 if parent is None else parent)
            lent.append(shared)
            f = len(prefixes[anchor])
            borrow = None if parent is None else (keys[parent], shared)
            pages = arena.activate(keys[anchor], f, capacity_tokens=f + 1, borrow=borrow)
            assert pages is not None
            specs.append(dict(key=keys[anchor], prefix=prefixes[anchor][shared:], f=f,
                              start=shared,
                              suffixes=mods["chunk"].Suffixes.of([suffixes[anchor].tolist()])))
        chunk = mods["chunk"].pack_chunk(torch, arena, specs, attention_mode="unified")
        u = chunk.meta["unified"]
        p = f"{name}/{pack}/"
        out[p + "docs"] = np.asarray(docs, dtype=np.int64)
        out[p + "lenders"] = np.asarray(lenders, dtype=np.int64)
        out[p + "lent"] = np.asarray(lent, dtype=np.int64)
        tables = [arena.accounting.table_pages(keys[d]) for d in docs]
        out[p + "table_lens"] = np.asarray([len(t) for t in tables], dtype=np.int64)
        out[p + "tables"] = np.asarray([x for t in tables for x in t], dtype=np.int64)
        out[p + "input_ids"] = arr(chunk.input_ids)
        out[p + "positions"] = arr(chunk.positions)
        out[p + "final_indices"] = arr(chunk.final_indices)
        out[p + "cu_a"] = arr(chunk.meta["cu_a"])
        for field in ("cu_q", "used", "src", "dst", "tail_src", "tail_dst"):
            out[p + field] = arr(u.get(field))
        table = u["table"]
        table = table.cpu().numpy() if torch.is_tensor(table) else np.asarray(table)
        out[p + "table_shape"] = np.asarray(table.shape, dtype=np.int64)
        out[p + "table"] = table.astype(np.int64).reshape(-1)
        # every answer arrives before the next pack is composed; no document
        # is released, so page ids are never reused
        for d in docs:
            adm.report(d, 0, 0, 1, [True])
        print(f"{name} pack {pack}: {len(docs)} documents, {chunk.tokens} rows, "
              f"{sum(lent)} borrowed tokens", flush=True)
    return out


def multi_question_vectors(mods):
    """pack_chunk of documents asked several questions each: the tiny
    corpus's 16 prompts, whole, each document activated for its prompt only
    (no room for questions: every question takes temporary pages, its first
    rows copied from the document's partial last page), documents 1..15
    borrowing document 0's first page when they share it. Questions are
    1-3 questions of 1-4 tokens drawn with numpy seed 5."""
    import torch

    sys.path.insert(0, str(ROOT))
    from quail_amd.workload import make_workload

    wl = make_workload("tiny", seed=0)
    prompts = [np.asarray(p, dtype=np.int64) for p in wl.prompts]
    rng = np.random.default_rng(5)
    questions = [[rng.integers(0, 1000, int(rng.integers(1, 5))).tolist()
                  for _ in range(int(rng.integers(1, 4)))] for _ in prompts]
    arena = mods["arena"].KVArena(num_layers=1, num_pages=4000, page_tokens=PAGE,
                                  num_kv_heads=1, d_head=2, dtype=torch.float32, device="cpu")
    specs = []
    lent = []
    for d, prompt in enumerate(prompts):
        key = ("doc", d)
        same = 0
        if d:
            n = min(len(prompt), len(prompts[0]))
            eq = np.flatnonzero(prompt[:n] != prompts[0][:n])
            same = (n if eq.size == 0 else int(eq[0])) // PAGE * PAGE
            same = min(same, (len(prompt) - 1) // PAGE * PAGE)
        borrow = (("doc", 0), same) if same else None
        assert arena.activate(key, len(prompt), borrow=borrow) is not None
        lent.append(same)
        specs.append(dict(key=key, prefix=prompt[same:], f=len(prompt), start=same,
                          suffixes=mods["chunk"].Suffixes.of(questions[d])))
    chunk = mods["chunk"].pack_chunk(torch, arena, specs, attention_mode="unified")
    u = chunk.meta["unified"]
    p = "multi/"
    out = {p + "lent": np.asarray(lent, dtype=np.int64),
           p + "question_lens": np.asarray([len(q) for qs in questions for q in qs], np.int64),
           p + "questions_per_doc": np.asarray([len(qs) for qs in questions], np.int64),
           p + "questions": np.asarray([t for qs in questions for q in qs for t in q], np.int64),
           p + "input_ids": arr(chunk.input_ids), p + "positions": arr(chunk.positions),
           p + "final_indices": arr(chunk.final_indices), p + "cu_a": arr(chunk.meta["cu_a"])}
    for field in ("cu_q", "used", "src", "dst", "tail_src", "tail_dst"):
        out[p + field] = arr(u.get(field))
    table = u["table"]
    table = table.cpu().numpy() if torch.is_tensor(table) else np.asarray(table)
    out[p + "table_shape"] = np.asarray(table.shape, dtype=np.int64)
    out[p + "table"] = table.astype(np.int64).reshape(-1)
    print(f"multi: {sum(len(q) for q in questions)} questions, {len(out[p + 'tail_src'])} "
          f"tail copies", flush=True)
    return out


class ReferenceStage:
    """The reference's one-stage driver loop over its own JoinAdmission,
    KVArena and pack_chunk, with a forward pass that computes nothing and a
    readout that answers every question True: StageExecutor.run
    (stage_executor.py:1191-1277) for one AI.IF stage, paged, unified
    attention, no decoder, no frames, finished documents freed (on_settled
    None, _settle :894-901). Each step below names the reference lines it
    follows. Records, per forward pass, the groups, the chunked prefill
    pieces, the borrows chosen, the page tables of the keys packed and the
    free pages, and the recoveries (evictions, evict-retries, splits)."""

    def __init__(self, mods, prefixes, questions, budget, arena, tree, retained=()):
        import torch
        self.mods, self.torch = mods, torch
        self.prefixes = prefixes
        self.questions = questions          # the stage's shared question list
        self.keys = [("doc", d) for d in range(len(prefixes))]
        self.arena = arena
        single = len(questions) == 1
        # a single suffix occupies document pages on the unified path
        # (stage_executor.py:392-399)
        self.extra = max(len(q) for q in questions) if single else 0
        self.single = single
        self.suffixes = mods["chunk"].Suffixes.of(questions)
        adm = mods["admission"]
        self.sched = adm.JoinAdmission(
            [len(p) for p in prefixes], [[len(q) for q in questions]], budget,
            arena.num_pages, arena.page_tokens, frame_tokens=[0],
            temporary_suffix_pages=True, page_cost=arena.page_cost, tree=tree,
            frame_writes=[False], extra_tokens=self.extra, reserve=self._reserve,
            chunked_prefill=True)
        b = self.borrowing = self.sched.borrowing
        b.can_borrow = self._borrow_check
        self.borrowers = b.borrowers()
        self.lowest = {}
        for d, parent in enumerate(b.tree_parent):
            if parent is not None:
                sh = b.tree_shared[d]
                self.lowest[parent] = min(self.lowest.get(parent, sh), sh)
        self.held = [self.keys[a] for a, n in enumerate(self.borrowers) if n]
        self.held_parents, self.reserved_parents = set(), {}
        self.outstanding = []
        self.passes = []
        self.events = []            # (kind, pass index, detail)
        self.reported = []          # per pass report: the documents settled

    def _borrow_check(self, document, parent, same_chunk):
        # borrow_check (stage_executor.py:93-107)
        shared = self.borrowing.tree_shared[document]
        if not same_chunk or self.arena.is_resident(self.keys[parent]):
            return self.arena.can_borrow(self.keys[parent], shared)
        return self.arena.origin(self.borrowing.shared(parent)) <= self.arena.origin(shared)

    def _reserve(self, anchor, borrow, rows):
        # _reserve / _reserved (stage_executor.py:584-620)
        key = self.keys[anchor]
        prefix = len(self.prefixes[anchor])
        parent, shared = (None, 0) if borrow is None else borrow
        borrowed = (self.keys[parent], shared) if shared else None
        evicted = self.arena.evicted_keys
        ok = self.arena.reserve(key, prefix, capacity_tokens=prefix + self.extra,
                                borrow=borrowed, extension=False, share_points=())
        if self.arena.evicted_keys != evicted:
            self.events.append(("reserve_evicted", len(self.passes),
                                self.arena.evicted_keys - evicted))
        if not ok:
            return False
        if parent is not None:
            self.arena.read_state((self.keys[parent],))
            self.reserved_parents[anchor] = self.keys[parent]
        if anchor not in self.held_parents and self.borrowers[anchor]:
            self.held_parents.add(anchor)
            self.arena.hold(key, self.borrowers[anchor])
            self.arena.keep_window(key, self.lowest[anchor])
        return True

    def _specs(self, groups, prefills):
        # _build (stage_executor.py:705-892), the paths a one-stage run takes
        Suffixes = self.mods["chunk"].Suffixes
        specs = []
        for a, j, start, end, carried in groups:
            key = self.keys[a]
            f = len(self.prefixes[a])
            parent, shared = ((self.borrowing.parent(a), self.borrowing.shared(a))
                              if carried else (None, 0))
            prefix = None
            if carried:
                prefix = self.prefixes[a][shared:] if shared else self.prefixes[a]
            sufs = Suffixes.of([self.questions[i] for i in range(start, end)])
            read_key = self.keys[parent] if shared and self.single else None
            carry = {}
            if prefix is not None:
                carry = dict(borrow_key=self.keys[parent] if shared else None,
                             share_points=())
            specs.append(dict(key=key, prefix=prefix, start=shared, read_key=read_key, f=f,
                              suffixes=sufs, read_all_rows=False, write_suffix_tokens=0,
                              single=self.single and end - start == 1, paths=None, **carry))
        for a, start, end in prefills:
            key = self.keys[a]
            parent, shared = self.borrowing.parent(a), self.borrowing.shared(a)
            specs.append(dict(
                key=key, prefix=self.prefixes[a][start:end], start=start, f=end,
                suffixes=Suffixes(np.empty(0, dtype=np.int64), []),
                borrow_key=(self.keys[parent] if start == shared and shared
                            else key if start else None),
                share_points=()))
        return specs

    def _run_one(self, groups, prefills):
        # _run_one (stage_executor.py:1115-1174): pack, forward (nothing),
        # free temporaries, report the earlier passes, then queue this one
        chunk = self.mods["chunk"].pack_chunk(self.torch, self.arena,
                                              self._specs(groups, prefills),
                                              attention_mode="unified")
        for key in chunk.temporary_keys:
            self.arena.free_key(key)
        keys = [self.keys[a] for a, *_ in groups] + [self.keys[a] for a, _, _ in prefills]
        self.passes.append(dict(
            groups=[(a, start, end, int(carried)) for a, _, start, end, carried in groups],
            prefills=list(prefills), rows=int(chunk.tokens),
            tables=[list(self.arena.accounting.table_pages(k)) for k in keys],
            free_pages=int(self.arena.free_pages)))
        while self.outstanding:
            self._report_next()
        self.outstanding.append(list(groups))

    def _run_part(self, part, prefills=()):
        # _run_part (stage_executor.py:1036-1062)
        try:
            self._run_one(part, prefills)
        except self.mods["chunk"].ArenaFullError:
            rows = sum((len(self.prefixes[a]) if carried else 0)
                       + sum(len(self.questions[i]) for i in range(start, end))
                       for a, _, start, end, carried in part)
            need = self.arena.page_cost(rows)
            if self.arena.evict_retained(need):
                self.events.append(("evict_retry", len(self.passes), len(part)))
                self._run_part(part, prefills)
                return
            if len(part) < 2:
                raise
            self.events.append(("split", len(self.passes), len(part)))
            half = len(part) // 2
            self._run_part(part[:half], prefills)
            self._run_part(part[half:])

    def _report_next(self):
        # _report_next / _report / _record (stage_executor.py:911-1000):
        # every question answered True; a finished document's pages go free
        groups = self.outstanding.pop(0)
        settled = []
        for a, j, start, end, _ in groups:
            result = self.sched.report(a, j, start, end, [True] * (end - start))
            for settlement in result.settlements:
                settled.append(settlement.anchor)
                key = self.keys[settlement.anchor]
                if self.arena.is_resident(key):
                    self.arena.free_key(key)
        self.reported.append((len(self.passes), settled))

    def _prefilled(self, prefills):
        # _prefilled (stage_executor.py:1176-1189)
        for a, start, _ in prefills:
            if start != self.borrowing.shared(a):
                continue
            parent = self.borrowing.tree_parent[a]
            if parent is not None:
                self.arena.release(self.keys[parent])
            if a in self.reserved_parents:
                self.arena.done_reading((self.reserved_parents.pop(a),))

    def _evict(self, pages):
        keys = self.arena.evict_retained(pages)
        if keys:
            self.events.append(("evict", len(self.passes), len(keys)))
        return keys

    def run(self):
        # run (stage_executor.py:1191-1277)
        sched, arena = self.sched, self.arena
        while True:
            for settlement in sched.take_settled():
                raise AssertionError("a document with nothing to ask")
            if sched.done():
                break
            if len(self.outstanding) > 1:
                self._report_next()
            if sched.blocked_pages:
                self._evict(sched.blocked_pages)
            groups = sched.next_chunk(arena.free_pages, room=sched.chunk_budget)
            prefills = sched.take_prefills()
            if not groups and prefills:
                self._run_part([], prefills)
                self._prefilled(prefills)
                continue
            if not groups:
                if sched.done():
                    continue
                if self.outstanding:
                    self._report_next()
                    continue
                if sched.blocked_pages and self._evict(sched.blocked_pages):
                    continue
                if arena.drop_holds(self.held):
                    self.events.append(("drop_holds", len(self.passes), 0))
                    continue
                raise AssertionError("nothing buildable and nothing in flight")
            self._run_part(groups, prefills)
            self._prefilled(prefills)
            for a, _, start, _, carried in groups:
                parent = self.borrowing.tree_parent[a]
                if carried and start == 0 and parent is not None:
                    arena.release(self.keys[parent])
                if a in self.reserved_parents:
                    arena.done_reading((self.reserved_parents.pop(a),))
        while self.outstanding:
            self._report_next()
        arena.drop_holds(self.held)
        return self


# Stage runs with binding pages and chunked prefill (name -> corpus, budget,
# arena pages, the stage's questions, retained keys filled before the run)
STAGE_RUNS = {
    # the tiny corpus, a pack budget below its longest documents (pieces)
    # and an arena of 40 pages (documents wait for answered ones' pages)
    "pieces": dict(corpus=("tiny", 0), budget=96, pages=40, questions=None, retained=()),
    # two questions per document (temporary question pages) and an arena
    # a third full of retained KV of an earlier operator (evictions)
    "evict": dict(corpus=("tiny", 1), budget=160, pages=36, questions=[[7, 8], [9, 10, 11]],
                  retained=(40, 60, 30)),
    # the Qwen3-4B AI.IF benchmark with the bench's 3,136-page arena
    "qwen3-4b": dict(corpus=("qwen3-4b", 0), budget=None, pages=3136, questions=None,
                     retained=()),
}


def stage_run_vectors(mods, name):
    import torch

    sys.path.insert(0, str(ROOT))
    from oracle.prefix_ref import PrefixIndex
    from quail_amd.workload import make_workload

    spec = STAGE_RUNS[name]
    wl = make_workload(*spec["corpus"])
    prompts = [np.asarray(p, dtype=np.int64) for p in wl.prompts]
    if spec["questions"] is None:
        prefixes = [p[:-1] for p in prompts]
        questions = [[0]]              # one 1-token question (its id does not matter)
        tree_docs = [p.tolist() for p in prompts]
    else:
        prefixes = prompts
        questions = spec["questions"]
        tree_docs = [p.tolist() + [t for q in questions for t in q] for p in prompts]
    budget = spec["budget"] or wl.chunk_budget
    order, parents, tree_shared = PrefixIndex(tree_docs).tree(PAGE)
    tree = types.SimpleNamespace(order=order, parent=parents, shared=tree_shared)
    arena = mods["arena"].KVArena(num_layers=1, num_pages=spec["pages"], page_tokens=PAGE,
                                  num_kv_heads=1, d_head=2, dtype=torch.float32, device="cpu")
    for i, tokens in enumerate(spec["retained"]):
        key = ("retained", i)
        assert arena.alloc(key, tokens) is not None
        arena.retain(key, tokens)
    run = ReferenceStage(mods, prefixes, questions, budget, arena, tree).run()
    p = f"stage/{name}/"
    out = {p + "budget": np.asarray([budget], np.int64),
           p + "pages": np.asarray([spec["pages"]], np.int64),
           p + "question_lens": np.asarray([len(q) for q in questions], np.int64),
           p + "retained": np.asarray(spec["retained"], np.int64)}
    g, pf, tb = [], [], []
    for i, ps in enumerate(run.passes):
        g += [(i, *x) for x in ps["groups"]]
        pf += [(i, *x) for x in ps["prefills"]]
        tb += [(i, len(t)) for t in ps["tables"]]
    out[p + "groups"] = np.asarray(g, np.int64).reshape(-1, 5)
    out[p + "prefills"] = np.asarray(pf, np.int64).reshape(-1, 4)
    out[p + "rows"] = np.asarray([ps["rows"] for ps in run.passes], np.int64)
    out[p + "free_pages"] = np.asarray([ps["free_pages"] for ps in run.passes], np.int64)
    out[p + "table_lens"] = np.asarray(tb, np.int64).reshape(-1, 2)
    out[p + "tables"] = np.asarray([x for ps in run.passes for t in ps["tables"] for x in t],
                                   np.int64)
    chosen = sorted(run.borrowing.chosen.items())
    out[p + "borrows"] = np.asarray([(d, par, sh) for d, (par, sh) in chosen],
                                    np.int64).reshape(-1, 3)
    kinds = {"evict": 0, "evict_retry": 1, "split": 2, "drop_holds": 3, "reserve_evicted": 4}
    out[p + "events"] = np.asarray([(kinds[k], i, n) for k, i, n in run.events],
                                   np.int64).reshape(-1, 3)
    out[p + "reported"] = np.asarray([(i, a) for i, docs in run.reported for a in docs],
                                     np.int64).reshape(-1, 2)
    counts = {k: sum(1 for e in run.events if e[0] == k) for k in kinds}
    print(f"stage {name}: {len(run.passes)} passes, {len(pf)} prefill pieces, "
          f"{len(chosen)} borrows, events {counts}", flush=True)
    return out


def main():
    mods = load_reference()
    cpu_staging(mods["chunk"])
    out = {}
    for name in PACKS:
        out.update(vectors(mods, name))
    out.update(multi_question_vectors(mods))
    for name in STAGE_RUNS:
        out.update(stage_run_vectors(mods, name))
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
