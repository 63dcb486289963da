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


def main():
    mods = load_reference()
    cpu_staging(mods["chunk"])
    out = {}
    for name in PACKS:
        out.update(vectors(mods, name))
    out.update(multi_question_vectors(mods))
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
