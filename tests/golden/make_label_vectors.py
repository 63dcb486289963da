"""Write tests/golden/label_vectors.json from the reference's own label trie code.

Run in the build container only (it reads the reference sources under
/root/reference; nothing it loads travels anywhere):

    python tests/golden/make_label_vectors.py

It loads, by file path, quail/labels.py (label_trie, read_nodes, fed_nodes;
dataclasses only) and quail/execution/labels.py (trie_paths, path_reads,
tree_scores, letter_scores; numpy), with stub parent packages so that
quail/__init__.py (which imports the Rust module, not built here) never
runs.

Inputs: seeded random label sets over a small vocabulary (so that labels
share prefixes, end where others continue, and repeat tokens), the two label
sets of the reference's planner tests (tests/planner/test_classify_cost.py:
16, 138-141), and sets of one-token labels. For each: the trie, the read
nodes, the paths (nodes, start, gathers) with every node read and with the
read nodes, which path rows are read, and tree_scores over seeded random
log-probability rows (some sets scored with log-softmax rows over exactly
the labels' tokens, some over extra target tokens too); letter_scores for
the one-token sets; and a label whose extension takes all (or nearly all) of
its probability.
"""

import importlib.util
import json
import sys
import types
from pathlib import Path

import numpy as np

REF = Path("/root/reference")
OUT = Path(__file__).resolve().parent / "label_vectors.json"


def load_reference():
    for name, path in (("quail", REF / "quail"), ("quail.execution", REF / "quail" / "execution")):
        pkg = types.ModuleType(name)
        pkg.__path__ = [str(path)]
        sys.modules[name] = pkg
    mods = {}
    for name, path in (("quail.labels", REF / "quail" / "labels.py"),
                       ("quail.execution.labels", REF / "quail" / "execution" / "labels.py")):
        spec = importlib.util.spec_from_file_location(name, path)
        mod = importlib.util.module_from_spec(spec)
        sys.modules[name] = mod
        spec.loader.exec_module(mod)
        mods[name] = mod
    return mods["quail.labels"], mods["quail.execution.labels"]


def label_sets():
    rng = np.random.default_rng(2024)
    sets = [[(10,), (20, 21, 22), (20, 25, 26, 27, 28), (30, 31, 32), (30, 31, 33)],
            [(10,), (20, 21), (20, 22), (30, 31, 32), (40,), (40, 41)]]
    for _ in range(40):
        n = int(rng.integers(2, 10))
        labels = []
        while len(labels) < n:
            ids = tuple(int(t) for t in rng.integers(1, 6, int(rng.integers(1, 6))))
            if ids not in labels:
                labels.append(ids)
        sets.append(labels)
    for n in (2, 5, 9):
        sets.append([(int(t),) for t in rng.choice(np.arange(1, 50), n, replace=False)])
    return sets


def _node(n):
    return [int(t) for t in n]


def main():
    base, ex = load_reference()
    rng = np.random.default_rng(7)
    cases = []
    for labels in label_sets():
        trie = base.label_trie(labels)
        read = base.read_nodes(labels)
        case = dict(labels=[_node(ids) for ids in labels],
                    trie=sorted([_node(k), [int(t) for t in v]] for k, v in trie.items()),
                    read=sorted(_node(n) for n in read),
                    fed=sorted(_node(n) for n in base.fed_nodes(read)))
        for key, r in (("all", None), ("read", read)):
            paths = ex.trie_paths(labels, r)
            case[f"paths_{key}"] = [[[_node(n) for n in nodes], int(start),
                                     [[int(p), int(c)] for p, c in gathers]]
                                    for nodes, start, gathers in paths]
            case[f"reads_{key}"] = [bool(x) for x in ex.path_reads(paths, r)]
        tokens = sorted({t for ids in labels for t in ids})
        extra = bool(rng.integers(0, 2))
        targets = tokens + ([int(t) for t in rng.choice(np.arange(60, 90), 3, replace=False)]
                            if extra else [])
        paths = ex.trie_paths(labels, read)
        rows = sum(ex.path_reads(paths, read))
        logits = rng.normal(0.0, 2.0, (rows, len(targets)))
        logprobs = logits - np.log(np.exp(logits).sum(axis=1, keepdims=True))
        case["targets"] = targets
        case["logprobs"] = logprobs.tolist()
        scores = ex.tree_scores(labels, paths, targets, logprobs, read)
        case["tree_scores"] = [float(x) if np.isfinite(x) else None for x in scores]
        if all(len(ids) == 1 for ids in labels):
            row = rng.normal(0.0, 2.0, len(targets))
            case["letter_row"] = row.tolist()
            case["letter_scores"] = [float(x) for x in ex.letter_scores(labels, targets, row)]
        cases.append(case)
    # a label whose extensions take all of its probability (log prob 0 for
    # the extending token at its node) scores minus infinity, and one whose
    # extension takes nearly all of it keeps the small rest
    for lp_ext in (0.0, -1e-6):
        labels = [(1,), (1, 2), (3,)]
        read = base.read_nodes(labels)
        paths = ex.trie_paths(labels, read)
        targets = [1, 2, 3]
        logprobs = np.array([[-0.5, -9.0, -1.2], [-30.0, lp_ext, -30.0]])
        scores = ex.tree_scores(labels, paths, targets, logprobs, read)
        cases.append(dict(labels=[_node(ids) for ids in labels],
                          trie=sorted([_node(k), [int(t) for t in v]]
                                      for k, v in base.label_trie(labels).items()),
                          read=sorted(_node(n) for n in read),
                          fed=sorted(_node(n) for n in base.fed_nodes(read)),
                          paths_read=[[[_node(n) for n in nodes], int(start),
                                       [[int(p), int(c)] for p, c in gathers]]
                                      for nodes, start, gathers in paths],
                          reads_read=[bool(x) for x in ex.path_reads(paths, read)],
                          targets=targets, logprobs=logprobs.tolist(),
                          tree_scores=[float(x) if np.isfinite(x) else None for x in scores]))
    OUT.write_text(json.dumps(dict(cases=cases), separators=(",", ":")))
    print(f"wrote {OUT} ({len(cases)} label sets)")


if __name__ == "__main__":
    main()
