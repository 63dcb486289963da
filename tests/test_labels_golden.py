"""The label trie of trie-scored AI.CLASSIFY against the reference's own code.

tests/golden/make_label_vectors.py ran the reference's label_trie,
read_nodes, fed_nodes (quail/labels.py) and trie_paths, path_reads,
tree_scores, letter_scores (quail/execution/labels.py:47-60, 151-260) on 47
label sets: the two of the reference's planner tests, 40 seeded random ones
over a five-token vocabulary (shared prefixes, labels that end where others
continue, repeated tokens), three sets of one-token labels, and a label
whose extension takes all (or all but 1e-6) of its probability. Here
quail_amd.labels must give the same trie, read and fed nodes, paths (nodes,
start, gathers) and read rows exactly, and the same scores to 1e-12 (minus
infinity where the reference gives it); the oracle's restatement
(oracle/labels_ref.py, which restates the trie and paths) the same trie,
nodes and paths.
"""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import labels_ref
from quail_amd import labels as qlabels

GOLDEN = json.loads((Path(__file__).parent / "golden" / "label_vectors.json").read_text())
CASES = GOLDEN["cases"]
IMPLS = {"quail_amd": qlabels, "oracle": labels_ref}


def _t(x):
    return tuple(int(v) for v in x)


def _paths(raw):
    return [([_t(n) for n in nodes], start, [(p, c) for p, c in gathers])
            for nodes, start, gathers in raw]


def _plain(paths):
    return [([_t(n) for n in nodes], int(start), [(int(p), int(c)) for p, c in gathers])
            for nodes, start, gathers in paths]


@pytest.mark.parametrize("impl", sorted(IMPLS))
@pytest.mark.parametrize("index", range(len(CASES)))
def test_label_trie_paths_and_scores_equal_the_reference(impl, index):
    mod = IMPLS[impl]
    case = CASES[index]
    labels = [_t(ids) for ids in case["labels"]]
    trie = mod.label_trie(labels)
    assert sorted([list(k), list(v)] for k, v in trie.items()) == case["trie"]
    read = mod.read_nodes(labels)
    assert sorted(list(n) for n in read) == case["read"]
    assert sorted(list(n) for n in mod.fed_nodes(read)) == case["fed"]
    for key, r in (("all", None), ("read", read)):
        if f"paths_{key}" not in case:
            continue
        paths = mod.trie_paths(labels, r)
        assert _plain(paths) == _paths(case[f"paths_{key}"]), key
        assert [bool(x) for x in mod.path_reads(paths, r)] == case[f"reads_{key}"], key
    if not hasattr(mod, "tree_scores"):
        return    # the oracle restates the trie and paths only
    paths = mod.trie_paths(labels, read)
    scores = mod.tree_scores(labels, paths, case["targets"], np.asarray(case["logprobs"]), read)
    want = np.array([-np.inf if x is None else x for x in case["tree_scores"]])
    assert np.array_equal(np.isneginf(scores), np.isneginf(want))
    finite = np.isfinite(want)
    np.testing.assert_allclose(scores[finite], want[finite], rtol=0, atol=1e-12)
    if "letter_scores" in case:
        got = mod.letter_scores(labels, case["targets"], np.asarray(case["letter_row"]))
        np.testing.assert_allclose(got, case["letter_scores"], rtol=0, atol=0)


def test_the_vectors_cover_what_they_are_meant_to():
    """Labels that extend others, several paths with gathers, a minus
    infinity score, one-token letter sets."""
    assert any(len(c["paths_read"]) >= 3 for c in CASES)
    assert any(g for c in CASES for _, _, gs in c["paths_read"] for g in gs)
    assert any(None in c["tree_scores"] for c in CASES)
    assert sum("letter_scores" in c for c in CASES) == 3
