"""quail_amd.labels: the label trie of trie-scored AI.CLASSIFY.

The trie, read nodes and path split equal the oracle's restatement
(oracle/labels_ref.py, itself pinned by the reference's known answers in
tests/test_pack_tree.py) on the reference's label sets and on seeded random
ones. tree_scores (quail/execution/labels.py:216-260) is pinned by what the
mathematics fixes: one-token labels score their token's log probability at
the root; a label that others extend keeps its probability minus theirs
(hand-computed); when every read row is a log-softmax over the targets and
the root's targets are the labels' first tokens, the label probabilities
add up to one; extensions that take all of a label's mass leave it -inf.
"""

import math

import numpy as np
import pytest

from oracle import labels_ref
from quail_amd import labels as qlabels

LABELS = ((10,), (20, 21, 22), (20, 25, 26, 27, 28), (30, 31, 32), (30, 31, 33))
SPLIT = ((10,), (20, 21), (20, 22), (30, 31, 32), (40,), (40, 41))


def _random_labels(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 9))
    return [tuple(rng.integers(1, 5, int(rng.integers(1, 6))).tolist()) for _ in range(n)]


def test_known_answers():
    # tests/planner/test_classify_cost.py:16, 106-108: LABELS feeds a 4-token
    # suffix and reads 3 of its rows; :138-142: where SPLIT's labels split
    read = qlabels.read_nodes(LABELS)
    paths = qlabels.trie_paths(LABELS, read)
    assert len(qlabels.path_tokens(paths, 7)) == 4 and sum(qlabels.path_reads(paths, read)) == 3
    assert read == {(), (20,), (30, 31)}
    assert qlabels.read_nodes(SPLIT) == {(), (20,), (40,)}
    with pytest.raises(ValueError):
        qlabels.LabelTrie([(1,), ()])


@pytest.mark.parametrize("seed", list(range(40)) + ["labels", "split"])
def test_trie_and_paths_equal_the_oracle(seed):
    labels = {"labels": LABELS, "split": SPLIT}.get(seed)
    if labels is None:
        labels = _random_labels(seed)
    assert qlabels.label_trie(labels) == labels_ref.label_trie(labels)
    read = qlabels.read_nodes(labels)
    assert read == labels_ref.read_nodes(labels)
    assert qlabels.fed_nodes(read) == labels_ref.fed_nodes(read)
    for r in (None, read):
        paths = qlabels.trie_paths(labels, r)
        assert paths == labels_ref.trie_paths(labels, r)
        assert qlabels.path_reads(paths, r) == labels_ref.path_reads(paths, r)
        assert qlabels.path_tokens(paths, 7) == labels_ref.path_tokens(paths, 7)


def _log_softmax(x):
    x = np.asarray(x, dtype=np.float64)
    m = x.max(axis=-1, keepdims=True)
    return x - m - np.log(np.exp(x - m).sum(axis=-1, keepdims=True))


def test_one_token_labels_score_their_root_log_probability():
    labels = [(5,), (9,), (7,), (9,)]
    read = qlabels.read_nodes(labels)
    paths = qlabels.trie_paths(labels, read)
    targets = [5, 7, 9, 11]
    lp = _log_softmax(np.random.default_rng(0).normal(size=(1, 4)))
    got = qlabels.tree_scores(labels, paths, targets, lp, read)
    want = [lp[0, 0], lp[0, 2], lp[0, 1], lp[0, 2]]
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-15)
    np.testing.assert_allclose(got, qlabels.letter_scores(labels, targets, lp[0]), atol=0)


def test_a_label_others_extend_keeps_its_probability_minus_theirs():
    # labels a, ab, ac, b (a=1, b=2, c=3): the root and node (1,) are read
    labels = [(1,), (1, 2), (1, 3), (2,)]
    read = qlabels.read_nodes(labels)
    assert read == {(), (1,)}
    paths = qlabels.trie_paths(labels, read)
    targets = [1, 2, 3]
    root = [math.log(0.6), math.log(0.3), math.log(0.1)]
    after_a = [math.log(0.5), math.log(0.2), math.log(0.3)]
    rows = {(): root, (1,): after_a}
    order = [n for nodes, _, _ in paths for n in nodes]
    lp = np.array([rows[n] for n in order if n in read])
    got = np.exp(qlabels.tree_scores(labels, paths, targets, lp, read))
    # P(a) = 0.6 (1 - 0.2 - 0.3), P(ab) = 0.6 * 0.2, P(ac) = 0.6 * 0.3, P(b) = 0.3
    np.testing.assert_allclose(got, [0.3, 0.12, 0.18, 0.3], rtol=1e-12)


def test_a_chain_of_labels_gives_each_its_nearest_extensions_share():
    # labels a, ab, abc: abc takes from ab (its nearest label prefix), ab from a
    labels = [(1,), (1, 2), (1, 2, 3)]
    read = qlabels.read_nodes(labels)
    assert read == {(), (1,), (1, 2)}
    paths = qlabels.trie_paths(labels, read)
    targets = [1, 2, 3]
    rows = {(): [0.0, -np.inf, -np.inf],                        # P(a) = 1
            (1,): [math.log(0.6), math.log(0.4), -np.inf],     # P(b | a) = 0.4
            (1, 2): [math.log(0.75), -np.inf, math.log(0.25)]}  # P(c | ab) = 0.25
    lp = np.array([rows[n] for nodes, _, _ in paths for n in nodes if n in read])
    got = np.exp(qlabels.tree_scores(labels, paths, targets, lp, read))
    np.testing.assert_allclose(got, [0.6, 0.4 * 0.75, 0.4 * 0.25], rtol=1e-12)


@pytest.mark.parametrize("seed", range(30))
def test_label_probabilities_add_up_to_one(seed):
    """Every read row a log-softmax over the targets and the root's mass
    only on the labels' first tokens: the label probabilities sum to 1
    (each read node's mass goes to its label, if one ends there, and to its
    children's labels). Half the label sets also hold prefixes of their
    labels (chains of labels extending labels)."""
    labels = _random_labels(seed)
    if seed % 2:
        rng = np.random.default_rng(seed)
        labels += [ids[:int(rng.integers(1, len(ids) + 1))] for ids in labels]
    labels = sorted(set(labels))
    read = qlabels.read_nodes(labels)
    paths = qlabels.trie_paths(labels, read)
    targets = sorted({t for ids in labels for t in ids})
    trie = qlabels.label_trie(labels)
    ends = set(labels)
    rng = np.random.default_rng(100 + seed)
    order = [n for nodes, _, _ in paths for n in nodes]
    rows = []
    for node in order:
        if node not in read:
            continue
        logits = rng.normal(size=len(targets))
        # only the node's children may take mass, unless a label ends here
        allowed = set(trie.get(node, ()))
        if node not in ends:
            logits = np.where([t in allowed for t in targets], logits, -np.inf)
        rows.append(_log_softmax(logits))
    scores = qlabels.tree_scores(labels, paths, targets, np.array(rows), read)
    assert math.isclose(float(np.exp(scores).sum()), 1.0, rel_tol=1e-12)


def test_extensions_taking_all_the_mass_leave_minus_infinity():
    labels = [(1,), (1, 2)]
    read = qlabels.read_nodes(labels)
    paths = qlabels.trie_paths(labels, read)
    lp = np.array([[0.0, -np.inf], [-np.inf, 0.0]])   # root: token 1; after it: token 2
    got = qlabels.tree_scores(labels, paths, [1, 2], lp, read)
    assert got[0] == -np.inf and got[1] == 0.0
