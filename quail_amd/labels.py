"""The label trie of trie-scored AI.CLASSIFY (the trie_tree rule).

The caller side of a label-path pack (`quail_amd.chunk.pack_chunk` with
`paths` and `read_mask`): which trie nodes a document's pass reads, how
the nodes it feeds split into causal paths, the suffix tokens that feed
them, and each label's log probability from the rows read. Follows
quail/labels.py:19-62, 129-131 (label_trie, read_nodes, fed_nodes),
quail/execution/labels.py:47-61, 151-260 (letter_scores, trie_paths,
path_reads, tree_scores) and
quail/backends/quail/executor/label_stages.py:93-99 (the suffix tokens
and the score call), with the same results.

A node is a label prefix, as a tuple of token ids; the root () is the
answer cue's row. A path is (nodes, start, gathers): the nodes whose rows
it holds in order (consecutive trie depths), the depth of its first node,
and the (path, leading rows) pairs that hold the first node's ancestors.
"""

import math

import numpy as np


class LabelTrie:
    """The trie of a label set.

    Args:
        label_ids: One token id sequence per label (duplicates allowed).

    Raises:
        ValueError: A label has no tokens.
    """

    def __init__(self, label_ids):
        self.labels = [tuple(int(t) for t in ids) for ids in label_ids]
        nexts = {}
        for ids in self.labels:
            if not ids:
                raise ValueError("a label has no tokens")
            for depth, token in enumerate(ids):
                nexts.setdefault(ids[:depth], set()).add(token)
        # every proper label prefix -> the tokens that may follow it, ascending
        self.children = {node: sorted(tokens) for node, tokens in nexts.items()}
        self.ends = set(self.labels)

    def read_nodes(self) -> set:
        """The root and every node where the labels part: two or more
        next tokens, or a label ending where another goes on."""
        return {()} | {node for node, tokens in self.children.items()
                       if len(tokens) > 1 or node in self.ends}

    def paths(self, read=None) -> list:
        """The fed nodes (the read nodes and their ancestors) split into
        paths that hold each once: a node's first fed child continues its
        path, every later one starts a new path, made when the walk (depth
        first, children by ascending token) reaches it."""
        if read is None:
            read = set(self.children)
        fed = fed_nodes(read)
        paths = []
        where = {}                  # node -> (path, row)
        pending = [((), None)]      # (node, its path; None: a new one)
        while pending:
            node, path = pending.pop()
            if path is None:
                paths.append(([], len(node), []))
                path = len(paths) - 1
            where[node] = (path, len(paths[path][0]))
            paths[path][0].append(node)
            kids = [node + (t,) for t in self.children.get(node, ()) if node + (t,) in fed]
            # popped first: the first child, on this path
            for i in range(len(kids) - 1, -1, -1):
                pending.append((kids[i], path if i == 0 else None))
        for nodes, _, gathers in paths[1:]:
            first = nodes[0]
            rows = {}
            for depth in range(len(first)):
                p, r = where[first[:depth]]
                rows[p] = max(rows.get(p, 0), r + 1)
            gathers.extend(sorted(rows.items()))
        return paths

    def scores(self, paths, targets, logprobs, read=None) -> np.ndarray:
        """Each label's log probability: the sum of its tokens' log
        probabilities at its read nodes, times, for a label that others
        extend, one minus the share its nearest label extensions take
        (minus infinity when they take all of it).

        Args:
            paths: From `paths` (or `trie_paths`).
            targets: The token id of each column of `logprobs`.
            logprobs: (read rows, targets): the paths' read rows in path
                order.
            read: The read nodes; None: every path row was read.
        """
        logprobs = np.asarray(logprobs, dtype=np.float64)
        row = {}
        for node, is_read in zip((n for nodes, _, _ in paths for n in nodes),
                                 path_reads(paths, read)):
            if is_read:
                row[node] = len(row)
        col = {int(t): c for c, t in enumerate(targets)}

        def tokens_logprob(ids, first=0):
            # the tokens at depths first.. whose preceding node was read
            return sum(float(logprobs[row[ids[:d]], col[ids[d]]])
                       for d in range(first, len(ids)) if ids[:d] in row)

        share = dict.fromkeys(self.labels, 0.0)
        for ids in share:
            parent = next((ids[:d] for d in range(len(ids) - 1, 0, -1) if ids[:d] in share),
                          None)
            if parent is not None:
                share[parent] += math.exp(tokens_logprob(ids, len(parent)))
        out = np.empty(len(self.labels), dtype=np.float64)
        for i, ids in enumerate(self.labels):
            # rounding may leave the extensions all of the mass, or more
            out[i] = (tokens_logprob(ids) + math.log1p(-share[ids])
                      if share[ids] < 1.0 else -math.inf)
        return out


def label_trie(label_ids) -> dict:
    """Every proper label prefix -> the sorted tokens that may follow it."""
    return LabelTrie(label_ids).children


def read_nodes(label_ids) -> set:
    """The trie nodes whose rows the trie_tree rule reads."""
    return LabelTrie(label_ids).read_nodes()


def fed_nodes(read) -> set:
    """The read nodes and all their ancestors (whose tokens are fed)."""
    return {node[:depth] for node in read for depth in range(len(node) + 1)}


def trie_paths(label_ids, read=None) -> list:
    """The fed trie nodes as paths, (nodes, start, gathers) each."""
    return LabelTrie(label_ids).paths(read)


def path_reads(paths, read=None) -> list:
    """For each path row in path order, whether it is read."""
    return [read is None or node in read for nodes, _, _ in paths for node in nodes]


def path_tokens(paths, cue) -> list:
    """The suffix that feeds the paths: the answer cue at the root, then
    each node's last token, path after path."""
    return [int(cue) if node == () else node[-1] for nodes, _, _ in paths for node in nodes]


def tree_scores(label_ids, paths, targets, logprobs, read=None) -> np.ndarray:
    """Each label's log probability from the paths' read rows."""
    return LabelTrie(label_ids).scores(paths, targets, logprobs, read)


def letter_scores(label_ids, targets, logprobs) -> np.ndarray:
    """The letters rule: each (one-token) label's log probability at the
    answer row, `logprobs` holding one value per target."""
    col = {int(t): c for c, t in enumerate(targets)}
    return np.asarray([float(logprobs[col[int(ids[0])]]) for ids in label_ids],
                      dtype=np.float64)
