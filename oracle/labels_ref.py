"""The label trie of trie-scored AI.CLASSIFY, in plain Python.

Test infrastructure (see oracle/__init__.py): it builds the `paths` and
`read_mask` a pack's label-path group carries, and each path row's
expected context, for the tree-layout tests. Restates the reference's
quail/labels.py:19-34 (label_trie), :47-62 (read_nodes), :129-131
(fed_nodes) and quail/execution/labels.py:151-210 (trie_paths,
path_reads) and label_stages.py:94-96 (the suffix tokens: the answer cue
at the root, then each node's last token).

Pinned by the reference's own known answers (tests/planner/
test_classify_cost.py:16, 106-108: LABELS reads 3 rows of a 4-token
suffix; :138-141: read_nodes of the splitting labels) and, in
tests/test_pack_tree.py, by invariants a wrong path split breaks: every
fed node is held exactly once, a path's rows are consecutive trie depths,
and a path's gathers are exactly its first node's ancestors.
"""


def label_trie(label_ids):
    """Each proper label prefix -> the sorted tokens that can follow it."""
    children = {}
    for ids in label_ids:
        if not ids:
            raise ValueError("a label has no tokens")
        for depth in range(len(ids)):
            children.setdefault(tuple(ids[:depth]), set()).add(ids[depth])
    return {prefix: sorted(tokens) for prefix, tokens in children.items()}


def read_nodes(label_ids):
    """The root and every node where labels split or one ends and another goes on."""
    trie = label_trie(label_ids)
    ends = {tuple(ids) for ids in label_ids}
    return {()} | {node for node, tokens in trie.items() if len(tokens) > 1 or node in ends}


def fed_nodes(read):
    """The read nodes and all their ancestors."""
    return {node[:depth] for node in read for depth in range(len(node) + 1)}


def trie_paths(label_ids, read=None):
    """[(nodes, first depth, gathers)] covering every fed node once: a path
    follows each node's first fed child; every other fed child opens a new
    path; gathers are the (earlier path, leading rows) holding the
    ancestors of a path's first node."""
    trie = label_trie(label_ids)
    fed = fed_nodes(set(trie) if read is None else read)
    paths, placed = [], {}

    def grow(path, node):
        placed[node] = (path, len(paths[path][0]))
        paths[path][0].append(node)
        kids = [node + (t,) for t in trie.get(node, ()) if node + (t,) in fed]
        for i, kid in enumerate(kids):
            if i:
                paths.append(([], len(kid), []))
                grow(len(paths) - 1, kid)
            else:
                grow(path, kid)

    paths.append(([], 0, []))
    grow(0, ())
    for nodes, _, gathers in paths[1:]:
        parent = nodes[0][:-1]
        need = {}
        for depth in range(len(parent) + 1):
            path, row = placed[parent[:depth]]
            need[path] = max(need.get(path, 0), row + 1)
        gathers.extend(sorted(need.items()))
    return paths


def path_reads(paths, read=None):
    """Per path row, in path order: is it read."""
    return [read is None or node in read for nodes, _, _ in paths for node in nodes]


def path_tokens(paths, cue):
    """The suffix a label-path group packs: the cue at the root, else the
    node's last token."""
    return [cue if node == () else node[-1] for nodes, _, _ in paths for node in nodes]


def path_contexts(paths, cue, document):
    """Per path row: the (token, position) list it must attend to, the
    document, the cue, then its node's tokens (positions from 0)."""
    f = len(document)
    base = [(int(t), p) for p, t in enumerate(document)] + [(int(cue), f)]
    return [base + [(int(t), f + 1 + i) for i, t in enumerate(node)]
            for nodes, _, _ in paths for node in nodes]
