"""Structural oracle for pack layouts: what every packed row's attention reads.

Test infrastructure (see oracle/__init__.py). It plays the role of the
reference's HashModel KV checker (tests/helpers/kv_checker.py:1-12, 77-115,
driven by tests/engine/test_kv_reads.py): a pool model records, per arena
row, the (token, position) a pack's scatter map wrote there (kv_row_scatter,
attention.py:885-897, then the tail copies of :1192-1195); each query row
then reads its sequence's keys through the block table exactly as the paged
causal call does (visible keys < used - q_len + i + 1, attention.py:1280-1306)
and must find precisely its own document's tokens at positions 0..its own
position, in order. Any wrong page, row, position, length or a stale page
read gives a different list.
"""

import numpy as np


class PoolModel:
    """Arena rows -> (token, position) of the KV written there."""

    def __init__(self):
        self.rows = {}

    def apply(self, ids, positions, unified):
        src = np.asarray(unified["src"], dtype=np.int64)
        dst = np.asarray(unified["dst"], dtype=np.int64)
        for s, d in zip(src.tolist(), dst.tolist()):
            if d >= 0:
                self.rows[d] = (int(ids[s]), int(positions[s]))
        if unified.get("tail_src") is not None:
            for s, d in zip(np.asarray(unified["tail_src"]).tolist(),
                            np.asarray(unified["tail_dst"]).tolist()):
                self.rows[d] = self.rows.get(s, ("unwritten", s))

    def forget_pages(self, pages, page):
        for p in pages:
            for r in range(p * page, p * page + page):
                self.rows.pop(r, None)


def visible_keys(unified, page, pool: PoolModel, causal=True):
    """Per packed row: the list of (token, position) its attention reads."""
    cu = np.asarray(unified["cu_q"], dtype=np.int64)
    used = np.asarray(unified["used"], dtype=np.int64)
    table = np.asarray(unified["table"], dtype=np.int64)
    out = {}
    for s in range(len(used)):
        q_len = int(cu[s + 1] - cu[s])
        seen = int(used[s])
        keys = []
        for j in range(seen):
            row = int(table[s, j // page]) * page + j % page
            keys.append(pool.rows.get(row, ("unwritten", row)))
        for i in range(q_len):
            lim = seen - q_len + i + 1 if causal else seen
            out[int(cu[s]) + i] = keys[:lim]
    return out


def check_pack(chunk, page, pool: PoolModel, prompt_of_key):
    """Apply the pack's writes to the pool model and check every row's reads.

    prompt_of_key(key) -> the document's full token list. Returns the number
    of rows checked; raises AssertionError naming the first bad row.
    """
    unified = chunk.host.get("unified", chunk.meta["unified"])
    ids = np.asarray(chunk.host_ids)
    positions = np.asarray(chunk.host_positions)
    pool.apply(ids, positions, unified)
    reads = visible_keys(unified, page, pool)
    checked = 0
    for key, row0, _, row1 in chunk.row_spans:
        prompt = list(prompt_of_key(key))
        for r in range(row0, row1):
            pos = int(positions[r])
            assert ids[r] == prompt[pos], f"row {r}: token {ids[r]} != prompt[{pos}]"
            want = [(int(t), p) for p, t in enumerate(prompt[:pos + 1])]
            got = reads[r]
            assert got == want, (f"row {r} of {key!r} at position {pos} reads "
                                 f"{got[:4]}...{got[-2:]} (len {len(got)}), want len {len(want)}")
            checked += 1
    return checked


def check_pack_tree(chunk, page, pool: PoolModel, prompt_of_key, context_of_row=None):
    """The tree layout's reads (attention.py:1395-1441): the pack's KV writes
    land in the pool first (kv_src -> kv_dst); a row then reads, in call B,
    its reader sequence's `used` keys through that sequence's table (not
    causal) when source[row] >= 0, in call C (label-path rows,
    reads["nodes"], :1424-1434) the gathered rows of its node sequence, and
    in call A the rows of its own cu_a segment up to itself. Together, in
    that order, they must be exactly its document's tokens at positions
    0..its own position, or context_of_row(key, row) when that gives a
    list. Returns the number of rows checked; raises AssertionError naming
    the first bad row."""
    meta = chunk.meta
    host = chunk.host or {}
    ids = np.asarray(chunk.host_ids)
    positions = np.asarray(chunk.host_positions)
    kv_src = host.get("kv_src", meta.get("kv_src"))
    kv_dst = host.get("kv_dst", meta.get("kv_dst"))
    if kv_src is not None:
        pool.apply(ids, positions, dict(src=kv_src, dst=kv_dst))
    reads = host.get("reads", meta.get("reads"))
    cu_a = np.asarray(host.get("segments", meta.get("segments"))["cu_q"], dtype=np.int64)
    b_keys, c_keys = {}, {}
    nodes = reads.get("nodes") if reads is not None else None
    if nodes is not None:
        q_rows = np.asarray(nodes["rows"], dtype=np.int64)
        k_rows = np.asarray(nodes["key_rows"], dtype=np.int64)
        ncu_q = np.asarray(nodes["cu_q"], dtype=np.int64)
        ncu_k = np.asarray(nodes["cu_k"], dtype=np.int64)
        b_index = np.asarray(nodes["b_index"], dtype=np.int64)
        for s in range(len(ncu_q) - 1):
            keys = [(int(ids[j]), int(positions[j])) for j in k_rows[ncu_k[s]:ncu_k[s + 1]]]
            for i in range(int(ncu_q[s]), int(ncu_q[s + 1])):
                c_keys[int(q_rows[i])] = keys
        for i, r in enumerate(q_rows.tolist()):
            assert int(np.asarray(reads["rows"])[b_index[i]]) == r, f"node row {r}: b_index"
    if reads is not None:
        rows = np.asarray(reads["rows"], dtype=np.int64)
        cu = np.asarray(reads["cu_q"], dtype=np.int64)
        used = np.asarray(reads["used"], dtype=np.int64)
        table = np.asarray(reads["table"], dtype=np.int64)
        source = np.asarray(reads["source"], dtype=np.int64)
        for s in range(len(used)):
            keys = [pool.rows.get(int(table[s, j // page]) * page + j % page, ("unwritten", j))
                    for j in range(int(used[s]))]
            for i in range(int(cu[s]), int(cu[s + 1])):
                b_keys[int(rows[i])] = keys
        for r in range(len(ids)):
            assert (source[r] >= 0) == (r in b_keys), f"row {r}: source map"
            if source[r] >= 0:
                assert rows[source[r]] == r, f"row {r}: source {source[r]}"
    seg_of = np.searchsorted(cu_a, np.arange(len(ids)), side="right") - 1
    checked = 0
    for key, row0, _, row1 in chunk.row_spans:
        prompt = list(prompt_of_key(key))
        for r in range(row0, row1):
            pos = int(positions[r])
            want = context_of_row(key, r) if context_of_row is not None else None
            if want is None:
                assert ids[r] == prompt[pos], f"row {r}: token {ids[r]} != prompt[{pos}]"
                want = [(int(t), p) for p, t in enumerate(prompt[:pos + 1])]
            a0 = int(cu_a[seg_of[r]])
            got = (list(b_keys.get(r, [])) + list(c_keys.get(r, []))
                   + [(int(ids[j]), int(positions[j])) for j in range(a0, r + 1)])
            assert got == want, (f"row {r} of {key!r} at position {pos} reads "
                                 f"{got[:4]}...{got[-2:]} (len {len(got)}), want len {len(want)}")
            checked += 1
    return checked
