"""Lay out scheduled document groups as one packed forward pass.

The unified causal path of the reference's pack_chunk
(quail/backends/quail/executor/chunk.py:505-1160, in particular the group
loop :606-684, the unified pools :913-1054, _PoolBuilder :407-502 and the
meta dict :1140-1158). Each group is

    dict(key=..., prefix=tokens or None, f=..., start=..., suffixes=[...])

where `prefix` is the document's fresh tokens past `start` (the tokens a
borrowed parent prefix already holds), `f` the document length the
suffixes follow, and `suffixes` the question token runs. Rows are laid out
as [prefix | suffix, suffix, ...] per group in order; positions continue
from `start` through the prefix and restart at `f` for every suffix.

For the one paged causal attention call every group becomes sequences:
  * "direct" (one suffix and the key's pages cover start + rows): one
    sequence reading the key's table with used = f + suffix rows, its rows
    scattered straight into the key's pages;
  * otherwise the prefix is one sequence (used = f) and each suffix gets a
    temporary key whose pages follow the key's full pages; a partial last
    page of the prefix is copied into the temporary first (tail copy).

Outputs match the reference's field for field: input_ids, positions,
final_indices (last row of each suffix), cu_a, and meta["unified"] =
{cu_q, used, table, src, dst, tail_src, tail_dst, max_q, max_used, causal,
cu_q_host, used_host, page_rows}. The layout is computed in C++
(csrc/host_pack.cpp, qx_pack_unified) against the arena's page accounting,
also C++; host arrays are numpy; `upload` moves them to the device in one
pinned staging copy per array.
"""

import ctypes
import time
from dataclasses import dataclass, field
from typing import Any

import numpy as np


class ArenaFullError(RuntimeError):
    """The KV arena has too few free pages to pack the chunk."""


@dataclass
class Chunk:
    input_ids: Any
    positions: Any
    final_indices: Any
    meta: dict
    attention_mode: str
    tokens: int
    layout: list
    row_spans: tuple = ()
    temporary_keys: tuple = ()
    fresh_keys: tuple = ()
    rows_per_answer: Any = None
    host_ids: np.ndarray = None
    host_positions: np.ndarray = None
    host: dict = field(default_factory=dict)


def pages_for_questions(arena, groups) -> int:
    """At most the temporary pages the groups' questions take in a unified
    pack (a question that does not fit its key's pages gets the prefix's
    partial last page and its own rows)."""
    t = arena.page_tokens
    return sum(arena.pages_needed(t + len(np.asarray(s).reshape(-1)))
               for g in groups for s in g["suffixes"])


def _as_suffixes(sufs):
    arrays = [np.asarray(s, dtype=np.int64) for s in sufs]
    lengths = np.asarray([len(a) for a in arrays], dtype=np.int64)
    ids = np.concatenate(arrays) if arrays else np.empty(0, dtype=np.int64)
    return ids, lengths


def _cat(parts, dtype=np.int64):
    parts = [np.asarray(p, dtype=dtype) for p in parts if len(p)]
    return np.concatenate(parts) if parts else np.empty(0, dtype=dtype)


# qx_pack_array indices (include/quail_mi355x.h)
(_IDS, _POSITIONS, _FINALS, _CU_A, _ROWS_PER_ANSWER, _SRC, _DST, _TAIL_SRC, _TAIL_DST, _CU_Q,
 _USED, _TABLE, _SEQ_PAGES, _TEMPORARIES, _ROW_SPANS, _SUFFIX_COUNTS, _FRESH_KEYS,
 _SCALARS) = range(18)
_EFULL = -4


def _pack_arrays(handle):
    """Copy a qx_pack_unified result into numpy arrays (int32 where noted)."""
    from quail_amd import _lib
    lib = _lib.load()
    data, count = ctypes.c_void_p(), ctypes.c_int64()
    out = []
    for which in range(18):
        rc = lib.qx_pack_array(handle, which, ctypes.byref(data), ctypes.byref(count))
        if rc:
            raise _lib.QxError(f"qx_pack_array: {lib.qx_last_error().decode()}")
        ctype = ctypes.c_int32 if which in (_CU_A, _CU_Q, _USED, _TABLE) else ctypes.c_int64
        dtype = np.int32 if ctype is ctypes.c_int32 else np.int64
        n = count.value
        if n:
            buf = (ctype * n).from_address(data.value)
            out.append(np.frombuffer(buf, dtype=dtype).copy())
        else:
            out.append(np.empty(0, dtype=dtype))
    return out


def _suffix_reads(g, s_row0, slen):
    """The answer rows of a group's suffixes (chunk.py:726-764): the marked
    rows of its one suffix (`read_mask`), the last `read_rows[j]` rows of
    suffix j, every row (`read_all_rows`), or each suffix's last row.
    Returns (rows, rows per answer, several rows per answer?)."""
    key = g["key"]
    n = len(slen)
    ends = s_row0 + np.cumsum(slen)
    total = int(slen.sum())
    if g.get("read_mask") is not None:
        marked = np.asarray(g["read_mask"], dtype=bool)
        if n != 1 or len(marked) != total:
            raise ValueError(f"group {key!r}: read_mask marks one suffix's rows")
        rows = s_row0 + np.flatnonzero(marked)
        return rows, np.array([len(rows)], dtype=np.int64), True
    if g.get("read_rows") is not None:
        counts = np.asarray(g["read_rows"], dtype=np.int64)
        if len(counts) != n or (counts > slen).any() or (counts < 0).any():
            raise ValueError(f"group {key!r}: read_rows must give each suffix at most its "
                             f"length")
        rows = (np.repeat(ends - counts, counts)
                + np.arange(int(counts.sum()), dtype=np.int64)
                - np.repeat(np.cumsum(counts) - counts, counts))
        return rows, counts, True
    if g.get("read_all_rows"):
        return np.arange(s_row0, s_row0 + total, dtype=np.int64), slen.astype(np.int64), True
    return ends - 1, np.ones(n, dtype=np.int64), False


def pack_chunk(arena, groups, *, attention_mode="unified", mask="causal", timing=None,
               attention_heads=None):
    """Pack groups for one unified causal forward pass (host arrays only).

    The layout runs in C++ (qx_pack_unified) against the arena's page
    accounting; this function flattens the groups, calls it, and wraps the
    arrays.

    attention_heads: (HQ, HK, D) of the model; with it the attention
    metadata also carries the work list of the paged calls (one item per
    query tile that holds rows, heaviest first, qx_paged_attention_work).

    Raises ValueError for layouts this path does not run and ArenaFullError
    when the suffixes' temporary pages do not fit (nothing stays allocated).
    """
    from quail_amd import _lib

    if mask != "causal":
        raise ValueError("this engine packs the causal mask")
    if attention_mode == "tree":
        return _pack_tree(arena, groups, timing=timing, attention_heads=attention_heads)
    if attention_mode != "unified":
        raise ValueError(f"attention_mode must be 'unified' or 'tree', got {attention_mode!r}")
    t0 = time.perf_counter()
    acct = arena.accounting
    keys, desc, prefixes, suffix_lens, suffix_ids = [], [], [], [], []
    for g in groups:
        key = g["key"]
        if not acct.is_resident(key):
            raise ValueError(f"group {key!r}: the paged unified path needs arena pages")
        if g.get("paths") is not None:
            raise ValueError(f"group {key!r}: paths pack one suffix, every row read, under "
                             f"tree attention")
        for name in ("canvas", "questions"):
            if g.get(name) is not None:
                raise ValueError(f"group {key!r}: this engine has no {name} rows")
        keys.append(key)
        fresh = g.get("prefix") is not None
        prefix = np.asarray(g["prefix"], dtype=np.int64) if fresh else None
        sids, slen = _as_suffixes(g["suffixes"])
        if g.get("read_mask") is not None or g.get("read_rows") is not None:
            _suffix_reads(g, 0, slen)   # refuse bad answer rows before pages move
        if fresh:
            prefixes.append(prefix)
        suffix_lens.append(slen)
        suffix_ids.append(sids)
        desc.append((acct.key_id(key), int(fresh), int(g["f"]), int(g.get("start", 0)),
                     len(prefix) if fresh else 0, len(slen),
                     int(g.get("write_suffix_tokens") or 0), int(bool(g.get("read_all_rows")))))
    desc = np.asarray(desc, dtype=np.int64).reshape(-1, 8)
    prefix_ids = _cat(prefixes)
    lens = _cat(suffix_lens)
    sids = _cat(suffix_ids)
    t1 = time.perf_counter()

    lib = _lib.load()
    handle, failed = ctypes.c_void_p(), ctypes.c_int64(-1)
    ptr = lambda a: a.ctypes.data if a.size else None  # noqa: E731
    rc = lib.qx_pack_unified(acct.handle, ptr(desc), len(desc), ptr(prefix_ids), ptr(lens),
                             ptr(sids), ctypes.byref(handle), ctypes.byref(failed))
    if rc:
        msg = lib.qx_last_error().decode(errors="replace")
        where = f"group {keys[failed.value]!r}: " if 0 <= failed.value < len(keys) else ""
        if rc == _EFULL:
            raise ArenaFullError(msg)
        raise ValueError(where + msg)
    try:
        (ids, positions, final, cu_a, rows_per_answer, src, dst, tail_src, tail_dst, cu_q, used,
         table, seq_pages, temporaries, row_spans, suffix_counts, fresh_ids,
         scalars) = _pack_arrays(handle)
    finally:
        lib.qx_pack_destroy(handle)
    n_tok, max_q, max_used, multi, has_tail, width = (int(v) for v in scalars)
    temporary_keys = tuple(acct.adopt(int(t)) for t in temporaries)
    table = table.reshape(-1, width)
    key_of = {acct.key_id(k): k for k in keys}
    spans = row_spans.reshape(-1, 3).tolist()
    if any(g.get("read_mask") is not None or g.get("read_rows") is not None for g in groups):
        # answer rows other than the last / every suffix row
        parts = [_suffix_reads(g, span[1], slen)
                 for g, span, slen in zip(groups, spans, suffix_lens) if len(slen)]
        final = _cat([p[0] for p in parts])
        rows_per_answer = _cat([p[1] for p in parts])
        multi = any(p[2] for p in parts)
    unified = dict(
        src=src, dst=dst,
        tail_src=tail_src if has_tail else None,
        tail_dst=tail_dst if has_tail else None,
        used=used, table=table, cu_q=cu_q, cu_q_host=cu_q.tolist(),
        used_host=used.tolist(),
        page_rows=[table[i, :c].tolist() for i, c in enumerate(seq_pages.tolist())],
        max_q=max_q, max_used=max_used, causal=True,
        # the scatter source is the pack's rows in order: row i's KV goes to
        # dst[i], which lets qk_norm_rope write it in place
        rows_in_order=bool(src.size == n_tok and np.array_equal(src, np.arange(n_tok))))
    meta = dict(layer=0, unified=unified, cu_a=cu_a,
                max_a=int(np.diff(cu_a).max()) if len(cu_a) > 1 else 0,
                final_query=_final_query(cu_q, used, table, final))
    if attention_heads is not None:
        for tables in (unified, meta["final_query"]):
            if tables is not None:
                tables["work"], tables["n_work"], tables["work_rows"] = _work_list(
                    tables, attention_heads, choose_rows=True)
    if timing is not None:
        timing["pack_py"] = timing.get("pack_py", 0.0) + (t1 - t0)
        timing["pack_unified"] = timing.get("pack_unified", 0.0) + (time.perf_counter() - t1)
    return Chunk(input_ids=ids, positions=positions, final_indices=final, meta=meta,
                 attention_mode="unified", tokens=n_tok,
                 layout=list(zip(keys, suffix_counts.tolist())),
                 row_spans=tuple((k, *span) for k, span in zip(keys, spans)),
                 temporary_keys=temporary_keys,
                 fresh_keys=tuple(key_of[int(i)] for i in fresh_ids),
                 rows_per_answer=rows_per_answer if multi else None,
                 host_ids=ids, host_positions=positions)


_TREE_UNSUPPORTED = ("canvas", "questions")


def _pack_tree(arena, groups, *, timing=None, attention_heads=None):
    """The tree attention layout (chunk.py:580-912, the reads of :1010-1054
    and the KV writes of :1060-1079 with attention_mode="tree").

    Call A is causal over the pack's own rows in `cu_a` segments: a fresh
    group's prefix is a segment (unless the group is `whole`, one segment
    with its suffix, or `stacked`), and each suffix is one. Call B reads
    resident KV, not causally: a borrowing prefix reads its key's pages
    before `start`; a suffix reads its key's pages [0, f); a stacked
    group (one suffix, a `read_key`) reads the read key's pages before
    `start` with all its rows, siblings with the same read key and start
    in one sequence. Fresh rows of paged keys (and kept suffix rows) are
    written to the key's pages first (kv_src -> kv_dst), so a later suffix
    or a child can read them.

    Label paths (`paths`, one suffix of a paged document holding the trie
    paths back to back, chunk.py:765-786; the document's rows may be in the
    same pack, as their own segment, never `whole` or `stacked`): each path
    is its own call A segment at positions f + its first node's depth
    onward, every path row reads the document's pages in call B, and a
    path's rows read the rows above its first node
    (leading rows of earlier paths, its `gathers`) in call C,
    `reads["nodes"]` (chunk.py:894-907). `read_mask` marks the one
    suffix's rows that feed the answer (chunk.py:726-741).
    """
    t0 = time.perf_counter()
    id_parts, pos_parts, finals, cu_a = [], [], [], [0]
    rows_per_answer, multi = [], False
    layout, row_spans, fresh_keys = [], [], []
    kv_writes, reader_rows, read_keys, read_used, cu_q = [], [], [], [], [0]
    node_q, node_k, node_cu_q, node_cu_k = [], [], [0], [0]
    # the pages each read sequence goes through: its read key's table; a
    # stacked run whose read key has left the arena (its last borrower was
    # admitted) reads its first document's table, whose leading pages are
    # the read key's borrowed ones
    table_keys = []
    max_q = 0
    n_tok = 0
    for g in groups:
        key = g["key"]
        for name in _TREE_UNSUPPORTED:
            if g.get(name) is not None:
                raise ValueError(f"group {key!r}: this engine has no {name} rows")
        fresh = g.get("prefix") is not None
        f = int(g["f"])
        start = int(g.get("start", 0))
        paged = arena.is_resident(key)
        row0 = n_tok
        sids, slen = _as_suffixes(g["suffixes"])
        n = len(slen)
        paths = g.get("paths")
        borrowing = fresh and start > 0
        # a group with label paths keeps its prefix rows a segment of their
        # own (its path rows read them from the pages, as a kept document's)
        stacked = borrowing and n == 1 and g.get("read_key") is not None and paths is None
        whole = (fresh and paged and not start and n == 1 and bool(g.get("single"))
                 and paths is None)
        prefix_len = 0
        if fresh:
            if not paged and n > 1:
                raise ValueError(f"group {key!r}: an unpaged fresh group packs [prefix | suffix] "
                                 f"as one causal segment, which only one suffix may join")
            if start and not paged:
                raise ValueError(f"group {key!r}: a borrowed prefix needs arena pages")
            prefix = np.asarray(g["prefix"], dtype=np.int64)
            prefix_len = len(prefix)
            id_parts.append(prefix)
            pos_parts.append(np.arange(start, start + prefix_len, dtype=np.int64))
            n_tok += prefix_len
            if (paged or not n) and not stacked and not whole:
                cu_a.append(n_tok)
            if borrowing and not stacked:
                reader_rows.append(np.arange(row0, n_tok, dtype=np.int64))
                cu_q.append(cu_q[-1] + prefix_len)
                read_keys.append(key)
                table_keys.append(key)
                read_used.append(start)
                max_q = max(max_q, prefix_len)
            if paged:
                kv_writes.append((key, row0, n_tok, start))
                fresh_keys.append(key)
        elif not paged:
            raise ValueError(f"group {key!r}: a kept group needs its arena pages")
        prefix_end = n_tok
        s_row0 = n_tok
        total = int(slen.sum())
        ends = np.cumsum(slen)
        begins = ends - slen
        if n:
            id_parts.append(sids)
            read, per_answer, several = _suffix_reads(g, s_row0, slen)
            finals.append(read)
            rows_per_answer.append(per_answer)
            multi = multi or several
            if paths is not None:
                if n != 1 or not g.get("read_all_rows") or not paged:
                    raise ValueError(f"group {key!r}: paths pack one suffix of a paged "
                                     f"document, every row read")
                lengths = np.asarray([len(nodes) for nodes, _, _ in paths], dtype=np.int64)
                if int(lengths.sum()) != total:
                    raise ValueError(f"group {key!r}: paths hold {int(lengths.sum())} rows, "
                                     f"the suffix {total}")
                starts = np.asarray([first for _, first, _ in paths], dtype=np.int64)
                path_ends = s_row0 + np.cumsum(lengths)
                path_row0 = path_ends - lengths
                pos_parts.append(f + np.repeat(starts, lengths)
                                 + np.arange(total, dtype=np.int64)
                                 - np.repeat(path_row0 - s_row0, lengths))
                cu_a.extend(path_ends.tolist())
                for index, (_, _, gathers) in enumerate(paths):
                    if not gathers:
                        continue
                    if any(c >= index or count > lengths[c] for c, count in gathers):
                        raise ValueError(f"group {key!r}: path {index} gathers rows outside "
                                         f"the earlier paths")
                    node_q.append(np.arange(path_row0[index], path_ends[index],
                                            dtype=np.int64))
                    node_k.append(np.concatenate([
                        np.arange(path_row0[c], path_row0[c] + count, dtype=np.int64)
                        for c, count in gathers]))
                    node_cu_q.append(node_cu_q[-1] + int(lengths[index]))
                    node_cu_k.append(node_cu_k[-1] + len(node_k[-1]))
            else:
                within = np.arange(total, dtype=np.int64) - np.repeat(begins, slen)
                pos_parts.append(f + within)
                cu_a.extend((s_row0 + ends).tolist())
            n_tok += total
            keep = int(g.get("write_suffix_tokens") or 0)
            if keep and paged:
                kv_writes.append((key, s_row0, s_row0 + keep, start + prefix_len if fresh else f))
        num_s = n_tok - s_row0
        layout.append((key, n))
        row_spans.append((key, row0, prefix_end, n_tok))
        if stacked:
            count = n_tok - row0
            reader_rows.append(np.arange(row0, n_tok, dtype=np.int64))
            read_key = g["read_key"]
            if read_keys and read_keys[-1] == read_key and read_used[-1] == start:
                cu_q[-1] += count
                max_q = max(max_q, cu_q[-1] - cu_q[-2])
            else:
                cu_q.append(cu_q[-1] + count)
                read_keys.append(read_key)
                table_keys.append(read_key if arena.is_resident(read_key) else key)
                read_used.append(start)
                max_q = max(max_q, count)
        elif num_s and f and paged and not whole:
            reader_rows.append(np.arange(s_row0, n_tok, dtype=np.int64))
            cu_q.append(cu_q[-1] + num_s)
            read_keys.append(key)
            table_keys.append(key)
            read_used.append(f)
            max_q = max(max_q, num_s)
    t1 = time.perf_counter()

    reads = None
    if read_keys:
        table = arena.block_table_rows([arena.owned_pages(k) for k in table_keys])
        rows = _cat(reader_rows)
        source = np.full(n_tok, -1, dtype=np.int32)
        source[rows] = np.arange(len(rows), dtype=np.int32)
        used = np.asarray(read_used, dtype=np.int32)
        reads = dict(rows=rows, cu_q=np.asarray(cu_q, dtype=np.int32), max_q=max_q, used=used,
                     max_used=int(used.max()), table=table, source=source, causal=False)
    if node_q:
        q_rows = _cat(node_q)
        if reads is None or (reads["source"][q_rows] < 0).any():
            raise ValueError("path rows read their document in call B; the document needs "
                             "arena pages")
        ncu_q = np.asarray(node_cu_q, dtype=np.int32)
        ncu_k = np.asarray(node_cu_k, dtype=np.int32)
        reads["nodes"] = dict(
            rows=q_rows, key_rows=_cat(node_k), cu_q=ncu_q, cu_k=ncu_k,
            used=np.diff(ncu_k).astype(np.int32), max_q=int(np.diff(ncu_q).max()),
            max_used=int(np.diff(ncu_k).max()), causal=False,
            # each node row's index among call B's rows
            b_index=reads["source"][q_rows].astype(np.int64))
        # where call C's gathered K/V rows land: 0..len(key_rows)-1
        reads["nodes"]["gather_rows"] = np.arange(len(reads["nodes"]["key_rows"]),
                                                  dtype=np.int64)
        reads["nodes"]["max_k"] = reads["nodes"]["max_used"]
    kv_src = kv_dst = None
    if kv_writes:
        src, dst = [], []
        for key, r0, r1, dest in kv_writes:
            rows = arena.capacity_rows(key)[dest:dest + (r1 - r0)]
            if len(rows) != r1 - r0:
                raise ValueError(f"group {key!r}: KV write of {r1 - r0} rows at {dest} exceeds "
                                 f"its reserved rows")
            src.append(np.arange(r0, r1, dtype=np.int64))
            dst.append(rows)
        kv_src, kv_dst = _cat(src), _cat(dst)
    # pool row per pack row (-1: none), for the qk-norm-rope pass to write
    # the KV of the pack's rows into the pages itself
    row_pool_dst = None
    if kv_src is not None and len(np.unique(kv_src)) == len(kv_src):
        row_pool_dst = np.full(n_tok, -1, dtype=np.int64)
        row_pool_dst[kv_src] = kv_dst
    cu_a_arr = np.asarray(cu_a, dtype=np.int32)
    segments = dict(cu_q=cu_a_arr, used=np.diff(cu_a_arr).astype(np.int32),
                    max_q=int(np.diff(cu_a_arr).max()) if len(cu_a) > 1 else 0, causal=True)
    segments["max_used"] = segments["max_q"]
    if attention_heads is not None:
        for tables in (segments, reads, reads and reads.get("nodes")):
            if tables:
                tables["work"], tables["n_work"], _ = _work_list(tables, attention_heads)
    ids = _cat(id_parts)
    positions = _cat(pos_parts)
    final = _cat(finals)
    meta = dict(layer=0, unified=None, kv_src=kv_src, kv_dst=kv_dst, row_pool_dst=row_pool_dst,
                reads=reads,
                segments=segments, cu_a=cu_a_arr, max_a=segments["max_q"])
    if timing is not None:
        timing["pack_py"] = timing.get("pack_py", 0.0) + (t1 - t0)
        timing["pack_reads"] = timing.get("pack_reads", 0.0) + (time.perf_counter() - t1)
    return Chunk(input_ids=ids, positions=positions, final_indices=final, meta=meta,
                 attention_mode="tree", tokens=n_tok, layout=layout, row_spans=tuple(row_spans),
                 fresh_keys=tuple(fresh_keys),
                 rows_per_answer=np.concatenate(rows_per_answer) if multi else None,
                 host_ids=ids, host_positions=positions)


def _work_list(tables, heads, choose_rows=False):
    """(work pairs, count, query rows per item) of a paged call over `tables`
    (host arrays). choose_rows: the tile height qx_paged_attention_tile_rows
    picks for these sequences (the call must then pass it); otherwise the
    default (0)."""
    from quail_amd import _lib
    hq, hk, d = heads
    cu_q = np.ascontiguousarray(tables["cu_q"], dtype=np.int32)
    used = np.ascontiguousarray(tables["used"], dtype=np.int32)
    seqs = len(used)
    causal = int(tables.get("causal", True))
    rows = 0
    if choose_rows:
        rows = _lib.count("qx_paged_attention_tile_rows", cu_q.ctypes.data, used.ctypes.data,
                          seqs, hq, hk, d, causal)
    cap = int(cu_q[-1]) + seqs if seqs else 1
    work = np.zeros(2 * max(cap, 1), dtype=np.int32)
    n = _lib.count("qx_paged_attention_work", cu_q.ctypes.data, used.ctypes.data, seqs, hq, hk,
                   d, causal, rows, work.ctypes.data, cap)
    return work[:2 * n], n, rows


def _final_query(cu_q, used, table, final):
    """Attention metadata with one query per final row: final row r of
    sequence s (i = r - cu_q[s], q_len rows) sees the keys [0, used[s] -
    q_len + i + 1) through table[s], so as a one-row sequence it reads
    exactly what it reads inside its own sequence. The last layer needs
    nothing else from the attention."""
    final = np.asarray(final, dtype=np.int64)
    if not len(final):
        return None
    seq = np.searchsorted(cu_q, final, side="right") - 1
    q_len = cu_q[seq + 1] - cu_q[seq]
    visible = (used[seq] - q_len + (final - cu_q[seq]) + 1).astype(np.int32)
    return dict(cu_q=np.arange(len(final) + 1, dtype=np.int32), used=visible,
                table=np.ascontiguousarray(table[seq]), max_q=1,
                max_used=int(visible.max()), causal=True)


# ---- staging ----------------------------------------------------------------

STAGING_DEPTH = 4


class InputStaging:
    """Pinned host buffers in a ring, reused across passes (chunk.py:317-361).

    Each name rotates through STAGING_DEPTH (pinned host, device, event)
    buffers; the host waits only on the upload STAGING_DEPTH passes back.
    """

    def __init__(self, device="cuda"):
        import torch
        self.torch = torch
        self.device = device
        self.rings = {}

    def copy(self, name, values, dtype):
        torch = self.torch
        src = torch.as_tensor(np.ascontiguousarray(values))
        count = src.numel()
        slot, ring = self.rings.get(name, (0, [None] * STAGING_DEPTH))
        entry = ring[slot]
        if entry is not None:
            entry[2].synchronize()
        if entry is None or entry[0].numel() < count or entry[0].dtype != dtype:
            cap = max(count, 64)
            entry = (torch.empty(cap, dtype=dtype, pin_memory=True),
                     torch.empty(cap, dtype=dtype, device=self.device), torch.cuda.Event())
        host, dev, event = entry
        host[:count].copy_(src.reshape(-1))
        dev[:count].copy_(host[:count], non_blocking=True)
        event.record()
        ring[slot] = entry
        self.rings[name] = ((slot + 1) % STAGING_DEPTH, ring)
        return dev[:count].view(src.shape)


def upload(chunk: Chunk, staging: InputStaging) -> Chunk:
    """Move a packed chunk's index arrays to the device (int64 ids/rows, int32 tables)."""
    import torch
    chunk.input_ids = staging.copy("tokens", chunk.host_ids, torch.int64)
    chunk.positions = staging.copy("positions", chunk.host_positions, torch.int64)
    chunk.final_indices = staging.copy("finals", chunk.final_indices, torch.int64)
    if chunk.attention_mode == "tree":
        return _upload_tree(chunk, staging)
    u = chunk.meta["unified"]
    dev = dict(u)
    dev["src"] = staging.copy("unified_src", u["src"], torch.int64)
    dev["dst"] = staging.copy("unified_dst", u["dst"], torch.int64)
    dev["row_dst"] = dev["dst"] if u.get("rows_in_order") else None
    if u["tail_src"] is not None:
        dev["tail_src"] = staging.copy("tail_src", u["tail_src"], torch.int64)
        dev["tail_dst"] = staging.copy("tail_dst", u["tail_dst"], torch.int64)
    dev["used"] = staging.copy("unified_lengths", u["used"], torch.int32)
    dev["cu_q"] = staging.copy("unified_cu_q", u["cu_q"], torch.int32)
    dev["table"] = staging.copy("block_table", u["table"], torch.int32)
    chunk.host["unified"] = u
    chunk.meta["unified"] = dev
    if u.get("work") is not None and u["n_work"]:
        dev["work"] = staging.copy("unified_work", u["work"], torch.int32)
    fq = chunk.meta.get("final_query")
    if fq is not None:
        chunk.host["final_query"] = fq
        chunk.meta["final_query"] = dict(
            fq, cu_q=staging.copy("final_cu_q", fq["cu_q"], torch.int32),
            used=staging.copy("final_used", fq["used"], torch.int32),
            table=staging.copy("final_table", fq["table"], torch.int32))
        if fq.get("work") is not None and fq["n_work"]:
            chunk.meta["final_query"]["work"] = staging.copy("final_work", fq["work"],
                                                             torch.int32)
    chunk.meta["cu_a"] = staging.copy("cu_a", chunk.meta["cu_a"], torch.int32)
    return chunk


def _upload_tree(chunk: Chunk, staging: InputStaging) -> Chunk:
    import torch
    meta = chunk.meta
    chunk.host["segments"], chunk.host["reads"] = meta["segments"], meta["reads"]
    chunk.host["kv_src"], chunk.host["kv_dst"] = meta["kv_src"], meta["kv_dst"]
    if meta["kv_src"] is not None:
        meta["kv_src"] = staging.copy("kv_src", meta["kv_src"], torch.int64)
        meta["kv_dst"] = staging.copy("kv_dst", meta["kv_dst"], torch.int64)
    if meta.get("row_pool_dst") is not None:
        chunk.host["row_pool_dst"] = meta["row_pool_dst"]
        meta["row_pool_dst"] = staging.copy("row_pool_dst", meta["row_pool_dst"], torch.int64)
    seg = meta["segments"]
    dev = dict(seg, cu_q=staging.copy("cu_a", seg["cu_q"], torch.int32),
               used=staging.copy("segment_lengths", seg["used"], torch.int32))
    if seg.get("work") is not None and seg["n_work"]:
        dev["work"] = staging.copy("segment_work", seg["work"], torch.int32)
    meta["segments"] = dev
    meta["cu_a"] = dev["cu_q"]
    reads = meta["reads"]
    if reads is not None:
        dev = dict(reads, rows=staging.copy("read_rows", reads["rows"], torch.int64),
                   cu_q=staging.copy("read_cu_q", reads["cu_q"], torch.int32),
                   used=staging.copy("read_used", reads["used"], torch.int32),
                   table=staging.copy("read_table", reads["table"], torch.int32),
                   source=staging.copy("read_source", reads["source"], torch.int32))
        if reads.get("work") is not None and reads["n_work"]:
            dev["work"] = staging.copy("read_work", reads["work"], torch.int32)
        nodes = reads.get("nodes")
        if nodes is not None:
            dev["nodes"] = dict(
                nodes, rows=staging.copy("node_rows", nodes["rows"], torch.int64),
                key_rows=staging.copy("node_key_rows", nodes["key_rows"], torch.int64),
                cu_q=staging.copy("node_cu_q", nodes["cu_q"], torch.int32),
                cu_k=staging.copy("node_cu_k", nodes["cu_k"], torch.int32),
                used=staging.copy("node_used", nodes["used"], torch.int32),
                b_index=staging.copy("node_b_index", nodes["b_index"], torch.int64),
                gather_rows=staging.copy("node_gather_rows", nodes["gather_rows"], torch.int64))
            if nodes.get("work") is not None and nodes["n_work"]:
                dev["nodes"]["work"] = staging.copy("node_work", nodes["work"], torch.int32)
        meta["reads"] = dev
    return chunk
