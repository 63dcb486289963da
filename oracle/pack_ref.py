"""The unified pack layout restated in plain Python: the oracle of the C++
packer (qx_pack_unified).

Test infrastructure (see oracle/__init__.py). It follows the reference's
pack_chunk with attention_mode="unified"
(quail/backends/quail/executor/chunk.py:505-1160: the group loop :606-684,
the unified pools :913-1054, _PoolBuilder :407-502) over an arena with the
KVArena surface (oracle.pages_ref.RefArena):

  * a group's rows are [prefix | suffix, suffix, ...]; positions continue
    from `start` through the prefix and restart at `f` for every suffix;
  * a group with one suffix whose key's pages cover start + its rows is one
    sequence scattered straight into the key's pages (used = f + suffix);
  * otherwise the prefix is a sequence (used = f) and each suffix gets a
    temporary key whose pages follow the key's full pages, a partial last
    page of the prefix copied into the temporary first (the tail copy).

Pinned by the reference's known answers (tests/engine/test_pack_chunk.py
:16-51,149-175, restated in tests/test_pack.py) and by the structural KV-read
check of oracle.packing_ref over seeded corpora.
"""

import numpy as np


class ArenaFullError(RuntimeError):
    """The arena has too few free pages for the pack's temporaries."""


def _as_suffixes(sufs):
    arrays = [np.asarray(s, dtype=np.int64) for s in sufs]
    lengths = np.asarray([len(a) for a in arrays], dtype=np.int64)
    ids = np.concatenate(arrays) if arrays else np.empty(0, dtype=np.int64)
    return ids, lengths


def _cat(parts, dtype=np.int64):
    parts = [np.asarray(p, dtype=dtype) for p in parts if len(p)]
    return np.concatenate(parts) if parts else np.empty(0, dtype=dtype)


def pack_unified_ref(arena, groups):
    """The unified causal layout of one pack, as dict of host arrays and
    lists (the fields of the product's Chunk and meta["unified"])."""
    id_parts, pos_parts, finals, cu_a = [], [], [], [0]
    rows_per_answer, multi = [], False
    layout, row_spans, fresh_keys, specs = [], [], [], []
    n_tok = 0
    for g in groups:
        key = g["key"]
        fresh = g.get("prefix") is not None
        f = int(g["f"])
        start = int(g.get("start", 0))
        paged = arena.is_resident(key)
        if not paged:
            raise ValueError(f"group {key!r}: the paged unified path needs arena pages")
        row0 = n_tok
        sids, slen = _as_suffixes(g["suffixes"])
        n = len(slen)
        if fresh:
            prefix = np.asarray(g["prefix"], dtype=np.int64)
            id_parts.append(prefix)
            pos_parts.append(np.arange(start, start + len(prefix), dtype=np.int64))
            n_tok += len(prefix)
            cu_a.append(n_tok)
        prefix_end = n_tok
        s_row0 = n_tok
        read_all = bool(g.get("read_all_rows"))
        total = int(slen.sum())
        ends = np.cumsum(slen)
        begins = ends - slen
        if n:
            id_parts.append(sids)
            within = np.arange(total, dtype=np.int64) - np.repeat(begins, slen)
            pos_parts.append(f + within)
            cu_a.extend((s_row0 + ends).tolist())
            if read_all:
                finals.append(np.arange(s_row0, s_row0 + total, dtype=np.int64))
                rows_per_answer.append(slen)
                multi = True
            else:
                finals.append(s_row0 + ends - 1)
                rows_per_answer.append(np.ones(n, dtype=np.int64))
            n_tok += total
        layout.append((key, n))
        row_spans.append((key, row0, prefix_end, n_tok))
        specs.append(dict(key=key, fresh=fresh, f=f, start=start, row0=row0,
                          prefix_end=prefix_end, row1=n_tok,
                          begins=s_row0 + begins, ends=s_row0 + ends,
                          keeps=int(g.get("write_suffix_tokens") or 0)))

    page = arena.page_tokens
    src, dst, tail_src, tail_dst = [], [], [], []
    seq_pages, seq_used, cu_q = [], [], [0]
    temporary_keys = []
    try:
        for spec in specs:
            key, f = spec["key"], spec["f"]
            r0, r1 = spec["row0"], spec["row1"]
            begins, ends = spec["begins"], spec["ends"]
            logical = spec["start"] if spec["fresh"] else f
            if spec["fresh"]:
                fresh_keys.append(key)
            count = r1 - r0
            rows = arena.capacity_rows(key)
            pages = arena.owned_pages(key)
            suffix_total = int((ends - begins).sum())
            direct = len(begins) == 1 and logical + count <= rows.size
            if spec["keeps"] and not direct:
                raise ValueError(f"group {key!r} keeps suffix KV but its pages hold "
                                 f"{rows.size} rows, not {logical + count}")
            if direct:
                src.append(np.arange(r0, r1, dtype=np.int64))
                dst.append(rows[logical:logical + count])
                seq_pages.append(list(pages))
                seq_used.append(f + suffix_total)
                cu_q.append(cu_q[-1] + count)
                continue
            n_prefix = spec["prefix_end"] - r0
            if n_prefix:
                src.append(np.arange(r0, spec["prefix_end"], dtype=np.int64))
                dst.append(rows[spec["start"]:spec["start"] + n_prefix])
                seq_pages.append(list(pages[:arena.pages_needed(f)]))
                seq_used.append(f)
                cu_q.append(cu_q[-1] + n_prefix)
            remainder = f % page
            for s0, s1 in zip(begins.tolist(), ends.tolist()):
                got = arena.alloc_temporary(remainder + (s1 - s0))
                if got is None:
                    raise ArenaFullError(
                        f"unified suffix pages exceed the free KV arena (asked "
                        f"{remainder + s1 - s0} rows, free pages {arena.free_pages})")
                temp, _ = got
                temporary_keys.append(temp)
                trows = arena.capacity_rows(temp)
                src.append(np.arange(s0, s1, dtype=np.int64))
                dst.append(trows[remainder:remainder + (s1 - s0)])
                if remainder:
                    base = pages[f // page] * page
                    tail_src.append(np.arange(base, base + remainder, dtype=np.int64))
                    tail_dst.append(trows[:remainder])
                seq_pages.append(list(pages[:f // page]) + arena.owned_pages(temp))
                seq_used.append(f + (s1 - s0))
                cu_q.append(cu_q[-1] + (s1 - s0))
    except Exception:
        for temp in temporary_keys:
            arena.free_key(temp)
        raise

    used = np.asarray(seq_used, dtype=np.int32)
    table = arena.block_table_rows(seq_pages) if seq_pages else np.zeros((0, 1), np.int32)
    cu_q_arr = np.asarray(cu_q, dtype=np.int32)
    unified = dict(
        src=_cat(src), dst=_cat(dst),
        tail_src=_cat(tail_src) if tail_src else None,
        tail_dst=_cat(tail_dst) if tail_dst else None,
        used=used, table=table, cu_q=cu_q_arr, cu_q_host=list(cu_q),
        used_host=used.tolist(), page_rows=seq_pages,
        max_q=int(np.diff(cu_q_arr).max()) if len(cu_q) > 1 else 0,
        max_used=int(used.max()) if len(used) else 0, causal=True)
    cu_a_arr = np.asarray(cu_a, dtype=np.int32)
    return dict(ids=_cat(id_parts), positions=_cat(pos_parts), finals=_cat(finals),
                cu_a=cu_a_arr, unified=unified, tokens=n_tok, layout=layout,
                row_spans=tuple(row_spans), temporary_keys=tuple(temporary_keys),
                fresh_keys=tuple(fresh_keys),
                rows_per_answer=np.concatenate(rows_per_answer) if multi else None)
