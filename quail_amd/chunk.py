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
cu_q_host, used_host, page_rows}. Host arrays are numpy; `upload` moves
them to the device in one pinned staging copy per array.
"""

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


def _as_suffixes(sufs):
    arrays = [np.asarray(s, dtype=np.int64) for s in sufs]
    lengths = np.asarray([len(a) for a in arrays], dtype=np.int64)
    ids = np.concatenate(arrays) if arrays else np.empty(0, dtype=np.int64)
    return ids, lengths


def _cat(parts, dtype=np.int64):
    parts = [np.asarray(p, dtype=dtype) for p in parts if len(p)]
    return np.concatenate(parts) if parts else np.empty(0, dtype=dtype)


def pack_chunk(arena, groups, *, attention_mode="unified", mask="causal", timing=None,
               attention_heads=None):
    """Pack groups for one unified causal forward pass (host arrays only).

    attention_heads: (HQ, HK, D) of the model; with it the attention
    metadata also carries the work list of the paged calls (one item per
    query tile that holds rows, heaviest first, qx_paged_attention_work).

    Raises ValueError for layouts this path does not run and ArenaFullError
    when the suffixes' temporary pages do not fit (temporaries allocated so
    far are freed first).
    """
    if attention_mode != "unified":
        raise ValueError("this engine packs the unified attention path")
    if mask != "causal":
        raise ValueError("this engine packs the causal mask")
    t0 = time.perf_counter()
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
    t1 = time.perf_counter()

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
    ids = _cat(id_parts)
    positions = _cat(pos_parts)
    final = _cat(finals)
    meta = dict(layer=0, unified=unified, cu_a=cu_a_arr,
                max_a=int(np.diff(cu_a_arr).max()) if len(cu_a) > 1 else 0,
                final_query=_final_query(cu_q_arr, used, table, final))
    if attention_heads is not None:
        for tables in (unified, meta["final_query"]):
            if tables is not None:
                tables["work"], tables["n_work"] = _work_list(tables, attention_heads)
    if timing is not None:
        timing["pack_py"] = timing.get("pack_py", 0.0) + (t1 - t0)
        timing["pack_unified"] = timing.get("pack_unified", 0.0) + (time.perf_counter() - t1)
    return Chunk(input_ids=ids, positions=positions, final_indices=final, meta=meta,
                 attention_mode="unified", tokens=n_tok, layout=layout,
                 row_spans=tuple(row_spans), temporary_keys=tuple(temporary_keys),
                 fresh_keys=tuple(fresh_keys),
                 rows_per_answer=np.concatenate(rows_per_answer) if multi else None,
                 host_ids=ids, host_positions=positions)


def _work_list(tables, heads):
    """(work pairs, count) of a paged call over `tables` (host arrays)."""
    from quail_amd import _lib
    hq, hk, d = heads
    cu_q = np.ascontiguousarray(tables["cu_q"], dtype=np.int32)
    used = np.ascontiguousarray(tables["used"], dtype=np.int32)
    seqs = len(used)
    cap = int(cu_q[-1]) + seqs if seqs else 1
    work = np.zeros(2 * max(cap, 1), dtype=np.int32)
    n = _lib.count("qx_paged_attention_work", cu_q.ctypes.data, used.ctypes.data, seqs, hq, hk,
                   d, int(tables.get("causal", True)), work.ctypes.data, cap)
    return work[:2 * n], n


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
    u = chunk.meta["unified"]
    chunk.input_ids = staging.copy("tokens", chunk.host_ids, torch.int64)
    chunk.positions = staging.copy("positions", chunk.host_positions, torch.int64)
    chunk.final_indices = staging.copy("finals", chunk.final_indices, torch.int64)
    dev = dict(u)
    dev["src"] = staging.copy("unified_src", u["src"], torch.int64)
    dev["dst"] = staging.copy("unified_dst", u["dst"], torch.int64)
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
