"""Paged KV arena on the GPU: per-layer K and V pools in 16-token pages.

The surface the packer and the attention path use, as the reference KVArena
(quail/backends/quail/executor/arena.py:1-24, 35-147, 347-437, 522-563,
644-648, 839-887) defines it for full-attention models: alloc / activate /
alloc_temporary / free_key / pin / retain, residency queries, capacity_rows,
layer_kv / paged_kv and block tables. Sliding-window pools and recurrent
state slots (other model families) are not part of this engine.

HBM layout: one allocation split [k0, v0, k1, v1, ...]; each pool is
(num_pages * page_tokens, num_kv_heads, head_dim) bf16, so page p holds pool
rows p*T .. p*T + T - 1 and a KV row is num_kv_heads * head_dim contiguous
bf16 (2 KiB for Qwen3-4B). At 16 tokens a page is 32 KiB per layer and pool.
"""

import numpy as np
import torch

from quail_amd.pages import PageArena


class _Claim:
    """What keeps a key's pages in the arena: queued borrowers that will
    read them (holds), admissions reading them now (reads), and whether a
    free was asked for meanwhile (done when the last claim goes)."""

    __slots__ = ("holds", "reads", "free_asked")

    def __init__(self):
        self.holds = 0
        self.reads = 0
        self.free_asked = False


class KVArena:
    def __init__(self, num_layers: int, num_pages: int, page_tokens: int, num_kv_heads: int,
                 d_head: int, dtype=torch.bfloat16, device="cuda", v_dtype=torch.float16):
        if dtype != torch.bfloat16 or v_dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("K pages are bf16; V pages bf16 or fp16")
        self.torch = torch
        self.dtype = dtype
        self.v_dtype = v_dtype
        self.device = device
        self.num_layers = num_layers
        self.kv_shape = (num_kv_heads, d_head)
        self.sliding_layers = frozenset()
        self.has_sliding = False
        self.num_state_slots = 0
        self._build(num_pages, page_tokens)
        self.evicted_keys = 0
        self.evicted_pages = 0
        self.evicted_prefix_tokens = 0

    def _build(self, num_pages, page_tokens):
        heads, dim = self.kv_shape
        self.accounting = PageArena(num_pages, page_tokens)
        rows = num_pages * page_tokens
        size = rows * heads * dim
        storage = torch.empty(2 * self.num_layers * size, dtype=self.dtype, device=self.device)
        parts = storage.split([size] * (2 * self.num_layers))
        self.k = [p.view(rows, heads, dim) for p in parts[0::2]]
        # V pages: bf16 as the reference's arena holds them, or fp16 (the
        # default here: the same 16-bit slots; bf16 V rows are converted once,
        # when written, and the PV product then keeps 11 bits of each
        # probability instead of 8)
        self.v = [p.view(self.v_dtype).view(rows, heads, dim) for p in parts[1::2]]
        self._claims = {}

    # ---- sizes -------------------------------------------------------------

    @property
    def page_tokens(self) -> int:
        return self.accounting.page_tokens

    @property
    def num_pages(self) -> int:
        return self.accounting.num_pages

    @property
    def free_pages(self) -> int:
        return self.accounting.free_pages

    @property
    def retained_pages(self) -> int:
        return self.accounting.retained_pages

    def pages_needed(self, tokens: int) -> int:
        return self.accounting.pages_needed(tokens)

    def page_cost(self, tokens: int, sliding_tokens: int = 0) -> int:
        return self.accounting.pages_needed(tokens)

    # ---- residency ---------------------------------------------------------

    def is_resident(self, key) -> bool:
        return self.accounting.is_resident(key)

    def resident_keys(self):
        return self.accounting.resident_keys()

    def owned_pages(self, key) -> list:
        """The page ids the key's block table reads: borrowed, then its own."""
        return self.accounting.table_pages(key)

    def tokens(self, key) -> int:
        return self.accounting.key_tokens(key)

    def capacity_rows(self, key) -> np.ndarray:
        """Pool row of every row in the key's pages, in logical order (host int64)."""
        pages = np.asarray(self.accounting.table_pages(key), dtype=np.int64)
        t = self.page_tokens
        return (pages[:, None] * t + np.arange(t, dtype=np.int64)).reshape(-1)

    # ---- allocation ----------------------------------------------------------

    def _borrow_plan(self, borrow):
        if borrow is None:
            return []
        parent, shared = borrow
        return self.accounting.shared_pages(parent, shared)

    def can_borrow(self, parent, shared: int) -> bool:
        acct = self.accounting
        return acct.is_resident(parent) and shared <= acct.key_tokens(parent)

    def alloc(self, key, tokens: int, capacity_tokens=None, base_tokens=None, borrow=None):
        """Pages for a fresh key, or None when the free list is short.
        borrow = (parent key, shared tokens): the key reads the parent's
        first pages as its own leading pages."""
        return self.accounting.alloc(key, tokens, capacity_tokens,
                                     borrowed=self._borrow_plan(borrow))

    def _evict_until(self, satisfied) -> tuple:
        """Free retained keys in the accounting's victim order until
        satisfied() holds (arena.py:478-492); a key a queued borrower will
        read (held) or that an admission is reading is never a victim.
        Returns the evicted keys."""
        acct = self.accounting
        keep = frozenset(self._claims)
        keys = []
        while not satisfied():
            victim = acct.pop_retained_victim(keep=keep)
            if victim is None:
                break
            key, _, tokens = victim
            self.evicted_keys += 1
            self.evicted_prefix_tokens += tokens
            self.evicted_pages += self.free_key(key)
            keys.append(key)
        return tuple(keys)

    def _evict_for_pages(self, need: int) -> None:
        self._evict_until(lambda: self.accounting.free_pages >= need)

    def evict_retained(self, pages_needed: int) -> tuple:
        """Free retained keys until pages_needed pages have come free
        (arena.py:468-476). Returns the evicted keys."""
        start = self.accounting.free_pages
        return self._evict_until(lambda: self.accounting.free_pages - start >= pages_needed)

    def reserve(self, key, tokens: int, *, capacity_tokens: int, borrow=None,
                extension=False, share_points=()) -> bool:
        """Pages for an admitted document (arena.py:584-642): retained KV is
        evicted until its capacity fits, never the document's own pages or
        the parent it borrows from; then it is activated (pinned). False
        leaves it as it was (evictions may have happened)."""
        acct = self.accounting
        if acct.is_resident(key):
            held = len(acct.table_pages(key))
        else:
            held = len(self._borrow_plan(borrow))
        need = max(0, acct.pages_needed(capacity_tokens) - held)
        protected = (key,) if borrow is None else (key, borrow[0])
        self.read_state(protected)
        try:
            self._evict_until(lambda: acct.free_pages >= need)
            if acct.free_pages < need:
                return False
            return self.activate(key, tokens, capacity_tokens=capacity_tokens,
                                 borrow=borrow) is not None
        finally:
            self.done_reading(protected)

    def activate(self, key, tokens: int, capacity_tokens=None, base_tokens=None, borrow=None):
        """Make a prefix active (pinned), evicting retained KV when needed."""
        acct = self.accounting
        capacity = tokens if capacity_tokens is None else capacity_tokens
        if acct.is_resident(key):
            acct.pin(key)
            need = max(0, acct.pages_needed(capacity) - len(acct.table_pages(key)))
            self._evict_for_pages(need)
            if need > acct.free_pages:
                return None
            acct.grow(key, capacity)
            acct.set_tokens(key, tokens)
            return acct.owned_pages(key)
        borrowed = self._borrow_plan(borrow)
        self._evict_for_pages(acct.pages_needed(capacity) - len(borrowed))
        pages = self.alloc(key, tokens, capacity, base_tokens, borrow=borrow)
        if pages is not None:
            acct.pin(key)
        return pages

    def alloc_temporary(self, tokens: int, sliding_tokens=None):
        key = object()
        pages = self.alloc(key, tokens, base_tokens=0)
        return None if pages is None else (key, pages)

    def free_key(self, key) -> int:
        """Free a key's pages, or once its holds and reads are over (a key
        queued borrowers will read, or that an admission reads, waits for
        them). Returns the pages that went free now."""
        claim = self._claims.get(key)
        if claim is not None:
            claim.free_asked = True
            return 0
        return self.accounting.free_key(key)

    def pin(self, key) -> None:
        self.accounting.pin(key)

    def retain(self, key, tokens=None, priority=None) -> None:
        """Keep a key's first `tokens` (all of them by default) for a later
        operator; it becomes evictable."""
        if tokens is not None:
            self.accounting.rewind(key, tokens)
        self.accounting.retain(key, priority)

    # ---- holds and reads: keys that admitted or queued readers need -------------

    def _claim(self, key) -> "_Claim":
        claim = self._claims.get(key)
        if claim is None:
            claim = self._claims[key] = _Claim()
        return claim

    def _settle(self, key) -> None:
        """Forget a key's claim once nothing keeps it; free its pages then
        if a free was asked for while it was kept."""
        claim = self._claims[key]
        if claim.holds or claim.reads:
            return
        del self._claims[key]
        if claim.free_asked:
            self.accounting.free_key(key)

    def hold(self, key, borrowers: int) -> None:
        """Keep a key for `borrowers` documents that will read its pages."""
        if borrowers:
            self._claim(key).holds += borrowers

    def release(self, key) -> None:
        """One borrower of the key was admitted, or will not come."""
        claim = self._claims.get(key)
        if claim is not None and claim.holds:
            claim.holds -= 1
            self._settle(key)

    def drop_holds(self, keys=None) -> bool:
        """Release every hold on the keys (all by default): freed keys go
        free, retained ones become evictable. True when any hold went."""
        pool = self._claims if keys is None else keys
        held = [k for k in pool if k in self._claims and self._claims[k].holds]
        for key in held:
            self._claims[key].holds = 0
            self._settle(key)
        return bool(held)

    def read_state(self, keys) -> None:
        """Keep each key's pages until done_reading for the same keys."""
        for key in keys:
            self._claim(key).reads += 1

    def done_reading(self, keys) -> None:
        for key in keys:
            self._claims[key].reads -= 1
            self._settle(key)

    def origin(self, tokens: int) -> int:
        """The first row a key's pages must hold for a borrower of `tokens`
        rows: 0 (every layer keeps every row; no sliding window)."""
        return 0

    def keep_window(self, key, shared: int) -> None:
        """No sliding window: every row a borrower reads stays."""

    # ---- tensors read by attention ---------------------------------------------

    def layer_kv(self, layer: int):
        """Flat K and V pools of one layer: (rows, num_kv_heads, head_dim)."""
        return self.k[layer], self.v[layer]

    def paged_kv(self, layer: int):
        heads, dim = self.kv_shape
        shape = (-1, self.page_tokens, heads, dim)
        return self.k[layer].view(shape), self.v[layer].view(shape)

    def block_table_rows(self, pages, pad_to=None) -> np.ndarray:
        """(len(pages), width) int32 table, each row zero-padded on the right."""
        width = max(len(p) for p in pages)
        if pad_to:
            width = max(width, pad_to)
        table = np.zeros((len(pages), width), dtype=np.int32)
        for row, p in enumerate(pages):
            table[row, :len(p)] = p
        return table

    def block_table(self, keys, pad_to=None):
        table = self.block_table_rows([self.owned_pages(k) for k in keys], pad_to)
        used = np.asarray([self.accounting.key_tokens(k) for k in keys], dtype=np.int32)
        return table, used
