"""Page accounting restated in plain Python: the oracle of the C++ page pool.

Test infrastructure (see oracle/__init__.py). It follows the reference
PageArena (quail/backends/quail/executor/pages.py:8-275) step by step:

  * the free list is a stack initialised [P-1, ..., 1, 0], so the first
    allocations take pages 0, 1, 2, ... in order (pages.py:26);
  * a key owns the pages it writes and may borrow the leading pages of a
    resident key; its table is borrowed pages then its own (pages.py:96-98);
  * a page goes back on the stack when its last holder releases it, in the
    order the releasing list names it (pages.py:103-109);
  * retention keeps freed documents evictable by a priority heap
    (pages.py:191-250).

Pinned by the reference's known answers (tests/engine/test_arena.py:10-138,
restated in tests/test_pages.py, which runs them on this class and on the
product) and by the invariant that no page is double-owned or leaked.
`RefArena` adds the KVArena surface the packer reads (arena.py:106-147,
522-563, 839-887) without device tensors.
"""

import heapq

import numpy as np


class RefPageArena:
    def __init__(self, num_pages: int, page_tokens: int):
        self.num_pages = num_pages
        self.page_tokens = page_tokens
        self.free = list(range(num_pages - 1, -1, -1))
        self.owned = {}
        self.borrowed = {}
        self.holds = np.zeros(num_pages, dtype=np.int32)
        self.tokens = {}
        self.pinned = set()
        self.retained = {}
        self._retained_sizes = {}
        self._retained_pages = 0
        self._heap = []
        self._versions = {}
        self._version = 0

    # ---- sizes -----------------------------------------------------------

    def pages_needed(self, tokens: int) -> int:
        return -(-tokens // self.page_tokens)

    @property
    def free_pages(self) -> int:
        return len(self.free)

    @property
    def resident_tokens(self) -> int:
        return sum(self.tokens.values())

    @property
    def retained_pages(self) -> int:
        return self._retained_pages

    @property
    def retained_prefix_tokens(self) -> int:
        return sum(self.tokens[k] for k in self.retained)

    # ---- allocation ------------------------------------------------------

    def alloc(self, key, tokens: int, capacity_tokens=None, borrowed=()):
        """Own pages for a new key, or None when the free stack is short."""
        if key in self.owned:
            raise KeyError(f"{key!r} already resident")
        capacity = tokens if capacity_tokens is None else capacity_tokens
        if capacity < tokens:
            raise ValueError("capacity_tokens must cover logical tokens")
        borrowed = list(borrowed)
        if len(borrowed) * self.page_tokens > tokens:
            raise ValueError("a key cannot borrow past its own tokens")
        need = self.pages_needed(capacity) - len(borrowed)
        if need > len(self.free):
            return None
        pages = [self.free.pop() for _ in range(need)]
        self.owned[key] = pages
        self.borrowed[key] = borrowed
        self.tokens[key] = tokens
        self.holds[borrowed + pages] += 1
        return pages

    def shared_pages(self, parent, shared: int, start: int = 0) -> list:
        """The parent's pages holding its tokens [start, shared) (whole pages)."""
        if start % self.page_tokens or (shared - start) % self.page_tokens:
            raise ValueError("a borrowed prefix is a whole number of pages")
        if parent not in self.owned:
            raise KeyError(f"borrow parent {parent!r} is not resident")
        if shared > self.tokens[parent]:
            raise ValueError(f"{parent!r} holds fewer tokens than borrowed")
        table = self.table_pages(parent)
        return table[start // self.page_tokens:shared // self.page_tokens]

    def table_pages(self, key) -> list:
        return self.borrowed[key] + self.owned[key]

    def borrowed_tokens(self, key) -> int:
        return len(self.borrowed[key]) * self.page_tokens

    def release_pages(self, pages) -> int:
        """Drop one hold per page; pages reaching zero go back on the stack."""
        pages = np.asarray(pages, dtype=np.int64)
        if pages.size == 0:
            return 0
        self.holds[pages] -= 1
        freed = pages[self.holds[pages] == 0]
        self.free.extend(int(p) for p in freed)
        return int(freed.size)

    def drop_leading(self, key, pages: int) -> int:
        b = self.borrowed[key]
        take_b = min(pages, len(b))
        dropped = b[:take_b] + self.owned[key][:pages - take_b]
        self.borrowed[key] = b[take_b:]
        self.owned[key] = self.owned[key][pages - take_b:]
        return self.release_pages(dropped)

    def free_key(self, key) -> int:
        pages = self.owned.pop(key)
        borrowed = self.borrowed.pop(key)
        self.tokens.pop(key)
        self.pinned.discard(key)
        self._forget(key)
        return self.release_pages(borrowed + pages)

    def rewind(self, key, tokens: int) -> int:
        if key not in self.owned:
            raise KeyError(key)
        low = self.borrowed_tokens(key)
        high = low + len(self.owned[key]) * self.page_tokens
        if tokens < low or tokens > high:
            raise ValueError("rewind tokens leave the resident capacity")
        keep = self.pages_needed(tokens) - len(self.borrowed[key])
        released = self.owned[key][keep:]
        self.owned[key] = self.owned[key][:keep]
        self.tokens[key] = tokens
        freed = self.release_pages(released)
        if key in self.retained:
            self.retain(key)
        return freed

    def grow(self, key, capacity_tokens: int):
        if key not in self.owned:
            raise KeyError(key)
        need = (self.pages_needed(capacity_tokens) - len(self.borrowed[key])
                - len(self.owned[key]))
        if need <= 0:
            return 0
        if need > len(self.free):
            return None
        added = [self.free.pop() for _ in range(need)]
        self.owned[key].extend(added)
        self.holds[added] += 1
        return need

    def row_indices(self, key, tokens=None):
        """Flat pool rows of the key's tokens: page p holds rows p*T .. p*T+T-1."""
        left = self.tokens[key] if tokens is None else tokens
        rows = []
        for p in self.table_pages(key):
            take = min(left, self.page_tokens)
            rows.extend(range(p * self.page_tokens, p * self.page_tokens + take))
            left -= take
        return rows

    # ---- pins and retention ------------------------------------------------

    def pin(self, key) -> None:
        if key not in self.owned:
            raise KeyError(key)
        self._forget(key)
        self.pinned.add(key)

    def _forget(self, key):
        self._retained_pages -= self._retained_sizes.pop(key, 0)
        self.retained.pop(key, None)
        self._versions.pop(key, None)

    def retain(self, key, priority=None) -> None:
        """Make a resident key evictable; priority defaults to tokens per
        page it alone holds (higher is kept longer)."""
        if key not in self.owned:
            raise KeyError(key)
        self.pinned.discard(key)
        tokens = self.tokens[key]
        self._forget(key)
        alone = int((self.holds[self.table_pages(key)] == 1).sum())
        self.retained[key] = tokens
        self._retained_sizes[key] = alone
        self._retained_pages += alone
        self._version += 1
        self._versions[key] = self._version
        if priority is None:
            priority = (tokens / max(1, alone),)
        heapq.heappush(self._heap, (priority, self._version, key, alone, tokens))

    def pop_retained_victim(self, keep=frozenset()):
        passed, victim = [], None
        while self._heap:
            entry = heapq.heappop(self._heap)
            _, version, key, pages, tokens = entry
            if self._versions.get(key) != version:
                continue
            if key in keep:
                passed.append(entry)
                continue
            self._forget(key)
            victim = (key, pages, tokens)
            break
        for entry in passed:
            heapq.heappush(self._heap, entry)
        return victim


class RefArena:
    """KVArena's host surface over RefPageArena (no tensors)."""

    def __init__(self, num_pages: int, page_tokens: int):
        self.accounting = RefPageArena(num_pages, page_tokens)
        self.page_tokens = page_tokens

    @property
    def free_pages(self) -> int:
        return self.accounting.free_pages

    def pages_needed(self, tokens: int) -> int:
        return self.accounting.pages_needed(tokens)

    def is_resident(self, key) -> bool:
        return key in self.accounting.owned

    def owned_pages(self, key) -> list:
        return self.accounting.table_pages(key)

    def capacity_rows(self, key) -> np.ndarray:
        pages = np.asarray(self.accounting.table_pages(key), dtype=np.int64)
        t = self.page_tokens
        return (pages[:, None] * t + np.arange(t, dtype=np.int64)).reshape(-1)

    def activate(self, key, tokens: int, capacity_tokens=None, borrow=None):
        borrowed = [] if borrow is None else self.accounting.shared_pages(*borrow)
        pages = self.accounting.alloc(key, tokens, capacity_tokens, borrowed=borrowed)
        if pages is not None:
            self.accounting.pin(key)
        return pages

    def alloc_temporary(self, tokens: int):
        key = object()
        pages = self.accounting.alloc(key, tokens)
        return None if pages is None else (key, pages)

    def free_key(self, key) -> int:
        return self.accounting.free_key(key)

    def block_table_rows(self, pages) -> np.ndarray:
        width = max(len(p) for p in pages)
        table = np.zeros((len(pages), width), dtype=np.int32)
        for row, p in enumerate(pages):
            table[row, :len(p)] = p
        return table
