"""Page accounting of the KV arena: a free-page stack and per-key page lists.

The accounting runs in C++ (`csrc/host_pack.cpp`, qx_pages_*), where the
packer (quail_amd.chunk.pack_chunk) reads it without a Python round trip per
group. This class is its Python face, with the interface of the reference
PageArena (quail/backends/quail/executor/pages.py:8-275), whose behaviour
fixes the page ids every block table holds, so tables built here match the
reference's bit for bit:

  * the free list is a stack initialised [P-1, ..., 1, 0], so the first
    allocations take pages 0, 1, 2, ... in order (pages.py:26);
  * a key owns the pages it writes and may borrow the leading pages of a
    resident key; its table is borrowed pages then its own (pages.py:96-98);
  * a page goes back on the stack when its last holder releases it, in the
    order the releasing list names it (pages.py:103-109);
  * retention keeps freed documents evictable by a priority heap, lowest
    priority first, ties in the order they were retained (pages.py:191-250).

Keys are any hashable Python values; the C++ side knows them by integer
ids (positive for keys made here, negative for the temporary keys the
packer allocates, which `adopt` names on the Python side).
"""

import ctypes
import itertools

from quail_amd import _lib

ENOKEY, EEXISTS, EFULL = -2, -3, -4


class TemporaryKey:
    """A temporary key the packer allocated (one suffix's pages)."""

    __slots__ = ("id",)

    def __init__(self, ident: int):
        self.id = ident

    def __repr__(self):
        return f"TemporaryKey({self.id})"


def _pages_call(name, *args):
    """Call a qx_pages_* entry point; a missing key raises KeyError, an
    argument error ValueError."""
    lib = _lib.load()
    rc = getattr(lib, name)(*args)
    if rc == 0:
        return
    msg = lib.qx_last_error().decode(errors="replace")
    if rc in (ENOKEY, EEXISTS):
        raise KeyError(msg)
    if rc == -1:
        raise ValueError(msg)
    raise _lib.QxError(f"{name}: {msg}")


class PageArena:
    def __init__(self, num_pages: int, page_tokens: int):
        self.num_pages = num_pages
        self.page_tokens = page_tokens
        handle = ctypes.c_void_p()
        _lib.call("qx_pages_create", num_pages, page_tokens, ctypes.byref(handle))
        self.handle = handle
        self._lib = _lib.load()
        self._ids = {}          # key -> id
        self._keys = {}         # id -> key
        self._next = itertools.count(1)
        self._buf = (ctypes.c_int32 * max(1, num_pages))()
        self._info = (ctypes.c_int64 * 6)()
        self._out = ctypes.c_int64()

    def __del__(self):
        handle = getattr(self, "handle", None)
        if handle is not None and handle.value and _lib is not None:
            try:
                _lib.load().qx_pages_destroy(handle)
            except Exception:
                pass
            self.handle = None

    # ---- ids -------------------------------------------------------------

    def key_id(self, key) -> int:
        """The C++ id of a resident key (KeyError when it is not resident)."""
        if isinstance(key, TemporaryKey):
            if key.id not in self._keys:
                raise KeyError(key)
            return key.id
        return self._ids[key]

    def adopt(self, ident: int) -> TemporaryKey:
        """Name a temporary key the packer allocated."""
        key = TemporaryKey(ident)
        self._keys[ident] = key
        return key

    def _drop(self, ident: int) -> None:
        key = self._keys.pop(ident)
        if not isinstance(key, TemporaryKey):
            del self._ids[key]

    # ---- sizes -------------------------------------------------------------

    def pages_needed(self, tokens: int) -> int:
        return -(-tokens // self.page_tokens)

    def _stats(self):
        stats = (ctypes.c_int64 * 5)()
        _pages_call("qx_pages_stats", self.handle, stats)
        return stats

    @property
    def free_pages(self) -> int:
        return self._stats()[0]

    @property
    def resident_tokens(self) -> int:
        return self._stats()[2]

    @property
    def retained_pages(self) -> int:
        return self._stats()[1]

    @property
    def retained_prefix_tokens(self) -> int:
        return self._stats()[3]

    # ---- per-key state -------------------------------------------------------

    def is_resident(self, key) -> bool:
        if isinstance(key, TemporaryKey):
            return key.id in self._keys
        return key in self._ids

    def _table(self, key):
        """(tokens, borrowed pages, owned pages, pinned, retained)."""
        ident = self.key_id(key)
        _pages_call("qx_pages_table", self.handle, ident, self._buf, len(self._buf), self._info)
        t, nb, no, pinned, retained = list(self._info)[:5]
        pages = self._buf[:nb + no]
        return t, pages[:nb], pages[nb:], bool(pinned), bool(retained)

    def table_pages(self, key) -> list:
        _, borrowed, owned, _, _ = self._table(key)
        return borrowed + owned

    def owned_pages(self, key) -> list:
        return self._table(key)[2]

    def borrowed_pages(self, key) -> list:
        return self._table(key)[1]

    def key_tokens(self, key) -> int:
        return self._table(key)[0]

    def set_tokens(self, key, tokens: int) -> None:
        _pages_call("qx_pages_set_tokens", self.handle, self.key_id(key), tokens)

    def borrowed_tokens(self, key) -> int:
        return len(self._table(key)[1]) * self.page_tokens

    def resident_keys(self) -> list:
        n = ctypes.c_int64()
        _pages_call("qx_pages_keys", self.handle, None, 0, ctypes.byref(n))
        ids = (ctypes.c_int64 * max(1, n.value))()
        _pages_call("qx_pages_keys", self.handle, ids, n.value, ctypes.byref(n))
        return [self._keys[i] for i in ids[:n.value]]

    def free_list(self) -> list:
        """The free stack, bottom first (the last entry is handed out next)."""
        n = ctypes.c_int64()
        _pages_call("qx_pages_free_list", self.handle, self._buf, len(self._buf),
                    ctypes.byref(n))
        return self._buf[:n.value]

    # views of the whole state, keyed like the reference's dictionaries
    @property
    def owned(self) -> dict:
        return {k: self.owned_pages(k) for k in self.resident_keys()}

    @property
    def borrowed(self) -> dict:
        return {k: self.borrowed_pages(k) for k in self.resident_keys()}

    @property
    def tokens(self) -> dict:
        return {k: self.key_tokens(k) for k in self.resident_keys()}

    @property
    def pinned(self) -> set:
        return {k for k in self.resident_keys() if self._table(k)[3]}

    @property
    def retained(self) -> dict:
        return {k: t for k in self.resident_keys()
                for t, _, _, _, kept in [self._table(k)] if kept}

    # ---- allocation ------------------------------------------------------

    def alloc(self, key, tokens: int, capacity_tokens=None, borrowed=()):
        """Own pages for a new key, or None when the free stack is short."""
        if self.is_resident(key):
            raise KeyError(f"{key!r} already resident")
        capacity = tokens if capacity_tokens is None else capacity_tokens
        borrowed = list(borrowed)
        arr = (ctypes.c_int32 * max(1, len(borrowed)))(*borrowed)
        ident = next(self._next)
        _pages_call("qx_pages_alloc", self.handle, ident, tokens, capacity, arr, len(borrowed),
                    ctypes.byref(self._out))
        if self._out.value < 0:
            return None
        self._ids[key] = ident
        self._keys[ident] = key
        return self.owned_pages(key)

    def shared_pages(self, parent, shared: int, start: int = 0) -> list:
        """The parent's pages holding its tokens [start, shared) (whole pages)."""
        if not self.is_resident(parent):
            raise KeyError(f"borrow parent {parent!r} is not resident")
        _pages_call("qx_pages_shared", self.handle, self.key_id(parent), shared, start,
                    self._buf, len(self._buf), ctypes.byref(self._out))
        return self._buf[:self._out.value]

    def drop_leading(self, key, pages: int) -> int:
        _pages_call("qx_pages_drop_leading", self.handle, self.key_id(key), pages,
                    ctypes.byref(self._out))
        return self._out.value

    def free_key(self, key) -> int:
        ident = self.key_id(key)
        _pages_call("qx_pages_free_key", self.handle, ident, ctypes.byref(self._out))
        self._drop(ident)
        return self._out.value

    def rewind(self, key, tokens: int) -> int:
        _pages_call("qx_pages_rewind", self.handle, self.key_id(key), tokens,
                    ctypes.byref(self._out))
        return self._out.value

    def grow(self, key, capacity_tokens: int):
        _pages_call("qx_pages_grow", self.handle, self.key_id(key), capacity_tokens,
                    ctypes.byref(self._out))
        return None if self._out.value < 0 else self._out.value

    def row_indices(self, key, tokens=None):
        """Flat pool rows of the key's tokens: page p holds rows p*T .. p*T+T-1."""
        left = self.key_tokens(key) if tokens is None else tokens
        rows = []
        for p in self.table_pages(key):
            take = min(left, self.page_tokens)
            rows.extend(range(p * self.page_tokens, p * self.page_tokens + take))
            left -= take
        return rows

    # ---- pins and retention ------------------------------------------------

    def pin(self, key) -> None:
        _pages_call("qx_pages_pin", self.handle, self.key_id(key))

    def retain(self, key, priority=None) -> None:
        """Make a resident key evictable; priority (a number, or a 1-tuple
        of one) defaults to tokens per page it alone holds (higher is kept
        longer)."""
        if isinstance(priority, tuple):
            if len(priority) != 1:
                raise TypeError("priority is a number or a 1-tuple")
            priority = priority[0]
        has = priority is not None
        _pages_call("qx_pages_retain", self.handle, self.key_id(key), int(has),
                    float(priority) if has else 0.0)

    def pop_retained_victim(self, keep=frozenset()):
        ids = [self._ids[k] if not isinstance(k, TemporaryKey) else k.id
               for k in keep if self.is_resident(k)]
        arr = (ctypes.c_int64 * max(1, len(ids)))(*ids)
        victim = (ctypes.c_int64 * 4)()
        _pages_call("qx_pages_pop_victim", self.handle, arr, len(ids), victim)
        if not victim[0]:
            return None
        return self._keys[victim[1]], victim[2], victim[3]
