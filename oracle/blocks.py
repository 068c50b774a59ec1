"""Block manager model on the CPU (oracle; test infrastructure only).

The reference has no block-level refcounts, copy-on-write or block LRU
(muserve/model/prefix_cache.py caches whole prefixes). This model fixes the
semantics the GPU block manager implements, built from the reference's pieces:
the LIFO free stack of muserve/kv_cache.py:77-91, the prefix key of
muserve/model/prefix_cache.py:31-34 evaluated per 16-token page, and the
OrderedDict LRU of muserve/model/prefix_cache.py:71,92,95-96 over cached pages
nobody holds.

admit(r, hashes, n_tokens):
  * k = number of leading page hashes present in the table (the longest run
    of consecutive hits from page 0);
  * OOM check before any change: the pages to take (n_pages - k, plus one for
    copy-on-write when the last page is partial) must not exceed
    free + evictable - (hits currently evictable);
  * hits: refcount += 1, leaving the LRU if they were in it;
  * new pages: pop the free stack, and when it is empty evict the LRU's
    oldest page (its hash leaves the table);
  * full pages k..m-1 register their hash (unless the hash is already
    present); the partial last page is never cached;
  * fork: a child shares every page (refcount += 1); when the last page is
    partial the child's first append copies it to a freshly taken page
    (copy-on-write) and detaches from it.
release(r): child then parent, each tail first: refcount -= 1; at 0 a cached
  page goes to the LRU's newest end, any other page onto the free stack.
"""
from __future__ import annotations

from collections import OrderedDict

PAGE = 16

OK, OOM = 0, 1


class BlockManagerModel:
    def __init__(self, num_pages: int, free_order: list[int] | None = None):
        self.P = num_pages
        self.free = list(range(num_pages)) if free_order is None else list(free_order)
        self.ref = [0] * num_pages
        self.hash: list[int | None] = [None] * num_pages
        self.table: dict[int, int] = {}
        self.lru: OrderedDict[int, None] = OrderedDict()
        self.evicted: list[int] = []
        self.reqs: dict[int, tuple[list[int], list[int]]] = {}

    def _take(self) -> int:
        if self.free:
            return self.free.pop()
        p, _ = self.lru.popitem(last=False)
        del self.table[self.hash[p]]
        self.hash[p] = None
        self.evicted.append(p)
        return p

    def admit(self, r: int, hashes: list[int], n_tokens: int) -> dict:
        n_pages = -(-n_tokens // PAGE)
        m = len(hashes)
        assert m == n_tokens // PAGE
        k = 0
        while k < m and hashes[k] in self.table:
            k += 1
        hits = [self.table[h] for h in hashes[:k]]
        cow = n_tokens % PAGE != 0
        need = n_pages - k + (1 if cow else 0)
        pinned = sum(1 for p in hits if self.ref[p] == 0)
        if need > len(self.free) + len(self.lru) - pinned:
            return {"status": OOM, "hits": 0, "table": [], "child_last": -1,
                    "cow_src": -1, "cow_dst": -1}
        for p in hits:
            if self.ref[p] == 0:
                del self.lru[p]
            self.ref[p] += 1
        new = [self._take() for _ in range(n_pages - k)]
        for p in new:
            self.ref[p] = 1
        table = hits + new
        for i in range(k, m):
            if hashes[i] not in self.table:
                self.table[hashes[i]] = table[i]
                self.hash[table[i]] = hashes[i]
        child = list(table)
        for p in table:
            self.ref[p] += 1
        cow_src = cow_dst = -1
        if cow:
            cow_src = table[-1]
            cow_dst = self._take()
            self.ref[cow_dst] = 1
            self.ref[cow_src] -= 1
            child[-1] = cow_dst
        self.reqs[r] = (table, child)
        return {"status": OK, "hits": k, "table": table,
                "child_last": child[-1] if child else -1, "cow_src": cow_src, "cow_dst": cow_dst}

    def release(self, r: int) -> None:
        table, child = self.reqs.pop(r)
        for tbl in (child, table):
            for p in reversed(tbl):
                self.ref[p] -= 1
                if self.ref[p] == 0:
                    if self.hash[p] is not None:
                        self.lru[p] = None
                    else:
                        self.free.append(p)

    # -- views used by the parity tests --
    def lru_order(self) -> list[int]:
        return list(self.lru)

    def check_invariants(self) -> None:
        """refcount = number of live tables holding the page; every page is in
        exactly one of free / LRU / held; table <-> cached pages is a bijection."""
        holders = [0] * self.P
        for table, child in self.reqs.values():
            for p in table:
                holders[p] += 1
            for p in child:
                holders[p] += 1
        assert holders == self.ref, "refcounts differ from holder counts"
        free, lru = set(self.free), set(self.lru)
        assert len(free) == len(self.free) and not (free & lru)
        held = {p for p in range(self.P) if self.ref[p] > 0}
        assert not (held & free) and not (held & lru)
        assert free | lru | held == set(range(self.P)), "a page is lost"
        assert all(self.ref[p] == 0 and self.hash[p] is not None for p in lru)
        assert {p: h for h, p in self.table.items()} == {
            p: h for p, h in enumerate(self.hash) if h is not None}


class TimestampLRUModel:
    """Independent restatement for pinning BlockManagerModel on small traces:
    the evictable set is derived by scanning all pages, and the eviction victim
    is the cached ref-0 page with the oldest release time (pure-Python loops)."""

    def __init__(self, num_pages: int, free_order: list[int] | None = None):
        self.P = num_pages
        self.free = list(range(num_pages)) if free_order is None else list(free_order)
        self.ref = [0] * num_pages
        self.hash: list[int | None] = [None] * num_pages
        self.released_at = [0] * num_pages
        self.clock = 0
        self.evicted: list[int] = []
        self.reqs: dict[int, tuple[list[int], list[int]]] = {}

    def _lookup(self, h: int) -> int:
        for p in range(self.P):
            if self.hash[p] == h:
                return p
        return -1

    def _evictable(self) -> list[int]:
        return [p for p in range(self.P) if self.hash[p] is not None and self.ref[p] == 0]

    def _take(self) -> int:
        if self.free:
            return self.free.pop()
        cand = self._evictable()
        p = min(cand, key=lambda q: self.released_at[q])
        self.hash[p] = None
        self.evicted.append(p)
        return p

    def admit(self, r: int, hashes: list[int], n_tokens: int) -> dict:
        n_pages = -(-n_tokens // PAGE)
        hits = []
        for h in hashes:
            p = self._lookup(h)
            if p < 0:
                break
            hits.append(p)
        k = len(hits)
        cow = n_tokens % PAGE != 0
        need = n_pages - k + (1 if cow else 0)
        evictable = [p for p in self._evictable() if p not in hits]
        if need > len(self.free) + len(evictable):
            return {"status": OOM, "hits": 0, "table": [], "child_last": -1,
                    "cow_src": -1, "cow_dst": -1}
        for p in hits:
            self.ref[p] += 1
        new = []
        for _ in range(n_pages - k):
            p = self._take()
            self.ref[p] = 1
            new.append(p)
        table = hits + new
        for i in range(k, len(hashes)):
            if self._lookup(hashes[i]) < 0:
                self.hash[table[i]] = hashes[i]
        child = list(table)
        for p in table:
            self.ref[p] += 1
        cow_src = cow_dst = -1
        if cow:
            cow_src = table[-1]
            cow_dst = self._take()
            self.ref[cow_dst] = 1
            self.ref[cow_src] -= 1
            child[-1] = cow_dst
        self.reqs[r] = (table, child)
        return {"status": OK, "hits": k, "table": table,
                "child_last": child[-1] if child else -1, "cow_src": cow_src, "cow_dst": cow_dst}

    def release(self, r: int) -> None:
        table, child = self.reqs.pop(r)
        for tbl in (child, table):
            for p in reversed(tbl):
                self.ref[p] -= 1
                if self.ref[p] == 0:
                    if self.hash[p] is not None:
                        self.clock += 1
                        self.released_at[p] = self.clock
                    else:
                        self.free.append(p)

    def lru_order(self) -> list[int]:
        return sorted(self._evictable(), key=lambda q: self.released_at[q])
