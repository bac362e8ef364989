"""CPU restatement of the reference's paged-KV page tables.

TEST INFRASTRUCTURE ONLY.  Only ``tests/`` imports this module, as the checker
of ``cfa_kv_cache_*`` (cudaforge_amd/csrc/kv_cache.cpp).  The product never
imports it.

Follows ``csrc/src/memory/paged_kv_cache.cpp`` of the reference step by step
(the reference's C++ needs CUDA, spdlog and its BlockAllocator, so it is not
built here):

  block hash                 :80-88
  LRU eviction               :101-124
  page allocation (LIFO)     :126-144
  page release / LRU insert  :146-165
  register_sequence_with_prefix :167-253
  append_tokens              :255-286
  unregister_sequence        :288-299
  fork_sequence              :301-316
  prepare_batch_metadata     :318-396 (context length :359-364)
  get_stats                  :423-445

``reference_quirks=True`` keeps four behaviours of the reference that the
library deliberately does not reproduce:

  * eviction erases the page's hash from the flat map but leaves its trie
    node under its parent (:101-124), so a later prompt can match a page that
    was recycled -- the library unlinks the node;
  * fork onto an already registered child overwrites the child's table
    without releasing its pages (:301-316) -- the library releases them;
  * register / append throw OutOfPagesException midway and keep the pages
    taken so far (:216-249, :272-284) -- the library checks the free and
    evictable pages first and leaves the tables unchanged on failure;
  * after a fork, append fills the shared, partly filled last page for every
    table holding it (:265-271) -- the library copies it on write (a private
    page for the appending sequence plus a queued page copy, ``copies``).

``truncate`` restates the library's rollback, which has no counterpart in the
reference; it is pinned by the invariants in tests/test_kv_cache.py (token
ledger, reference counts, free/cached/allocated partition), not by reference
vectors.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional

M64 = (1 << 64) - 1


class OracleError(Exception):
    """kind: 'state' (runtime_error), 'range' (out_of_range),
    'pages' (OutOfPagesException), 'arg' (invalid argument)."""

    def __init__(self, kind: str, msg: str):
        super().__init__(msg)
        self.kind = kind


@dataclass
class Page:
    refs: int = 0
    filled: int = 0
    hash: int = 0
    cached: bool = False
    node: Optional["TrieNode"] = None


@dataclass(eq=False)
class TrieNode:
    hash: int = 0
    page: int = -1
    parent: Optional["TrieNode"] = None
    kids: Dict[int, "TrieNode"] = field(default_factory=dict)


def block_hash(tokens, parent: int) -> int:
    """paged_kv_cache.cpp:80-88 (std::hash<int32_t> is the value widened to
    64 bits; arithmetic modulo 2**64)."""
    h = (parent ^ 0x9E3779B97F4A7C15) & M64
    for t in tokens:
        h ^= ((int(t) & M64) + 0x9E3779B9 + ((h << 6) & M64) + (h >> 2)) & M64
    return h


class PageTables:
    def __init__(self, *, num_blocks: int, block_size: int, prefix_caching: bool = True,
                 max_batch: int = 256, max_blocks_per_seq: int = 512,
                 bytes_per_block: int = 0, reference_quirks: bool = False):
        self.bs = block_size
        self.n = num_blocks
        self.caching = prefix_caching
        self.max_batch = max_batch
        self.max_blocks = max_blocks_per_seq
        self.bytes_per_block = bytes_per_block
        self.quirks = reference_quirks
        self.pages = [Page() for _ in range(num_blocks)]
        # the stack holds n-1 .. 0 with 0 on top (constructor, :45-54)
        self.free: List[int] = list(range(num_blocks - 1, -1, -1))
        self.lru: List[int] = []  # index 0 = most recently released
        self.root = TrieNode()
        self.tables: Dict[int, List[int]] = {}
        self.hits = self.misses = self.evictions = 0
        self.copies: List[tuple] = []  # (src page, dst page, slots)

    # -- :101-144 ---------------------------------------------------------
    def _evict(self) -> bool:
        for pid in reversed(self.lru):
            pg = self.pages[pid]
            if pg.refs == 0:
                self.lru.remove(pid)
                if not self.quirks and pg.node is not None:
                    nd = pg.node
                    if nd.parent is not None and nd.parent.kids.get(nd.hash) is nd:
                        del nd.parent.kids[nd.hash]
                pg.node = None
                pg.cached = False
                pg.hash = 0
                pg.filled = 0
                self.free.append(pid)
                self.evictions += 1
                return True
        return False

    def _alloc(self) -> int:
        if not self.free and not self._evict():
            raise OracleError("pages", "OutOfPagesException")
        pid = self.free.pop()
        pg = self.pages[pid]
        pg.refs, pg.filled, pg.cached = 1, 0, False
        if not self.quirks:
            pg.hash = 0
        return pid

    # -- :146-165 ---------------------------------------------------------
    def _release(self, pid: int) -> None:
        if pid < 0 or pid >= self.n:
            return
        pg = self.pages[pid]
        if pg.refs == 0:
            return
        pg.refs -= 1
        if pg.refs == 0:
            if self.caching and pg.hash != 0:
                pg.cached = True
                self.lru.insert(0, pid)
            else:
                pg.filled = 0
                self.free.append(pid)

    def _table(self, seq: int) -> List[int]:
        if seq not in self.tables:
            raise OracleError("state", f"Sequence ID {seq} not registered")
        return self.tables[seq]

    # -- :167-253 ---------------------------------------------------------
    def register(self, seq: int, tokens) -> int:
        if seq in self.tables:
            return 0
        bs = self.bs
        full = len(tokens) // bs
        hashes = []
        h = 0
        for b in range(full):
            h = block_hash(tokens[b * bs:(b + 1) * bs], h)
            hashes.append(h)
        hit: List[TrieNode] = []
        node = self.root
        if self.caching:
            for h in hashes:
                kid = node.kids.get(h)
                if kid is None:
                    break
                hit.append(kid)
                node = kid
        tail = len(tokens) - full * bs
        if not self.quirks:
            needed = (full - len(hit)) + (1 if tail > 0 or full == 0 else 0)
            cached_hits = sum(1 for k in hit if self.pages[k.page].cached)
            if needed > len(self.free) + len(self.lru) - cached_hits:
                raise OracleError("pages", "OutOfPagesException")
        table: List[int] = []
        for kid in hit:
            pg = self.pages[kid.page]
            pg.refs += 1
            if pg.cached:
                pg.cached = False
                self.lru.remove(kid.page)
            table.append(kid.page)
            self.hits += 1
        node = hit[-1] if hit else self.root
        for b in range(len(hit), full):
            pid = self._alloc()
            pg = self.pages[pid]
            pg.filled = bs
            pg.hash = hashes[b]
            if self.caching or self.quirks:
                nd = TrieNode(hash=hashes[b], page=pid, parent=node)
                node.kids[hashes[b]] = nd
                pg.node = nd
                node = nd
            table.append(pid)
            self.misses += 1
        if tail > 0 or not table:
            pid = self._alloc()
            self.pages[pid].filled = tail
            table.append(pid)
        self.tables[seq] = table
        return len(hit) * bs

    # -- :255-286 ---------------------------------------------------------
    def _make_private_last(self, table: List[int], slots: int) -> None:
        src = table[-1]
        dst = self._alloc()
        self.pages[dst].filled = slots
        self.pages[src].refs -= 1
        table[-1] = dst
        if slots:
            self.copies.append((src, dst, slots))

    def append(self, seq: int, n: int = 1) -> None:
        table = self._table(seq)
        if n == 0 and not self.quirks:
            return
        room = self.bs - self.pages[table[-1]].filled
        cow = not self.quirks and room > 0 and self.pages[table[-1]].refs > 1
        extra = -(-(n - room) // self.bs) if n > room else 0
        if not self.quirks and int(cow) + extra > len(self.free) + len(self.lru):
            raise OracleError("pages", "OutOfPagesException")
        if cow:
            self._make_private_last(table, self.pages[table[-1]].filled)
        last = self.pages[table[-1]]
        if n <= room:
            last.filled += n
            return
        rest = n - room
        last.filled = self.bs
        for _ in range(extra):
            pid = self._alloc()
            add = min(rest, self.bs)
            self.pages[pid].filled = add
            rest -= add
            table.append(pid)

    # -- :288-299 ---------------------------------------------------------
    def unregister(self, seq: int) -> None:
        table = self.tables.pop(seq, None)
        for pid in table or ():
            self._release(pid)

    # -- :301-316 ---------------------------------------------------------
    def fork(self, parent: int, child: int) -> None:
        if parent == child and not self.quirks:
            raise OracleError("arg", "fork onto itself")
        src = list(self._table(parent))
        for pid in src:
            self.pages[pid].refs += 1
        if not self.quirks:
            self.unregister(child)
        self.tables[child] = src

    # -- rollback (library extension) -------------------------------------
    def truncate(self, seq: int, new_len: int) -> None:
        table = self._table(seq)
        if new_len > self.context_length(seq):
            raise OracleError("arg", "new length exceeds the sequence")
        keep = max(1, -(-new_len // self.bs))
        last_fill = new_len - (keep - 1) * self.bs
        cut = table[keep - 1]
        changes = last_fill != self.pages[cut].filled
        cow = changes and self.pages[cut].refs > 1
        if cow:
            avail = len(self.free) + len(self.lru) + sum(
                1 for p in table[keep:] if self.pages[p].refs == 1)
            if avail == 0:
                raise OracleError("pages", "OutOfPagesException")
        for pid in table[keep:]:
            self._release(pid)
        del table[keep:]
        if cow:
            self._make_private_last(table, last_fill)
        elif changes:
            pg = self.pages[cut]
            if pg.hash != 0:
                nd = pg.node
                if nd is not None and nd.parent is not None and nd.parent.kids.get(nd.hash) is nd:
                    del nd.parent.kids[nd.hash]
                pg.node = None
                pg.hash = 0
            pg.filled = last_fill

    # -- :359-364 ---------------------------------------------------------
    def context_length(self, seq: int) -> int:
        table = self._table(seq)
        return (len(table) - 1) * self.bs + self.pages[table[-1]].filled

    # -- :318-396 ---------------------------------------------------------
    def prepare_batch(self, seqs):
        if len(seqs) > self.max_batch:
            raise OracleError("range", "batch size exceeds max_supported_batch_size")
        mb = max((len(self._table(s)) for s in seqs), default=0)
        if mb > self.max_blocks:
            raise OracleError("range", "blocks exceed max_blocks_per_sequence")
        tables = [self.tables[s] + [-1] * (mb - len(self.tables[s])) for s in seqs]
        ctx = [self.context_length(s) for s in seqs]
        return tables, ctx, mb

    # -- :423-445 ---------------------------------------------------------
    def stats(self) -> dict:
        free = len(self.free)
        cached = len(self.lru)
        alloc = self.n - free - cached
        return dict(
            total_blocks=self.n, free_blocks=free, allocated_blocks=alloc,
            cached_prefix_blocks=cached,
            total_memory_bytes=self.n * self.bytes_per_block * 2,
            used_memory_bytes=(alloc + cached) * self.bytes_per_block * 2,
            pool_utilization_ratio=(self.n - free) / self.n,
            active_sequences_count=len(self.tables),
            prefix_cache_hits=self.hits, prefix_cache_misses=self.misses,
            lru_evictions_count=self.evictions)
