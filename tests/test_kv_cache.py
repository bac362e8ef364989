"""CPU tier: paged-KV page tables (cfa_kv_cache_* in libcfa.so, host code
only -- no GPU call is made here) against the oracle restatement
(oracle/kv_pages.py) of csrc/src/memory/paged_kv_cache.cpp.

Pinning of the oracle:
  * the reference's own test (tests/cpp/test_paged_kv_cache.cpp:38-80):
    prompts of 32 and 48 tokens give context lengths 32 / 48 and a batch
    descriptor with max_blocks_per_seq 3;
  * a scripted scenario whose block tables, hit/miss/eviction counts and
    partition were derived by hand from the reference's code (LIFO free
    stack, LRU release order, eviction from the LRU tail), including the
    reference's stale-trie aliasing after eviction (reference_quirks=True);
  * invariants checked on random scripts: reference counts equal the number
    of tables holding each page, free/cached/allocated partition, a token
    ledger kept by the test equals every context length, and a prefix match
    never returns a page whose contents differ from the prompt's (contents
    tracked by the test), re-registering a prompt right after itself
    matches every full block.
The library is then checked against the oracle call by call on random
scripts (tables, matches, lengths, stats, page states, error kinds).
"""
from __future__ import annotations

import random

import pytest

from oracle.kv_pages import OracleError, PageTables

from cudaforge_amd import _lib
from cudaforge_amd.kv_cache import KVCacheConfig, OutOfPagesException, PagedKVCache


def _cache(**kw) -> PagedKVCache:
    return PagedKVCache(KVCacheConfig(**kw), device="cpu")


def _oracle(cfg: KVCacheConfig, quirks: bool = False) -> PageTables:
    return PageTables(num_blocks=cfg.total_gpu_blocks, block_size=cfg.block_size,
                      prefix_caching=cfg.enable_prefix_caching,
                      max_batch=cfg.max_supported_batch_size,
                      max_blocks_per_seq=cfg.max_blocks_per_sequence,
                      bytes_per_block=cfg.bytes_per_block, reference_quirks=quirks)


KAT_CFG = dict(num_layers=2, num_kv_heads=2, head_dim=64, block_size=16, element_size_bytes=2,
               total_gpu_blocks=32, max_supported_batch_size=16, max_blocks_per_sequence=32)


def test_reference_kat_prepare_batch_metadata():
    """tests/cpp/test_paged_kv_cache.cpp:38-80."""
    kv = _cache(**KAT_CFG)
    orc = _oracle(KVCacheConfig(**KAT_CFG))
    for c in (kv, orc):
        reg = c.register_sequence_with_prefix if c is kv else c.register
        reg(100, [1] * 32)
        reg(200, [2] * 48)
    d = kv.prepare_batch_metadata([100, 200])
    assert d.batch_size == 2 and d.max_blocks_per_seq == 3
    assert d.context_lens.tolist() == [32, 48]
    assert d.block_tables.tolist() == [[0, 1, -1], [2, 3, 4]]
    assert d.block_size == 16 and d.num_kv_heads == 2 and d.head_dim == 64
    assert d.layer_block_bytes == 2 * 16 * 64 * 2 and d.bytes_per_block == 2 * d.layer_block_bytes
    tables, ctx, mb = orc.prepare_batch([100, 200])
    assert (tables, ctx, mb) == ([[0, 1, -1], [2, 3, 4]], [32, 48], 3)
    kv.unregister_sequence(100)
    kv.unregister_sequence(200)
    st = kv.get_stats()
    assert st.active_sequences_count == 0 and st.free_blocks + st.cached_prefix_blocks == 32


SCRIPT_CFG = dict(num_layers=1, num_kv_heads=1, head_dim=8, block_size=4, total_gpu_blocks=7,
                  max_supported_batch_size=8, max_blocks_per_sequence=8)


def _run_script(reg, unreg, stats):
    """The scripted scenario; expected values were derived by hand from
    paged_kv_cache.cpp (free stack 6..0 with 0 on top; released hashed pages
    go to the LRU front; eviction takes the LRU tail)."""
    A = [1, 2, 3, 4, 5, 6, 7, 8, 9]
    assert reg(1, A) == (0, [0, 1, 2])            # 2 hashed pages + tail
    assert reg(2, A[:8] + [10, 11]) == (8, [0, 1, 3])  # both full pages shared
    assert reg(3, [1, 2, 3, 4, 9, 9, 9, 9]) == (4, [0, 4])
    unreg(1)                                      # page 2 -> free stack
    unreg(2)                                      # page 1 -> LRU, page 3 -> free
    s = stats()
    assert (s["free_blocks"], s["cached_prefix_blocks"], s["allocated_blocks"]) == (4, 1, 2)
    assert reg(4, [7] * 13) == (0, [3, 2, 5, 6])  # pops 3, 2, 5, 6
    assert reg(5, [8] * 4) == (0, [1])            # free list empty: evicts page 1
    s = stats()
    assert (s["lru_evictions_count"], s["prefix_cache_hits"], s["prefix_cache_misses"]) == (1, 3, 7)
    unreg(4)                                      # 3, 2, 5 -> LRU; 6 -> free
    return reg(6, A[:8])


def test_scripted_scenario_library_and_oracle():
    cfg = KVCacheConfig(**SCRIPT_CFG)
    kv = _cache(**SCRIPT_CFG)

    def reg(seq, toks):
        m = kv.register_sequence_with_prefix(seq, toks)
        return m, kv.get_block_table(seq)

    def stats():
        return vars(kv.get_stats())

    # page 1 was recycled for sequence 5, so only page 0 may match
    assert _run_script(reg, kv.unregister_sequence, stats) == (4, [0, 6])
    assert kv.block_info(1) == (1, 4, False)

    orc = _oracle(cfg)
    assert _run_script(lambda s, t: (orc.register(s, t), list(orc.tables[s])),
                       orc.unregister, orc.stats) == (4, [0, 6])


def test_reference_quirk_stale_trie_aliases_recycled_page():
    """With the reference's eviction (the trie node stays under its parent,
    paged_kv_cache.cpp:101-124) the last prompt matches page 1, which now
    holds sequence 5's tokens [8, 8, 8, 8]: two sequences alias one page."""
    orc = _oracle(KVCacheConfig(**SCRIPT_CFG), quirks=True)
    got = _run_script(lambda s, t: (orc.register(s, t), list(orc.tables[s])),
                      orc.unregister, orc.stats)
    assert got == (8, [0, 1])
    assert orc.tables[5] == [1] and orc.pages[1].refs == 2


def test_reference_quirk_fork_onto_registered_child_leaks():
    """paged_kv_cache.cpp:301-316 overwrites a registered child's table; its
    pages keep their references for ever.  The library releases them."""
    cfg = KVCacheConfig(**SCRIPT_CFG)
    for quirks, free_after in ((True, 6), (False, 7)):  # page 1 leaks with the quirk
        orc = _oracle(cfg, quirks=quirks)
        orc.register(1, [5] * 3)   # page 0
        orc.register(2, [6] * 3)   # page 1
        orc.fork(1, 2)
        orc.unregister(1)
        orc.unregister(2)
        assert orc.stats()["free_blocks"] == free_after
    kv = _cache(**SCRIPT_CFG)
    kv.register_sequence_with_prefix(1, [5] * 3)
    kv.register_sequence_with_prefix(2, [6] * 3)
    kv.fork_sequence(1, 2)
    kv.unregister_sequence(1)
    kv.unregister_sequence(2)
    assert kv.get_stats().free_blocks == 7


def test_lifo_reuse_and_append_growth():
    kv = _cache(**SCRIPT_CFG)
    kv.register_sequence_with_prefix(1, [])           # one empty page
    assert kv.get_block_table(1) == [0] and kv.context_length(1) == 0
    kv.append_tokens(1)                               # default num_tokens = 1
    kv.append_tokens(1, 3)
    assert kv.get_block_table(1) == [0] and kv.context_length(1) == 4
    kv.append_tokens(1, 9)                            # 4 + 9 = 13 tokens, 4 pages
    assert kv.get_block_table(1) == [0, 1, 2, 3] and kv.context_length(1) == 13
    kv.unregister_sequence(1)                         # unhashed: back on the stack
    kv.register_sequence_with_prefix(2, [1, 2])
    assert kv.get_block_table(2) == [3]               # last freed, first reused


def test_truncate_rollback():
    kv = _cache(**SCRIPT_CFG)
    kv.register_sequence_with_prefix(1, [1, 2, 3, 4, 5])   # [0 (hashed), 1 (1 token)]
    kv.append_tokens(1, 8)                                 # 13 tokens: [0, 1, 2, 3]
    kv.truncate_sequence(1, 6)
    assert kv.get_block_table(1) == [0, 1] and kv.context_length(1) == 6
    assert kv.get_stats().free_blocks == 5
    kv.truncate_sequence(1, 6)                             # no-op
    with pytest.raises(ValueError):
        kv.truncate_sequence(1, 7)
    # cutting inside the hashed prompt page drops its prefix entry
    kv.truncate_sequence(1, 2)
    assert kv.get_block_table(1) == [0] and kv.context_length(1) == 2
    assert kv.register_sequence_with_prefix(2, [1, 2, 3, 4]) == 0
    kv.truncate_sequence(1, 0)
    assert kv.get_block_table(1) == [0] and kv.context_length(1) == 0


def test_copy_on_write_after_fork():
    kv = _cache(**SCRIPT_CFG)
    kv.register_sequence_with_prefix(1, [1, 2, 3, 4, 5, 6])  # [0 (hashed), 1 (2 tokens)]
    kv.fork_sequence(1, 2)
    assert kv.block_info(1)[0] == 2
    kv.append_tokens(2, 1)             # the child gets a private copy of page 1
    assert kv.get_block_table(2) == [0, 2] and kv.get_block_table(1) == [0, 1]
    assert kv.pop_page_copies() == [(1, 2, 2)]
    assert kv.context_length(1) == 6 and kv.context_length(2) == 7
    assert kv.block_info(1) == (1, 2, False) and kv.block_info(2) == (1, 3, False)
    kv.append_tokens(1, 1)             # page 1 is private again: no copy
    assert kv.pop_page_copies() == [] and kv.get_block_table(1) == [0, 1]
    # a cut inside a shared page copies the kept part
    kv.fork_sequence(1, 3)
    kv.truncate_sequence(3, 5)
    assert kv.get_block_table(3) == [0, 3] and kv.pop_page_copies() == [(1, 3, 1)]
    assert kv.context_length(1) == 7 and kv.context_length(3) == 5
    # a cut at a page end shares on
    kv.fork_sequence(1, 4)
    kv.truncate_sequence(4, 4)
    assert kv.get_block_table(4) == [0] and kv.pop_page_copies() == []
    assert kv.block_info(0)[0] == 4


def test_error_mapping():
    kv = _cache(**SCRIPT_CFG)
    with pytest.raises(RuntimeError, match="not registered"):
        kv.append_tokens(9)
    with pytest.raises(RuntimeError):
        kv.get_block_table(9)
    with pytest.raises(RuntimeError):
        kv.fork_sequence(9, 10)
    kv.unregister_sequence(9)                             # unknown id: ignored
    with pytest.raises(ValueError):
        kv.fork_sequence(1, 1)
    kv.register_sequence_with_prefix(1, [0] * 20)         # 5 pages
    assert kv.register_sequence_with_prefix(1, [3] * 4) == 0   # already registered: no-op
    assert kv.context_length(1) == 20
    with pytest.raises(OutOfPagesException):
        kv.register_sequence_with_prefix(2, [1] * 12)
    assert issubclass(OutOfPagesException, RuntimeError)
    with pytest.raises(IndexError):
        kv.prepare_batch_metadata(list(range(9)))
    kv2 = _cache(**dict(SCRIPT_CFG, max_blocks_per_sequence=2))
    kv2.register_sequence_with_prefix(1, [0] * 9)
    with pytest.raises(IndexError):
        kv2.prepare_batch_metadata([1])
    with pytest.raises(ValueError):
        _cache(**dict(SCRIPT_CFG, block_size=0))


def test_stats_formulas():
    cfg = KVCacheConfig(**KAT_CFG)
    kv = PagedKVCache(cfg, device="cpu")
    kv.register_sequence_with_prefix(1, [1] * 40)          # 2 hashed + tail
    kv.register_sequence_with_prefix(2, [1] * 32)          # shares both
    kv.unregister_sequence(1)
    s = kv.get_stats()
    assert s.total_blocks == 32 and s.free_blocks == 30 and s.cached_prefix_blocks == 0
    assert s.allocated_blocks == 2 and s.active_sequences_count == 1
    assert s.total_memory_bytes == 32 * cfg.bytes_per_block * 2
    assert s.used_memory_bytes == 2 * cfg.bytes_per_block * 2
    assert s.pool_utilization_ratio == pytest.approx(2 / 32)
    assert (s.prefix_cache_hits, s.prefix_cache_misses) == (2, 2)
    kv.unregister_sequence(2)
    s = kv.get_stats()
    assert s.cached_prefix_blocks == 2 and s.allocated_blocks == 0


def test_prefix_caching_disabled():
    kv = _cache(**dict(SCRIPT_CFG, enable_prefix_caching=False))
    assert kv.register_sequence_with_prefix(1, [1, 2, 3, 4]) == 0
    assert kv.register_sequence_with_prefix(2, [1, 2, 3, 4]) == 0
    assert kv.get_block_table(1) == [0] and kv.get_block_table(2) == [1]
    kv.unregister_sequence(1)
    s = kv.get_stats()
    assert s.cached_prefix_blocks == 0 and s.free_blocks == 6 and s.prefix_cache_misses == 2


# ---------------------------------------------------------------------------
# Random scripts: invariants (oracle and library) and differential parity.
# ---------------------------------------------------------------------------
class _Lib:
    """Adapter giving the library the oracle's method names."""

    def __init__(self, kv: PagedKVCache, cfg: KVCacheConfig):
        self.kv, self.cfg = kv, cfg

    def call(self, op, *a):
        f = {"register": self.kv.register_sequence_with_prefix, "append": self.kv.append_tokens,
             "unregister": self.kv.unregister_sequence, "fork": self.kv.fork_sequence,
             "truncate": self.kv.truncate_sequence}[op]
        try:
            return (f(*a), self.kv.pop_page_copies()), None
        except OutOfPagesException:
            return None, "pages"
        except IndexError:
            return None, "range"
        except ValueError:
            return None, "arg"
        except RuntimeError:
            return None, "state"

    def table(self, s):
        return self.kv.get_block_table(s)

    def length(self, s):
        return self.kv.context_length(s)

    def page(self, p):
        return self.kv.block_info(p)

    def stats(self):
        return vars(self.kv.get_stats())


class _Orc:
    def __init__(self, orc: PageTables):
        self.o = orc

    def call(self, op, *a):
        try:
            res = getattr(self.o, op)(*a)
            copies, self.o.copies = self.o.copies, []
            return (res, copies), None
        except OracleError as e:
            return None, e.kind

    def table(self, s):
        return list(self.o.tables[s])

    def length(self, s):
        return self.o.context_length(s)

    def page(self, p):
        pg = self.o.pages[p]
        return pg.refs, pg.filled, pg.cached

    def stats(self):
        return self.o.stats()


def _random_ops(rng: random.Random, n_ops: int, bs: int):
    live: list = []
    next_id = 1
    prompts = [[rng.randrange(3) for _ in range(rng.randrange(0, 5 * bs))] for _ in range(6)]
    for _ in range(n_ops):
        r = rng.random()
        if r < 0.35 or not live:
            base = rng.choice(prompts)
            cut = rng.randrange(0, len(base) + 1)
            toks = base[:cut] + [rng.randrange(3) for _ in range(rng.randrange(0, bs + 2))]
            if rng.random() < 0.15 and live:
                yield ("register", rng.choice(live), toks)   # already registered
                continue
            yield ("register", next_id, toks)
            live.append(next_id)
            next_id += 1
        elif r < 0.55:
            yield ("append", rng.choice(live), rng.choice([1, 1, 2, bs, bs + 3]))
        elif r < 0.7:
            s = rng.choice(live)
            live.remove(s)
            yield ("unregister", s)
        elif r < 0.8:
            p = rng.choice(live)
            if rng.random() < 0.2:
                yield ("fork", p, rng.choice(live))
            else:
                yield ("fork", p, next_id)
                live.append(next_id)
                next_id += 1
        else:
            yield ("truncate", rng.choice(live), None)
        if rng.random() < 0.02:
            yield ("unregister", 10 ** 6)


def _check_invariants(c, cfg: KVCacheConfig, seqs, ledger, content):
    refs = {}
    for s in seqs:
        t = c.table(s)
        assert c.length(s) == ledger[s], (s, c.length(s), ledger[s])
        assert len(t) >= 1 and (len(t) - 1) * cfg.block_size < max(ledger[s], 1) + cfg.block_size
        for p in t:
            refs[p] = refs.get(p, 0) + 1
    n_free = n_cached = n_alloc = 0
    for p in range(cfg.total_gpu_blocks):
        r, _, cached = c.page(p)
        assert r == refs.get(p, 0), (p, r, refs.get(p, 0))
        if cached:
            assert r == 0
            n_cached += 1
        elif r:
            n_alloc += 1
        else:
            n_free += 1
    st = c.stats()
    assert (st["free_blocks"], st["cached_prefix_blocks"], st["allocated_blocks"]) == \
        (n_free, n_cached, n_alloc)
    assert st["active_sequences_count"] == len(seqs)


def _play(c, cfg: KVCacheConfig, ops, check_every: int = 1):
    bs = cfg.block_size
    seqs, ledger, content = set(), {}, {}
    log = []
    for k, op in enumerate(ops):
        name = op[0]
        if name == "register":
            _, s, toks = op
            res, err = c.call("register", s, toks)
            log.append((op[:2], res, err))
            res = res[0] if res else res
            if err is None and s not in seqs:
                seqs.add(s)
                ledger[s] = len(toks)
                t = c.table(s)
                full = len(toks) // bs
                # a match never returns a page holding other tokens
                for j in range(res // bs):
                    assert content.get(t[j]) == tuple(toks[:(j + 1) * bs]), (s, j)
                for j in range(res // bs, len(t)):
                    content[t[j]] = tuple(toks[:(j + 1) * bs]) if j < full else None
                if cfg.enable_prefix_caching:
                    # the same prompt registered again at once matches every full page
                    probe = 10 ** 7 + k
                    r2, e2 = c.call("register", probe, toks)
                    if e2 is None:
                        assert r2[0] == full * bs
                        c.call("unregister", probe)
            elif err is None:
                assert res == 0
        elif name == "append":
            _, s, n = op
            before = c.table(s) if s in seqs else []
            res, err = c.call("append", s, n)
            log.append((op, res, err))
            if err is None:
                ledger[s] += n
                for p in c.table(s)[len(before):]:
                    content[p] = None
        elif name == "unregister":
            res, err = c.call("unregister", op[1])
            log.append((op, res, err))
            seqs.discard(op[1])
            ledger.pop(op[1], None)
        elif name == "fork":
            _, p, ch = op
            res, err = c.call("fork", p, ch)
            log.append((op, res, err))
            if err is None:
                seqs.add(ch)
                ledger[ch] = ledger[p]
        elif name == "truncate":
            _, s, n = op
            if n is None:
                n = (ledger.get(s, 0) * 7 + k) % (ledger.get(s, 0) + 2)
            res, err = c.call("truncate", s, n)
            log.append((("truncate", s, n), res, err))
            if err is None:
                if n % bs or n == 0:
                    # the cut page no longer holds a whole prompt block
                    content[c.table(s)[-1]] = None
                ledger[s] = n
        if k % check_every == 0:
            _check_invariants(c, cfg, seqs, ledger, content)
        for s in seqs:
            log.append(("state", s, tuple(c.table(s)), c.length(s)))
    log.append(("stats", c.stats()))
    return log


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize("caching", [True, False])
def test_random_scripts_library_matches_oracle(seed, caching):
    rng = random.Random(seed * 2 + caching)
    bs = rng.choice([1, 2, 4, 16])
    n_blocks = rng.choice([6, 12, 40])
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=1, head_dim=4, block_size=bs,
                        total_gpu_blocks=n_blocks, enable_prefix_caching=caching,
                        max_supported_batch_size=64, max_blocks_per_sequence=256)
    ops = list(_random_ops(rng, 160, bs))
    log_orc = _play(_Orc(_oracle(cfg)), cfg, ops)
    log_lib = _play(_Lib(PagedKVCache(cfg, device="cpu"), cfg), cfg, ops)
    assert len(log_orc) == len(log_lib)
    for a, b in zip(log_orc, log_lib):
        assert a == b


def test_random_scripts_exercise_every_path():
    """The random scripts above reach eviction, out-of-pages, shared-page
    truncation refusals and prefix hits."""
    kinds = set()
    evictions = hits = 0
    for seed in range(12):
        rng = random.Random(seed * 2 + 1)
        bs = rng.choice([1, 2, 4, 16])
        n_blocks = rng.choice([6, 12, 40])
        cfg = KVCacheConfig(num_layers=1, num_kv_heads=1, head_dim=4, block_size=bs,
                            total_gpu_blocks=n_blocks, max_supported_batch_size=64,
                            max_blocks_per_sequence=256)
        log = _play(_Orc(_oracle(cfg)), cfg, list(_random_ops(rng, 160, bs)), check_every=50)
        kinds |= {e[2] for e in log if len(e) == 3 and e[0] not in ("state",) and e[2]}
        evictions += log[-1][1]["lru_evictions_count"]
        hits += log[-1][1]["prefix_cache_hits"]
    assert {"pages", "state"} <= kinds
    assert evictions > 0 and hits > 0


def test_library_symbols_present():
    lib = _lib.load()
    for name in _lib.SIGNATURES:
        if name.startswith("cfa_kv_cache_"):
            assert hasattr(lib, name)
