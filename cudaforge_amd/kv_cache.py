"""Paged KV cache: page tables in libcfa.so, K/V pools in HBM.

Mirror of the reference's ``PagedKVCache`` as its Python layer sees it
(``csrc/bindings/pybind_module.cpp:20-99``: ``KVCacheConfig``,
``KVCacheStats``, ``PagedKVCache.register_sequence_with_prefix``,
``append_tokens``, ``unregister_sequence``, ``get_block_table``,
``get_config``, ``get_stats``), plus the C++-only calls the verification path
needs (``fork_sequence``, ``prepare_batch_metadata``, ``get_key_block_ptr``,
``get_value_block_ptr``; ``csrc/include/cudaforge/memory/paged_kv_cache.h:
99-139``) and the rollback of rejected draft tokens (``truncate_sequence``,
``commit_tree_paths``), which the reference does not have.

The page tables (reference counts, free list, prefix trie, LRU) live in C++
behind the C ABI (``cfa_kv_cache_*``); this module owns the device memory:
the two pools ``[total_gpu_blocks, num_layers, num_kv_heads, block_size,
head_dim]`` (the byte layout of ``paged_kv_cache.cpp:13-21, 409-421``), the
pinned host staging buffers and the device block tables the kernels read.
"""
from __future__ import annotations

import ctypes
from dataclasses import asdict, dataclass
from typing import Callable, List, Optional, Sequence

import torch

from . import _lib
from ._lib import OutOfPagesException

__all__ = [
    "KVCacheConfig",
    "KVCacheStats",
    "KVCacheBatchDescriptor",
    "OutOfPagesException",
    "PagedKVCache",
]


@dataclass
class KVCacheConfig:
    """paged_kv_cache.h:36-46 (same fields and defaults)."""

    num_layers: int = 32
    num_kv_heads: int = 8
    head_dim: int = 128
    block_size: int = 16
    element_size_bytes: int = 2
    total_gpu_blocks: int = 1024
    enable_prefix_caching: bool = True
    max_supported_batch_size: int = 256
    max_blocks_per_sequence: int = 512

    @property
    def layer_block_bytes(self) -> int:
        return self.num_kv_heads * self.block_size * self.head_dim * self.element_size_bytes

    @property
    def bytes_per_block(self) -> int:
        return self.num_layers * self.layer_block_bytes

    def _c(self) -> _lib.KVCacheConfigC:
        return _lib.KVCacheConfigC(
            self.num_layers, self.num_kv_heads, self.head_dim, self.block_size,
            self.element_size_bytes, self.total_gpu_blocks, 1 if self.enable_prefix_caching else 0,
            0, self.max_supported_batch_size, self.max_blocks_per_sequence)


@dataclass
class KVCacheStats:
    """paged_kv_cache.h:63-75."""

    total_blocks: int = 0
    free_blocks: int = 0
    allocated_blocks: int = 0
    cached_prefix_blocks: int = 0
    total_memory_bytes: int = 0
    used_memory_bytes: int = 0
    pool_utilization_ratio: float = 0.0
    active_sequences_count: int = 0
    prefix_cache_hits: int = 0
    prefix_cache_misses: int = 0
    lru_evictions_count: int = 0


@dataclass
class KVCacheBatchDescriptor:
    """paged_kv_cache.h:81-94.  ``block_tables`` ([batch_size,
    max_blocks_per_seq], -1 padded) and ``context_lens`` ([batch_size]) are
    int32 views of the cache's device staging buffers: the next
    ``prepare_batch_metadata`` call overwrites them, in stream order, as in
    the reference."""

    block_tables: torch.Tensor
    context_lens: torch.Tensor
    batch_size: int
    max_blocks_per_seq: int
    block_size: int
    num_kv_heads: int
    head_dim: int
    bytes_per_block: int
    layer_block_bytes: int
    key_pool_ptr: int
    val_pool_ptr: int


_POOL_DTYPES = {1: torch.uint8, 2: torch.bfloat16, 4: torch.float32}


class PagedKVCache:
    """Page tables of a paged KV cache plus its two device pools.

    ``allocator`` (optional) is a callable ``(nbytes, device) -> tensor`` that
    provides the pool memory (the role of the reference's ``BlockAllocator``
    arena); by default the pools come from torch's caching allocator.
    ``device=None`` picks the current HIP device; on a host without one the
    cache holds page tables only (no pools, host-side batch metadata).
    ``dtype`` overrides the pool element type chosen from
    ``element_size_bytes`` (bf16 for 2 bytes).
    """

    def __init__(self, config: KVCacheConfig, allocator: Optional[Callable] = None, *,
                 device: Optional[torch.device] = None, dtype: Optional[torch.dtype] = None):
        self._cfg = KVCacheConfig(**asdict(config))
        lib = _lib.load()
        handle = ctypes.c_void_p()
        _lib.check(lib.cfa_kv_cache_create(ctypes.byref(self._cfg._c()), ctypes.byref(handle)),
                   "PagedKVCache")
        self._h = handle
        self._lib = lib
        c = self._cfg
        if device is None and torch.cuda.is_available():
            device = torch.device("cuda", torch.cuda.current_device())
        self.device = torch.device(device) if device is not None else None
        cap = c.max_supported_batch_size * c.max_blocks_per_sequence
        self.key_pool: Optional[torch.Tensor] = None
        self.value_pool: Optional[torch.Tensor] = None
        self._event = None
        if self.device is not None and self.device.type == "cuda":
            dt = dtype or _POOL_DTYPES.get(c.element_size_bytes)
            if dt is None or torch.empty((), dtype=dt).element_size() != c.element_size_bytes:
                raise ValueError("element_size_bytes does not match the pool dtype")
            shape = (c.total_gpu_blocks, c.num_layers, c.num_kv_heads, c.block_size, c.head_dim)
            self.key_pool = self._pool(shape, dt, allocator)
            self.value_pool = self._pool(shape, dt, allocator)
            self._h_tables = torch.empty(cap, dtype=torch.int32, pin_memory=True)
            self._h_ctx = torch.empty(c.max_supported_batch_size, dtype=torch.int32,
                                      pin_memory=True)
            self._d_tables = torch.empty(cap, dtype=torch.int32, device=self.device)
            self._d_ctx = torch.empty(c.max_supported_batch_size, dtype=torch.int32,
                                      device=self.device)
        else:
            self._h_tables = torch.empty(cap, dtype=torch.int32)
            self._h_ctx = torch.empty(c.max_supported_batch_size, dtype=torch.int32)
            self._d_tables = self._d_ctx = None

    def _pool(self, shape, dt, allocator):
        nbytes = 1
        for s in shape:
            nbytes *= s
        nbytes *= torch.empty((), dtype=dt).element_size()
        if allocator is None:
            return torch.empty(shape, dtype=dt, device=self.device)
        raw = allocator(nbytes, self.device)
        if not isinstance(raw, torch.Tensor) or raw.numel() * raw.element_size() < nbytes:
            raise ValueError("allocator returned too little memory")
        return raw.view(torch.uint8).reshape(-1)[:nbytes].view(dt).view(shape)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                if self._event is not None:
                    self._event.synchronize()
                self._lib.cfa_kv_cache_destroy(h)
            except Exception:
                pass
            self._h = None

    # -- reference interface (pybind_module.cpp:83-99) ----------------------
    def register_sequence_with_prefix(self, sequence_id: int, prompt_tokens: Sequence[int]) -> int:
        """paged_kv_cache.cpp:167-253; returns the tokens served from the
        prefix cache."""
        toks = torch.as_tensor(list(prompt_tokens), dtype=torch.int32)
        matched = ctypes.c_uint32(0)
        ptr = ctypes.cast(toks.data_ptr(), _lib._i32p) if toks.numel() else None
        _lib.check(self._lib.cfa_kv_cache_register_sequence(
            self._h, sequence_id, ptr, toks.numel(), ctypes.byref(matched)),
            "register_sequence_with_prefix")
        return matched.value

    def append_tokens(self, sequence_id: int, num_tokens: int = 1) -> None:
        """paged_kv_cache.cpp:255-286, with copy on write of a page shared
        after fork_sequence (the copy runs on the current stream)."""
        _lib.check(self._lib.cfa_kv_cache_append_tokens(self._h, sequence_id, num_tokens),
                   "append_tokens")
        self._apply_page_copies()

    def unregister_sequence(self, sequence_id: int) -> None:
        """paged_kv_cache.cpp:288-299."""
        _lib.check(self._lib.cfa_kv_cache_unregister_sequence(self._h, sequence_id),
                   "unregister_sequence")

    def get_block_table(self, sequence_id: int) -> List[int]:
        """paged_kv_cache.cpp:398-407."""
        n = ctypes.c_int64(0)
        _lib.check(self._lib.cfa_kv_cache_get_block_table(self._h, sequence_id, None, 0,
                                                          ctypes.byref(n)), "get_block_table")
        out = (ctypes.c_int32 * max(1, n.value))()
        _lib.check(self._lib.cfa_kv_cache_get_block_table(self._h, sequence_id, out, n.value,
                                                          ctypes.byref(n)), "get_block_table")
        return list(out[:n.value])

    def get_config(self) -> KVCacheConfig:
        return KVCacheConfig(**asdict(self._cfg))

    def get_stats(self) -> KVCacheStats:
        """paged_kv_cache.cpp:423-445."""
        s = _lib.KVCacheStatsC()
        _lib.check(self._lib.cfa_kv_cache_get_stats(self._h, ctypes.byref(s)), "get_stats")
        return KVCacheStats(**{f: getattr(s, f) for f in KVCacheStats.__dataclass_fields__})

    # -- C++-side interface (paged_kv_cache.h:109-135) ----------------------
    def fork_sequence(self, parent_sequence_id: int, child_sequence_id: int) -> None:
        """paged_kv_cache.cpp:301-316 (a registered child first releases its
        own pages)."""
        _lib.check(self._lib.cfa_kv_cache_fork_sequence(self._h, parent_sequence_id,
                                                        child_sequence_id), "fork_sequence")

    def prepare_batch_metadata(self, active_sequence_ids: Sequence[int],
                               stream: Optional[torch.cuda.Stream] = None
                               ) -> KVCacheBatchDescriptor:
        """paged_kv_cache.cpp:318-396: stage the batch's block tables and
        context lengths for the kernels (host-to-device copies enqueued on
        `stream`, default the current stream)."""
        ids = (ctypes.c_uint64 * max(1, len(active_sequence_ids)))(*active_sequence_ids)
        c = self._cfg
        mb = ctypes.c_int32(0)
        B = len(active_sequence_ids)
        on_dev = self._d_tables is not None
        if on_dev:
            st = stream if stream is not None else torch.cuda.current_stream(self.device)
            # the pinned buffers may still feed the previous call's copy
            if self._event is not None:
                self._event.synchronize()
        with (torch.cuda.device(self.device) if on_dev else _nullctx()):
            rc = self._lib.cfa_kv_cache_prepare_batch(
                self._h, ids, B, self._h_tables.data_ptr(), self._h_ctx.data_ptr(),
                self._h_tables.numel(),
                self._d_tables.data_ptr() if on_dev else None,
                self._d_ctx.data_ptr() if on_dev else None,
                self._d_tables.numel() if on_dev else 0, ctypes.byref(mb),
                st.cuda_stream if on_dev else None)
            _lib.check(rc, "prepare_batch_metadata")
            if on_dev:
                self._event = torch.cuda.Event()
                self._event.record(st)
        n = B * mb.value
        src_t, src_c = (self._d_tables, self._d_ctx) if on_dev else (self._h_tables, self._h_ctx)
        return KVCacheBatchDescriptor(
            block_tables=src_t[:n].view(B, mb.value), context_lens=src_c[:B], batch_size=B,
            max_blocks_per_seq=mb.value, block_size=c.block_size, num_kv_heads=c.num_kv_heads,
            head_dim=c.head_dim, bytes_per_block=c.bytes_per_block,
            layer_block_bytes=c.layer_block_bytes,
            key_pool_ptr=self.key_pool.data_ptr() if self.key_pool is not None else 0,
            val_pool_ptr=self.value_pool.data_ptr() if self.value_pool is not None else 0)

    def get_key_block_ptr(self, block_id: int, layer_idx: int) -> int:
        """paged_kv_cache.cpp:409-414 (device address)."""
        return self._block_ptr(self.key_pool, block_id, layer_idx)

    def get_value_block_ptr(self, block_id: int, layer_idx: int) -> int:
        """paged_kv_cache.cpp:416-421 (device address)."""
        return self._block_ptr(self.value_pool, block_id, layer_idx)

    def _block_ptr(self, pool, block_id: int, layer_idx: int) -> int:
        if pool is None:
            raise RuntimeError("this cache has no device pools")
        c = self._cfg
        if not (0 <= block_id < c.total_gpu_blocks and 0 <= layer_idx < c.num_layers):
            raise IndexError("block or layer index out of range")
        return pool.data_ptr() + block_id * c.bytes_per_block + layer_idx * c.layer_block_bytes

    # -- extensions ---------------------------------------------------------
    def context_length(self, sequence_id: int) -> int:
        """(pages - 1) * block_size + fill of the last page
        (paged_kv_cache.cpp:359-364)."""
        n = ctypes.c_uint32(0)
        _lib.check(self._lib.cfa_kv_cache_context_length(self._h, sequence_id, ctypes.byref(n)),
                   "context_length")
        return n.value

    def truncate_sequence(self, sequence_id: int, new_length: int) -> None:
        """Keep the first `new_length` tokens; pages past them are released
        (a cut inside a page shared after a fork copies the kept part to a
        private page).  ValueError when new_length exceeds the sequence."""
        _lib.check(self._lib.cfa_kv_cache_truncate_sequence(self._h, sequence_id, new_length),
                   "truncate_sequence")
        self._apply_page_copies()

    def pop_page_copies(self) -> List[tuple]:
        """Queued copy-on-write page copies ``(src_block, dst_block,
        n_slots)``, oldest first.  A cache with device pools runs them itself
        after every append / truncate; a page-table-only cache leaves them
        to the caller."""
        n = ctypes.c_int64(0)
        _lib.check(self._lib.cfa_kv_cache_pop_page_copies(self._h, None, 0, ctypes.byref(n)),
                   "pop_page_copies")
        if n.value == 0:
            return []
        arr = (_lib.KVPageCopyC * n.value)()
        _lib.check(self._lib.cfa_kv_cache_pop_page_copies(self._h, arr, n.value, ctypes.byref(n)),
                   "pop_page_copies")
        return [(c.src_block, c.dst_block, c.n_slots) for c in arr[:n.value]]

    def _apply_page_copies(self) -> None:
        if self.key_pool is None:
            return
        for src, dst, n in self.pop_page_copies():
            for pool in (self.key_pool, self.value_pool):
                pool[dst, :, :, :n].copy_(pool[src, :, :, :n])

    def block_info(self, block_id: int) -> tuple:
        """(reference count, tokens filled, is cached) of one page."""
        r, f, c = ctypes.c_uint32(0), ctypes.c_uint32(0), ctypes.c_int32(0)
        _lib.check(self._lib.cfa_kv_cache_block_info(self._h, block_id, ctypes.byref(r),
                                                     ctypes.byref(f), ctypes.byref(c)),
                   "block_info")
        return r.value, f.value, bool(c.value)

    def commit_tree_paths(self, sequence_ids: Sequence[int], descriptor: KVCacheBatchDescriptor,
                          base_lens: torch.Tensor, paths: torch.Tensor,
                          path_lens: torch.Tensor) -> List[int]:
        """Keep the accepted path of a verified draft tree and roll back the
        rest.

        Each sequence held ``base_lens[b]`` tokens before its N tree nodes
        were appended (``append_tokens(seq, N)``) and written at slots
        ``base + node``; ``descriptor`` is the batch's metadata taken after
        that append.  The accepted nodes ``paths[b, :path_lens[b]]`` move to
        slots ``base .. base + L - 1`` on the device (``cfa_kv_commit``), then
        each sequence is truncated to ``base + L``.  Returns the new lengths
        (this reads them back to the host, which waits for the stream).
        """
        from .verify import kv_commit

        if self.key_pool is None:
            raise RuntimeError("this cache has no device pools")
        out = kv_commit(self.key_pool, self.value_pool, descriptor.block_tables, base_lens,
                        paths, path_lens)
        new_lens = out.new_ctx_lens.cpu().tolist()
        status = out.status.cpu().tolist()
        for seq, n in zip(sequence_ids, new_lens):
            self.truncate_sequence(seq, n)
        bad = [seq for seq, s in zip(sequence_ids, status) if s != 0]
        if bad:
            raise RuntimeError(f"commit_tree_paths: malformed path or unmapped page for "
                               f"sequences {bad} (rolled back to their base length)")
        return new_lens


class _nullctx:
    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False
