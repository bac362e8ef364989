"""ctypes binding of ``libcfa.so`` (the C ABI declared in include/cudaforge_amd.h).

The library is loaded from the package directory (it is built in-tree by
``cudaforge_amd._build``); ``CFA_LIB_PATH`` selects another build of the same
library, such as a host-sanitizer variant for CPU test runs.  There is no
fallback: if the library is missing, every entry point raises
``RuntimeError`` naming the build command.

Error mapping follows the reference's pybind layer: a C-ABI ``CFA_ERR_ARG`` is
the ``std::invalid_argument`` of ``csrc/src/scheduler/speculative.cpp:58-62``
and surfaces as ``ValueError``; ``CFA_ERR_RANGE`` is a ``std::out_of_range``
(``IndexError``); ``CFA_ERR_OUT_OF_PAGES`` is the reference's
``OutOfPagesException`` (a ``RuntimeError``); ``CFA_ERR_STATE`` (a
``std::runtime_error``) and ``CFA_ERR_HIP`` surface as ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.environ.get("CFA_LIB_PATH") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), "libcfa.so")

CFA_OK = 0
CFA_ERR_ARG = -1
CFA_ERR_HIP = -2
CFA_ERR_STATE = -3
CFA_ERR_RANGE = -4
CFA_ERR_OUT_OF_PAGES = -5

CFA_INPUT_PROBS = 0
CFA_INPUT_LOGITS = 1

CFA_MODE_CPP = 0
CFA_MODE_PYTHON = 1
CFA_MODE_GREEDY = 2

CFA_SAMPLE_MULTINOMIAL = 0
CFA_SAMPLE_FILTERED = 1
CFA_SAMPLE_GREEDY = 2

_i = ctypes.c_int
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_f = ctypes.c_float
_sz = ctypes.c_size_t
_p = ctypes.c_void_p
_i32p = ctypes.POINTER(ctypes.c_int32)
_f32p = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)
_ip = ctypes.POINTER(ctypes.c_int)

_u32 = ctypes.c_uint32
_u32p = ctypes.POINTER(ctypes.c_uint32)
_i64p = ctypes.POINTER(ctypes.c_int64)


class KVCacheConfigC(ctypes.Structure):
    """cfa_kv_cache_config."""

    _fields_ = [
        ("num_layers", ctypes.c_uint32),
        ("num_kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("block_size", ctypes.c_uint32),
        ("element_size_bytes", ctypes.c_uint64),
        ("total_gpu_blocks", ctypes.c_uint64),
        ("enable_prefix_caching", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("max_supported_batch_size", ctypes.c_uint64),
        ("max_blocks_per_sequence", ctypes.c_uint64),
    ]


class KVCacheStatsC(ctypes.Structure):
    """cfa_kv_cache_stats."""

    _fields_ = [
        ("total_blocks", ctypes.c_uint64),
        ("free_blocks", ctypes.c_uint64),
        ("allocated_blocks", ctypes.c_uint64),
        ("cached_prefix_blocks", ctypes.c_uint64),
        ("total_memory_bytes", ctypes.c_uint64),
        ("used_memory_bytes", ctypes.c_uint64),
        ("pool_utilization_ratio", ctypes.c_double),
        ("active_sequences_count", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("prefix_cache_hits", ctypes.c_uint64),
        ("prefix_cache_misses", ctypes.c_uint64),
        ("lru_evictions_count", ctypes.c_uint64),
    ]


class KVPageCopyC(ctypes.Structure):
    """cfa_kv_page_copy."""

    _fields_ = [("src_block", ctypes.c_int32), ("dst_block", ctypes.c_int32),
                ("n_slots", ctypes.c_int32)]


# The ABI these signatures describe (CFA_ABI_VERSION of include/cudaforge_amd.h).
ABI_VERSION = 200

# name -> (restype, argtypes); every symbol the header declares.
SIGNATURES: dict[str, tuple] = {
    "cfa_last_error": (ctypes.c_char_p, []),
    "cfa_version": (_i, []),
    "cfa_chain_verify_workspace_size": (_sz, [_i, _i, _i, _i, _i]),
    "cfa_chain_verify": (
        _i,
        [_p, _i64, _i64, _p, _i64, _i64, _i, _p, _p, _i, _i, _i, _f, _f, _i, _i32,
         _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p],
    ),
    "cfa_chain_verify_noalloc": (
        _i,
        [_p, _i64, _i64, _p, _i64, _i64, _i, _p, _p, _i, _i, _i, _f, _f, _i, _i32,
         _p, _p, _p, _p, _p, _p, _p, _p],
    ),
    "cfa_sample_workspace_size": (_sz, [_i, _i, _i, _i]),
    "cfa_sample": (
        _i, [_p, _i64, _i, _i, _i, _i, _f, _i, _f, _i, _p, _p, _p, _p, _sz, _p]),
    "cfa_tree_attention_workspace_size": (_sz, [_i, _i, _i, _i, _i, _i, _i]),
    "cfa_tree_attention": (
        _i,
        [_p, _p, _p, _p, _i, _p, _i, _i, _i, _i, _p, _i64, _i, _i, _i, _i, _i, _i, _f, _i, _i,
         _p, _p, _sz, _p],
    ),
    "cfa_tree_verify_workspace_size": (_sz, [_i]),
    "cfa_tree_verify": (
        _i,
        [_p, _i64, _i64, _p, _i64, _i64, _i, _p, _i64, _p, _p, _i, _i, _i, _i, _f, _i, _i32,
         _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _sz, _p],
    ),
    "cfa_kv_commit": (
        _i,
        [_p, _p, _p, _i, _p, _p, _i, _p, _i, _i, _i, _i, _i, _i, _i, _p, _p, _p],
    ),
    "cfa_w4a16_dequant": (_i, [_p, _p, _p, _i, _i, _i, _i, _p, _p]),
    "cfa_w4a16_dequant_t": (_i, [_p, _p, _p, _i, _i, _i, _i, _p, _p]),
    "cfa_w4a16_gemm": (_i, [_p, _p, _p, _i, _i, _i, _i, _i, _p, _p]),
    "cfa_w4a16_gemm_zp_workspace_size": (_sz, [_i, _i, _i]),
    "cfa_w4a16_gemm_zp": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _p, _p, _sz, _p]),
    "cfa_w4a16_gemm_zp_silu": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _p, _p, _sz, _p]),
    "cfa_w4a16_gemm_zp_splits": (_i, [_i, _i, _i]),
    "cfa_w4a16_gemm_zp_partials": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _p, _sz, _p]),
    "cfa_rmsnorm": (_i, [_p, _p, _p, _p, _i, _i, _f, _p]),
    "cfa_rmsnorm_partials": (_i, [_p, _p, _i, _p, _p, _i, _i, _f, _p]),
    "cfa_rope_kv_paged": (
        _i, [_p, _p, _i, _i, _i, _i, _i, _f, _p, _p, _p, _i, _i, _i, _p, _i, _p, _p]),
    "cfa_rope_kv_paged_partials": (
        _i, [_p, _i, _p, _i, _i, _i, _i, _i, _f, _p, _p, _p, _i, _i, _i, _p, _i, _p, _p]),
    "cfa_rope_kv_strided": (
        _i, [_p, _p, _i, _i, _i, _i, _i, _f, _p, _p, _i64p, _p, _i64p, _p, _p]),
    "cfa_silu_mul": (_i, [_p, _p, _i, _i, _p]),
    "cfa_gemm_bf16_skinny_workspace_size": (_sz, [_i, _i, _i, _i]),
    "cfa_gemm_bf16_skinny": (_i, [_p, _p, _p, _i, _i, _i, _i, _p, _sz, _p]),
    "cfa_gemm_bf16_skinny_silu": (_i, [_p, _p, _p, _i, _i, _i, _i, _p, _sz, _p]),
    "cfa_kv_cache_create": (_i, [ctypes.POINTER(KVCacheConfigC), ctypes.POINTER(_p)]),
    "cfa_kv_cache_destroy": (None, [_p]),
    "cfa_kv_cache_register_sequence": (_i, [_p, _u64, _i32p, _i64, _u32p]),
    "cfa_kv_cache_append_tokens": (_i, [_p, _u64, _u32]),
    "cfa_kv_cache_unregister_sequence": (_i, [_p, _u64]),
    "cfa_kv_cache_fork_sequence": (_i, [_p, _u64, _u64]),
    "cfa_kv_cache_truncate_sequence": (_i, [_p, _u64, _u32]),
    "cfa_kv_cache_context_length": (_i, [_p, _u64, _u32p]),
    "cfa_kv_cache_get_block_table": (_i, [_p, _u64, _i32p, _i64, _i64p]),
    "cfa_kv_cache_prepare_batch": (
        _i, [_p, ctypes.POINTER(_u64), _i, _p, _p, _i64, _p, _p, _i64, _i32p, _p]),
    "cfa_kv_cache_get_stats": (_i, [_p, ctypes.POINTER(KVCacheStatsC)]),
    "cfa_kv_cache_pop_page_copies": (_i, [_p, ctypes.POINTER(KVPageCopyC), _i64, _i64p]),
    "cfa_kv_cache_block_info": (_i, [_p, _i32, _u32p, _u32p, _i32p]),
    "cfa_rng_create": (_p, [_u64]),
    "cfa_rng_destroy": (None, [_p]),
    "cfa_rng_peek": (_i, [_p, _i, _f32p]),
    "cfa_rng_advance": (_i, [_p, _i]),
    "cfa_profile_enable": (_i, [_i]),
    "cfa_profile_reset": (_i, []),
    "cfa_profile_query": (_i, [ctypes.c_char_p, _ip, _dp]),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load libcfa.so (once) and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build the HIP library with "
                    "`python -m cudaforge_amd._build` (there is no CPU fallback)")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            if lib.cfa_version() // 100 != ABI_VERSION // 100:
                raise RuntimeError(
                    f"{LIB_PATH} has ABI version {lib.cfa_version()}, these bindings need "
                    f"{ABI_VERSION}: rebuild with `python -m cudaforge_amd._build`")
            _lib = lib
    return _lib


def last_error() -> str:
    msg = load().cfa_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    """Raise the Python exception that corresponds to a C-ABI return code."""
    if rc == CFA_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc == CFA_ERR_ARG:
        raise ValueError(msg)
    if rc == CFA_ERR_RANGE:
        raise IndexError(msg)
    if rc == CFA_ERR_OUT_OF_PAGES:
        raise OutOfPagesException(msg)
    raise RuntimeError(msg)


class OutOfPagesException(RuntimeError):
    """No free or evictable KV page (paged_kv_cache.h:31-34, raised at
    paged_kv_cache.cpp:126-135)."""


def profile_enable(on: bool) -> None:
    check(load().cfa_profile_enable(1 if on else 0), "cfa_profile_enable")


def profile_reset() -> None:
    check(load().cfa_profile_reset(), "cfa_profile_reset")


def profile_query(kernel: str) -> tuple[int, float]:
    """(launch count, summed duration in ms) of `kernel` since the last reset."""
    n = ctypes.c_int(0)
    ms = ctypes.c_double(0.0)
    check(load().cfa_profile_query(kernel.encode(), ctypes.byref(n), ctypes.byref(ms)),
          "cfa_profile_query")
    return n.value, ms.value
