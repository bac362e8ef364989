"""CPU tier: the C-ABI library loads and exports every declared entry point,
its host-only parts (the reference's uniform stream) match the golden stream,
and host-side validation raises before any device work."""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from cudaforge_amd import _lib
from tests import helpers as H

HEADER_DIR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")


def declared_functions():
    names = []
    for fn in sorted(os.listdir(HEADER_DIR)):
        if not fn.endswith(".h"):
            continue
        text = open(os.path.join(HEADER_DIR, fn)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b(cfa_[a-z0-9_]+)\s*\(", text):
            names.append(m.group(1))
    return sorted(set(names))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "cfa_chain_verify" in names and "cfa_last_error" in names


@pytest.mark.parametrize("name", declared_functions())
def test_library_exports_declared_symbol(name):
    lib = _lib.load()
    assert hasattr(lib, name), f"libcfa.so does not export {name}"
    assert name in _lib.SIGNATURES, f"cudaforge_amd._lib has no signature for {name}"


def test_rng_stream_matches_reference_stream():
    lib = _lib.load()
    seeds, draws = H.mt_stream()
    for s, row in zip(seeds, draws):
        r = lib.cfa_rng_create(ctypes.c_uint64(int(s)))
        out = np.zeros(1000, np.float32)
        assert lib.cfa_rng_peek(r, 600, out.ctypes.data_as(_lib._f32p)) == 0
        assert lib.cfa_rng_advance(r, 600) == 0
        assert lib.cfa_rng_peek(r, 400, out[600:].ctypes.data_as(_lib._f32p)) == 0
        lib.cfa_rng_destroy(r)
        np.testing.assert_array_equal(out, row[:1000])


def test_argument_errors_map_to_valueerror():
    lib = _lib.load()
    rc = lib.cfa_chain_verify(None, 0, 0, None, 0, 0, 1, None, None, 0, 1, 10,
                              ctypes.c_float(1.0), ctypes.c_float(1.0), 0, -1,
                              None, None, None, None, None, None, None, None, 0, None)
    assert rc == _lib.CFA_ERR_ARG
    with pytest.raises(ValueError):
        _lib.check(rc, "cfa_chain_verify")
    assert "positive" in _lib.last_error()


@pytest.mark.parametrize("first_node,head_dim,msg", [(15, 128, "first_node"), (-1, 128, "first_node"),
                                                   (0, 96, "head_dim")])
def test_tree_attention_argument_errors(first_node, head_dim, msg):
    """Shape checks run before anything touches a device (dummy pointers)."""
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    rc = lib.cfa_tree_attention(p, p, p, p, 4, p, 8, 1, 0, 16, p, 0, 2, 15, first_node, 8, 2,
                                head_dim, ctypes.c_float(0.1), 64, 0, p, p, 1 << 20, None)
    assert rc == _lib.CFA_ERR_ARG
    assert msg in _lib.last_error()
    ws = lib.cfa_tree_attention_workspace_size(2, 15, 8, 2, head_dim, 64, 0)
    assert (ws == 0) == (head_dim == 96)


def test_host_validation_rejects_cpu_tensors():
    from cudaforge_amd.verify import chain_verify

    t = torch.zeros(2, 3, 8)
    with pytest.raises(ValueError):
        chain_verify(t, torch.zeros(2, 2, 8), torch.zeros(2, 2, dtype=torch.int32),
                     torch.zeros(2, 3))


def test_compat_engine_dimension_errors_match_reference_message():
    from cudaforge_amd import SpeculativeConfig, SpeculativeEngine

    eng = SpeculativeEngine(SpeculativeConfig())
    with pytest.raises(ValueError, match="Incompatible draft and target"):
        eng.verify_candidates([1, 2], [[0.5, 0.5]], [[0.5, 0.5]] * 3, 0)
    with pytest.raises(ValueError, match="Incompatible draft and target"):
        eng.verify_candidates([1], [[0.5, 0.5]], [[0.5, 0.5]], 0)
    with pytest.raises(ValueError):
        eng.verify_candidates([5], [[0.5, 0.5]], [[0.5, 0.5]] * 2, 0)  # id >= V


def test_compat_config_defaults_and_no_reseed():
    from cudaforge_amd import SpeculativeConfig, SpeculativeEngine

    c = SpeculativeConfig()
    assert (c.gamma, c.temperature, c.top_p, c.rng_seed) == (5, 1.0, 1.0, 42)
    eng = SpeculativeEngine(c)
    c2 = SpeculativeConfig(gamma=3, rng_seed=7)
    eng.set_config(c2)
    assert eng.get_config().gamma == 3
    seeds, draws = H.mt_stream()
    idx = list(seeds).index(42)
    np.testing.assert_array_equal(eng._peek(8), draws[idx][:8])  # still seeded with 42


@pytest.mark.parametrize("M,N,K,splits,msg", [
    (0, 64, 128, 1, "M must be"),
    (129, 64, 128, 1, "M must be"),
    (8, 100, 128, 1, "N must be"),
    (8, 64, 100, 1, "K must be"),
    (8, 64, 512, 3, "splits must divide"),
    (8, 64, 512, 8, "splits must divide"),
    (8, 64, 512, 2, "workspace smaller"),
])
def test_skinny_gemm_argument_errors(M, N, K, splits, msg):
    """Shape, split and workspace checks run before anything touches a device
    (dummy pointers)."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    rc = lib.cfa_gemm_bf16_skinny(p, p, p, M, N, K, splits, p, 16, None)
    assert rc == _lib.CFA_ERR_ARG
    assert msg in _lib.last_error()


def test_skinny_gemm_workspace_size():
    lib = _lib.load()
    # one split needs none; S splits need the 64 KiB counter region plus S
    # fp32 partial tiles of 16 * m_tiles rows x 64 columns per column tile
    assert lib.cfa_gemm_bf16_skinny_workspace_size(8, 3072, 2048, 1) == 0
    assert lib.cfa_gemm_bf16_skinny_workspace_size(8, 3072, 2048, 4) == 65536 + 48 * 4 * 4096
    assert lib.cfa_gemm_bf16_skinny_workspace_size(100, 2048, 8192, 8) == 65536 + 32 * 8 * 32 * 1024
    assert lib.cfa_gemm_bf16_skinny_workspace_size(129, 64, 128, 1) == 0


def test_w4a16_split_counts():
    """Split-K counts of the fused W4A16 GEMM (one work-group per CU; the
    host without a GPU assumes 256 CUs): the verify step's target shapes at
    M = 504, and 0 for shapes the kernel does not take."""
    lib = _lib.load()
    assert lib.cfa_w4a16_gemm_zp_splits(504, 28672, 4096) == 1     # gate/up: 224 tiles
    assert lib.cfa_w4a16_gemm_zp_splits(504, 6144, 4096) == 5      # QKV: 48 tiles
    assert lib.cfa_w4a16_gemm_zp_splits(504, 4096, 4096) == 8      # O
    assert lib.cfa_w4a16_gemm_zp_splits(504, 4096, 14336) == 8     # down
    assert lib.cfa_w4a16_gemm_zp_splits(1, 256, 128) == 1
    assert lib.cfa_w4a16_gemm_zp_splits(504, 4100, 4096) == 0
    assert lib.cfa_w4a16_gemm_zp_splits(0, 256, 128) == 0
    # the workspace of the reducing entry point is the same partials
    assert lib.cfa_w4a16_gemm_zp_workspace_size(504, 4096, 4096) == 8 * 504 * 4096 * 4


def test_fused_layer_argument_errors():
    """The partial-summing and SiLU-gated entry points validate before any
    device work (dummy pointers)."""
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    rc = lib.cfa_w4a16_gemm_zp_partials(p, p, p, None, 504, 4100, 4096, 128, p, 1 << 30, None)
    assert rc == _lib.CFA_ERR_ARG and "multiple of 256" in _lib.last_error()
    rc = lib.cfa_w4a16_gemm_zp_partials(p, p, p, None, 504, 4096, 4096, 128, p, 1024, None)
    assert rc == _lib.CFA_ERR_ARG and "part too small" in _lib.last_error()
    rc = lib.cfa_w4a16_gemm_zp_silu(p, p, p, None, 504, 4096, 4000, 128, p, p, 1 << 30, None)
    assert rc == _lib.CFA_ERR_ARG and "multiple of 32" in _lib.last_error()
    rc = lib.cfa_rmsnorm_partials(p, p, 0, p, p, 504, 4096, 1e-5, None)
    assert rc == _lib.CFA_ERR_ARG and "splits" in _lib.last_error()
    rc = lib.cfa_rmsnorm_partials(p, None, 8, p, p, 504, 4096, 1e-5, None)
    assert rc == _lib.CFA_ERR_ARG and "null" in _lib.last_error()
    rc = lib.cfa_rope_kv_paged_partials(None, 5, p, 8, 63, 32, 8, 128, 5e5, p, p, p, 0, 32, 16,
                                        p, 200, p, None)
    assert rc == _lib.CFA_ERR_ARG and "null" in _lib.last_error()
    rc = lib.cfa_rope_kv_paged_partials(p, 0, p, 8, 63, 32, 8, 128, 5e5, p, p, p, 0, 32, 16,
                                        p, 200, p, None)
    assert rc == _lib.CFA_ERR_ARG and "splits" in _lib.last_error()


def test_abi_version_matches_bindings():
    """The library reports the ABI of its header, which the bindings require."""
    with open(os.path.join(HEADER_DIR, "cudaforge_amd.h")) as f:
        hdr = int(re.search(r"#define CFA_ABI_VERSION (\d+)", f.read()).group(1))
    assert _lib.load().cfa_version() == hdr == _lib.ABI_VERSION


def test_tree_status_check_raises_on_failures():
    """check_status: 0 passes; 1 (uniforms ran out) and 2 (a team wait timed
    out) raise RuntimeError naming the sequences."""
    from cudaforge_amd.verify import check_status

    check_status(torch.zeros(4, dtype=torch.int32))
    with pytest.raises(RuntimeError, match=r"ran out .*\[2\]"):
        check_status(torch.tensor([0, 0, 1, 0], dtype=torch.int32))
    with pytest.raises(RuntimeError, match=r"timed out .*\[0, 3\]"):
        check_status(torch.tensor([2, 0, 0, 2], dtype=torch.int32))
