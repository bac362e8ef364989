"""GPU tier: cfa_chain_verify_noalloc (the allocation-free chain verification,
whose workspace is the library's static 32 MiB device array) against
cfa_chain_verify with a caller workspace, called through the C ABI.

Two calls in a row, the second with a smaller input, in each mode; the
outputs must be identical (bit-exact) to the workspace entry point's.  A
shape whose workspace exceeds 32 MiB is refused with CFA_ERR_ARG before any
work is enqueued.
"""
import ctypes

import numpy as np
import pytest
import torch

from cudaforge_amd import _lib
from tests.golden.recipes import c2_inputs

pytestmark = pytest.mark.gpu

MODES = {"cpp": _lib.CFA_MODE_CPP, "python": _lib.CFA_MODE_PYTHON,
         "greedy": _lib.CFA_MODE_GREEDY}


def _lib_noalloc():
    lib = _lib.load()
    return lib, lib.cfa_chain_verify_noalloc


def _inputs(device, B, K, V, mode, seed):
    tl, dl, tok, U = c2_inputs(seed=seed, B=B, K=K, V=V, temperature=0.7)
    if mode == "python":
        extra = np.random.default_rng(seed).random((B, 1)).astype(np.float32)
        U = np.concatenate([U, extra], axis=1)
    return [torch.from_numpy(np.ascontiguousarray(a)).to(device) for a in (tl, dl, tok, U)]


def _outputs(device, B, K, V, probs):
    i32 = dict(dtype=torch.int32, device=device)
    o = [torch.full((B,), -7, **i32), torch.full((B, K + 1), -7, **i32),
         torch.full((B,), -7, **i32), torch.full((B,), -7, **i32), torch.full((B,), -7, **i32)]
    if probs:
        o += [torch.empty(B, K + 1, V, device=device), torch.empty(B, K, V, device=device)]
    return o


def _call(fn, t, d, tok, U, mode, outs, stream, workspace=None):
    B, K1, V = t.shape
    K = K1 - 1
    ptr = [x.data_ptr() for x in outs[:5]]
    probs = [outs[5].data_ptr(), outs[6].data_ptr()] if len(outs) > 5 else [None, None]
    greedy = mode == "greedy"
    args = [t.data_ptr(), t.stride(0), t.stride(1),
            None if greedy else d.data_ptr(), d.stride(0), d.stride(1),
            _lib.CFA_INPUT_LOGITS, tok.data_ptr(), None if greedy else U.data_ptr(),
            B, K, V, ctypes.c_float(0.7), ctypes.c_float(0.9), MODES[mode], -1,
            *ptr, *probs]
    if workspace is not None:
        args += [workspace.data_ptr(), workspace.numel()]
    return fn(*args, stream)


@pytest.mark.parametrize("mode", ["cpp", "python", "greedy"])
def test_noalloc_matches_workspace_entry_point(device, mode):
    lib, noalloc = _lib_noalloc()
    stream = torch.cuda.current_stream(device).cuda_stream
    # the full chain-sampling shape, then a smaller one: the static scratch
    # keeps the first call's contents and must not leak into the second
    for (B, K, V, seed, probs) in ((64, 8, 128256, 5, False), (5, 3, 1001, 6, True)):
        t, d, tok, U = _inputs(device, B, K, V, mode, seed)
        ref = _outputs(device, B, K, V, probs)
        ws_bytes = lib.cfa_chain_verify_workspace_size(B, K, V, _lib.CFA_INPUT_LOGITS,
                                                       MODES[mode])
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
        _lib.check(_call(lib.cfa_chain_verify, t, d, tok, U, mode, ref, stream, ws),
                   "cfa_chain_verify")
        got = _outputs(device, B, K, V, probs)
        _lib.check(_call(noalloc, t, d, tok, U, mode, got, stream), "cfa_chain_verify_noalloc")
        torch.cuda.synchronize()
        for name, a, b in zip(("accept_len", "tokens", "num_emitted", "final", "eos",
                               "target_probs", "draft_probs"), ref, got):
            if mode == "greedy" and name == "draft_probs":
                continue
            assert torch.equal(a, b), (mode, B, K, V, name)


def test_noalloc_refuses_shapes_beyond_its_scratch(device):
    lib, noalloc = _lib_noalloc()
    B, K, V = 200, 8, 128256  # needs about 58 MiB of workspace
    assert lib.cfa_chain_verify_workspace_size(B, K, V, _lib.CFA_INPUT_LOGITS,
                                               _lib.CFA_MODE_CPP) > (32 << 20)
    x = torch.empty(1, device=device)
    i = torch.empty(1, dtype=torch.int32, device=device)
    rc = noalloc(x.data_ptr(), (K + 1) * V, V, x.data_ptr(), K * V, V, _lib.CFA_INPUT_LOGITS,
                 i.data_ptr(), x.data_ptr(), B, K, V, ctypes.c_float(1.0), ctypes.c_float(1.0),
                 _lib.CFA_MODE_CPP, -1, i.data_ptr(), i.data_ptr(), i.data_ptr(), i.data_ptr(),
                 i.data_ptr(), None, None, torch.cuda.current_stream(device).cuda_stream)
    assert rc == _lib.CFA_ERR_ARG
    assert "32 MiB" in _lib.last_error()
