"""Shared test helpers: golden-fixture access and reference-stream replay."""
from __future__ import annotations

import hashlib
import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def small_cases():
    """Yield (name, seed, eos, tokens, dprobs, tprobs, outputs_by_mode)."""
    z = np.load(os.path.join(GOLDEN, "chain_cpp.npz"))
    names = sorted({k.split("__")[0] for k in z.files})
    for name in names:
        seed, eos = (int(x) for x in z[f"{name}__meta"])
        outs = {}
        for mode in ("cpp", "greedy"):
            outs[mode] = {k: z[f"{name}__{mode}_{k}"] for k in
                          ("accepted", "num_accepted", "final", "eos")}
        yield (name, seed, eos, z[f"{name}__tokens"], z[f"{name}__dprobs"],
               z[f"{name}__tprobs"], outs)


def large_cases():
    with open(os.path.join(GOLDEN, "chain_cpp_large.json")) as f:
        return json.load(f)


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def mt_stream():
    z = np.load(os.path.join(GOLDEN, "mt19937.npz"))
    return z["seeds"], z["draws"]


def draws_used(n: int, K: int, accepted_last, eos: int) -> int:
    """Uniforms the reference consumes in one verify_candidates call
    (speculative.cpp:64-97): one per acceptance test, plus the final draw
    unless an accepted EOS ended the call."""
    if n > 0 and accepted_last == eos:
        return n
    return n + 2 if n < K else K + 1


def replay(verify_one, tok, d, t, eos, stream, greedy):
    """Successive calls on one engine: verify_one(tok_c, d_c, t_c, eos, U_c)
    returns (accepted list, final, eos flag); the stream position advances by
    the draws each call consumed.  Returns arrays shaped like the fixtures."""
    C, K = tok.shape
    acc = np.full((C, K), -1, np.int32)
    na = np.zeros(C, np.int32)
    fin = np.zeros(C, np.int32)
    ef = np.zeros(C, np.int32)
    pos = 0
    for c in range(C):
        U = stream[pos:pos + K + 1]
        a, f, e = verify_one(tok[c], d[c], t[c], eos, U)
        n = len(a)
        acc[c, :n] = a
        na[c], fin[c], ef[c] = n, f, int(e)
        if not greedy:
            pos += draws_used(n, K, a[-1] if n else None, eos)
    return dict(accepted=acc, num_accepted=na, final=fin, eos=ef)


def paged_pools(K, V, block_size, num_layers=1, layer=0, extra_blocks=3, seed=0):
    """Scatter contiguous per-sequence K/V ([B][L_b, Hkv, D] lists or a
    [B, L, Hkv, D] tensor) into a paged pool [blocks, layers, Hkv, bs, D] with
    a random block permutation (paged_kv_cache.cpp:13-21, 409-421).
    Returns (k_pool, v_pool, block_tables [B, max_blocks] int32); unused
    table entries are -1, as prepare_batch_metadata leaves them
    (paged_kv_cache.cpp:346-347)."""
    import torch

    B = len(K)
    lens = [int(k.shape[0]) for k in K]
    Hkv, D = K[0].shape[1], K[0].shape[2]
    nb = [(L + block_size - 1) // block_size for L in lens]
    total = sum(nb) + extra_blocks
    g = torch.Generator().manual_seed(seed)
    perm = torch.randperm(total, generator=g)
    kp = torch.randn(total, num_layers, Hkv, block_size, D, generator=g).to(K[0].dtype)
    vp = torch.randn(total, num_layers, Hkv, block_size, D, generator=g).to(V[0].dtype)
    maxb = max(nb)
    bt = torch.full((B, maxb), -1, dtype=torch.int32)
    nxt = 0
    for b in range(B):
        for p in range(nb[b]):
            blk = int(perm[nxt])
            nxt += 1
            bt[b, p] = blk
            lo, hi = p * block_size, min((p + 1) * block_size, lens[b])
            kp[blk, layer, :, : hi - lo, :] = K[b][lo:hi].transpose(0, 1)
            vp[blk, layer, :, : hi - lo, :] = V[b][lo:hi].transpose(0, 1)
    return kp, vp, bt
