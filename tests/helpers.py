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
