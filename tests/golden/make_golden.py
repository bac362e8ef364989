"""Write the golden vectors of the chain-verification path.

Run in a container where /root/reference is mounted and ``make -C oracle`` has
compiled the reference's own engine (csrc/src/scheduler/speculative.cpp +
speculative.h, driven by oracle/ref_driver.cpp) into oracle/_ref/:

    python tests/golden/make_golden.py

Outputs (committed; the tests read them, never the reference):
  chain_cpp.npz   small cases: inputs and the reference engine's outputs for
                  successive verify_candidates / verify_candidates_greedy calls
                  on one engine per case (so its mt19937 stream carries over)
  chain_cpp_large.json  V = 128256 cases: the input recipe (seeded numpy), a
                  SHA-256 of the generated inputs, and the reference outputs
  mt19937.npz     the reference's uniform stream for a few rng_seed values
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import oracle as O  # noqa: E402
from tests.golden.recipes import chain_case  # noqa: E402


SMALL = [
    # name, seed, calls, K, V, recipe kwargs
    ("v5_k3", 1, 12, 3, 5, {}),
    ("v5_k1_onehot", 2, 6, 1, 5, {"onehot": True}),
    ("v64_k4", 3, 10, 4, 64, {}),
    ("v64_k8_eos", 4, 10, 8, 64, {"eos_bias": True}),
    ("v64_k0", 5, 6, 0, 64, {}),
    ("v64_k4_equal", 6, 6, 4, 64, {"equal": True}),
    ("v64_k4_zero_q", 7, 6, 4, 64, {"zero_q": True}),
    ("v1000_k8", 8, 6, 8, 1000, {"sigma": 3.0}),
    ("v1000_k5_sharp", 9, 6, 5, 1000, {"sigma": 8.0}),
    ("v1_k2", 10, 4, 2, 1, {}),
]

LARGE = [
    ("v128256_k3", 100, 3, 3, 128256, {"sigma": 2.0}),
    ("v128256_k8", 101, 2, 8, 128256, {"sigma": 2.0}),
]


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main() -> None:
    assert O.ref_lib() is not None, "build oracle/_ref first (make -C oracle)"
    small = {}
    for name, seed, calls, K, V, kw in SMALL:
        tok, d, t, eos = chain_case(seed, calls, K, V, **kw)
        small[f"{name}__tokens"] = tok
        small[f"{name}__dprobs"] = d
        small[f"{name}__tprobs"] = t
        small[f"{name}__meta"] = np.array([seed, eos], np.int64)
        for greedy in (False, True):
            out = O.ref_verify(seed, tok, d, t, eos, greedy=greedy)
            mode = "greedy" if greedy else "cpp"
            for k, v in out.items():
                small[f"{name}__{mode}_{k}"] = v
    np.savez_compressed(os.path.join(HERE, "chain_cpp.npz"), **small)

    large = []
    for name, seed, calls, K, V, kw in LARGE:
        tok, d, t, eos = chain_case(seed, calls, K, V, **kw)
        out = O.ref_verify(seed, tok, d, t, eos, greedy=False)
        large.append(dict(name=name, seed=seed, calls=calls, K=K, V=V, kwargs=kw, eos=eos,
                          sha256=digest(tok, d, t),
                          out={k: v.tolist() for k, v in out.items()}))
    with open(os.path.join(HERE, "chain_cpp_large.json"), "w") as f:
        json.dump(large, f, indent=1)

    seeds = [0, 1, 42, 2**32 + 7]
    np.savez_compressed(os.path.join(HERE, "mt19937.npz"),
                        seeds=np.array(seeds, np.uint64),
                        draws=np.stack([O.ref_uniforms(s, 4096) for s in seeds]))
    print("wrote", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
