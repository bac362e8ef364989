"""CPU tier: the exact parallel replay of a sequential fp32 accumulation
(cudaforge_amd/csrc/seqsum.hpp) -- host emulation of the work-group algorithm
with the same helpers, fuzzed against a plain left-to-right fp32 loop on the
inputs that break naive parallel sums (ties, subnormals, wide ranges)."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "native", "seqsum_emu.cpp")
LIB = os.path.join(HERE, "native", "libseqsum_emu.so")


def build_emu(lib: str = LIB, extra: tuple = ()) -> str:
    """Compile the host emulation (extra: e.g. sanitizer flags) unless current."""
    hdr = os.path.join(os.path.dirname(HERE), "cudaforge_amd", "csrc", "seqsum.hpp")
    if not os.path.exists(lib) or os.path.getmtime(lib) < max(os.path.getmtime(SRC),
                                                               os.path.getmtime(hdr)):
        subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-fPIC", "-shared",
                        *extra, SRC, "-o", lib], check=True)
    return lib


@pytest.fixture(scope="module")
def emu():
    # SEQSUM_EMU_LIB: another build of the emulation (the sanitizer runs)
    L = ctypes.CDLL(os.environ.get("SEQSUM_EMU_LIB") or build_emu())
    L.emu_seq.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_longlong, ctypes.c_int,
                          ctypes.c_float, ctypes.c_int, ctypes.c_float,
                          ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_longlong),
                          ctypes.POINTER(ctypes.c_longlong)]

    def run(x, cdf, r, nt):
        x = np.ascontiguousarray(x, np.float32)
        s, i, ns = ctypes.c_float(), ctypes.c_longlong(), ctypes.c_longlong()
        L.emu_seq(x.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), x.size, cdf,
                  np.float32(r), nt, np.float32(0.0), ctypes.byref(s), ctypes.byref(i),
                  ctypes.byref(ns))
        return np.float32(s.value), i.value
    return run


def seq_prefix(x):
    return np.cumsum(x.astype(np.float32), dtype=np.float32)  # sequential fp32 adds


def generators(rng):
    def softmax(V, sig):
        l = rng.normal(0, sig, V)
        p = np.exp(l - l.max())
        return (p / p.sum()).astype(np.float32)
    return [
        lambda V: softmax(V, 2.86),
        lambda V: softmax(V, 6.0),
        lambda V: np.where(rng.random(V) < 0.7, 0, softmax(V, 2.0)).astype(np.float32),
        lambda V: (rng.integers(0, 64, V) * 2.0 ** -20).astype(np.float32),
        lambda V: (rng.integers(0, 2 ** 10, V) * 2.0 ** -30).astype(np.float32),
        lambda V: (rng.integers(0, 8, V) * 2.0 ** -149).astype(np.float32),
        lambda V: np.exp(rng.uniform(-100, 0, V)).astype(np.float32),
        lambda V: np.sort(softmax(V, 3.0)),
        lambda V: np.sort(softmax(V, 3.0))[::-1].copy(),
        lambda V: np.zeros(V, np.float32),
    ]


def test_cumsum_is_sequential():
    x = np.array([1.0, 2.0 ** -24, 2.0 ** -24], np.float32)
    assert seq_prefix(x)[-1] == np.float32(1.0)  # sequential rounding, not pairwise


@pytest.mark.parametrize("seed", range(4))
def test_emulated_replay_is_bit_exact(emu, seed):
    rng = np.random.default_rng(seed)
    gens = generators(rng)
    for trial in range(40):
        V = int(rng.choice([1, 5, 1000, 16384, 20000, 128256]))
        x = gens[trial % len(gens)](V)
        pref = seq_prefix(x)
        nt = int(rng.choice([64, 256, 1024]))
        s, _ = emu(x, 0, 0.0, nt)
        assert s == pref[-1], (trial, V)
        for rk in range(4):
            if rk == 0:
                r = np.float32(rng.random()) * (pref[-1] if pref[-1] > 0 else 1)
            elif rk == 1:
                r = pref[rng.integers(0, V)]
            elif rk == 2:
                r = np.nextafter(pref[rng.integers(0, V)], np.float32(0))
            else:
                r = np.float32(rng.random())
            hit = np.nonzero(r <= pref)[0]
            _, idx = emu(x, 1, r, nt)
            assert idx == (int(hit[0]) if hit.size else -1), (trial, V, r)
