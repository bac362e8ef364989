"""CPU tier: the host code under sanitizers.

* libcfa.so's host side (entry points, argument checks, the page tables of
  csrc/kv_cache.cpp, the host RNG) built with AddressSanitizer +
  UndefinedBehaviorSanitizer (cudaforge_amd._build --sanitize address: host
  pass only), running the page-table and C-ABI CPU tests.
* The oracle (oracle/spec_oracle.c) and the host emulation of the exact
  sequential-sum algorithm (tests/native/seqsum_emu.cpp over
  cudaforge_amd/csrc/seqsum.hpp) built with gcc's ASan + UBSan, running their
  CPU tests.
* libcfa.so's host side built with ThreadSanitizer, driven by eight native
  threads sharing one page table (tests/native/threaded_host_calls.cpp).

Each configuration runs in a child process with its sanitizer runtime
preloaded; no GPU call is made.  A sanitizer report fails the test.
"""
import glob
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
NATIVE = os.path.join(ROOT, "tests", "native")
SAN = os.path.join(ROOT, "cudaforge_amd", "_san")


def _clang_rt(name):
    hits = sorted(glob.glob(f"/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.{name}-x86_64.so"))
    return hits[-1] if hits else None


def _gcc_rt(name):
    if not shutil.which("gcc"):
        return None
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True,
                       text=True).stdout.strip()
    return p if os.path.isabs(p) and os.path.exists(p) else None


def _stale(target, sources):
    return not os.path.exists(target) or os.path.getmtime(target) < max(
        os.path.getmtime(s) for s in sources)


def _lib_variant(kind):
    from cudaforge_amd import _build

    lib = os.path.join(SAN, f"libcfa_{kind}.so")
    srcs = _build.sources() + glob.glob(os.path.join(_build.CSRC, "*.hpp"))
    if _stale(lib, srcs):
        _build.build(sanitize=kind)
    return lib


def _run(cmd, env, timeout=900):
    full = dict(os.environ)
    full.update(env)
    p = subprocess.run(cmd, cwd=ROOT, env=full, capture_output=True, text=True, timeout=timeout)
    out = p.stdout + p.stderr
    for marker in ("ERROR: AddressSanitizer", "runtime error:", "WARNING: ThreadSanitizer"):
        assert marker not in out, out[-6000:]
    assert p.returncode == 0, out[-6000:]
    return out


@pytest.fixture(scope="module")
def hipcc():
    if not (shutil.which("hipcc") or os.path.exists("/opt/rocm/bin/hipcc")):
        pytest.skip("hipcc not available")


def test_libcfa_host_under_asan_ubsan(hipcc):
    rt = _clang_rt("asan")
    if rt is None:
        pytest.skip("clang ASan runtime not found")
    lib = _lib_variant("address")
    out = _run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider", "-m",
                "not gpu", "tests/test_kv_cache.py", "tests/test_abi.py"],
               {"CFA_LIB_PATH": lib, "LD_PRELOAD": rt, "ASAN_OPTIONS": "detect_leaks=0"})
    assert " passed" in out


def test_oracle_and_seqsum_emulation_under_asan_ubsan():
    asan, ubsan = _gcc_rt("libasan.so"), _gcc_rt("libubsan.so")
    if asan is None or ubsan is None or not shutil.which("make"):
        pytest.skip("gcc sanitizer runtimes not found")
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "_san/liboracle_asan.so"],
                   check=True)
    emu = os.path.join(NATIVE, "libseqsum_emu_asan.so")
    sys.path.insert(0, ROOT)
    from tests.test_seqsum_emu import build_emu

    build_emu(emu, ("-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"))
    out = _run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                "tests/test_oracle.py", "tests/test_python_mode_oracle.py",
                "tests/test_sampling_oracle.py", "tests/test_tree_oracle.py",
                "tests/test_seqsum_emu.py"],
               {"ORACLE_LIB_PATH": os.path.join(ROOT, "oracle", "_san", "liboracle_asan.so"),
                "SEQSUM_EMU_LIB": emu, "LD_PRELOAD": f"{asan}:{ubsan}",
                "ASAN_OPTIONS": "detect_leaks=0"})
    assert " passed" in out


def test_libcfa_host_page_tables_under_tsan(hipcc):
    clangxx = "/opt/rocm/llvm/bin/clang++"
    if not os.path.exists(clangxx) or _clang_rt("tsan") is None:
        pytest.skip("clang ThreadSanitizer not found")
    lib = _lib_variant("thread")
    src = os.path.join(NATIVE, "threaded_host_calls.cpp")
    exe = os.path.join(SAN, "threaded_host_calls_tsan")
    if _stale(exe, [src, lib, os.path.join(ROOT, "include", "cudaforge_amd.h")]):
        subprocess.run([clangxx, "-std=c++17", "-O1", "-g", "-fsanitize=thread",
                        "-I" + os.path.join(ROOT, "include"), src, "-L" + SAN, "-lcfa_thread",
                        "-Wl,-rpath," + SAN, "-Wl,-rpath,/opt/rocm/lib", "-o", exe], check=True)
    out = _run([exe], {"TSAN_OPTIONS": "halt_on_error=1"}, timeout=600)
    assert "bad=0" in out
