"""Build driver for ``libcfa.so`` -- the gfx950 HIP kernels behind the C ABI.

Every ``csrc/*.hip`` and ``csrc/*.cpp`` file is compiled by ``hipcc`` for
gfx950 into an object under ``csrc/_build/`` (in parallel), then linked into
``cudaforge_amd/libcfa.so``.  ``hipcc`` cross-compiles without a GPU, so this
runs on any host with ROCm installed.

Run ``python -m cudaforge_amd._build`` (or ``__graft_entry__.build()``).

``--sanitize address`` / ``--sanitize thread`` builds a variant whose HOST
code (entry points, argument checks, page tables, the host RNG) is
instrumented with AddressSanitizer + UndefinedBehaviorSanitizer or
ThreadSanitizer, into ``cudaforge_amd/_san/libcfa_<kind>.so``; device code is
compiled as usual.  These variants are for CPU-only test runs (the sanitizer
runtime is preloaded into the test process, and ``CFA_LIB_PATH`` points the
package at the variant); they are never run on a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG, "csrc")
OBJ = os.path.join(CSRC, "_build")
LIB = os.path.join(PKG, "libcfa.so")
ARCH = os.environ.get("CFA_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: hipcc must not emit v_pk_{add,mul,fma}_f32 (some of their
# forms have produced wrong results on this hardware pool).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I" + os.path.join(os.path.dirname(PKG), "include"),
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def sources() -> list[str]:
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp"))
    )


# host-only instrumentation: each -fsanitize= applies to the host pass only
SANITIZE_FLAGS = {
    "address": ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host",
                "-fno-omit-frame-pointer", "-g"],
    "thread": ["-Xarch_host", "-fsanitize=thread", "-Xarch_host", "-fno-omit-frame-pointer",
               "-g"],
}
SAN_DIR = os.path.join(PKG, "_san")


def _compile(src: str, hipcc: str, verbose: bool, objdir: str = OBJ,
             extra: tuple = ()) -> str:
    obj = os.path.join(objdir, os.path.basename(src) + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, *extra, "-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass warns that it does not know the packed-fp32 feature
    noise = [ln for ln in (res.stderr or "").splitlines() if "packed-fp32-ops" not in ln]
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n" + "\n".join(noise))
    if verbose and any(ln.strip() for ln in noise):
        sys.stderr.write("\n".join(noise) + "\n")
    return obj


def build(verbose: bool = False, jobs: int | None = None, sanitize: str | None = None) -> str:
    """Compile every kernel source and link libcfa.so (or, with `sanitize`,
    the host-instrumented variant under _san/); returns its path."""
    hipcc = _hipcc()
    objdir, lib, extra = OBJ, LIB, ()
    if sanitize is not None:
        if sanitize not in SANITIZE_FLAGS:
            raise ValueError(f"sanitize must be one of {sorted(SANITIZE_FLAGS)}")
        objdir = os.path.join(SAN_DIR, "obj_" + sanitize)
        lib = os.path.join(SAN_DIR, f"libcfa_{sanitize}.so")
        extra = tuple(SANITIZE_FLAGS[sanitize])
    os.makedirs(objdir, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc, verbose, objdir, extra), srcs))
    tmp = lib + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link of {os.path.basename(lib)} failed:\n" + res.stderr)
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    san = None
    if "--sanitize" in sys.argv:
        san = sys.argv[sys.argv.index("--sanitize") + 1]
    print(build(verbose=True, sanitize=san))
