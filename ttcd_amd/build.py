"""Build libttcd_amd.so (gfx950) in-tree with hipcc.

Each HIP source is compiled to an object in parallel, then linked into
ttcd_amd/lib/libttcd_amd.so. The library is a plain C ABI (include/ttcd.h);
Python binds it with ctypes (ttcd_amd/_lib.py), so no torch headers are
compiled and the same .so serves any C/C++/FFI caller.

    python -m ttcd_amd.build            # build
    python -m ttcd_amd.build --verbose
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libttcd_amd.so")

SOURCES = ["attn.hip", "conv.hip", "merge.hip", "prologue.hip", "epilogue.hip", "ttt.hip", "api.hip"]
# attn.hip has no NaN-dependent logic; without IEEE mode max/min of MFMA
# results need no canonicalising moves.
SOURCE_FLAGS = {"attn.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"]}
ARCH = "gfx950"

# -packed-fp32-ops: keep hipcc from emitting v_pk_{add,mul,fma}_f32.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n"
                           f"{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        # hipcc's host pass warns about the gfx-only target feature; keep other output.
        lines = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
        if lines:
            print("\n".join(lines), flush=True)


def build(verbose: bool = False, jobs: int | None = None, out: str | None = None,
          defines: tuple[str, ...] = ()) -> str:
    """Compile every HIP source for gfx950 and link the shared library (to `out`,
    default ttcd_amd/lib/libttcd_amd.so; `defines` are extra -D flags)."""
    hipcc = _hipcc()
    out = out or LIB_PATH
    build_dir = BUILD_DIR if out == LIB_PATH else out + ".objs"
    os.makedirs(build_dir, exist_ok=True)
    os.makedirs(os.path.dirname(out), exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(build_dir, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, *SOURCE_FLAGS.get(src, []), *[f"-D{d}" for d in defines],
                     "-I", INCLUDE, "-I", CSRC, "-c", os.path.join(CSRC, src), "-o", obj])
    jobs = jobs or min(len(cmds), max(1, (os.cpu_count() or 4) // 2))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = out + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose="--verbose" in sys.argv))
