"""Builds libtmoe.so (the C-ABI library of include/tmoe.h) for gfx950 with hipcc.

The library is built in-tree, next to this file, so that it travels with the
source tree. `python -m` is not needed: call build() (the repository's
__graft_entry__.build() does).
"""
from __future__ import annotations

import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libtmoe.so")

SOURCES = ["tmoe_kernels.hip", "tmoe_static.hip", "tmoe_api.cpp"]
# the measurement harness's hardware probes (include/tmoe_probe.h), a library of
# their own so that libtmoe.so holds only the layer
PROBE_SOURCES = ["tmoe_probe.hip"]
PROBE_LIB = os.path.join(HERE, "libtmoe_probe.so")
ARCH = "gfx950"

# Packed FP32 vector instructions are disabled for all device code: hipcc -O3
# would otherwise form them from ordinary float code.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 library cannot be built")


def build(verbose: bool = False) -> str:
    """Compiles every source (concurrently) and links libtmoe.so and
    libtmoe_probe.so; returns libtmoe.so's path."""
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    cmds, groups = [], []
    for lib, sources in ((LIB, SOURCES), (PROBE_LIB, PROBE_SOURCES)):
        objs = []
        for src in sources:
            obj = os.path.join(objdir, src + ".o")
            lang = ["-x", "hip"] if src.endswith(".hip") else []
            cmds.append([hipcc(), *HIPCC_FLAGS, "-I", INCLUDE, "-I", CSRC, *lang, "-c",
                         os.path.join(CSRC, src), "-o", obj])
            objs.append(obj)
        groups.append((lib, objs))
    _run_all(cmds, verbose)
    for lib, objs in groups:
        tmp = lib + ".tmp"
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
               "-Wl,-rpath,/opt/rocm/lib"]
        _run(cmd, verbose)
        os.replace(tmp, lib)
    return LIB


# hipcc's host pass does not know the packed-fp32 feature and says so: harmless.
_NOISE = "'-packed-fp32-ops' is not a recognized feature"


def _run_all(cmds, verbose):
    """Runs the compile commands side by side; raises on the first that failed."""
    procs = []
    for cmd in cmds:
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                                            text=True)))
    failed = None
    for cmd, pr in procs:
        _, stderr = pr.communicate()
        err = "\n".join(l for l in stderr.splitlines() if _NOISE not in l)
        if pr.returncode != 0 and failed is None:
            failed = f"build failed ({pr.returncode}): {' '.join(cmd)}\n{err}"
        elif verbose and err.strip():
            print(err)
    if failed:
        raise RuntimeError(failed)


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in res.stderr.splitlines() if _NOISE not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err)


if __name__ == "__main__":
    print(build(verbose=True))
