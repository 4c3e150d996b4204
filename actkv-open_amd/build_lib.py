"""Build libactkv_hip.so (the gfx950 C-ABI library) in-tree with hipcc.

    python actkv-open_amd/build_lib.py          # compile every csrc/*.hip, link the .so

Objects go to actkv-open_amd/_build/, the library to actkv-open_amd/actkv/libactkv_hip.so,
where actkv/_hip.py loads it.  hipcc cross-compiles for gfx950 without a GPU.  gcc builds
csrc/pyglue.c into actkv/_glue*.so, the CPython module _hip.py calls the hot entry points through.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "actkv", "libactkv_hip.so")
GLUE = os.path.join(HERE, "actkv", "_glue" + sysconfig.get_config_var("EXT_SUFFIX"))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed fp32 VALU ops stay disabled: the kernels' fp32 math is plain scalar code.
FLAGS = ["--offload-arch=" + ARCH, "-O3", "-std=c++17", "-fPIC", "-Wall",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]


def _run(cmd):
    p = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the gfx950 feature name; that warning is harmless
    err = "\n".join(l for l in p.stderr.splitlines() if "packed-fp32-ops" not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{err}")
    return err


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    objs = [os.path.join(BUILD, os.path.basename(s)[:-4] + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        futs = [ex.submit(_run, [HIPCC, *FLAGS, "-c", s, "-o", o]) for s, o in zip(srcs, objs)]
        for f in futs:
            msg = f.result()
            if verbose and msg.strip():
                print(msg, file=sys.stderr)
    tmp = LIB + ".tmp"
    _run([HIPCC, "--offload-arch=" + ARCH, "-shared", "-fPIC", *objs, "-o", tmp])
    os.replace(tmp, LIB)
    build_glue()
    return LIB


def build_glue() -> str:
    """The CPython module that calls the library's hot entry points (host code only: gcc)."""
    tmp = GLUE + ".tmp"
    _run(["gcc", "-O2", "-shared", "-fPIC", "-Wall", "-Wextra", "-Wconversion", "-Werror",
          "-Wno-unused-parameter", "-I" + sysconfig.get_paths()["include"],
          "-I" + os.path.join(ROOT, "include"), os.path.join(CSRC, "pyglue.c"), "-o", tmp])
    os.replace(tmp, GLUE)
    return GLUE


if __name__ == "__main__":
    print(build(verbose=True))
