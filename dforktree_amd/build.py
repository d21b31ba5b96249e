"""Build the gfx950 HIP library in-tree: dforktree_amd/libdforktree_amd.so.

    python -m dforktree_amd.build        (or __graft_entry__.build())

Every csrc/*.hip is compiled to an object with hipcc (in parallel) and linked
into one shared library that exports the C ABI of include/dforktree_amd.h.
calib/stream_copy.hip, the streaming copy that bench.py times as the
achievable-bandwidth reference, goes into a library of its own
(dforktree_amd/libdft_stream_copy.so, ``build_calibration``), outside the C
ABI; a failure there is reported as a warning and leaves the product
library in place.
Packed-fp32 instruction selection is disabled for all device code.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
INCLUDE = PKG.parent / "include"
BUILD = PKG / "_build"
LIB = PKG / "libdforktree_amd.so"
CALIB_SRC = PKG / "calib" / "stream_copy.hip"
CALIB_LIB = PKG / "libdft_stream_copy.so"
ARCH = os.environ.get("DFT_OFFLOAD_ARCH", "gfx950")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # the host pass does not know the packed-fp32 feature and says so: drop that line
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    return r.returncode, out


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [BUILD / (s.stem + ".o") for s in sources]
    cmds = [[HIPCC, *COMMON, "-c", str(s), "-o", str(o)] for s, o in zip(sources, objs)]
    with ThreadPoolExecutor(max_workers=min(len(cmds), os.cpu_count() or 4)) as ex:
        results = list(ex.map(_run, cmds))
    for cmd, (rc, out) in zip(cmds, results):
        if verbose and out.strip():
            print(out, file=sys.stderr)
        if rc != 0:
            raise RuntimeError(f"hipcc failed ({rc}): {' '.join(cmd)}\n{out}")
    tmp = LIB.with_suffix(".so.tmp")
    rc, out = _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    if rc != 0:
        raise RuntimeError(f"link failed ({rc}):\n{out}")
    os.replace(tmp, LIB)
    try:
        build_calibration()
    except RuntimeError as e:  # a bench-only artefact: the product library is built
        print(f"warning: {e}", file=sys.stderr)
    return LIB


def build_calibration() -> Path:
    """Compile the streaming-copy library that bench.py times as the
    achievable-bandwidth reference (outside the C ABI); returns its path."""
    tmp = CALIB_LIB.with_suffix(".so.tmp")
    rc, out = _run([HIPCC, *COMMON, "-shared", str(CALIB_SRC), "-o", str(tmp)])
    if rc != 0:
        raise RuntimeError(f"hipcc failed ({rc}) on {CALIB_SRC}:\n{out}")
    os.replace(tmp, CALIB_LIB)
    return CALIB_LIB


if __name__ == "__main__":
    print(build(verbose=True))
