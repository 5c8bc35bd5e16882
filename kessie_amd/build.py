"""Build recipe for libkessie_mi355x.so (gfx950), in-tree.

    python -m kessie_amd.build            # compile every csrc/*.hip and link

Each translation unit is compiled to an object with hipcc in parallel, then
linked into ``kessie_amd/libkessie_mi355x.so``.  The library is what the ctypes
loader (kessie_amd/kessie_hip_ctypes.py) opens; nothing is JIT-compiled at
import time.  The same call builds the measurement-only companion
``kessie_amd/probes/libkessie_probes.so`` (HBM ceiling probes that bench.py
loads; not part of the product library).
"""
from __future__ import annotations

import concurrent.futures as _fut
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libkessie_mi355x.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
PROBES_DIR = os.path.join(PKG_DIR, "probes")
PROBES_LIB_PATH = os.path.join(PROBES_DIR, "libkessie_probes.so")
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: never emit packed fp32 VALU ops (v_pk_fma_f32 & co).
# -ffp-contract=fast-honor-pragmas: contraction allowed except where a kernel
#  turns it off with `#pragma clang fp contract(off)` (the RoPE remap does, to
#  round each product separately).
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=fast-honor-pragmas",
    "-fno-gpu-rdc",
    "-fvisibility=hidden",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def sources() -> list[str]:
    return sorted(
        os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip")
    )


def _compile(src: str, extra: list[str], subdir: str = "") -> str:
    out_dir = os.path.join(BUILD_DIR, subdir)
    os.makedirs(out_dir, exist_ok=True)
    obj = os.path.join(out_dir, os.path.basename(src)[:-4] + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *extra, "-c", src, "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            f"hipcc failed for {os.path.basename(src)}:\n{' '.join(cmd)}\n"
            f"{proc.stdout}\n{proc.stderr}"
        )
    # Surface warnings other than the known harmless host-pass notice about
    # the packed-fp32 feature flag.
    warn = "\n".join(
        ln for ln in proc.stderr.splitlines()
        if ln.strip() and "packed-fp32-ops" not in ln and "not a recognized feature" not in ln
    )
    if warn:
        print(warn, file=sys.stderr)
    return obj


def build(verbose: bool = True, jobs: int | None = None, extra: list[str] | None = None) -> str:
    """Compile all HIP sources for gfx950 and link the shared library.

    Always recompiles (the caller asked for a build).  Returns the .so path.
    """
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    extra = list(extra or [])
    jobs = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    probe_srcs = sorted(os.path.join(PROBES_DIR, f) for f in os.listdir(PROBES_DIR) if f.endswith(".hip"))
    with _fut.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra), srcs))
        probe_objs = list(ex.map(lambda s: _compile(s, extra, "probes"), probe_srcs))
    _link(objs, LIB_PATH)
    _link(probe_objs, PROBES_LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(srcs)} sources and {PROBES_LIB_PATH}")
    return LIB_PATH


def _link(objs: list[str], path: str) -> None:
    tmp = path + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, path)


def clean() -> None:
    shutil.rmtree(BUILD_DIR, ignore_errors=True)
    for path in (LIB_PATH, PROBES_LIB_PATH):
        if os.path.exists(path):
            os.remove(path)


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "clean":
        clean()
    else:
        build()
