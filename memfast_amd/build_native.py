"""Ahead-of-time build of libmemfast_hip.so for gfx950.

Replaces the reference's per-Config NVRTC compilation (memfast/cuda.py:130-204):
every kernel is compiled once, with the physical constants passed at run time
in the mf_config descriptor.  Run ``python -m memfast_amd.build_native``.
"""

import concurrent.futures
import hashlib
import os
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
SOURCES = PACKAGE / "csrc"
HEADER = PACKAGE.parent / "include" / "memfast_hip.h"
OBJECTS = PACKAGE / "_build"
LIBRARY = PACKAGE / "lib" / "libmemfast_hip.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # No implicit FMA contraction: the CPU reference rounds every product and
    # sum separately (explicit fma() calls are kept where intended).
    "-ffp-contract=off",
    # Packed FP32 VALU forms are kept out of every kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def source_files():
    return sorted(SOURCES.glob("*.hip"))


def source_hash():
    """SHA-256 over every native source and the public header."""
    digest = hashlib.sha256(" ".join(FLAGS).encode())
    for path in [*sorted(SOURCES.glob("*")), HEADER]:
        if path.is_file() and path.suffix in (".hip", ".h"):
            digest.update(path.name.encode())
            digest.update(path.read_bytes())
    return digest.hexdigest()


def _compile(source, defines):
    obj = OBJECTS / (source.stem + ".o")
    cmd = [HIPCC, *FLAGS, *defines, "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{proc.stderr}")
    return obj


def build(verbose=False):
    OBJECTS.mkdir(exist_ok=True)
    LIBRARY.parent.mkdir(exist_ok=True)
    defines = [f'-DMF_SOURCE_HASH="{source_hash()}"']
    files = source_files()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(files))) as pool:
        objects = list(pool.map(lambda s: _compile(s, defines), files))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
