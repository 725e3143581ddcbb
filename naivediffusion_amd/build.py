"""Builds libndx.so (the HIP library behind include/ndx.h) for gfx950.

Every source under csrc/ is compiled by hipcc into _build/ and linked into
naivediffusion_amd/libndx.so, in-tree, so the built library travels with the
repository snapshot to the machine that runs it. Run as
``python -m naivediffusion_amd.build`` or through ``__graft_entry__.build()``.
"""

from __future__ import annotations

import concurrent.futures
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libndx.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-fvisibility=hidden",
    # Packed fp32 instructions stay off: hipcc emits ordinary scalar fp32.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Small per-thread arrays (staged tile chunks) stay in registers: every
    # kernel here manages its LDS explicitly, and an array moved into LDS
    # costs a workgroup slot per CU and extra LDS traffic.
    "-mllvm", "-disable-promote-alloca-to-lds",
    "-Wno-unused-result",
]


def source_hash() -> str:
    """SHA-256 (first 16 hex digits) of every source the library is built
    from and the flags it is built with. The build embeds it in
    ndx_version(); the loader compares it with the sources beside the
    library and refuses a library built from other sources."""
    h = hashlib.sha256()
    files = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp")) + sorted(CSRC.glob("*.h"))
    files.append(PACKAGE.parent / "include" / "ndx.h")
    for f in files:
        h.update(f.name.encode())
        h.update(b"\0")
        h.update(f.read_bytes())
        h.update(b"\0")
    h.update(" ".join(HIPCC_FLAGS).encode())
    return h.hexdigest()[:16]


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found: the HIP library cannot be built")


def _compile(src: Path, digest: str) -> Path:
    obj = BUILD / (src.name + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, f'-DNDX_SOURCE_HASH="{digest}"', "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd.insert(1, "-xhip")
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature flag; that
    # warning is expected and harmless.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))
    digest = source_hash()
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as pool:
        objects = list(pool.map(lambda src: _compile(src, digest), sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking libndx.so failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(sources)} sources (source hash {digest})")
    return LIBRARY


if __name__ == "__main__":
    build()
