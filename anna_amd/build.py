"""Builds libanna_mi.so (the C-ABI HIP library) in-tree for gfx950.

Run as ``python -m anna_amd.build``.  Sources are compiled in parallel with hipcc
and linked with ``hipcc -shared``; the result lands next to this file so it
travels with the source tree.
"""

from __future__ import annotations

import concurrent.futures
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
OBJ_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libanna_mi.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # packed FP32 instructions are kept out of every kernel
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the anna_mi HIP library cannot be built")


def _sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def source_hash() -> str:
    """sha256 over every file of csrc/ and include/ (names and contents, sorted).

    The library is stamped with it (anna_mi_source_hash) and the loader refuses a binary
    whose stamp differs from the sources next to it, so a run provably uses the kernels of
    the tree it ships with."""
    h = hashlib.sha256()
    inc = PKG_DIR.parent / "include"
    files = sorted(p for p in CSRC.iterdir() if p.is_file() and p.suffix in (".hip", ".cpp", ".hpp", ".h"))
    if inc.is_dir():
        files += sorted(p for p in inc.iterdir() if p.is_file() and p.suffix == ".h")
    for p in files:
        h.update(p.name.encode())
        h.update(b"\0")
        h.update(p.read_bytes())
        h.update(b"\0")
    return h.hexdigest()


def _up_to_date(src: Path, obj: Path) -> bool:
    if not obj.exists():
        return False
    deps = [src, *CSRC.glob("*.hpp"), *(PKG_DIR.parent / "include").glob("*.h")]
    return obj.stat().st_mtime > max(p.stat().st_mtime for p in deps)


def _compile(src: Path, stamp: str, force: bool = True) -> Path:
    obj = OBJ_DIR / (src.stem + ".o")
    if not force and src.name != "runtime.cpp" and _up_to_date(src, obj):
        return obj
    cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.name == "runtime.cpp":
        cmd.insert(-4, f'-DANNA_MI_SOURCE_HASH="{stamp}"')
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns about the device-only feature flag; drop that noise.
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(l for l in (proc.stdout + proc.stderr).splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{msgs}")
    if msgs.strip():
        print(msgs, file=sys.stderr)
    return obj


def build(verbose: bool = True, force: bool = True) -> Path:
    """Compiles every source (force=False reuses objects newer than their sources and the
    shared headers; the stamped runtime.cpp is always rebuilt) and links the library."""
    OBJ_DIR.mkdir(exist_ok=True)
    sources = _sources()
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as ex:
        stamp = source_hash()
        objs = list(ex.map(lambda src: _compile(src, stamp, force), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build(force="--incremental" not in sys.argv)
