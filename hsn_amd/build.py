"""Build the HIP library ``hsn_amd/libhsn_amd.so`` for gfx950 (MI355X), in-tree.

``python -m hsn_amd.build`` (or ``__graft_entry__.build()``) compiles every source under
``hsn_amd/csrc`` with ``hipcc --offload-arch=gfx950`` in parallel and links one shared library
exporting the C ABI of ``include/hsn_window.h`` and ``include/hsn_ops.h``. A manifest
(``hsn_amd/libhsn_amd.json``) records the SHA-256 of every source and of the library, so the
loader can refuse a library built from other sources.
"""

from __future__ import annotations

import concurrent.futures
import hashlib
import json
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = ROOT / "_build"
LIBRARY = PKG / "libhsn_amd.so"
MANIFEST = PKG / "libhsn_amd.json"
ARCH = "gfx950"

#: hipcc flags. Packed fp32 arithmetic is switched off (the compiler would otherwise form
#: v_pk_* fp32 ops from scalar code); a*b+c may fuse where written apart, except where a file
#: says `#pragma clang fp contract(off)` (the router: the CPU path rounds every operation).
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-ffp-contract=fast-honor-pragmas",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def headers() -> list[Path]:
    return sorted(list(CSRC.glob("*.h")) + list(CSRC.glob("*.cuh")) +
                  list((ROOT / "include").glob("*.h")))


def _sha(path: Path) -> str:
    return hashlib.sha256(path.read_bytes()).hexdigest()


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: the HIP library cannot be built")
    return found


def _stamp(src: Path) -> str:
    """Digest of what an object depends on: the source, every header and the flags."""
    h = hashlib.sha256(" ".join(HIP_FLAGS).encode())
    for path in [src, *headers()]:
        h.update(path.read_bytes())
    return h.hexdigest()


def _compile(src: Path, incremental: bool = False) -> Path:
    obj = BUILD / (src.name + ".o")
    stamp = BUILD / (src.name + ".stamp")
    digest = _stamp(src)
    if incremental and obj.is_file() and stamp.is_file() and stamp.read_text() == digest:
        return obj
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr[-6000:]}")
    stamp.write_text(digest)
    return obj


def build(verbose: bool = False, incremental: bool = False) -> Path:
    """Compile and link the library; returns its path. ``incremental`` reuses an object whose
    source, headers and flags are unchanged since it was compiled (the default compiles all)."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(jobs, 1)) as pool:
        objs = list(pool.map(lambda src: _compile(src, incremental), srcs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-6000:]}")
    os.replace(tmp, LIBRARY)
    manifest = {
        "arch": ARCH,
        "library_sha256": _sha(LIBRARY),
        "sources": {str(p.relative_to(ROOT)): _sha(p) for p in srcs + headers()},
        "flags": HIP_FLAGS,
    }
    MANIFEST.write_text(json.dumps(manifest, indent=1, sort_keys=True) + "\n")
    if verbose:
        print(f"built {LIBRARY} ({LIBRARY.stat().st_size} bytes) from {len(srcs)} sources")
    return LIBRARY


#: The host helper module (``hsn_amd/host/tables.cpp``): the trainer's pointer tables, built with
#: the host compiler against the installed PyTorch's headers and libraries.
HOST_SOURCE = PKG / "host" / "tables.cpp"
HOST_MODULE = PKG / "_tables.so"
HOST_MANIFEST = PKG / "_tables.json"


def build_host(verbose: bool = False) -> Path:
    """Compile ``hsn_amd/_tables.so`` (CPython extension, host code only); returns its path."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    torch_lib = str(Path(torch.__file__).resolve().parent / "lib")
    tmp = HOST_MODULE.with_suffix(".so.tmp")
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           *[f"-isystem{p}" for p in cpp_extension.include_paths()],
           f"-isystem{sysconfig.get_paths()['include']}",
           str(HOST_SOURCE), "-o", str(tmp),
           f"-L{torch_lib}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python",
           f"-Wl,-rpath,{torch_lib}"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"host helper build failed:\n{proc.stderr[-6000:]}")
    os.replace(tmp, HOST_MODULE)
    HOST_MANIFEST.write_text(json.dumps({"source_sha256": _sha(HOST_SOURCE),
                                         "module_sha256": _sha(HOST_MODULE)}, indent=1) + "\n")
    if verbose:
        print(f"built {HOST_MODULE} ({HOST_MODULE.stat().st_size} bytes)")
    return HOST_MODULE


def host_stale() -> str | None:
    """Why ``hsn_amd/_tables.so`` is not the build of the current source, or None."""
    if not HOST_MODULE.is_file() or not HOST_MANIFEST.is_file():
        return "hsn_amd/_tables.so is not built"
    manifest = json.loads(HOST_MANIFEST.read_text())
    if manifest.get("module_sha256") != _sha(HOST_MODULE):
        return "hsn_amd/_tables.so differs from its build manifest"
    if manifest.get("source_sha256") != _sha(HOST_SOURCE):
        return "hsn_amd/host/tables.cpp changed since hsn_amd/_tables.so was built"
    return None


def stale() -> str | None:
    """Why the built library does not match the sources (None: it matches)."""
    if not LIBRARY.is_file() or not MANIFEST.is_file():
        return "the HIP library is not built (python -m hsn_amd.build)"
    manifest = json.loads(MANIFEST.read_text())
    if manifest.get("library_sha256") != _sha(LIBRARY):
        return "libhsn_amd.so differs from its build manifest"
    for name, digest in manifest.get("sources", {}).items():
        path = ROOT / name
        if not path.is_file() or _sha(path) != digest:
            return f"source changed since the build: {name}"
    for path in sources() + headers():
        if str(path.relative_to(ROOT)) not in manifest.get("sources", {}):
            return f"source added since the build: {path.relative_to(ROOT)}"
    return None


if __name__ == "__main__":
    build(verbose=True, incremental="--incremental" in sys.argv[1:])
    build_host(verbose=True)
    sys.exit(0)
