"""Build the gfx950 backend library ``oxmera_amd/liboxm.so`` in-tree.

Each HIP / C++ translation unit under ``oxmera_amd/csrc`` is compiled with
``hipcc --offload-arch=gfx950`` into ``oxmera_amd/_build`` (in parallel),
then linked into one shared library exporting the C-ABI of
``include/oxm.h``.  hipcc cross-compiles, so this runs without a GPU.

Usage: ``python -m oxmera_amd.build`` (or ``__graft_entry__.build()``);
``python -m oxmera_amd.build --changed`` recompiles only out-of-date units.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "liboxm.so"
ARCH = os.environ.get("OXM_GFX", "gfx950")

SOURCES = ["oxm_capi.cpp", "gemm.hip", "gemm_f32.hip", "gemm_bf16.hip", "gemm_f16.hip", "gemm_strip.hip",
           "glue.hip", "elementwise.hip", "elementwise_int.hip"]

# -packed-fp32-ops off: hipcc must not form v_pk_{add,mul,fma}_f32 on this pool.
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wno-unused-command-line-argument"]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the gfx950 backend cannot be built")
    return exe


def _compile(src: str) -> Path:
    obj = BUILD / (src.replace(".", "_") + ".o")
    lang = ["-x", "hip"]
    cmd = [_hipcc(), *COMMON, *lang, "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


CLI_SRC = PKG / "cli" / "doctor.cpp"
CLI = PKG / "bin" / "oxmera"


def build_cli(verbose: bool = True) -> Path:
    """Compile the ``oxmera`` command (``oxmera doctor``) with the host C++
    compiler; returns its path."""
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("no host C++ compiler: the oxmera command cannot be built")
    CLI.parent.mkdir(exist_ok=True)
    tmp = CLI.with_suffix(".tmp")
    cmd = [cxx, "-O2", "-std=c++17", "-Wall", "-o", str(tmp), str(CLI_SRC)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, CLI)
    if verbose:
        print(f"built {CLI}", flush=True)
    return CLI


def _deps(path: Path, seen: set) -> set:
    """The file and every local header it includes, transitively."""
    import re
    if path in seen or not path.exists():
        return seen
    seen.add(path)
    for inc in re.findall(r'^\s*#\s*include\s+"([^"]+)"', path.read_text(), re.M):
        _deps((path.parent / inc).resolve(), seen)
    return seen


def _stale(src: str) -> bool:
    """Whether a unit's object is older than its source or a header it
    includes."""
    obj = BUILD / (src.replace(".", "_") + ".o")
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    return any(d.stat().st_mtime > t for d in _deps((CSRC / src).resolve(), set()))


def build(verbose: bool = True, changed_only: bool = False) -> Path:
    """Compile every translation unit (with ``changed_only``, only those whose
    object is out of date) and link ``liboxm.so``; returns its path."""
    BUILD.mkdir(exist_ok=True)
    todo = [s for s in SOURCES if not changed_only or _stale(s)]
    jobs = min(max(1, len(todo)), max(1, min(os.cpu_count() or 1, 16)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_compile, todo))
    objs = [BUILD / (s.replace(".", "_") + ".o") for s in SOURCES]
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", flush=True)
    return LIB


if __name__ == "__main__":
    build(changed_only="--changed" in sys.argv[1:])
    build_cli()
    sys.exit(0)
