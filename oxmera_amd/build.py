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

# the GEMM instantiations are spread over several units, compiled in parallel
# (a full build: ~10.5 minutes on 8 cores, against ~25 as three units)
SOURCES = ["oxm_capi.cpp", "gemm.hip", "gemm_f32.hip", "gemm_f32_rs.hip", "gemm_f32_dl256.hip", "gemm_f32_dl64.hip",
           "gemm_bf16.hip", "gemm_bf16_1w.hip", "gemm_f16.hip", "gemm_f16_1w.hip", "gemm_strip.hip", "glue.hip",
           "elementwise.hip", "elementwise_int.hip"]

# -packed-fp32-ops off: hipcc must not form v_pk_{add,mul,fma}_f32 on this pool.
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wno-unused-command-line-argument"]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found: the gfx950 backend cannot be built")
    return exe


# Units whose kernels issue global_load_lds with the short hazard pad: their
# device assembly is kept (-save-temps) and checked by check_dma_hazards.
CHECKED = ("gemm_bf16.hip", "gemm_bf16_1w.hip", "gemm_f16.hip", "gemm_f16_1w.hip", "gemm_f32.hip",
           "gemm_f32_rs.hip", "gemm_f32_dl256.hip", "gemm_f32_dl64.hip")


def _compile(src: str) -> Path:
    obj = BUILD / (src.replace(".", "_") + ".o")
    lang = ["-x", "hip"]
    extra = []
    if src in CHECKED:
        tmp = BUILD / ("tmp_" + src.replace(".", "_"))
        tmp.mkdir(exist_ok=True)
        extra = [f"-save-temps={'obj'}"]
        obj_in_tmp = tmp / obj.name
        cmd = [_hipcc(), *COMMON, *extra, *lang, "-c", str(CSRC / src), "-o", str(obj_in_tmp)]
    else:
        cmd = [_hipcc(), *COMMON, *lang, "-c", str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    if src in CHECKED:
        asm = [f for f in tmp.iterdir() if f.name.endswith("gfx950.s")]
        problems = [p for f in asm for p in check_dma_hazards(f.read_text())]
        if not asm:
            problems = [f"no device assembly for {src}"]
        if problems:
            raise RuntimeError(f"{src}: DMA hazard check failed:\n" + "\n".join(problems[:20]))
        os.replace(obj_in_tmp, obj)
        shutil.rmtree(tmp, ignore_errors=True)
    return obj


def _sgprs(tok: str) -> set:
    """SGPR numbers named by an operand token: s5, s[2:3]."""
    import re
    m = re.fullmatch(r"s(\d+)", tok)
    if m:
        return {int(m.group(1))}
    m = re.fullmatch(r"s\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    return set()


def check_dma_hazards(asm: str) -> list:
    """Every global_load_lds_dwordx4 preceded by the short pad (s_nop 0) must
    have no VALU write of its base SGPRs within the 5 wait states a VMEM read
    of a VALU-written SGPR needs (each instruction counts one, s_nop N counts
    N + 1; a label ends the search as unsafe, since a predecessor block could
    end with such a write).  Returns a description of each violation."""
    import re
    lines = []
    for raw in asm.splitlines():
        t = raw.split(";", 1)[0].strip()
        if not t or (t.startswith(".") and not t.endswith(":")):
            continue  # blank or a directive (labels such as .LBB0_3: are kept)
        lines.append(t)
    problems = []
    for i, t in enumerate(lines):
        if not t.startswith("global_load_lds_dwordx4"):
            continue
        ops = [o.strip() for o in t.split(None, 1)[1].split(",")]
        base = _sgprs(ops[1]) if len(ops) > 1 else set()
        # the asm block: s_mov_b32 m0, sX / s_nop N / the load
        if i < 2 or not lines[i - 1].startswith("s_nop") or not lines[i - 2].startswith("s_mov_b32 m0"):
            problems.append(f"unexpected sequence before: {t}")
            continue
        if int(lines[i - 1].split()[1], 0) >= 4:
            continue  # the full pad
        waits, j = 0, i - 1
        while j >= 0 and waits < 5:
            u = lines[j]
            if u.endswith(":"):
                problems.append(f"block boundary within 5 wait states of a short-pad DMA: {t}")
                break
            mn = u.split()[0]
            if mn.startswith("v_"):
                dst = [o.strip() for o in u.split(None, 1)[1].split(",")][:2] if " " in u else []
                if any(_sgprs(d) & base for d in dst):
                    problems.append(f"VALU write of the DMA base within {waits} wait states: {u} -> {t}")
                    break
            waits += int(u.split()[1], 0) + 1 if mn == "s_nop" else 1
            j -= 1
    return problems


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
