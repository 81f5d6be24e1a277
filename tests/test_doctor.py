"""`oxmera doctor` (oxmera_amd/cli/doctor.cpp): the reference's own doctor
tests (crates/oxmera-cli/tests/doctor.rs:65-124) on its own fixtures and
goldens, copied as data into tests/golden/doctor/, plus the ROCm shapes.

A golden's first line is the terminal-size / cursor header of the
reference's PTY capture ("size: 100x45  cursor: <row>,0"); the rest is the
rendered report, compared after trimming trailing blanks per line
(doctor.rs:34-41).  The cursor row is the number of lines printed.
Regenerate the ROCm goldens after an intentional change with
OXMERA_BLESS=1 (the reference's goldens are never rewritten).
"""
import os
import stat
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
GOLD = ROOT / "tests" / "golden" / "doctor"
REFERENCE_SHAPES = ["no-gpu", "metal", "cuda"]
ROCM_SHAPES = ["rocm-mi355x", "rocm-other-gpu", "rocm-toolkit-only", "rocm-absent"]


@pytest.fixture(scope="module")
def oxmera():
    exe = ROOT / "oxmera_amd" / "bin" / "oxmera"
    if not exe.exists():
        from oxmera_amd import build as b
        b.build_cli(verbose=False)
    return exe


def run(exe, *args, env=None, cwd=None):
    return subprocess.run([str(exe), *args], capture_output=True, text=True, env=env, cwd=cwd, timeout=30)


def normalize(text: str) -> str:
    return "\n".join(l.rstrip() for l in text.splitlines()).rstrip()


def screen(exe, shape):
    r = run(exe, "doctor", "--fixture", str(GOLD / f"{shape}.toml"), env={}, cwd=str(GOLD))
    assert r.returncode == 0, r.stderr
    assert r.stdout.endswith("doctor: report complete\n")
    return r.stdout


def check_golden(name, out, bless=False):
    header = f"size: 100x45  cursor: {out.count(chr(10))},0"
    path = GOLD / name
    if bless and os.environ.get("OXMERA_BLESS"):
        path.write_text(header + "\n" + normalize(out) + "\n")
    lines = path.read_text().split("\n", 1)
    assert lines[0].strip() == header
    assert normalize(lines[1]) == normalize(out), f"frame differs from golden {name}"


@pytest.mark.parametrize("shape", REFERENCE_SHAPES)
def test_reference_goldens_byte_identical(oxmera, shape):
    out = screen(oxmera, shape)
    check_golden(f"doctor-{shape}-100x45.txt", out)
    if shape == "no-gpu":
        assert "install cargo-reconverge" in out and "metered" in out
    if shape == "metal":
        assert "no convergence gate exists on this path" in out and "1 solved" in out
    if shape == "cuda":
        assert "metered — approved GPU sessions only" in out and "per-part" in out
    assert "rocm" not in out and "hipcc" not in out     # no gpu.rocm key: the reference's frame


@pytest.mark.parametrize("shape", ROCM_SHAPES)
def test_rocm_goldens(oxmera, shape):
    out = screen(oxmera, shape)
    check_golden(f"doctor-{shape}-100x45.txt", out, bless=True)
    rocm = [l for l in out.splitlines() if l.startswith("  rocm    ")]
    assert len(rocm) == 1
    want = {"rocm-mi355x": "gfx950 visible", "rocm-other-gpu": "devices gfx942",
            "rocm-toolkit-only": "no device listed", "rocm-absent": "no ROCm toolkit here"}[shape]
    assert want in rocm[0]
    assert "AMD execution (hip-gfx950)        metered" in out   # a visible GPU is not permission to spend


def test_stress_100_iterations_are_identical(oxmera):
    first = normalize(screen(oxmera, "no-gpu"))
    for i in range(1, 100):
        assert normalize(screen(oxmera, "no-gpu")) == first, f"iteration {i}"


def test_usage_and_errors(oxmera, tmp_path):
    r = run(oxmera)
    assert r.returncode == 1 and "usage: oxmera <doctor [--fixture <path>] | --version>" in r.stderr
    r = run(oxmera, "doctor", "--bogus")
    assert r.returncode == 1 and "usage: oxmera doctor [--fixture <path>]" in r.stderr
    r = run(oxmera, "doctor", "--fixture", str(tmp_path / "missing.toml"))
    assert r.returncode == 1 and "cannot read fixture" in r.stderr
    bad = tmp_path / "bad.toml"
    bad.write_text('os = "linux"\narch = "x86_64"\n[toolchain]\ncontainer = false\n')   # no [gpu]
    r = run(oxmera, "doctor", "--fixture", str(bad))
    assert r.returncode == 1 and "cannot parse fixture" in r.stderr and "gpu" in r.stderr
    bad.write_text('os = "linux\n')
    r = run(oxmera, "doctor", "--fixture", str(bad))
    assert r.returncode == 1 and "unterminated string" in r.stderr
    r = run(oxmera, "--version")
    assert r.returncode == 0 and r.stdout.startswith("oxmera ")


def _fake_tool(dirpath: Path, name: str, text: str):
    p = dirpath / name
    body = text.replace("'", "'\\''")
    p.write_text("#!/bin/sh\nprintf '%s' '" + body + "'\n")   # printf: a shell builtin, PATH-independent
    p.chmod(p.stat().st_mode | stat.S_IXUSR | stat.S_IXGRP | stat.S_IXOTH)


def test_probe_detects_gfx950_through_rocminfo(oxmera, tmp_path):
    # stand-ins for rocminfo / hipcc on PATH: the probe parses their output
    _fake_tool(tmp_path, "rocminfo", "ROCk module is loaded\n*******\nAgent 1\n  Name:                    AMD EPYC\n"
                                     "Agent 2\n  Name:                    gfx950\n  Marketing Name: AMD Instinct MI355X\n"
                                     "Agent 3\n  Name:                    gfx950\n")
    _fake_tool(tmp_path, "hipcc", "HIP version: 9.9.9-stand-in\nclang\n")
    r = run(oxmera, "doctor", env={"PATH": str(tmp_path)}, cwd=str(tmp_path))
    assert r.returncode == 0, r.stderr
    assert "  hipcc        HIP version: 9.9.9-stand-in" in r.stdout
    assert "  rocm    gfx950 visible — the hip-gfx950 backend can run" in r.stdout
    assert "no exercises/manifest.toml found from here" in r.stdout


def test_probe_without_rocm_and_with_a_ladder(oxmera, tmp_path):
    (tmp_path / "exercises").mkdir()
    (tmp_path / "exercises" / "manifest.toml").write_text(
        '[[exercise]]\nid = "a1"\nname = "shape and strides"\ntools = ["cargo"]\nstatus = "solved"\n\n'
        '[[exercise]]\nid = "b1"\nname = "first kernel"\nstatus = "todo"\n')
    sub = tmp_path / "exercises" / "deeper"
    sub.mkdir()
    r = run(oxmera, "doctor", env={"PATH": str(tmp_path / "nothing-here")}, cwd=str(sub))
    assert r.returncode == 0, r.stderr
    assert "  rocm    no ROCm toolkit here" in r.stdout and "  hipcc        not found" in r.stdout
    assert "1 solved, 1 todo, 0 planned" in r.stdout and "[x] a1   shape and strides" in r.stdout
