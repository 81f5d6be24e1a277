"""`oxmera doctor` on the MI355X box, live: the probe runs the real
rocminfo (crates/oxmera-cli/src/probe.rs:48-72 is where the reference probes
its toolchains) and the report's ROCm backend path must say a gfx950 is
visible.  The fixture-driven goldens are in tests/test_doctor.py."""
import shutil
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent.parent / "oxmera_amd" / "bin" / "oxmera"


def test_doctor_sees_the_gfx950_live():
    assert EXE.exists(), "oxmera_amd/bin/oxmera is not built"
    assert shutil.which("rocminfo") or Path("/opt/rocm/bin/rocminfo").exists(), "no rocminfo on this box"
    print("doctor live", flush=True)
    res = subprocess.run([str(EXE), "doctor"], capture_output=True, text=True, timeout=60)
    print(res.stdout, flush=True)
    assert res.returncode == 0, res.stderr
    rocm = [ln for ln in res.stdout.splitlines() if ln.strip().startswith("rocm ")]
    assert len(rocm) == 1, res.stdout
    assert "gfx950 visible" in rocm[0], rocm[0]
    assert "hip-gfx950 backend can run" in rocm[0], rocm[0]
    hipcc = [ln for ln in res.stdout.splitlines() if ln.strip().startswith("hipcc ")]
    assert hipcc and "not found" not in hipcc[0], res.stdout
