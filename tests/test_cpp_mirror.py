"""The C++ host mirror (include/oxmera.hpp) and the spec ladder restated in
C++ (tests/cpp/spec_tests.cpp): host-side cases here, A4 on the GPU."""
import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIBDIR = ROOT / "oxmera_amd"


@pytest.fixture(scope="module")
def spec_binary(tmp_path_factory):
    exe = tmp_path_factory.mktemp("cpp") / "spec_tests"
    cmd = ["g++", "-std=c++17", "-O1", "-Wall", "-I", str(ROOT / "include"), str(ROOT / "tests/cpp/spec_tests.cpp"),
           "-L", str(LIBDIR), "-loxm", f"-Wl,-rpath,{LIBDIR}", "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return exe


def test_cpp_spec_host(spec_binary):
    res = subprocess.run([str(spec_binary)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert " 0 failed" in res.stdout


@pytest.mark.gpu
def test_cpp_spec_gpu(spec_binary):
    res = subprocess.run([str(spec_binary), "--gpu"], capture_output=True, text=True, timeout=120)
    print(res.stdout, flush=True)
    assert res.returncode == 0, res.stdout + res.stderr
    assert " 0 failed" in res.stdout
