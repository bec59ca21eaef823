"""Run the C++ host-layer test program (tests/cpp/test_host.cpp): GGUF
parsing, the reference's name map and quantized/f32 classification, malformed
files (CPU), then loading the tiny GGUF onto the device and QMatMul::forward
parity against the committed expectations (GPU)."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_host")
GGUF = os.path.join(ROOT, "tests", "golden", "tiny_llama_q4_0.gguf")
EXPECT = os.path.join(ROOT, "tests", "golden", "tiny_llama_q4_0.expect")


def _run(mode):
    assert os.path.exists(BIN), "build first: python -m unillm_amd.build"
    r = subprocess.run([BIN, mode, GGUF, EXPECT], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    assert "0 failed" in r.stdout


def test_host_cpu():
    _run("cpu")


@pytest.mark.gpu
def test_host_gpu():
    _run("gpu")
