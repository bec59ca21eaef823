"""Run the C++ host-layer test program (tests/cpp/test_host.cpp): GGUF
parsing, the reference's name map and quantized/f32 classification, malformed
files (CPU), then loading the tiny GGUFs onto the device and QMatMul::forward
parity against the committed expectations, load-time QKV / gate+up fusion, and
the KV-cache mirror (LayerKVCache / KVCache with closed-form attention checks and
the reference's overflow message), and LlamaModel::forward_with_cache over the
tiny Q4_0 model against the f64 logits of tests/golden/tiny_llama_q4_0.step (GPU);
the same for tiny_llama_f16 (dense F16 / F32 / BF16 projections).  The K-quant files
(tiny_llama_q4_k_m: Q4_K + Q6_K; tiny_llama_q5_k_m: Q5_K + Q6_K) are checked for their
plan, per-tensor parity and fusion."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "test_host")
GOLDEN = os.path.join(ROOT, "tests", "golden")


def _run(mode, stem="tiny_llama_q4_0", data=".expect"):
    assert os.path.exists(BIN), "build first: python -m unillm_amd.build"
    gguf, expect = (os.path.join(GOLDEN, stem + ext) for ext in (".gguf", data))
    r = subprocess.run([BIN, mode, gguf, expect], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    assert "0 failed" in r.stdout


def test_host_cpu():
    _run("cpu")


@pytest.mark.gpu
def test_host_gpu():
    _run("gpu")


def test_host_k_quants_cpu():
    _run("cpu-kq", "tiny_llama_q4_k_m")


@pytest.mark.gpu
def test_host_k_quants_gpu():
    _run("gpu-kq", "tiny_llama_q4_k_m")


def test_host_q5_k_m_cpu():
    _run("cpu-kq", "tiny_llama_q5_k_m")


@pytest.mark.gpu
def test_host_q5_k_m_gpu():
    _run("gpu-kq", "tiny_llama_q5_k_m")


@pytest.mark.gpu
def test_host_model_step_gpu():
    _run("gpu-step", data=".step")


@pytest.mark.gpu
def test_host_dense_gpu():
    # F16 / F32 / BF16 projections (candle's dequantized QMatMul), loaded and fused
    _run("gpu-dense", "tiny_llama_f16")


@pytest.mark.gpu
def test_host_dense_model_step_gpu():
    # the whole step, eager and captured, on the dense model against its f64 logits
    _run("gpu-step", "tiny_llama_f16", data=".step")
