"""Runs the C++ mirror's unit tests (tests/cpp/test_mirror.cpp) on the GPU.

They restate the reference's Rust unit tests of the quantization module
(crates/woolly-tensor/src/quantization.rs:1293-1407) and of gguf dequantize
(crates/woolly-gguf/src/dequantize.rs:613-633) through include/woolly_hip.hpp.
"""
import subprocess
from pathlib import Path

import pytest

CPP = Path(__file__).resolve().parent / "cpp"


@pytest.mark.gpu
def test_cpp_mirror_unit_tests():
    subprocess.run(["make", "-s", "-C", str(CPP)], check=True)
    res = subprocess.run([str(CPP / "_build" / "test_mirror")], capture_output=True, text=True,
                         timeout=90)
    print(res.stdout, res.stderr)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "PASSED: 0 failed" in res.stdout
