"""The C++ operator layer (include/marketforge_gpu.hpp) through its own test
program, tests/cpp/host_api_test.cpp (built by __graft_entry__.build() or,
on the CPU, on demand)."""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
BIN = os.path.join(HERE, "cpp", "_build", "host_api_test")


def _build() -> None:
    import oracle
    oracle.lib()  # builds oracle/liboracle.so when absent
    from market_sim_amd import abi
    abi.lib()     # the product library must exist (built by build())
    subprocess.run(["make", "-s", "-C", os.path.join(HERE, "cpp")], check=True)


def _run(mode: str, timeout: int):
    r = subprocess.run([BIN, mode], capture_output=True, text=True, timeout=timeout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert " 0 failures" in r.stdout, r.stdout
    return r.stdout


def test_cpp_layer_types_and_validation():
    _build()
    out = _run("--cpu", 60)
    assert "--cpu:" in out


@pytest.mark.gpu
def test_cpp_layer_reference_cases_and_decode_tail(hip):
    if not os.path.exists(BIN):
        pytest.fail("tests/cpp/_build/host_api_test is not built: run __graft_entry__.build()")
    out = _run("--gpu", 120)
    assert "decode tail (mul-add chain)" in out
