"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer (no GPU
code is built with them): the CPU oracle with its own driver
(tests/cpp/oracle_sanitize.c), the C++ operator layer's test program in its
CPU mode, and the operator shim's reference-case harness.  Built by
tests/cpp/Makefile (`make sanitize`) with -fno-sanitize-recover=all, so any
report fails the run.  Leak checking is off: the HIP runtime the library
loads keeps allocations until exit."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
BUILD = os.path.join(HERE, "cpp", "_build")
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer",
       "-g", "-O1"]
ENV = {**os.environ, "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0",
       "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}


@pytest.fixture(scope="module")
def built():
    if shutil.which("gcc") is None or shutil.which("g++") is None:
        pytest.skip("gcc/g++ absent")
    from market_sim_amd import abi
    abi.lib()  # the product library must exist (built by build())
    subprocess.run(["make", "-s", "-C", os.path.join(HERE, "cpp"), "sanitize"], check=True,
                   timeout=600)
    return BUILD


def _run(cmd, timeout=300):
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout, env=ENV)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error" not in r.stderr, r.stderr
    return r.stdout


def test_oracle_under_asan_ubsan(built):
    out = _run([os.path.join(built, "oracle_sanitize")])
    assert " 0 failures" in out, out


def test_cpp_operator_layer_under_asan_ubsan(built):
    out = _run([os.path.join(built, "host_api_test_san"), "--cpu"])
    assert "--cpu:" in out and " 0 failures" in out, out


def test_shim_reference_cases_under_asan_ubsan(tmp_path):
    ref_include = "/root/reference/include"
    if not os.path.isdir(os.path.join(ref_include, "marketforge", "cuda")):
        pytest.skip("reference headers absent")
    if shutil.which("g++") is None:
        pytest.skip("g++ absent")
    from market_sim_amd import abi
    libdir = os.path.dirname(abi.lib()._name)
    exe = tmp_path / "shim_reference_cases_san"
    cmd = ["g++", "-std=c++20", "-Wall", "-Werror", *SAN, "-I", ref_include,
           "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "market_sim_amd", "shim", "operators_shim.cpp"),
           os.path.join(HERE, "cpp", "shim_reference_cases.cpp"),
           "-L", libdir, "-lmarketforge_hip", f"-Wl,-rpath,{libdir}", "-o", str(exe)]
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=ENV)
    if r.returncode == 77:
        pytest.skip(r.stdout.strip())
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "19 checks, 0 failures" in r.stdout, r.stdout
