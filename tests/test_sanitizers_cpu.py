"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer, no GPU.

Two builds, both of host code only (gcc / g++, no .hip file):
  * tests/host/test_host_san: the C++ host interface (mc_candle.cpp) and the
    safetensors checkpoint reader / writer (checkpoint.cpp, which parses
    untrusted files) compiled in from source, run over its --cpu cases: the
    validation and message cases, the checkpoint round trips, the malformed
    headers and the mutated-file sweep (every truncation of a valid header,
    byte substitutions at every header position, bad length prefixes);
  * oracle/liboracle_san.so: the CPU oracle, loaded into a Python process
    (libasan preloaded) in place of liboracle.so, running the oracle tests:
    the reference's known answers, the golden fixtures, finite differences.
Any sanitizer report fails the run (leaks included for the host program;
the Python interpreter's own allocations are not leak-checked).
"""
import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def _asan_runtime():
    p = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True)
    path = p.stdout.strip()
    if p.returncode != 0 or not os.path.isabs(path) or not os.path.exists(path):
        pytest.skip("gcc's libasan is not available")
    return path


def _make(target, directory):
    subprocess.run(["make", "-s", "-C", directory, target], check=True, timeout=600)


def test_host_interface_under_asan_ubsan():
    _asan_runtime()
    _make("test_host_san", os.path.join(HERE, "host"))
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    p = subprocess.run([os.path.join(HERE, "host", "test_host_san"), "--cpu"], capture_output=True, text=True,
                       timeout=300, env=env)
    out = p.stdout + p.stderr
    assert p.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert "checkpoint_mutated_files" in out and " 0 failed" in out, out[-4000:]


def test_oracle_under_asan_ubsan():
    asan = _asan_runtime()
    _make("liboracle_san.so", os.path.join(ROOT, "oracle"))
    san_lib = os.path.join(ROOT, "oracle", "liboracle_san.so")
    env = dict(os.environ, MC_ORACLE_LIB=san_lib, LD_PRELOAD=asan, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1", PYTHONPATH=ROOT)
    # the sanitizer build is the one that gets loaded
    probe = subprocess.run([sys.executable, "-c",
                            "import oracle; oracle.lib(); print(open('/proc/self/maps').read().count('liboracle_san.so') > 0)"],
                           capture_output=True, text=True, timeout=300, env=env, cwd=ROOT)
    assert probe.returncode == 0 and probe.stdout.strip() == "True", probe.stdout + probe.stderr
    tests = [os.path.join(HERE, f) for f in ("test_oracle.py", "test_oracle_rowops.py", "test_oracle_adamw.py",
                                             "test_oracle_attention.py")]
    p = subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider", *tests], capture_output=True,
                       text=True, timeout=900, env=env, cwd=ROOT)
    out = p.stdout + p.stderr
    assert p.returncode == 0, out[-4000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
