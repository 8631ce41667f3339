"""The CPU test suites again, under AddressSanitizer and
UndefinedBehaviorSanitizer, in child processes:

- the oracle (oracle/liboracle_san.so, gcc) under the oracle and golden tests;
- the host code of libmiaie.so and libmiaie_xaie.so (aiehlc_amd/lib_san,
  built by aiehlc_amd/build.py with the sanitizers on the host pass only)
  under the ABI, facade and front-end tests.

Both builds stop at the first error (-fno-sanitize-recover=all), so a report
fails the child run.  Leak checking is off: the Python interpreter and the
HIP runtime keep allocations until exit by design."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
from aiehlc_amd import build as hip_build  # noqa: E402

ORACLE_SAN = os.path.join(ROOT, "oracle", "liboracle_san.so")
LIB_SAN = os.path.join(ROOT, "aiehlc_amd", "lib_san")


def _gcc_asan():
    r = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True)
    path = r.stdout.strip()
    return path if os.path.isabs(path) and os.path.exists(path) else None


def _run_under(preload, env_extra, tests):
    env = dict(os.environ, LD_PRELOAD=preload, ASAN_OPTIONS="detect_leaks=0:abort_on_error=0",
               UBSAN_OPTIONS="print_stacktrace=1", **env_extra)
    cmd = [sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider", *tests]
    r = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert r.returncode == 0, out[-4000:]
    return out


def test_oracle_under_asan_and_ubsan():
    rt = _gcc_asan()
    if rt is None or not os.path.exists(ORACLE_SAN):
        pytest.skip("gcc ASan runtime or oracle/liboracle_san.so missing")
    out = _run_under(rt, {"MIAIE_ORACLE_LIB": "liboracle_san.so"},
                     ["tests/test_oracle.py", "tests/test_golden.py"])
    assert " passed" in out


def test_library_host_code_under_asan_and_ubsan():
    rt = hip_build.asan_runtime()
    if rt is None or not os.path.exists(os.path.join(LIB_SAN, "libmiaie_xaie.so")):
        pytest.skip("clang ASan runtime or aiehlc_amd/lib_san missing")
    out = _run_under(rt, {"MIAIE_LIB_DIR": LIB_SAN},
                     ["tests/test_abi.py", "tests/test_xaie.py", "tests/test_hlc.py"])
    assert " passed" in out
