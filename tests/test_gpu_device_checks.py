"""The device-checked build (aiehlc_amd/lib_dbg/libmiaie.so, MIAIE_DEVICE_CHECKS=1):
every kernel family on valid buffers equals the oracle with no fault
reported, and accesses past a buffer's declared extent are named by
miaie_wait (MIAIE_EFAULT) and not performed.  The declared extents are
shorter than the real allocations, so nothing the kernels do reaches memory
the process does not own.

The library is loaded in a process of its own (tests/device_checks_child.py):
this process already holds the product build."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DBG = os.path.join(ROOT, "aiehlc_amd", "lib_dbg")

pytestmark = pytest.mark.gpu


@pytest.mark.skipif(not os.path.exists(os.path.join(LIB_DBG, "libmiaie.so")),
                    reason="device-checked build missing (aiehlc_amd/build.py builds it)")
def test_device_checked_build_passes_clean_runs_and_names_planted_faults():
    print("[case] device-checked build, child process", flush=True)
    env = dict(os.environ, MIAIE_LIB_DIR=LIB_DBG)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "tests", "device_checks_child.py")], env=env,
                       capture_output=True, text=True, timeout=240)
    sys.stderr.write(r.stderr[-4000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    out = json.loads(r.stdout.strip().splitlines()[-1])
    print(json.dumps(out, indent=1), flush=True)
    assert len(out["cases"]) >= 15
    kinds = " ".join(p["message"] for p in out["planted"])
    for word in ("copy", "store", "load"):
        assert word in kinds, kinds
