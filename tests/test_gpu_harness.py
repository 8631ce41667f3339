"""The reference's example flows, run end to end through the C++ host
surface (include/miaie.hpp) by aiehlc_amd/harness/miaie_examples on the GPU.
Each subcommand computes its CPU golden the way the reference example does
and exits 0 only when the device output matches."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "aiehlc_amd", "harness", "miaie_examples")

CASES = [
    (["mm", "16", "0"], "CPU result matches"),        # aieml_mm.cc
    (["mm", "8", "0"], "CPU result matches"),         # aieoob.c
    (["perf"], "CPU result matches"),                 # aieml_perf.cc
    (["nokernelload"], "CPU result matches"),         # aie_nokernelload.cc
    (["multi_tile"], "out[0] = 26"),                  # multi_tile.cpp:150
    (["seq_full_col"], "out[0] = 23"),                # seq_full_col.cpp:163
    (["vek385"], "out[0] = 108"),                     # vek385_verification.cpp:138
    (["gemm", "4096", "4096", "4096", "10"], "CPU result matches"),
    (["gemm", "512", "384", "192", "9"], "CPU result matches"),
    (["conv"], "CPU result matches"),
    (["conv", "200", "2"], "CPU result matches"),  # also two streams, each output against the first
    (["conv", "300", "3"], "from 3 threads"),  # three streams, one issuing thread each, outputs compared
    (["mlp", "256", "4096", "11008", "4096"], "CPU result matches"),
]


def test_harness_usage_without_arguments():
    """Runs on the CPU: the binary is built and rejects a missing subcommand."""
    assert os.path.exists(EXE), "build() did not produce the harness"
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=60)
    assert r.returncode == 64 and "usage" in r.stderr


@pytest.mark.gpu
@pytest.mark.parametrize("args,needle", CASES, ids=[" ".join(c[0]) for c in CASES])
def test_harness_example(args, needle):
    print("[case] miaie_examples", *args, flush=True)
    r = subprocess.run([EXE, *args], capture_output=True, text=True, timeout=110)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, (r.returncode, r.stdout, r.stderr)
    assert needle in r.stdout
    if args[0] == "conv":
        assert "CPU result matches" in r.stdout
    if args[:4] == ["gemm", "4096", "4096", "4096"]:  # the planner, read through miaie::Context
        assert "plan: kernel 1, tile 256x256, 256 workgroups of 256 threads" in r.stdout
