"""The reference's own example host programs through the front end and the
aie-rt facade, on the CPU.

Each example (read from the reference tree at test time; nothing of it is
kept in this repository) is rewritten by aiehlc_amd/hlc.py, then compiled
with g++ against include/miaie_xaie.h (which the rewrite puts in place of
aie-rt's xaiengine.h) and the reference's own BSP headers
(thirdparty/arch/psv_cortexa72_0/bsp/include).  The object must compile, every
XAie_* symbol it references must be exported by libmiaie_xaie.so, and the
only other symbols it needs beyond the C/C++ runtime are the three BSP
services a host program replaces (cache disables and the timer).  The kernel
list must place each kernel's windows where the reference's compiler does
(AieFrontEnd.cc:297-394) and where the example's own moves expect them.

Skipped when the reference tree is absent (it is not on the GPU boxes)."""
import os
import subprocess

import pytest

from aiehlc_amd import hlc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
BSP = os.path.join(REF, "thirdparty", "arch", "psv_cortexa72_0", "bsp", "include")
XAIE_LIB = os.path.join(ROOT, "aiehlc_amd", "lib", "libmiaie_xaie.so")

pytestmark = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "example")),
                                reason="reference tree absent")

# example -> {kernel name: (keyword, gfx950 target, ping addresses of its windows)}
EXAMPLES = {
    # __global__ mm with annotated windows in 0x1000 / out 0x6000 (aieml_mm.cc:41-42)
    "example/matrixmultiply/aieml_mm.cc": {"mm": ("__global__", "miaie_xaie_mm", [0x1000, 0x6000])},
    # __global__ perf, unannotated windows placed by the default rule (aieml_perf.cc:61)
    "example/perf/aieml_perf.cc": {"perf": ("__global__", "miaie_xaie_perf", [0x1000, 0x6000])},
    # __kernel__ perf, launched as perf<1,1,4,4,256,16,64>(phy, phy_out) (aie_nokernelload.cc:130)
    "example/nokernelload/aie_nokernelload.cc": {"perf": ("__kernel__", "perf_u8", [0x1000, 0x6000])},
    # k1 -> k2 (multi_tile.cpp:39-47), windows at the default placement 0x1000 / 0x5000
    "example/multi/multi_tile.cpp": {"k1": ("__global__", "miaie_xaie_k1", [0x1000, 0x5000]),
                                     "k2": ("__global__", "miaie_xaie_k2", [0x1000, 0x5000])},
    "example/multi/seq_full_col.cpp": {"k1": ("__global__", "miaie_xaie_k1", [0x1000, 0x5000]),
                                       "k2": ("__global__", "miaie_xaie_k2", [0x1000, 0x5000])},
}

# BSP services a host program supplies (Xil_*CacheDisable: nothing to do on a
# coherent host; XTime_GetTime: a host clock)
BSP_SERVICES = {"Xil_DCacheDisable", "Xil_ICacheDisable", "XTime_GetTime"}
RUNTIME_PREFIXES = ("_Z", "__cxa", "__gxx", "_Unwind", "__stack_chk", "__dso_handle", "_GLOBAL_OFFSET_TABLE_")
LIBC = {"printf", "puts", "fflush", "stdout", "strlen", "putchar", "memcpy", "memset", "abort", "exit"}


def _undefined(obj):
    out = subprocess.run(["nm", "-u", obj], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def _exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if len(line.split()) == 3}


@pytest.mark.parametrize("rel", sorted(EXAMPLES))
def test_reference_example_rewrites_compiles_and_resolves(tmp_path, rel):
    path = os.path.join(REF, rel)
    src = open(path).read()
    host, kernels, warnings = hlc.rewrite(src, filename=path)
    # the kernels and where their windows go
    got = {k.name: (k.keyword, k.target, list(k.ping)) for k in kernels}
    assert got == EXAMPLES[rel], got
    # BSP includes are reported, not silently dropped
    assert any("BSP header" in w for w in warnings)
    assert '#include "miaie_xaie.h"' in host and '"xaiengine.h"' not in host
    # compiles against the facade header and the reference's own BSP headers
    cc = tmp_path / (os.path.basename(rel) + ".host.cc")
    cc.write_text(host)
    obj = tmp_path / "host.o"
    r = subprocess.run(["g++", "-std=c++17", "-c", "-w", "-I", os.path.join(ROOT, "include"), "-I", BSP, str(cc),
                        "-o", str(obj)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    # every aie-rt call (and kernel descriptor) resolves to the facade;
    # nothing else is missing
    undef = _undefined(str(obj))
    xaie = {s for s in undef if s.startswith(("XAie_", "miaie_"))}
    assert xaie, "the example makes aie-rt calls"
    missing = xaie - _exported(XAIE_LIB)
    assert not missing, sorted(missing)
    rest = {s for s in undef - xaie if not s.startswith(RUNTIME_PREFIXES) and s not in LIBC}
    assert rest <= BSP_SERVICES, sorted(rest - BSP_SERVICES)
