"""The aiehlc source front end retargeted to gfx950 (aiehlc_amd/hlc.py).

CPU: the rewrite does what aiehlc.cc:469-607 does to a host source:
kernel definitions cut out (wherever they sit, whatever their bodies hold),
`__kernel__` names given a template, XAie_LoadElfMem pointed at the
kernel, windows placed by the reference compiler's rule.  Keywords inside
comments and strings are left alone, and a kernel with no gfx950
counterpart is an error.  GPU: the two sample programs in the dialect
(aiehlc_amd/harness/hlc/), rewritten and compiled by build(), run and
check their results."""
import os
import subprocess
import tempfile

import pytest

from aiehlc_amd import hlc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HARNESS = os.path.join(ROOT, "aiehlc_amd", "harness")

SRC = r'''#include "xaiengine.h"
#include "xil_printf.h"
// __global__ void not_a_kernel(int* a, int* b) { }
const char* s = "__kernel__ void nor_this(int x) {}";
__global__ void mm(input_window_int32 * win __attribute__((annotate("mem_address:0x1000"), annotate("size_hint:512"))),
        output_window_int32 *out __attribute__((annotate("mem_address:0x6000"), annotate("size_hint:512")))) {
#define INNER 16
  if (1) { { aie::vector<int32_t, INNER> v = window_readincr_v<INNER>(win); } }
  const char* brace = "}";  /* } */
}
__kernel__ void perf(input_window_int32 * win, output_window_int32 * out)
{
  uint32_t x = '}';
}
__global__ void k1(int *in, int *out);
int main() {
  XAie_LoadElfMem(dev, XAie_TileLoc(4,4), (unsigned char *)mm);
  XAie_LoadElfMem(dev,
                  XAie_TileLoc(1, 3), (unsigned char *) k1);
  perf<1,1,4,4,256,16,64>(phy, phy_out);
}
'''


def test_finds_definitions_outside_comments_and_strings():
    ks = hlc.find_kernels(SRC)
    assert [(k.keyword, k.name) for k in ks] == [("__global__", "mm"), ("__kernel__", "perf"), ("__global__", "k1")]
    mm = ks[0]
    assert [p.name for p in mm.params] == ["win", "out"]
    assert [(p.mem_address, p.size_hint) for p in mm.params] == [(0x1000, 512), (0x6000, 512)]
    assert SRC[mm.start:mm.end].rstrip().endswith("}") and "brace" in SRC[mm.start:mm.end]
    assert SRC[ks[2].start:ks[2].end].endswith(";")  # a declaration


def test_rewrite_output():
    out, ks, warnings = hlc.rewrite(SRC, filename="prog.cc")
    body = out.split('#line 1 "prog.cc"\n', 1)[1]
    # definitions are gone, line count kept
    assert "window_readincr_v" not in body and "uint32_t x" not in body
    assert body.count("\n") == SRC.count("\n")
    # keywords in comments and strings untouched
    assert "// __global__ void not_a_kernel" in body and '"__kernel__ void nor_this(int x) {}"' in body
    # aie-rt header swapped, BSP header reported
    assert '#include "miaie_xaie.h"' in body and "xaiengine.h" not in body
    assert any("xil_printf.h" in w for w in warnings)
    # LoadElfMem points at the descriptors (the reference rewrites it to _binary_kernel_<k>_start)
    assert "XAie_LoadElfMem(dev, XAie_TileLoc(4,4), (const unsigned char *)&miaie_xaie_mm)" in body
    assert "(const unsigned char *)&miaie_xaie_k1)" in body
    # the __kernel__ template forwards to the gfx950 launch
    head = out.split("#line 1")[0]
    assert "inline void perf(Args&&... args)" in head
    assert "miaie_hlc::launch<miaie_hlc::Kernel::perf_u8, Col, Row, colstart, rowstart, M, N, K>" in head
    assert "perf<1,1,4,4,256,16,64>(phy, phy_out);" in body
    assert [k.target for k in ks] == ["miaie_xaie_mm", "perf_u8", "miaie_xaie_k1"]


def test_window_placement_rule():
    # AieFrontEnd.cc:297-394: ping at the annotation or after the previous
    # pong; each buffer 4 * size_hint words (size_hint 512 by default)
    P = hlc.Param
    assert hlc.window_layout([P("", "int *", "a"), P("", "int *", "b")]) == [0x1000, 0x5000]
    assert hlc.window_layout([P("", "w", "a", 0x1000, 512), P("", "w", "b", 0x6000, 512)]) == [0x1000, 0x6000]
    assert hlc.window_layout([P("", "w", "a", 0, 256), P("", "w", "b"), P("", "w", "c", 0x20000)]) == \
        [0x1000, 0x3000, 0x20000]


def test_unknown_kernels_are_errors_and_map_overrides():
    src = "__global__ void saxpy(float* x, float* y) { }\n"
    with pytest.raises(hlc.HlcError, match="no gfx950 counterpart.*saxpy"):
        hlc.rewrite(src)
    out, ks, _ = hlc.rewrite(src, {"saxpy": "k1"})
    assert ks[0].target == "miaie_xaie_k1"
    with pytest.raises(hlc.HlcError, match="unknown __global__ target"):
        hlc.rewrite(src, {"saxpy": "nope"})
    with pytest.raises(hlc.HlcError, match="not a __global__ kernel"):
        hlc.rewrite("__global__ void k1(int* a, int* b) {}\nint f(){ XAie_LoadElfMem(d, l, (unsigned char*)k9); }\n")
    # the vek385 kernel: `mm` on uint64_t pointers is the 3x3 replicated kernel
    _, ks, _ = hlc.rewrite("__global__ void mm(uint64_t *in, uint64_t *out) { while(true) {} }\n")
    assert ks[0].target == "miaie_xaie_mm3_u64"


def test_command_line_and_compile(tmp_path):
    """The CLI writes the host file and kernel list; g++ compiles the output
    against the headers (syntax only: no device is needed)."""
    src = tmp_path / "prog.cc"
    src.write_text('#include "xaiengine.h"\n#include "miaie.hpp"\n'
                   '__kernel__ void gemm_i8(const int8_t* A, const int8_t* B, int8_t* Y, int s) { aie::stuff(); }\n'
                   '__global__ void k2(int* in, int* out) { *out = *in + 10; }\n'
                   'int main() { XAie_DevInst d = {}; XAie_LoadElfMem(&d, XAie_TileLoc(1, 4), (unsigned char*)k2);\n'
                   '  gemm_i8<1, 1, 0, 0, 256, 256, 64>((const int8_t*)0, (const int8_t*)0, (int8_t*)0, 10); }\n')
    out, kl = tmp_path / "host.cc", tmp_path / "kernel_list"
    r = subprocess.run(["python", "-m", "aiehlc_amd.hlc", str(src), "-o", str(out), "--kernel-list", str(kl)],
                       cwd=ROOT, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert kl.read_text() == "gemm_i8 __kernel__ gemm_i8 0x1000 0x5000 0x9000 0xd000\nk2 __global__ miaie_xaie_k2 0x1000 0x5000\n"
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-I", os.path.join(ROOT, "include"),
                        str(out)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    bad = tmp_path / "bad.cc"
    bad.write_text("__kernel__ void conv(int* a) {}\n")
    r = subprocess.run(["python", "-m", "aiehlc_amd.hlc", str(bad), "-o", str(tmp_path / "o.cc")], cwd=ROOT,
                       capture_output=True, text=True)
    assert r.returncode == 1 and "no gfx950 counterpart" in r.stderr


def test_samples_are_built():
    for name in ("hlc_elf_flow", "hlc_kernel_flow"):
        assert os.path.exists(os.path.join(HARNESS, name)), f"build() did not produce {name}"


@pytest.mark.gpu
@pytest.mark.parametrize("name,needles", [
    ("hlc_elf_flow", ["mm: C[0][0] = 31960, C[15][15] = 1994200, 0 mismatches", "chain: out[0] = 26, 0 mismatches",
                      "elf_flow: all results match"]),
    ("hlc_kernel_flow", ["perf: out = {3145728, 4567, 811597824, 3, 2}, 0 mismatches",
                         "gemm_i8: 256 x 256 x 512, 0 mismatches", "kernel_flow: all results match"]),
])
def test_rewritten_programs_run(name, needles):
    print(f"[case] {name}", flush=True)
    r = subprocess.run([os.path.join(HARNESS, name)], capture_output=True, text=True, timeout=110)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, (r.stdout, r.stderr)
    for n in needles:
        assert n in r.stdout, n
