"""The 16x16 GEMM kernels issue their MFMAs through inline assembly (int8:
aiehlc_amd/csrc/gemm_i8_kernels.hpp, mfma16; bf16: aiehlc_amd/csrc/
gemm_bf16.hip, mfma16_bf16), which the compiler's hazard recognizer does not
see.  These checks compile the kernels for gfx950 and read the generated
assembly (of this build, CPU only):

- no scratch memory (a spill would put the accumulators' neighbours through
  memory, and VGPR pressure is what makes the compiler move accumulators);
- every asm MFMA updates its accumulator in place;
- no non-MFMA instruction touches an MFMA's accumulator registers before the
  worst-case MFMA result latency (18 wait states) has passed, and no VALU
  instruction writes an MFMA's operand registers within 3 wait states before
  it.  The compiler would insert these waits for its own MFMA instructions;
  for the inline ones the kernel relies on the order it writes (in-place
  accumulation, operands straight from LDS reads, the drain before the
  epilogue).
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

KERNELS = [
    "gemm_i8_pipe16<256, 256, 4, false, Y_HI, false>",
    "gemm_i8_pipe16<256, 128, 4, false, Y_HI, false>",
    "gemm_i8_pipe16<256, 256, 4, false, Y_NONE, true>",
    "gemm_i8_pipe16<256, 256, 4, true, Y_MED3, true>",
    "gemm_i8_pipe16<256, 256, 4, false, Y_HI_RELU, false, false, true>",
]
MIXED = ["gemm_i8_pipe16_mixed<false, Y_HI_RELU, false>", "gemm_i8_pipe16_mixed<false, Y_MED3, false, true>"]

SRC = """
#include "gemm_i8_kernels.hpp"
namespace miaie { namespace gemm {
%s
}}
"""
ARGS = ("const int8_t*, const int8_t*, int8_t*, int32_t*, int, int, int, int, int, int, int, int, int")

MFMA = "v_mfma_i32_16x16x64_i8"
MFMA_BF16 = "v_mfma_f32_16x16x32_bf16"
RESULT_WAIT = 18  # XDL result -> VALU access, worst case over pass counts
OPERAND_WAIT = 3  # VALU write -> MFMA source read


def _regs(tok):
    m = re.match(r"([va])\[(\d+):(\d+)\]", tok)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", tok)
    if m:
        return {(m.group(1), int(m.group(2)))}
    return set()


FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
         "-mllvm", "-amdgpu-kernarg-preload-count=16", "--cuda-device-only", "-S",
         f"-I{os.path.join(ROOT, 'aiehlc_amd', 'csrc')}", f"-I{os.path.join(ROOT, 'include')}"]


def _have_hipcc():
    return shutil.which(HIPCC) or os.path.exists(HIPCC)


@pytest.fixture(scope="module")
def asm_bf16(tmp_path_factory):
    if not _have_hipcc():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm16bf") / "bf16.s"
    subprocess.run([HIPCC, *FLAGS, os.path.join(ROOT, "aiehlc_amd", "csrc", "gemm_bf16.hip"), "-o", str(out)],
                   check=True, capture_output=True)
    return out.read_text()


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not _have_hipcc():
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("asm16")
    inst = [f"template __global__ void {k}({ARGS}, unsigned long long*);" for k in KERNELS]
    inst += [f"template __global__ void {k}({ARGS}, int);" for k in MIXED]
    src = d / "k.hip"
    src.write_text(SRC % "\n".join(inst))
    out = d / "k.s"
    subprocess.run([HIPCC, *FLAGS, str(src), "-o", str(out)], check=True, capture_output=True)
    return out.read_text()


def _functions(s, pattern=r"_ZN5miaie4gemm\S*pipe16\S*"):
    for m in re.finditer(r"^(%s):[^\n]*$" % pattern, s, re.M):
        name = m.group(1)
        end = s.index(".Lfunc_end", m.end())
        yield name, s[m.end():end]


def _instructions(body):
    out = []
    for line in body.split("\n"):
        t = line.strip()
        if not t or t.startswith((";", ".")) or t.endswith(":"):
            continue
        out.append(t.split(";")[0].strip())
    return out


def test_all_kernels_compiled(asm):
    names = [n for n, _ in _functions(asm)]
    assert len(names) == len(KERNELS) + len(MIXED), names


def _check_no_scratch(s, key):
    meta = s[s.index("amdhsa.kernels:"):]
    seen = 0
    for blk in meta.split("\n  - ")[1:]:
        m = re.search(r"\.name:\s+(\S+)", blk)
        if not m or key not in m.group(1):
            continue
        seen += 1
        priv = int(re.search(r"\.private_segment_fixed_size:\s+(\d+)", blk).group(1))
        spill = int(re.search(r"\.vgpr_spill_count:\s+(\d+)", blk).group(1))
        assert priv == 0 and spill == 0, (m.group(1), priv, spill)
    assert seen


def _check_hazards(s, pattern, mfma):
    checked = 0
    for name, body in _functions(s, pattern):
        ins = _instructions(body)
        pending = []  # AGPRs written by an MFMA still inside the result latency
        waits = []    # wait states elapsed since each pending MFMA
        recent_valu = []  # (wait states ago, registers written) for the last few VALU ops
        for t in ins:
            op = t.split()[0]
            ops = [o.rstrip(",") for o in t.split()[1:]]
            step = int(ops[0]) + 1 if op == "s_nop" and ops else 1
            if op == mfma:
                checked += 1
                dst, a, b, c = ops[:4]
                assert dst == c, f"{name}: MFMA not in place: {t}"
                srcs = _regs(a) | _regs(b)
                for ago, regs in recent_valu:
                    assert not (regs & (srcs | _regs(c))) or ago >= OPERAND_WAIT, f"{name}: VALU result read too soon by {t}"
                pending.append(_regs(dst))
                waits.append(0)
            else:
                touched = set()
                for o in ops:
                    touched |= _regs(o)
                for regs, w in zip(pending, waits):
                    assert not (regs & touched), f"{name}: {t} touches MFMA result registers after {w} wait states"
            waits = [w + step for w in waits]
            keep = [i for i, w in enumerate(waits) if w < RESULT_WAIT]
            pending = [pending[i] for i in keep]
            waits = [waits[i] for i in keep]
            recent_valu = [(ago + step, r) for ago, r in recent_valu if ago + step < OPERAND_WAIT]
            if op.startswith("v_") and op != mfma and ops:
                recent_valu.append((0, _regs(ops[0])))
    return checked


def test_no_scratch(asm):
    _check_no_scratch(asm, "pipe16")


def test_mfma_in_place_and_hazard_free(asm):
    assert _check_hazards(asm, r"_ZN5miaie4gemm\S*pipe16\S*", MFMA) > 1000


def test_bf16_no_scratch(asm_bf16):
    _check_no_scratch(asm_bf16, "gemm_bf16_pair16")


def test_bf16_mfma_in_place_and_hazard_free(asm_bf16):
    assert _check_hazards(asm_bf16, r"\S*gemm_bf16_pair16\S*", MFMA_BF16) > 500
