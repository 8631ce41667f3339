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
  it, along every branch: the state at a backward branch (the loop tail) is
  carried into the loop head.  The int8 check reads the library's own
  gemm_i8.hip, i.e. every instantiation its launchers use.  The compiler would insert these waits for its own MFMA instructions;
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

# Every pipe16 instantiation the library's launch tables name (gemm_i8.hip):
# both tile widths, both B layouts, every output form, the mixed launch and
# the MLP's cached-Y forms.
N_PIPE16 = 48
EXPECT = [
    "gemm_i8_pipe16ILi256ELi128ELi4ELb1ELi3ELb1ELb0ELb0E",   # 256x128 NT, Y_HI_RELU and C
    "gemm_i8_pipe16ILi256ELi256ELi4ELb1ELi2ELb0ELb0ELb0E",   # 256x256 NT, Y_HI
    "gemm_i8_pipe16_mixedILb1ELi3ELb0ELb0E",                 # mixed NT, Y_HI_RELU
    "gemm_i8_pipe16ILi256ELi256ELi4ELb0ELi2ELb0ELb0ELb0E",   # the benchmarked kernel
]

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
    """The device assembly of the library's own int8 GEMM translation unit."""
    if not _have_hipcc():
        pytest.skip("hipcc not available")
    out = tmp_path_factory.mktemp("asm16") / "gemm_i8.s"
    subprocess.run([HIPCC, *FLAGS, os.path.join(ROOT, "aiehlc_amd", "csrc", "gemm_i8.hip"), "-o", str(out)],
                   check=True, capture_output=True)
    return out.read_text()


def _functions(s, pattern=r"_ZN5miaie4gemm\S*pipe16\S*"):
    for m in re.finditer(r"^(%s):[^\n]*$" % pattern, s, re.M):
        name = m.group(1)
        end = s.index(".Lfunc_end", m.end())
        yield name, s[m.end():end]


def _items(body):
    """("label", name) and ("ins", text) in text order; directives dropped."""
    out = []
    for line in body.split("\n"):
        t = line.split(";")[0].strip()
        if not t:
            continue
        m = re.match(r"^([.\w$]+):$", t)
        if m:
            out.append(("label", m.group(1)))
        elif not t.startswith("."):
            out.append(("ins", t))
    return out


def test_all_kernels_compiled(asm):
    names = [n for n, _ in _functions(asm)]
    assert len(names) == N_PIPE16, names
    for key in EXPECT:
        assert any(key in n for n in names), key


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


def _step(name, t, state, mfma):
    """Advance (pending MFMA results, recent VALU writes) over instruction t,
    asserting the two hazards; returns the new state and 1 for an MFMA."""
    pending, recent = state
    op = t.split()[0]
    ops = [o.rstrip(",") for o in t.split()[1:]]
    step = int(ops[0]) + 1 if op == "s_nop" and ops else 1
    n = 0
    if op == mfma:
        n = 1
        dst, a, b, c = ops[:4]
        assert dst == c, f"{name}: MFMA not in place: {t}"
        srcs = _regs(a) | _regs(b) | _regs(c)
        for ago, regs in recent:
            assert not (regs & srcs) or ago >= OPERAND_WAIT, f"{name}: VALU result read too soon by {t}"
        pending = pending + [(_regs(dst), 0)]
    else:
        touched = set()
        for o in ops:
            touched |= _regs(o)
        for regs, w in pending:
            assert not (regs & touched), f"{name}: {t} touches MFMA result registers after {w} wait states"
    pending = [(r, w + step) for r, w in pending if w + step < RESULT_WAIT]
    recent = [(ago + step, r) for ago, r in recent if ago + step < OPERAND_WAIT]
    if op.startswith("v_") and op != mfma and ops:
        recent.append((0, _regs(ops[0])))
    return (pending, recent), n


def _is_branch(op):
    return op == "s_branch" or op.startswith("s_cbranch")


def _check_hazards(s, pattern, mfma):
    """Walk each kernel in text order; the state at a branch also flows to its
    target: a forward branch's into the label when the walk reaches it, a
    backward branch's (the loop tail's MFMAs and VALU writes) into the loop
    head, walked again from there until that state has expired."""
    checked = 0
    for name, body in _functions(s, pattern):
        items = _items(body)
        label_at = {t: i for i, (k, t) in enumerate(items) if k == "label"}
        incoming, back = {}, []
        state = ([], [])
        for i, (kind, t) in enumerate(items):
            if kind == "label":
                for p, r in incoming.pop(t, []):
                    state = (state[0] + p, state[1] + r)
                continue
            state, n = _step(name, t, state, mfma)
            checked += n
            op = t.split()[0]
            if _is_branch(op):
                j = label_at.get(t.split()[1])
                if j is not None and j > i:
                    incoming.setdefault(items[j][1], []).append(state)
                elif j is not None:
                    back.append((j, state))
                if op == "s_branch":
                    state = ([], [])  # nothing falls through
        for j, st in back:
            for kind, t in items[j + 1:]:
                if not (st[0] or st[1]):
                    break
                if kind == "ins":
                    st, _ = _step(name, t, st, mfma)
                    if _is_branch(t.split()[0]):
                        break
    return checked


def test_no_scratch(asm):
    _check_no_scratch(asm, "pipe16")


def test_mfma_in_place_and_hazard_free(asm):
    assert _check_hazards(asm, r"_ZN5miaie4gemm\S*pipe16\S*", MFMA) > 1000


def test_bf16_no_scratch(asm_bf16):
    _check_no_scratch(asm_bf16, "gemm_bf16_pair16")


def test_bf16_mfma_in_place_and_hazard_free(asm_bf16):
    assert _check_hazards(asm_bf16, r"\S*gemm_bf16_pair16\S*", MFMA_BF16) > 500


def _synthetic(loop_tail):
    return ("f:\n.LBB0_1:\n\tv_mfma_i32_16x16x64_i8 a[0:3], v[0:3], v[4:7], a[0:3]\n"
            + "".join(f"\ts_nop 7\n" for _ in range(3)) + loop_tail + "\ts_cbranch_scc1 .LBB0_1\n\ts_endpgm\n.Lfunc_end0:\n")


def test_hazard_check_follows_the_loop_back_edge():
    # a VALU write of an MFMA operand at the loop bottom, read by the MFMA at
    # the loop top one instruction later: only the back edge shows it
    with pytest.raises(AssertionError, match="VALU result read too soon"):
        _check_hazards(_synthetic("\tv_mov_b32 v1, 0\n"), "f", MFMA)
    # an MFMA at the loop bottom whose result the loop top's VALU reads
    bad = ("f:\n.LBB0_1:\n\tv_accvgpr_read_b32 v9, a1\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n"
           "\tv_mfma_i32_16x16x64_i8 a[0:3], v[0:3], v[4:7], a[0:3]\n\ts_cbranch_scc1 .LBB0_1\n\ts_endpgm\n.Lfunc_end0:\n")
    with pytest.raises(AssertionError, match="touches MFMA result registers"):
        _check_hazards(bad, "f", MFMA)
    # the same with the wait states in between passes
    assert _check_hazards(_synthetic("\tv_mov_b32 v1, 0\n\ts_nop 3\n"), "f", MFMA) == 1
