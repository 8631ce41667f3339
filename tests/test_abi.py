"""CPU checks of the C-ABI boundary: the gfx950 library loads on a host
without a GPU and exports exactly the entry points include/miaie.h declares.
No compute entry point is called here."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

import aiehlc_amd as mi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _exported(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_header_declares_the_boundary():
    names = mi.header_functions()
    assert len(names) == len(set(names))
    for must in ("miaie_init", "miaie_finish", "miaie_alloc", "miaie_copy_h2d", "miaie_copy_d2h", "miaie_wait",
                 "miaie_mm_window_i32", "miaie_gemm_i8_i32", "miaie_gemm_i8_rq", "miaie_gemm_bf16_f32",
                 "miaie_conv2d_i8_nhwc", "miaie_mlp_i8"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = mi.load_library()
    declared = set(mi.header_functions())
    for name in declared:
        assert hasattr(lib, name), name
    exported = {s for s in _exported(mi.LIB_PATH) if s.startswith("miaie_")}
    # hidden visibility: nothing beyond the header leaks out of the library
    assert exported == declared, (exported ^ declared)
    # the Python binding table covers the whole header
    assert set(mi._SIGS) == declared


def test_version_and_init_error_without_gpu():
    lib = mi.load_library()
    assert mi.version().startswith("miaie")
    h = ctypes.c_void_p()
    rc = lib.miaie_init(ctypes.byref(h), 0)
    if rc != mi.MIAIE_OK:  # no device here: a clean error, never a crash
        assert rc in (mi.MIAIE_EHIP, mi.MIAIE_EINVAL, mi.MIAIE_EUNSUPPORTED)
        assert lib.miaie_last_error_string(None)
        assert h.value is None
    else:
        assert lib.miaie_finish(h) == mi.MIAIE_OK


def test_null_context_is_rejected():
    lib = mi.load_library()
    assert lib.miaie_wait(None, 0) == mi.MIAIE_EINVAL
    assert lib.miaie_gemm_i8_rq(None, None, None, None, 1, 1, 1, 10, 0, None, 0) == mi.MIAIE_EINVAL
    assert b"NULL" in lib.miaie_last_error_string(None)
    assert lib.miaie_finish(None) == mi.MIAIE_OK


def test_status_codes_match_header():
    text = open(mi.HEADER_PATH).read()
    for name in ("MIAIE_OK", "MIAIE_EINVAL", "MIAIE_EHIP", "MIAIE_ETIMEDOUT", "MIAIE_ENOMEM", "MIAIE_EUNSUPPORTED",
                 "MIAIE_EFAULT"):
        m = re.search(rf"#define {name} \(?(-?\d+)\)?", text)
        assert m and int(m.group(1)) == getattr(mi, name), name
    # the conv planner's kernel ids, as the Python binding names them
    for name, label in (("MIAIE_CONV_ROWS", "rows"), ("MIAIE_CONV_IGEMM", "igemm"), ("MIAIE_CONV_DIRECT", "direct"),
                        ("MIAIE_CONV_TAPS", "taps"), ("MIAIE_CONV_ROWS_DEEP", "rows_deep")):
        m = re.search(rf"#define {name} (\d+)", text)
        assert m and mi.CONV_KERNELS[int(m.group(1))] == label, name


def test_conv_planner_keeps_32_bit_offsets_in_range():
    """The row-block conv kernel indexes X, Y and W with 32-bit offsets; shapes
    whose weights (Cout * R*S*Cin bytes) reach 2^31 must go to a kernel that
    indexes in 64 bits.  Host-only: the planner needs no device."""
    assert mi.plan_conv2d_i8(8, 56, 56, 64, 64) == "rows"            # config 4
    assert mi.plan_conv2d_i8(1, 1, 1, 128, 64) == "rows"
    big = (1 << 31) // (9 * 128)                                      # 1864135 channels
    cout = big - big % 64                                             # multiple of 64 below the bound
    assert cout * 9 * 128 < 1 << 31
    assert mi.plan_conv2d_i8(1, 1, 1, 128, cout) == "rows"
    cout2 = cout + 64                                                 # weights reach 2^31 bytes
    assert cout2 * 9 * 128 >= 1 << 31
    assert mi.plan_conv2d_i8(1, 1, 1, 128, cout2) == "igemm"
    assert mi.plan_conv2d_i8(1, 1, 1, 128, cout2 + 32) == "direct"   # not a multiple of 64
    # X and Y offsets: a batch whose activations reach 2^31 bytes
    n_big = (1 << 31) // (56 * 56 * 64) + 1
    assert mi.plan_conv2d_i8(n_big, 56, 56, 64, 64) == "igemm"
    assert mi.plan_conv2d_i8(2, 56, 56, 64, 64, stride=2) == "igemm"
    assert mi.plan_conv2d_i8(1, 5, 5, 4, 8) == "direct"
    # deep 3x3 stride-1 layers: the chunked row-block kernel or the taps
    # kernel, whichever the launch-time estimate favours; strided ones: taps
    assert mi.plan_conv2d_i8(8, 14, 14, 256, 256) == "rows_deep"
    assert mi.plan_conv2d_i8(8, 56, 56, 256, 256) == "rows_deep"
    assert mi.plan_conv2d_i8(8, 28, 28, 512, 512) == "rows_deep"
    assert mi.plan_conv2d_i8(8, 56, 56, 192, 96) == "rows_deep"          # Cin not a multiple of 128
    assert mi.plan_conv2d_i8(8, 7, 7, 512, 512) == "taps"                # 56 tiles split 4 ways
    assert mi.plan_conv2d_i8(32, 28, 28, 512, 512) == "rows_deep"        # 32-column blocks
    assert mi.plan_conv2d_i8(32, 28, 28, 512, 512, 1, 1, 1, 0) == "taps"  # 1x1: not the row-block kernel
    assert mi.plan_conv2d_i8(1, 3, 3, 4032, 64) == "rows_deep"
    assert mi.plan_conv2d_i8(1, 3, 3, 4160, 64) == "igemm"               # above the 4096 bound, not a multiple of 128
    assert mi.plan_conv2d_i8(8, 56, 56, 256, 256, 5, 5, 1, 2) == "taps"  # not 3x3
    assert mi.plan_conv2d_i8(8, 112, 112, 128, 128) == "rows"              # rows wider than 64: column blocks
    assert mi.plan_conv2d_i8(8, 28, 28, 128, 128) == "rows"                # one round of row blocks
    assert mi.plan_conv2d_i8(32, 28, 28, 128, 128) == "rows_deep"          # narrow, several rounds: 32-column blocks
    assert mi.plan_conv2d_i8(8, 112, 112, 128, 128, stride=2) == "taps"     # stride 2: not the row-block kernel
    n_deep = (1 << 31) // (14 * 14 * 256) + 1                             # X reaches 2^31 bytes
    assert mi.plan_conv2d_i8(n_deep, 14, 14, 256, 256) == "igemm"
    big_deep = (1 << 31) // (9 * 256)                                     # weights reach 2^31 bytes
    assert mi.plan_conv2d_i8(1, 1, 1, 256, big_deep + 64 - big_deep % 64) == "igemm"
    with pytest.raises(mi.MiaieError):
        mi.plan_conv2d_i8(1, 2, 2, 4, 4, 5, 5, 1, 0)                  # filter larger than the input


def test_device_checked_build_exports_the_same_boundary():
    """aiehlc_amd/lib_dbg/libmiaie.so (device-side bounds checks) exports
    exactly the header's entry points and says it checks; the product build
    says it does not.  The debug build is loaded in a process of its own."""
    dbg = os.path.join(ROOT, "aiehlc_amd", "lib_dbg", "libmiaie.so")
    if not os.path.exists(dbg):
        pytest.skip("device-checked build missing")
    exported = {s for s in _exported(dbg) if s.startswith("miaie_")}
    assert exported == set(mi.header_functions()), exported ^ set(mi.header_functions())
    assert mi.load_library().miaie_debug_device_checks() == 0
    code = f"import ctypes; print(ctypes.CDLL({dbg!r}).miaie_debug_device_checks())"
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, check=True).stdout
    assert out.strip() == "1"
