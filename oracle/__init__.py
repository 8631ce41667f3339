"""CPU oracle for the miaie GEMM/conv path — TEST INFRASTRUCTURE ONLY.

ctypes bindings over oracle/liboracle.so (built from oracle/miaie_oracle.c by
oracle/build.py).  Only tests/, __graft_entry__.smoke() and the cpu_baseline
leg of bench.py may import this package, and only as the checker or as the
timed CPU baseline; the product path (aiehlc_amd) never touches it.

Each wrapper names the C function it calls; the C file cites the reference
file:line each one restates.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIBS: dict[str, C.CDLL] = {}

_p = C.c_void_p
_i = C.c_int
_sz = C.c_size_t
_u64 = C.c_uint64


def _lib(name: str | None = None) -> C.CDLL:
    # MIAIE_ORACLE_LIB selects another build of the same source (the
    # sanitized liboracle_san.so)
    name = name or os.environ.get("MIAIE_ORACLE_LIB") or "liboracle.so"
    if name in _LIBS:
        return _LIBS[name]
    path = os.path.join(_HERE, name)
    if not os.path.exists(path):
        from . import build as _build

        _build.build()
    lib = C.CDLL(path)
    sigs = {
        "oracle_tensor_seed": (_u64, [_u64]),
        "oracle_sm64_at": (_u64, [_u64, _u64]),
        "oracle_fill_i8": (None, [_p, _sz, _u64]),
        "oracle_fill_shift": (None, [_p, _sz, _u64]),
        "oracle_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "oracle_bf16_to_f32": (C.c_float, [C.c_uint16]),
        "oracle_fill_bf16_normal": (None, [_p, _sz, _u64, C.c_double]),
        "oracle_mm_window_i32": (None, [_p, _p, _i]),
        "oracle_count_mismatch_i32": (_i, [_p, _p, _sz]),
        "oracle_gemm_i8_nt_rows": (None, [_p, _p, _p] + [_i] * 9),
        "oracle_transpose_i8": (None, [_p, _p, _i, _i, _i]),
        "oracle_gemm_i8_nn_rows": (_i, [_p, _p, _p] + [_i] * 9),
        "oracle_requant": (C.c_int8, [C.c_int32, _i, _i]),
        "oracle_requant_buf": (None, [_p, _p, _sz, _i, _i]),
        "oracle_gemm_i8_rq_rows": (_i, [_p, _p, _p, _p] + [_i] * 9),
        "oracle_gemm_bf16_rows": (None, [_p, _p, _p] + [_i] * 6),
        "oracle_gemm_bf16_f64_rows": (None, [_p, _p, _p] + [_i] * 6),
        "oracle_conv2d_nhwc_i8": (None, [_p, _p, _p, _p, _p] + [_i] * 11),
        "oracle_mlp_i8_rows": (_i, [_p, _p, _p, _p, _p] + [_i] * 9),
        "oracle_dot_u8_probe": (None, [_p, _p]),
        "oracle_mm_square_u64": (None, [_p, _p, _i, _u64]),
        "oracle_chain_add": (None, [_p, _p, _i, _p, _i]),
        "oracle_num_threads": (_i, []),
    }
    for fn, (res, args) in sigs.items():
        f = getattr(lib, fn)
        f.restype = res
        f.argtypes = args
    _LIBS[name] = lib
    return lib


def _ptr(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def default_threads() -> int:
    return int(os.environ.get("MIAIE_ORACLE_THREADS", min(16, os.cpu_count() or 1)))


# ---------------------------------------------------------------- generators
def tensor_seed(tensor_id: int) -> int:
    return int(_lib().oracle_tensor_seed(tensor_id))


def fill_i8(n: int, tensor_id: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int8)
    _lib().oracle_fill_i8(_ptr(out), n, tensor_id)
    return out


def fill_shift(n: int, tensor_id: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint8)
    _lib().oracle_fill_shift(_ptr(out), n, tensor_id)
    return out


def fill_bf16_normal(n: int, tensor_id: int, scale: float) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    _lib().oracle_fill_bf16_normal(_ptr(out), n, tensor_id, scale)
    return out


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- reference goldens
def mm_window_i32(win: np.ndarray, n: int) -> np.ndarray:
    """oracle_mm_window_i32: aieml_mm.cc:194-230 on a packed A||B window."""
    win = np.ascontiguousarray(win, dtype=np.int32)
    assert win.size == 2 * n * n
    out = np.zeros(n * n, dtype=np.int32)
    _lib().oracle_mm_window_i32(_ptr(win), _ptr(out), n)
    return out


def count_mismatch_i32(want: np.ndarray, got: np.ndarray) -> int:
    want = np.ascontiguousarray(want, dtype=np.int32)
    got = np.ascontiguousarray(got, dtype=np.int32)
    return int(_lib().oracle_count_mismatch_i32(_ptr(want), _ptr(got), want.size))


def gemm_i8(A: np.ndarray, B: np.ndarray, b_nt: bool = False, rows=None, nthreads=None,
            lib: str | None = None) -> np.ndarray:
    """int8 GEMM with int32 accumulation.  NT: oracle_gemm_i8_nt_rows; NN: oracle_gemm_i8_nn_rows.

    Returns C[row0:row1, :] (all rows by default)."""
    A = np.ascontiguousarray(A, dtype=np.int8)
    B = np.ascontiguousarray(B, dtype=np.int8)
    M, K = A.shape
    N = B.shape[0] if b_nt else B.shape[1]
    assert (B.shape[1] if b_nt else B.shape[0]) == K
    r0, r1 = rows if rows is not None else (0, M)
    nt = nthreads or default_threads()
    Cfull = np.zeros((r1 - r0, N), dtype=np.int32)
    Asub = np.ascontiguousarray(A[r0:r1])
    L = _lib(lib)
    if b_nt:
        L.oracle_gemm_i8_nt_rows(_ptr(Asub), _ptr(B), _ptr(Cfull), r1 - r0, N, K, K, K, N, 0, r1 - r0, nt)
    else:
        rc = L.oracle_gemm_i8_nn_rows(_ptr(Asub), _ptr(B), _ptr(Cfull), r1 - r0, N, K, K, N, N, 0, r1 - r0, nt)
        assert rc == 0
    return Cfull


def requant(acc: np.ndarray, shift: int, relu: bool = False) -> np.ndarray:
    """oracle_requant_buf: sat_int8((acc + 2^(s-1)) >> s), optional ReLU."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    y = np.empty(acc.shape, dtype=np.int8)
    _lib().oracle_requant_buf(_ptr(acc), _ptr(y), acc.size, shift, int(relu))
    return y


def requant_scalar(acc: int, shift: int, relu: bool = False) -> int:
    return int(_lib().oracle_requant(acc, shift, int(relu)))


def gemm_i8_rq(A, B, shift, relu=False, b_nt=False, rows=None, nthreads=None, want_acc=False):
    """oracle_gemm_i8_rq_rows: GEMM + requant; returns Y rows (and the int32 accumulators)."""
    A = np.ascontiguousarray(A, dtype=np.int8)
    B = np.ascontiguousarray(B, dtype=np.int8)
    M, K = A.shape
    N = B.shape[0] if b_nt else B.shape[1]
    r0, r1 = rows if rows is not None else (0, M)
    Y = np.zeros((M, N), dtype=np.int8)
    Cd = np.zeros((M, N), dtype=np.int32) if want_acc else None
    rc = _lib().oracle_gemm_i8_rq_rows(_ptr(A), _ptr(B), _ptr(Y), _ptr(Cd) if want_acc else None,
                                       M, N, K, int(b_nt), shift, int(relu), r0, r1,
                                       nthreads or default_threads())
    assert rc == 0
    if want_acc:
        return Y[r0:r1], Cd[r0:r1]
    return Y[r0:r1]


def gemm_bf16(A_bits: np.ndarray, B_bits: np.ndarray, rows=None, nthreads=None, f64=False):
    """oracle_gemm_bf16_rows (fp32 accumulate) or oracle_gemm_bf16_f64_rows."""
    A_bits = np.ascontiguousarray(A_bits, dtype=np.uint16)
    B_bits = np.ascontiguousarray(B_bits, dtype=np.uint16)
    M, K = A_bits.shape
    N = B_bits.shape[1]
    r0, r1 = rows if rows is not None else (0, M)
    out = np.zeros((r1 - r0, N), dtype=np.float64 if f64 else np.float32)
    fn = _lib().oracle_gemm_bf16_f64_rows if f64 else _lib().oracle_gemm_bf16_rows
    fn(_ptr(A_bits), _ptr(B_bits), _ptr(out), M, N, K, r0, r1, nthreads or default_threads())
    return out


def conv2d_nhwc_i8(X, W, shifts, stride=1, pad=1, relu=False, want_acc=False, nthreads=None):
    """oracle_conv2d_nhwc_i8: direct 7-loop NHWC x OHWI conv + per-channel requant."""
    X = np.ascontiguousarray(X, dtype=np.int8)
    W = np.ascontiguousarray(W, dtype=np.int8)
    shifts = np.ascontiguousarray(shifts, dtype=np.uint8)
    N, H, Wd, Cin = X.shape
    Cout, R, S, Cin2 = W.shape
    assert Cin == Cin2 and shifts.size == Cout
    Ho = (H + 2 * pad - R) // stride + 1
    Wo = (Wd + 2 * pad - S) // stride + 1
    Y = np.zeros((N, Ho, Wo, Cout), dtype=np.int8)
    Y32 = np.zeros((N, Ho, Wo, Cout), dtype=np.int32) if want_acc else None
    _lib().oracle_conv2d_nhwc_i8(_ptr(X), _ptr(W), _ptr(shifts), _ptr(Y),
                                 _ptr(Y32) if want_acc else None, N, H, Wd, Cin, Cout, R, S,
                                 stride, pad, int(relu), nthreads or default_threads())
    return (Y, Y32) if want_acc else Y


def mlp_i8(X, W1, W2, s1, s2, rows=None, nthreads=None, want_h=False):
    """oracle_mlp_i8_rows: Y = rq_s2(relu(rq_s1(X W1)) W2)."""
    X = np.ascontiguousarray(X, dtype=np.int8)
    W1 = np.ascontiguousarray(W1, dtype=np.int8)
    W2 = np.ascontiguousarray(W2, dtype=np.int8)
    M, K = X.shape
    F = W1.shape[1]
    Nout = W2.shape[1]
    r0, r1 = rows if rows is not None else (0, M)
    Y = np.zeros((M, Nout), dtype=np.int8)
    H = np.zeros((M, F), dtype=np.int8) if want_h else None
    rc = _lib().oracle_mlp_i8_rows(_ptr(X), _ptr(W1), _ptr(W2), _ptr(Y), _ptr(H) if want_h else None,
                                   M, K, F, Nout, s1, s2, r0, r1, nthreads or default_threads())
    assert rc == 0
    return (Y[r0:r1], H[r0:r1]) if want_h else Y[r0:r1]


def dot_u8_probe(param_nn: int) -> np.ndarray:
    """oracle_dot_u8_probe: aie_nokernelload.cc:50-83."""
    inp = np.zeros(512, dtype=np.uint32)
    inp[0] = param_nn
    out = np.zeros(5, dtype=np.uint32)
    _lib().oracle_dot_u8_probe(_ptr(inp), _ptr(out))
    return out


def mm_square_u64(inp: np.ndarray, n: int, iters: int = 1) -> np.ndarray:
    """oracle_mm_square_u64: vek385_verification.cpp:56-69."""
    inp = np.ascontiguousarray(inp, dtype=np.uint64)
    out = np.zeros(n * n + 1, dtype=np.uint64)
    _lib().oracle_mm_square_u64(_ptr(inp), _ptr(out), n, iters)
    return out


def chain_add(inp: np.ndarray, length: int, addends) -> np.ndarray:
    """oracle_chain_add: multi_tile.cpp:39-47 / seq_full_col.cpp:39-47 chains."""
    inp = np.ascontiguousarray(inp, dtype=np.int32)
    add = np.ascontiguousarray(np.asarray(addends, dtype=np.int32))
    out = np.zeros(length, dtype=np.int32)
    _lib().oracle_chain_add(_ptr(inp), _ptr(out), length, _ptr(add), add.size)
    return out
