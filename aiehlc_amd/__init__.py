"""aiehlc_amd — host-side mirror of the miaie C ABI (include/miaie.h).

The product is the gfx950 library aiehlc_amd/lib/libmiaie.so; this module
binds it with ctypes and mirrors the reference harness flow
(example/matrixmultiply/aieml_mm.cc:108-249): allocate device memory, move
data in, run a kernel, wait for it, move data back.  There is no fallback:
if the library is missing, importing the bindings raises.

    import aiehlc_amd as mi
    with mi.Context(0) as ctx:
        a = ctx.upload(A); b = ctx.upload(B); y = ctx.empty((M, N), np.int8)
        ctx.gemm_i8_rq(a, b, y, M, N, K, shift=10)
        ctx.wait(10_000)
        Y = ctx.download(y)
"""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np

from . import synth  # noqa: F401  (re-exported)

HERE = os.path.dirname(os.path.abspath(__file__))
# MIAIE_LIB_DIR selects another build of the same library (the host-sanitized
# one in aiehlc_amd/lib_san, the device-checked one in aiehlc_amd/lib_dbg, see
# aiehlc_amd/build.py); default aiehlc_amd/lib
LIB_DIR = os.environ.get("MIAIE_LIB_DIR") or os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libmiaie.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "miaie.h")

MIAIE_OK = 0
MIAIE_EINVAL = -1
MIAIE_EHIP = -2
MIAIE_ETIMEDOUT = -3
MIAIE_ENOMEM = -4
MIAIE_EUNSUPPORTED = -5
MIAIE_EFAULT = -6
B_NN = 0
B_NT = 1

_ERR_NAMES = {
    MIAIE_EINVAL: "MIAIE_EINVAL",
    MIAIE_EHIP: "MIAIE_EHIP",
    MIAIE_ETIMEDOUT: "MIAIE_ETIMEDOUT",
    MIAIE_ENOMEM: "MIAIE_ENOMEM",
    MIAIE_EUNSUPPORTED: "MIAIE_EUNSUPPORTED",
}


class MiaieError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{_ERR_NAMES.get(code, code)}: {msg}")
        self.code = code


_p, _i, _sz, _u64 = C.c_void_p, C.c_int, C.c_size_t, C.c_uint64
_SIGS = {
    "miaie_init": (_i, [C.POINTER(_p), _i]),
    "miaie_init_on_stream": (_i, [C.POINTER(_p), _i, _p]),
    "miaie_finish": (_i, [_p]),
    "miaie_last_error_string": (C.c_char_p, [_p]),
    "miaie_get_stream": (_i, [_p, C.POINTER(_p)]),
    "miaie_alloc": (_i, [_p, _sz, C.POINTER(_p)]),
    "miaie_free": (_i, [_p, _p]),
    "miaie_copy_h2d": (_i, [_p, _p, _p, _sz]),
    "miaie_copy_d2h": (_i, [_p, _p, _p, _sz]),
    "miaie_copy_d2d": (_i, [_p, _p, _p, _sz]),
    "miaie_wait": (_i, [_p, _i]),
    "miaie_debug_device_checks": (_i, []),
    "miaie_debug_register": (_i, [_p, _p, _sz]),
    "miaie_debug_unregister": (_i, [_p, _p]),
    "miaie_mm_window_i32": (_i, [_p, _p, _p, _i]),
    "miaie_perf_window_u32": (_i, [_p, _p, _p, _i]),
    "miaie_dot_u8_probe": (_i, [_p, _p, _p]),
    "miaie_mm_square_u64": (_i, [_p, _p, _p, _i, _i, _u64]),
    "miaie_chain_add_i32": (_i, [_p, _p, _p, _i, _p, _i]),
    "miaie_gemm_i8_i32": (_i, [_p, _p, _p, _p] + [_i] * 7),
    "miaie_gemm_i8_rq": (_i, [_p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _i]),
    "miaie_gemm_bf16_f32": (_i, [_p, _p, _p, _p, _i, _i, _i]),
    "miaie_conv2d_i8_nhwc": (_i, [_p, _p, _p, _p, _p] + [_i] * 9),
    "miaie_mlp_i8": (_i, [_p, _p, _p, _p, _p, _p] + [_i] * 6),
    "miaie_mlp_i8_noalloc": (_i, [_p, _p, _p, _p, _p] + [_i] * 6),
    "miaie_fill_i8": (_i, [_p, _p, _sz, _u64]),
    "miaie_plan_gemm_i8": (_i, [_p, _i, _i, _i, _p]),
    "miaie_plan_set_cus": (_i, [_p, _i, C.POINTER(_i)]),
    "miaie_plan_conv2d_i8": (_i, [_i] * 9 + [C.POINTER(_i)]),
    "miaie_graph_begin": (_i, [_p]),
    "miaie_graph_end": (_i, [_p, C.POINTER(_p)]),
    "miaie_graph_launch": (_i, [_p, _p]),
    "miaie_graph_destroy": (_i, [_p]),
    "miaie_version": (C.c_char_p, []),
}

_lib: C.CDLL | None = None


def load_library(path: str = LIB_PATH) -> C.CDLL:
    """Load libmiaie.so (built by aiehlc_amd/build.py).  Raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                          "(there is no CPU fallback)")
    lib = C.CDLL(path)
    for name, (res, args) in _SIGS.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib


def header_functions(path: str = HEADER_PATH) -> list[str]:
    """Names of every MIAIE_API function declared in include/miaie.h."""
    text = open(path).read()
    return re.findall(r"MIAIE_API\s+[\w\s\*]+?\b(miaie_\w+)\s*\(", text)


CONV_KERNELS = {0: "rows", 1: "igemm", 2: "direct", 3: "taps", 4: "rows_deep"}  # MIAIE_CONV_*


def plan_conv2d_i8(N, H, W, Cin, Cout, R=3, S=3, stride=1, pad=1) -> str:
    """Which conv kernel miaie_conv2d_i8_nhwc runs for this shape (16-byte
    aligned buffers).  A host function: needs no device."""
    k = _i(-1)
    rc = load_library().miaie_plan_conv2d_i8(N, H, W, Cin, Cout, R, S, stride, pad, C.byref(k))
    if rc != MIAIE_OK:
        raise MiaieError(rc, load_library().miaie_last_error_string(None).decode())
    return CONV_KERNELS[k.value]


class DeviceBuffer:
    """Device allocation owned by a Context (XAie_MemInst analogue)."""

    def __init__(self, ctx: "Context", ptr: int, nbytes: int, dtype=None, shape=None):
        self.ctx, self.ptr, self.nbytes = ctx, ptr, nbytes
        self.dtype = np.dtype(dtype) if dtype is not None else None
        self.shape = tuple(shape) if shape is not None else None

    @property
    def value(self) -> int:
        return self.ptr

    def free(self) -> None:
        if self.ptr:
            self.ctx._call("miaie_free", self.ptr)
            self.ptr = 0


def _addr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


KERNEL_TILE64 = 0
KERNEL_PIPE = 1
KERNEL_PIPE_MIXED = 2  # 256x256 tiles, then 256x128 tiles over the last columns


class GemmPlan(C.Structure):
    """miaie_gemm_plan (include/miaie.h)."""
    _fields_ = [("kernel", C.c_int), ("tile_m", C.c_int), ("tile_n", C.c_int), ("workgroups", C.c_int),
                ("threads", C.c_int)]

    def as_dict(self) -> dict:
        return {f: getattr(self, f) for f, _ in self._fields_}


class Graph:
    """A recorded chain of entry points (miaie_graph_*), replayed by launch()."""

    def __init__(self, ctx: "Context"):
        self.ctx = ctx
        self.handle = None

    def launch(self) -> None:
        if not self.handle:
            raise MiaieError(MIAIE_EINVAL, "graph is not recorded yet")
        self.ctx._call("miaie_graph_launch", self.handle)

    def destroy(self) -> None:
        if self.handle:
            self.ctx.lib.miaie_graph_destroy(self.handle)
            self.handle = None


class _Recording:
    def __init__(self, ctx: "Context"):
        self.ctx = ctx
        self.graph = Graph(ctx)

    def __enter__(self) -> Graph:
        self.ctx._call("miaie_graph_begin")
        return self.graph

    def __exit__(self, exc_type, *exc):
        h = _p()
        rc = self.ctx.lib.miaie_graph_end(self.ctx.handle, C.byref(h) if exc_type is None else None)
        if exc_type is None:
            if rc != MIAIE_OK:
                raise MiaieError(rc, self.ctx.last_error())
            self.graph.handle = h.value
        return False


class Context:
    """One miaie context: a device, a stream, and the last error text."""

    def __init__(self, device: int = 0, stream: int | None = None):
        self.lib = load_library()
        h = _p()
        if stream is None:
            rc = self.lib.miaie_init(C.byref(h), device)
        else:
            rc = self.lib.miaie_init_on_stream(C.byref(h), device, stream)
        if rc != MIAIE_OK:
            raise MiaieError(rc, self.lib.miaie_last_error_string(None).decode())
        self.handle = h.value
        self.device = device
        self._bufs: list[DeviceBuffer] = []

    # -- plumbing
    def _call(self, name: str, *args) -> int:
        rc = getattr(self.lib, name)(self.handle, *args)
        if rc != MIAIE_OK:
            raise MiaieError(rc, self.lib.miaie_last_error_string(self.handle).decode())
        return rc

    def call_status(self, name: str, *args) -> int:
        """Call an entry point and return its status instead of raising."""
        return getattr(self.lib, name)(self.handle, *args)

    def last_error(self) -> str:
        return self.lib.miaie_last_error_string(self.handle).decode()

    def close(self) -> None:
        if self.handle:
            for b in self._bufs:
                b.free()
            self._bufs.clear()
            rc = self.lib.miaie_finish(self.handle)
            self.handle = None
            if rc != MIAIE_OK:
                raise MiaieError(rc, "miaie_finish")

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def stream(self) -> int:
        s = _p()
        self._call("miaie_get_stream", C.byref(s))
        return s.value or 0

    # -- memory (MemAllocate / MoveData analogues)
    def alloc(self, nbytes: int, dtype=None, shape=None) -> DeviceBuffer:
        p = _p()
        self._call("miaie_alloc", _sz(max(1, nbytes)), C.byref(p))
        b = DeviceBuffer(self, p.value, nbytes, dtype, shape)
        self._bufs.append(b)
        return b

    def empty(self, shape, dtype) -> DeviceBuffer:
        shape = tuple(shape) if np.ndim(shape) else (int(shape),)
        dt = np.dtype(dtype)
        return self.alloc(int(np.prod(shape)) * dt.itemsize, dt, shape)

    def upload(self, arr: np.ndarray) -> DeviceBuffer:
        arr = np.ascontiguousarray(arr)
        b = self.alloc(arr.nbytes, arr.dtype, arr.shape)
        self._call("miaie_copy_h2d", b.ptr, arr.ctypes.data, _sz(arr.nbytes))
        return b

    def copy_h2d(self, dst: DeviceBuffer, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= dst.nbytes
        self._call("miaie_copy_h2d", dst.ptr, arr.ctypes.data, _sz(arr.nbytes))

    def download(self, buf: DeviceBuffer, dtype=None, shape=None) -> np.ndarray:
        dt = np.dtype(dtype) if dtype is not None else buf.dtype
        shape = shape if shape is not None else buf.shape
        out = np.empty(shape if shape is not None else buf.nbytes // dt.itemsize, dtype=dt)
        self._call("miaie_copy_d2h", out.ctypes.data, buf.ptr, _sz(out.nbytes))
        return out

    def copy_d2d(self, dst, src, nbytes: int) -> None:
        self._call("miaie_copy_d2d", _addr(dst), _addr(src), _sz(nbytes))

    def wait(self, timeout_ms: int = -1) -> None:
        self._call("miaie_wait", timeout_ms)

    # -- device bounds checks (the debug build; no-ops in the product build)
    def device_checks(self) -> bool:
        return bool(self.lib.miaie_debug_device_checks())

    def debug_register(self, buf, nbytes: int) -> None:
        self._call("miaie_debug_register", _addr(buf), _sz(nbytes))

    def debug_unregister(self, buf) -> None:
        self._call("miaie_debug_unregister", _addr(buf))

    def fill_i8(self, buf, n: int, tensor_id: int) -> None:
        self._call("miaie_fill_i8", _addr(buf), _sz(n), _u64(tensor_id))

    def plan_gemm_i8(self, M: int, N: int, K: int) -> dict:
        plan = GemmPlan()
        self._call("miaie_plan_gemm_i8", M, N, K, C.addressof(plan))
        return plan.as_dict()

    def plan_set_cus(self, cus: int) -> int:
        """Plan GEMM tiles for `cus` compute units; returns the previous value."""
        prev = _i(0)
        self._call("miaie_plan_set_cus", cus, C.byref(prev))
        return prev.value

    def record(self) -> _Recording:
        """`with ctx.record() as g: <entry points>` records them into g
        instead of running them; g.launch() replays the chain."""
        return _Recording(self)

    # -- reference kernels
    def mm_window_i32(self, win, out, n: int) -> None:
        self._call("miaie_mm_window_i32", _addr(win), _addr(out), n)

    def perf_window_u32(self, win, out, n: int) -> None:
        self._call("miaie_perf_window_u32", _addr(win), _addr(out), n)

    def dot_u8_probe(self, inp, out) -> None:
        self._call("miaie_dot_u8_probe", _addr(inp), _addr(out))

    def mm_square_u64(self, inp, out, n: int, batch: int, iters: int = 1) -> None:
        self._call("miaie_mm_square_u64", _addr(inp), _addr(out), n, batch, _u64(iters))

    def chain_add_i32(self, inp, out, length: int, addends) -> None:
        add = np.ascontiguousarray(np.asarray(addends, dtype=np.int32))
        self._call("miaie_chain_add_i32", _addr(inp), _addr(out), length,
                   add.ctypes.data if add.size else None, add.size)

    # -- typed GEMM / conv
    def gemm_i8_i32(self, A, B, Cm, M, N, K, lda=None, ldb=None, ldc=None, b_layout=B_NN) -> None:
        lda = K if lda is None else lda
        ldb = (K if b_layout == B_NT else N) if ldb is None else ldb
        ldc = N if ldc is None else ldc
        self._call("miaie_gemm_i8_i32", _addr(A), _addr(B), _addr(Cm), M, N, K, lda, ldb, ldc, b_layout)

    def gemm_i8_rq(self, A, B, Y, M, N, K, shift, relu=False, C_dbg=None, b_layout=B_NN) -> None:
        self._call("miaie_gemm_i8_rq", _addr(A), _addr(B), _addr(Y), M, N, K, shift, int(relu),
                   _addr(C_dbg), b_layout)

    def gemm_bf16_f32(self, A, B, Cm, M, N, K) -> None:
        self._call("miaie_gemm_bf16_f32", _addr(A), _addr(B), _addr(Cm), M, N, K)

    def conv2d_i8_nhwc(self, X, W, shifts, Y, N, H, Wd, Cin, Cout, R=3, S=3, stride=1, pad=1) -> None:
        self._call("miaie_conv2d_i8_nhwc", _addr(X), _addr(W), _addr(shifts), _addr(Y), N, H, Wd, Cin, Cout,
                   R, S, stride, pad)

    def mlp_i8(self, X, W1, W2, H, Y, M, K, F, Nout, s1, s2) -> None:
        self._call("miaie_mlp_i8", _addr(X), _addr(W1), _addr(W2), _addr(H), _addr(Y), M, K, F, Nout, s1, s2)

    def mlp_i8_noalloc(self, X, W1, W2, Y, M, K, F, Nout, s1, s2) -> None:
        """miaie_mlp_i8 with H in the library's own device array (allocates nothing)."""
        self._call("miaie_mlp_i8_noalloc", _addr(X), _addr(W1), _addr(W2), _addr(Y), M, K, F, Nout, s1, s2)


def version() -> str:
    return load_library().miaie_version().decode()
