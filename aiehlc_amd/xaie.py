"""ctypes binding of the aie-rt-shaped facade (include/miaie_xaie.h,
aiehlc_amd/lib/libmiaie_xaie.so).

The structures mirror the header field for field; `Device` wraps the
partition set-up the reference examples perform in main()
(example/perf/aieml_perf.cc:265-313) and raises `XAieError` on a status
other than XAIE_OK.  There is no fallback: a missing library raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
# MIAIE_LIB_DIR selects another build of the same library (the host-sanitized
# one in aiehlc_amd/lib_san, see aiehlc_amd/build.py); default aiehlc_amd/lib
LIB_DIR = os.environ.get("MIAIE_LIB_DIR") or os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libmiaie_xaie.so")
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "miaie_xaie.h")

XAIE_OK = 0
XAIE_ERR = 1
XAIE_INVALID_DEVICE = 2
XAIE_INVALID_ARGS = 3
XAIE_INVALID_TILE = 4
XAIE_INVALID_DATA_MEM_ADDR = 5
XAIE_INVALID_ELF = 6
XAIE_CORE_STATUS_TIMEOUT = 7
XAIE_ERR_NO_ROUTE = 8
XAIE_NOT_SUPPORTED = 9

XAIE_DEV_GEN_AIEML = 2
XAIE_MEM_CACHEABLE = 1
XAIE_IO_BACKEND_BAREMETAL = 0
MIAIE_XAIE_KERNEL_MAGIC = 0x4B45494D
MIAIE_XAIE_MAX_PARAMS = 4
MIAIE_XAIE_KERNEL_FOREVER = 1


class LocType(C.Structure):
    _fields_ = [("Row", C.c_uint8), ("Col", C.c_uint8)]


def tile(col: int, row: int) -> LocType:
    """XAie_TileLoc(col, row)."""
    return LocType(row, col)


class Config(C.Structure):
    _fields_ = [("AieGen", C.c_uint8), ("BaseAddr", C.c_uint64), ("ColShift", C.c_uint8), ("RowShift", C.c_uint8),
                ("NumCols", C.c_uint8), ("NumRows", C.c_uint8), ("ShimRowNum", C.c_uint8),
                ("MemTileRowStart", C.c_uint8), ("MemTileNumRows", C.c_uint8), ("AieTileRowStart", C.c_uint8),
                ("AieTileNumRows", C.c_uint8)]


class Backend(C.Structure):
    _fields_ = [("Type", C.c_int), ("Name", C.c_char_p)]


class DevInst(C.Structure):
    _fields_ = [("Backend", C.POINTER(Backend)), ("IsReady", C.c_uint8), ("AieGen", C.c_uint8),
                ("BaseAddr", C.c_uint64), ("NumCols", C.c_uint8), ("NumRows", C.c_uint8), ("ShimRow", C.c_uint8),
                ("MemTileRowStart", C.c_uint8), ("MemTileNumRows", C.c_uint8), ("AieTileRowStart", C.c_uint8),
                ("AieTileNumRows", C.c_uint8), ("StartCol", C.c_uint8), ("PartNumCols", C.c_uint8),
                ("PartBaseAddr", C.c_uint64), ("Priv", C.c_void_p)]


LaunchFn = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_void_p, C.POINTER(C.c_uint32), C.c_uint32, C.POINTER(C.c_uint32),
                       C.c_uint32, C.c_uint32, C.c_void_p)


class Kernel(C.Structure):
    _fields_ = [("Magic", C.c_uint32), ("Name", C.c_char_p), ("NumParams", C.c_uint32),
                ("MemAddress", C.c_uint32 * MIAIE_XAIE_MAX_PARAMS), ("SizeHint", C.c_uint32 * MIAIE_XAIE_MAX_PARAMS),
                ("Flags", C.c_uint32), ("Launch", LaunchFn), ("User", C.c_void_p), ("Builtin", C.c_uint32)]


def kernel(name: str, mem_address=(), size_hint=(), nparams: int = 2, launch=None, flags: int = 0) -> Kernel:
    """A user kernel descriptor: window annotations per parameter (0 = none)."""
    k = Kernel()
    k.Magic = MIAIE_XAIE_KERNEL_MAGIC
    k.Name = name.encode()
    k.NumParams = nparams
    for i, a in enumerate(mem_address):
        k.MemAddress[i] = a
    for i, s in enumerate(size_hint):
        k.SizeHint[i] = s
    k.Flags = flags
    if launch is not None:
        k.Launch = launch
    return k


class XAieError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"AieRC {code}: {msg}")
        self.code = code


_p, _u8, _u32, _u64 = C.c_void_p, C.c_uint8, C.c_uint32, C.c_uint64
_rc = C.c_int
_dev = C.POINTER(DevInst)
SIGS = {
    "XAie_MiaieWindowLayout": (_rc, [C.POINTER(Kernel), C.POINTER(_u32), C.POINTER(_u32)]),
    "XAie_MiaieLastError": (C.c_char_p, [_dev]),
    "XAie_MiaieTileMemBytes": (_u32, [_dev, LocType]),
    "XAie_SetupPartitionConfig": (_rc, [_dev, _u64, _u32, _u32]),
    "XAie_CfgInitialize": (_rc, [_dev, C.POINTER(Config)]),
    "XAie_SetIOBackend": (_rc, [_dev, C.c_int]),
    "XAie_UpdateNpiAddr": (_rc, [_dev, _u64]),
    "XAie_PartitionInitialize": (_rc, [_dev, _p]),
    "XAie_PmRequestTiles": (_rc, [_dev, _p, _u32]),
    "XAie_PartitionTeardown": (_rc, [_dev]),
    "XAie_Finish": (_rc, [_dev]),
    "XAie_CoreReset": (_rc, [_dev, LocType]),
    "XAie_CoreUnreset": (_rc, [_dev, LocType]),
    "XAie_LoadElfMem": (_rc, [_dev, LocType, _p]),
    "XAie_CoreEnable": (_rc, [_dev, LocType]),
    "XAie_CoreDisable": (_rc, [_dev, LocType]),
    "XAie_CoreWaitForDone": (_rc, [_dev, LocType, _u32]),
    "XAie_CoreReadDoneBit": (_rc, [_dev, LocType, C.POINTER(_u8)]),
    "XAie_CoreGetStatus": (_rc, [_dev, LocType, C.POINTER(_u32)]),
    "XAie_DataMemBlockWrite": (_rc, [_dev, LocType, _u64, _p, _u32]),
    "XAie_DataMemBlockRead": (_rc, [_dev, LocType, _u64, _p, _u32]),
    "XAie_DataMemWrWord": (_rc, [_dev, LocType, _u64, _u32]),
    "XAie_DataMemRdWord": (_rc, [_dev, LocType, _u64, C.POINTER(_u32)]),
    "XAie_MemAllocate": (_p, [_dev, _u64, C.c_int]),
    "XAie_MemFree": (_rc, [_p]),
    "XAie_MemGetVAddr": (_p, [_p]),
    "XAie_MemGetDevAddr": (_u64, [_p]),
    "XAie_MemSyncForDev": (_rc, [_p]),
    "XAie_MemSyncForCPU": (_rc, [_p]),
    "XAie_InitRoutingHandler": (_p, [_dev]),
    "XAie_Route": (_rc, [_p, _p, LocType, LocType]),
    "XAie_MoveData": (_rc, [_p, LocType, _p, _u32, _p, LocType]),
    "XAie_MoveDataExternal2Aie": (_rc, [_p, LocType, _p, _u32, _u64, LocType]),
    "XAie_MoveDataAie2External": (_rc, [_p, LocType, _u64, _u32, _p, LocType]),
    "XAie_RouteDmaWait": (_rc, [_p, LocType, LocType, _u8]),
    "XAie_Run": (_rc, [_p, _u32]),
    "XAie_RoutingInstanceFree": (_rc, [_p]),
    "XAie_LoadKernel": (_p, [C.c_char_p, C.c_int, C.c_int]),
    "XAie_RoutingHostToAie": (_rc, [_p, LocType]),
    "XAie_RoutingAieToHost": (_rc, [_p, LocType]),
    "XAie_MoveDataToAie": (_rc, [_p, C.c_int, _p, C.c_size_t]),
    "XAie_RunCore": (_rc, [_p]),
    "XAie_WaitOutData": (_rc, [_p]),
    "XAie_MoveAieToData": (_rc, [_p, C.c_int, _p, C.c_size_t]),
    "XAie_KernelFree": (_rc, [_p]),
    "XAie_MiaieRunOnDdr": (_rc, [C.POINTER(Kernel), _u32, _u32, _u32, _u32, _u64, _u64]),
}
BUILTINS = ("miaie_xaie_mm", "miaie_xaie_mm8", "miaie_xaie_perf", "miaie_xaie_k1", "miaie_xaie_k2", "miaie_xaie_mm3_u64",
            "miaie_xaie_perf_u8")

_lib = None


def load_library(path: str = LIB_PATH) -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = C.CDLL(path)
    for name, (res, args) in SIGS.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    _lib = lib
    return lib


def builtin(name: str) -> Kernel:
    """One of the built-in kernel descriptors (e.g. "miaie_xaie_k1")."""
    return Kernel.in_dll(load_library(), name)


def header_functions(path: str = HEADER_PATH) -> list[str]:
    """Names of every MIAIE_XAIE_API function declared in include/miaie_xaie.h."""
    text = open(path).read()
    return re.findall(r"MIAIE_XAIE_API\s+(?!extern)[\w\s\*]+?\b(XAie_\w+)\s*\(", text)


def header_objects(path: str = HEADER_PATH) -> list[str]:
    """Names of the kernel descriptors the header exports."""
    return re.findall(r"MIAIE_XAIE_API\s+extern\s+const\s+XAie_MiaieKernel\s+(\w+)\s*;", open(path).read())


def window_layout(k: Kernel) -> tuple[list[int], list[int]]:
    lib = load_library()
    ping = (C.c_uint32 * MIAIE_XAIE_MAX_PARAMS)()
    pong = (C.c_uint32 * MIAIE_XAIE_MAX_PARAMS)()
    rc = lib.XAie_MiaieWindowLayout(C.byref(k), ping, pong)
    if rc != XAIE_OK:
        raise XAieError(rc, lib.XAie_MiaieLastError(None).decode())
    return list(ping)[: k.NumParams], list(pong)[: k.NumParams]


class Device:
    """An initialised partition (XAie_SetupConfig + XAie_CfgInitialize +
    XAie_SetIOBackend + XAie_PartitionInitialize) with the examples'
    AIE-ML geometry, 38 columns x 11 rows (example/matrixmultiply/aieml_mm.cc:19-31)."""

    def __init__(self, cols: int = 38, rows: int = 11, start_col: int = 0, part_cols: int = 0):
        self.lib = load_library()
        self.inst = DevInst()
        self.cfg = Config(XAIE_DEV_GEN_AIEML, 0x20000000000, 25, 20, cols, rows, 0, 1, 2, 3, rows - 3)
        if part_cols:
            self.check(self.lib.XAie_SetupPartitionConfig(C.byref(self.inst), 0x20000000000 + (start_col << 25),
                                                          start_col, part_cols))
        self.check(self.lib.XAie_CfgInitialize(C.byref(self.inst), C.byref(self.cfg)))
        self.check(self.lib.XAie_SetIOBackend(C.byref(self.inst), XAIE_IO_BACKEND_BAREMETAL))
        self.check(self.lib.XAie_PartitionInitialize(C.byref(self.inst), None))

    @property
    def ref(self):
        return C.byref(self.inst)

    def check(self, rc: int) -> None:
        if rc != XAIE_OK:
            raise XAieError(rc, self.lib.XAie_MiaieLastError(C.byref(self.inst)).decode())

    def call(self, name: str, *args) -> int:
        """Call XAie_<name>(&DevInst, *args) and return its status."""
        return getattr(self.lib, "XAie_" + name)(self.ref, *args)

    def close(self) -> None:
        if self.inst.IsReady:
            self.check(self.lib.XAie_PartitionTeardown(self.ref))

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
