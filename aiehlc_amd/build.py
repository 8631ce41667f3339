"""Build step for the miaie HIP library (gfx950 only).

Compiles every aiehlc_amd/csrc/*.hip translation unit with hipcc for gfx950
and links them into aiehlc_amd/lib/libmiaie.so, builds the aie-rt-shaped
facade aiehlc_amd/csrc/xaie/*.hip into aiehlc_amd/lib/libmiaie_xaie.so on top
of it, then the harness programs in aiehlc_amd/harness/ (C++ against
miaie.hpp, C against miaie_xaie.h, and the aiehlc-dialect samples in
harness/hlc/ through the hlc.py front end) and the measurement probes in
aiehlc_amd/probes/.  Runs on a machine without a GPU
(hipcc cross-compiles).

The same sources are also built twice more: with host-side AddressSanitizer
and UndefinedBehaviorSanitizer (aiehlc_amd/lib_san/), and with device-side
bounds checks in every kernel (aiehlc_amd/lib_dbg/, MIAIE_DEVICE_CHECKS=1,
csrc/dbg_checks.hpp).  A process selects either with MIAIE_LIB_DIR.

Flags: -O3, C++17, hidden visibility (only the MIAIE_API symbols of
include/miaie.h are exported), packed-FP32 instruction selection turned
off (`-Xclang -target-feature -Xclang -packed-fp32-ops`), and kernel
arguments preloaded into SGPRs (`-mllvm -amdgpu-kernarg-preload-count=16`).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
LIBDIR = os.path.join(HERE, "lib")
SANDIR = os.path.join(HERE, "lib_san")
DBGDIR = os.path.join(HERE, "lib_dbg")
LIB = os.path.join(LIBDIR, "libmiaie.so")
HARNESS = os.path.join(HERE, "harness")
XAIE_SRC = os.path.join(CSRC, "xaie")
XAIE_LIB = os.path.join(LIBDIR, "libmiaie_xaie.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # kernel arguments arrive in SGPRs at wave launch instead of through a
    # scalar load from the (cold) kernarg segment on each kernel's critical path
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall", "-Wno-unused-function",
    f"-I{os.path.join(ROOT, 'include')}",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = (r.stdout + r.stderr).strip()
    # hipcc's host pass does not know the packed-fp32 feature: harmless, drop it
    lines = [l for l in out.splitlines() if "packed-fp32-ops" not in l and l.strip()
             and "not a recognized feature for this target" not in l]
    if r.returncode != 0:
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}\n" + "\n".join(lines))
    if lines and verbose:
        print("\n".join(lines), flush=True)


# Host code of the libraries built again with AddressSanitizer and
# UndefinedBehaviorSanitizer (device code is built as usual: the flags apply
# to the host pass only).  The result, aiehlc_amd/lib_san/, is loaded by
# setting MIAIE_LIB_DIR and preloading clang's ASan runtime (asan_runtime()).
SAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer", "-Xarch_host", "-g"]


def asan_runtime() -> str | None:
    """clang's shared ASan runtime (the one hipcc's host pass instruments for)."""
    import glob

    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def build(verbose: bool = False, jobs: int | None = None) -> str:
    os.makedirs(OBJ, exist_ok=True)
    os.makedirs(LIBDIR, exist_ok=True)
    # the device-checked library's objects take longest (its int8 GEMM unit
    # alone about 3.5 minutes): compile them beside everything else
    dbg_pool = cf.ThreadPoolExecutor(2)
    dbg_futs = _device_checked_objects(dbg_pool, verbose)
    srcs = sources()
    objs = [os.path.join(OBJ, os.path.basename(s)[:-4] + ".o") for s in srcs]
    jobs = jobs or min(8, len(srcs))
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", s, "-o", o], verbose) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    tmp = LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB)
    build_xaie(verbose)
    build_harness(verbose)
    build_hlc_samples(verbose)
    build_probes(verbose)
    build_sanitized(verbose, jobs)
    for f in dbg_futs:
        f.result()
    dbg_pool.shutdown()
    _link_device_checked(verbose)
    return LIB


def build_sanitized(verbose: bool = False, jobs: int | None = None) -> str:
    """aiehlc_amd/lib_san/libmiaie.so and libmiaie_xaie.so with sanitized host code."""
    sobj = os.path.join(OBJ, "san")
    os.makedirs(sobj, exist_ok=True)
    os.makedirs(SANDIR, exist_ok=True)
    srcs = sources()
    xsrcs = sorted(os.path.join(XAIE_SRC, f) for f in os.listdir(XAIE_SRC) if f.endswith(".hip"))
    objs = [os.path.join(sobj, os.path.basename(s)[:-4] + ".o") for s in srcs]
    xobjs = [os.path.join(sobj, "xaie_" + os.path.basename(s)[:-4] + ".o") for s in xsrcs]
    jobs = jobs or min(8, len(srcs) + len(xsrcs))
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, *SAN_FLAGS, "-c", s, "-o", o], verbose)
                for s, o in zip(srcs + xsrcs, objs + xobjs)]
        for f in futs:
            f.result()
    lib = os.path.join(SANDIR, "libmiaie.so")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", lib + ".tmp", *objs], verbose)
    os.replace(lib + ".tmp", lib)
    xlib = os.path.join(SANDIR, "libmiaie_xaie.so")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", xlib + ".tmp", *xobjs, f"-L{SANDIR}", "-lmiaie",
          "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(xlib + ".tmp", xlib)
    return lib


def _device_checked_objects(pool: cf.Executor, verbose: bool) -> list:
    dobj = os.path.join(OBJ, "dbg")
    os.makedirs(dobj, exist_ok=True)
    # longest first (gemm_i8.hip)
    srcs = sorted(sources(), key=lambda p: os.path.basename(p) != "gemm_i8.hip")
    return [pool.submit(_run, [HIPCC, *HIP_FLAGS, "-DMIAIE_DEVICE_CHECKS=1", "-c", s,
                               "-o", os.path.join(dobj, os.path.basename(s)[:-4] + ".o")], verbose) for s in srcs]


def _link_device_checked(verbose: bool) -> str:
    os.makedirs(DBGDIR, exist_ok=True)
    dobj = os.path.join(OBJ, "dbg")
    objs = [os.path.join(dobj, os.path.basename(s)[:-4] + ".o") for s in sources()]
    lib = os.path.join(DBGDIR, "libmiaie.so")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", lib + ".tmp", *objs], verbose)
    os.replace(lib + ".tmp", lib)
    return lib


def build_device_checked(verbose: bool = False, jobs: int | None = None) -> str:
    """aiehlc_amd/lib_dbg/libmiaie.so: the same library with device-side
    bounds checks (MIAIE_DEVICE_CHECKS=1, csrc/dbg_checks.hpp): every global
    access of every kernel is checked against the runtime's buffer table."""
    with cf.ThreadPoolExecutor(jobs or 8) as pool:
        for f in _device_checked_objects(pool, verbose):
            f.result()
    return _link_device_checked(verbose)


def build_xaie(verbose: bool = False) -> str:
    """libmiaie_xaie.so: the aie-rt-shaped facade (include/miaie_xaie.h), a
    client of libmiaie.so with its own tile-array kernels."""
    srcs = sorted(os.path.join(XAIE_SRC, f) for f in os.listdir(XAIE_SRC) if f.endswith(".hip"))
    objs = [os.path.join(OBJ, "xaie_" + os.path.basename(s)[:-4] + ".o") for s in srcs]
    for s, o in zip(srcs, objs):
        _run([HIPCC, *HIP_FLAGS, "-c", s, "-o", o], verbose)
    tmp = XAIE_LIB + ".tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, f"-L{LIBDIR}", "-lmiaie",
          "-Wl,-rpath,$ORIGIN"], verbose)
    os.replace(tmp, XAIE_LIB)
    return XAIE_LIB


def build_harness(verbose: bool = False) -> None:
    if not os.path.isdir(HARNESS):
        return
    for f in sorted(os.listdir(HARNESS)):
        if f.endswith(".cpp"):
            exe = os.path.join(HARNESS, f[:-4])
            cmd = ["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", f"-I{os.path.join(ROOT, 'include')}",
                   os.path.join(HARNESS, f), "-o", exe + ".tmp", f"-L{LIBDIR}", "-lmiaie", "-pthread",
                   "-Wl,-rpath,$ORIGIN/../lib"]
        elif f.endswith(".c"):
            # C programs written against the aie-rt-shaped facade
            exe = os.path.join(HARNESS, f[:-2])
            cmd = ["gcc", "-O2", "-std=c11", "-Wall", "-Wextra", f"-I{os.path.join(ROOT, 'include')}",
                   os.path.join(HARNESS, f), "-o", exe + ".tmp", f"-L{LIBDIR}", "-lmiaie_xaie", "-lmiaie",
                   "-Wl,-rpath,$ORIGIN/../lib"]
        else:
            continue
        _run(cmd, verbose)
        os.replace(exe + ".tmp", exe)


def build_hlc_samples(verbose: bool = False) -> None:
    """Programs in the aiehlc dialect (aiehlc_amd/harness/hlc/*.cc), rewritten
    by aiehlc_amd/hlc.py and compiled with g++ into aiehlc_amd/harness/hlc_<name>."""
    sdir = os.path.join(HARNESS, "hlc")
    if not os.path.isdir(sdir):
        return
    sys.path.insert(0, ROOT)
    from aiehlc_amd import hlc  # noqa: E402  (the front end is part of the package)
    os.makedirs(OBJ, exist_ok=True)
    for f in sorted(os.listdir(sdir)):
        if not f.endswith(".cc"):
            continue
        src = os.path.join(sdir, f)
        out, _, _ = hlc.rewrite(open(src).read(), filename=src)
        host = os.path.join(OBJ, "hlc_" + f)
        with open(host, "w") as fh:
            fh.write(out)
        exe = os.path.join(HARNESS, "hlc_" + f[:-3])
        _run(["g++", "-O2", "-std=c++17", "-Wall", "-Wextra", f"-I{os.path.join(ROOT, 'include')}", host, "-o",
              exe + ".tmp", f"-L{LIBDIR}", "-lmiaie_xaie", "-lmiaie", "-Wl,-rpath,$ORIGIN/../lib"], verbose)
        os.replace(exe + ".tmp", exe)


def build_probes(verbose: bool = False) -> None:
    """Standalone measurement programs (aiehlc_amd/probes/*.hip) used by bench.py."""
    pdir = os.path.join(HERE, "probes")
    if not os.path.isdir(pdir):
        return
    for f in sorted(os.listdir(pdir)):
        if not f.endswith(".hip"):
            continue
        exe = os.path.join(pdir, f[:-4])
        _run([HIPCC, *HIP_FLAGS, os.path.join(pdir, f), "-o", exe + ".tmp"], verbose)
        os.replace(exe + ".tmp", exe)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
