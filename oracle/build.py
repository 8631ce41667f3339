"""Build recipe for the CPU oracle (test infrastructure only).

Compiles oracle/miaie_oracle.c with gcc into two shared libraries:
  oracle/liboracle.so     -O2 -fopenmp   (checker, and the timed CPU baseline)
  oracle/liboracle_os.so  -Os -fopenmp   (the reference host's -Os flag,
                                          script/aiehlc.sh:343, reported beside it)
  oracle/liboracle_san.so -O1 -fopenmp with ASan and UBSan (the CPU tests run
                                          under it, tests/test_sanitizers.py)

The reference's own golden loops cannot be compiled here: they live inside
harness programs that include aie-rt's xaiengine.h and the Xilinx BSP
(example/matrixmultiply/aieml_mm.cc:8-14), neither of which is vendored, so
there is no oracle/_ref build.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "miaie_oracle.c")
OUTS = {
    "liboracle.so": ["-O2"],
    "liboracle_os.so": ["-Os"],
    # AddressSanitizer + UndefinedBehaviorSanitizer build, loaded by setting
    # MIAIE_ORACLE_LIB=liboracle_san.so with gcc's libasan preloaded
    "liboracle_san.so": ["-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                         "-fno-omit-frame-pointer"],
}


def build(verbose: bool = False) -> None:
    for name, opt in OUTS.items():
        out = os.path.join(HERE, name)
        tmp = out + ".tmp"
        cmd = ["gcc", *opt, "-std=c11", "-fPIC", "-shared", "-fopenmp", "-fvisibility=hidden",
               "-Wall", "-Wextra", "-o", tmp, SRC, "-lm"]
        if verbose:
            print(" ".join(cmd), flush=True)
        subprocess.run(cmd, check=True)
        os.replace(tmp, out)


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
