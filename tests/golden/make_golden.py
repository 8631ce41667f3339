"""Writes tests/golden/golden.npz: small input/output vectors for the hot path,
computed with numpy integer/float64 arithmetic only (independent of the C
oracle and of the GPU kernels).  Run from the repository root:

    python tests/golden/make_golden.py

Cases:
  mm16_i        the packed window of example/matrixmultiply/aieml_mm.cc:137-140
                (word i = i), golden C = A . B^T with B stored [N][K] (:194-230)
  mm16_ip1      example/perf/aieml_perf.cc:141-144 (word i = i + 1)
  mm8_i         example/other/aieoob.c:83-86 (n = 8)
  gemm64        benchmark config 1: 64x64x64 int8 NN from the SplitMix64 streams
                (A id 1, B id 2) -> int32 C and Y = requant(C, 10)
  gemm_ragged   37x50x70 int8 NN (numpy default_rng(20261201)) -> C, Y (shift 9, ReLU)
  conv          N=1 H=W=6 Cin=32 Cout=64 3x3 stride 1 pad 1 (default_rng) -> Y
  mlp           X 8x64, W1 64x96, W2 96x32 (default_rng) -> H, Y (shifts 11, 12)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from aiehlc_amd import synth  # noqa: E402  (numpy SplitMix64 generator)


def rq(acc, s, relu=False):
    acc = np.asarray(acc, dtype=np.int64)
    q = np.floor_divide(acc + (2 ** (s - 1) if s else 0), 2 ** s)
    return np.clip(q, 0 if relu else -128, 127).astype(np.int8)


def window_case(n, base):
    win = (np.arange(2 * n * n, dtype=np.int64) + base)
    A = win[: n * n].reshape(n, n)
    Bnk = win[n * n:].reshape(n, n)
    C = (A @ Bnk.T).astype(np.int64)
    return win.astype(np.int32), ((C + 2**31) % 2**32 - 2**31).astype(np.int32)


def main():
    out = {}
    for name, n, base in (("mm16_i", 16, 0), ("mm16_ip1", 16, 1), ("mm8_i", 8, 0)):
        win, C = window_case(n, base)
        out[f"{name}_in"], out[f"{name}_out"] = win, C.reshape(-1)

    A = synth.int8((64, 64), 1)
    B = synth.int8((64, 64), 2)
    C = A.astype(np.int64) @ B.astype(np.int64)
    out["gemm64_A"], out["gemm64_B"] = A, B
    out["gemm64_C"], out["gemm64_Y10"] = C.astype(np.int32), rq(C, 10)

    rng = np.random.default_rng(20261201)
    A = rng.integers(-128, 128, size=(37, 70), dtype=np.int8)
    B = rng.integers(-128, 128, size=(70, 50), dtype=np.int8)
    C = A.astype(np.int64) @ B.astype(np.int64)
    out["ragged_A"], out["ragged_B"] = A, B
    out["ragged_C"], out["ragged_Y9r"] = C.astype(np.int32), rq(C, 9, relu=True)

    X = rng.integers(-128, 128, size=(1, 6, 6, 32), dtype=np.int8)
    W = rng.integers(-128, 128, size=(64, 3, 3, 32), dtype=np.int8)
    sh = rng.integers(8, 13, size=64).astype(np.uint8)
    Xp = np.zeros((1, 8, 8, 32), dtype=np.int64)
    Xp[:, 1:7, 1:7] = X
    acc = np.zeros((1, 6, 6, 64), dtype=np.int64)
    for r in range(3):
        for s in range(3):
            acc += np.einsum("nhwc,oc->nhwo", Xp[:, r:r + 6, s:s + 6], W[:, r, s].astype(np.int64))
    q = np.floor_divide(acc + (1 << (sh.astype(np.int64) - 1)), 1 << sh.astype(np.int64))
    out["conv_X"], out["conv_W"], out["conv_shifts"] = X, W, sh
    out["conv_Y"] = np.clip(q, -128, 127).astype(np.int8)

    X = rng.integers(-128, 128, size=(8, 64), dtype=np.int8)
    W1 = rng.integers(-128, 128, size=(64, 96), dtype=np.int8)
    W2 = rng.integers(-128, 128, size=(96, 32), dtype=np.int8)
    H = rq(X.astype(np.int64) @ W1.astype(np.int64), 11, relu=True)
    Y = rq(H.astype(np.int64) @ W2.astype(np.int64), 12)
    out["mlp_X"], out["mlp_W1"], out["mlp_W2"], out["mlp_H"], out["mlp_Y"] = X, W1, W2, H, Y

    np.savez_compressed(os.path.join(HERE, "golden.npz"), **out)
    print("wrote", os.path.join(HERE, "golden.npz"), len(out), "arrays")


if __name__ == "__main__":
    main()
