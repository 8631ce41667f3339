"""Run by tests/test_gpu_device_checks.py in a process of its own, with
MIAIE_LIB_DIR pointing at the device-checked build (aiehlc_amd/lib_dbg).

1. Every kernel family runs on valid buffers with its results compared to
   the CPU oracle bit for bit (bf16 to the 1e-2 normwise bar) and miaie_wait
   reporting no access outside a known buffer.
2. Planted mistakes, in the buffer table only: a buffer is declared shorter
   than its real allocation (miaie_debug_register with the same address), so
   the kernel's accesses past the declared end stay inside memory the process
   owns.  The check must name them (MIAIE_EFAULT), and a store past the
   declared end must not have reached memory (the bytes there keep their
   sentinel).

Prints one JSON object: {"cases": [...], "planted": [...]} and exits 0 when
every check passed."""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import aiehlc_amd as mi  # noqa: E402
import oracle  # noqa: E402
from aiehlc_amd import synth  # noqa: E402


def say(*a):
    print("[step]", *a, file=sys.stderr, flush=True)


def main() -> int:
    assert os.path.abspath(mi.LIB_DIR).endswith("lib_dbg"), mi.LIB_DIR
    ctx = mi.Context(0)
    assert ctx.device_checks(), "the library at MIAIE_LIB_DIR is not the device-checked build"
    rng = np.random.default_rng(2024)
    cases, planted = [], []

    def i8(*shape):
        return rng.integers(-128, 128, size=shape, dtype=np.int8)

    # ---- 1. valid buffers, every kernel family
    gemm_shapes = [((512, 512, 256), mi.B_NN), ((512, 384, 192), mi.B_NT), ((256, 256, 128), mi.B_NN),
                   ((128, 128, 64), mi.B_NN), ((100, 50, 300), mi.B_NN), ((129, 77, 64), mi.B_NT)]
    for (M, N, K), lay in gemm_shapes:
        say("gemm_i8", M, N, K, lay)
        A, B = i8(M, K), (i8(N, K) if lay == mi.B_NT else i8(K, N))
        dA, dB, dY, dC = ctx.upload(A), ctx.upload(B), ctx.empty((M, N), np.int8), ctx.empty((M, N), np.int32)
        ctx.gemm_i8_rq(dA, dB, dY, M, N, K, 10, False, dC, lay)
        ctx.wait(120_000)
        Yo, Co = oracle.gemm_i8_rq(A, B, 10, b_nt=lay == mi.B_NT, want_acc=True)
        assert np.array_equal(ctx.download(dC), Co) and np.array_equal(ctx.download(dY), Yo), ("gemm_i8", M, N, K)
        ctx.gemm_i8_rq(dA, dB, dY, M, N, K, 11, True, None, lay)  # Y only
        ctx.wait(120_000)
        assert np.array_equal(ctx.download(dY), oracle.gemm_i8_rq(A, B, 11, True, b_nt=lay == mi.B_NT))
        for b in (dA, dB, dY, dC):
            b.free()
        cases.append(f"gemm_i8 {M}x{N}x{K} {'NT' if lay == mi.B_NT else 'NN'}")

    for M, N, K in [(512, 256, 128), (256, 256, 96), (300, 264, 128), (100, 130, 40), (70, 70, 64)]:
        say("gemm_bf16", M, N, K)
        A = synth.bf16_normal((M, K), 1, 1.0 / np.sqrt(K))
        B = synth.bf16_normal((K, N), 2, 1.0 / np.sqrt(K))
        dA, dB, dC = ctx.upload(A), ctx.upload(B), ctx.empty((M, N), np.float32)
        ctx.gemm_bf16_f32(dA, dB, dC, M, N, K)
        ctx.wait(120_000)
        R = oracle.gemm_bf16(A, B, f64=True)
        err = np.abs(ctx.download(dC).astype(np.float64) - R).max() / np.abs(R).max()
        assert err <= 1e-2, ("gemm_bf16", M, N, K, err)
        for b in (dA, dB, dC):
            b.free()
        cases.append(f"gemm_bf16 {M}x{N}x{K}")

    conv_shapes = [(1, 6, 56, 64, 64, 3, 3, 1, 1),     # row-block kernel
                   (1, 8, 8, 256, 64, 3, 3, 1, 1),      # chunked row-block kernel
                   (1, 16, 16, 256, 64, 3, 3, 2, 1),    # taps kernel, split K (workspace)
                   (1, 5, 9, 96, 64, 3, 3, 1, 1),       # implicit GEMM
                   (1, 5, 5, 4, 8, 3, 3, 1, 1)]         # direct
    for (N, H, W, Cin, Cout, R, S, st, pad) in conv_shapes:
        say("conv", N, H, W, Cin, Cout, R, S, st, pad)
        X, Wt = i8(N, H, W, Cin), i8(Cout, R, S, Cin)
        sh = rng.integers(8, 13, size=Cout, dtype=np.uint8)
        Ho, Wo = (H + 2 * pad - R) // st + 1, (W + 2 * pad - S) // st + 1
        dX, dW, dS, dY = ctx.upload(X), ctx.upload(Wt), ctx.upload(sh), ctx.empty((N, Ho, Wo, Cout), np.int8)
        ctx.conv2d_i8_nhwc(dX, dW, dS, dY, N, H, W, Cin, Cout, R, S, st, pad)
        ctx.wait(120_000)
        assert np.array_equal(ctx.download(dY), oracle.conv2d_nhwc_i8(X, Wt, sh, st, pad)), ("conv", Cin, Cout)
        for b in (dX, dW, dS, dY):
            b.free()
        cases.append(f"conv2d {mi.plan_conv2d_i8(N, H, W, Cin, Cout, R, S, st, pad)} {N}x{H}x{W}x{Cin}->{Cout}")

    say("mlp")
    M, K, F, Nout = 256, 128, 512, 256
    X, W1, W2 = i8(M, K), i8(K, F), i8(F, Nout)
    dX, d1, d2 = ctx.upload(X), ctx.upload(W1), ctx.upload(W2)
    dH, dY, dYn = ctx.empty((M, F), np.int8), ctx.empty((M, Nout), np.int8), ctx.empty((M, Nout), np.int8)
    ctx.mlp_i8(dX, d1, d2, dH, dY, M, K, F, Nout, 11, 12)
    ctx.mlp_i8_noalloc(dX, d1, d2, dYn, M, K, F, Nout, 11, 12)  # H in the scratch array
    ctx.wait(120_000)
    Yo = oracle.mlp_i8(X, W1, W2, 11, 12)
    assert np.array_equal(ctx.download(dY), Yo) and np.array_equal(ctx.download(dYn), Yo)
    for b in (dX, d1, d2, dH, dY, dYn):
        b.free()
    cases.append("mlp_i8 and mlp_i8_noalloc 256x128x512x256")

    say("reference kernels, copy, fill")
    win = np.arange(512, dtype=np.int32)
    dwin, dout = ctx.upload(win), ctx.empty((256,), np.int32)
    ctx.mm_window_i32(dwin, dout, 16)
    ctx.wait(60_000)
    assert np.array_equal(ctx.download(dout), oracle.mm_window_i32(win, 16))
    dsrc, ddst = ctx.empty((4099,), np.int8), ctx.empty((4099,), np.int8)
    ctx.fill_i8(dsrc, 4099, 5)
    ctx.copy_d2d(ddst, dsrc, 4099)
    ctx.wait(60_000)
    assert np.array_equal(ctx.download(ddst), synth.int8((4099,), 5))
    for b in (dwin, dout, dsrc, ddst):
        b.free()
    cases.append("mm_window_i32, fill_i8, copy_d2d")

    # ---- 2. planted: buffers declared shorter than their allocations
    def expect_fault(kind, source):
        rc = ctx.call_status("miaie_wait", 120_000)
        msg = ctx.last_error()
        assert rc == mi.MIAIE_EFAULT, (rc, msg)
        assert kind in msg and f"({source}, line " in msg, msg
        return msg

    say("planted: A declared half its rows (pipelined GEMM copies)")
    M = N = K = 512
    A, B = i8(M, K), i8(K, N)
    dA, dB, dY = ctx.upload(A), ctx.upload(B), ctx.empty((M, N), np.int8)
    ctx.debug_register(dA, (M // 2) * K)
    ctx.gemm_i8_rq(dA, dB, dY, M, N, K, 10, False, None, mi.B_NN)
    planted.append({"case": "A declared 256 of 512 rows, 512^3 int8 GEMM", "message": expect_fault("global->LDS copy", "gemm_i8_kernels.hpp")})
    ctx.debug_register(dA, M * K)  # the true extent again: clean
    ctx.gemm_i8_rq(dA, dB, dY, M, N, K, 10, False, None, mi.B_NN)
    ctx.wait(120_000)
    assert np.array_equal(ctx.download(dY), oracle.gemm_i8_rq(A, B, 10))

    say("planted: Y declared half its rows (stores dropped)")
    sentinel = np.full((M, N), 0x5A, dtype=np.int8)
    ctx.copy_h2d(dY, sentinel)
    ctx.debug_register(dY, (M // 2) * N)
    ctx.gemm_i8_rq(dA, dB, dY, M, N, K, 10, False, None, mi.B_NN)
    msg = expect_fault("store of 16 bytes", "gemm_i8_kernels.hpp")
    got = ctx.download(dY)
    assert np.array_equal(got[: M // 2], oracle.gemm_i8_rq(A, B, 10)[: M // 2])
    assert (got[M // 2:] == 0x5A).all(), "a store past the declared extent reached memory"
    planted.append({"case": "Y declared 256 of 512 rows: the rows past it keep their sentinel", "message": msg})
    ctx.debug_register(dY, M * N)
    for b in (dA, dB, dY):
        b.free()

    say("planted: conv X declared short (plain loads)")
    N_, H, W, Cin, Cout = 1, 6, 56, 64, 64
    X, Wt = i8(N_, H, W, Cin), i8(Cout, 3, 3, Cin)
    sh = np.full(Cout, 10, np.uint8)
    dX, dW, dS, dY = ctx.upload(X), ctx.upload(Wt), ctx.upload(sh), ctx.empty((N_, H, W, Cout), np.int8)
    ctx.debug_register(dX, X.nbytes // 2)
    ctx.conv2d_i8_nhwc(dX, dW, dS, dY, N_, H, W, Cin, Cout, 3, 3, 1, 1)
    planted.append({"case": "conv X declared half its rows", "message": expect_fault("load of 16 bytes", "conv2d_i8_rows.hpp")})
    ctx.debug_register(dX, X.nbytes)
    ctx.conv2d_i8_nhwc(dX, dW, dS, dY, N_, H, W, Cin, Cout, 3, 3, 1, 1)
    ctx.wait(120_000)
    assert np.array_equal(ctx.download(dY), oracle.conv2d_nhwc_i8(X, Wt, sh, 1, 1))
    for b in (dX, dW, dS, dY):
        b.free()

    # the table refuses overlapping declarations
    d = ctx.empty((4096,), np.int8)
    rc = ctx.call_status("miaie_debug_register", d.ptr + 16, mi._sz(64))
    assert rc == mi.MIAIE_EINVAL, rc
    d.free()
    ctx.close()
    print(json.dumps({"cases": cases, "planted": planted}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
