"""GPU parity of the int8 GEMM (+requant), bf16 GEMM, int8 conv2d and the
chained int8 MLP, through the miaie C ABI, against the CPU oracle.

Integer paths are compared bit-exactly.  bf16 uses the normwise metric
max|C - R| / max|R| <= 1e-2 against the fp64 oracle on the same bf16 inputs.
The integer benchmark shapes (configs 1, 2, 4 and 5) are compared with the
oracle over every element; bf16 8192^3 on one row of every 16-row block (every
workgroup's output) plus checks that hold over the whole output.
"""
import numpy as np
import pytest

import aiehlc_amd as mi
import oracle
from aiehlc_amd import synth

pytestmark = pytest.mark.gpu

BF16_TOL = 1e-2


def _say(*a):
    print("[case]", *a, flush=True)


def _run_gemm_i8(ctx, A, B, b_layout, shift=None, relu=False, want_c=True):
    M, K = A.shape
    N = B.shape[0] if b_layout == mi.B_NT else B.shape[1]
    dA, dB = ctx.upload(A), ctx.upload(B)
    dC = ctx.empty((M, N), np.int32) if want_c else None
    if shift is None:
        ctx.gemm_i8_i32(dA, dB, dC, M, N, K, b_layout=b_layout)
        ctx.wait(60_000)
        out = (None, ctx.download(dC))
    else:
        dY = ctx.empty((M, N), np.int8)
        ctx.gemm_i8_rq(dA, dB, dY, M, N, K, shift, relu, dC, b_layout)
        ctx.wait(60_000)
        out = (ctx.download(dY), ctx.download(dC) if want_c else None)
    for b in (dA, dB, dC):
        if b is not None:
            b.free()
    return out


SMALL = [(1, 1, 1), (16, 16, 16), (64, 64, 64), (17, 33, 65), (100, 50, 300), (128, 96, 7), (3, 200, 129)]
BIG = [(256, 256, 64), (512, 768, 256), (768, 512, 128)]


@pytest.mark.parametrize("shape", SMALL + BIG)
@pytest.mark.parametrize("layout", [mi.B_NN, mi.B_NT])
def test_gemm_i8_i32(ctx, shape, layout):
    M, N, K = shape
    _say("gemm_i8_i32", shape, layout)
    rng = np.random.default_rng(M * 131 + N * 7 + K)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    B = rng.integers(-128, 128, size=(N, K) if layout == mi.B_NT else (K, N), dtype=np.int8)
    _, Cg = _run_gemm_i8(ctx, A, B, layout)
    assert np.array_equal(Cg, oracle.gemm_i8(A, B, b_nt=layout == mi.B_NT))


def test_gemm_i8_single_tile_config(ctx):
    """Config 1: 64x64 int8 NN from seed (A id 1, B id 2) -> int32."""
    _say("gemm 64^3 seeded")
    A = synth.int8((64, 64), 1)
    B = synth.int8((64, 64), 2)
    _, Cg = _run_gemm_i8(ctx, A, B, mi.B_NN)
    assert np.array_equal(Cg, oracle.gemm_i8(A, B))


@pytest.mark.parametrize("shape,layout", [((512, 384, 128), mi.B_NN), ((512, 384, 192), mi.B_NT),
                                          ((4096, 4096, 128), mi.B_NN), ((4096, 4096, 128), mi.B_NT),
                                          ((2048, 1024, 256), mi.B_NN)])
def test_gemm_i8_pipeline_tile_widths(ctx, shape, layout):
    """Shapes that select the 128-wide (N % 256 != 0, or a grid under one round
    of CUs) and the 256-wide (4096^2 grid) pipelined tiles, both B layouts."""
    M, N, K = shape
    _say("gemm_i8 pipeline widths", shape, layout)
    rng = np.random.default_rng(M + N + K + layout)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    B = rng.integers(-128, 128, size=(N, K) if layout == mi.B_NT else (K, N), dtype=np.int8)
    Yg, Cg = _run_gemm_i8(ctx, A, B, layout, 9, False)
    Yo, Co = oracle.gemm_i8_rq(A, B, 9, b_nt=layout == mi.B_NT, want_acc=True)
    assert np.array_equal(Cg, Co)
    assert np.array_equal(Yg, Yo)


@pytest.mark.parametrize("shape", [(64, 64, 64), (100, 50, 300), (256, 256, 64), (512, 512, 512)])
@pytest.mark.parametrize("shift,relu", [(10, False), (11, True), (0, False), (1, False), (31, False), (7, True)])
def test_gemm_i8_rq(ctx, shape, shift, relu):
    M, N, K = shape
    _say("gemm_i8_rq", shape, shift, relu)
    rng = np.random.default_rng(shift * 1000 + M)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    Yg, Cg = _run_gemm_i8(ctx, A, B, mi.B_NN, shift, relu)
    Yo, Co = oracle.gemm_i8_rq(A, B, shift, relu, want_acc=True)
    assert np.array_equal(Cg, Co)
    assert np.array_equal(Yg, Yo)


def test_gemm_i8_rq_without_debug_output(ctx):
    _say("gemm_i8_rq no C_dbg")
    rng = np.random.default_rng(3)
    A = rng.integers(-128, 128, size=(512, 256), dtype=np.int8)
    B = rng.integers(-128, 128, size=(256, 256), dtype=np.int8)
    Yg, _ = _run_gemm_i8(ctx, A, B, mi.B_NN, 10, False, want_c=False)
    assert np.array_equal(Yg, oracle.gemm_i8_rq(A, B, 10))


def _mismatches(got, want):
    """The reference's check: count differing elements over the whole output
    (example/matrixmultiply/aieml_mm.cc:232-245)."""
    assert got.shape == want.shape, (got.shape, want.shape)
    return int(np.count_nonzero(got != want))


def test_gemm_i8_rq_4096_config(ctx):
    """Config 2: M=N=K=4096 NN, shift 10, compared with the oracle over every
    element.  First the benchmarked launch itself (Y only, C_dbg = NULL: the
    kernel bench.py times), then the launch that also writes the int32
    accumulators, whose C and Y are compared in full as well."""
    M = N = K = 4096
    _say("gemm_i8_rq 4096^3")
    A = synth.int8((M, K), 1)
    B = synth.int8((K, N), 2)
    Yo, Co = oracle.gemm_i8_rq(A, B, 10, want_acc=True)
    Yb, _ = _run_gemm_i8(ctx, A, B, mi.B_NN, 10, False, want_c=False)
    assert _mismatches(Yb, Yo) == 0
    del Yb
    Yg, Cg = _run_gemm_i8(ctx, A, B, mi.B_NN, 10, False)
    assert _mismatches(Cg, Co) == 0
    assert _mismatches(Yg, Yo) == 0


@pytest.mark.parametrize("shape", [(1, 1, 1), (64, 64, 64), (37, 70, 45), (256, 256, 32), (512, 256, 512),
                                   (300, 1000, 256), (129, 77, 64), (1000, 40, 96),  # prefetching 64x64
                                   (100, 130, 40), (33, 65, 8), (70, 70, 1000)])     # ... with K % 32 != 0
def test_gemm_bf16(ctx, shape):
    M, N, K = shape
    _say("gemm_bf16", shape)
    A = synth.bf16_normal((M, K), 1, 1.0 / np.sqrt(K))
    B = synth.bf16_normal((K, N), 2, 1.0 / np.sqrt(K))
    dA, dB, dC = ctx.upload(A), ctx.upload(B), ctx.empty((M, N), np.float32)
    ctx.gemm_bf16_f32(dA, dB, dC, M, N, K)
    ctx.wait(60_000)
    Cg = ctx.download(dC).astype(np.float64)
    R = oracle.gemm_bf16(A, B, f64=True)
    err = np.abs(Cg - R).max() / max(np.abs(R).max(), 1e-30)
    assert err <= BF16_TOL, err
    # fp32 accumulation of exact bf16 products: far tighter than the bar
    assert err <= 1e-5, err


# M and N that 256 does not divide, on the 256x256 bf16 kernels: the last
# tile row and column are moved back over their neighbours.  The launcher
# takes them there when the tiles fill at least half the CUs, so the small
# shapes plan for one CU; (4000, 2056, 128) fills the device as it is.
@pytest.mark.parametrize("shape,cus", [((300, 264, 128), 1), ((300, 264, 96), 1), ((513, 520, 64), 1),
                                       ((256, 1000, 192), 1), ((4000, 2056, 128), 0)])
def test_gemm_bf16_ragged_256(ctx, shape, cus):
    M, N, K = shape
    _say("gemm_bf16 ragged 256x256", shape, "cus", cus)
    A = synth.bf16_normal((M, K), 3, 1.0 / np.sqrt(K))
    B = synth.bf16_normal((K, N), 4, 1.0 / np.sqrt(K))
    prev = ctx.plan_set_cus(cus) if cus else None
    try:
        dA, dB, dC = ctx.upload(A), ctx.upload(B), ctx.empty((M, N), np.float32)
        ctx.gemm_bf16_f32(dA, dB, dC, M, N, K)
        ctx.wait(60_000)
        Cg = ctx.download(dC).astype(np.float64)
        for b in (dA, dB, dC):
            b.free()
    finally:
        if cus:
            ctx.plan_set_cus(prev)
    R = oracle.gemm_bf16(A, B, f64=True)
    err = np.abs(Cg - R).max() / np.abs(R).max()
    assert err <= BF16_TOL, err
    assert err <= 1e-5, err


def _random_bf16_cases(n=12, seed=7):
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        M = int(rng.choice([int(rng.integers(1, 300)), int(rng.integers(256, 900))]))
        N = int(rng.choice([int(rng.integers(1, 300)), 8 * int(rng.integers(32, 110))]))
        K = int(rng.choice([32 * int(rng.integers(1, 20)), int(rng.integers(1, 400))]))
        cases.append((M, N, K, int(rng.choice([0, 1]))))
    return cases


@pytest.mark.parametrize("M,N,K,one_cu", _random_bf16_cases())
def test_gemm_bf16_random_shapes(ctx, M, N, K, one_cu):
    """Seeded random shapes; planned for one CU half the time, so that
    ragged shapes take the 256x256 kernels with overlapping last tiles."""
    _say("gemm_bf16 random", (M, N, K), "one CU" if one_cu else "")
    A = synth.bf16_normal((M, K), 8, 1.0 / np.sqrt(K))
    B = synth.bf16_normal((K, N), 9, 1.0 / np.sqrt(K))
    prev = ctx.plan_set_cus(1) if one_cu else None
    try:
        dA, dB, dC = ctx.upload(A), ctx.upload(B), ctx.empty((M, N), np.float32)
        ctx.gemm_bf16_f32(dA, dB, dC, M, N, K)
        ctx.wait(60_000)
        Cg = ctx.download(dC).astype(np.float64)
        for b in (dA, dB, dC):
            b.free()
    finally:
        if one_cu:
            ctx.plan_set_cus(prev)
    R = oracle.gemm_bf16(A, B, f64=True)
    err = np.abs(Cg - R).max() / max(np.abs(R).max(), 1e-30)
    assert err <= BF16_TOL, err
    assert err <= 1e-5, err


# K sweep over the 256x256 bf16 kernels: K % 64 == 0 takes the pair-staged
# kernel (A staged two k-tiles at a time; its waits change over the last six
# k-tiles and in the prologue below six), odd multiples of 32 the per-k-tile
# kernel.
@pytest.mark.parametrize("K", [32, 64, 96, 128, 192, 256, 320, 384, 448, 512, 576, 1088, 2112])
def test_gemm_bf16_k_sweep(ctx, K):
    M, N = 512, 256
    _say("gemm_bf16 k-sweep", (M, N, K))
    A = synth.bf16_normal((M, K), 5, 1.0 / np.sqrt(K))
    B = synth.bf16_normal((K, N), 6, 1.0 / np.sqrt(K))
    dA, dB, dC = ctx.upload(A), ctx.upload(B), ctx.empty((M, N), np.float32)
    ctx.gemm_bf16_f32(dA, dB, dC, M, N, K)
    ctx.wait(60_000)
    Cg = ctx.download(dC).astype(np.float64)
    for b in (dA, dB, dC):
        b.free()
    R = oracle.gemm_bf16(A, B, f64=True)
    err = np.abs(Cg - R).max() / np.abs(R).max()
    assert err <= BF16_TOL, err
    assert err <= 1e-5, err


def test_gemm_bf16_8192_config(ctx):
    """Config 3: 8192^3 bf16, N(0,1)/sqrt(K).

    The output buffer is filled with NaN before the launch, so an element the
    kernel never writes fails the finiteness check over the whole output.

    Against the fp64 oracle on 512 rows, one from every 16-row block (row
    16b + b mod 16): every 256-row tile row, every wave's half of it and
    every 16-row MFMA block of a wave is compared on all 8192 columns, so
    every one of the 1024 workgroups' output is checked.  Reported: the
    normwise error (the bar, max|C-R| / max|R| <= 1e-2), the elementwise
    relative error where |R| >= 1e-3 max|R|, and the Frobenius relative
    error (also held to 1e-2).

    Over the whole output: C(2A) == 2 C(A) bit for bit (doubling a bf16
    operand is exact and the accumulation order does not depend on the
    data)."""
    M = N = K = 8192
    _say("gemm_bf16 8192^3")
    A = synth.bf16_normal((M, K), 1, 1.0 / np.sqrt(K))
    B = synth.bf16_normal((K, N), 2, 1.0 / np.sqrt(K))
    A2 = synth.f32_to_bf16_bits(2.0 * synth.bf16_bits_to_f32(A))
    assert np.array_equal(synth.bf16_bits_to_f32(A2), 2.0 * synth.bf16_bits_to_f32(A))
    nan_fill = np.full((M, N), np.nan, dtype=np.float32)
    dA, dB, dC = ctx.upload(A), ctx.upload(B), ctx.upload(nan_fill)
    ctx.gemm_bf16_f32(dA, dB, dC, M, N, K)
    ctx.wait(120_000)
    Cg = ctx.download(dC)
    ctx.copy_h2d(dC, nan_fill)
    del nan_fill
    ctx.copy_h2d(dA, A2)
    ctx.gemm_bf16_f32(dA, dB, dC, M, N, K)
    ctx.wait(120_000)
    C2 = ctx.download(dC)
    for b in (dA, dB, dC):
        b.free()
    assert np.isfinite(Cg).all()
    assert np.array_equal(C2, 2.0 * Cg)
    del C2
    blocks = np.arange(M // 16)
    rows = 16 * blocks + blocks % 16
    assert np.array_equal(np.unique(rows // 16), blocks)
    R = oracle.gemm_bf16(A[rows], B, f64=True)
    D = Cg[rows].astype(np.float64) - R
    err = np.abs(D).max() / np.abs(R).max()
    big = np.abs(R) >= 1e-3 * np.abs(R).max()
    elem = (np.abs(D)[big] / np.abs(R)[big]).max()
    frob = np.linalg.norm(D) / np.linalg.norm(R)
    print(f"[bf16 8192^3] normwise {err:.3e} elementwise(|R|>=1e-3 max) {elem:.3e} frobenius {frob:.3e}", flush=True)
    assert err <= BF16_TOL, err
    assert frob <= BF16_TOL, frob


CONV_SHAPES = [
    # N, H, W, Cin, Cout, R, S, stride, pad
    (1, 5, 5, 32, 64, 3, 3, 1, 1),
    (2, 7, 9, 64, 64, 3, 3, 1, 1),
    (1, 8, 8, 64, 128, 3, 3, 2, 1),
    (1, 6, 6, 96, 64, 1, 1, 1, 0),
    (1, 9, 9, 32, 64, 5, 5, 1, 2),
    (1, 7, 64, 64, 128, 3, 3, 1, 1),  # odd Ho, Wo = 64, two Cout blocks
    (3, 5, 33, 32, 64, 3, 3, 1, 0),   # no padding
    (2, 56, 56, 64, 64, 3, 3, 1, 1),  # config shape, fewer images (row-block 4 rows x 32 channels)
    (1, 5, 48, 64, 64, 3, 3, 1, 1),   # row-pair (2 x 64, Ho < 8): odd Ho (last workgroup half outside the image)
    (2, 6, 50, 64, 128, 3, 3, 1, 0),  # row-pair, no padding, two Cout blocks
    (1, 9, 60, 64, 64, 3, 3, 1, 2),   # row-block 4 x 32, pad 2 (two zero columns each side), Ho 11: last block 3 rows
    (1, 4, 64, 64, 64, 3, 3, 1, 0),   # row-pair, widest row, no padding
    (1, 7, 56, 64, 32, 3, 3, 1, 1),   # row-block 4 rows x 32 channels (Cout 32), last block half outside
    (2, 5, 30, 32, 96, 3, 3, 1, 1),   # row-block 4 x 32, three channel blocks, Cin 32
    (2, 7, 28, 128, 128, 3, 3, 1, 1),  # row-block 2 x 64 at Cin 128 (116 KiB of LDS), Ho < 8 and odd
    (1, 6, 60, 128, 96, 3, 3, 1, 2),  # row-block 4 x 32 at Cin 128, pad 2
    (1, 10, 64, 128, 128, 3, 3, 1, 1),  # row-block 4 x 32 at Cin 128, four channel blocks, last block half outside
    (2, 11, 40, 32, 64, 3, 3, 1, 1),  # row-block 4 x 32 at Cin 32, Cout 64, last block 3 rows
    (1, 8, 30, 64, 128, 3, 3, 1, 1),  # Ho = 8, the first height on 4 x 32 at Cout % 64 == 0: two whole row blocks
    (3, 8, 66, 32, 64, 3, 3, 1, 1),   # 4 x 32, Wo 66: two column blocks (the second 2 columns wide), N % 8 != 0 grid
    (1, 5, 9, 96, 64, 3, 3, 1, 1),    # Cin 96: implicit-GEMM kernel
    (1, 8, 8, 256, 64, 3, 3, 1, 1),   # chunked row-block kernel: four 64-channel chunks, one workgroup
    (1, 16, 16, 256, 64, 3, 3, 2, 1),  # taps kernel (LDS-staged), stride 2: one tile split 4 ways over k (partials + reduce)
    (2, 7, 7, 512, 128, 3, 3, 1, 1),  # taps: 4 tiles split 8 ways, the last pixel block partial
    (1, 6, 6, 320, 64, 3, 3, 2, 1),   # Cin 320: implicit GEMM, stride 2, split over k
    (1, 5, 70, 128, 64, 3, 3, 1, 1),  # row-block kernel at Cin 128, rows wider than 64: two column blocks
    (1, 5, 70, 128, 64, 5, 5, 1, 2),  # taps, 5x5: pixel tiles across rows (left and right padding)
    (1, 9, 9, 128, 128, 3, 3, 2, 1),  # taps, stride 2
    (8, 14, 14, 256, 256, 3, 3, 1, 1),  # deep CNN layer on the chunked row-block kernel (32 x 32 waves, 256 workgroups)
    (8, 7, 7, 512, 512, 3, 3, 1, 1),    # deepest, on taps: 56 tiles, split 4 ways
    (2, 6, 70, 192, 96, 3, 3, 1, 1),  # chunked row-block: 3 chunks (odd), Cout 96 (4 rows x 32), two column blocks
    (32, 14, 14, 128, 128, 3, 3, 1, 1),  # Cin 128 on the chunked row-block kernel (narrow layer, several rounds)
    (1, 5, 5, 4, 8, 3, 3, 1, 1),      # fallback kernel (channels not multiples of 32/64)
    (2, 6, 7, 3, 5, 3, 3, 2, 0),      # fallback kernel
]


@pytest.mark.parametrize("shape", CONV_SHAPES)
def test_conv2d_i8(ctx, shape):
    N, H, W, Cin, Cout, R, S, stride, pad = shape
    _say("conv2d", shape)
    rng = np.random.default_rng(sum(shape))
    X = rng.integers(-128, 128, size=(N, H, W, Cin), dtype=np.int8)
    Wt = rng.integers(-128, 128, size=(Cout, R, S, Cin), dtype=np.int8)
    sh = rng.integers(8, 13, size=Cout, dtype=np.uint8)
    Ho = (H + 2 * pad - R) // stride + 1
    Wo = (W + 2 * pad - S) // stride + 1
    dX, dW, dS = ctx.upload(X), ctx.upload(Wt), ctx.upload(sh)
    dY = ctx.empty((N, Ho, Wo, Cout), np.int8)
    ctx.conv2d_i8_nhwc(dX, dW, dS, dY, N, H, W, Cin, Cout, R, S, stride, pad)
    ctx.wait(60_000)
    Yg = ctx.download(dY)
    assert np.array_equal(Yg, oracle.conv2d_nhwc_i8(X, Wt, sh, stride, pad))


def _random_conv_cases(n=16, seed=1202):
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        Cin = int(rng.choice([3, 32, 64, 96, 128, 192, 256, 320, 384]))
        Cout = int(rng.choice([8, 32, 64, 96, 128, 192, 256]))
        R = int(rng.choice([1, 3, 3, 3, 5]))
        stride = int(rng.choice([1, 1, 2]))
        pad = int(rng.integers(0, R // 2 + 1))
        H = int(rng.integers(R, 20))
        W = int(rng.integers(R, 80))
        N = int(rng.integers(1, 4))
        cases.append((N, H, W, Cin, Cout, R, R, stride, pad))
    return cases


@pytest.mark.parametrize("shape", _random_conv_cases())
def test_conv2d_i8_random_shapes(ctx, shape):
    """Seeded random shapes over the conv kernels (whichever the planner
    picks), shifts over [0, 31], bit-exact against the oracle."""
    N, H, W, Cin, Cout, R, S, stride, pad = shape
    _say("conv2d random", shape, mi.plan_conv2d_i8(N, H, W, Cin, Cout, R, S, stride, pad))
    rng = np.random.default_rng(sum(shape) * 13)
    X = rng.integers(-128, 128, size=(N, H, W, Cin), dtype=np.int8)
    Wt = rng.integers(-128, 128, size=(Cout, R, S, Cin), dtype=np.int8)
    sh = rng.integers(0, 32, size=Cout, dtype=np.uint8)
    Ho = (H + 2 * pad - R) // stride + 1
    Wo = (W + 2 * pad - S) // stride + 1
    dX, dW, dS = ctx.upload(X), ctx.upload(Wt), ctx.upload(sh)
    dY = ctx.empty((N, Ho, Wo, Cout), np.int8)
    ctx.conv2d_i8_nhwc(dX, dW, dS, dY, N, H, W, Cin, Cout, R, S, stride, pad)
    ctx.wait(60_000)
    assert np.array_equal(ctx.download(dY), oracle.conv2d_nhwc_i8(X, Wt, sh, stride, pad))


def _random_rows_cases(n=48, seed=20261202):
    """3x3 stride-1 layers for the row-block kernels: Cin 32/64/128, Cout a
    multiple of 32 (both workgroup shapes), heights across the 4-row block
    boundary, widths over one to three 64-column blocks, batch sizes on both
    grid forms, pads 0-2, planned for 1 to 256 CUs."""
    rng = np.random.default_rng(seed)
    cases = []
    while len(cases) < n:
        Cin = int(rng.choice([32, 64, 128]))
        Cout = int(rng.choice([32, 64, 96, 128, 160, 256]))
        H, W = int(rng.integers(3, 22)), int(rng.integers(3, 150))
        N, pad = int(rng.choice([1, 2, 3, 8, 9, 16])), int(rng.integers(0, 3))
        if N * H * W * Cout * Cin > 6e8:
            N = 1
        cases.append(((N, H, W, Cin, Cout, 3, 3, 1, pad), int(rng.choice([256, 256, 64, 8, 1]))))
    return cases


@pytest.mark.parametrize("shape,cus", _random_rows_cases())
def test_conv2d_i8_rows_random(ctx, shape, cus):
    """Seeded random layers on the row-block kernels (4 x 32 and 2 x 64
    workgroups, and the chunked kernel where a CU count makes it the
    choice), per-channel shifts over [0, 31], bit-exact against the oracle."""
    N, H, W, Cin, Cout, R, S, stride, pad = shape
    _say("conv2d rows random", shape, "cus", cus)
    rng = np.random.default_rng(sum(shape) * 31 + cus)
    X = rng.integers(-128, 128, size=(N, H, W, Cin), dtype=np.int8)
    Wt = rng.integers(-128, 128, size=(Cout, R, S, Cin), dtype=np.int8)
    sh = rng.integers(0, 32, size=Cout, dtype=np.uint8)
    Ho, Wo = H + 2 * pad - 2, W + 2 * pad - 2
    prev = ctx.plan_set_cus(cus)
    try:
        dX, dW, dS = ctx.upload(X), ctx.upload(Wt), ctx.upload(sh)
        dY = ctx.empty((N, Ho, Wo, Cout), np.int8)
        ctx.conv2d_i8_nhwc(dX, dW, dS, dY, N, H, W, Cin, Cout, R, S, stride, pad)
        ctx.wait(60_000)
        Yg = ctx.download(dY)
    finally:
        ctx.plan_set_cus(prev)
    assert np.array_equal(Yg, oracle.conv2d_nhwc_i8(X, Wt, sh, stride, pad))


@pytest.mark.parametrize("shape", [
    (1, 9, 70, 256, 128, 3, 3, 2, 1),   # stride 2: 2 pixel tiles, the last partial
    (2, 7, 7, 256, 256, 5, 5, 1, 2),    # 5x5: one partial pixel tile, two channel tiles
    (1, 17, 17, 128, 256, 3, 3, 2, 1),  # stride 2
    (1, 6, 6, 384, 128, 3, 3, 1, 0),    # no padding, three 128-channel chunks per tap
])
def test_conv2d_i8_taps_128_tiles(ctx, shape):
    """The taps kernel's 128 x 128 workgroup tile, which the launcher takes
    when those tiles fill a round of CUs: planned here for one CU so that
    small shapes take it.  Bit-exact against the oracle."""
    N, H, W, Cin, Cout, R, S, stride, pad = shape
    _say("conv2d taps 128x128", shape)
    assert mi.plan_conv2d_i8(N, H, W, Cin, Cout, R, S, stride, pad) == "taps"
    rng = np.random.default_rng(sum(shape) + 7)
    X = rng.integers(-128, 128, size=(N, H, W, Cin), dtype=np.int8)
    Wt = rng.integers(-128, 128, size=(Cout, R, S, Cin), dtype=np.int8)
    sh = rng.integers(8, 13, size=Cout, dtype=np.uint8)
    Ho = (H + 2 * pad - R) // stride + 1
    Wo = (W + 2 * pad - S) // stride + 1
    prev = ctx.plan_set_cus(1)
    try:
        dX, dW, dS = ctx.upload(X), ctx.upload(Wt), ctx.upload(sh)
        dY = ctx.empty((N, Ho, Wo, Cout), np.int8)
        ctx.conv2d_i8_nhwc(dX, dW, dS, dY, N, H, W, Cin, Cout, R, S, stride, pad)
        ctx.wait(60_000)
        Yg = ctx.download(dY)
    finally:
        ctx.plan_set_cus(prev)
    assert np.array_equal(Yg, oracle.conv2d_nhwc_i8(X, Wt, sh, stride, pad))


@pytest.mark.parametrize("shape,cus", [
    ((1, 8, 8, 256, 128, 3, 3, 1, 1), 256),   # 32 x 32 waves (more workgroups), 64-column blocks
    ((1, 8, 8, 192, 128, 3, 3, 1, 1), 1),     # 32 x 64 waves (two MFMAs per pixel fragment), 32-column blocks
    #                                           (Cin 192: at 1 CU the taps kernel would be estimated faster for Cin 256)
    ((2, 6, 70, 192, 128, 3, 3, 1, 0), 1),    # 3 chunks, two 64-column blocks, no padding, 32 x 64 waves
    ((16, 5, 9, 320, 128, 3, 3, 1, 1), 1),    # 5 chunks, image-per-XCD grid over 16 images, 32 x 64 waves
    ((2, 9, 20, 192, 128, 3, 3, 1, 1), 1),    # 8 rows x 32 columns, 32 x 64 waves, last row block partial
    ((1, 9, 20, 256, 96, 3, 3, 1, 1), 1),     # 8 rows x 32 columns, 32 x 32 waves (Cout 96)
    ((1, 2, 10, 256, 64, 3, 3, 1, 1), 256),   # fewer output rows than a row block
    ((1, 3, 3, 4032, 64, 3, 3, 1, 1), 256),   # 63 chunks: Cin near the 4096 bound of the rounding term
])
@pytest.mark.parametrize("extreme", [False, True])
def test_conv2d_i8_rows_deep(ctx, shape, cus, extreme):
    """The chunked row-block kernel (Cin a multiple of 64 above 128, 3x3,
    stride 1): both wave tiles, odd and even chunk counts, column blocks, both
    grid forms, shifts over [0, 31].  `extreme` fills X and W with -128, the
    largest |acc| (9 * Cin * 2^14) on top of the rounding term."""
    N, H, W, Cin, Cout, R, S, stride, pad = shape
    _say("conv2d rows_deep", shape, cus, extreme)
    assert mi.plan_conv2d_i8(N, H, W, Cin, Cout, R, S, stride, pad) == "rows_deep"
    rng = np.random.default_rng(sum(shape) + cus + extreme)
    if extreme:
        X = np.full((N, H, W, Cin), -128, np.int8)
        Wt = np.full((Cout, R, S, Cin), -128, np.int8)
    else:
        X = rng.integers(-128, 128, size=(N, H, W, Cin), dtype=np.int8)
        Wt = rng.integers(-128, 128, size=(Cout, R, S, Cin), dtype=np.int8)
    sh = rng.integers(0, 32, size=Cout, dtype=np.uint8)
    sh[:3] = [0, 31, 7]
    Ho = (H + 2 * pad - R) // stride + 1
    Wo = (W + 2 * pad - S) // stride + 1
    prev = ctx.plan_set_cus(cus)
    try:
        dX, dW, dS = ctx.upload(X), ctx.upload(Wt), ctx.upload(sh)
        dY = ctx.empty((N, Ho, Wo, Cout), np.int8)
        ctx.conv2d_i8_nhwc(dX, dW, dS, dY, N, H, W, Cin, Cout, R, S, stride, pad)
        ctx.wait(60_000)
        Yg = ctx.download(dY)
    finally:
        ctx.plan_set_cus(prev)
    assert np.array_equal(Yg, oracle.conv2d_nhwc_i8(X, Wt, sh, stride, pad))


@pytest.mark.parametrize("shape", [
    (1, 6, 56, 64, 64, 3, 3, 1, 1),   # row-block 2 rows x 64 channels (Ho < 8)
    (1, 9, 56, 64, 64, 3, 3, 1, 1),   # row-block 4 rows x 32 channels, two channel blocks (config 4's workgroup)
    (1, 5, 20, 32, 96, 3, 3, 1, 1),   # row-block 4 rows x 32 channels, three channel blocks
    (1, 4, 24, 128, 64, 3, 3, 1, 1),  # row-block at Cin 128
    (1, 8, 8, 64, 64, 3, 3, 2, 1),    # implicit-GEMM kernel
    (1, 16, 16, 256, 64, 3, 3, 2, 1),  # taps kernel split over k (requantize in the reduce kernel)
    (1, 56, 100, 128, 64, 1, 1, 1, 0),  # taps kernel, not split: requantize in its own epilogue
    (1, 4, 20, 192, 96, 3, 3, 1, 1),  # chunked row-block kernel
    (1, 5, 5, 4, 8, 3, 3, 1, 1),      # direct kernel
])
@pytest.mark.parametrize("small", [False, True])
def test_conv2d_i8_shift_range(ctx, shape, small):
    """Per-channel shifts over the whole documented range [0, 31], mixed
    within each 32-channel block (so waves take the general epilogue), then
    with every shift >= 8 but one channel at 7, and with every shift >= 8
    (the high-byte epilogue).  `small` draws X in [-3, 3] so that small
    shifts land inside the int8 range instead of saturating."""
    N, H, W, Cin, Cout, R, S, stride, pad = shape
    _say("conv2d shift range", shape, small)
    rng = np.random.default_rng(7 + Cout + small)
    lo, hi = (-3, 4) if small else (-128, 128)
    X = rng.integers(lo, hi, size=(N, H, W, Cin), dtype=np.int8)
    Wt = rng.integers(-128, 128, size=(Cout, R, S, Cin), dtype=np.int8)
    Ho = (H + 2 * pad - R) // stride + 1
    Wo = (W + 2 * pad - S) // stride + 1
    full = rng.integers(0, 32, size=Cout, dtype=np.uint8)
    full[:4] = [0, 31, 7, 8]
    one7 = rng.integers(8, 32, size=Cout, dtype=np.uint8)
    one7[Cout // 2 + 1] = 7
    ge8 = rng.integers(8, 32, size=Cout, dtype=np.uint8)
    ge8[:2] = [8, 31]
    dX, dW = ctx.upload(X), ctx.upload(Wt)
    for sh in (full, one7, ge8):
        dS = ctx.upload(sh)
        dY = ctx.empty((N, Ho, Wo, Cout), np.int8)
        ctx.conv2d_i8_nhwc(dX, dW, dS, dY, N, H, W, Cin, Cout, R, S, stride, pad)
        ctx.wait(60_000)
        assert np.array_equal(ctx.download(dY), oracle.conv2d_nhwc_i8(X, Wt, sh, stride, pad)), sh


def test_conv2d_i8_config(ctx):
    """Config 4: N=8, 56x56, Cin=Cout=64, 3x3, stride 1, pad 1, shifts in [8,12]; full bit-exact compare."""
    _say("conv2d config 4")
    X = synth.int8((8, 56, 56, 64), 3)
    Wt = synth.int8((64, 3, 3, 64), 4)
    sh = synth.shifts(64, 7)
    dX, dW, dS = ctx.upload(X), ctx.upload(Wt), ctx.upload(sh)
    dY = ctx.empty((8, 56, 56, 64), np.int8)
    ctx.conv2d_i8_nhwc(dX, dW, dS, dY, 8, 56, 56, 64, 64, 3, 3, 1, 1)
    ctx.wait(60_000)
    Yg = ctx.download(dY)
    assert np.array_equal(Yg, oracle.conv2d_nhwc_i8(X, Wt, sh, 1, 1))


@pytest.mark.parametrize("shape", [(64, 64, 128, 64), (256, 256, 512, 256), (100, 70, 90, 30),
                                   (1000, 512, 1088, 528)])  # M, F and Nout that no tile divides
def test_mlp_i8(ctx, shape):
    M, K, F, Nout = shape
    _say("mlp", shape)
    rng = np.random.default_rng(M + F)
    X = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    W1 = rng.integers(-128, 128, size=(K, F), dtype=np.int8)
    W2 = rng.integers(-128, 128, size=(F, Nout), dtype=np.int8)
    dX, d1, d2 = ctx.upload(X), ctx.upload(W1), ctx.upload(W2)
    dH, dY = ctx.empty((M, F), np.int8), ctx.empty((M, Nout), np.int8)
    ctx.mlp_i8(dX, d1, d2, dH, dY, M, K, F, Nout, 11, 12)
    ctx.wait(60_000)
    Yo, Ho = oracle.mlp_i8(X, W1, W2, 11, 12, want_h=True)
    assert np.array_equal(ctx.download(dH), Ho)
    assert np.array_equal(ctx.download(dY), Yo)


@pytest.mark.parametrize("form,s1,s2", [("uniform", 5, 12), ("uniform", 11, 7), ("mixed", 6, 12),
                                        ("mixed", 11, 12)])
def test_mlp_i8_cached_h_forms(ctx, form, s1, s2):
    """The up-projection writes H with ordinary stores (it is read right
    after) in both requant forms (shift < 8: clamp; >= 8: high byte), from
    the uniform 256x256 kernel and from the mixed-tile one.  Planned for one
    CU, so that these small shapes take 256-row tiles."""
    M, K, F, Nout = (256, 256, 512, 256) if form == "uniform" else (256, 256, 384, 256)
    prev = ctx.plan_set_cus(1)
    try:
        up = ctx.plan_gemm_i8(M, F, K)
        _say("mlp cached H", (M, K, F, Nout), form, "shifts", s1, s2, "plan", up)
        want = mi.KERNEL_PIPE if form == "uniform" else mi.KERNEL_PIPE_MIXED
        assert (up["kernel"], up["tile_m"], up["tile_n"]) == (want, 256, 256)
        rng = np.random.default_rng(1000 + 10 * s1 + s2)
        X = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
        W1 = rng.integers(-128, 128, size=(K, F), dtype=np.int8)
        W2 = rng.integers(-128, 128, size=(F, Nout), dtype=np.int8)
        dX, d1, d2 = ctx.upload(X), ctx.upload(W1), ctx.upload(W2)
        dH, dY = ctx.empty((M, F), np.int8), ctx.empty((M, Nout), np.int8)
        ctx.mlp_i8(dX, d1, d2, dH, dY, M, K, F, Nout, s1, s2)
        ctx.wait(60_000)
    finally:
        assert ctx.plan_set_cus(prev) == 1
    Yo, Ho = oracle.mlp_i8(X, W1, W2, s1, s2, want_h=True)
    assert np.array_equal(ctx.download(dH), Ho)
    assert np.array_equal(ctx.download(dY), Yo)


def test_mlp_i8_config(ctx):
    """Config 5: X 2048x4096 -> W1 4096x11008 (rq 11 + ReLU) -> W2 11008x4096
    (rq 12).  H and Y compared with the oracle over every element."""
    M, K, F, Nout = 2048, 4096, 11008, 4096
    _say("mlp config 5")
    X = synth.int8((M, K), 3)
    W1 = synth.int8((K, F), 5)
    W2 = synth.int8((F, Nout), 6)
    dX, d1, d2 = ctx.upload(X), ctx.upload(W1), ctx.upload(W2)
    dH, dY = ctx.empty((M, F), np.int8), ctx.empty((M, Nout), np.int8)
    ctx.mlp_i8(dX, d1, d2, dH, dY, M, K, F, Nout, 11, 12)
    ctx.wait(120_000)
    Hg, Yg = ctx.download(dH), ctx.download(dY)
    for b in (dX, d1, d2, dH, dY):
        b.free()
    Yo, Ho = oracle.mlp_i8(X, W1, W2, 11, 12, want_h=True)
    assert _mismatches(Hg, Ho) == 0
    assert _mismatches(Yg, Yo) == 0
    assert Ho.min() >= 0 and Ho.max() > 0  # ReLU, and not all zero


def test_fill_i8_matches_host_generator(ctx):
    _say("fill_i8")
    for n, tid in [(1, 1), (15, 2), (16, 3), (12345, 4), (1 << 20, 5)]:
        d = ctx.empty((n,), np.int8)
        ctx.fill_i8(d, n, tid)
        ctx.wait(10_000)
        got = ctx.download(d)
        assert np.array_equal(got, synth.int8((n,), tid))
        assert np.array_equal(got, oracle.fill_i8(n, tid))
        d.free()


@pytest.mark.parametrize("nbytes,offset", [(1, 0), (4096, 0), (1000003, 0), (4096, 3)])
def test_copy_d2d(ctx, nbytes, offset):
    _say("copy_d2d", nbytes, offset)
    src = np.random.default_rng(nbytes).integers(0, 256, size=nbytes + 16, dtype=np.uint8)
    d_src = ctx.upload(src)
    d_dst = ctx.upload(np.zeros(nbytes + 16, dtype=np.uint8))
    ctx.copy_d2d(d_dst.ptr + offset, d_src.ptr + offset, nbytes)
    ctx.wait(10_000)
    got = ctx.download(d_dst)
    assert np.array_equal(got[offset:offset + nbytes], src[offset:offset + nbytes])
    assert not got[:offset].any() and not got[offset + nbytes:].any()


def test_argument_errors(ctx):
    """Invalid arguments are rejected on the host with MIAIE_EINVAL and a message; nothing launches."""
    _say("argument errors")
    d = ctx.empty((4096,), np.int8)
    assert ctx.call_status("miaie_gemm_i8_i32", None, d.ptr, d.ptr, 4, 4, 4, 4, 4, 4, 0) == mi.MIAIE_EINVAL
    assert "A is NULL" in ctx.last_error()
    assert ctx.call_status("miaie_gemm_i8_i32", d.ptr, d.ptr, d.ptr, 0, 4, 4, 4, 4, 4, 0) == mi.MIAIE_EINVAL
    assert ctx.call_status("miaie_gemm_i8_i32", d.ptr, d.ptr, d.ptr, 4, 4, 4, 3, 4, 4, 0) == mi.MIAIE_EINVAL
    assert ctx.call_status("miaie_gemm_i8_i32", d.ptr, d.ptr, d.ptr, 4, 4, 4, 4, 4, 4, 2) == mi.MIAIE_EINVAL
    assert ctx.call_status("miaie_gemm_i8_rq", d.ptr, d.ptr, d.ptr, 4, 4, 4, 32, 0, None, 0) == mi.MIAIE_EINVAL
    assert "shift=32" in ctx.last_error()
    assert ctx.call_status("miaie_gemm_i8_rq", d.ptr, d.ptr, d.ptr, 4, 4, 4, 5, 2, None, 0) == mi.MIAIE_EINVAL
    assert ctx.call_status("miaie_conv2d_i8_nhwc", d.ptr, d.ptr, d.ptr, d.ptr, 1, 2, 2, 4, 4, 5, 5, 1, 0) == mi.MIAIE_EINVAL
    assert ctx.call_status("miaie_mm_window_i32", d.ptr, d.ptr, 0) == mi.MIAIE_EINVAL
    assert ctx.call_status("miaie_mlp_i8", d.ptr, d.ptr, d.ptr, None, d.ptr, 4, 4, 4, 4, 11, 12) == mi.MIAIE_EINVAL
    ctx.wait(10_000)
    d.free()


def test_launch_status_ignores_earlier_runtime_errors(ctx):
    """A failed HIP call of the caller's own (here hipSetDevice on a device
    that does not exist) before an entry point does not make its launches
    report a failure: each launch's status is the launch's own."""
    import ctypes

    _say("launch status after a caller's failed runtime call")
    hip = ctypes.CDLL("libamdhip64.so")
    count = ctypes.c_int()
    assert hip.hipGetDeviceCount(ctypes.byref(count)) == 0
    M = N = K = 256
    rng = np.random.default_rng(5)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    B = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    dA, dB, dY = ctx.upload(A), ctx.upload(B), ctx.empty((M, N), np.int8)
    X = rng.integers(-128, 128, size=(1, 8, 8, 64), dtype=np.int8)
    Wt = rng.integers(-128, 128, size=(64, 3, 3, 64), dtype=np.int8)
    sh = np.full(64, 9, dtype=np.uint8)
    dX, dW, dS, dC = ctx.upload(X), ctx.upload(Wt), ctx.upload(sh), ctx.empty((1, 8, 8, 64), np.int8)
    for call in (lambda: ctx.call_status("miaie_gemm_i8_rq", dA.ptr, dB.ptr, dY.ptr, M, N, K, 10, 0, None, mi.B_NN),
                 lambda: ctx.call_status("miaie_conv2d_i8_nhwc", dX.ptr, dW.ptr, dS.ptr, dC.ptr, 1, 8, 8, 64, 64, 3, 3,
                                         1, 1)):
        assert hip.hipSetDevice(count.value + 7) != 0  # the caller's own failed call
        assert call() == mi.MIAIE_OK, ctx.last_error()
    ctx.wait(10_000)
    assert np.array_equal(ctx.download(dY), oracle.requant(oracle.gemm_i8(A, B), 10))
    assert np.array_equal(ctx.download(dC), oracle.conv2d_nhwc_i8(X, Wt, sh, 1, 1))
    for b in (dA, dB, dY, dX, dW, dS, dC):
        b.free()
    hip.hipGetLastError()  # clear the planted error for whatever runs next


def test_wait_deadline(ctx):
    """miaie_wait returns MIAIE_ETIMEDOUT when the deadline passes first and OK once drained."""
    _say("wait deadline")
    inp = np.zeros(4, dtype=np.uint32)
    inp[0] = 0xFFFFFFFF  # ~1.6e12 MACs: milliseconds of work, then it ends
    d_in, d_out = ctx.upload(inp), ctx.empty((8,), np.uint32)
    ctx.dot_u8_probe(d_in, d_out)
    rc = ctx.call_status("miaie_wait", 0)
    assert rc in (mi.MIAIE_ETIMEDOUT, mi.MIAIE_OK)
    ctx.wait(60_000)
    assert ctx.download(d_out)[1] == 4567
