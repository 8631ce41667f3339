"""The tiling planner (miaie_plan_gemm_i8) and the tiles it picks.

The planner chooses the pipelined kernel's workgroup tile (256x256,
256x128 or 128x128) from the shape and the device's CU count; every choice
must give the oracle's bits exactly, in every output mode and both B
layouts.  Small-M products (one GPU's share of a GEMM sharded over M) are
where the 128x128 tile is chosen."""
import numpy as np
import pytest

import aiehlc_amd as mi
import oracle

pytestmark = pytest.mark.gpu


def test_planner_choices(ctx):
    full = ctx.plan_gemm_i8(4096, 4096, 4096)
    assert (full["kernel"], full["tile_m"], full["tile_n"]) == (mi.KERNEL_PIPE, 256, 256)
    assert full["workgroups"] == 256 and full["threads"] == 256
    # one GPU's 512-row share of the 4096^3 GEMM: more, smaller tiles
    shard = ctx.plan_gemm_i8(512, 4096, 4096)
    assert (shard["tile_m"], shard["tile_n"], shard["workgroups"]) == (128, 128, 128)
    # the MLP's up-projection: 256 wide tiles fill one round, 176 narrow ones
    # the next (344 wide tiles would take 2 rounds, 688 narrow ones 2.7)
    up = ctx.plan_gemm_i8(2048, 11008, 4096)
    assert (up["kernel"], up["tile_m"], up["tile_n"], up["workgroups"]) == (mi.KERNEL_PIPE_MIXED, 256, 256, 256 + 176)
    # its down-projection: exactly one round of 256x128 tiles
    down = ctx.plan_gemm_i8(2048, 4096, 11008)
    assert (down["kernel"], down["tile_m"], down["tile_n"]) == (mi.KERNEL_PIPE, 256, 128)
    # M and N that no tile divides: the same tiles, the last row and column
    # overlapping their neighbours (16 x 16 tiles of 256 cover 4000)
    ragged = ctx.plan_gemm_i8(4000, 4000, 4096)
    assert (ragged["kernel"], ragged["tile_m"], ragged["tile_n"], ragged["workgroups"]) == (mi.KERNEL_PIPE, 256, 256, 256)
    assert ctx.plan_gemm_i8(4000, 4004, 4096)["kernel"] == mi.KERNEL_TILE64  # N % 16 != 0 and no tile divides N
    assert ctx.plan_gemm_i8(4000, 4096, 4096)["kernel"] == mi.KERNEL_PIPE    # only M ragged: any N a tile divides
    # shapes the pipelined kernel cannot take
    assert ctx.plan_gemm_i8(100, 50, 30)["kernel"] == mi.KERNEL_TILE64
    assert ctx.plan_gemm_i8(128, 128, 100)["kernel"] == mi.KERNEL_TILE64
    assert ctx.call_status("miaie_plan_gemm_i8", 0, 1, 1, None) == mi.MIAIE_EINVAL
    # planning for fewer CUs: one CU takes the widest tile that fits
    prev = ctx.plan_set_cus(1)
    try:
        assert (ctx.plan_gemm_i8(512, 512, 256)["tile_m"], ctx.plan_gemm_i8(512, 512, 256)["tile_n"]) == (256, 256)
        assert ctx.plan_gemm_i8(256, 384, 256)["kernel"] == mi.KERNEL_PIPE_MIXED  # one wide + one narrow tile
        assert ctx.plan_gemm_i8(256, 384, 192)["tile_n"] == 128  # K % 128 != 0: no mixed kernel
        assert ctx.plan_gemm_i8(128, 256, 256)["tile_m"] == 128
    finally:
        assert ctx.plan_set_cus(prev) == 1
    assert ctx.plan_gemm_i8(4096, 4096, 4096)["tile_n"] == 256
    assert ctx.call_status("miaie_plan_set_cus", 0, None) == mi.MIAIE_EINVAL


SHAPES = [(512, 4096, 4096, mi.B_NN), (256, 1024, 2048, mi.B_NT), (128, 2048, 1024, mi.B_NN),
          (384, 640, 512, mi.B_NT), (128, 128, 64, mi.B_NN)]


@pytest.mark.parametrize("M,N,K,layout", SHAPES)
def test_128_tiles_match_the_oracle(ctx, M, N, K, layout):
    plan = ctx.plan_gemm_i8(M, N, K)
    print(f"[case] gemm {M}x{N}x{K} layout {layout} plan {plan}", flush=True)
    assert (plan["tile_m"], plan["tile_n"]) == (128, 128)
    rng = np.random.default_rng(M + N + K + layout)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    B = rng.integers(-128, 128, size=(N, K) if layout == mi.B_NT else (K, N), dtype=np.int8)
    dA, dB = ctx.upload(A), ctx.upload(B)
    dC, dY, dY2, dC2 = (ctx.empty((M, N), np.int32), ctx.empty((M, N), np.int8), ctx.empty((M, N), np.int8),
                        ctx.empty((M, N), np.int32))
    ctx.gemm_i8_i32(dA, dB, dC, M, N, K, b_layout=layout)          # C only
    ctx.gemm_i8_rq(dA, dB, dY, M, N, K, 10, False, None, layout)    # Y only
    ctx.gemm_i8_rq(dA, dB, dY2, M, N, K, 11, True, dC2, layout)     # Y + C, ReLU
    ctx.wait(60_000)
    C = ctx.download(dC)
    slabs = [(0, M)] if M * N * K <= 2**31 else [(0, 64), (M - 64, M)]
    for r0, r1 in slabs:
        assert np.array_equal(C[r0:r1], oracle.gemm_i8(A, B, b_nt=layout == mi.B_NT, rows=(r0, r1)))
    assert np.array_equal(ctx.download(dY), oracle.requant(C, 10))
    assert np.array_equal(ctx.download(dY2), oracle.requant(C, 11, relu=True))
    assert np.array_equal(ctx.download(dC2), C)
    if len(slabs) > 1:  # full-size check by linearity in A: C(2A') = 2 C(A')
        A2 = (A // 2).astype(np.int8)
        dA2 = ctx.upload((2 * A2.astype(np.int16)).astype(np.int8))
        dAh, dCh = ctx.upload(A2), ctx.empty((M, N), np.int32)
        ctx.gemm_i8_i32(dA2, dB, dC, M, N, K, b_layout=layout)
        ctx.gemm_i8_i32(dAh, dB, dCh, M, N, K, b_layout=layout)
        ctx.wait(60_000)
        assert np.array_equal(ctx.download(dC), 2 * ctx.download(dCh))


# K sweep over the pipelined kernels: K % 128 == 0 takes the pair-staged
# kernel (A staged two k-tiles at a time, a copy schedule whose waits change
# over the last six k-tiles and in the prologue below 6 k-tiles), other
# multiples of 64 the per-k-tile kernel.  Every k-tile count from the
# smallest up to well past the steady state, at each tile width (planned for
# one CU, M x N picks 256x256, 256x128 and 128x128, and 256 x 384 one wide
# and one narrow tile in a mixed launch), both B layouts and every output
# mode.
K_SWEEP = [64, 128, 192, 256, 320, 384, 512, 640, 768, 896, 1024, 1152, 1280, 2176, 2240]
TILE_SHAPES = [(512, 512), (256, 128), (128, 256), (256, 384)]


@pytest.mark.parametrize("K", K_SWEEP)
@pytest.mark.parametrize("MN", TILE_SHAPES)
@pytest.mark.parametrize("layout", [mi.B_NN, mi.B_NT])
def test_pipelined_k_sweep(ctx, K, MN, layout):
    M, N = MN
    # planning for one CU makes the planner take the widest tile that fits
    prev = ctx.plan_set_cus(1)
    try:
        _k_sweep(ctx, M, N, K, MN, layout)
    finally:
        ctx.plan_set_cus(prev)


def _k_sweep(ctx, M, N, K, MN, layout):
    plan = ctx.plan_gemm_i8(M, N, K)
    print(f"[case] k-sweep gemm {M}x{N}x{K} layout {layout} plan {plan}", flush=True)
    if MN == (256, 384) and K % 128 == 0:
        # one 256x256 and one 256x128 tile in one launch (the pair-staged kernel needs K % 128 == 0)
        assert (plan["kernel"], plan["workgroups"]) == (mi.KERNEL_PIPE_MIXED, 2)
    else:
        assert plan["kernel"] == mi.KERNEL_PIPE
        assert (plan["tile_m"], plan["tile_n"]) == {(512, 512): (256, 256), (256, 128): (256, 128),
                                                    (128, 256): (128, 128), (256, 384): (256, 128)}[MN]
    rng = np.random.default_rng(7 * K + M + layout)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    B = rng.integers(-128, 128, size=(N, K) if layout == mi.B_NT else (K, N), dtype=np.int8)
    dA, dB = ctx.upload(A), ctx.upload(B)
    dC, dY, dY2, dC2, dY3 = (ctx.empty((M, N), np.int32), ctx.empty((M, N), np.int8), ctx.empty((M, N), np.int8),
                             ctx.empty((M, N), np.int32), ctx.empty((M, N), np.int8))
    ctx.gemm_i8_i32(dA, dB, dC, M, N, K, b_layout=layout)          # C only
    ctx.gemm_i8_rq(dA, dB, dY, M, N, K, 10, False, None, layout)    # Y only, shift >= 8
    ctx.gemm_i8_rq(dA, dB, dY2, M, N, K, 11, True, dC2, layout)     # Y + C, ReLU
    ctx.gemm_i8_rq(dA, dB, dY3, M, N, K, 5, True, None, layout)     # Y only, shift < 8, ReLU
    ctx.wait(60_000)
    C = ctx.download(dC)
    assert np.array_equal(C, oracle.gemm_i8(A, B, b_nt=layout == mi.B_NT))
    assert np.array_equal(ctx.download(dY), oracle.requant(C, 10))
    assert np.array_equal(ctx.download(dY2), oracle.requant(C, 11, relu=True))
    assert np.array_equal(ctx.download(dC2), C)
    assert np.array_equal(ctx.download(dY3), oracle.requant(C, 5, relu=True))
    for b in (dA, dB, dC, dY, dY2, dC2, dY3):
        b.free()


# Operands inside larger row-major arrays (row pitch > the product's extent):
# 16-byte multiples keep the pipelined kernels (per-k-tile and pair-staged),
# other pitches take the bounds-checked 64x64 kernel.  C = A.B is checked on
# the product's rows and columns, and C's padding must stay untouched.
@pytest.mark.parametrize("M,N,K,lda,ldb,ldc,layout", [
    (512, 512, 256, 320, 640, 528, mi.B_NN),   # pair-staged 256x256
    (512, 512, 256, 336, 272, 520, mi.B_NT),
    (512, 512, 192, 208, 528, 512, mi.B_NN),   # per-k-tile 256x256 (K % 128 != 0)
    (256, 384, 384, 400, 400, 392, mi.B_NN),   # 256x128
    (128, 256, 256, 288, 304, 260, mi.B_NT),   # 128x128
    (128, 256, 256, 260, 256, 256, mi.B_NN),   # lda % 16 != 0: fallback
    (300, 400, 256, 320, 416, 408, mi.B_NN),   # ragged M and N, pair-staged 256x256 (overlapping last tiles)
    (500, 304, 192, 208, 224, 312, mi.B_NT),   # ragged M and N, per-k-tile 256x128
])
def test_strided_operands(ctx, M, N, K, lda, ldb, ldc, layout):
    prev = ctx.plan_set_cus(1)
    try:
        print(f"[case] strided gemm {M}x{N}x{K} lda {lda} ldb {ldb} ldc {ldc} layout {layout}", flush=True)
        rng = np.random.default_rng(lda + ldb + ldc + layout)
        Ab = rng.integers(-128, 128, size=(M, lda), dtype=np.int8)
        Bb = rng.integers(-128, 128, size=(N, ldb) if layout == mi.B_NT else (K, ldb), dtype=np.int8)
        Cb = np.full((M, ldc), 0x5A5A5A5A, dtype=np.int32)
        dA, dB, dC = ctx.upload(Ab), ctx.upload(Bb), ctx.upload(Cb)
        ctx.gemm_i8_i32(dA, dB, dC, M, N, K, lda=lda, ldb=ldb, ldc=ldc, b_layout=layout)
        ctx.wait(60_000)
        Cg = ctx.download(dC)
        A = np.ascontiguousarray(Ab[:, :K])
        B = np.ascontiguousarray(Bb[:, :K] if layout == mi.B_NT else Bb[:, :N])
        assert np.array_equal(Cg[:, :N], oracle.gemm_i8(A, B, b_nt=layout == mi.B_NT))
        assert (Cg[:, N:] == 0x5A5A5A5A).all()
        for b in (dA, dB, dC):
            b.free()
    finally:
        ctx.plan_set_cus(prev)


# Shapes the pipelined kernels cannot take (M or N below the smallest tile,
# N % 16 != 0 where no tile divides N, K % 64 != 0) with K % 16 == 0 and
# 16-byte aligned A rows run the prefetching 64x64 kernel (vector loads from
# clamped addresses, zeroed outside the matrix); bit-exact in every output
# mode and both B layouts, including products smaller than one tile and row
# pitches above the extent.
@pytest.mark.parametrize("M,N,K,layout,lda_pad", [
    (1000, 1000, 256, mi.B_NN, 0),  # N % 16 == 8
    (300, 4004, 128, mi.B_NT, 0),
    (129, 77, 64, mi.B_NN, 0),    # N not a multiple of 16: byte gathers down B's columns
    (33, 250, 192, mi.B_NT, 0),
    (2000, 100, 128, mi.B_NT, 0),
    (1, 1, 64, mi.B_NN, 0),
    (70, 130, 128, mi.B_NN, 16),  # lda = K + 16
    (70, 130, 128, mi.B_NT, 32),  # lda = K + 32, ldb = K + 32
    (100, 130, 80, mi.B_NN, 0),   # K % 64 == 16: the last k-tile is one chunk deep
    (65, 33, 48, mi.B_NT, 0),     # K % 64 == 48, one k-tile
    (300, 272, 1008, mi.B_NN, 0),
    (64, 64, 16, mi.B_NT, 16),    # K = 16, lda = ldb = 32
])
def test_ragged_fallback_matches_the_oracle(ctx, M, N, K, layout, lda_pad):
    plan = ctx.plan_gemm_i8(M, N, K)
    print(f"[case] ragged gemm {M}x{N}x{K} layout {layout} pad {lda_pad} plan {plan}", flush=True)
    assert plan["kernel"] == mi.KERNEL_TILE64
    rng = np.random.default_rng(M * 7 + N * 3 + K + layout + lda_pad)
    lda = K + lda_pad
    Ab = rng.integers(-128, 128, size=(M, lda), dtype=np.int8)
    if layout == mi.B_NT:
        ldb = K + lda_pad
        Bb = rng.integers(-128, 128, size=(N, ldb), dtype=np.int8)
        B = np.ascontiguousarray(Bb[:, :K])
    else:
        ldb = N
        Bb = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
        B = Bb
    A = np.ascontiguousarray(Ab[:, :K])
    C = oracle.gemm_i8(A, B, b_nt=layout == mi.B_NT)
    dA, dB = ctx.upload(Ab), ctx.upload(Bb)
    dC = ctx.empty((M, N), np.int32)
    ctx.gemm_i8_i32(dA, dB, dC, M, N, K, lda=lda, ldb=ldb, ldc=N, b_layout=layout)
    ctx.wait(60_000)
    assert np.array_equal(ctx.download(dC), C)
    if lda_pad == 0:  # the requantizing entry takes dense operands
        dY, dY2, dC2 = ctx.empty((M, N), np.int8), ctx.empty((M, N), np.int8), ctx.empty((M, N), np.int32)
        ctx.gemm_i8_rq(dA, dB, dY, M, N, K, 10, False, None, layout)
        ctx.gemm_i8_rq(dA, dB, dY2, M, N, K, 5, True, dC2, layout)
        ctx.wait(60_000)
        assert np.array_equal(ctx.download(dY), oracle.requant(C, 10))
        assert np.array_equal(ctx.download(dY2), oracle.requant(C, 5, relu=True))
        assert np.array_equal(ctx.download(dC2), C)
        for b in (dY, dY2, dC2):
            b.free()
    for b in (dA, dB, dC):
        b.free()


# M and N that no tile divides, on the pipelined kernels: the last tile row
# (column) is moved back to end at M (N) and overlaps the one before it.
# (cus, expected kernel, tile): planned for `cus` CUs (0: the device's).
RAGGED = [
    (1000, 1008, 256, mi.B_NN, 0, None, None),
    (1000, 1008, 256, mi.B_NT, 0, None, None),
    (300, 4000, 128, mi.B_NN, 0, None, None),
    (300, 400, 256, mi.B_NN, 1, mi.KERNEL_PIPE, (256, 256)),   # pair-staged, both edges
    (300, 400, 256, mi.B_NT, 1, mi.KERNEL_PIPE, (256, 256)),
    (500, 304, 192, mi.B_NN, 1, mi.KERNEL_PIPE, (256, 128)),   # per-k-tile kernel (K % 128 == 64)
    (500, 304, 192, mi.B_NT, 1, mi.KERNEL_PIPE, (256, 128)),
    (130, 208, 256, mi.B_NN, 1, mi.KERNEL_PIPE, (128, 128)),
    (500, 528, 256, mi.B_NN, 1, mi.KERNEL_PIPE_MIXED, (256, 256)),  # narrow part 272 columns
    (500, 528, 256, mi.B_NT, 1, mi.KERNEL_PIPE_MIXED, (256, 256)),
    (2048, 10992, 256, mi.B_NN, 0, mi.KERNEL_PIPE_MIXED, (256, 256)),
]


@pytest.mark.parametrize("M,N,K,layout,cus,kernel,tile", RAGGED)
def test_ragged_pipelined_matches_the_oracle(ctx, M, N, K, layout, cus, kernel, tile):
    prev = ctx.plan_set_cus(cus) if cus else None
    try:
        plan = ctx.plan_gemm_i8(M, N, K)
        print(f"[case] ragged pipelined gemm {M}x{N}x{K} layout {layout} cus {cus} plan {plan}", flush=True)
        assert plan["kernel"] in (mi.KERNEL_PIPE, mi.KERNEL_PIPE_MIXED)
        if kernel is not None:
            assert (plan["kernel"], (plan["tile_m"], plan["tile_n"])) == (kernel, tile), plan
        rng = np.random.default_rng(M * 5 + N + K + layout)
        A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
        B = rng.integers(-128, 128, size=(N, K) if layout == mi.B_NT else (K, N), dtype=np.int8)
        dA, dB = ctx.upload(A), ctx.upload(B)
        dC, dY, dY2, dC2, dY3 = (ctx.empty((M, N), np.int32), ctx.empty((M, N), np.int8),
                                 ctx.empty((M, N), np.int8), ctx.empty((M, N), np.int32), ctx.empty((M, N), np.int8))
        ctx.gemm_i8_i32(dA, dB, dC, M, N, K, b_layout=layout)          # C only
        ctx.gemm_i8_rq(dA, dB, dY, M, N, K, 10, False, None, layout)    # Y only, shift >= 8
        ctx.gemm_i8_rq(dA, dB, dY2, M, N, K, 11, True, dC2, layout)     # Y + C, ReLU
        ctx.gemm_i8_rq(dA, dB, dY3, M, N, K, 5, True, None, layout)     # Y only, shift < 8, ReLU
        ctx.wait(60_000)
        C, Y, Y2, C2, Y3 = (ctx.download(d) for d in (dC, dY, dY2, dC2, dY3))
        for b in (dA, dB, dC, dY, dY2, dC2, dY3):
            b.free()
    finally:
        if cus:
            ctx.plan_set_cus(prev)
    Co = oracle.gemm_i8(A, B, b_nt=layout == mi.B_NT)
    assert np.array_equal(C, Co)
    assert np.array_equal(C2, Co)
    assert np.array_equal(Y, oracle.requant(Co, 10))
    assert np.array_equal(Y2, oracle.requant(Co, 11, relu=True))
    assert np.array_equal(Y3, oracle.requant(Co, 5, relu=True))


# Mixed launches (gemm_i8_pipe16_mixed): 256x256 tiles over the first
# columns, 256x128 tiles over the rest.  Planned for fewer CUs where that
# makes small shapes choose the mix; every output mode and both B layouts,
# bit-exact against the oracle.
MIXED = [(512, 1408, 256, 16, mi.B_NN), (512, 1408, 256, 16, mi.B_NT), (256, 640, 384, 2, mi.B_NN),
         (768, 896, 128, 5, mi.B_NT), (2048, 11008, 256, 256, mi.B_NN)]


@pytest.mark.parametrize("M,N,K,cus,layout", MIXED)
def test_mixed_tiles_match_the_oracle(ctx, M, N, K, cus, layout):
    prev = ctx.plan_set_cus(cus)
    try:
        plan = ctx.plan_gemm_i8(M, N, K)
        print(f"[case] mixed gemm {M}x{N}x{K} cus {cus} layout {layout} plan {plan}", flush=True)
        assert plan["kernel"] == mi.KERNEL_PIPE_MIXED, plan
        rng = np.random.default_rng(M * 3 + N + K + layout)
        A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
        B = rng.integers(-128, 128, size=(N, K) if layout == mi.B_NT else (K, N), dtype=np.int8)
        dA, dB = ctx.upload(A), ctx.upload(B)
        dC, dY, dY2, dC2 = (ctx.empty((M, N), np.int32), ctx.empty((M, N), np.int8), ctx.empty((M, N), np.int8),
                            ctx.empty((M, N), np.int32))
        ctx.gemm_i8_i32(dA, dB, dC, M, N, K, b_layout=layout)          # C only
        ctx.gemm_i8_rq(dA, dB, dY, M, N, K, 10, False, None, layout)    # Y only (int16-saturation form)
        ctx.gemm_i8_rq(dA, dB, dY2, M, N, K, 5, True, dC2, layout)      # Y + C, med3 form, ReLU
        ctx.wait(60_000)
        C, Y, Y2, C2 = ctx.download(dC), ctx.download(dY), ctx.download(dY2), ctx.download(dC2)
        for b in (dA, dB, dC, dY, dY2, dC2):
            b.free()
    finally:
        ctx.plan_set_cus(prev)
    Co = oracle.gemm_i8(A, B, b_nt=layout == mi.B_NT)
    assert np.array_equal(C, Co)
    assert np.array_equal(C2, Co)
    assert np.array_equal(Y, oracle.requant(Co, 10))
    assert np.array_equal(Y2, oracle.requant(Co, 5, relu=True))


# Seeded random shapes across every planner branch (uniform, mixed and ragged
# pipelined tiles, the 64x64 fallbacks), both B layouts, every output mode and
# shifts on both sides of 8, each against the oracle.  Sizes are drawn so that
# the pipelined kernels' conditions (K % 64, N % 16, M and N at least one
# tile) are met about half the time.
def _random_gemm_cases(n=24, seed=20261202):
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        M = int(rng.choice([int(rng.integers(1, 130)), int(rng.integers(128, 1100))]))
        N = int(rng.choice([int(rng.integers(1, 130)), 16 * int(rng.integers(8, 70)), int(rng.integers(128, 1100))]))
        K = int(rng.choice([64 * int(rng.integers(1, 9)), 16 * int(rng.integers(1, 40)), int(rng.integers(1, 300))]))
        cases.append((M, N, K, int(rng.integers(0, 2)), int(rng.integers(3, 14)), bool(rng.integers(0, 2)),
                      int(rng.choice([0, 1, 4, 256]))))
    return cases


@pytest.mark.parametrize("M,N,K,layout,shift,relu,cus", _random_gemm_cases())
def test_random_shapes_match_the_oracle(ctx, M, N, K, layout, shift, relu, cus):
    prev = ctx.plan_set_cus(cus) if cus else None
    try:
        plan = ctx.plan_gemm_i8(M, N, K)
        print(f"[case] random gemm {M}x{N}x{K} layout {layout} shift {shift} relu {relu} cus {cus} plan {plan}",
              flush=True)
        rng = np.random.default_rng(M * 1009 + N * 31 + K)
        A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
        B = rng.integers(-128, 128, size=(N, K) if layout == mi.B_NT else (K, N), dtype=np.int8)
        dA, dB = ctx.upload(A), ctx.upload(B)
        dC, dY, dY2, dC2 = (ctx.empty((M, N), np.int32), ctx.empty((M, N), np.int8), ctx.empty((M, N), np.int8),
                            ctx.empty((M, N), np.int32))
        ctx.gemm_i8_i32(dA, dB, dC, M, N, K, b_layout=layout)
        ctx.gemm_i8_rq(dA, dB, dY, M, N, K, shift, relu, None, layout)
        ctx.gemm_i8_rq(dA, dB, dY2, M, N, K, shift, relu, dC2, layout)
        ctx.wait(60_000)
        C, Y, Y2, C2 = (ctx.download(d) for d in (dC, dY, dY2, dC2))
        for b in (dA, dB, dC, dY, dY2, dC2):
            b.free()
    finally:
        if cus:
            ctx.plan_set_cus(prev)
    Co = oracle.gemm_i8(A, B, b_nt=layout == mi.B_NT)
    Yo = oracle.requant(Co, shift, relu=relu)
    assert np.array_equal(C, Co)
    assert np.array_equal(C2, Co)
    assert np.array_equal(Y, Yo)
    assert np.array_equal(Y2, Yo)


# The pipelined kernels start the accumulators of a Y-only launch at the
# rounding term 2^(s-1), exact while |acc| + 2^(s-1) < 2^31, which the
# launcher holds to K < 2^16 (|acc| <= K * 2^14); K = 65472 is the largest
# such K the pipelined kernels take, where an all -128 row times an all -128
# column gives acc = 2^30 - 2^20 and, at s = 31, acc + 2^30 lies 2^20 below
# 2^31.  K = 65536 takes the 64x64 kernel, whose requant rounds without the
# add ((acc >> s) + bit s-1 of acc).  Rows 0-2 of A and columns 0-2 of B are
# constant (-128, -128, 127) so that the top-left 3x3 block of accumulators
# sits at the extremes +-K*2^14; the rest is random.
@pytest.mark.parametrize("K,MN", [(65472, 256), (65536, 128)])
@pytest.mark.parametrize("layout", [mi.B_NN, mi.B_NT])
def test_requant_round_term_at_the_largest_k(ctx, K, MN, layout):
    M = N = MN
    plan = ctx.plan_gemm_i8(M, N, K)
    print(f"[case] requant boundary gemm {M}x{N}x{K} layout {layout} plan {plan}", flush=True)
    assert (plan["kernel"] == mi.KERNEL_TILE64) == (K >= 1 << 16)
    rng = np.random.default_rng(K + MN + layout)
    A = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    Bkn = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    for r, v in enumerate((-128, -128, 127)):
        A[r, :] = v
        Bkn[:, r] = v
    B = np.ascontiguousarray(Bkn.T) if layout == mi.B_NT else Bkn
    Co = oracle.gemm_i8(A, B, b_nt=layout == mi.B_NT)
    assert Co[0, 0] == K * 16384 and Co[0, 2] == -K * 16256
    dA, dB = ctx.upload(A), ctx.upload(B)
    dY, dY2, dC2 = ctx.empty((M, N), np.int8), ctx.empty((M, N), np.int8), ctx.empty((M, N), np.int32)
    try:
        for shift in (0, 1, 16, 29, 30, 31):
            for relu in (False, True):
                ctx.gemm_i8_rq(dA, dB, dY, M, N, K, shift, relu, None, layout)
                ctx.gemm_i8_rq(dA, dB, dY2, M, N, K, shift, relu, dC2, layout)
                ctx.wait(60_000)
                Yo = oracle.requant(Co, shift, relu=relu)
                Y, Y2, C2 = ctx.download(dY), ctx.download(dY2), ctx.download(dC2)
                assert np.array_equal(Y, Yo), (shift, relu, int(np.count_nonzero(Y != Yo)))
                assert np.array_equal(Y2, Yo), (shift, relu)
                assert np.array_equal(C2, Co), (shift, relu)
    finally:
        for b in (dA, dB, dY, dY2, dC2):
            b.free()
