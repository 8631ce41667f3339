"""GPU parity of the reference's single-tile kernels, through the miaie C ABI.

Each test runs the reference harness flow (allocate, move in, run, wait,
move out, compare: example/matrixmultiply/aieml_mm.cc:108-249) and checks
the result against the CPU oracle and against the reference's own known
answers.
"""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _say(*a):
    print("[case]", *a, flush=True)


@pytest.mark.parametrize("n,base", [(16, 0), (16, 1), (8, 0), (1, 5), (33, 0), (100, 7)])
def test_mm_window_i32(ctx, n, base):
    """aieml_mm.cc (inputs i) / aieml_perf.cc (inputs i+1) / aieoob.c (n=8)."""
    _say("mm_window_i32", n, base)
    win = (np.arange(2 * n * n, dtype=np.int64) + base).astype(np.int32)
    d_in = ctx.upload(win)
    d_out = ctx.upload(np.zeros(n * n, dtype=np.int32))
    ctx.mm_window_i32(d_in, d_out, n)
    ctx.wait(10_000)
    got = ctx.download(d_out)
    want = oracle.mm_window_i32(win, n)
    assert oracle.count_mismatch_i32(want, got) == 0
    if (n, base) == (16, 0):
        c = got.reshape(16, 16)
        assert (c[0, 0], c[0, 1], c[1, 0], c[15, 15], int(c.sum())) == (31960, 33880, 99416, 1994200, 200366080)
    if (n, base) == (16, 1):
        c = got.reshape(16, 16)
        assert (c[0, 0], c[15, 15], int(c.sum())) == (36312, 2006232, 202463232)
    if (n, base) == (8, 0):
        c = got.reshape(8, 8)
        assert (c[0, 0], c[7, 7], int(c.sum())) == (1932, 58828, 1542912)


def test_perf_window_u32_wraparound(ctx):
    """aieml_perf.cc:61-83 is uint32: large inputs must wrap exactly like the golden."""
    _say("perf_window_u32 wrap")
    n = 16
    rng = np.random.default_rng(5)
    win = rng.integers(0, 2**32, size=2 * n * n, dtype=np.uint64).astype(np.uint32)
    d_in = ctx.upload(win)
    d_out = ctx.upload(np.zeros(n * n, dtype=np.uint32))
    ctx.perf_window_u32(d_in, d_out, n)
    ctx.wait(10_000)
    got = ctx.download(d_out).view(np.int32)
    want = oracle.mm_window_i32(win.view(np.int32), n)
    assert np.array_equal(got, want)


def test_nokernelload_window_kat(ctx):
    """aie_nokernelload.cc:121-125 inputs (word 0 = 2^20) through the golden of :137-173."""
    _say("nokernelload window")
    win = np.arange(512, dtype=np.int32)
    win[0] = 1 << 20
    d_in = ctx.upload(win)
    d_out = ctx.upload(np.zeros(256, dtype=np.int32))
    ctx.mm_window_i32(d_in, d_out, 16)
    ctx.wait(10_000)
    c = ctx.download(d_out)
    assert (c[0], c[1]) == (268467416, 285246552)


@pytest.mark.parametrize("param", [1 << 20, 1, 0, 1023, 1025, (1 << 24) + 3, 0xFFFFFFFF])
def test_dot_u8_probe(ctx, param):
    """aie_nokernelload.cc:50-83; 2^20 gives {3145728, 4567, 811597824, 3, 2}."""
    _say("dot_u8_probe", param)
    inp = np.zeros(512, dtype=np.uint32)
    inp[0] = param
    d_in = ctx.upload(inp)
    d_out = ctx.upload(np.zeros(8, dtype=np.uint32))
    ctx.dot_u8_probe(d_in, d_out)
    ctx.wait(60_000)
    got = ctx.download(d_out)[:5]
    assert np.array_equal(got, oracle.dot_u8_probe(param))
    if param == 1 << 20:
        assert list(got) == [3145728, 4567, 811597824, 3, 2]


def test_mm_square_replicated(ctx):
    """vek385_verification.cpp:56-69,117-138: tiles with all-v inputs give 3*v^2 = {27,48,75,108}."""
    _say("mm_square_u64")
    n, vals, iters = 3, [3, 4, 5, 6], 5
    inp = np.concatenate([np.full(n * n, v, dtype=np.uint64) for v in vals])
    d_in = ctx.upload(inp)
    d_out = ctx.upload(np.zeros(len(vals) * (n * n + 1), dtype=np.uint64))
    ctx.mm_square_u64(d_in, d_out, n, len(vals), iters)
    ctx.wait(10_000)
    got = ctx.download(d_out).reshape(len(vals), n * n + 1)
    for t, v in enumerate(vals):
        want = oracle.mm_square_u64(inp[t * 9:(t + 1) * 9], n, iters)
        assert np.array_equal(got[t], want)
        assert set(got[t, :9].tolist()) == {3 * v * v} and got[t, 9] == iters
    assert got[:, 0].tolist() == [27, 48, 75, 108]


def test_mm_square_wraps_like_int(ctx):
    _say("mm_square_u64 wrap")
    rng = np.random.default_rng(9)
    n, batch = 7, 33
    inp = rng.integers(0, 2**63, size=batch * n * n, dtype=np.uint64)
    d_in = ctx.upload(inp)
    d_out = ctx.upload(np.zeros(batch * (n * n + 1), dtype=np.uint64))
    ctx.mm_square_u64(d_in, d_out, n, batch, 1)
    ctx.wait(10_000)
    got = ctx.download(d_out).reshape(batch, -1)
    for t in range(batch):
        assert np.array_equal(got[t], oracle.mm_square_u64(inp[t * n * n:(t + 1) * n * n], n, 1))


@pytest.mark.parametrize("addends,expect", [([1, 10], 26), ([1] * 8, 23), ([], 15)])
def test_chain(ctx, addends, expect):
    """multi_tile.cpp:150 (15+1+10 = 26) and seq_full_col.cpp:163 (15 + 8 stages of +1 = 23)."""
    _say("chain", addends)
    inp = np.full(20, 15, dtype=np.int32)
    d_in = ctx.upload(inp)
    d_out = ctx.upload(np.full(20, 9999, dtype=np.int32))
    ctx.chain_add_i32(d_in, d_out, 20, addends)
    ctx.wait(10_000)
    got = ctx.download(d_out)
    assert np.array_equal(got, oracle.chain_add(inp, 20, addends))
    assert set(got.tolist()) == {expect}
