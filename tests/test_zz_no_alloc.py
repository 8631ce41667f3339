"""miaie_mlp_i8_noalloc (H in the library's file-scope device array) through
the C ABI, bit-exact as every integer path:

- against the CPU oracle's Y directly, and against miaie_mlp_i8 (H from the
  caller), whose H is compared with the oracle's H;
- two calls in a row, the second smaller, so the second reads a scratch array
  the first left full of its own H;
- two contexts (two streams) issuing interleaved calls without waiting in
  between: the calls share the one array and are ordered through its event,
  so each result still equals its own oracle."""
import numpy as np
import pytest

import aiehlc_amd as mi
import oracle

pytestmark = pytest.mark.gpu

MAX_H = 32 << 20  # MIAIE_MLP_NOALLOC_MAX_H


def _inputs(shape, seed):
    M, K, F, Nout = shape
    rng = np.random.default_rng(seed)
    X = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    W1 = rng.integers(-128, 128, size=(K, F), dtype=np.int8)
    W2 = rng.integers(-128, 128, size=(F, Nout), dtype=np.int8)
    return X, W1, W2


def test_noalloc_mlp_matches_the_oracle_and_the_allocating_entry_point(ctx):
    # first call: a large H (config 5's F, 1024 rows: 11 MiB of the 32 MiB);
    # second call: smaller and ragged (the 64x64 fallback GEMMs)
    for shape, seed in (((1024, 512, 11008, 1024), 1), ((100, 70, 90, 30), 2)):
        print(f"[case] mlp_i8_noalloc {shape}", flush=True)
        M, K, F, Nout = shape
        X, W1, W2 = _inputs(shape, seed)
        dX, d1, d2 = ctx.upload(X), ctx.upload(W1), ctx.upload(W2)
        dH, dY, dYn = ctx.empty((M, F), np.int8), ctx.empty((M, Nout), np.int8), ctx.empty((M, Nout), np.int8)
        ctx.mlp_i8_noalloc(dX, d1, d2, dYn, M, K, F, Nout, 11, 12)
        ctx.mlp_i8(dX, d1, d2, dH, dY, M, K, F, Nout, 11, 12)
        ctx.wait(60_000)
        got, want_y, got_h = ctx.download(dYn), ctx.download(dY), ctx.download(dH)
        for b in (dX, d1, d2, dH, dY, dYn):
            b.free()
        Yo, Ho = oracle.mlp_i8(X, W1, W2, 11, 12, want_h=True)
        assert np.array_equal(got_h, Ho), (shape, int(np.count_nonzero(got_h != Ho)))
        assert np.array_equal(got, Yo), (shape, int(np.count_nonzero(got != Yo)))
        assert np.array_equal(want_y, Yo)
        assert Yo.any() and Ho.any()


def test_noalloc_mlp_two_streams_share_the_array_in_order(ctx):
    # two contexts, each with its own stream, issue calls of different shapes
    # alternately without waiting: every call writes its whole H into the
    # shared array, so unordered calls would read another call's H
    shapes = [((512, 256, 4096, 512), 11), ((768, 128, 2048, 256), 12)]
    ctxs = [ctx, mi.Context(0)]
    try:
        assert ctxs[0].stream != ctxs[1].stream
        cases = []
        for c, (shape, seed) in zip(ctxs, shapes):
            M, K, F, Nout = shape
            X, W1, W2 = _inputs(shape, seed)
            bufs = [c.upload(X), c.upload(W1), c.upload(W2)] + [c.empty((M, Nout), np.int8) for _ in range(3)]
            c.wait(60_000)
            cases.append((c, shape, (X, W1, W2), bufs))
        print("[case] mlp_i8_noalloc on two streams, interleaved", flush=True)
        for r in range(3):
            for c, (M, K, F, Nout), _, b in cases:
                c.mlp_i8_noalloc(b[0], b[1], b[2], b[3 + r], M, K, F, Nout, 11, 12)
        for c, shape, (X, W1, W2), b in cases:
            c.wait(60_000)
            Yo = oracle.mlp_i8(X, W1, W2, 11, 12)
            for r in range(3):
                got = c.download(b[3 + r])
                assert np.array_equal(got, Yo), (shape, r, int(np.count_nonzero(got != Yo)))
            for x in b:
                x.free()
    finally:
        ctxs[1].close()


def test_noalloc_mlp_rejects_an_h_beyond_the_array(ctx):
    d = ctx.empty((4096,), np.int8)
    # M*F one byte past the array: refused on the host, nothing launched
    F = 4096
    M = MAX_H // F + 1
    rc = ctx.call_status("miaie_mlp_i8_noalloc", d.ptr, d.ptr, d.ptr, d.ptr, M, 16, F, 16, 11, 12)
    assert rc == mi.MIAIE_EINVAL
    assert "MIAIE_MLP_NOALLOC_MAX_H" in ctx.last_error()
    assert ctx.call_status("miaie_mlp_i8_noalloc", d.ptr, None, d.ptr, d.ptr, 4, 4, 4, 4, 11, 12) == mi.MIAIE_EINVAL
    ctx.wait(10_000)
    d.free()
