"""miaie_mlp_i8_noalloc (H in the library's file-scope device array) against
miaie_mlp_i8 (H from the caller), through the C ABI: two calls in a row, the
second smaller, so the second reads a scratch array the first left full of
its own H.  Bit-exact, as every integer path."""
import numpy as np
import pytest

import aiehlc_amd as mi

pytestmark = pytest.mark.gpu

MAX_H = 32 << 20  # MIAIE_MLP_NOALLOC_MAX_H


def _mlp_both(ctx, shape, seed):
    M, K, F, Nout = shape
    rng = np.random.default_rng(seed)
    X = rng.integers(-128, 128, size=(M, K), dtype=np.int8)
    W1 = rng.integers(-128, 128, size=(K, F), dtype=np.int8)
    W2 = rng.integers(-128, 128, size=(F, Nout), dtype=np.int8)
    dX, d1, d2 = ctx.upload(X), ctx.upload(W1), ctx.upload(W2)
    dH, dY, dYn = ctx.empty((M, F), np.int8), ctx.empty((M, Nout), np.int8), ctx.empty((M, Nout), np.int8)
    ctx.mlp_i8(dX, d1, d2, dH, dY, M, K, F, Nout, 11, 12)
    ctx.mlp_i8_noalloc(dX, d1, d2, dYn, M, K, F, Nout, 11, 12)
    ctx.wait(60_000)
    want, got = ctx.download(dY), ctx.download(dYn)
    for b in (dX, d1, d2, dH, dY, dYn):
        b.free()
    return want, got


def test_noalloc_mlp_matches_the_allocating_entry_point(ctx):
    # first call: a large H (config 5's F, 1024 rows: 11 MiB of the 32 MiB);
    # second call: smaller and ragged (the 64x64 fallback GEMMs)
    for shape, seed in (((1024, 512, 11008, 1024), 1), ((100, 70, 90, 30), 2)):
        print(f"[case] mlp_i8_noalloc {shape}", flush=True)
        want, got = _mlp_both(ctx, shape, seed)
        assert np.array_equal(got, want), (shape, int(np.count_nonzero(got != want)))
        assert want.any()


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
