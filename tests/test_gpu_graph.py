"""Recorded kernel chains (miaie_graph_*): a chain of entry points recorded
once and replayed must give, on every replay, exactly what the CPU oracle
computes from that replay's inputs.  Eager work (refilling the inputs with
new seeds) runs between replays, so each replay reads fresh buffer contents
through the pointers fixed at recording time."""
import numpy as np
import pytest

import aiehlc_amd as mi
import oracle

pytestmark = pytest.mark.gpu


def _chain(ctx, b, out):
    """GEMM+requant, conv2d, the two-GEMM MLP and a device copy: the calls the
    graph records, writing into the buffers of `out`."""
    ctx.gemm_i8_rq(b["A"], b["B"], out["Y1"], 320, 384, 256, 10, False, None, mi.B_NN)
    ctx.conv2d_i8_nhwc(b["X"], b["W"], b["S"], out["Y2"], 2, 14, 14, 64, 64, 3, 3, 1, 1)
    ctx.mlp_i8(b["Xm"], b["W1"], b["W2"], out["H"], out["Y3"], 128, 256, 512, 192, 11, 12)
    ctx.copy_d2d(out["Y4"], out["Y1"], 320 * 384)


def _buffers(ctx):
    b = {
        "A": ctx.empty((320, 256), np.int8), "B": ctx.empty((256, 384), np.int8),
        "X": ctx.empty((2, 14, 14, 64), np.int8), "W": ctx.empty((64, 3, 3, 64), np.int8),
        "S": ctx.upload(mi.synth.shifts(64, 7)),
        "Xm": ctx.empty((128, 256), np.int8), "W1": ctx.empty((256, 512), np.int8),
        "W2": ctx.empty((512, 192), np.int8),
    }
    return b


def _outputs(ctx):
    return {"Y1": ctx.empty((320, 384), np.int8), "Y2": ctx.empty((2, 14, 14, 64), np.int8),
            "H": ctx.empty((128, 512), np.int8), "Y3": ctx.empty((128, 192), np.int8),
            "Y4": ctx.empty((320, 384), np.int8)}


def _refill(ctx, b, seed):
    for i, k in enumerate(("A", "B", "X", "W", "Xm", "W1", "W2")):
        ctx.fill_i8(b[k], b[k].nbytes, 1000 * seed + i)


def _oracle_outputs(ctx, b):
    """What the chain must produce, from the CPU oracle on the inputs the
    buffers hold (downloaded after the eager refill)."""
    A, B = ctx.download(b["A"]), ctx.download(b["B"])
    X, W, S = ctx.download(b["X"]), ctx.download(b["W"]), ctx.download(b["S"])
    Xm, W1, W2 = ctx.download(b["Xm"]), ctx.download(b["W1"]), ctx.download(b["W2"])
    Y1 = oracle.gemm_i8_rq(A, B, 10)
    Y3, H = oracle.mlp_i8(Xm, W1, W2, 11, 12, want_h=True)
    return {"Y1": Y1, "Y2": oracle.conv2d_nhwc_i8(X, W, S, 1, 1), "H": H, "Y3": Y3, "Y4": Y1}


def test_replays_match_the_oracle(ctx):
    """Every replay's outputs equal the CPU oracle's on that replay's inputs
    (the reference checks its chains against known answers: multi_tile.cpp:150,
    seq_full_col.cpp:163), and equal the same calls run directly."""
    b = _buffers(ctx)
    g_out, e_out = _outputs(ctx), _outputs(ctx)
    _refill(ctx, b, 1)
    ctx.wait(60_000)
    with ctx.record() as g:
        _chain(ctx, b, g_out)
    try:
        for replay in range(4):
            print(f"[case] replay {replay}", flush=True)
            _refill(ctx, b, 2 + replay)      # eager work between replays
            g.launch()
            _chain(ctx, b, e_out)            # the same calls, run directly
            ctx.wait(60_000)
            want = _oracle_outputs(ctx, b)
            for k in g_out:
                got = ctx.download(g_out[k])
                assert np.array_equal(got, want[k]), (replay, k, int(np.count_nonzero(got != want[k])))
                assert np.array_equal(ctx.download(e_out[k]), want[k]), (replay, k, "direct")
            # the replay really used the new inputs: outputs change with the seed
            if replay == 0:
                first = ctx.download(g_out["Y1"])
            else:
                assert not np.array_equal(first, ctx.download(g_out["Y1"]))
    finally:
        g.destroy()


def test_waits_and_allocations_are_refused_while_recording(ctx):
    buf = ctx.empty((4096,), np.int8)
    ref = ctx.empty((4096,), np.int8)
    host = np.zeros(4096, np.int8)
    with ctx.record() as g:
        ctx.fill_i8(buf, 4096, 77)
        assert ctx.call_status("miaie_copy_h2d", buf.ptr, host.ctypes.data, 4096) == mi.MIAIE_EINVAL
        assert "recorded" in ctx.last_error()
        assert ctx.call_status("miaie_copy_d2h", host.ctypes.data, buf.ptr, 4096) == mi.MIAIE_EINVAL
        assert ctx.call_status("miaie_wait", 0) == mi.MIAIE_EINVAL
        p = mi.C.c_void_p()
        assert ctx.call_status("miaie_alloc", mi.C.c_size_t(64), mi.C.byref(p)) == mi.MIAIE_EINVAL
        assert ctx.call_status("miaie_graph_begin") == mi.MIAIE_EINVAL   # no nesting
        # an invalid call is refused and records nothing
        assert ctx.call_status("miaie_gemm_i8_rq", None, None, None, 1, 1, 1, 10, 0, None, 0) == mi.MIAIE_EINVAL
    try:
        g.launch()
        ctx.fill_i8(ref, 4096, 77)
        ctx.wait(10_000)
        assert np.array_equal(ctx.download(buf), ctx.download(ref))
    finally:
        g.destroy()


def test_graph_replays_only_on_its_context(ctx):
    """A recorded chain may use its context's workspace (split-K conv), so
    another context of the same device may not replay it."""
    buf = ctx.empty((4096,), np.int8)
    with ctx.record() as g:
        ctx.fill_i8(buf, 4096, 5)
    other = mi.Context(ctx.device)
    try:
        assert other.call_status("miaie_graph_launch", g.handle) == mi.MIAIE_EINVAL
        assert "another context" in other.last_error()
        g.launch()  # its own context replays it
        ctx.wait(10_000)
    finally:
        g.destroy()
        other.close()


def test_graph_misuse(ctx):
    h = mi.C.c_void_p()
    assert ctx.call_status("miaie_graph_end", mi.C.byref(h)) == mi.MIAIE_EINVAL      # not recording
    assert ctx.call_status("miaie_graph_launch", None) == mi.MIAIE_EINVAL
    ctx._call("miaie_graph_begin")
    assert ctx.call_status("miaie_graph_end", mi.C.byref(h)) == mi.MIAIE_EINVAL      # empty recording
    assert "nothing was recorded" in ctx.last_error()
    assert ctx.lib.miaie_graph_destroy(None) == mi.MIAIE_OK
    # the context works normally afterwards
    buf = ctx.empty((256,), np.int8)
    ctx.fill_i8(buf, 256, 3)
    ctx.wait(10_000)
