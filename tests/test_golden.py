"""Committed fixtures (tests/golden/golden.npz, written by numpy integer
arithmetic in tests/golden/make_golden.py) checked against the CPU oracle
(CPU) and against the gfx950 kernels through the C ABI (GPU); the recorded
synthetic inputs of the benchmark configurations (tests/golden/
synthetic_manifest.json) against the host generators (CPU) and the device
fill (GPU)."""
import hashlib
import json
import os

import numpy as np
import pytest

import oracle
from aiehlc_amd import synth

G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz"))


# ---------------------------------------------------------------- CPU: oracle vs fixtures
@pytest.mark.parametrize("name,n", [("mm16_i", 16), ("mm16_ip1", 16), ("mm8_i", 8)])
def test_oracle_window_fixtures(name, n):
    assert np.array_equal(oracle.mm_window_i32(G[f"{name}_in"], n), G[f"{name}_out"])


def test_window_fixture_holds_reference_known_answers():
    c = G["mm16_i_out"].reshape(16, 16)  # aieml_mm.cc inputs
    assert (c[0, 0], c[0, 1], c[1, 0], c[15, 15]) == (31960, 33880, 99416, 1994200)
    c = G["mm16_ip1_out"].reshape(16, 16)  # aieml_perf.cc inputs
    assert (c[0, 0], c[15, 15]) == (36312, 2006232)


def test_oracle_gemm_fixtures():
    Y, C = oracle.gemm_i8_rq(G["gemm64_A"], G["gemm64_B"], 10, want_acc=True)
    assert np.array_equal(C, G["gemm64_C"]) and np.array_equal(Y, G["gemm64_Y10"])
    Y, C = oracle.gemm_i8_rq(G["ragged_A"], G["ragged_B"], 9, relu=True, want_acc=True)
    assert np.array_equal(C, G["ragged_C"]) and np.array_equal(Y, G["ragged_Y9r"])


def test_oracle_conv_and_mlp_fixtures():
    assert np.array_equal(oracle.conv2d_nhwc_i8(G["conv_X"], G["conv_W"], G["conv_shifts"], 1, 1), G["conv_Y"])
    Y, H = oracle.mlp_i8(G["mlp_X"], G["mlp_W1"], G["mlp_W2"], 11, 12, want_h=True)
    assert np.array_equal(H, G["mlp_H"]) and np.array_equal(Y, G["mlp_Y"])


# ------------------------------------------------- CPU: the benchmark's synthetic inputs
MANIFEST = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                                       "synthetic_manifest.json")))


def _sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _int8_entries():
    for c, tensors in sorted(MANIFEST["configs"].items()):
        for name, t in sorted(tensors.items()):
            if isinstance(t, dict) and t.get("dtype") == "int8":
                yield c, name, t


@pytest.mark.parametrize("c,name,t", list(_int8_entries()), ids=lambda v: v if isinstance(v, str) else "")
def test_synthetic_int8_inputs_match_the_manifest(c, name, t):
    """The numpy generator and the C oracle's generator both reproduce the
    recorded bytes of every int8 benchmark input (tests/golden/make_manifest.py)."""
    shape = tuple(t["shape"])
    assert _sha(synth.int8(shape, t["stream"])) == t["sha256"], (c, name)
    if int(np.prod(shape)) <= (1 << 24):
        assert _sha(oracle.fill_i8(int(np.prod(shape)), t["stream"])) == t["sha256"], (c, name)


def test_synthetic_shifts_and_bf16_match_the_manifest():
    cfg = MANIFEST["configs"]
    assert synth.shifts(64, 7).tolist() == cfg["4"]["shifts"]["values"]
    assert oracle.fill_shift(64, 7).tolist() == cfg["4"]["shifts"]["values"]
    for name, sid in (("A", 1), ("B", 2)):
        assert synth.bf16_normal((16,), sid, 1.0 / np.sqrt(8192)).tolist() == cfg["3"][name]["first16_bits"]


# ---------------------------------------------------------------- GPU: kernels vs fixtures
@pytest.mark.gpu
@pytest.mark.parametrize("name,n", [("mm16_i", 16), ("mm16_ip1", 16), ("mm8_i", 8)])
def test_gpu_window_fixtures(ctx, name, n):
    print("[case] golden window", name, flush=True)
    d_in = ctx.upload(G[f"{name}_in"])
    d_out = ctx.empty((n * n,), np.int32)
    ctx.mm_window_i32(d_in, d_out, n)
    ctx.wait(10_000)
    assert np.array_equal(ctx.download(d_out), G[f"{name}_out"])


@pytest.mark.gpu
@pytest.mark.parametrize("case,shift,relu", [("gemm64", 10, False), ("ragged", 9, True)])
def test_gpu_gemm_fixtures(ctx, case, shift, relu):
    print("[case] golden gemm", case, flush=True)
    A, B = G[f"{case}_A"], G[f"{case}_B"]
    M, K = A.shape
    N = B.shape[1]
    dA, dB = ctx.upload(A), ctx.upload(B)
    dY, dC = ctx.empty((M, N), np.int8), ctx.empty((M, N), np.int32)
    ctx.gemm_i8_rq(dA, dB, dY, M, N, K, shift, relu, dC)
    ctx.wait(10_000)
    Ywant = G["gemm64_Y10"] if case == "gemm64" else G["ragged_Y9r"]
    assert np.array_equal(ctx.download(dC), G[f"{case}_C"])
    assert np.array_equal(ctx.download(dY), Ywant)


@pytest.mark.gpu
def test_gpu_conv_and_mlp_fixtures(ctx):
    print("[case] golden conv + mlp", flush=True)
    X, W, sh = G["conv_X"], G["conv_W"], G["conv_shifts"]
    dX, dW, dS, dY = ctx.upload(X), ctx.upload(W), ctx.upload(sh), ctx.empty(G["conv_Y"].shape, np.int8)
    ctx.conv2d_i8_nhwc(dX, dW, dS, dY, 1, 6, 6, 32, 64, 3, 3, 1, 1)
    ctx.wait(10_000)
    assert np.array_equal(ctx.download(dY), G["conv_Y"])
    X, W1, W2 = G["mlp_X"], G["mlp_W1"], G["mlp_W2"]
    dX, d1, d2 = ctx.upload(X), ctx.upload(W1), ctx.upload(W2)
    dH, dYm = ctx.empty(G["mlp_H"].shape, np.int8), ctx.empty(G["mlp_Y"].shape, np.int8)
    ctx.mlp_i8(dX, d1, d2, dH, dYm, 8, 64, 96, 32, 11, 12)
    ctx.wait(10_000)
    assert np.array_equal(ctx.download(dH), G["mlp_H"])
    assert np.array_equal(ctx.download(dYm), G["mlp_Y"])


@pytest.mark.gpu
def test_gpu_fill_matches_the_manifest(ctx):
    """miaie_fill_i8 on the device writes the recorded bytes of config 2's A
    and B and config 4's X and W, the inputs bench.py generates on the device."""
    print("[case] device fill vs manifest", flush=True)
    cfg = MANIFEST["configs"]
    for c, name in (("2", "A"), ("2", "B"), ("4", "X"), ("4", "W")):
        t = cfg[c][name]
        n = int(np.prod(t["shape"]))
        d = ctx.empty((n,), np.int8)
        ctx.fill_i8(d, n, t["stream"])
        ctx.wait(10_000)
        assert _sha(ctx.download(d)) == t["sha256"], (c, name)
        d.free()
