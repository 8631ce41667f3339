"""Writes tests/golden/synthetic_manifest.json: the seeded synthetic inputs of
the five benchmark configurations (the bytes bench.py measures on), recorded
as shapes, generator streams and SHA-256 digests of the generated int8
tensors, so that a change to the generator or to a stream assignment shows
up as a test failure.  Run from the repository root:

    python tests/golden/make_manifest.py

The generator (aiehlc_amd/synth.py; miaie_fill_i8 on the device produces the
same int8 bytes) is SplitMix64: draw i of tensor t is
mix(s0 + (i+1)*gamma) with s0 = mix(0x5EED0000 + t + gamma); int8 values are
(int8)(draw >> 56), shifts 8 + (draw >> 32) % 5, bf16 values N(0,1)*scale by
Box-Muller on 53-bit uniforms rounded to nearest even.  bf16 tensors are
recorded by their first 16 bit patterns (the full tensors are 128 MiB each).
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from aiehlc_amd import synth  # noqa: E402

OUT = os.path.join(HERE, "synthetic_manifest.json")

# (config, tensor name, shape, stream id); all int8
INT8 = [
    ("1", "A", (64, 64), 1), ("1", "B", (64, 64), 2),
    ("2", "A", (4096, 4096), 1), ("2", "B", (4096, 4096), 2),
    ("4", "X", (8, 56, 56, 64), 3), ("4", "W", (64, 3, 3, 64), 4),
    ("5", "X", (2048, 4096), 3), ("5", "W1", (4096, 11008), 5), ("5", "W2", (11008, 4096), 6),
]
BF16 = [("3", "A", (8192, 8192), 1), ("3", "B", (8192, 8192), 2)]
EXTRA = {"1": {"layout": "NN", "out": "int32 C, Y = requant(C, 10)"},
         "2": {"layout": "NN", "shift": 10, "out": "int8 Y (int32 C on the debug launch)"},
         "3": {"layout": "NN", "scale": "1/sqrt(8192)", "out": "fp32 C"},
         "4": {"stride": 1, "pad": 1, "layout": "NHWC x OHWI", "out": "int8 Y[8][56][56][64]"},
         "5": {"s1": 11, "s2": 12, "relu": "after requant s1", "out": "int8 H[2048][11008], Y[2048][4096]"}}


def sha256(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def build() -> dict:
    man = {"generator": "SplitMix64 streams, aiehlc_amd/synth.py (see the docstring of tests/golden/make_manifest.py)",
           "configs": {}}
    cfg = man["configs"]
    for c, name, shape, sid in INT8:
        cfg.setdefault(c, dict(EXTRA[c]))[name] = {"shape": list(shape), "dtype": "int8", "stream": sid,
                                                     "sha256": sha256(synth.int8(shape, sid))}
    cfg["4"]["shifts"] = {"shape": [64], "dtype": "uint8", "stream": 7, "values": synth.shifts(64, 7).tolist()}
    for c, name, shape, sid in BF16:
        first = synth.bf16_normal((16,), sid, 1.0 / np.sqrt(8192))
        cfg.setdefault(c, dict(EXTRA[c]))[name] = {"shape": list(shape), "dtype": "bf16", "stream": sid,
                                                     "first16_bits": [int(v) for v in first]}
    return man


if __name__ == "__main__":
    with open(OUT, "w") as f:
        json.dump(build(), f, indent=1, sort_keys=True)
        f.write("\n")
    print("wrote", OUT)
