"""Seeded synthetic inputs for the benchmark shapes (numpy, host side).

SplitMix64 (Steele, Lea & Flood, 2014) is counter based: draw i of a stream
whose state starts at s0 is mix(s0 + (i+1)*gamma), so whole tensors are
generated with vectorised uint64 arithmetic.  Tensor streams start at
s0 = mix(0x5EED0000 + tensor_id + gamma).  Tensor ids: A=1, B=2, X=3, W=4,
W1=5, W2=6, shifts=7.

  int8   : (int8)(draw >> 56), uniform over [-128, 127]
  shift  : 8 + (draw >> 32) % 5, uniform over [8, 12]
  bf16   : N(0,1)*scale by Box-Muller (z0 of draws 2i, 2i+1 on 53-bit
           uniforms), rounded to bf16 with round-to-nearest-even

miaie_fill_i8 on the device produces the same int8 bytes.
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
TENSOR_IDS = {"A": 1, "B": 2, "X": 3, "W": 4, "W1": 5, "W2": 6, "shifts": 7}


def _mix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def tensor_seed(tensor_id: int) -> np.uint64:
    with np.errstate(over="ignore"):
        return _mix(np.array([0x5EED0000 + tensor_id], dtype=np.uint64) + GAMMA)[0]


def draws(tensor_id: int, n: int, start: int = 0) -> np.ndarray:
    """Raw 64-bit draws start .. start+n-1 of the tensor's stream."""
    s0 = tensor_seed(tensor_id)
    idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        return _mix(s0 + idx * GAMMA)


def int8(shape, tensor_id: int, chunk: int = 1 << 24) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.int8)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        out[s:e] = (draws(tensor_id, e - s, s) >> np.uint64(56)).astype(np.uint8).view(np.int8)
    return out.reshape(shape)


def shifts(n: int, tensor_id: int = 7) -> np.ndarray:
    return (np.uint64(8) + (draws(tensor_id, n) >> np.uint64(32)) % np.uint64(5)).astype(np.uint8)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (NaNs kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & np.uint32(0x7F800000)) == np.uint32(0x7F800000)
    nan &= (u & np.uint32(0x007FFFFF)) != 0
    lsb = (u >> np.uint32(16)) & np.uint32(1)
    with np.errstate(over="ignore"):
        r = ((u + np.uint32(0x7FFF) + lsb) >> np.uint32(16)).astype(np.uint16)
    r[nan] = ((u[nan] >> np.uint32(16)) | np.uint32(0x40)).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def bf16_normal(shape, tensor_id: int, scale: float, chunk: int = 1 << 23) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16)
    two53 = 1.0 / 9007199254740992.0
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        d = draws(tensor_id, 2 * (e - s), 2 * s)
        u1 = ((d[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * two53
        u2 = (d[1::2] >> np.uint64(11)).astype(np.float64) * two53
        z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
        out[s:e] = f32_to_bf16_bits((z * scale).astype(np.float32))
    return out.reshape(shape)
