"""Synthetic inputs for benchmarks and GGUF fixtures: the reference Rng and ggml quantisers.

* ``Rng`` restates the reference's SplitMix64 + Box-Muller generator (src/tensor.rs:155-199),
  vectorised: SplitMix64 output i depends only on ``seed ^ GAMMA`` + (i+1) * GAMMA, so a block of
  outputs is one numpy expression.  Integer streams and uniforms are bit-identical to the
  reference; normals use numpy's float32 ``log``/``cos`` and so may differ from the reference's
  libm in the last ulp.
* ``quantize_q4_0`` / ``quantize_q8_0`` follow ggml's reference quantisers (the ones GGUF
  writers use for these formats): Q4_0 maps the signed largest element of a 32-block to -8,
  codes ``min(15, trunc(x/d + 8.5))``; Q8_0 uses ``d = amax/127`` and rounds half away from zero.
  Scales are stored as IEEE half (round to nearest even).
"""
from __future__ import annotations

import numpy as np

GAMMA = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


class Rng:
    def __init__(self, seed: int):
        self.state = np.uint64(seed) ^ GAMMA

    def next_u64(self, n: int) -> np.ndarray:
        with np.errstate(over="ignore"):
            i = np.arange(1, n + 1, dtype=np.uint64)
            z = self.state + i * GAMMA
            self.state = self.state + np.uint64(n) * GAMMA
            z = (z ^ (z >> np.uint64(30))) * _M1
            z = (z ^ (z >> np.uint64(27))) * _M2
            return z ^ (z >> np.uint64(31))

    def uniform(self, n: int) -> np.ndarray:
        return (self.next_u64(n) >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24)

    def vec_normal(self, n: int, std: float) -> np.ndarray:
        u = self.uniform(2 * n).reshape(n, 2)
        u1 = np.maximum(u[:, 0], np.float32(1e-12))
        u2 = u[:, 1]
        two_pi = np.float32(2.0) * np.float32(np.pi)
        z = np.sqrt(np.float32(-2.0) * np.log(u1)) * np.cos(two_pi * u2)
        return (z.astype(np.float32) * np.float32(std)).astype(np.float32)


def _f16_bits(d: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return d.astype(np.float16).view(np.uint16)


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """[n x k] float32 -> uint8 [n, k/32*18] GGUF Q4_0 blocks."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    assert k % 32 == 0
    x = w.reshape(-1, 32)
    idx = np.argmax(np.abs(x), axis=1)
    mx = x[np.arange(x.shape[0]), idx]
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.minimum(15, (x * inv[:, None] + np.float32(8.5)).astype(np.int32)).astype(np.uint8)
    out = np.empty((x.shape[0], 18), dtype=np.uint8)
    out[:, 0:2] = _f16_bits(d).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q[:, :16] | (q[:, 16:] << 4)
    return out.reshape(n, k // 32 * 18)


def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """[n x k] float32 -> uint8 [n, k/32*34] GGUF Q8_0 blocks."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    assert k % 32 == 0
    x = w.reshape(-1, 32)
    amax = np.abs(x).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    v = (x * inv[:, None]).astype(np.float32).astype(np.float64)
    q = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int8)
    out = np.empty((x.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = _f16_bits(d).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(n, k // 32 * 34)


QUANTIZERS = {2: quantize_q4_0, 8: quantize_q8_0}
