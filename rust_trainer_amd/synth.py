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
* ``quantize_q4_k`` / ``quantize_q6_k`` are valid K-quant encoders (ggml's search-based encoder is
  not restated); every consumer reads the bytes they produce, so parity does not depend on them.
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


def _rne(v: np.ndarray) -> np.ndarray:
    """nearest integer, ties to even (ggml's nearest_int)"""
    return np.rint(v).astype(np.int32)


def quantize_q4_k(w: np.ndarray) -> np.ndarray:
    """[n x k] float32 -> uint8 [n, k/256*144] GGUF Q4_K super-blocks.

    A valid (not ggml's search-based) encoder: per 32-element sub-block the affine fit
    x ~ (d*sc)*q - dmin*m with q in [0, 15] spanning [min(x, 0), max(x)]; the super-block d, dmin
    map the largest sub-block scale / min to 63 (6-bit sc, m); q = nearest((x + dmin*m) / (d*sc)).
    """
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    assert k % 256 == 0
    x = w.reshape(-1, 8, 32)
    f = np.float32
    mn = np.minimum(x.min(axis=2), f(0.0))
    mx = x.max(axis=2)
    scale = ((mx - mn) / f(15.0)).astype(f)
    mins = (-mn).astype(f)
    max_scale = np.maximum(scale.max(axis=1), f(0.0))
    max_min = np.maximum(mins.max(axis=1), f(0.0))
    dh = (max_scale / f(63.0)).astype(np.float16)
    mh = (max_min / f(63.0)).astype(np.float16)
    d, dmin = dh.astype(f), mh.astype(f)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(d[:, None] > 0, _rne(scale / d[:, None]), 0).clip(0, 63)
        m = np.where(dmin[:, None] > 0, _rne(mins / dmin[:, None]), 0).clip(0, 63)
        es = (d[:, None] * sc.astype(f)).astype(f)
        em = (dmin[:, None] * m.astype(f)).astype(f)
        q = np.where(es[:, :, None] > 0, _rne(((x + em[:, :, None]).astype(f) / es[:, :, None]).astype(f)), 0)
    q = q.clip(0, 15).astype(np.uint8)
    out = np.zeros((x.shape[0], 144), dtype=np.uint8)
    out[:, 0:2] = dh.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = mh.view(np.uint8).reshape(-1, 2)
    sc8, m8 = sc.astype(np.uint8), m.astype(np.uint8)
    out[:, 4:8] = (sc8[:, :4] & 63) | ((sc8[:, 4:] >> 4) << 6)
    out[:, 8:12] = (m8[:, :4] & 63) | ((m8[:, 4:] >> 4) << 6)
    out[:, 12:16] = (sc8[:, 4:] & 0xF) | ((m8[:, 4:] & 0xF) << 4)
    L = q.reshape(-1, 4, 2, 32)  # [chunk c][half][l]: elements 64c + 32 half + l
    out[:, 16:] = (L[:, :, 0, :] | (L[:, :, 1, :] << 4)).reshape(-1, 128)
    return out.reshape(n, k // 256 * 144)


def quantize_q6_k(w: np.ndarray) -> np.ndarray:
    """[n x k] float32 -> uint8 [n, k/256*210] GGUF Q6_K super-blocks.

    A valid encoder: per 16-element sub-block the signed element of largest |x| (first on ties)
    maps to -32; the sub-block scales are int8 against a super-block d that maps the
    largest-magnitude scale to -128 (clamped to [-128, 127]); q = nearest(x / (d*sc)) in [-32, 31].
    """
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    assert k % 256 == 0
    f = np.float32
    x = w.reshape(-1, 16, 16)
    nsb = x.shape[0]
    idx = np.argmax(np.abs(x), axis=2)
    mx = np.take_along_axis(x, idx[:, :, None], axis=2)[:, :, 0]
    scl = (mx / f(-32.0)).astype(f)
    j = np.argmax(np.abs(scl), axis=1)
    max_scale = scl[np.arange(nsb), j]
    nz = np.abs(max_scale) > 0
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        iscale = np.where(nz, f(-128.0) / np.where(nz, max_scale, f(1.0)), f(0.0)).astype(f)
        dh = np.where(nz, (f(1.0) / np.where(nz, iscale, f(1.0))).astype(f), f(0.0)).astype(np.float16)
        d = dh.astype(f)
        scales = np.where(nz[:, None], _rne((iscale[:, None] * scl).astype(f)), 0).clip(-128, 127)
        es = (d[:, None] * scales.astype(f)).astype(f)
        q = np.where(es[:, :, None] != 0, _rne((x / np.where(es != 0, es, f(1.0))[:, :, None]).astype(f)), 0)
    L = (q.clip(-32, 31) + 32).astype(np.uint8).reshape(-1, 2, 4, 32)  # [half h][quarter][l]
    out = np.zeros((nsb, 210), dtype=np.uint8)
    q1, q2, q3, q4 = L[:, :, 0], L[:, :, 1], L[:, :, 2], L[:, :, 3]
    ql = np.concatenate([(q1 & 0xF) | ((q3 & 0xF) << 4), (q2 & 0xF) | ((q4 & 0xF) << 4)], axis=2)  # [h][64]
    qh = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    out[:, 0:128] = ql.reshape(-1, 128)
    out[:, 128:192] = qh.reshape(-1, 64)
    out[:, 192:208] = scales.astype(np.int8).view(np.uint8)
    out[:, 208:210] = dh.view(np.uint8).reshape(-1, 2)
    return out.reshape(n, k // 256 * 210)


QUANTIZERS = {2: quantize_q4_0, 8: quantize_q8_0, 12: quantize_q4_k, 14: quantize_q6_k}
