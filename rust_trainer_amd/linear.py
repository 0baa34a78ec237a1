"""Frozen linear layer with an optional trainable LoRA adapter: ``y = W.x + b + (alpha/r) B.A.x``.

Mirrors ``src/linear.rs``: ``Lora`` (rank, alpha, a [r x in], b [out x r], ga, gb as host float32
vectors that an optimiser mutates in place) and ``Linear`` (name, w, bias, lora, lora_enabled).
When ``w`` is a :class:`HipFrozen`, the whole forward (frozen product, bias, LoRA down/up) and the
whole backward (dx, dA, dB) run on the GPU through ``rtq_linear_forward`` /
``rtq_linear_backward``; the LoRA tensors stay host arrays, as in the reference, and are uploaded
per call.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np

from . import _ffi
from .frozen import FrozenMatmul, HipFrozen


class Lora:
    """Trainable low-rank adapter (src/linear.rs:8-36). ``a`` is [r x in], ``b`` is [out x r]."""

    def __init__(self, rank: int, alpha: float, a: np.ndarray, b: np.ndarray):
        self.rank = int(rank)
        self.alpha = float(alpha)
        self.a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
        self.b = np.ascontiguousarray(b, dtype=np.float32).reshape(-1)
        self.ga = np.zeros_like(self.a)
        self.gb = np.zeros_like(self.b)

    @classmethod
    def new(cls, rank: int, alpha: float, inp: int, out: int, rng) -> "Lora":
        """PEFT-style init (src/linear.rs:21-25): A ~ U(-1/sqrt(in), 1/sqrt(in)), B = 0."""
        bound = np.float32(1.0) / np.float32(math.sqrt(inp))
        a = rng.vec_uniform_sym(rank * inp, float(bound))
        return cls(rank, alpha, a, np.zeros(out * rank, np.float32))

    def scale(self) -> float:
        return float(np.float32(self.alpha) / np.float32(self.rank))

    def zero_grad(self) -> None:
        self.ga[...] = 0.0
        self.gb[...] = 0.0

    def num_params(self) -> int:
        return self.a.size + self.b.size


class Linear:
    """src/linear.rs:38-122."""

    def __init__(self, name: str, w: FrozenMatmul, bias=None):
        if bias is not None:
            bias = np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
            assert bias.size == w.out_dim()
        self.name = name
        self.w = w
        self.bias = bias
        self.lora: Lora | None = None
        self.lora_enabled = True

    def in_dim(self) -> int:
        return self.w.in_dim()

    def out_dim(self) -> int:
        return self.w.out_dim()

    def attach_lora(self, rank: int, alpha: float, rng) -> None:
        self.lora = Lora.new(rank, alpha, self.in_dim(), self.out_dim(), rng)

    def active_lora(self) -> Lora | None:
        return self.lora if self.lora_enabled else None

    def _lora_view(self, l: Lora | None) -> _ffi.RtqLora | None:
        if l is None:
            return None
        assert l.a.size == l.rank * self.in_dim() and l.b.size == self.out_dim() * l.rank, "lora shapes"
        return _ffi.RtqLora(l.rank, l.alpha, l.a.ctypes.data, l.b.ctypes.data, 1)

    def forward(self, x, t: int) -> np.ndarray:
        """``x`` is [t x in]; returns [t x out] (flat)."""
        inp, out = self.in_dim(), self.out_dim()
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        assert x.size == t * inp, f"{self.name}: input shape"
        if isinstance(self.w, HipFrozen):
            y = np.empty(t * out, dtype=np.float32)
            lv = self._lora_view(self.active_lora())
            _ffi.check(_ffi.lib().rtq_linear_forward(
                self.w.ctx.handle, self.w.handle, None if self.bias is None else self.bias.ctypes.data,
                ctypes.byref(lv) if lv is not None else None, x.ctypes.data, t, y.ctypes.data), "rtq_linear_forward")
            return y
        raise TypeError("Linear on the GPU path needs a HipFrozen weight")

    def backward(self, x, dy, t: int) -> np.ndarray:
        """Back-propagates ``dy`` [t x out]; accumulates LoRA gradients; returns ``dx`` [t x in]."""
        inp, out = self.in_dim(), self.out_dim()
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        dy = np.ascontiguousarray(dy, dtype=np.float32).reshape(-1)
        assert dy.size == t * out
        assert x.size == t * inp
        if not isinstance(self.w, HipFrozen):
            raise TypeError("Linear on the GPU path needs a HipFrozen weight")
        dx = np.empty(t * inp, dtype=np.float32)
        l = self.lora if self.lora_enabled else None
        lv = self._lora_view(l)
        _ffi.check(_ffi.lib().rtq_linear_backward(
            self.w.ctx.handle, self.w.handle, ctypes.byref(lv) if lv is not None else None, x.ctypes.data,
            dy.ctypes.data, t, dx.ctypes.data, None if l is None else l.ga.ctypes.data,
            None if l is None else l.gb.ctypes.data), "rtq_linear_backward")
        return dx
