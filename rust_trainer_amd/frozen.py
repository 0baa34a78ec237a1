"""Frozen quantised weights on the GPU — the ``FrozenMatmul`` plugin point.

Mirrors the reference's contract (``src/frozen.rs:13-27``) and its GGUF implementation
``RieFrozen`` (``src/rie.rs:50-129``): the frozen weight provides only the forward product
``y = x . W^T`` (fresh output) and the input gradient ``dx += dy . W`` (accumulated), plus
``row`` (dequantise one row) and ``nbytes``.  Arrays are row-major float32; like ``&[f32]`` /
``Vec<f32>`` in the reference, inputs may be flat or 2-D and outputs are flat.

``HipFrozen`` keeps the packed GGUF blocks on the device (uploaded once) and runs the gfx950
kernels of librtq.so.  Shape errors raise ``AssertionError`` where the reference asserts;
device failures raise ``RtqError``.
"""
from __future__ import annotations

import abc
import ctypes
import weakref

import numpy as np

from . import _ffi


class Context:
    """One device, one stream, the loaded gfx950 code object (``rtq_ctx``).

    Replaces the engine ThreadPool the reference threads through ``RieFrozen``
    (``src/rie.rs:53,182``).
    """

    def __init__(self, device: int = 0):
        L = _ffi.lib()
        h = ctypes.c_void_p()
        _ffi.check(L.rtq_ctx_create(device, ctypes.byref(h)), "rtq_ctx_create")
        self._h = h
        self.device = device
        # weights and models created on this context, closed before it (a model or weight that
        # outlives its context - held by a traceback, say - must not reach the freed context later)
        self._owned: weakref.WeakSet = weakref.WeakSet()

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("context destroyed")
        return self._h

    @property
    def stream(self) -> int:
        return int(_ffi.lib().rtq_ctx_stream(self.handle) or 0)

    def reserve(self, max_t: int, max_rows: int, max_cols: int, max_rank: int = 0) -> None:
        _ffi.check(_ffi.lib().rtq_ctx_reserve(self.handle, max_t, max_rows, max_cols, max_rank), "rtq_ctx_reserve")

    def set_timing(self, on: bool, only_kernel: str | None = None) -> None:
        """HIP events around kernel launches (all kernels, or only ``only_kernel``)."""
        _ffi.check(_ffi.lib().rtq_ctx_set_timing(self.handle, int(on), only_kernel.encode() if only_kernel else None),
                   "rtq_ctx_set_timing")

    def timing(self) -> dict[str, tuple[int, float]]:
        """{kernel name: (launches, total ms)} for kernels launched since the last reset."""
        L = _ffi.lib()
        n = L.rtq_ctx_timing_count(self.handle)
        out = {}
        for i in range(n):
            name = ctypes.c_char_p()
            cnt = ctypes.c_int64()
            ms = ctypes.c_double()
            _ffi.check(L.rtq_ctx_timing_get(self.handle, i, ctypes.byref(name), ctypes.byref(cnt), ctypes.byref(ms)),
                       "rtq_ctx_timing_get")
            if cnt.value:
                out[name.value.decode()] = (cnt.value, ms.value)
        return out

    def timing_work(self) -> dict[str, tuple[float, float]]:
        """{kernel name: (flops, bytes)}: the algorithmic work of the timed launches (frozen-linear
        kernels; see rtq_ctx_timing_work)."""
        L = _ffi.lib()
        out = {}
        for i in range(L.rtq_ctx_timing_count(self.handle)):
            name = ctypes.c_char_p()
            cnt = ctypes.c_int64()
            ms = ctypes.c_double()
            fl, by = ctypes.c_double(), ctypes.c_double()
            _ffi.check(L.rtq_ctx_timing_get(self.handle, i, ctypes.byref(name), ctypes.byref(cnt), ctypes.byref(ms)),
                       "rtq_ctx_timing_get")
            _ffi.check(L.rtq_ctx_timing_work(self.handle, i, ctypes.byref(fl), ctypes.byref(by)), "rtq_ctx_timing_work")
            if cnt.value and fl.value:
                out[name.value.decode()] = (fl.value, by.value)
        return out

    def reset_timing(self) -> None:
        _ffi.lib().rtq_ctx_timing_reset(self.handle)

    def close(self) -> None:
        """Destroys the weights and models still alive on this context, then the context itself."""
        if self._h is not None:
            for w in list(self._owned):
                w.close()
            _ffi.lib().rtq_ctx_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


_DEFAULT_CTX: Context | None = None


def default_context() -> Context:
    global _DEFAULT_CTX
    if _DEFAULT_CTX is None:
        _DEFAULT_CTX = Context(0)
    return _DEFAULT_CTX


def _f32(a, n: int, what: str) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    assert a.size == n, f"{what}: expected {n} elements, got {a.size}"
    return a


class FrozenMatmul(abc.ABC):
    """A frozen ``[out x in]`` weight matrix (``trait FrozenMatmul``, src/frozen.rs:14-25)."""

    @abc.abstractmethod
    def out_dim(self) -> int: ...

    @abc.abstractmethod
    def in_dim(self) -> int: ...

    @abc.abstractmethod
    def forward(self, x, t: int) -> np.ndarray:
        """``y[t x out] = x[t x in] . W^T``"""

    @abc.abstractmethod
    def backward_input(self, dy, t: int, dx: np.ndarray) -> None:
        """``dx[t x in] += dy[t x out] . W`` (gradient to the input only; W is frozen)."""

    @abc.abstractmethod
    def row(self, r: int, out: np.ndarray) -> None:
        """Dequantise one row into ``out``."""

    @abc.abstractmethod
    def nbytes(self) -> int: ...


def pack_trainer_q8_0(w, out: int, inp: int) -> np.ndarray:
    """FrozenWeight::q8_0's quantiser (src/frozen.rs:53-73) into the TYPE_TQ8_0 packing: per
    32-element block d = amax / 127 (f32), q = round(x / d) with halves away from zero (Rust
    f32::round), clamped to +-127; the scales [out x inp/32] (f32) then the codes (i8), as bytes."""
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(out, inp)
    assert inp % 32 == 0, "TQ8_0 needs whole 32-element blocks"
    blk = w.reshape(-1, 32)
    amax = np.abs(blk).max(axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.zeros_like(d)
    nz = d > 0
    inv[nz] = np.float32(1.0) / d[nz]
    v = blk * inv[:, None]                       # f32 products, as x * id in the reference
    tr = np.trunc(v)
    q = tr + np.where(np.abs(v - tr) >= np.float32(0.5), np.sign(v), np.float32(0.0))  # exact half-away rounding
    q = np.clip(q, -127.0, 127.0).astype(np.int8)
    return np.concatenate([d.view(np.uint8), q.reshape(-1).view(np.uint8)])


class HipFrozen(FrozenMatmul):
    """Frozen weight on an MI355X (``RieFrozen::new``, src/rie.rs:58-60; ``FrozenWeight``,
    src/frozen.rs:33-75).

    ``blocks`` are the weight's packed bytes: GGUF blocks (``Weight::data()``) for Q4_0 (2), Q8_0 (8),
    Q4_K (12), Q6_K (14); a float32 [rows x cols] array for F32 (0); the ``pack_trainer_q8_0``
    bytes for the trainer-native Q8_0 with f32 scales (TYPE_TQ8_0).  ``rows`` = out, ``cols`` = in.
    """

    @classmethod
    def f32(cls, w, out: int, inp: int, ctx: Context | None = None) -> "HipFrozen":
        """``FrozenWeight::f32`` (src/frozen.rs:48-51)."""
        w = np.ascontiguousarray(w, dtype=np.float32)
        assert w.size == out * inp, "weight shape mismatch"
        return cls(_ffi.TYPE_F32, w, out, inp, ctx=ctx)

    @classmethod
    def q8_0(cls, w, out: int, inp: int, ctx: Context | None = None) -> "HipFrozen":
        """``FrozenWeight::q8_0`` (src/frozen.rs:53-73): quantised when ``inp`` is a multiple of 32,
        else kept f32."""
        w = np.ascontiguousarray(w, dtype=np.float32)
        assert w.size == out * inp
        if inp % 32:
            return cls.f32(w, out, inp, ctx=ctx)
        return cls(_ffi.TYPE_TQ8_0, pack_trainer_q8_0(w, out, inp), out, inp, ctx=ctx)

    @classmethod
    def from_gguf(cls, file, name: str, ctx: Context | None = None) -> "HipFrozen":
        """Uploads GGUF tensor ``name`` of an open ``gguf.GgufFile`` straight from the mapped
        image (the loader's ``fz(&l.wq)``, src/rie.rs:183, :218-231)."""
        t = file.tensor(name)
        assert t is not None, f"no tensor {name}"
        self = cls.__new__(cls)
        self.ctx = ctx or default_context()
        h = ctypes.c_void_p()
        _ffi.check(_ffi.lib().rtq_weight_from_gguf(self.ctx.handle, file.handle, name.encode(), ctypes.byref(h)),
                   "rtq_weight_from_gguf")
        self._adopt(h, t.ty, t.n_rows(), t.row_len())
        return self

    def __init__(self, ggml_type: int, blocks, rows: int, cols: int, ctx: Context | None = None):
        self.ctx = ctx or default_context()
        arr = np.ascontiguousarray(blocks)
        b = arr.view(np.uint8).reshape(-1) if arr.dtype != np.uint8 else arr  # bytes as they are
        h = ctypes.c_void_p()
        _ffi.check(_ffi.lib().rtq_weight_create(self.ctx.handle, ggml_type, b.ctypes.data, b.nbytes, rows, cols,
                                                ctypes.byref(h)), "rtq_weight_create")
        self._adopt(h, ggml_type, rows, cols)

    def _adopt(self, h: ctypes.c_void_p, ggml_type: int, rows: int, cols: int) -> None:
        self._h = h
        self.ggml_type = ggml_type
        self._rows, self._cols = rows, cols
        self.ctx._owned.add(self)

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def out_dim(self) -> int:
        return self._rows

    def in_dim(self) -> int:
        return self._cols

    def nbytes(self) -> int:
        return int(_ffi.lib().rtq_weight_nbytes(self._h))

    def forward(self, x, t: int) -> np.ndarray:
        x = _f32(x, t * self._cols, "forward input")
        y = np.empty(t * self._rows, dtype=np.float32)
        _ffi.check(_ffi.lib().rtq_frozen_forward(self.ctx.handle, self._h, x.ctypes.data, t, y.ctypes.data),
                   "rtq_frozen_forward")
        return y

    def backward_input(self, dy, t: int, dx: np.ndarray) -> None:
        dy = _f32(dy, t * self._rows, "backward dy")
        assert isinstance(dx, np.ndarray) and dx.dtype == np.float32 and dx.flags["C_CONTIGUOUS"], \
            "dx must be a C-contiguous float32 array (accumulated in place)"
        assert dx.size == t * self._cols, f"dx: expected {t * self._cols} elements, got {dx.size}"
        _ffi.check(_ffi.lib().rtq_frozen_backward_input(self.ctx.handle, self._h, dy.ctypes.data, t, dx.ctypes.data),
                   "rtq_frozen_backward_input")

    def row(self, r: int, out: np.ndarray) -> None:
        assert isinstance(out, np.ndarray) and out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
        assert out.size == self._cols
        _ffi.check(_ffi.lib().rtq_frozen_row(self.ctx.handle, self._h, r, out.ctypes.data), "rtq_frozen_row")

    # ---- device-pointer variants (ints are device addresses; stream 0 = the HIP null stream)
    def forward_d(self, x_ptr: int, t: int, y_ptr: int, stream: int = 0) -> None:
        _ffi.check(_ffi.lib().rtq_frozen_forward_d(self.ctx.handle, self._h, x_ptr, t, y_ptr, stream or None),
                   "rtq_frozen_forward_d")

    def backward_input_d(self, dy_ptr: int, t: int, dx_ptr: int, stream: int = 0) -> None:
        _ffi.check(_ffi.lib().rtq_frozen_backward_input_d(self.ctx.handle, self._h, dy_ptr, t, dx_ptr,
                                                          stream or None), "rtq_frozen_backward_input_d")

    def rows_d(self, r0: int, count: int, out_ptr: int, stream: int = 0) -> None:
        _ffi.check(_ffi.lib().rtq_frozen_rows_d(self.ctx.handle, self._h, r0, count, out_ptr, stream or None),
                   "rtq_frozen_rows_d")

    # ---- parity hooks
    def debug_quantize_acts(self, x, t: int) -> np.ndarray:
        """The activation blocks (ggml layout) the GPU forward uses for ``x``."""
        x = _f32(x, t * self._cols, "acts")
        per = {2: 34 * (self._cols // 32), 8: 34 * (self._cols // 32)}.get(self.ggml_type,
                                                                            292 * (self._cols // 256))
        out = np.empty((t, per), dtype=np.uint8)
        _ffi.check(_ffi.lib().rtq_debug_quantize_acts(self.ctx.handle, self._h, x.ctypes.data, t, out.ctypes.data),
                   "rtq_debug_quantize_acts")
        return out

    def debug_block_isums(self, x, t: int) -> np.ndarray:
        """Integer block sums computed by the GPU forward kernel: int32 [t, out, isums_per_row]."""
        x = _f32(x, t * self._cols, "acts")
        m = int(_ffi.lib().rtq_debug_isums_per_row(self._h))
        out = np.empty((t, self._rows, m), dtype=np.int32)
        _ffi.check(_ffi.lib().rtq_debug_block_isums(self.ctx.handle, self._h, x.ctypes.data, t, out.ctypes.data),
                   "rtq_debug_block_isums")
        return out

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            _ffi.lib().rtq_weight_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
