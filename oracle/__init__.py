"""CPU oracle for the frozen quantised-matmul path (TEST INFRASTRUCTURE ONLY).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
this package, and only as the checker or the timed CPU baseline.  The product library
(``rust_trainer_amd``) never imports it and has no CPU fallback.

It wraps ``oracle/liboracle.so`` (built from ``rtq_oracle.c`` by ``oracle/Makefile``), a C
restatement of the reference's CPU path:

* ``src/frozen.rs:14-25`` FrozenMatmul contract; ``src/rie.rs:74-124`` RieFrozen forward
  (activation quantisation + integer block dots), backward_input (32-row dequant + axpy),
  row (dequant_row);
* ``src/linear.rs:73-121`` Linear LoRA forward/backward; ``src/tensor.rs:24-120`` primitives;
* ``src/tensor.rs:155-199`` Rng;
* ggml block semantics for Q4_0 / Q8_0 / Q4_K / Q6_K weights and Q8_0 / Q8_K activations
  (rie-core, pinned at f3be365b41f929cc81ee08afaa994d02bbeee2f5 in Cargo.lock:529-540, is
  absent from the container; parity against it is unpinned).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K = 0, 1, 2, 8, 12, 14, 15
# not a ggml type: the trainer-native FrozenWeight::Q8_0 (src/frozen.rs:38-45), f32 scale per 32
# elements, packed as scales [n][k/32] (f32) then codes [n][k] (i8)
TQ8_0 = 264
TYPE_NAMES = {F32: "F32", F16: "F16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K", Q8_K: "Q8_K",
              TQ8_0: "TQ8_0"}
BLOCK_ELEMS = {F32: 1, F16: 1, Q4_0: 32, Q8_0: 32, Q4_K: 256, Q6_K: 256, Q8_K: 256}
BLOCK_BYTES = {F32: 4, F16: 2, Q4_0: 18, Q8_0: 34, Q4_K: 144, Q6_K: 210, Q8_K: 292}

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_f = ctypes.c_float
_i = ctypes.c_int


class OrLinear(ctypes.Structure):
    _fields_ = [("wtype", ctypes.c_int), ("w", ctypes.c_void_p), ("out", ctypes.c_int64), ("in_", ctypes.c_int64),
                ("bias", ctypes.c_void_p), ("rank", ctypes.c_int64), ("alpha", ctypes.c_float),
                ("A", ctypes.c_void_p), ("B", ctypes.c_void_p), ("ga", ctypes.c_void_p), ("gb", ctypes.c_void_p)]


class OrLayer(ctypes.Structure):
    _fields_ = [("attn_norm", ctypes.c_void_p), ("ffn_norm", ctypes.c_void_p), ("q_norm", ctypes.c_void_p),
                ("k_norm", ctypes.c_void_p)] + [(n, OrLinear) for n in ("q", "k", "v", "o", "gate", "up", "down")]


class OrModel(ctypes.Structure):
    _fields_ = [("n_layer", ctypes.c_int), ("d", ctypes.c_int64), ("n_head", ctypes.c_int64),
                ("n_kv", ctypes.c_int64), ("hd", ctypes.c_int64), ("rot", ctypes.c_int64), ("n_ff", ctypes.c_int64),
                ("eps", ctypes.c_float), ("off", ctypes.c_float), ("theta", ctypes.c_float),
                ("freq_scale", ctypes.c_float), ("neox", ctypes.c_int), ("kv_f16", ctypes.c_int),
                ("embed", OrLinear), ("lm_head", OrLinear), ("out_norm", ctypes.c_void_p),
                ("layers", ctypes.POINTER(OrLayer)), ("rope_factors", ctypes.c_void_p), ("n_factors", ctypes.c_int64)]


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            raise RuntimeError(f"{path} is not built; run __graft_entry__.build() (or make -C oracle)")
        L = ctypes.CDLL(path)
        sig = {
            "or_rng_seed": (ctypes.c_uint64, [ctypes.c_uint64]),
            "or_rng_next_u64": (ctypes.c_uint64, [_p]),
            "or_rng_uniform": (_f, [_p]),
            "or_rng_normal": (_f, [_p]),
            "or_rng_fill_normal": (None, [_p, _p, _i64, _f]),
            "or_rng_fill_uniform_sym": (None, [_p, _p, _i64, _f]),
            "or_fp32_to_fp16": (ctypes.c_uint16, [_f]),
            "or_fp16_to_fp32": (_f, [ctypes.c_uint16]),
            "or_row_bytes": (_i64, [_i, _i64]),
            "or_quantize": (_i, [_i, _p, _i64, _p]),
            "or_tq8_quantize": (_i, [_p, _i64, _i64, _p]),
            "or_dequant_row": (_i, [_i, _p, _i64, _p]),
            "or_act_type_for": (_i, [_i]),
            "or_quantize_acts_q8_0": (None, [_p, _i64, _p]),
            "or_quantize_acts_q8_k": (None, [_p, _i64, _p]),
            "or_isums_per_row": (_i64, [_i, _i64]),
            "or_block_isums": (_i, [_i, _p, _p, _i64, _p]),
            "or_frozen_forward": (_i, [_i, _p, _i64, _i64, _p, _i64, _p, _i]),
            "or_frozen_forward_f64": (_i, [_i, _p, _i64, _i64, _p, _i64, _p]),
            "or_frozen_backward_input": (_i, [_i, _p, _i64, _i64, _p, _i64, _p, _i]),
            "or_frozen_row": (_i, [_i, _p, _i64, _i64, _i64, _p]),
            "or_dot": (_f, [_p, _p, _i64]),
            "or_pin_threads": (_i, [_i]),
            "or_matmul_nt": (None, [_p, _p, _i64, _i64, _i64, _p, _i]),
            "or_matmul_nn": (None, [_p, _p, _i64, _i64, _i64, _p, _i]),
            "or_matmul_tn_acc": (None, [_p, _p, _p, _i64, _i64, _i64, _i]),
            "or_linear_forward": (_i, [_i, _p, _i64, _i64, _p, _i64, _f, _p, _p, _i, _p, _i64, _p, _i]),
            "or_linear_backward": (_i, [_i, _p, _i64, _i64, _i64, _f, _p, _p, _i, _p, _p, _i64, _p, _p, _p, _i]),
            "or_lm_head": (_i, [_i, _p, _i64, _i64, _p, _f, _f, _p, _i64, _p, _p, _p, _i64, _i64, _p, _p, _p, _i]),
            "or_round_f16": (_f, [_f]),
            "or_rope_table": (None, [_i64, _i64, _f, _f, _p, _p]),
            "or_model_forward_backward": (_i, [ctypes.POINTER(OrModel), _p, _i64, _p, _p, _p, _i64, _p,
                                               ctypes.POINTER(_i64), _i]),
            "or_model_forward_backward_layout": (_i, [ctypes.POINTER(OrModel), _p, _i64, _p, _p, _p, _p, _p, _i64,
                                                      _p, ctypes.POINTER(_i64), _i]),
            "or_rope_table_at": (None, [_p, _i64, _i64, _f, _f, _p, _i64, _p, _p]),
            "or_allowed": (_i, [_p, _i64, _i64]),
            "or_rmsnorm": (None, [_p, _p, _i64, _i64, _f, _f, _i, _p, _p]),
            "or_rmsnorm_backward": (None, [_p, _p, _p, _p, _i64, _i64, _f, _p]),
            "or_qk_prep": (None, [ctypes.POINTER(OrModel), _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _p]),
            "or_qk_backward": (None, [ctypes.POINTER(OrModel), _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p,
                                      _p]),
            "or_attention_forward": (None, [ctypes.POINTER(OrModel), _p, _p, _p, _i64, _p, _p, _p, _i]),
            "or_attention_backward": (None, [ctypes.POINTER(OrModel), _p, _p, _p, _p, _p, _i64, _p, _p, _p, _p, _i]),
            "or_swiglu": (None, [_p, _p, _i64, _p]),
            "or_swiglu_backward": (None, [_p, _p, _p, _i64, _p, _p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _check(rc: int, what: str):
    if rc != 0:
        raise ValueError(f"oracle {what} failed with code {rc}")


class Rng:
    """SplitMix64 + Box-Muller, src/tensor.rs:155-199 (same seeds give the same streams)."""

    def __init__(self, seed: int):
        self._state = np.array([lib().or_rng_seed(seed)], dtype=np.uint64)

    @property
    def state(self) -> int:
        return int(self._state[0])

    def next_u64(self) -> int:
        return int(lib().or_rng_next_u64(_ptr(self._state)))

    def uniform(self) -> float:
        return float(lib().or_rng_uniform(_ptr(self._state)))

    def normal(self) -> float:
        return float(lib().or_rng_normal(_ptr(self._state)))

    def vec_normal(self, n: int, std: float) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        lib().or_rng_fill_normal(_ptr(self._state), _ptr(out), n, std)
        return out

    def vec_uniform_sym(self, n: int, bound: float) -> np.ndarray:
        out = np.empty(n, dtype=np.float32)
        lib().or_rng_fill_uniform_sym(_ptr(self._state), _ptr(out), n, bound)
        return out


def fp32_to_fp16_bits(v: float) -> int:
    return int(lib().or_fp32_to_fp16(v))


def fp16_bits_to_fp32(h: int) -> float:
    return float(lib().or_fp16_to_fp32(h))


def row_bytes(wtype: int, k: int) -> int:
    return int(lib().or_row_bytes(wtype, k))


def quantize(wtype: int, w: np.ndarray) -> np.ndarray:
    """Quantise an [n x k] f32 matrix row-major into GGUF blocks (uint8 [n, row_bytes]); TQ8_0: the
    trainer-native packing (flat uint8: scales then codes, src/frozen.rs:53-73)."""
    w = _f32(w)
    n, k = w.shape
    if wtype == TQ8_0:
        out = np.empty(n * (k // 32) * 4 + n * k, dtype=np.uint8)
        _check(lib().or_tq8_quantize(_ptr(w), n, k, _ptr(out)), "tq8_quantize")
        return out
    out = np.empty((n, row_bytes(wtype, k)), dtype=np.uint8)
    _check(lib().or_quantize(wtype, _ptr(w), w.size, _ptr(out)), "quantize")
    return out


def dequantize(wtype: int, blocks: np.ndarray, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    n = blocks.size // row_bytes(wtype, k)
    out = np.empty((n, k), dtype=np.float32)
    _check(lib().or_dequant_row(wtype, _ptr(blocks), n * k, _ptr(out)), "dequant")
    return out


def act_type_for(wtype: int) -> int:
    return int(lib().or_act_type_for(wtype))


def quantize_acts(wtype: int, x: np.ndarray) -> np.ndarray:
    """QuantActs::prepare for the activation format paired with ``wtype``: uint8 [t, act_row_bytes]."""
    x = _f32(x)
    t, k = x.shape
    at = act_type_for(wtype)
    out = np.empty((t, row_bytes(at, k)), dtype=np.uint8)
    fn = lib().or_quantize_acts_q8_0 if at == Q8_0 else lib().or_quantize_acts_q8_k
    for i in range(t):
        fn(_ptr(x[i]), k, _ptr(out[i]))
    return out


def block_isums(wtype: int, wblocks: np.ndarray, acts: np.ndarray, k: int) -> np.ndarray:
    """Integer block sums for every (token, row): int32 [t, n, isums_per_row]."""
    wblocks = np.ascontiguousarray(wblocks, dtype=np.uint8)
    acts = np.ascontiguousarray(acts, dtype=np.uint8)
    n, t = wblocks.shape[0], acts.shape[0]
    m = int(lib().or_isums_per_row(wtype, k))
    out = np.empty((t, n, m), dtype=np.int32)
    for i in range(t):
        for o in range(n):
            _check(lib().or_block_isums(wtype, _ptr(wblocks[o]), _ptr(acts[i]), k, _ptr(out[i, o])), "isums")
    return out


def frozen_forward(wtype, wblocks, n, k, x, nthreads=1) -> np.ndarray:
    x = _f32(x).reshape(-1, k)
    t = x.shape[0]
    y = np.empty((t, n), dtype=np.float32)
    _check(lib().or_frozen_forward(wtype, _ptr(np.ascontiguousarray(wblocks)), n, k, _ptr(x), t, _ptr(y), nthreads),
           "forward")
    return y


def frozen_forward_f64(wtype, wblocks, n, k, x) -> np.ndarray:
    x = _f32(x).reshape(-1, k)
    t = x.shape[0]
    y = np.empty((t, n), dtype=np.float64)
    _check(lib().or_frozen_forward_f64(wtype, _ptr(np.ascontiguousarray(wblocks)), n, k, _ptr(x), t, _ptr(y)),
           "forward_f64")
    return y


def frozen_backward_input(wtype, wblocks, n, k, dy, dx=None, nthreads=1) -> np.ndarray:
    dy = _f32(dy).reshape(-1, n)
    t = dy.shape[0]
    dx = np.zeros((t, k), dtype=np.float32) if dx is None else _f32(dx).copy()
    _check(lib().or_frozen_backward_input(wtype, _ptr(np.ascontiguousarray(wblocks)), n, k, _ptr(dy), t, _ptr(dx),
                                          nthreads), "backward_input")
    return dx


def frozen_row(wtype, wblocks, n, k, r) -> np.ndarray:
    out = np.empty(k, dtype=np.float32)
    _check(lib().or_frozen_row(wtype, _ptr(np.ascontiguousarray(wblocks)), n, k, r, _ptr(out)), "row")
    return out


def dot(a, b) -> float:
    a, b = _f32(a), _f32(b)
    return float(lib().or_dot(_ptr(a), _ptr(b), a.size))


def matmul_nt(a, b, nthreads=1):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[0]
    out = np.empty((m, n), dtype=np.float32)
    lib().or_matmul_nt(_ptr(a), _ptr(b), m, k, n, _ptr(out), nthreads)
    return out


def matmul_nn(a, b, nthreads=1):
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[1]
    out = np.empty((m, n), dtype=np.float32)
    lib().or_matmul_nn(_ptr(a), _ptr(b), m, k, n, _ptr(out), nthreads)
    return out


def matmul_tn_acc(out, a, b, nthreads=1):
    a, b = _f32(a), _f32(b)
    k, m = a.shape
    n = b.shape[1]
    assert out.shape == (m, n) and out.dtype == np.float32 and out.flags["C_CONTIGUOUS"]
    lib().or_matmul_tn_acc(_ptr(out), _ptr(a), _ptr(b), k, m, n, nthreads)
    return out


def linear_forward(wtype, wblocks, n, k, x, bias=None, A=None, B=None, alpha=0.0, lora_enabled=True, nthreads=1):
    x = _f32(x).reshape(-1, k)
    t = x.shape[0]
    rank = 0 if A is None else A.shape[0]
    y = np.empty((t, n), dtype=np.float32)
    _check(lib().or_linear_forward(wtype, _ptr(np.ascontiguousarray(wblocks)), n, k,
                                   _ptr(None if bias is None else _f32(bias)), rank, alpha,
                                   _ptr(None if A is None else _f32(A)), _ptr(None if B is None else _f32(B)),
                                   int(lora_enabled), _ptr(x), t, _ptr(y), nthreads), "linear_forward")
    return y


def linear_backward(wtype, wblocks, n, k, x, dy, A=None, B=None, alpha=0.0, ga=None, gb=None, lora_enabled=True,
                    nthreads=1):
    """Returns (dx, ga, gb); ga/gb accumulate into copies of the given arrays (zeros if None)."""
    x = _f32(x).reshape(-1, k)
    dy = _f32(dy).reshape(-1, n)
    t = x.shape[0]
    rank = 0 if A is None else A.shape[0]
    dx = np.empty((t, k), dtype=np.float32)
    ga = np.zeros((rank, k), np.float32) if ga is None else _f32(ga).copy()
    gb = np.zeros((n, rank), np.float32) if gb is None else _f32(gb).copy()
    _check(lib().or_linear_backward(wtype, _ptr(np.ascontiguousarray(wblocks)), n, k, rank, alpha,
                                    _ptr(None if A is None else _f32(A)), _ptr(None if B is None else _f32(B)),
                                    int(lora_enabled), _ptr(x), _ptr(dy), t, _ptr(dx), _ptr(ga), _ptr(gb), nthreads),
           "linear_backward")
    return dx, ga, gb


def lm_head(wtype, wblocks, V, d, norm, x, pos, tok, wts=None, eps=1e-6, off=0.0, chunk=64, nthreads=1):
    """Model::head (src/model.rs:561-609): returns (logp [n], hits, dx [t x d] or None)."""
    x = _f32(x).reshape(-1, d)
    t = x.shape[0]
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    tok = np.ascontiguousarray(tok, dtype=np.int32)
    n = pos.size
    logp = np.empty(n, np.float32)
    hits = ctypes.c_int64()
    dx = np.empty((t, d), np.float32) if wts is not None else None
    _check(lib().or_lm_head(wtype, _ptr(np.ascontiguousarray(wblocks)), V, d, _ptr(_f32(norm)), eps, off, _ptr(x), t,
                            _ptr(pos), _ptr(tok), _ptr(None if wts is None else _f32(wts)), n, chunk, _ptr(logp),
                            ctypes.byref(hits), _ptr(dx), nthreads), "lm_head")
    return logp, hits.value, dx


def pin_threads(n: int) -> int:
    """Pins an OpenMP team of ``n`` (and the pool threads later teams reuse) to the process's allowed
    CPUs, one each, for timed runs; returns the number of allowed CPUs (-1: affinity unavailable)."""
    return lib().or_pin_threads(n)


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the timed baselines' records."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def round_f16(x: float) -> float:
    return float(lib().or_round_f16(x))


def rope_table(t: int, rot: int, theta: float, freq_scale: float = 1.0, positions=None, factors=None):
    """Rope::at_positions (src/ops.rs:141-167): cos / sin [t x rot/2] for positions (default 0..t-1)."""
    cos_ = np.empty((t, rot // 2), np.float32)
    sin_ = np.empty((t, rot // 2), np.float32)
    if positions is None and factors is None:
        lib().or_rope_table(t, rot, theta, freq_scale, _ptr(cos_), _ptr(sin_))
        return cos_, sin_
    pos = None if positions is None else np.ascontiguousarray(positions, np.int32)
    fac = None if factors is None else _f32(factors)
    lib().or_rope_table_at(_ptr(pos), t, rot, theta, freq_scale, _ptr(fac), 0 if fac is None else fac.size,
                           _ptr(cos_), _ptr(sin_))
    return cos_, sin_


def allowed(seg, i: int, j: int) -> bool:
    """Rope::allowed (src/ops.rs:160-167)"""
    s = None if seg is None else np.ascontiguousarray(seg, np.int32)
    return bool(lib().or_allowed(_ptr(s), i, j))


LINEARS = ("q", "k", "v", "o", "gate", "up", "down")


def _model_struct(m: dict, keep: list, grads: list | None = None):
    """(OrModel, per-layer grads) for the dict description of model_forward_backward"""

    def arr(a, dt=np.float32):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=dt)
        keep.append(a)
        return a.ctypes.data

    def lin(d_, gl=None):
        A, B = d_.get("A"), d_.get("B")
        r = 0 if A is None else int(np.asarray(A).shape[0])
        ga = gb = None
        if r:
            ga = np.zeros((r, d_["in"]), np.float32)
            gb = np.zeros((d_["out"], r), np.float32)
            keep.extend([ga, gb])
            if gl is not None:
                gl.append((ga, gb))
        elif gl is not None:
            gl.append(None)
        blocks = np.ascontiguousarray(d_["blocks"])
        keep.append(blocks)
        return OrLinear(d_["wtype"], blocks.ctypes.data, d_["out"], d_["in"], arr(d_.get("bias")), r,
                        float(d_.get("alpha", 0.0)), arr(A), arr(B), None if ga is None else ga.ctypes.data,
                        None if gb is None else gb.ctypes.data)

    n_layer = m["n_layer"]
    L = (OrLayer * max(n_layer, 1))()
    keep.append(L)
    for i, ld in enumerate(m["layers"][:n_layer]):
        gl = []
        L[i] = OrLayer(arr(ld["attn_norm"]), arr(ld["ffn_norm"]), arr(ld.get("q_norm")), arr(ld.get("k_norm")),
                       *[lin(ld[n], gl) for n in LINEARS])
        if grads is not None:
            grads.append(dict(zip(LINEARS, gl)))
    e, h = m["embed"], m["lm_head"]
    fac = m.get("rope_factors")
    M = OrModel(n_layer, m["d"], m["n_head"], m["n_kv"], m["hd"], m["rot"], m["n_ff"], m["eps"], m["off"],
                m["theta"], m["freq_scale"], int(m["neox"]), int(m["kv_f16"]),
                lin(dict(wtype=e[0], blocks=e[1], out=e[2], **{"in": e[3]})),
                lin(dict(wtype=h[0], blocks=h[1], out=h[2], **{"in": h[3]})), arr(m["out_norm"]), L,
                arr(fac), 0 if fac is None else int(np.asarray(fac).size))
    return M


def model_forward_backward(m: dict, tokens, pos, tok, wts=None, nthreads=1, positions=None, segments=None):
    """Model::forward_backward (src/model.rs:615-687) of a model described by ``m``:
    scalars n_layer, d, n_head, n_kv, hd, rot, n_ff, eps, off, theta, freq_scale, neox, kv_f16
    (optional rope_factors); ``embed`` / ``lm_head`` = (wtype, blocks, out, in); ``out_norm``;
    ``layers`` = list of dicts with attn_norm, ffn_norm, q_norm, k_norm (or None) and per linear name
    a dict wtype, blocks, out, in, optional bias, A [r x in], B [out x r], alpha.  ``positions`` /
    ``segments`` (both [t]) give a packed layout (Model::forward_backward_packed, :634-642).
    Returns (logp, hits, grads) with grads[l][name] = (ga, gb) accumulated from zero."""
    keep: list = []
    grads: list = []
    M = _model_struct(m, keep, grads)
    tokens = np.ascontiguousarray(tokens, np.int32)
    pos = np.ascontiguousarray(pos, np.int32)
    tok = np.ascontiguousarray(tok, np.int32)
    ps = None if positions is None else np.ascontiguousarray(positions, np.int32)
    sg = None if segments is None else np.ascontiguousarray(segments, np.int32)
    w = None if wts is None else _f32(wts)
    logp = np.empty(pos.size, np.float32)
    hits = ctypes.c_int64()
    _check(lib().or_model_forward_backward_layout(ctypes.byref(M), _ptr(tokens), tokens.size, _ptr(ps), _ptr(sg),
                                                  _ptr(pos), _ptr(tok), _ptr(w), pos.size, _ptr(logp),
                                                  ctypes.byref(hits), nthreads), "model_forward_backward")
    return logp, hits.value, grads


class BlockOps:
    """The operations of one decoder block (src/model.rs:165-197, src/attention.rs:162-367,
    src/model.rs:113-134) as separate calls on host arrays, for checking a device step op by op on
    the device's own inputs.  ``m`` is the dict description of model_forward_backward."""

    def __init__(self, m: dict):
        self._keep: list = []
        self.m = m
        self.M = _model_struct(dict(m, n_layer=0, layers=[]), self._keep)

    def rmsnorm(self, x, w, fused=False):
        x = _f32(x)
        rows, d = x.shape
        y, inv = np.empty_like(x), np.empty(rows, np.float32)
        lib().or_rmsnorm(_ptr(x), _ptr(_f32(w)), rows, d, self.m["eps"], self.m["off"], int(fused), _ptr(y), _ptr(inv))
        return y, inv

    def rmsnorm_backward(self, x, w, inv, dy):
        x, dy = _f32(x), _f32(dy)
        dx = np.empty_like(x)
        lib().or_rmsnorm_backward(_ptr(x), _ptr(_f32(w)), _ptr(_f32(inv)), _ptr(dy), x.shape[0], x.shape[1],
                                  self.m["off"], _ptr(dx))
        return dx

    def qk_prep(self, q_norm, k_norm, cos_, sin_, q_raw, k_raw, v_raw):
        m, t = self.m, q_raw.shape[0]
        q_raw, k_raw, v_raw = _f32(q_raw), _f32(k_raw), _f32(v_raw)
        q, k, v = np.empty_like(q_raw), np.empty_like(k_raw), np.empty_like(v_raw)
        qi, ki = np.empty(t * m["n_head"], np.float32), np.empty(t * m["n_kv"], np.float32)
        qn = None if q_norm is None else _f32(q_norm)
        kn = None if k_norm is None else _f32(k_norm)
        lib().or_qk_prep(ctypes.byref(self.M), _ptr(qn), _ptr(kn), _ptr(_f32(cos_)), _ptr(_f32(sin_)), _ptr(q_raw),
                         _ptr(k_raw), _ptr(v_raw), t, _ptr(q), _ptr(k), _ptr(v), _ptr(qi), _ptr(ki))
        return q, k, v, qi, ki

    def qk_backward(self, q_norm, k_norm, cos_, sin_, q_raw, k_raw, q_inv, k_inv, dq, dk):
        t = q_raw.shape[0]
        dq_raw, dk_raw = np.empty_like(_f32(q_raw)), np.empty_like(_f32(k_raw))
        qn = None if q_norm is None else _f32(q_norm)
        kn = None if k_norm is None else _f32(k_norm)
        args = [_f32(a) for a in (cos_, sin_, q_raw, k_raw, q_inv, k_inv, dq, dk)]
        lib().or_qk_backward(ctypes.byref(self.M), _ptr(qn), _ptr(kn), *[_ptr(a) for a in args], t, _ptr(dq_raw),
                             _ptr(dk_raw))
        return dq_raw, dk_raw

    def attention(self, q, k, v, seg=None, nthreads=16):
        m, t = self.m, q.shape[0]
        q, k, v = _f32(q), _f32(k), _f32(v)
        probs = np.empty((m["n_head"], t, t), np.float32)
        o = np.empty((t, m["n_head"] * m["hd"]), np.float32)
        sg = None if seg is None else np.ascontiguousarray(seg, np.int32)
        lib().or_attention_forward(ctypes.byref(self.M), _ptr(q), _ptr(k), _ptr(v), t, _ptr(sg), _ptr(probs), _ptr(o),
                                   nthreads)
        return probs, o

    def attention_backward(self, q, k, v, probs, d_o, seg=None, nthreads=16):
        t = q.shape[0]
        q, k, v, probs, d_o = (_f32(a) for a in (q, k, v, probs, d_o))
        dq, dk, dv = np.empty_like(q), np.empty_like(k), np.empty_like(v)
        sg = None if seg is None else np.ascontiguousarray(seg, np.int32)
        lib().or_attention_backward(ctypes.byref(self.M), _ptr(q), _ptr(k), _ptr(v), _ptr(probs), _ptr(d_o), t,
                                    _ptr(sg), _ptr(dq), _ptr(dk), _ptr(dv), nthreads)
        return dq, dk, dv

    def swiglu(self, g, u):
        g, u = _f32(g), _f32(u)
        hm = np.empty_like(g)
        lib().or_swiglu(_ptr(g), _ptr(u), g.size, _ptr(hm))
        return hm

    def swiglu_backward(self, g, u, dhm):
        g, u, dhm = _f32(g), _f32(u), _f32(dhm)
        dg, du = np.empty_like(g), np.empty_like(g)
        lib().or_swiglu_backward(_ptr(g), _ptr(u), _ptr(dhm), g.size, _ptr(dg), _ptr(du))
        return dg, du
