"""GGUF v3 container (``rie_core::gguf::{GgufFile, GgufWriter}``) and the synthetic-model builder
(``rie_core::testing::SyntheticSpec``) over librtq.so's native reader / writer.

* ``GgufFile.open(path)`` maps the file, ``GgufFile.from_bytes(b)`` borrows the bytes (kept alive
  by the handle) — src/rie.rs:159, :370; tests/engine.rs:27-31.  ``get_str`` / ``get_f32``
  (src/rie.rs:371-379) return None when the key is absent; ``tensor(name)`` returns a
  ``TensorInfo`` (``ty``, ``n_rows()``, ``row_len()``) and ``tensor_data(t)`` a zero-copy uint8
  view into the image (src/rie.rs:381-384).
* ``GgufWriter`` (src/rie.rs:349-363): ``kv(key, Value.String(...))``, ``tensor(name, dims,
  ggml_type, bytes)``, ``to_bytes()``; ``write(path)`` writes ``path.tmp`` then renames.
* ``SyntheticSpec`` (src/main.rs:648-677, examples/bench_train.rs:28-32): random-weight llama /
  qwen3 models with per-tensor quant types, tensors named as the loader reads them
  (``blk.{i}.attn_q.weight`` ... src/rie.rs:207-231).
* ``HipFrozen.from_gguf`` (frozen.py) uploads a tensor straight from an open file.

Shape convention (GGUF): ``dims[0]`` is the row length (columns), ``dims[1:]`` the rows.
"""
from __future__ import annotations

import ctypes
import dataclasses
import os
import struct

import numpy as np

from . import _ffi
from .synth import QUANTIZERS, Rng

# GGUF metadata value types (public GGUF v3 specification)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}
_NP = {U8: np.uint8, I8: np.int8, U16: np.uint16, I16: np.int16, U32: np.uint32, I32: np.int32, F32: np.float32,
       BOOL: np.bool_, U64: np.uint64, I64: np.int64, F64: np.float64}

# ggml tensor types the writer and ``TensorInfo.nbytes`` know: id -> (block elements, block bytes)
GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q4_K, GGML_Q6_K = 0, 1, 2, 8, 12, 14
GGML_BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36),
              10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 15: (256, 292),
              24: (1, 1), 25: (1, 2), 26: (1, 4), 27: (1, 8), 28: (1, 8), 30: (1, 2)}
GGML_NAMES = {"F32": 0, "F16": 1, "Q4_0": 2, "Q8_0": 8, "Q4_K": 12, "Q6_K": 14}


def ggml_nbytes(ggml_type: int, n: int) -> int:
    be, bb = GGML_BLOCK[ggml_type]
    assert n % be == 0, f"{n} elements is not a whole number of type-{ggml_type} blocks"
    return n // be * bb


@dataclasses.dataclass(frozen=True)
class Value:
    """A typed metadata value (``rie_core::gguf::Value``): ``Value.String("lora")``,
    ``Value.F32(8.0)``, ``Value.Array(U32, [1, 2])``."""
    type: int
    value: object
    elem: int = -1

    @staticmethod
    def String(s: str) -> "Value":  # noqa: N802 - mirrors Value::String
        return Value(STRING, s)

    @staticmethod
    def F32(x: float) -> "Value":  # noqa: N802
        return Value(F32, float(x))

    @staticmethod
    def F64(x: float) -> "Value":  # noqa: N802
        return Value(F64, float(x))

    @staticmethod
    def U32(x: int) -> "Value":  # noqa: N802
        return Value(U32, int(x))

    @staticmethod
    def I32(x: int) -> "Value":  # noqa: N802
        return Value(I32, int(x))

    @staticmethod
    def U64(x: int) -> "Value":  # noqa: N802
        return Value(U64, int(x))

    @staticmethod
    def I64(x: int) -> "Value":  # noqa: N802
        return Value(I64, int(x))

    @staticmethod
    def Bool(x: bool) -> "Value":  # noqa: N802
        return Value(BOOL, bool(x))

    @staticmethod
    def Array(elem: int, items) -> "Value":  # noqa: N802
        return Value(ARRAY, list(items), elem)


@dataclasses.dataclass(frozen=True)
class TensorInfo:
    """One tensor's directory entry (``GgufFile::tensor``)."""
    index: int
    name: str
    ty: int
    dims: tuple
    nbytes: int

    def row_len(self) -> int:
        return int(self.dims[0])

    def n_rows(self) -> int:
        return int(np.prod(self.dims[1:], dtype=np.int64)) if len(self.dims) > 1 else 1


class GgufFile:
    """A parsed GGUF image (``rtq_gguf``)."""

    def __init__(self, handle: ctypes.c_void_p, keep=None):
        self._h = handle
        self._keep = keep  # the borrowed bytes of from_bytes
        L = _ffi.lib()
        self.version = int(L.rtq_gguf_version(handle))
        self._tensors = [self._info(i) for i in range(int(L.rtq_gguf_tensor_count(handle)))]
        self._by_name = {t.name: t for t in self._tensors}

    @classmethod
    def open(cls, path: str | os.PathLike) -> "GgufFile":
        h = ctypes.c_void_p()
        _ffi.check(_ffi.lib().rtq_gguf_open(os.fsencode(path), ctypes.byref(h)), "rtq_gguf_open")
        return cls(h)

    @classmethod
    def from_bytes(cls, data) -> "GgufFile":
        buf = np.frombuffer(data, dtype=np.uint8) if not isinstance(data, np.ndarray) else \
            np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        h = ctypes.c_void_p()
        _ffi.check(_ffi.lib().rtq_gguf_from_bytes(buf.ctypes.data, buf.nbytes, ctypes.byref(h)), "rtq_gguf_from_bytes")
        return cls(h, keep=(data, buf))

    @property
    def handle(self) -> ctypes.c_void_p:
        if self._h is None:
            raise RuntimeError("GGUF file closed")
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            _ffi.lib().rtq_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- metadata
    def keys(self) -> list[str]:
        return [self._kv(i)[0] for i in range(int(_ffi.lib().rtq_gguf_kv_count(self.handle)))]

    def _kv(self, i: int):
        key, data = ctypes.c_void_p(), ctypes.c_void_p()
        ty, elem, count = ctypes.c_int(), ctypes.c_int(), ctypes.c_uint64()
        _ffi.check(_ffi.lib().rtq_gguf_kv(self.handle, i, ctypes.byref(key), ctypes.byref(ty), ctypes.byref(elem),
                                          ctypes.byref(count), ctypes.byref(data)), "rtq_gguf_kv")
        return ctypes.string_at(key.value).decode(), ty.value, elem.value, count.value, data.value

    def value_type(self, key: str) -> int | None:
        i = int(_ffi.lib().rtq_gguf_find_kv(self.handle, key.encode()))
        return None if i < 0 else self._kv(i)[1]

    def get(self, key: str):
        """The decoded value of ``key`` (str, int, float, bool, list of str, or a numpy array for
        numeric arrays), or None."""
        i = int(_ffi.lib().rtq_gguf_find_kv(self.handle, key.encode()))
        if i < 0:
            return None
        _, ty, elem, count, ptr = self._kv(i)
        if ty == STRING:
            return ctypes.string_at(ptr, count).decode("utf-8", errors="replace") if count else ""
        if ty == ARRAY:
            if elem == STRING:
                out, at = [], ptr
                for _ in range(count):
                    n = struct.unpack("<Q", ctypes.string_at(at, 8))[0]
                    out.append(ctypes.string_at(at + 8, n).decode("utf-8", errors="replace") if n else "")
                    at += 8 + n
                return out
            nb = count * np.dtype(_NP[elem]).itemsize
            return np.frombuffer(ctypes.string_at(ptr, nb) if nb else b"", dtype=_NP[elem]).copy()
        v = struct.unpack(_SCALAR[ty], ctypes.string_at(ptr, struct.calcsize(_SCALAR[ty])))[0]
        return v

    def get_str(self, key: str) -> str | None:
        """``GgufFile::get_str``: the string value, None if absent or not a string."""
        return self.get(key) if self.value_type(key) == STRING else None

    def get_f32(self, key: str) -> float | None:
        """``GgufFile::get_f32``: a numeric value as float32, None if absent or not a number."""
        if self.value_type(key) in (None, STRING, ARRAY):
            return None
        v = ctypes.c_double()
        _ffi.check(_ffi.lib().rtq_gguf_get_f64(self.handle, key.encode(), ctypes.byref(v)), "rtq_gguf_get_f64")
        return float(np.float32(v.value))

    def get_u32(self, key: str) -> int | None:
        ty = self.value_type(key)
        return int(self.get(key)) if ty in (U8, U16, U32, I8, I16, I32, U64, I64) else None

    # ---- tensors
    def _info(self, i: int) -> TensorInfo:
        name, data = ctypes.c_char_p(), ctypes.c_void_p()
        ty, nd = ctypes.c_int(), ctypes.c_int()
        ne = (ctypes.c_int64 * 4)()
        nb = ctypes.c_size_t()
        _ffi.check(_ffi.lib().rtq_gguf_tensor(self._h, i, ctypes.byref(name), ctypes.byref(ty), ctypes.byref(nd), ne,
                                              ctypes.byref(data), ctypes.byref(nb)), "rtq_gguf_tensor")
        return TensorInfo(i, name.value.decode(), ty.value, tuple(int(ne[d]) for d in range(nd.value)), int(nb.value))

    def tensors(self) -> list[TensorInfo]:
        return list(self._tensors)

    def tensor(self, name: str) -> TensorInfo | None:
        return self._by_name.get(name)

    def tensor_data(self, t: TensorInfo) -> np.ndarray:
        """The tensor's bytes: a read-only uint8 view into the image (valid while the file is open)."""
        data = ctypes.c_void_p()
        _ffi.check(_ffi.lib().rtq_gguf_tensor(self.handle, t.index, None, None, None, None, ctypes.byref(data), None),
                   "rtq_gguf_tensor")
        if t.nbytes == 0:
            return np.empty(0, dtype=np.uint8)
        view = np.ctypeslib.as_array((ctypes.c_uint8 * t.nbytes).from_address(data.value))
        view.flags.writeable = False
        return view

    def tensor_f32(self, t: TensorInfo) -> np.ndarray:
        """An F32 / F16 tensor as float32 [n_rows, row_len] (norm weights, adapters)."""
        raw = self.tensor_data(t)
        if t.ty == GGML_F32:
            return raw.view(np.float32).reshape(t.n_rows(), t.row_len()).copy()
        if t.ty == GGML_F16:
            return raw.view(np.float16).astype(np.float32).reshape(t.n_rows(), t.row_len())
        raise ValueError(f"{t.name}: type {t.ty} is not F32/F16")


class GgufWriter:
    """Builds a GGUF v3 image (``GgufWriter``, src/rie.rs:349-363)."""

    def __init__(self):
        h = ctypes.c_void_p()
        _ffi.check(_ffi.lib().rtq_gguf_writer_create(ctypes.byref(h)), "rtq_gguf_writer_create")
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            _ffi.lib().rtq_gguf_writer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def kv(self, key: str, v: Value) -> None:
        L = _ffi.lib()
        if v.type == STRING:
            b = v.value.encode()
            st = L.rtq_gguf_writer_kv(self._h, key.encode(), STRING, -1, len(b), ctypes.c_char_p(b))
        elif v.type == ARRAY and v.elem == STRING:
            items = [s.encode() for s in v.value]
            arr = (ctypes.c_char_p * max(1, len(items)))(*items)
            st = L.rtq_gguf_writer_kv(self._h, key.encode(), ARRAY, STRING, len(items), ctypes.cast(arr, ctypes.c_void_p))
        elif v.type == ARRAY:
            a = np.ascontiguousarray(np.asarray(v.value, dtype=_NP[v.elem]))
            st = L.rtq_gguf_writer_kv(self._h, key.encode(), ARRAY, v.elem, a.size, a.ctypes.data if a.size else None)
        else:
            b = struct.pack(_SCALAR[v.type], v.value)
            st = L.rtq_gguf_writer_kv(self._h, key.encode(), v.type, -1, 1, ctypes.c_char_p(b))
        _ffi.check(st, f"rtq_gguf_writer_kv({key})")

    def tensor(self, name: str, dims, ggml_type: int, data) -> None:
        """``dims`` as GGUF stores them: ``[row_len, n_rows, ...]``; ``data`` the packed bytes."""
        a = np.ascontiguousarray(data)
        a = a.view(np.uint8).reshape(-1) if a.dtype != np.uint8 else a.reshape(-1)
        ne = (ctypes.c_int64 * len(dims))(*[int(d) for d in dims])
        _ffi.check(_ffi.lib().rtq_gguf_writer_tensor(self._h, name.encode(), ggml_type, len(dims), ne, a.ctypes.data,
                                                     a.nbytes), f"rtq_gguf_writer_tensor({name})")

    def to_bytes(self) -> bytes:
        data, n = ctypes.c_void_p(), ctypes.c_size_t()
        _ffi.check(_ffi.lib().rtq_gguf_writer_bytes(self._h, ctypes.byref(data), ctypes.byref(n)),
                   "rtq_gguf_writer_bytes")
        if not n.value:
            return b""
        # through a ctypes array (string_at takes a C int size: images over 2 GiB)
        return bytes((ctypes.c_char * n.value).from_address(data.value))

    def write(self, path: str | os.PathLike) -> None:
        _ffi.check(_ffi.lib().rtq_gguf_writer_write(self._h, os.fsencode(path)), "rtq_gguf_writer_write")


# ------------------------------------------------------------------ synthetic models
@dataclasses.dataclass
class SyntheticSpec:
    """A random-weight llama / qwen3 GGUF (``rie_core::testing::SyntheticSpec``; fields as the
    reference sets them in src/main.rs:662-675).

    Linear weights are N(0, ``std``) from the reference's SplitMix64 generator, one stream per
    tensor (seed ``seed * 1_000_003 + tensor index``), quantised with ``synth.QUANTIZERS``; norm
    weights are 1.  ``wtype`` is the default type of every matrix; ``tensor_types`` overrides it
    per tensor role (``attn_q``, ``attn_k``, ``attn_v``, ``attn_output``, ``ffn_gate``, ``ffn_up``,
    ``ffn_down``, ``token_embd``, ``output``).  A K-quant falls back to Q8_0 on a tensor whose row
    length is not a multiple of 256 (Q8_0 to F32 below 32).
    """
    arch: str = "qwen3"
    wtype: int = GGML_Q4_0
    seed: int = 1
    n_layer: int = 2
    n_embd: int = 256
    n_head: int = 4
    n_head_kv: int = 2
    head_dim: int = 64
    rope_dim: int = 64
    n_ff: int = 512
    n_vocab: int = 512
    tied_output: bool = True
    rope_base: float = 1e6
    rms_eps: float = 1e-6
    std: float = 0.02
    tensor_types: dict = dataclasses.field(default_factory=dict)
    # weights from numpy's PCG64 (N(0, std) per tensor, seeded as above) instead of the reference's
    # SplitMix64 stream: 6x faster to draw, for the multi-billion-parameter benchmark models
    fast: bool = False

    # name -> (arch, layers, hidden, heads, kv heads, head dim, ff, vocab, tied, rope base, per-role types)
    PRESETS = {
        "qwen3-0.6b": ("qwen3", 28, 1024, 16, 8, 128, 3072, 151936, True, 1e6, {}),
        "qwen3-4b": ("qwen3", 36, 2560, 32, 8, 128, 9728, 151936, True, 1e6,
                     {"attn_q": GGML_Q4_K, "attn_k": GGML_Q4_K, "attn_v": GGML_Q4_K, "attn_output": GGML_Q4_K,
                      "ffn_gate": GGML_Q4_K, "ffn_up": GGML_Q4_K, "ffn_down": GGML_Q6_K, "token_embd": GGML_Q6_K,
                      "output": GGML_Q6_K}),
        "llama3-8b": ("llama", 32, 4096, 32, 8, 128, 14336, 128256, False, 5e5, {}),
    }

    @classmethod
    def preset(cls, name: str, wtype: int) -> "SyntheticSpec | None":
        p = cls.PRESETS.get(name)
        if p is None:
            return None
        arch, nl, d, nh, nkv, hd, ff, nv, tied, base, types = p
        return cls(arch=arch, wtype=wtype, n_layer=nl, n_embd=d, n_head=nh, n_head_kv=nkv, head_dim=hd, rope_dim=hd,
                   n_ff=ff, n_vocab=nv, tied_output=tied, rope_base=base, tensor_types=dict(types))

    @classmethod
    def tiny(cls, arch: str, wtype: int) -> "SyntheticSpec":
        return cls(arch=arch, wtype=wtype)

    def _type_for(self, role: str, row_len: int) -> int:
        ty = self.tensor_types.get(role, self.wtype)
        if ty in (GGML_Q4_K, GGML_Q6_K) and row_len % 256:
            ty = GGML_Q8_0
        if ty in (GGML_Q4_0, GGML_Q8_0) and row_len % 32:
            ty = GGML_F32
        return ty

    def plan(self) -> list[tuple[str, int, tuple]]:
        """(name, ggml type, dims) of every tensor, in file order."""
        d, q, kv = self.n_embd, self.n_head * self.head_dim, self.n_head_kv * self.head_dim
        out = [("token_embd.weight", self._type_for("token_embd", d), (d, self.n_vocab))]
        for i in range(self.n_layer):
            p = f"blk.{i}."
            out += [(p + "attn_norm.weight", GGML_F32, (d,)),
                    (p + "attn_q.weight", self._type_for("attn_q", d), (d, q)),
                    (p + "attn_k.weight", self._type_for("attn_k", d), (d, kv)),
                    (p + "attn_v.weight", self._type_for("attn_v", d), (d, kv)),
                    (p + "attn_output.weight", self._type_for("attn_output", q), (q, d))]
            if self.arch == "qwen3":
                out += [(p + "attn_q_norm.weight", GGML_F32, (self.head_dim,)),
                        (p + "attn_k_norm.weight", GGML_F32, (self.head_dim,))]
            out += [(p + "ffn_norm.weight", GGML_F32, (d,)),
                    (p + "ffn_gate.weight", self._type_for("ffn_gate", d), (d, self.n_ff)),
                    (p + "ffn_up.weight", self._type_for("ffn_up", d), (d, self.n_ff)),
                    (p + "ffn_down.weight", self._type_for("ffn_down", self.n_ff), (self.n_ff, d))]
        out.append(("output_norm.weight", GGML_F32, (d,)))
        if not self.tied_output:
            out.append(("output.weight", self._type_for("output", d), (d, self.n_vocab)))
        return out

    def tensor_values(self, index: int, name: str, ggml_type: int, dims) -> np.ndarray:
        """The packed bytes of tensor ``index`` of ``plan()``."""
        n = int(np.prod(dims, dtype=np.int64))
        if name.endswith("norm.weight"):
            return np.ones(n, dtype=np.float32).view(np.uint8)
        if self.fast:
            return np.concatenate([self._fast_rows(index, ggml_type, dims, r0, r1)
                                   for r0, r1 in self._fast_chunks(dims)])
        else:
            w = Rng(self.seed * 1_000_003 + index).vec_normal(n, self.std).reshape(-1, dims[0])
        if ggml_type == GGML_F32:
            return w.view(np.uint8).reshape(-1)
        return QUANTIZERS[ggml_type](w).reshape(-1)

    FAST_CHUNK = 1 << 24  # elements per independently seeded row chunk of a fast tensor

    def _fast_chunks(self, dims) -> list[tuple[int, int]]:
        rows = int(np.prod(dims[1:], dtype=np.int64)) if len(dims) > 1 else 1
        step = max(1, self.FAST_CHUNK // int(dims[0]))
        return [(r, min(rows, r + step)) for r in range(0, rows, step)]

    def _fast_rows(self, index: int, ggml_type: int, dims, r0: int, r1: int) -> np.ndarray:
        """rows [r0, r1) of a fast tensor: N(0, std) from PCG64 seeded by (tensor, first row)"""
        rng = np.random.default_rng([self.seed * 1_000_003 + index, r0])
        w = (rng.standard_normal((r1 - r0) * int(dims[0]), dtype=np.float32) * np.float32(self.std))
        w = w.reshape(r1 - r0, int(dims[0]))
        if ggml_type == GGML_F32:
            return w.view(np.uint8).reshape(-1)
        return QUANTIZERS[ggml_type](w).reshape(-1)

    def metadata(self) -> list[tuple[str, Value]]:
        a = self.arch
        return [("general.architecture", Value.String(a)),
                ("general.name", Value.String(f"synthetic-{a}")),
                ("general.alignment", Value.U32(32)),
                (f"{a}.block_count", Value.U32(self.n_layer)),
                (f"{a}.context_length", Value.U32(4096)),
                (f"{a}.embedding_length", Value.U32(self.n_embd)),
                (f"{a}.feed_forward_length", Value.U32(self.n_ff)),
                (f"{a}.attention.head_count", Value.U32(self.n_head)),
                (f"{a}.attention.head_count_kv", Value.U32(self.n_head_kv)),
                (f"{a}.attention.key_length", Value.U32(self.head_dim)),
                (f"{a}.attention.value_length", Value.U32(self.head_dim)),
                (f"{a}.attention.layer_norm_rms_epsilon", Value.F32(self.rms_eps)),
                (f"{a}.rope.dimension_count", Value.U32(self.rope_dim)),
                (f"{a}.rope.freq_base", Value.F32(self.rope_base)),
                (f"{a}.vocab_size", Value.U32(self.n_vocab))]

    def writer(self, workers: int = 1) -> GgufWriter:
        """The image's writer; ``workers`` > 1 draws and quantises the tensors in that many forked
        processes (the bytes are the same)."""
        w = GgufWriter()
        for k, v in self.metadata():
            w.kv(k, v)
        plan = self.plan()
        if workers > 1 and len(plan) > 1:
            import concurrent.futures as cf
            import multiprocessing as mp

            with cf.ProcessPoolExecutor(max_workers=workers, mp_context=mp.get_context("fork")) as ex:
                if self.fast:  # row chunks, so one large tensor keeps every worker busy
                    futs = [[ex.submit(self._fast_rows, i, ty, dims, r0, r1) for r0, r1 in self._fast_chunks(dims)]
                            if not name.endswith("norm.weight") else [ex.submit(self.tensor_values, i, name, ty, dims)]
                            for i, (name, ty, dims) in enumerate(plan)]
                    for (name, ty, dims), fs in zip(plan, futs):
                        w.tensor(name, dims, ty, np.concatenate([f.result() for f in fs]))
                else:
                    futs = [ex.submit(self.tensor_values, i, name, ty, dims) for i, (name, ty, dims) in enumerate(plan)]
                    for (name, ty, dims), f in zip(plan, futs):
                        w.tensor(name, dims, ty, f.result())
        else:
            for i, (name, ty, dims) in enumerate(plan):
                w.tensor(name, dims, ty, self.tensor_values(i, name, ty, dims))
        return w

    def build(self, workers: int = 1) -> bytes:
        """The whole GGUF image (``SyntheticSpec::build``)."""
        w = self.writer(workers)
        try:
            return w.to_bytes()
        finally:
            w.close()
