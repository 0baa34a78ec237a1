"""Device-resident training step of a GGUF decoder (``Model`` of the reference over the GPU
``FrozenMatmul``): ``Model::attach_lora``, ``zero_grad``, ``forward_backward`` and ``score``
(src/model.rs:406-436, :547-687), with every frozen tensor, activation and adapter in HBM.

``GpuModel.from_gguf(file)`` loads an open ``gguf.GgufFile`` as ``load_gguf_from`` does
(src/rie.rs:164-260).  Adapters are numbered in (block, q, k, v, o, gate, up, down) order; ``lora(i)``
returns host copies ``(a, b, ga, gb)``.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _ffi
from .frozen import Context, default_context

LINEARS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")
GGUF_LINEARS = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up", "ffn_down")
DEFAULT_TARGETS = LINEARS  # src/model.rs:321-322 (the DeltaNet projections do not occur in GGUF models)


def model_config(file) -> dict:
    """The hyper-parameters ``GpuModel.from_gguf`` would load from ``file`` (an open
    ``gguf.GgufFile``), with the same refusals (``RtqError``), without a device."""
    c = _ffi.RtqModelConfig()
    _ffi.check(_ffi.lib().rtq_model_config_from_gguf(file.handle, ctypes.byref(c)), "rtq_model_config_from_gguf")
    return {n: getattr(c, n) for n, _ in c._fields_}


def _target_mask(targets) -> int:
    mask = 0
    for t in targets:
        name = GGUF_LINEARS[LINEARS.index(t)] if t in LINEARS else t
        if name in GGUF_LINEARS:
            mask |= 1 << GGUF_LINEARS.index(name)
    return mask


class GpuModel:
    def __init__(self, handle: ctypes.c_void_p, ctx: Context, keep=None):
        self._h = handle
        self.ctx = ctx
        ctx._owned.add(self)
        self._keep = keep
        c = _ffi.RtqModelConfig()
        _ffi.check(_ffi.lib().rtq_model_get_config(handle, ctypes.byref(c)), "rtq_model_get_config")
        self.config = {n: getattr(c, n) for n, _ in c._fields_}

    @classmethod
    def from_gguf(cls, file, ctx: Context | None = None) -> "GpuModel":
        ctx = ctx or default_context()
        h = ctypes.c_void_p()
        _ffi.check(_ffi.lib().rtq_model_from_gguf(ctx.handle, file.handle, ctypes.byref(h)), "rtq_model_from_gguf")
        return cls(h, ctx, keep=file)

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            _ffi.lib().rtq_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def attach_lora(self, rank: int, alpha: float, targets=DEFAULT_TARGETS, seed: int = 1) -> int:
        """``Model::attach_lora``: returns the number of adapter parameters."""
        n = ctypes.c_int64()
        _ffi.check(_ffi.lib().rtq_model_attach_lora(self._h, rank, alpha, _target_mask(targets), seed, ctypes.byref(n)),
                   "rtq_model_attach_lora")
        return n.value

    def lora_count(self) -> int:
        return int(_ffi.lib().rtq_model_lora_count(self._h))

    def lora_info(self, i: int) -> dict:
        layer, which = ctypes.c_int(), ctypes.c_int()
        rank, inp, out = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        alpha = ctypes.c_float()
        _ffi.check(_ffi.lib().rtq_model_lora_info(self._h, i, ctypes.byref(layer), ctypes.byref(which),
                                                  ctypes.byref(rank), ctypes.byref(inp), ctypes.byref(out),
                                                  ctypes.byref(alpha)), "rtq_model_lora_info")
        return dict(layer=layer.value, name=f"blk.{layer.value}.{GGUF_LINEARS[which.value]}", which=which.value,
                    rank=rank.value, in_dim=inp.value, out_dim=out.value, alpha=alpha.value)

    def lora(self, i: int):
        """Host copies (a [r x in], b [out x r], ga, gb) of adapter i."""
        inf = self.lora_info(i)
        r, k, n = inf["rank"], inf["in_dim"], inf["out_dim"]
        a, ga = np.empty((r, k), np.float32), np.empty((r, k), np.float32)
        b, gb = np.empty((n, r), np.float32), np.empty((n, r), np.float32)
        _ffi.check(_ffi.lib().rtq_model_lora_get(self._h, i, a.ctypes.data, b.ctypes.data, ga.ctypes.data,
                                                 gb.ctypes.data), "rtq_model_lora_get")
        return a, b, ga, gb

    def set_lora(self, i: int, a=None, b=None) -> None:
        inf = self.lora_info(i)
        av = None if a is None else np.ascontiguousarray(a, np.float32).reshape(inf["rank"], inf["in_dim"])
        bv = None if b is None else np.ascontiguousarray(b, np.float32).reshape(inf["out_dim"], inf["rank"])
        _ffi.check(_ffi.lib().rtq_model_lora_set(self._h, i, None if av is None else av.ctypes.data,
                                                 None if bv is None else bv.ctypes.data), "rtq_model_lora_set")

    def lora_device(self, i: int) -> tuple[int, int, int, int, int]:
        """Device addresses of adapter i's (a, b, ga, gb) and the row stride of b / gb in floats
        (the adapters of fused linears share one B matrix)."""
        ps = [ctypes.c_void_p() for _ in range(4)]
        ld = ctypes.c_int64()
        _ffi.check(_ffi.lib().rtq_model_lora_device(self._h, i, *[ctypes.byref(p) for p in ps], ctypes.byref(ld)),
                   "rtq_model_lora_device")
        return tuple(int(p.value or 0) for p in ps) + (ld.value,)

    def zero_grad(self) -> None:
        _ffi.check(_ffi.lib().rtq_model_zero_grad(self._h), "rtq_model_zero_grad")

    def forward_backward(self, tokens, targets, weights=None) -> tuple[np.ndarray, int]:
        """``Model::forward_backward``: log-probs of the targets (and the greedy hits); with
        ``weights`` the adapters' gradients of ``L = -sum w_i logp_i`` accumulate."""
        toks = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
        pos = np.array([t.pos for t in targets], dtype=np.int32)
        tok = np.array([t.token for t in targets], dtype=np.int32)
        w = None if weights is None else np.ascontiguousarray(weights, dtype=np.float32)
        if w is not None:
            assert w.size == pos.size, "one weight per target"
        logp = np.empty(pos.size, dtype=np.float32)
        hits = ctypes.c_int64()
        _ffi.check(_ffi.lib().rtq_model_forward_backward(self._h, toks.ctypes.data, toks.size, pos.ctypes.data,
                                                         tok.ctypes.data, None if w is None else w.ctypes.data,
                                                         pos.size, logp.ctypes.data, ctypes.byref(hits)),
                   "rtq_model_forward_backward")
        self._stepped = True
        return logp, int(hits.value)

    def forward_backward_packed(self, packed, targets, weights=None) -> tuple[np.ndarray, int]:
        """``Model::forward_backward_packed`` (src/model.rs:634-642) over a ``packing.Packed`` batch:
        RoPE at each token's own position, attention within the segment layout; ``targets`` index
        ``packed.tokens`` (``Packed.map_targets``)."""
        toks = np.ascontiguousarray(packed.tokens, dtype=np.int32).reshape(-1)
        ps = np.ascontiguousarray(packed.positions, dtype=np.int32).reshape(-1)
        sg = np.ascontiguousarray(packed.segments, dtype=np.int32).reshape(-1)
        assert ps.size == toks.size and sg.size == toks.size, "one position and segment per token"
        pos = np.array([t.pos for t in targets], dtype=np.int32)
        tok = np.array([t.token for t in targets], dtype=np.int32)
        w = None if weights is None else np.ascontiguousarray(weights, dtype=np.float32)
        if w is not None:
            assert w.size == pos.size, "one weight per target"
        logp = np.empty(pos.size, dtype=np.float32)
        hits = ctypes.c_int64()
        _ffi.check(_ffi.lib().rtq_model_forward_backward_packed(
            self._h, toks.ctypes.data, toks.size, ps.ctypes.data, sg.ctypes.data, pos.ctypes.data, tok.ctypes.data,
            None if w is None else w.ctypes.data, pos.size, logp.ctypes.data, ctypes.byref(hits)),
            "rtq_model_forward_backward_packed")
        self._stepped = True
        return logp, int(hits.value)

    @property
    def checkpointing(self):
        """``Model::checkpointing``: True recomputes each block's forward in the backward, False keeps
        every block's activations, None (default) decides per step by memory.  Reading it gives the
        last step's choice (None before any step)."""
        v = int(_ffi.lib().rtq_model_checkpointing(self._h))
        return None if not getattr(self, "_stepped", False) else bool(v)

    @checkpointing.setter
    def checkpointing(self, on) -> None:
        mode = -1 if on is None else (1 if on else 0)
        _ffi.check(_ffi.lib().rtq_model_set_checkpointing(self._h, mode), "rtq_model_set_checkpointing")

    @property
    def fused_attention(self):
        """Attention kernels: True the fused kernels (no probability matrix; head_dim 64 / 128),
        False the probability-matrix path, None (default) the fused kernels whenever the head size
        allows.  Reading it gives the last step's choice (None before any step)."""
        v = int(_ffi.lib().rtq_model_attention_fused(self._h))
        return None if not getattr(self, "_stepped", False) else bool(v)

    @fused_attention.setter
    def fused_attention(self, on) -> None:
        mode = -1 if on is None else (1 if on else 0)
        _ffi.check(_ffi.lib().rtq_model_set_attention(self._h, mode), "rtq_model_set_attention")

    @property
    def graph_replays(self) -> int:
        """Steps so far that replayed the captured step graph (a step whose sizes, layout, choices,
        adapters and buffers equal the previous step's is captured; later ones replay it)."""
        return int(_ffi.lib().rtq_model_graph_replays(self._h))

    def debug_capture(self, layer: int) -> None:
        """Copy block ``layer``'s tensors during each step (-1: off); read them with ``debug_tensor``."""
        _ffi.check(_ffi.lib().rtq_model_debug_capture(self._h, layer), "rtq_model_debug_capture")

    def debug_tensor(self, name: str, shape) -> np.ndarray:
        out = np.empty(shape, np.float32)
        _ffi.check(_ffi.lib().rtq_model_debug_tensor(self._h, name.encode(), out.ctypes.data, out.size),
                   "rtq_model_debug_tensor")
        return out

    def score(self, tokens, targets) -> tuple[np.ndarray, int]:
        """``Model::score`` (src/model.rs:553-557): log-probs and hits, no backward."""
        return self.forward_backward(tokens, targets, None)
