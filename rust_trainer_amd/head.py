"""LM head + cross-entropy and the embedding gather on the GPU (``Model::head`` and
``Model::embed_tokens``, src/model.rs:446-454, :561-609).

``head(lm_head, final_norm, x, targets, weights)`` returns ``(logp, dx, hits)`` as the reference's
``Model::head`` does: the log-probability of each target token at its position (final RMSNorm,
``lm_head.forward``, log-softmax with an f64 normaliser), the number of targets that are the greedy
argmax, and — when ``weights`` is given — ``dL/dx`` of ``L = -sum w_i logp_i`` (zero rows outside
the target positions; an empty array otherwise).  ``embed_tokens(embed, tokens)`` gathers
dequantised rows.
"""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np

from . import _ffi
from .frozen import HipFrozen


@dataclasses.dataclass(frozen=True)
class Target:
    """A supervised target (src/model.rs:223-226): predict ``token`` from position ``pos``."""
    pos: int
    token: int


def answer_targets(tokens, answer_start: int) -> list[Target]:
    """Every answer token ``tokens[i]`` (``i >= answer_start``) predicted from position ``i - 1``
    (src/model.rs:230-232)."""
    return [Target(i - 1, int(tokens[i])) for i in range(max(answer_start, 1), len(tokens))]


def embed_tokens(embed: HipFrozen, tokens) -> np.ndarray:
    """x[t x d] = row(token) per token (src/model.rs:446-454); out-of-vocab tokens raise."""
    ids = np.ascontiguousarray(tokens, dtype=np.int32).reshape(-1)
    out = np.empty((ids.size, embed.in_dim()), dtype=np.float32)
    _ffi.check(_ffi.lib().rtq_frozen_gather(embed.ctx.handle, embed.handle, ids.ctypes.data, ids.size,
                                            out.ctypes.data), "rtq_frozen_gather")
    return out.reshape(-1)


def head(lm_head: HipFrozen, final_norm, x, targets, weights=None, eps: float = 1e-6,
         offset: float = 0.0) -> tuple[np.ndarray, np.ndarray, int]:
    """``Model::head`` (src/model.rs:561-609) on the GPU; ``x`` is [t x d] final hidden states."""
    d = lm_head.in_dim()
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size % d == 0, "x is not a whole number of rows"
    t = x.size // d
    norm = np.ascontiguousarray(final_norm, dtype=np.float32)
    assert norm.size == d, "final_norm length != hidden size"
    pos = np.array([tg.pos for tg in targets], dtype=np.int32)
    tok = np.array([tg.token for tg in targets], dtype=np.int32)
    n = pos.size
    w = None
    if weights is not None:
        w = np.ascontiguousarray(weights, dtype=np.float32)
        assert w.size == n, "one weight per target"
    logp = np.empty(n, dtype=np.float32)
    hits = ctypes.c_int64()
    dx = np.empty(t * d, dtype=np.float32) if w is not None else np.empty(0, dtype=np.float32)
    _ffi.check(_ffi.lib().rtq_lm_head(lm_head.ctx.handle, lm_head.handle, norm.ctypes.data, eps, offset,
                                      x.ctypes.data, t, pos.ctypes.data, tok.ctypes.data,
                                      None if w is None else w.ctypes.data, n, logp.ctypes.data,
                                      ctypes.byref(hits), dx.ctypes.data if w is not None else None), "rtq_lm_head")
    return logp, dx, int(hits.value)


def head_d(lm_head: HipFrozen, norm_ptr: int, x_ptr: int, t: int, pos_ptr: int, tok_ptr: int, weights_ptr: int,
           n: int, logp_ptr: int, hit_ptr: int, dx_ptr: int, eps: float = 1e-6, offset: float = 0.0,
           stream: int = 0) -> None:
    """Device-pointer variant (ints are device addresses; hit is int32 per target)."""
    _ffi.check(_ffi.lib().rtq_lm_head_d(lm_head.ctx.handle, lm_head.handle, norm_ptr, eps, offset, x_ptr, t, pos_ptr,
                                        tok_ptr, weights_ptr or None, n, logp_ptr, hit_ptr, dx_ptr or None,
                                        stream or None), "rtq_lm_head_d")
