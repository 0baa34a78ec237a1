"""rust_trainer_amd — MI355X (gfx950) frozen quantised-matmul path for Rust_Trainer-style LoRA training.

The product is ``librtq.so`` (C ABI, ``include/rtq.h``): hand-written gfx950 kernels for the GGUF
frozen linear's forward (``y = W_q.x + (alpha/r) B.A.x``), input gradient (``dx = W_q^T.dy``) and
LoRA gradients, plus the GGUF v3 container reader / writer the loader reads weights through.
This package is the host-side mirror of the reference's plugin interface (``FrozenMatmul``,
``Lora``, ``Linear``, ``GgufFile``, ``GgufWriter``, ``SyntheticSpec``) over that C ABI.
"""
from ._ffi import RtqError, TYPE_F32, TYPE_Q4_0, TYPE_Q4_K, TYPE_Q6_K, TYPE_Q8_0, TYPE_TQ8_0, lib  # noqa: F401
from .frozen import Context, FrozenMatmul, HipFrozen, default_context, pack_trainer_q8_0  # noqa: F401
from .gguf import GgufFile, GgufWriter, SyntheticSpec, Value  # noqa: F401
from .head import Target, answer_targets, embed_tokens, head  # noqa: F401
from .linear import Linear, Lora  # noqa: F401
from .model import GpuModel  # noqa: F401

__all__ = ["Context", "FrozenMatmul", "HipFrozen", "Linear", "Lora", "RtqError", "default_context", "lib",
           "TYPE_Q4_0", "TYPE_Q8_0", "TYPE_Q4_K", "TYPE_Q6_K", "TYPE_F32", "TYPE_TQ8_0", "pack_trainer_q8_0",
           "GgufFile", "GgufWriter", "SyntheticSpec", "Value", "Target", "answer_targets", "embed_tokens", "head", "GpuModel"]
