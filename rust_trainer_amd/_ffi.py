"""ctypes binding of librtq.so (include/rtq.h).

The library is built in-tree by ``__graft_entry__.build()`` (``rust_trainer_amd/csrc/build.py``).
There is no CPU fallback: a missing library, a missing device or a failing call raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "librtq.so")

RTQ_OK = 0
STATUS_NAMES = {0: "OK", 1: "ERR_INVALID", 2: "ERR_UNSUPPORTED", 3: "ERR_HIP", 4: "ERR_NO_DEVICE"}

TYPE_Q4_0, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K = 2, 8, 12, 14
# trainer-native FrozenWeight storage (src/frozen.rs:33-45): f32, and Q8_0 with f32 block scales
TYPE_F32, TYPE_TQ8_0 = 0, 264

# every symbol include/rtq.h declares, with (restype, argtypes)
_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i = ctypes.c_int
_f = ctypes.c_float
_sz = ctypes.c_size_t


class RtqLora(ctypes.Structure):
    _fields_ = [("rank", ctypes.c_int64), ("alpha", ctypes.c_float), ("a", ctypes.c_void_p),
                ("b", ctypes.c_void_p), ("enabled", ctypes.c_int)]


_LP = ctypes.POINTER(RtqLora)


class RtqModelConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ("n_layer", "n_embd", "n_head", "n_head_kv", "head_dim", "rope_dim",
                                              "n_ff", "n_vocab")] + \
               [(n, ctypes.c_float) for n in ("rms_eps", "norm_offset", "rope_base", "rope_freq_scale")] + \
               [(n, ctypes.c_int) for n in ("rope_neox", "qk_norm", "kv_f16", "tied")] + \
               [("n_rope_factors", ctypes.c_int64)]

SIGNATURES = {
    "rtq_version": (ctypes.c_char_p, []),
    "rtq_last_error": (ctypes.c_char_p, []),
    "rtq_ctx_create": (_i, [_i, ctypes.POINTER(_p)]),
    "rtq_ctx_destroy": (None, [_p]),
    "rtq_ctx_stream": (_p, [_p]),
    "rtq_ctx_reserve": (_i, [_p, _i64, _i64, _i64, _i64]),
    "rtq_ctx_set_timing": (_i, [_p, _i, ctypes.c_char_p]),
    "rtq_ctx_timing_count": (_i, [_p]),
    "rtq_ctx_timing_get": (_i, [_p, _i, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_i64),
                                ctypes.POINTER(ctypes.c_double)]),
    "rtq_ctx_timing_work": (_i, [_p, _i, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    "rtq_ctx_timing_reset": (None, [_p]),
    "rtq_weight_create": (_i, [_p, _i, _p, _sz, _i64, _i64, ctypes.POINTER(_p)]),
    "rtq_weight_destroy": (None, [_p]),
    "rtq_weight_out_dim": (_i64, [_p]),
    "rtq_weight_in_dim": (_i64, [_p]),
    "rtq_weight_nbytes": (_sz, [_p]),
    "rtq_weight_type": (_i, [_p]),
    "rtq_frozen_forward": (_i, [_p, _p, _p, _i64, _p]),
    "rtq_frozen_backward_input": (_i, [_p, _p, _p, _i64, _p]),
    "rtq_frozen_row": (_i, [_p, _p, _i64, _p]),
    "rtq_linear_forward": (_i, [_p, _p, _p, _LP, _p, _i64, _p]),
    "rtq_linear_backward": (_i, [_p, _p, _LP, _p, _p, _i64, _p, _p, _p]),
    "rtq_frozen_forward_d": (_i, [_p, _p, _p, _i64, _p, _p]),
    "rtq_frozen_backward_input_d": (_i, [_p, _p, _p, _i64, _p, _p]),
    "rtq_frozen_rows_d": (_i, [_p, _p, _i64, _i64, _p, _p]),
    "rtq_linear_forward_d": (_i, [_p, _p, _p, _LP, _p, _i64, _p, _p]),
    "rtq_linear_backward_d": (_i, [_p, _p, _LP, _p, _p, _i64, _p, _p, _p, _p]),
    "rtq_debug_quantize_acts": (_i, [_p, _p, _p, _i64, _p]),
    "rtq_debug_isums_per_row": (_i64, [_p]),
    "rtq_debug_block_isums": (_i, [_p, _p, _p, _i64, _p]),
    "rtq_frozen_gather": (_i, [_p, _p, _p, _i64, _p]),
    "rtq_frozen_gather_d": (_i, [_p, _p, _p, _i64, _p, _p]),
    "rtq_lm_head": (_i, [_p, _p, _p, _f, _f, _p, _i64, _p, _p, _p, _i64, _p, ctypes.POINTER(_i64), _p]),
    "rtq_lm_head_d": (_i, [_p, _p, _p, _f, _f, _p, _i64, _p, _p, _p, _i64, _p, _p, _p, _p]),
    # device-resident training step
    "rtq_linear_forward_noalloc_d": (_i, [_p, _p, _p, _LP, _p, _i64, _p, _p]),
    "rtq_model_from_gguf": (_i, [_p, _p, ctypes.POINTER(_p)]),
    "rtq_model_config_from_gguf": (_i, [_p, _p]),
    "rtq_model_destroy": (None, [_p]),
    "rtq_model_get_config": (_i, [_p, _p]),
    "rtq_model_attach_lora": (_i, [_p, _i64, _f, ctypes.c_uint32, ctypes.c_uint64, ctypes.POINTER(_i64)]),
    "rtq_model_lora_count": (_i64, [_p]),
    "rtq_model_lora_info": (_i, [_p, _i64, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i64),
                                 ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_f)]),
    "rtq_model_lora_get": (_i, [_p, _i64, _p, _p, _p, _p]),
    "rtq_model_lora_set": (_i, [_p, _i64, _p, _p]),
    "rtq_model_lora_device": (_i, [_p, _i64, ctypes.POINTER(_p), ctypes.POINTER(_p), ctypes.POINTER(_p),
                                   ctypes.POINTER(_p), ctypes.POINTER(_i64)]),
    "rtq_model_zero_grad": (_i, [_p]),
    "rtq_model_forward_backward": (_i, [_p, _p, _i64, _p, _p, _p, _i64, _p, ctypes.POINTER(_i64)]),
    "rtq_model_forward_backward_packed": (_i, [_p, _p, _i64, _p, _p, _p, _p, _p, _i64, _p, ctypes.POINTER(_i64)]),
    "rtq_model_set_checkpointing": (_i, [_p, _i]),
    "rtq_model_checkpointing": (_i, [_p]),
    "rtq_model_set_attention": (_i, [_p, _i]),
    "rtq_model_attention_fused": (_i, [_p]),
    "rtq_model_graph_replays": (_i64, [_p]),
    "rtq_model_debug_capture": (_i, [_p, _i64]),
    "rtq_model_debug_tensor": (_i, [_p, ctypes.c_char_p, _p, _i64]),
    # GGUF v3 container
    "rtq_gguf_open": (_i, [ctypes.c_char_p, ctypes.POINTER(_p)]),
    "rtq_gguf_from_bytes": (_i, [_p, _sz, ctypes.POINTER(_p)]),
    "rtq_gguf_close": (None, [_p]),
    "rtq_gguf_version": (ctypes.c_uint32, [_p]),
    "rtq_gguf_kv_count": (_i64, [_p]),
    "rtq_gguf_find_kv": (_i64, [_p, ctypes.c_char_p]),
    "rtq_gguf_kv": (_i, [_p, _i64, ctypes.POINTER(_p), ctypes.POINTER(_i), ctypes.POINTER(_i),
                         ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(_p)]),
    "rtq_gguf_get_str": (_i, [_p, ctypes.c_char_p, ctypes.POINTER(_p), ctypes.POINTER(ctypes.c_uint64)]),
    "rtq_gguf_get_f64": (_i, [_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_double)]),
    "rtq_gguf_tensor_count": (_i64, [_p]),
    "rtq_gguf_find_tensor": (_i64, [_p, ctypes.c_char_p]),
    "rtq_gguf_tensor": (_i, [_p, _i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_i), ctypes.POINTER(_i),
                             ctypes.POINTER(_i64), ctypes.POINTER(_p), ctypes.POINTER(_sz)]),
    "rtq_weight_from_gguf": (_i, [_p, _p, ctypes.c_char_p, ctypes.POINTER(_p)]),
    "rtq_gguf_writer_create": (_i, [ctypes.POINTER(_p)]),
    "rtq_gguf_writer_destroy": (None, [_p]),
    "rtq_gguf_writer_kv": (_i, [_p, ctypes.c_char_p, _i, _i, ctypes.c_uint64, _p]),
    "rtq_gguf_writer_tensor": (_i, [_p, ctypes.c_char_p, _i, _i, ctypes.POINTER(_i64), _p, _sz]),
    "rtq_gguf_writer_bytes": (_i, [_p, ctypes.POINTER(_p), ctypes.POINTER(_sz)]),
    "rtq_gguf_writer_write": (_i, [_p, ctypes.c_char_p]),
}

_LIB = None


class RtqError(RuntimeError):
    def __init__(self, status: int, what: str, msg: str):
        super().__init__(f"{what} failed: {STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


def _share_torch_hip_runtime() -> None:
    """PyTorch-ROCm ships its own libamdhip64.so.7.  Loading it first makes librtq.so's dependency
    on libamdhip64.so.7 resolve to that same runtime, so tensors and streams from torch and the
    library's kernels live in one HIP runtime (two runtimes in one process do not share devices)."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def lib() -> ctypes.CDLL:
    """Loads librtq.so (raises if it has not been built)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        _share_torch_hip_runtime()
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(status: int, what: str) -> None:
    if status != RTQ_OK:
        msg = lib().rtq_last_error()
        raise RtqError(status, what, msg.decode() if msg else "")
