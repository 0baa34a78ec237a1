"""Adapter writers and readers over the device model's LoRA adapters — format-only consumers of
``Lora.a`` / ``Lora.b``, as in the reference:

* llama.cpp LoRA GGUF (``write_gguf_adapter`` / ``read_gguf_adapter``, src/rie.rs:342-411):
  ``general.architecture``, ``general.type = "adapter"``, ``adapter.type = "lora"``,
  ``adapter.lora.alpha``; per module ``<name>.weight.lora_a`` (ggml dims ``[in, r]``) and
  ``<name>.weight.lora_b`` (``[r, out]``), F32;
* PEFT directory (``save_adapter`` / ``load_adapter_into``, src/adapter.rs:68-175):
  ``adapter_model.safetensors`` (``base_model.model.<module>.lora_A.weight`` ``[r, in]``,
  ``lora_B.weight`` ``[out, r]``, F32), ``adapter_config.json``, ``trainer_meta.json``, and the GGUF
  adapter beside it (``adapter.gguf``) for GGUF-named modules;
* agentos-llm ``AGLORA1`` (``save_aglora`` / ``load_aglora``, src/agentd.rs:163-265): attention
  q / k / v / o only.

``src`` is any object with ``lora_count()``, ``lora_info(i)`` (``name``, ``which``, ``layer``,
``rank``, ``in_dim``, ``out_dim``, ``alpha``) and ``lora(i) -> (a, b, ga, gb)`` — ``GpuModel``.
Loaders re-attach the model's adapters with the file's rank (one rank for all modules, as
``attach_lora`` draws them) and set every A and B; linears of an attached kind that the file does
not hold get A = B = 0, which is an exact no-op whose gradients stay zero.  All writes go to
``<path>.tmp`` and are renamed into place.
"""
from __future__ import annotations

import dataclasses
import json
import os
import struct

import numpy as np

from .gguf import GGML_F32, GgufFile, GgufWriter, Value
from .model import GGUF_LINEARS, LINEARS

GGUF_ADAPTER_FILE = "adapter.gguf"  # src/rie.rs:44
WEIGHTS_FILE = "adapter_model.safetensors"  # src/adapter.rs:26-28
CONFIG_FILE = "adapter_config.json"
META_FILE = "trainer_meta.json"


def _atomic_bytes(path: str, data: bytes) -> None:
    tmp = str(path) + ".tmp"
    with open(tmp, "wb") as f:
        f.write(data)
    os.replace(tmp, path)


def _modules(src):
    """[(name, which, a [r x in], b [out x r], alpha)] in (block, linear) order"""
    out = []
    for i in range(src.lora_count()):
        inf = src.lora_info(i)
        a, b, _, _ = src.lora(i)
        out.append((inf["name"], inf["which"], a, b, inf["alpha"]))
    return out


# ------------------------------------------------------------------ llama.cpp LoRA GGUF
def write_gguf_adapter(src, path, arch: str) -> None:
    """src/rie.rs:346-364."""
    mods = _modules(src)
    if not mods:
        raise ValueError("no LoRA adapters")
    w = GgufWriter()
    w.kv("general.architecture", Value.String(arch))
    w.kv("general.type", Value.String("adapter"))
    w.kv("adapter.type", Value.String("lora"))
    w.kv("adapter.lora.alpha", Value.F32(mods[0][4]))
    for name, _, a, b, _ in mods:
        w.tensor(f"{name}.weight.lora_a", [a.shape[1], a.shape[0]], GGML_F32, np.ascontiguousarray(a, np.float32))
        w.tensor(f"{name}.weight.lora_b", [b.shape[1], b.shape[0]], GGML_F32, np.ascontiguousarray(b, np.float32))
    w.write(path)
    w.close()


def _install(model, found: dict, rank: int, alpha: float) -> int:
    """Re-attaches the model's adapters at ``rank`` on the kinds present in ``found``
    {(layer, which): (a, b)} and sets every A and B (zeros where the file holds none)."""
    kinds = sorted({w for (_, w) in found})
    model.attach_lora(rank, alpha, targets=[LINEARS[k] for k in kinds], seed=0)
    n = 0
    for i in range(model.lora_count()):
        inf = model.lora_info(i)
        ab = found.get((inf["layer"], inf["which"]))
        if ab is None:
            model.set_lora(i, np.zeros((rank, inf["in_dim"]), np.float32), np.zeros((inf["out_dim"], rank), np.float32))
            continue
        a, b = ab
        if a.shape != (rank, inf["in_dim"]) or b.shape != (inf["out_dim"], rank):
            raise ValueError(f"{inf['name']}: adapter shape mismatch")
        model.set_lora(i, a, b)
        n += 1
    return n


def _parse_module(name: str):
    """(layer, which) of a GGUF module name blk.{i}.{attn_q,...}"""
    parts = name.split(".")
    if len(parts) != 3 or parts[0] != "blk" or parts[2] not in GGUF_LINEARS:
        return None
    return int(parts[1]), GGUF_LINEARS.index(parts[2])


def read_gguf_adapter(model, path, arch: str | None = None) -> int:
    """src/rie.rs:369-411: returns the number of adapted modules."""
    g = GgufFile.open(path)
    try:
        if g.get_str("adapter.type") != "lora":
            raise ValueError("not a LoRA adapter GGUF")
        a_arch = g.get_str("general.architecture")
        if arch is not None and a_arch is not None and a_arch != arch:
            raise ValueError(f"adapter is for '{a_arch}', model is '{arch}'")
        alpha = g.get_f32("adapter.lora.alpha") or 0.0
        found, rank = {}, None
        for t in g.tensors():
            if not t.name.endswith(".weight.lora_a"):
                continue
            mod = t.name[: -len(".weight.lora_a")]
            key = _parse_module(mod)
            tb = g.tensor(mod + ".weight.lora_b")
            if key is None or tb is None:
                continue
            a = g.tensor_f32(t)  # [r x in]
            b = g.tensor_f32(tb)  # [out x r]
            if b.shape[1] != a.shape[0]:
                raise ValueError(f"{mod}: adapter shape mismatch")
            if rank is not None and a.shape[0] != rank:
                raise ValueError("adapters of different ranks in one file are not supported")
            rank = a.shape[0]
            found[key] = (a, b)
        if not found:
            raise ValueError("adapter matched no modules")
        n = _install(model, found, rank, alpha if alpha > 0 else float(rank))
        if n == 0:
            raise ValueError("adapter matched no modules")
        return n
    finally:
        g.close()


# ------------------------------------------------------------------ PEFT directory
@dataclasses.dataclass
class AdapterMeta:
    """trainer_meta.json (src/adapter.rs:32-46)."""
    id: str = ""
    base_model: str = ""
    base_fingerprint: str = ""
    rank: int = 0
    alpha: float = 0.0
    targets: list = dataclasses.field(default_factory=list)
    created_unix: int = 0
    train_steps: int = 0
    train_examples: int = 0
    final_train_loss: float | None = None
    eval: dict | None = None


def base_fingerprint(config: dict) -> str:
    """FNV-1a 64 over the model's hyper-parameters (src/adapter.rs:48-66: config and linear shapes,
    which the hyper-parameters fix), so an adapter is never applied to a different model shape.  The
    text hashed is this package's JSON of the device model's config, so the digest differs from the
    reference's for the same model."""
    h = 0xCBF29CE484222325
    text = json.dumps(config, sort_keys=True)
    for byte in text.encode():
        h ^= byte
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return f"{h:016x}"


def _peft(module: str, which: str) -> str:
    return f"base_model.model.{module}.lora_{which}.weight"


def _model_fingerprint(model) -> str:
    return base_fingerprint(getattr(model, "config", {}))


def save_adapter(model, directory, meta: AdapterMeta, arch: str | None = None) -> None:
    """src/adapter.rs:68-114."""
    from safetensors.numpy import save  # noqa: PLC0415 (optional dependency of this writer)

    os.makedirs(directory, exist_ok=True)
    mods = _modules(model)
    if not mods:
        raise ValueError("model has no LoRA adapters")
    tensors, targets = {}, []
    rank, alpha = mods[0][2].shape[0], mods[0][4]
    for name, _, a, b, al in mods:
        tensors[_peft(name, "A")] = np.ascontiguousarray(a, np.float32)
        tensors[_peft(name, "B")] = np.ascontiguousarray(b, np.float32)
        short = name.rsplit(".", 1)[-1]
        if short not in targets:
            targets.append(short)
    meta = dataclasses.replace(meta, rank=rank, alpha=alpha, targets=targets,
                               base_fingerprint=meta.base_fingerprint or _model_fingerprint(model))
    _atomic_bytes(os.path.join(directory, WEIGHTS_FILE),
                  save(tensors, metadata={"format": "pt", "base_fingerprint": meta.base_fingerprint}))
    cfg = {"peft_type": "LORA", "task_type": "CAUSAL_LM", "base_model_name_or_path": meta.base_model, "r": rank,
           "lora_alpha": alpha, "lora_dropout": 0.0, "bias": "none", "fan_in_fan_out": False, "use_rslora": False,
           "target_modules": targets}
    _atomic_bytes(os.path.join(directory, CONFIG_FILE), json.dumps(cfg, indent=2).encode())
    _atomic_bytes(os.path.join(directory, META_FILE), json.dumps(dataclasses.asdict(meta), indent=2).encode())
    if arch is not None and all(n.startswith("blk.") for n, *_ in mods):
        write_gguf_adapter(model, os.path.join(directory, GGUF_ADAPTER_FILE), arch)


def read_meta(directory) -> AdapterMeta:
    d = json.load(open(os.path.join(directory, META_FILE)))
    return AdapterMeta(**{k: v for k, v in d.items() if k in {f.name for f in dataclasses.fields(AdapterMeta)}})


def load_adapter_into(model, directory) -> AdapterMeta:
    """src/adapter.rs:131-165."""
    from safetensors.numpy import load_file  # noqa: PLC0415

    meta = read_meta(directory)
    fp = _model_fingerprint(model)
    if meta.base_fingerprint and meta.base_fingerprint != fp:
        raise ValueError(f"adapter was trained for base {meta.base_fingerprint} but this model is {fp}")
    st = load_file(os.path.join(directory, WEIGHTS_FILE))
    found, rank = {}, None
    for key, a in st.items():
        if not (key.startswith("base_model.model.") and key.endswith(".lora_A.weight")):
            continue
        mod = key[len("base_model.model."): -len(".lora_A.weight")]
        lk = _parse_module(mod)
        b = st.get(_peft(mod, "B"))
        if lk is None or b is None:
            continue
        if rank is not None and a.shape[0] != rank:
            raise ValueError("adapters of different ranks in one file are not supported")
        rank = a.shape[0]
        found[lk] = (a, b)
    if not found:
        raise ValueError("adapter matched no modules")
    _install(model, found, rank, meta.alpha)
    return meta


# ------------------------------------------------------------------ agentos-llm AGLORA1
_AG_TAGS = {0: b"q", 1: b"k", 2: b"v", 3: b"o"}  # q_proj, k_proj, v_proj, o_proj (Q < K < V < O)


def save_aglora(model, path) -> None:
    """src/agentd.rs:177-219: "AGLORA1\\0", rank u32, alpha f32, count u32, then per (layer, tag)
    in (layer, Q < K < V < O) order: layer u32, tag u8, in u32, out u32, A [r x in] f32, B [out x r] f32."""
    mods = _modules(model)
    items = []
    for name, which, a, b, alpha in mods:
        if which not in _AG_TAGS:
            raise ValueError(f"{name}: AGLORA1 holds attention q/k/v/o only")
        items.append((int(name.split(".")[1]), which, a, b, alpha))
    items.sort(key=lambda x: (x[0], x[1]))
    rank = items[0][2].shape[0] if items else 0
    alpha = items[0][4] if items else 0.0
    out = bytearray(b"AGLORA1\0")
    out += struct.pack("<IfI", rank, alpha, len(items))
    for layer, which, a, b, _ in items:
        out += struct.pack("<I", layer) + _AG_TAGS[which] + struct.pack("<II", a.shape[1], b.shape[0])
        out += np.ascontiguousarray(a, "<f4").tobytes() + np.ascontiguousarray(b, "<f4").tobytes()
    _atomic_bytes(path, bytes(out))


def load_aglora(model, path) -> int:
    """src/agentd.rs:221-265: returns the pair count."""
    b = open(path, "rb").read()
    if len(b) < 20 or b[:8] != b"AGLORA1\0":
        raise ValueError("not an agentos LoRA adapter")
    rank, alpha, n = struct.unpack_from("<IfI", b, 8)
    at, found = 20, {}
    tags = {v: k for k, v in _AG_TAGS.items()}
    for _ in range(n):
        if at + 13 > len(b):
            raise ValueError("adapter file is cut short")
        layer, = struct.unpack_from("<I", b, at)
        tag = b[at + 4: at + 5]
        inp, outd = struct.unpack_from("<II", b, at + 5)
        at += 13
        count = rank * inp + outd * rank
        if at + count * 4 > len(b):
            raise ValueError("adapter file is cut short")
        vals = np.frombuffer(b, "<f4", count, at).astype(np.float32)
        at += count * 4
        if tag not in tags:
            raise ValueError(f"unknown AGLORA1 tag {tag!r}")
        found[(layer, tags[tag])] = (vals[: rank * inp].reshape(rank, inp), vals[rank * inp:].reshape(outd, rank))
    loaded = _install(model, found, rank, alpha)
    if loaded != len(found):
        raise ValueError(f"adapter has {len(found)} pairs, {loaded} matched the model")
    return loaded
