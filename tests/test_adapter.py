"""Adapter writers / readers (llama.cpp LoRA GGUF, PEFT directory, AGLORA1) on the host, over a
stand-in for the device model's adapter accessors.  The AGLORA1 bytes are compared with a layout
encoded here from the format's definition (src/agentd.rs:177-181); the GGUF adapter is read back
with the container reader and checked against write_gguf_adapter's layout (src/rie.rs:342-364)."""
import json
import os
import struct

import numpy as np
import pytest

from rust_trainer_amd import adapter as AD
from rust_trainer_amd import gguf as G
from rust_trainer_amd.model import GGUF_LINEARS, LINEARS


class FakeModel:
    """lora_count / lora_info / lora / attach_lora / set_lora like GpuModel, on host arrays"""

    def __init__(self, n_layer, shapes, rank, alpha, kinds, seed=0):
        self.n_layer, self.shapes = n_layer, shapes
        self.config = {"n_layer": n_layer, "shapes": [list(x) for x in shapes]}
        self.attach_lora(rank, alpha, [LINEARS[k] for k in kinds])
        rng = np.random.default_rng(seed)
        for m in self.mods:
            m["a"] = rng.standard_normal(m["a"].shape).astype(np.float32)
            m["b"] = rng.standard_normal(m["b"].shape).astype(np.float32)

    def attach_lora(self, rank, alpha, targets=LINEARS, seed=1):
        kinds = [LINEARS.index(t) for t in targets]
        self.mods = []
        for layer in range(self.n_layer):
            for k in sorted(kinds):
                out, inp = self.shapes[k]
                self.mods.append(dict(layer=layer, which=k, name=f"blk.{layer}.{GGUF_LINEARS[k]}", rank=rank,
                                      in_dim=inp, out_dim=out, alpha=alpha, a=np.zeros((rank, inp), np.float32),
                                      b=np.zeros((out, rank), np.float32)))
        return 0

    def lora_count(self):
        return len(self.mods)

    def lora_info(self, i):
        return {k: v for k, v in self.mods[i].items() if k not in ("a", "b")}

    def lora(self, i):
        m = self.mods[i]
        return m["a"].copy(), m["b"].copy(), np.zeros_like(m["a"]), np.zeros_like(m["b"])

    def set_lora(self, i, a, b):
        self.mods[i]["a"] = np.asarray(a, np.float32).copy()
        self.mods[i]["b"] = np.asarray(b, np.float32).copy()


SHAPES = [(64, 32), (16, 32), (16, 32), (32, 64), (96, 32), (96, 32), (32, 96)]  # (out, in) per linear kind


def same_adapters(m1, m2):
    assert m1.lora_count() == m2.lora_count()
    for i in range(m1.lora_count()):
        assert m1.lora_info(i)["name"] == m2.lora_info(i)["name"]
        np.testing.assert_array_equal(m1.lora(i)[0], m2.lora(i)[0])
        np.testing.assert_array_equal(m1.lora(i)[1], m2.lora(i)[1])


def test_aglora_bytes_follow_the_format(tmp_path):
    m = FakeModel(2, SHAPES, 4, 8.0, [3, 0, 2])  # o, q, v
    p = tmp_path / "a.lora"
    AD.save_aglora(m, p)
    want = bytearray(b"AGLORA1\0") + struct.pack("<I", 4) + struct.pack("<f", 8.0) + struct.pack("<I", 6)
    for layer in range(2):
        for k, tag in ((0, b"q"), (2, b"v"), (3, b"o")):  # Q < K < V < O within a layer
            a, b, _, _ = m.lora([i for i in range(m.lora_count()) if m.lora_info(i)["layer"] == layer and
                                 m.lora_info(i)["which"] == k][0])
            want += struct.pack("<I", layer) + tag + struct.pack("<II", a.shape[1], b.shape[0])
            want += a.astype("<f4").tobytes() + b.astype("<f4").tobytes()
    assert p.read_bytes() == bytes(want)
    assert not os.path.exists(str(p) + ".tmp")
    fresh = FakeModel(2, SHAPES, 1, 1.0, [4])
    assert AD.load_aglora(fresh, p) == 6
    same_adapters(m, fresh)
    assert fresh.lora_info(0)["alpha"] == 8.0 and fresh.lora_info(0)["rank"] == 4
    p.write_bytes(p.read_bytes()[:-4])
    with pytest.raises(ValueError):
        AD.load_aglora(fresh, p)
    with pytest.raises(ValueError):
        AD.save_aglora(FakeModel(1, SHAPES, 2, 4.0, [4]), tmp_path / "mlp.lora")  # gate is not attention


def test_gguf_adapter_layout_and_round_trip(tmp_path):
    m = FakeModel(2, SHAPES, 4, 8.0, range(7))
    p = tmp_path / "adapter.gguf"
    AD.write_gguf_adapter(m, p, "qwen3")
    g = G.GgufFile.open(p)
    assert (g.get_str("general.architecture"), g.get_str("general.type"), g.get_str("adapter.type")) == \
        ("qwen3", "adapter", "lora")
    assert g.get_f32("adapter.lora.alpha") == 8.0
    ta = g.tensor("blk.1.ffn_down.weight.lora_a")
    tb = g.tensor("blk.1.ffn_down.weight.lora_b")
    assert ta.dims == (96, 4) and tb.dims == (4, 32) and ta.ty == tb.ty == 0  # ne [in, r] and [r, out], F32
    i = [k for k in range(m.lora_count()) if m.lora_info(k)["name"] == "blk.1.ffn_down"][0]
    np.testing.assert_array_equal(g.tensor_f32(ta), m.lora(i)[0])
    np.testing.assert_array_equal(g.tensor_f32(tb), m.lora(i)[1])
    g.close()
    fresh = FakeModel(2, SHAPES, 2, 2.0, [0])
    assert AD.read_gguf_adapter(fresh, p, "qwen3") == 14
    same_adapters(m, fresh)
    with pytest.raises(ValueError):
        AD.read_gguf_adapter(fresh, p, "llama")


def test_gguf_adapter_subset_gets_zero_adapters(tmp_path):
    """a file adapting only some blocks: the other blocks' adapters of those kinds are exact zeros"""
    m = FakeModel(1, SHAPES, 4, 8.0, [0, 2])
    p = tmp_path / "adapter.gguf"
    AD.write_gguf_adapter(m, p, "qwen3")
    fresh = FakeModel(3, SHAPES, 2, 2.0, [5])
    assert AD.read_gguf_adapter(fresh, p) == 2
    for i in range(fresh.lora_count()):
        inf = fresh.lora_info(i)
        a, b, _, _ = fresh.lora(i)
        if inf["layer"] == 0:
            np.testing.assert_array_equal(a, m.lora(inf["which"] // 2)[0])
        else:
            assert not a.any() and not b.any()


def test_peft_directory_round_trip(tmp_path):
    from safetensors.numpy import load_file

    m = FakeModel(2, SHAPES, 4, 8.0, range(7))
    d = tmp_path / "adapter"
    AD.save_adapter(m, d, AD.AdapterMeta(id="x", base_model="synthetic-qwen3"), arch="qwen3")
    st = load_file(str(d / AD.WEIGHTS_FILE))
    assert st["base_model.model.blk.0.attn_q.lora_A.weight"].shape == (4, 32)
    assert st["base_model.model.blk.0.attn_q.lora_B.weight"].shape == (64, 4)
    cfg = json.load(open(d / AD.CONFIG_FILE))
    assert cfg["peft_type"] == "LORA" and cfg["r"] == 4 and cfg["lora_alpha"] == 8.0
    assert cfg["target_modules"] == list(GGUF_LINEARS)
    meta = AD.read_meta(d)
    assert meta.rank == 4 and meta.alpha == 8.0 and meta.base_fingerprint
    assert (d / AD.GGUF_ADAPTER_FILE).exists()  # GGUF-named modules: the engine's adapter beside
    fresh = FakeModel(2, SHAPES, 4, 1.0, range(7))
    AD.load_adapter_into(fresh, d)
    same_adapters(m, fresh)
    other = FakeModel(2, [(o + 16, i) for o, i in SHAPES], 4, 1.0, range(7))
    with pytest.raises(ValueError):
        AD.load_adapter_into(other, d)  # fingerprint of a different model shape
