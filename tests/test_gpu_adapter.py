"""GPU: adapters written from a device model and read into a fresh one (llama.cpp LoRA GGUF, PEFT
directory, AGLORA1) give the same adapters and bit-identical log-probs."""
import numpy as np
import pytest

import oracle as O
import rust_trainer_amd as rt
from model_cases import sequence, tiny_spec
from rust_trainer_amd import adapter as AD
from rust_trainer_amd import gguf as G

pytestmark = pytest.mark.gpu


def trained_model(ctx, g, targets):
    m = rt.GpuModel.from_gguf(g, ctx=ctx)
    m.attach_lora(4, 8.0, targets=targets, seed=3)
    rng = np.random.default_rng(0)
    for i in range(m.lora_count()):
        inf = m.lora_info(i)
        m.set_lora(i, rng.standard_normal((4, inf["in_dim"])).astype(np.float32) * 0.1,
                   rng.standard_normal((inf["out_dim"], 4)).astype(np.float32) * 0.05)
    return m


@pytest.mark.parametrize("fmt", ["gguf", "peft", "aglora"])
def test_adapter_round_trip_on_device(ctx, tmp_path, fmt):
    g = G.GgufFile.from_bytes(tiny_spec(O.Q4_0, n_layer=2).build())
    targets = rt.model.LINEARS if fmt != "aglora" else ("q_proj", "k_proj", "v_proj", "o_proj")
    m = trained_model(ctx, g, targets)
    toks, pos, tok = sequence(512, 32, 12)
    tg = [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)]
    lp0, _ = m.score(toks, tg)
    path = tmp_path / ("adapter.gguf" if fmt == "gguf" else "adapter.lora" if fmt == "aglora" else "dir")
    fresh = rt.GpuModel.from_gguf(g, ctx=ctx)
    if fmt == "gguf":
        AD.write_gguf_adapter(m, path, "qwen3")
        assert AD.read_gguf_adapter(fresh, path, "qwen3") == m.lora_count()
    elif fmt == "peft":
        AD.save_adapter(m, path, AD.AdapterMeta(id="t"), arch="qwen3")
        AD.load_adapter_into(fresh, path)
    else:
        AD.save_aglora(m, path)
        assert AD.load_aglora(fresh, path) == m.lora_count()
    assert fresh.lora_count() == m.lora_count()
    for i in range(m.lora_count()):
        a0, b0, _, _ = m.lora(i)
        a1, b1, _, _ = fresh.lora(i)
        np.testing.assert_array_equal(a0, a1)
        np.testing.assert_array_equal(b0, b1)
        assert fresh.lora_info(i)["alpha"] == 8.0
    lp1, _ = fresh.score(toks, tg)
    np.testing.assert_array_equal(lp0, lp1)
    m.close()
    fresh.close()
