"""The model loader's hyper-parameters and refusals (rtq_model_config_from_gguf, the device-free
part of rtq_model_from_gguf), against load_gguf_from (src/rie.rs:164-260), and the packed-batch
layout (pack / Packed, src/model.rs:234-290).  CPU only: synthetic GGUF images carrying the keys.

The GGUF key names for the settings the reference's loader refuses follow llama.cpp's conventions
(``<arch>.attention.sliding_window``, ``<arch>.attn_logit_softcapping``, ...); rie-core, which reads
them in the reference, is absent, so which spelling it reads is unpinned.
"""
import numpy as np
import pytest

from rust_trainer_amd import RtqError, gguf as G
from rust_trainer_amd.model import model_config
from rust_trainer_amd.packing import answer_targets, pack

UNSUPPORTED = 2


def image(arch="qwen3", extra=(), tensors=(), n_layer=1):
    s = G.SyntheticSpec(arch=arch, wtype=G.GGML_F32, n_layer=n_layer, n_embd=64, n_head=4, n_head_kv=2, head_dim=16,
                        rope_dim=16, n_ff=96, n_vocab=40)
    w = s.writer()
    try:
        for k, v in extra:
            w.kv(k, v)
        for name, dims, data in tensors:
            w.tensor(name, dims, G.GGML_F32, np.ascontiguousarray(data, np.float32).view(np.uint8))
        return G.GgufFile.from_bytes(w.to_bytes())
    finally:
        w.close()


def test_plain_config():
    c = model_config(image())
    assert (c["n_layer"], c["n_embd"], c["n_head"], c["n_head_kv"], c["head_dim"], c["n_ff"], c["n_vocab"]) == \
        (1, 64, 4, 2, 16, 96, 40)
    assert c["rope_neox"] == 1 and c["qk_norm"] == 1 and c["kv_f16"] == 1 and c["tied"] == 1
    assert c["rope_freq_scale"] == 1.0 and c["n_rope_factors"] == 0
    c = model_config(image("llama"))
    assert c["rope_neox"] == 0 and c["qk_norm"] == 0


@pytest.mark.parametrize("arch", ["gemma2", "phi3", "qwen3moe", "mamba"])
def test_untrainable_architectures_are_refused(arch):
    s = G.SyntheticSpec(arch="qwen3", wtype=G.GGML_F32, n_layer=1, n_embd=64, n_head=4, n_head_kv=2, head_dim=16,
                        rope_dim=16, n_ff=96, n_vocab=40)
    w = G.GgufWriter()
    try:
        for k, v in s.metadata():
            w.kv(k.replace("qwen3", arch) if k != "general.architecture" else k,
                 G.Value.String(arch) if k == "general.architecture" else v)
        for i, (name, ty, dims) in enumerate(s.plan()):
            w.tensor(name, dims, ty, s.tensor_values(i, name, ty, dims))
        g = G.GgufFile.from_bytes(w.to_bytes())
    finally:
        w.close()
    with pytest.raises(RtqError) as e:
        model_config(g)
    assert e.value.status == UNSUPPORTED and "not trainable" in str(e.value)


@pytest.mark.parametrize("key,value", [
    ("qwen3.attention.sliding_window", G.Value.U32(4096)),
    ("qwen3.attn_logit_softcapping", G.Value.F32(50.0)),
    ("qwen3.final_logit_softcapping", G.Value.F32(30.0)),
    ("qwen3.logit_scale", G.Value.F32(0.5)),
    ("qwen3.embedding_scale", G.Value.F32(8.0)),
    ("qwen3.residual_scale", G.Value.F32(0.2)),
    ("qwen3.attention.scale", G.Value.F32(0.125)),
    ("qwen3.expert_count", G.Value.U32(8)),
    ("qwen3.rope.scaling.type", G.Value.String("yarn")),
])
def test_non_plain_settings_are_refused(key, value):
    with pytest.raises(RtqError) as e:
        model_config(image(extra=[(key, value)]))
    assert e.value.status == UNSUPPORTED


@pytest.mark.parametrize("key,value", [
    ("qwen3.attention.sliding_window", G.Value.U32(0)),
    ("qwen3.logit_scale", G.Value.F32(1.0)),
    ("qwen3.attention.scale", G.Value.F32(0.25)),  # 1 / sqrt(head_dim 16)
    ("qwen3.rope.scaling.type", G.Value.String("none")),
])
def test_plain_values_of_those_keys_load(key, value):
    assert model_config(image(extra=[(key, value)]))["n_layer"] == 1


def test_post_norm_layers_are_refused():
    with pytest.raises(RtqError) as e:
        model_config(image(tensors=[("blk.0.post_attention_norm.weight", (64,), np.ones(64))]))
    assert e.value.status == UNSUPPORTED and "post-norm" in str(e.value)


def test_linear_rope_scaling_and_frequency_factors():
    c = model_config(image(extra=[("qwen3.rope.scaling.type", G.Value.String("linear")),
                                  ("qwen3.rope.scaling.factor", G.Value.F32(4.0))]))
    assert c["rope_freq_scale"] == 0.25
    c = model_config(image(extra=[("qwen3.rope.scale_linear", G.Value.F32(2.0))]))
    assert c["rope_freq_scale"] == 0.5
    c = model_config(image(tensors=[("rope_freqs.weight", (8,), np.linspace(1, 8, 8))]))
    assert c["n_rope_factors"] == 8
    with pytest.raises(RtqError):  # longer than rope_dim / 2
        model_config(image(tensors=[("rope_freqs.weight", (9,), np.ones(9))]))


def test_pack_layout_as_the_reference():
    prompt = list(range(100, 113))
    seqs = [prompt + [1, 2, 3, 4, 5], prompt + [6, 7, 8, 9, 10, 11, 12, 13, 14], prompt + [15, 16, 17]]
    p = pack(seqs)
    assert p.shared == 13
    assert p.tokens == prompt + seqs[0][13:] + seqs[1][13:] + seqs[2][13:]
    assert p.positions == list(range(13)) + list(range(13, 18)) + list(range(13, 22)) + list(range(13, 16))
    assert p.segments == [0] * 13 + [1] * 5 + [2] * 9 + [3] * 3
    assert p.offsets == [13, 18, 27]
    for k, s in enumerate(seqs):
        for i in range(len(s)):
            assert p.tokens[p.index(k, i)] == s[i] and p.positions[p.index(k, i)] == i
        for t, u in zip(answer_targets(s, 12), p.map_targets(k, answer_targets(s, 12))):
            assert p.tokens[u.pos] == s[t.pos] and u.token == t.token
    # a batch of one is just the sequence; identical sequences keep a token of their own
    one = pack(seqs[:1])
    assert one.shared == 0 and one.tokens == seqs[0]
    same = pack([prompt, prompt])
    assert same.shared == 12 and same.segments == [0] * 12 + [1, 2]
