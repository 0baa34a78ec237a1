"""The configs[2] training step at full size - Qwen3-0.6B shape, all 28 blocks, the tied 151936-row
Q4_0 head, LoRA r = 16 on every projection, 512 tokens with loss on the last 256 - through the
tile plans that size picks, checked by properties that need no oracle run of the whole model (the
per-op parity of one block at this shape is in tests/test_gpu_block_ops.py):

* the log-probs are finite and the loss is that of an untrained model (mean -log p within
  [0.5, 2] x log(vocab));
* activation recomputation changes nothing beyond f32 rounding (tests/gradcheck.rs:199-212:
  log-probs and every adapter gradient within 1e-5 x max(|a|, 1));
* a step replayed from the captured HIP graph equals the same step run eagerly, bit for bit;
* the same step repeated reproduces every bit (no atomics in the step's reductions);
* the block's RMSNorms formed inside the next linear's activation kernel give the bits of the norm
  kernel run first (a model loaded with RTQ_NORM_FUSE=0), on 16-, 8- and 4-token tiles.
"""
import numpy as np
import pytest

import rust_trainer_amd as rt
from model_cases import adapters
from rust_trainer_amd import gguf as G
from rust_trainer_amd import synth

pytestmark = pytest.mark.gpu

NAMES = ("q", "k", "v", "o", "gate", "up", "down")


def grads(model):
    return [np.concatenate([ga.ravel(), gb.ravel()]) for ga, gb in (model.lora(i)[2:] for i in range(model.lora_count()))]


def test_config2_full_step_properties(ctx, monkeypatch):
    spec = G.SyntheticSpec.preset("qwen3-0.6b", G.GGML_Q4_0)
    g = G.GgufFile.from_bytes(spec.build(workers=16))
    lora = adapters(g, 16, 32.0, b_std=0.01)
    t, n = 512, 256
    toks = (synth.Rng(7).next_u64(t) % np.uint64(spec.n_vocab)).astype(np.int32)
    targets = [rt.Target(int(p), int(toks[p + 1])) for p in range(t - n - 1, t - 1)]
    wts = np.full(n, 1.0 / n, np.float32)

    def load(graph, c=None):
        if graph:
            monkeypatch.delenv("RTQ_STEP_GRAPH", raising=False)
        else:
            monkeypatch.setenv("RTQ_STEP_GRAPH", "0")
        m = rt.GpuModel.from_gguf(g, ctx=c or ctx)
        monkeypatch.delenv("RTQ_STEP_GRAPH", raising=False)
        m.attach_lora(16, 32.0, seed=1)
        for i in range(m.lora_count()):
            inf = m.lora_info(i)
            m.set_lora(i, *lora[(inf["layer"], NAMES[inf["which"]])])
        return m

    def step(m):
        m.zero_grad()
        lp, hits = m.forward_backward(toks, targets, wts)
        return lp, hits, grads(m)

    model = load(graph=True)
    assert model.config["n_layer"] == 28 and model.lora_count() == 28 * 7
    runs = [step(model) for _ in range(5)]  # eager, eager (the first allocated), captured, replays
    assert model.graph_replays >= 2
    lp, hits, gr = runs[0]
    assert np.isfinite(lp).all() and all(np.isfinite(x).all() for x in gr)
    loss = float(-lp.mean())
    print(f"mean loss {loss:.3f} (log vocab {np.log(spec.n_vocab):.3f}), hits {hits}")
    assert 0.5 * np.log(spec.n_vocab) <= loss <= 2.0 * np.log(spec.n_vocab)
    for lp_r, hits_r, gr_r in runs[1:]:  # replays (and the captured step) equal the eager step bitwise
        np.testing.assert_array_equal(lp_r, lp)
        assert hits_r == hits
        for a, b in zip(gr_r, gr):
            np.testing.assert_array_equal(a, b)
    eager = load(graph=False)
    lp_e, hits_e, gr_e = step(eager)
    assert eager.graph_replays == 0
    np.testing.assert_array_equal(lp_e, lp)
    for a, b in zip(gr_e, gr):
        np.testing.assert_array_equal(a, b)
    eager.close()
    monkeypatch.setenv("RTQ_NORM_FUSE", "0")
    unfused = load(graph=False)
    monkeypatch.delenv("RTQ_NORM_FUSE")
    lp_u, hits_u, gr_u = step(unfused)
    np.testing.assert_array_equal(lp_u, lp)
    assert hits_u == hits
    for a, b in zip(gr_u, gr):
        np.testing.assert_array_equal(a, b)
    unfused.close()
    for tt in ("16", "4"):  # the norms' activation kernel on 16- and 4-token tiles (default 8): same bits
        monkeypatch.setenv("RTQ_ACT_TT", tt)
        c2 = rt.Context(0)
        monkeypatch.delenv("RTQ_ACT_TT")
        other = load(graph=False, c=c2)
        lp_o, hits_o, gr_o = step(other)
        np.testing.assert_array_equal(lp_o, lp)
        assert hits_o == hits
        for a, b in zip(gr_o, gr):
            np.testing.assert_array_equal(a, b)
        other.close()
        c2.close()
    model.checkpointing = True
    lp_c, hits_c, gr_c = step(model)
    assert model.checkpointing is True and hits_c == hits
    assert np.all(np.abs(lp_c - lp) <= 1e-5 * np.maximum(np.abs(lp), 1.0))
    worst = max(float((np.abs(a - b) / np.maximum(np.abs(b), 1.0)).max()) for a, b in zip(gr_c, gr))
    print(f"recompute vs keep: max |d logp| {np.abs(lp_c - lp).max():.2e}, worst gradient {worst:.2e}")
    assert worst <= 1e-5
    model.close()
