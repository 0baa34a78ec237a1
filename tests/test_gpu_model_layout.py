"""Step-level invariants of the device training step, restated from the reference's own tests:

* checkpointing (recomputing each block's forward in the backward) changes nothing
  (tests/gradcheck.rs:199-210: log-probs and every ga / gb within 1e-5 * max(|a|, 1));
* a packed shared-prompt batch gives the log-probs and adapter gradients of running its examples
  separately (tests/gradcheck.rs:279-338 on an F32 model: 1e-5; tests/engine.rs:296-326 on a
  quantised model: 1e-4 on log-probs; the device's log-probs are bit-identical, its gradients
  within 1e-5);
* the packed step agrees with the oracle's packed step (F32 weights, 1e-3);
* linear RoPE scaling and rope_freqs.weight factors reach the device step (F32 weights against the
  oracle with the same scaling, 1e-3).
"""
import numpy as np
import pytest

import oracle as O
import rust_trainer_amd as rt
from model_cases import adapters, oracle_model, sequence, tiny_spec
from rust_trainer_amd import gguf as G
from rust_trainer_amd.packing import answer_targets, pack

pytestmark = pytest.mark.gpu

NAMES = O.LINEARS


def model_with(ctx, g, rank, alpha, b_std=0.05, seed=11):
    model = rt.GpuModel.from_gguf(g, ctx=ctx)
    model.attach_lora(rank, alpha, seed=1)
    lora = adapters(g, rank, alpha, seed=seed, b_std=b_std)
    for i in range(model.lora_count()):
        inf = model.lora_info(i)
        model.set_lora(i, *lora[(inf["layer"], NAMES[inf["which"]])])
    return model, lora


def all_grads(model):
    return [np.concatenate([ga.ravel(), gb.ravel()]) for ga, gb in (model.lora(i)[2:] for i in range(model.lora_count()))]


@pytest.mark.parametrize("wtype,fused", [(O.F32, False), (O.Q4_0, False), (O.Q6_K, False), (O.Q4_0, True)])
def test_checkpointing_changes_nothing(ctx, wtype, fused):
    spec = tiny_spec(wtype, n_layer=3)
    g = G.GgufFile.from_bytes(spec.build())
    model, _ = model_with(ctx, g, 4, 8.0)
    model.fused_attention = fused
    toks, pos, tok = sequence(spec.n_vocab, 48, 20, 3)
    targets = [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)]
    wts = np.full(20, 0.05, np.float32)
    out = {}
    for ck in (True, False, True):
        model.checkpointing = ck
        model.zero_grad()
        lp, hits = model.forward_backward(toks, targets, wts)
        assert model.checkpointing is ck
        out.setdefault(ck, []).append((lp, hits, all_grads(model)))
    (lp1, h1, g1), (lp3, h3, g3) = out[True]
    lp0, h0, g0 = out[False][0]
    assert h1 == h0
    assert np.all(np.abs(lp1 - lp0) <= 1e-5 * np.maximum(np.abs(lp0), 1.0))
    for a, b in zip(g1, g0):
        assert np.all(np.abs(a - b) <= 1e-5 * np.maximum(np.abs(b), 1.0)), "checkpointing changed grads"
    # the device step is deterministic: a repeated step reproduces every bit
    np.testing.assert_array_equal(lp1, lp3)
    for a, b in zip(g1, g3):
        np.testing.assert_array_equal(a, b)
    model.close()


def packed_batch(V, prompt_len, extras, seed):
    rng = O.Rng(seed)
    prompt = [int(v) for v in (rng.vec_uniform_sym(prompt_len, 1.0) * 0.5 + 0.5) * (V - 1)]
    seqs = []
    for extra, start in extras:
        seqs.append((prompt + [int(v) for v in (rng.vec_uniform_sym(extra, 1.0) * 0.5 + 0.5) * (V - 1)], start))
    return seqs


MIXED = "Q4_K/Q6_K"  # configs[3]'s mix: Q4_K attention / gate / up, Q6_K down and output


PACKED_CASES = {
    # three examples sharing a 70-token prompt (more than one 64-token block), one answer starting
    # inside the shared part (tests/gradcheck.rs:289-295)
    "short": (dict(), 70, [(50, 72), (90, 71), (30, 69)]),
    # head size 128 (the half-wave QK kernels) and rows long enough to be cut into pieces (blocks
    # 0-7 in pieces of 3 key tiles, later ones of 6) whose partials are merged
    "long128": (dict(n_head=4, n_head_kv=2, head_dim=128, rope_dim=128), 130, [(450, 131), (600, 128), (20, 140)]),
}


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("wtype,case", [(O.F32, "short"), (O.Q4_0, "short"), (MIXED, "short"), (O.Q4_0, "long128")])
def test_packed_batch_equals_separate_examples(ctx, wtype, case, fused):
    """A packed shared-prompt batch against its examples run one by one, on the same attention path.
    The reference asserts log-probs within 1e-4 on a Q4_0 model (tests/engine.rs:296-326) and
    log-probs and gradients within 1e-5 on an F32 one (tests/gradcheck.rs:325-336).  The device
    runs a packed layout's forward attention over each example's logical sequence (the shared rows,
    then its own) with the key tiles and pieces of that example's own step, so every log-prob is
    bit-identical, on quantised weights too.  Gradients: the shared rows' key / value gradients sum
    every example's queries in one reduction (separately, one run each, added as ga / gb
    accumulate), so they agree to f32 rounding: 1e-5 of the largest."""
    kw, prompt, extras = PACKED_CASES[case]
    if wtype == MIXED:
        spec = tiny_spec(O.Q4_K, n_layer=2, n_vocab=500, tied=False,
                         tensor_types={"ffn_down": O.Q6_K, "output": O.Q6_K, "token_embd": O.Q6_K}, **kw)
    else:
        spec = tiny_spec(wtype, n_layer=2, n_vocab=500, **kw)
    g = G.GgufFile.from_bytes(spec.build())
    model, _ = model_with(ctx, g, 3, 6.0)
    model.fused_attention = fused  # the same attention kernels for the packed batch and the examples
    seqs = packed_batch(spec.n_vocab, prompt, extras, 44)
    model.zero_grad()
    sep = []
    for s, start in seqs:
        tg = answer_targets(s, start)
        lp, _ = model.forward_backward(s, tg, np.full(len(tg), 0.1, np.float32))
        sep += list(lp)
    g_sep = np.concatenate(all_grads(model))
    p = pack([s for s, _ in seqs])
    assert p.shared == prompt
    targets = []
    for k, (s, start) in enumerate(seqs):
        targets += p.map_targets(k, answer_targets(s, start))
    model.zero_grad()
    lp, _ = model.forward_backward_packed(p, targets, np.full(len(targets), 0.1, np.float32))
    g_pack = np.concatenate(all_grads(model))
    sep = np.array(sep, np.float32)
    err = np.abs(sep - lp).max()
    gerr = np.abs(g_sep - g_pack).max() / max(np.abs(g_sep).max(), 1.0)
    print(f"packed vs separate: max |d logp| {err:.2e} ({int((sep != lp).sum())} of {lp.size} differ), "
          f"max |d grad| / max |grad| {gerr:.2e}")
    np.testing.assert_array_equal(lp, sep)
    assert gerr <= 1e-5
    model.close()


@pytest.mark.parametrize("fused", [True, False])
def test_packed_step_matches_oracle(ctx, fused):
    spec = tiny_spec(O.F32, n_layer=2, n_vocab=400)
    g = G.GgufFile.from_bytes(spec.build())
    model, lora = model_with(ctx, g, 4, 8.0)
    model.fused_attention = fused
    seqs = packed_batch(spec.n_vocab, 40, [(30, 41), (55, 38), (12, 45), (70, 60)], 9)
    p = pack([s for s, _ in seqs])
    targets = []
    for k, (s, start) in enumerate(seqs):
        targets += p.map_targets(k, answer_targets(s, start))
    wts = np.linspace(0.5, 1.5, len(targets)).astype(np.float32)
    model.zero_grad()
    lp, hits = model.forward_backward_packed(p, targets, wts)
    lp_o, hits_o, grads = O.model_forward_backward(oracle_model(g, lora, 8.0), p.tokens, [t.pos for t in targets],
                                                   [t.token for t in targets], wts, nthreads=16,
                                                   positions=p.positions, segments=p.segments)
    assert np.abs(lp - lp_o).max() <= 1e-3 * np.abs(lp_o).max() and hits == hits_o
    worst = 0.0
    for i in range(model.lora_count()):
        inf = model.lora_info(i)
        _, _, ga, gb = model.lora(i)
        ga_o, gb_o = grads[inf["layer"]][NAMES[inf["which"]]]
        worst = max(worst, np.abs(ga - ga_o).max() / np.abs(ga_o).max(), np.abs(gb - gb_o).max() / np.abs(gb_o).max())
    assert worst <= 1e-3
    model.close()


def test_rope_scaling_reaches_the_device_step(ctx):
    spec = tiny_spec(O.F32, n_layer=2, arch="llama", tied=False)
    w = spec.writer()
    factors = np.linspace(1.0, 4.0, spec.rope_dim // 2 - 3).astype(np.float32)
    try:
        w.kv("llama.rope.scaling.type", G.Value.String("linear"))
        w.kv("llama.rope.scaling.factor", G.Value.F32(2.0))
        w.tensor("rope_freqs.weight", (factors.size,), G.GGML_F32, factors.view(np.uint8))
        g = G.GgufFile.from_bytes(w.to_bytes())
    finally:
        w.close()
    model, lora = model_with(ctx, g, 4, 8.0)
    assert model.config["rope_freq_scale"] == 0.5 and model.config["n_rope_factors"] == factors.size
    toks, pos, tok = sequence(spec.n_vocab, 40, 16, 5)
    wts = np.linspace(0.5, 1.5, 16).astype(np.float32)
    model.zero_grad()
    lp, _ = model.forward_backward(toks, [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)], wts)
    m = oracle_model(g, lora, 8.0)
    m["freq_scale"], m["rope_factors"] = 0.5, factors
    lp_o, _, _ = O.model_forward_backward(m, toks, pos, tok, wts, nthreads=16)
    assert np.abs(lp - lp_o).max() <= 1e-3 * np.abs(lp_o).max()
    m_plain = oracle_model(g, lora, 8.0)
    lp_plain, _, _ = O.model_forward_backward(m_plain, toks, pos, tok, wts, nthreads=16)
    assert np.abs(lp_plain - lp_o).max() > 1e-3 * np.abs(lp_o).max()  # the scaling matters here
    model.close()


def test_reattached_adapters_free_the_previous_ones(ctx):
    """rtq_model_attach_lora releases the previous adapters' memory: eight re-attaches take less
    device memory than one adapter set (a leak would take eight)"""
    import torch

    g = G.GgufFile.from_bytes(tiny_spec(O.Q4_0, n_layer=2).build())
    model = rt.GpuModel.from_gguf(g, ctx=ctx)
    n = model.attach_lora(128, 8.0, seed=1)
    one_set = 2 * 4 * n  # A, B and their gradients
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(0)[0]
    for _ in range(8):
        model.attach_lora(128, 8.0, seed=2)
    torch.cuda.synchronize()
    used = free0 - torch.cuda.mem_get_info(0)[0]
    print(f"one adapter set {one_set} B, device memory taken by eight re-attaches {used} B")
    assert used < one_set
    assert model.lora_count() == 2 * 7 and model.lora_info(0)["rank"] == 128
    model.close()
