"""GPU parity of the device-resident training step (rtq_model_*) against the oracle's restatement
of Model::forward_backward (src/model.rs:644-687) on synthetic GGUF models.

Errors are max |gpu - oracle| / max |oracle| per tensor (log-probs, each adapter's ga and gb).

* F32 weights (no activation quantisation): <= 1e-3, as for a single linear.
* Quantised weights: a whole-model step is not a continuous function of its inputs.  Every linear
  re-quantises its input to Q8 codes and K / V are rounded to f16, so a one-ulp difference in any
  f32 sum can move a code across a rounding boundary, and that step propagates.  The oracle shows
  the same: the oracle against itself, with every norm weight moved by one ulp, differs by up to
  ~2e-3 in log-probs and ~4e-2 in gradients.  That noise floor is measured in the test (four
  perturbations), and the GPU must stay within max(1e-3, 2 x floor).
* Always: greedy hits equal, the adapters' initial A equal to the reference Rng's draw.
"""
import numpy as np
import pytest

import oracle as O
import rust_trainer_amd as rt
from model_cases import adapters, oracle_model, sequence, tiny_spec
from rust_trainer_amd import gguf as G

pytestmark = pytest.mark.gpu

TOL = 1e-3
NAMES = O.LINEARS  # adapter order within a block: q, k, v, o, gate, up, down


def rel_err(got, want):
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    assert got.shape == want.shape
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def run_both(ctx, spec, rank=4, alpha=8.0, t=40, n=16, seed=5, weights=True, fused=None):
    g = G.GgufFile.from_bytes(spec.build())
    model = rt.GpuModel.from_gguf(g, ctx=ctx)
    model.fused_attention = fused
    model.attach_lora(rank, alpha, seed=1)
    lora = adapters(g, rank, alpha)
    for i in range(model.lora_count()):
        inf = model.lora_info(i)
        A, B = lora[(inf["layer"], NAMES[inf["which"]])]
        model.set_lora(i, A, B)
    toks, pos, tok = sequence(spec.n_vocab, t, n, seed)
    wts = np.linspace(0.5, 1.5, n).astype(np.float32) if weights else None
    targets = [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)]
    model.zero_grad()
    logp, hits = model.forward_backward(toks, targets, wts)
    lp_o, hits_o, grads = O.model_forward_backward(oracle_model(g, lora, alpha, kv_f16=True), toks, pos, tok, wts,
                                                   nthreads=16)
    return model, logp, hits, lp_o, hits_o, grads


def grad_err(model, grads):
    worst = 0.0
    for i in range(model.lora_count()):
        inf = model.lora_info(i)
        _, _, ga, gb = model.lora(i)
        ga_o, gb_o = grads[inf["layer"]][NAMES[inf["which"]]]
        worst = max(worst, rel_err(ga, ga_o), rel_err(gb, gb_o))
    return worst


def noise_floor(g, lora, alpha, toks, pos, tok, wts, seeds=4):
    """(log-prob, gradient) error of the oracle against itself with every norm weight moved by
    one ulp up or down at random"""
    base = O.model_forward_backward(oracle_model(g, lora, alpha), toks, pos, tok, wts, nthreads=16)
    fl, fg = 0.0, 0.0
    for seed in range(seeds):
        m = oracle_model(g, lora, alpha)
        rng = np.random.default_rng(seed)

        def nudge(w):
            w = w.copy()
            r = rng.random(w.size)
            w[r < 1 / 3] = np.nextafter(w[r < 1 / 3], np.float32(np.inf))
            w[r > 2 / 3] = np.nextafter(w[r > 2 / 3], np.float32(-np.inf))
            return w

        for L in m["layers"]:
            for k in ("attn_norm", "ffn_norm", "q_norm", "k_norm"):
                if L.get(k) is not None:
                    L[k] = nudge(L[k])
        m["out_norm"] = nudge(m["out_norm"])
        lp, _, gr = O.model_forward_backward(m, toks, pos, tok, wts, nthreads=16)
        fl = max(fl, rel_err(lp, base[0]))
        fg = max(fg, max(rel_err(gr[li][n][k], base[2][li][n][k]) for li in range(len(gr)) for n in NAMES
                         if gr[li][n] is not None for k in range(2)))
    return fl, fg


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("t", [40, 37, 150])
def test_model_step_f32_weights_matches_oracle(ctx, t, fused):
    """F32 weights: no activation quantisation, so the step is smooth and the 1e-3 bar holds
    (t = 37: attention rows of odd length, so the attention products take single-float loads;
    t = 150: several key tiles), with either attention path"""
    model, logp, hits, lp_o, hits_o, grads = run_both(ctx, tiny_spec(O.F32, n_layer=2), t=t, fused=fused)
    assert model.fused_attention is fused
    assert rel_err(logp, lp_o) <= TOL and hits == hits_o
    assert grad_err(model, grads) <= TOL
    model.close()


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0, O.Q4_K, O.Q6_K])
def test_model_step_matches_oracle(ctx, wtype):
    spec = tiny_spec(wtype, n_layer=2)
    model, logp, hits, lp_o, hits_o, grads = run_both(ctx, spec)
    g = G.GgufFile.from_bytes(spec.build())
    toks, pos, tok = sequence(spec.n_vocab, 40, 16, 5)
    fl, fg = noise_floor(g, adapters(g, 4, 8.0), 8.0, toks, pos, tok, np.linspace(0.5, 1.5, 16).astype(np.float32))
    el, eg = rel_err(logp, lp_o), grad_err(model, grads)
    print(f"log-probs {el:.2e} (oracle floor {fl:.2e}), gradients {eg:.2e} (floor {fg:.2e})")
    assert el <= max(TOL, 2 * fl) and eg <= max(TOL, 2 * fg)
    assert hits == hits_o
    model.close()


@pytest.mark.parametrize("targets", [("q_proj", "v_proj", "up_proj"), ("k_proj", "gate_proj", "down_proj")])
def test_model_step_adapter_subset_matches_oracle(ctx, targets):
    """adapters on some members of the fused q|k|v and gate|up groups only (quantised weights, so
    the block-diagonal backward runs with unadapted members in between)"""
    spec = tiny_spec(O.Q8_0, n_layer=2)
    g = G.GgufFile.from_bytes(spec.build())
    model = rt.GpuModel.from_gguf(g, ctx=ctx)
    model.attach_lora(4, 8.0, targets=targets, seed=1)
    full = adapters(g, 4, 8.0)
    names = {t.replace("_proj", "") for t in targets}
    lora = {key: v for key, v in full.items() if key[1] in names}
    for i in range(model.lora_count()):
        inf = model.lora_info(i)
        model.set_lora(i, *lora[(inf["layer"], NAMES[inf["which"]])])
    toks, pos, tok = sequence(spec.n_vocab, 40, 16, 5)
    wts = np.linspace(0.5, 1.5, 16).astype(np.float32)
    model.zero_grad()
    logp, hits = model.forward_backward(toks, [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)], wts)
    lp_o, hits_o, grads = O.model_forward_backward(oracle_model(g, lora, 8.0), toks, pos, tok, wts, nthreads=16)
    fl, fg = noise_floor(g, lora, 8.0, toks, pos, tok, wts)
    el, eg = rel_err(logp, lp_o), grad_err(model, grads)
    print(f"log-probs {el:.2e} (oracle floor {fl:.2e}), gradients {eg:.2e} (floor {fg:.2e})")
    assert el <= max(TOL, 2 * fl) and eg <= max(TOL, 2 * fg)
    assert hits == hits_o and model.lora_count() == 2 * len(targets)
    model.close()


def test_model_step_config3_layer_shape(ctx):
    """two blocks of the configs[2] shape (hidden 1024, 16 / 8 heads of 128, FFN 3072, NEOX RoPE,
    QK-norm), 512 tokens, loss on the last 256, rank 16; vocabulary cut to 8192 (the full head is
    covered by the LM head tests)"""
    spec = tiny_spec(O.Q4_0, n_layer=2, n_embd=1024, n_head=16, n_head_kv=8, head_dim=128, rope_dim=128, n_ff=3072,
                     n_vocab=8192)
    model, logp, hits, lp_o, hits_o, grads = run_both(ctx, spec, rank=16, alpha=32.0, t=512, n=256)
    g = G.GgufFile.from_bytes(spec.build())
    toks, pos, tok = sequence(spec.n_vocab, 512, 256, 5)
    fl, fg = noise_floor(g, adapters(g, 16, 32.0), 32.0, toks, pos, tok,
                         np.linspace(0.5, 1.5, 256).astype(np.float32), seeds=2)
    el, eg = rel_err(logp, lp_o), grad_err(model, grads)
    print(f"log-probs {el:.2e} (oracle floor {fl:.2e}), gradients {eg:.2e} (floor {fg:.2e})")
    assert el <= max(TOL, 2 * fl) and eg <= max(TOL, 2 * fg)
    model.close()


@pytest.mark.parametrize("fused", [True, False])
def test_model_step_f32_hd128_long_rows_matches_oracle(ctx, fused, monkeypatch):
    """head size = RoPE size = 128 (the half-wave QK-norm + RoPE kernels, whose backward also sums
    the cut blocks' partial slots on every layer but a captured one) at 600 tokens (fused: rows of
    up to ten key tiles cut into pieces and merged), F32 weights against the oracle at 1e-3; then
    the same step with nothing cut (RTQ_ATTN_ITEMS=0) against the default: log-probs within 1e-5
    (f32 rounding of the forward merges), gradients within 5e-5 (the attention backward's products
    carry 16 significant bits, about 2^-16 each, and cut rows sum them in another order; measured
    1.5e-5)"""
    spec = tiny_spec(O.F32, n_layer=2, head_dim=128, rope_dim=128)
    model, logp, hits, lp_o, hits_o, grads = run_both(ctx, spec, t=600, n=200, fused=fused)
    assert rel_err(logp, lp_o) <= TOL and hits == hits_o
    assert grad_err(model, grads) <= TOL
    monkeypatch.setenv("RTQ_ATTN_ITEMS", "0")
    whole, lp_w, hits_w, _, _, _ = run_both(ctx, spec, t=600, n=200, fused=fused)
    monkeypatch.delenv("RTQ_ATTN_ITEMS")
    assert rel_err(lp_w, logp) <= 1e-5 and hits_w == hits
    for i in range(model.lora_count()):
        for a, b in zip(whole.lora(i)[2:], model.lora(i)[2:]):
            assert rel_err(a, b) <= 5e-5
    whole.close()
    model.close()


def test_model_step_llama_untied_and_score(ctx):
    """normal (adjacent-pair) RoPE, no QK-norm, untied output head (F32 weights: the 1e-3 bar);
    score() = log-probs only"""
    spec = tiny_spec(O.F32, n_layer=2, arch="llama", tied=False)
    model, logp, hits, lp_o, hits_o, grads = run_both(ctx, spec)
    assert model.config["rope_neox"] == 0 and model.config["qk_norm"] == 0 and model.config["tied"] == 0
    assert rel_err(logp, lp_o) <= TOL and hits == hits_o
    assert grad_err(model, grads) <= TOL
    toks, pos, tok = sequence(spec.n_vocab, 40, 16, 5)
    lp2, h2 = model.score(toks, [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)])
    np.testing.assert_array_equal(lp2, logp)
    assert h2 == hits
    model.close()


def test_attach_lora_draws_the_reference_init(ctx):
    g = G.GgufFile.from_bytes(tiny_spec(O.F32, n_layer=2).build())
    model = rt.GpuModel.from_gguf(g, ctx=ctx)
    n = model.attach_lora(8, 16.0, targets=("q_proj", "v_proj", "down_proj"), seed=7)
    assert model.lora_count() == 2 * 3
    rng = O.Rng(7)
    total = 0
    for i in range(model.lora_count()):
        inf = model.lora_info(i)
        a, b, ga, gb = model.lora(i)
        want = rng.vec_uniform_sym(8 * inf["in_dim"], 1.0 / np.sqrt(inf["in_dim"])).reshape(8, -1)
        np.testing.assert_array_equal(a, want)
        assert not b.any() and not ga.any() and not gb.any()
        total += a.size + b.size
    assert n == total and [model.lora_info(i)["name"] for i in range(2)] == ["blk.0.attn_q", "blk.0.attn_v"]
    # a fresh adapter is a no-op: the same log-probs as with adapters disabled on the oracle
    toks, pos, tok = sequence(512, 24, 8, 3)
    lp, _ = model.score(toks, [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)])
    lp_o, _, _ = O.model_forward_backward(oracle_model(g, None), toks, pos, tok, None, nthreads=16)
    assert rel_err(lp, lp_o) <= TOL
    model.close()


def test_model_rejects_bad_inputs(ctx):
    g = G.GgufFile.from_bytes(tiny_spec(O.Q4_0, n_layer=1).build())
    model = rt.GpuModel.from_gguf(g, ctx=ctx)
    with pytest.raises(rt.RtqError):
        model.forward_backward([0, 512], [rt.Target(0, 1)], [1.0])
    with pytest.raises(rt.RtqError):
        model.forward_backward([0, 1], [rt.Target(2, 1)], [1.0])
    model.close()
