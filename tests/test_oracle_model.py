"""The oracle's model-level training step (or_model_forward_backward) pinned on the CPU:

* round_f16 against IEEE half conversion (and the reference's own edge at 65520);
* RoPE tables against f64 trigonometry;
* the forward log-probs against an independent float64 numpy restatement of the model
  (src/model.rs, src/attention.rs, src/ops.rs) on an F32 synthetic model;
* every LoRA gradient kind against central finite differences of L = -sum w_i logp_i
  (F32 model without f16 K/V rounding, so L is smooth in the adapters).
"""
import numpy as np
import pytest

import oracle as O
from model_cases import GGUF_NAMES, adapters, oracle_model, sequence, tiny_spec
from rust_trainer_amd import gguf as G


def test_round_f16_matches_ieee_half():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(3000) * 10.0 ** rng.integers(-9, 5, 3000), [0.0, -0.0, 6.1e-5, 5.96e-8,
                                                                                        2.98e-8, 65504.0, -65519.0]])
    x = x.astype(np.float32)
    got = np.array([O.round_f16(float(v)) for v in x], np.float32)
    want = x.astype(np.float16).astype(np.float32)
    np.testing.assert_array_equal(got, want)
    # the reference's rounding grid at the top of the range rounds 65520 up to 65536 (not inf)
    assert O.round_f16(65520.0) == 65536.0 and O.round_f16(70000.0) == np.inf and O.round_f16(-1e6) == -np.inf


def test_rope_table_matches_f64():
    t, rot, theta = 300, 64, 1e6
    c, s = O.rope_table(t, rot, theta)
    i = np.arange(rot // 2)
    f = (np.float32(theta) ** (-2.0 * i / rot)).astype(np.float64)
    ang = np.arange(t)[:, None] * f[None, :]
    assert np.abs(c - np.cos(ang)).max() < 1e-4 and np.abs(s - np.sin(ang)).max() < 1e-4
    assert c[0].tolist() == [1.0] * (rot // 2) and not s[0].any()


def f64_logp(m, tokens, pos, tok, lora_scale):
    """Independent float64 forward of the model (F32 weights only)."""
    d, nh, nkv, hd, rot = m["d"], m["n_head"], m["n_kv"], m["hd"], m["rot"]

    def W(lin):
        w = np.frombuffer(np.ascontiguousarray(lin["blocks"]).tobytes(), np.float32).reshape(lin["out"], lin["in"])
        return w.astype(np.float64)

    def linear(lin, x):
        y = x @ W(lin).T
        if lin.get("A") is not None:
            y = y + lora_scale * (x @ lin["A"].astype(np.float64).T) @ lin["B"].astype(np.float64).T
        return y

    def rms(x, w, fused):
        ir = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + m["eps"])
        return x * ir * w

    t = tokens.size
    half = rot // 2
    f = m["theta"] ** (-2.0 * np.arange(half) / rot)
    ang = np.arange(t)[:, None] * f[None, :]
    cos, sin = np.cos(ang), np.sin(ang)

    def rope(x):  # x [t, heads, hd], NEOX pairs (i, i + half)
        x = x.copy()
        a, b = x[..., :half].copy(), x[..., half:rot].copy()
        x[..., :half] = a * cos[:, None, :] - b * sin[:, None, :]
        x[..., half:rot] = b * cos[:, None, :] + a * sin[:, None, :]
        return x

    emb = np.frombuffer(np.ascontiguousarray(m["embed"][1]).tobytes(), np.float32).reshape(m["embed"][2], d)
    x = emb[tokens].astype(np.float64)
    for L in m["layers"]:
        n1 = rms(x, L["attn_norm"], False)
        q = linear(L["q"], n1).reshape(t, nh, hd)
        k = linear(L["k"], n1).reshape(t, nkv, hd)
        v = linear(L["v"], n1).reshape(t, nkv, hd)
        q, k = rope(rms(q, L["q_norm"], True)), rope(rms(k, L["k_norm"], True))
        o = np.zeros((t, nh, hd))
        for h in range(nh):
            g = h // (nh // nkv)
            s = (q[:, h] / np.sqrt(hd)) @ k[:, g].T
            s[np.triu_indices(t, 1)] = -np.inf
            p = np.exp(s - s.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            o[:, h] = p @ v[:, g]
        hres = x + linear(L["o"], o.reshape(t, nh * hd))
        n2 = rms(hres, L["ffn_norm"], False)
        gg, uu = linear(L["gate"], n2), linear(L["up"], n2)
        x = hres + linear(L["down"], gg / (1.0 + np.exp(-gg)) * uu)
    ns = rms(x[pos], m["out_norm"], False)
    logits = ns @ emb.astype(np.float64).T
    mx = logits.max(1, keepdims=True)
    lse = (mx + np.log(np.exp(logits - mx).sum(1, keepdims=True)))[:, 0]
    return logits[np.arange(pos.size), tok] - lse


@pytest.fixture(scope="module")
def f32_model():
    s = tiny_spec(G.GGML_F32, n_layer=2, n_embd=64, n_head=4, n_head_kv=2, head_dim=16, rope_dim=16, n_ff=96,
                  n_vocab=80)
    g = G.GgufFile.from_bytes(s.build())
    return g


def test_model_forward_matches_f64_restatement(f32_model):
    g = f32_model
    lora = adapters(g, rank=4, alpha=8.0)
    m = oracle_model(g, lora, alpha=8.0, kv_f16=False)
    m["layers"][1]["q_norm"] = (1.0 + 0.1 * O.Rng(3).vec_normal(16, 1.0)).astype(np.float32)  # non-trivial norm
    tokens, pos, tok = sequence(80, 24, 10)
    logp, hits, _ = O.model_forward_backward(m, tokens, pos, tok, None)
    want = f64_logp(m, tokens, pos, tok, 8.0 / 4)
    assert np.abs(logp - want).max() <= 2e-5 * np.abs(want).max()
    # kv_f16 only rounds K and V: a small, non-zero change
    m["kv_f16"] = True
    lp16, _, _ = O.model_forward_backward(m, tokens, pos, tok, None)
    assert 0 < np.abs(lp16 - logp).max() < 1e-2 * np.abs(logp).max()


def test_model_lora_grads_finite_differences(f32_model):
    g = f32_model
    lora = adapters(g, rank=2, alpha=4.0, b_std=0.05)
    tokens, pos, tok = sequence(80, 12, 6)
    wts = np.linspace(0.5, 1.5, pos.size).astype(np.float32)

    def loss():
        lp, _, _ = O.model_forward_backward(oracle_model(g, lora, alpha=4.0, kv_f16=False), tokens, pos, tok, None)
        return -float((wts.astype(np.float64) * lp).sum())

    _, _, grads = O.model_forward_backward(oracle_model(g, lora, alpha=4.0, kv_f16=False), tokens, pos, tok, wts)
    rng = np.random.default_rng(1)
    h = 1e-2
    for (li, name) in [(0, "q"), (0, "k"), (1, "v"), (0, "o"), (1, "gate"), (0, "up"), (1, "down")]:
        A, B = lora[(li, name)]
        ga, gb = grads[li][name]
        for which, P, G_ in (("A", A, ga), ("B", B, gb)):
            for _ in range(2):
                idx = tuple(int(rng.integers(0, s)) for s in P.shape)
                old = P[idx]
                P[idx] = old + h
                lp_ = loss()
                P[idx] = old - h
                lm_ = loss()
                P[idx] = old
                fd = (lp_ - lm_) / (2 * h)
                assert abs(fd - G_[idx]) <= 5e-3 * max(abs(fd), 0.05), (li, name, which, idx, fd, G_[idx])


def test_model_rejects_bad_tokens(f32_model):
    m = oracle_model(f32_model, None)
    with pytest.raises(Exception):
        O.model_forward_backward(m, np.array([0, 80], np.int32), [0], [1], None)


def test_gguf_names_cover_every_linear():
    assert sorted(GGUF_NAMES) == sorted(O.LINEARS)
