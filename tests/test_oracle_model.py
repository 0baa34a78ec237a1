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


def f64_logp(m, tokens, pos, tok, lora_scale, positions=None, segments=None):
    """Independent float64 forward of the model (F32 weights only); positions / segments: a packed
    layout (RoPE at the given positions; token i sees j <= i with segment 0 or its own)."""
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
    f = m["theta"] ** (-2.0 * np.arange(half) / rot) * m["freq_scale"]
    fac = m.get("rope_factors")
    if fac is not None:
        f = f / np.where(np.asarray(fac, np.float64) != 0, np.asarray(fac, np.float64), 1.0)
    ps = np.arange(t) if positions is None else np.asarray(positions)
    ang = ps[:, None] * f[None, :]
    seg = np.zeros(t, np.int64) if segments is None else np.asarray(segments)
    banned = (np.arange(t)[None, :] > np.arange(t)[:, None]) | ((seg[None, :] != 0) & (seg[None, :] != seg[:, None]))
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
            s[banned] = -np.inf
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


def test_rope_table_at_positions_and_factors_matches_f64():
    rot, theta, scale = 32, 5e5, 0.25
    positions = np.array([0, 7, 3, 200, 199, 3000], np.int32)
    factors = np.array([1.0, 0.0, 2.0, 8.0, 0.5] + [1.0] * 6, np.float32)  # 11 of 16 pairs; a 0 keeps the pair
    c, s = O.rope_table(positions.size, rot, theta, scale, positions=positions, factors=factors)
    i = np.arange(rot // 2)
    f = (np.float32(theta) ** (-2.0 * i / rot)).astype(np.float64) * scale
    div = np.ones(rot // 2)
    div[: factors.size] = np.where(factors != 0, factors, 1.0)
    ang = positions[:, None].astype(np.float64) * (f / div)[None, :]
    assert np.abs(c - np.cos(ang)).max() < 2e-3 and np.abs(s - np.sin(ang)).max() < 2e-3
    # the identity layout reproduces the plain tables bit for bit
    c0, s0 = O.rope_table(50, rot, theta)
    c1, s1 = O.rope_table(50, rot, theta, positions=np.arange(50))
    assert np.array_equal(c0, c1) and np.array_equal(s0, s1)


def test_allowed_rule():
    seg = np.array([0, 0, 1, 1, 2, 2, 0], np.int32)
    for i in range(7):
        for j in range(7):
            want = j <= i and (seg[j] == 0 or seg[j] == seg[i])
            assert O.allowed(seg, i, j) == want
            assert O.allowed(None, i, j) == (j <= i)


def packed_case(V, prompt_len=13, extras=((5, 15), (9, 14), (3, 12)), seed=44):
    """The reference's packed_batch_equals_separate_examples layout (tests/gradcheck.rs:280-338):
    three examples sharing a prompt, one answer starting inside the shared part."""
    from rust_trainer_amd.packing import answer_targets, pack

    rng = O.Rng(seed)
    prompt = [int(v) for v in (O.Rng(seed).vec_uniform_sym(prompt_len, 1.0) * 0.5 + 0.5) * (V - 1)]
    seqs = []
    for k, (extra, start) in enumerate(extras):
        tail = (rng.vec_uniform_sym(extra, 1.0) * 0.5 + 0.5) * (V - 1)
        seqs.append((prompt + [int(v) for v in tail], start))
    p = pack([s for s, _ in seqs])
    targets = []
    for k, (s, start) in enumerate(seqs):
        targets += p.map_targets(k, answer_targets(s, start))
    return seqs, p, targets


def test_packed_forward_matches_f64_restatement(f32_model):
    g = f32_model
    lora = adapters(g, rank=4, alpha=8.0)
    m = oracle_model(g, lora, alpha=8.0, kv_f16=False)
    seqs, p, targets = packed_case(80)
    pos = np.array([t.pos for t in targets], np.int32)
    tok = np.array([t.token for t in targets], np.int32)
    toks = np.array(p.tokens, np.int32)
    lp, _, _ = O.model_forward_backward(m, toks, pos, tok, None, positions=p.positions, segments=p.segments)
    want = f64_logp(m, toks, pos, tok, 8.0 / 4, positions=p.positions, segments=p.segments)
    assert np.abs(lp - want).max() <= 2e-5 * np.abs(want).max()
    # without the segment rule the examples would see each other: the log-probs move
    lp_bad, _, _ = O.model_forward_backward(m, toks, pos, tok, None, positions=p.positions)
    assert np.abs(lp_bad - lp).max() > 1e-3


def test_rope_factors_forward_matches_f64_restatement(f32_model):
    g = f32_model
    m = oracle_model(g, adapters(g, rank=2, alpha=4.0), alpha=4.0, kv_f16=False)
    m["rope_factors"] = np.linspace(1.0, 8.0, m["rot"] // 2).astype(np.float32)
    m["freq_scale"] = 0.5
    tokens, pos, tok = sequence(80, 20, 8)
    lp, _, _ = O.model_forward_backward(m, tokens, pos, tok, None)
    want = f64_logp(m, tokens, pos, tok, 4.0 / 2)
    assert np.abs(lp - want).max() <= 2e-5 * np.abs(want).max()


@pytest.mark.parametrize("wtype", [G.GGML_F32, G.GGML_Q8_0])
def test_packed_batch_equals_separate_examples(wtype):
    """tests/gradcheck.rs:280-338 on the oracle: a packed batch gives the log-probs and LoRA
    gradients of running each example separately (1e-5, gradients relative to their max)."""
    from rust_trainer_amd.packing import answer_targets

    s = tiny_spec(wtype, n_layer=2, n_embd=64, n_head=4, n_head_kv=2, head_dim=16, rope_dim=16, n_ff=96, n_vocab=50)
    g = G.GgufFile.from_bytes(s.build())
    lora = adapters(g, rank=3, alpha=6.0, b_std=0.05)
    seqs, p, targets = packed_case(50)
    assert p.shared == 13

    def flat(grads):
        return np.concatenate([np.concatenate([ga.ravel(), gb.ravel()]) for gl in grads for ga, gb in gl.values()])

    sep_lp, sep_g = [], None
    for sq, start in seqs:
        tg = answer_targets(sq, start)
        w = np.full(len(tg), 0.1, np.float32)
        lp, _, gr = O.model_forward_backward(oracle_model(g, lora, 6.0), np.array(sq, np.int32),
                                             [t.pos for t in tg], [t.token for t in tg], w)
        sep_lp += list(lp)
        sep_g = flat(gr) if sep_g is None else sep_g + flat(gr)
    w = np.full(len(targets), 0.1, np.float32)
    lp, _, gr = O.model_forward_backward(oracle_model(g, lora, 6.0), np.array(p.tokens, np.int32),
                                         [t.pos for t in targets], [t.token for t in targets], w,
                                         positions=p.positions, segments=p.segments)
    assert np.abs(np.array(sep_lp) - lp).max() < 1e-5
    scale = max(np.abs(sep_g).max(), 1.0)
    assert np.abs(sep_g - flat(gr)).max() <= 1e-5 * scale
