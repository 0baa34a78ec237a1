"""Op-by-op parity of the device training step (rtq_model_*) against the oracle, teacher-forced.

A whole quantised step is not a continuous function of its inputs (every linear re-quantises its
input to Q8 codes, K / V are rounded to f16), so comparing only its end results cannot tell a bug
from a code that flipped.  Here one block's tensors are captured during a device step
(rtq_model_debug_capture) and every operation of the block (src/model.rs:165-197,
src/attention.rs:162-367, src/model.rs:113-134) is recomputed by the oracle from the device's own
inputs to that operation:

* the Q8 activation codes of every linear's input are bit-exact (the device's quantisation of its
  own n1, o, n2 and hm against the oracle's quantiser);
* every linear output, norm, QK-norm + RoPE, attention output and probabilities, SwiGLU, every
  input gradient and every adapter's dA and dB agree within max |device - oracle| / max |oracle|
  <= 1e-3 (no noise-floor scaling).

Cases: the configs[2] block shape (hidden 1024, 16 / 8 heads of 128, FFN 3072, NEOX RoPE, QK-norm,
512 tokens, rank 16) in all four formats; an odd shape (5 heads of 36 over 1 KV head: fused q|k|v
of 252 rows and gate|up of 320, neither a multiple of 64) at t = 16 and 700 with k_proj and
up_proj unadapted (the block-diagonal fused adapter with an unadapted member); a packed
shared-prompt batch at the configs[2] shape with activations recomputed; the configs[3] block
shape (Qwen3-4B: hidden 2560, 32 / 8 heads, FFN 9728, Q4_K attention / gate / up, Q6_K down) on a
packed batch of eight examples sharing a 200-token prompt (680 tokens, and the configuration's 6792); the configs[4] block shape
(Llama-3-8B: hidden 4096, 32 / 8 heads, FFN 14336, adjacent-pair RoPE 5e5, Q8_0, rank 64,
untied head) at 2048 tokens with loss on the last 1024, recomputed.
"""
import numpy as np
import pytest

import oracle as O
import rust_trainer_amd as rt
from model_cases import adapters, oracle_model, sequence, tiny_spec
from rust_trainer_amd import gguf as G
from rust_trainer_amd.packing import answer_targets, pack

pytestmark = pytest.mark.gpu

TOL = 1e-3
LIN = O.LINEARS  # q, k, v, o, gate, up, down


def rel(got, want, mask=None):
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    assert got.shape == want.shape
    if mask is not None:
        got, want = got[mask.reshape(-1)], want[mask.reshape(-1)]
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def lin_fwd(L, name, x, t):
    d = L[name]
    return O.linear_forward(d["wtype"], d["blocks"], d["out"], d["in"], x, A=d.get("A"), B=d.get("B"),
                            alpha=d.get("alpha", 0.0), nthreads=16).reshape(t, d["out"])


def lin_bwd(L, name, x, dy, t):
    d = L[name]
    dx, ga, gb = O.linear_backward(d["wtype"], d["blocks"], d["out"], d["in"], x, dy, A=d.get("A"), B=d.get("B"),
                                   alpha=d.get("alpha", 0.0), nthreads=16)
    return dx.reshape(t, d["in"]), ga, gb


def codes_exact(ctx, wtype, x, t):
    """the device's Q8 activation blocks of x equal the oracle's (x: the device's own tensor)"""
    k = x.shape[1]
    if wtype == O.F32:
        return
    w = O.quantize(wtype, O.Rng(9).vec_normal(64 * k, 0.02).reshape(64, k))
    hf = rt.HipFrozen(wtype, w, 64, k, ctx=ctx)
    assert np.array_equal(hf.debug_quantize_acts(x, t), O.quantize_acts(wtype, x)), "activation codes differ"


def check_block(ctx, g, model, m, layer, t, seg, lora_map, report):
    """compare every op of captured block `layer` with the oracle on the device's inputs"""
    c = model.config
    d, nh, nkv, hd, ff = c["n_embd"], c["n_head"], c["n_head_kv"], c["head_dim"], c["n_ff"]
    qd, kd = nh * hd, nkv * hd
    shapes = dict(x=(t, d), n1=(t, d), inv1=(t,), q_raw=(t, qd), k_raw=(t, kd), v_raw=(t, kd), q=(t, qd), k=(t, kd),
                  v=(t, kd), q_inv=(t * nh,), k_inv=(t * nkv,), o=(t, qd), h=(t, d), n2=(t, d),
                  inv2=(t,), gate=(t, ff), up=(t, ff), hm=(t, ff), y=(t, d), dy=(t, d), dhm=(t, ff), dgate=(t, ff),
                  dup=(t, ff), dn2=(t, d), dh=(t, d), d_o=(t, qd), dq=(t, qd), dk=(t, kd), dv=(t, kd),
                  dq_raw=(t, qd), dk_raw=(t, kd), dn1=(t, d), dx=(t, d))
    T = {n: model.debug_tensor(n, s) for n, s in shapes.items()}
    fused = model.fused_attention  # fused attention: each row's log-sum-exp is kept instead of P
    if fused:
        T["lse"] = model.debug_tensor("lse", (nh, t))
    else:
        T["P"] = model.debug_tensor("P", (nh, t, t))
    L = m["layers"][layer]
    ops = O.BlockOps(m)
    errs = {}
    wt = {n: L[n]["wtype"] for n in LIN}
    # forward (src/model.rs:166-180, src/attention.rs:162-240, src/model.rs:114-119)
    n1, inv1 = ops.rmsnorm(T["x"], L["attn_norm"])
    errs["n1"], errs["inv1"] = rel(T["n1"], n1), rel(T["inv1"], inv1)
    codes_exact(ctx, wt["q"], T["n1"], t)
    for n in ("q", "k", "v"):
        errs[n + "_raw"] = rel(T[n + "_raw"], lin_fwd(L, n, T["n1"], t))
    pos = np.arange(t) if report.get("positions") is None else np.asarray(report["positions"])
    cos_, sin_ = O.rope_table(t, m["rot"], m["theta"], m["freq_scale"], positions=pos)
    q, k, v, qi, ki = ops.qk_prep(L["q_norm"], L["k_norm"], cos_, sin_, T["q_raw"], T["k_raw"], T["v_raw"])
    errs["q"], errs["k"], errs["v"] = rel(T["q"], q), rel(T["k"], k), rel(T["v"], v)
    if L["q_norm"] is not None:
        errs["q_inv"], errs["k_inv"] = rel(T["q_inv"], qi), rel(T["k_inv"], ki)
    P, o = ops.attention(T["q"], T["k"], T["v"], seg)
    allowed = np.tril(np.ones((t, t), bool))
    if seg is not None:
        s = np.asarray(seg)
        allowed &= (s[None, :] == 0) | (s[None, :] == s[:, None])
    if fused:
        # the device's probabilities p = exp((q scale) . k - lse) from its own q, k and lse (f64)
        qs = (T["q"].reshape(t, nh, hd) * np.float32(1.0 / np.sqrt(hd))).astype(np.float64)
        kk = T["k"].reshape(t, nkv, hd).astype(np.float64)
        P_dev = np.zeros((nh, t, t), np.float32)
        for hh in range(nh):
            sc_ = qs[:, hh, :] @ kk[:, hh // (nh // nkv), :].T
            P_dev[hh] = np.where(allowed, np.exp(sc_ - T["lse"][hh][:, None]), 0.0)
    else:
        P_dev = np.where(np.broadcast_to(allowed, T["P"].shape), T["P"], 0.0).astype(np.float32)
    errs["P"] = rel(P_dev, P, np.broadcast_to(allowed, P.shape))
    errs["o"] = rel(T["o"], o)
    codes_exact(ctx, wt["o"], T["o"], t)
    errs["h"] = rel(T["h"], T["x"] + lin_fwd(L, "o", T["o"], t))
    n2, inv2 = ops.rmsnorm(T["h"], L["ffn_norm"])
    errs["n2"], errs["inv2"] = rel(T["n2"], n2), rel(T["inv2"], inv2)
    codes_exact(ctx, wt["gate"], T["n2"], t)
    errs["gate"], errs["up"] = rel(T["gate"], lin_fwd(L, "gate", T["n2"], t)), rel(T["up"], lin_fwd(L, "up", T["n2"], t))
    errs["hm"] = rel(T["hm"], ops.swiglu(T["gate"], T["up"]))
    codes_exact(ctx, wt["down"], T["hm"], t)
    errs["y"] = rel(T["y"], T["h"] + lin_fwd(L, "down", T["hm"], t))
    # backward (src/model.rs:183-194, src/attention.rs:243-355)
    grads = {}
    dhm, *grads["down"] = lin_bwd(L, "down", T["hm"], T["dy"], t)
    errs["dhm"] = rel(T["dhm"], dhm)
    dg, du = ops.swiglu_backward(T["gate"], T["up"], T["dhm"])
    errs["dgate"], errs["dup"] = rel(T["dgate"], dg), rel(T["dup"], du)
    dxg, *grads["gate"] = lin_bwd(L, "gate", T["n2"], T["dgate"], t)
    dxu, *grads["up"] = lin_bwd(L, "up", T["n2"], T["dup"], t)
    errs["dn2"] = rel(T["dn2"], dxg + dxu)
    errs["dh"] = rel(T["dh"], T["dy"] + ops.rmsnorm_backward(T["h"], L["ffn_norm"], T["inv2"], T["dn2"]))
    d_o, *grads["o"] = lin_bwd(L, "o", T["o"], T["dh"], t)
    errs["d_o"] = rel(T["d_o"], d_o)
    # (the unfused device path leaves blocks of a packed layout where no pair may attend unwritten:
    # only the allowed entries are its probabilities)
    dq, dk, dv = ops.attention_backward(T["q"], T["k"], T["v"], P_dev, T["d_o"], seg)
    errs["dq"], errs["dk"], errs["dv"] = rel(T["dq"], dq), rel(T["dk"], dk), rel(T["dv"], dv)
    dq_raw, dk_raw = ops.qk_backward(L["q_norm"], L["k_norm"], cos_, sin_, T["q_raw"], T["k_raw"], T["q_inv"],
                                     T["k_inv"], T["dq"], T["dk"])
    errs["dq_raw"], errs["dk_raw"] = rel(T["dq_raw"], dq_raw), rel(T["dk_raw"], dk_raw)
    dxq, *grads["q"] = lin_bwd(L, "q", T["n1"], T["dq_raw"], t)
    dxk, *grads["k"] = lin_bwd(L, "k", T["n1"], T["dk_raw"], t)
    dxv, *grads["v"] = lin_bwd(L, "v", T["n1"], T["dv"], t)
    errs["dn1"] = rel(T["dn1"], dxq + (dxk + dxv))
    errs["dx"] = rel(T["dx"], T["dh"] + ops.rmsnorm_backward(T["x"], L["attn_norm"], T["inv1"], T["dn1"]))
    # every adapter of the block: dA, dB from the device's own inputs of that linear
    for i in range(model.lora_count()):
        inf = model.lora_info(i)
        if inf["layer"] != layer:
            continue
        name = LIN[inf["which"]]
        _, _, ga, gb = model.lora(i)
        errs["dA_" + name] = rel(ga, grads[name][0])
        errs["dB_" + name] = rel(gb, grads[name][1])
    worst = max(errs, key=errs.get)
    print(" ".join(f"{k} {v:.1e}" for k, v in errs.items()))
    print(f"worst: {worst} {errs[worst]:.2e}")
    bad = {k: v for k, v in errs.items() if not v <= TOL}
    assert not bad, f"ops above {TOL}: {bad}"


def build(ctx, spec, rank, alpha, targets):
    g = G.GgufFile.from_bytes(spec.build())
    model = rt.GpuModel.from_gguf(g, ctx=ctx)
    model.attach_lora(rank, alpha, targets=targets, seed=1)
    full = adapters(g, rank, alpha, b_std=0.02)
    names = {x.replace("_proj", "") for x in targets}
    lora = {key: v for key, v in full.items() if key[1] in names}
    for i in range(model.lora_count()):
        inf = model.lora_info(i)
        model.set_lora(i, *lora[(inf["layer"], LIN[inf["which"]])])
    return g, model, oracle_model(g, lora, alpha)


CONFIG2_BLOCK = dict(n_layer=2, n_embd=1024, n_head=16, n_head_kv=8, head_dim=128, rope_dim=128, n_ff=3072,
                     n_vocab=8192)
ALL = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


@pytest.mark.parametrize("fused", [None, False])  # None: the default (fused kernels); False: probability matrix
@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0, O.Q4_K, O.Q6_K])
def test_config2_block_ops_match_oracle(ctx, wtype, fused):
    spec = tiny_spec(wtype, **CONFIG2_BLOCK)
    g, model, m = build(ctx, spec, 16, 32.0, ALL)
    model.fused_attention = fused
    t, n = 512, 256
    toks, pos, tok = sequence(spec.n_vocab, t, n, 5)
    wts = np.linspace(0.5, 1.5, n).astype(np.float32)
    for layer in (1, 0):
        model.debug_capture(layer)
        model.zero_grad()
        model.forward_backward(toks, [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)], wts)
        print(f"layer {layer} (recompute: {model.checkpointing})")
        check_block(ctx, g, model, m, layer, t, None, {}, {})
    model.close()


def test_config2_block_ops_fused_attention_match_oracle(ctx):
    """the configs[2] block with the fused attention kernels forced, equal target weights"""
    spec = tiny_spec(O.Q4_K, **CONFIG2_BLOCK)
    g, model, m = build(ctx, spec, 16, 32.0, ALL)
    model.fused_attention = True
    t, n = 512, 256
    toks, pos, tok = sequence(spec.n_vocab, t, n, 9)
    model.debug_capture(1)
    model.zero_grad()
    model.forward_backward(toks, [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)], np.full(n, 1.0 / n, np.float32))
    assert model.fused_attention is True
    check_block(ctx, g, model, m, 1, t, None, {}, {})
    model.close()


@pytest.mark.parametrize("t", [45, 333])
def test_fused_attention_head_dim_64_match_oracle(ctx, t):
    """the fused attention kernels at head_dim 64 (the other width they are built for), four query
    heads per KV head, ragged lengths (a partial last 64-row block)"""
    spec = tiny_spec(O.Q8_0, n_layer=1, n_embd=512, n_head=8, n_head_kv=2, head_dim=64, rope_dim=64, n_ff=768,
                     n_vocab=500)
    g, model, m = build(ctx, spec, 8, 16.0, ALL)
    model.fused_attention = True
    n = min(t - 1, 120)
    toks, pos, tok = sequence(spec.n_vocab, t, n, 5)
    model.debug_capture(0)
    model.zero_grad()
    model.forward_backward(toks, [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)],
                           np.linspace(0.5, 1.5, n).astype(np.float32))
    assert model.fused_attention is True
    check_block(ctx, g, model, m, 0, t, None, {}, {})
    model.close()


@pytest.mark.parametrize("t", [16, 700])
@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
def test_odd_fused_groups_block_ops_match_oracle(ctx, wtype, t):
    spec = tiny_spec(wtype, n_layer=1, n_embd=128, n_head=5, n_head_kv=1, head_dim=36, rope_dim=36, n_ff=160,
                     n_vocab=300)
    g, model, m = build(ctx, spec, 4, 8.0, ("q_proj", "v_proj", "o_proj", "gate_proj", "down_proj"))
    n = min(t - 1, 100)
    toks, pos, tok = sequence(spec.n_vocab, t, n, 7)
    model.debug_capture(0)
    model.zero_grad()
    model.forward_backward(toks, [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)],
                           np.linspace(0.5, 1.5, n).astype(np.float32))
    check_block(ctx, g, model, m, 0, t, None, {}, {})
    model.close()


def test_t16_many_split_finish_block_ops_match_oracle(ctx):
    """16 tokens through a block with 2560 or more rows per projection: every dx has 20 or more row
    splits, so each linear's partials (down_proj's as SwiGLU's dh) are summed by the
    workgroup-per-(token, 64 columns) finish"""
    spec = tiny_spec(O.Q4_0, n_layer=1, n_embd=2560, n_head=20, n_head_kv=4, head_dim=128, rope_dim=128, n_ff=3072,
                     n_vocab=512)
    g, model, m = build(ctx, spec, 16, 32.0, ALL)
    t, n = 16, 12
    toks, pos, tok = sequence(spec.n_vocab, t, n, 11)
    model.debug_capture(0)
    model.zero_grad()
    ctx.set_timing(True)
    ctx.reset_timing()
    model.forward_backward(toks, [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)],
                           np.linspace(0.5, 1.5, n).astype(np.float32))
    ran = ctx.timing()
    ctx.set_timing(False)
    assert ran.get("rtq_bwd_finish_rows", (0,))[0] >= 4, ran  # q|k|v, o, gate|up, down (dh)
    check_block(ctx, g, model, m, 0, t, None, {}, {})
    model.close()


def test_packed_block_ops_match_oracle_recomputed(ctx):
    """a packed batch of four examples sharing a 100-token prompt (512 tokens) at the configs[2]
    block shape, activations recomputed in the backward"""
    spec = tiny_spec(O.Q4_0, **CONFIG2_BLOCK)
    g, model, m = build(ctx, spec, 16, 32.0, ALL)
    rng = O.Rng(21)
    prompt = [int(v) for v in (rng.vec_uniform_sym(100, 1.0) * 0.5 + 0.5) * (spec.n_vocab - 1)]
    seqs = [prompt + [int(v) for v in (rng.vec_uniform_sym(103, 1.0) * 0.5 + 0.5) * (spec.n_vocab - 1)]
            for _ in range(4)]
    p = pack(seqs)
    assert len(p.tokens) == 512 and p.shared == 100
    targets = []
    for k, s in enumerate(seqs):
        targets += p.map_targets(k, answer_targets(s, 150))
    wts = np.linspace(0.5, 1.5, len(targets)).astype(np.float32)
    model.checkpointing = True
    model.debug_capture(0)
    model.zero_grad()
    model.forward_backward_packed(p, targets, wts)
    assert model.checkpointing is True
    check_block(ctx, g, model, m, 0, 512, np.array(p.segments), {}, {"positions": p.positions})
    model.close()


@pytest.mark.parametrize("extra,start", [(60, 230), (824, 724)], ids=["680", "6792"])
def test_config3_block_ops_packed_match_oracle(ctx, extra, start):
    """the configs[3] block shape on a packed batch of eight examples sharing a 200-token prompt:
    680 tokens, and the configuration's own 8 x 1024 tokens (6792 packed, loss on each example's
    last 300 positions)"""
    spec = tiny_spec(O.Q4_K, n_layer=1, n_embd=2560, n_head=32, n_head_kv=8, head_dim=128, rope_dim=128, n_ff=9728,
                     n_vocab=4096, tensor_types={"ffn_down": O.Q6_K, "token_embd": O.Q6_K})
    g, model, m = build(ctx, spec, 16, 32.0, ALL)
    rng = O.Rng(33)
    V = spec.n_vocab
    prompt = [int(v) for v in (rng.vec_uniform_sym(200, 1.0) * 0.5 + 0.5) * (V - 1)]
    seqs = [prompt + [int(v) for v in (rng.vec_uniform_sym(extra, 1.0) * 0.5 + 0.5) * (V - 1)] for _ in range(8)]
    p = pack(seqs)
    t = 200 + 8 * extra
    assert len(p.tokens) == t and p.shared == 200
    targets = []
    for k, s in enumerate(seqs):
        targets += p.map_targets(k, answer_targets(s, start))
    model.debug_capture(0)
    model.zero_grad()
    model.forward_backward_packed(p, targets, np.full(len(targets), 1.0 / len(targets), np.float32))
    check_block(ctx, g, model, m, 0, t, np.array(p.segments), {}, {"positions": p.positions})
    model.close()


@pytest.mark.parametrize("fused", [False, None])  # None: the default (fused kernels)
def test_config4_block_ops_match_oracle_recomputed(ctx, fused):
    spec = tiny_spec(O.Q8_0, n_layer=2, arch="llama", tied=False, n_embd=4096, n_head=32, n_head_kv=8, head_dim=128,
                     rope_dim=128, n_ff=14336, n_vocab=4096, rope_base=5e5)
    g, model, m = build(ctx, spec, 64, 128.0, ALL)
    model.fused_attention = fused
    t, n = 2048, 1024
    toks, pos, tok = sequence(spec.n_vocab, t, n, 17)
    model.checkpointing = True
    model.debug_capture(0)
    model.zero_grad()
    model.forward_backward(toks, [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)],
                           np.full(n, 1.0 / n, np.float32))
    assert model.checkpointing is True and model.config["rope_neox"] == 0 and model.config["tied"] == 0
    check_block(ctx, g, model, m, 0, t, None, {}, {})
    model.close()
