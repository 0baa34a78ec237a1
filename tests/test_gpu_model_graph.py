"""The training step replayed from its HIP graph against the same step run eagerly.

A model captures its step's kernels once two steps in a row share the launch key (sizes, packed
layout, choices, adapters, buffers) and replays the graph on later steps with that key.  Two models
of one GGUF image and one set of adapters run the same calls side by side: one with graphs (the
default), one loaded with RTQ_STEP_GRAPH=0 (every step eager).  Every step's log-probs, hits and
every adapter's accumulated dA / dB are compared, through a sequence that replays several times
with eager work and host synchronisations between the replays (the other model's steps, adapter
uploads, a score without backward, other sizes, a packed batch) and changes what a replay must see
(new tokens, targets, loss weights, adapter values, gradients accumulating over steps).

Tolerance (max |graph - eager| / max |eager| per tensor): both models launch the same kernels on the
same inputs; the small-model products split K across workgroups and sum the splits with atomics,
whose order varies from run to run.
* F32 weights: 1e-4 (f32 rounding only).
* Q4_0 weights: log-probs 4e-3, gradients 8e-2, twice the quantised step's own noise floor (each
  linear re-quantises its input, so a one-ulp change of an f32 sum can move a code; the oracle
  against itself with every norm weight moved by one ulp differs by up to ~2e-3 and ~4e-2).
A replay that read stale inputs, skipped a kernel or repeated an accumulation differs by O(1).
"""
import numpy as np
import pytest

import oracle as O
import rust_trainer_amd as rt
from model_cases import adapters, sequence, tiny_spec
from rust_trainer_amd import gguf as G
from rust_trainer_amd.packing import answer_targets, pack

pytestmark = pytest.mark.gpu

NAMES = O.LINEARS
TOL = {O.F32: (1e-4, 1e-4), O.Q4_0: (4e-3, 8e-2)}


def rel(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    assert a.shape == b.shape
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)) if b.size else 0.0


def load(ctx, g, lora, monkeypatch, graph):
    if graph:
        monkeypatch.delenv("RTQ_STEP_GRAPH", raising=False)
    else:
        monkeypatch.setenv("RTQ_STEP_GRAPH", "0")
    model = rt.GpuModel.from_gguf(g, ctx=ctx)
    monkeypatch.delenv("RTQ_STEP_GRAPH", raising=False)
    model.attach_lora(4, 8.0, seed=1)
    set_adapters(model, lora)
    return model


def set_adapters(model, lora):
    for i in range(model.lora_count()):
        inf = model.lora_info(i)
        model.set_lora(i, *lora[(inf["layer"], NAMES[inf["which"]])])


def grads(model):
    return [np.concatenate([ga.ravel(), gb.ravel()]) for ga, gb in (model.lora(i)[2:] for i in range(model.lora_count()))]


@pytest.mark.parametrize("wtype", [O.F32, O.Q4_0])
def test_step_graph_replays_equal_eager_steps(ctx, wtype, monkeypatch):
    spec = tiny_spec(wtype, n_layer=2)
    g = G.GgufFile.from_bytes(spec.build())
    lora = adapters(g, 4, 8.0, b_std=0.05)
    mg = load(ctx, g, lora, monkeypatch, graph=True)
    me = load(ctx, g, lora, monkeypatch, graph=False)
    V = spec.n_vocab
    tol_lp, tol_g = TOL[wtype]
    worst = [0.0, 0.0]

    def both(call, zero=True, check_grads=True):
        out = []
        for m in (mg, me):
            if zero:
                m.zero_grad()
            out.append(call(m))
        (lp_g, h_g), (lp_e, h_e) = out
        e_lp = rel(lp_g, lp_e)
        assert e_lp <= tol_lp, f"log-probs differ by {e_lp:.2e}"
        assert h_g == h_e
        worst[0] = max(worst[0], e_lp)
        if check_grads:
            for i, (a, b) in enumerate(zip(grads(mg), grads(me))):
                e_g = rel(a, b)
                assert e_g <= tol_g, f"adapter {i}: gradients differ by {e_g:.2e}"
                worst[1] = max(worst[1], e_g)

    def plain(t, n, seed, weights=True):
        toks, pos, tok = sequence(V, t, n, seed)
        tg = [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)]
        w = np.linspace(0.5, 1.5, n).astype(np.float32) * (1 + seed % 3) if weights else None
        return lambda m: m.forward_backward(toks, tg, w)

    # one shape, new tokens each step: eager, eager (the first step's allocations changed the key),
    # captured, then replays
    for seed in range(1, 6):
        both(plain(48, 16, seed))
    r0 = mg.graph_replays
    assert r0 >= 2, f"{r0} replays over five equal-shaped steps"
    # new adapter values (device contents only): the graph is still replayed and reads them
    lora2 = adapters(g, 4, 8.0, seed=23, b_std=0.05)
    for m in (mg, me):
        set_adapters(m, lora2)
    both(plain(48, 16, 6))
    both(plain(48, 16, 7), zero=False)  # gradients accumulate over two replays
    assert mg.graph_replays == r0 + 2
    # a score (no backward) between replays, then the same training step again: replayed directly
    both(plain(48, 16, 8, weights=False), check_grads=False)
    both(plain(48, 16, 9))
    assert mg.graph_replays == r0 + 3
    # another size, three times (captured, replayed), then the first size again
    for seed in range(10, 13):
        both(plain(72, 20, seed))
    for seed in range(13, 17):
        both(plain(48, 16, seed))
    # a packed batch (positions, segments), repeated with other answers' weights
    rng = O.Rng(31)
    prompt = [int(v) for v in (rng.vec_uniform_sym(30, 1.0) * 0.5 + 0.5) * (V - 1)]
    seqs = [(prompt + [int(v) for v in (rng.vec_uniform_sym(e, 1.0) * 0.5 + 0.5) * (V - 1)], s)
            for e, s in [(20, 31), (26, 33), (14, 30)]]
    p = pack([s for s, _ in seqs])
    targets = []
    for k, (s, start) in enumerate(seqs):
        targets += p.map_targets(k, answer_targets(s, start))
    for rep in range(4):
        w = np.full(len(targets), 0.1 * (rep + 1), np.float32)
        both(lambda m: m.forward_backward_packed(p, targets, w))
    assert me.graph_replays == 0
    assert mg.graph_replays >= r0 + 7, f"{mg.graph_replays} replays"
    print(f"{wtype}: {mg.graph_replays} replays, worst log-prob {worst[0]:.2e}, gradient {worst[1]:.2e}")
    mg.close()
    me.close()


@pytest.mark.parametrize("ckpt", [False, True])
def test_step_graph_replays_hd128_cut_rows(ctx, ckpt, monkeypatch):
    """the launch sequences of the larger configurations: head size 128 (half-wave QK kernels, whose
    backward sums the cut blocks' partial slots), 320 tokens (rows cut into pieces), activations
    kept or recomputed; F32 weights, 1e-4 as above"""
    spec = tiny_spec(O.F32, n_layer=2, head_dim=128, rope_dim=128)
    g = G.GgufFile.from_bytes(spec.build())
    lora = adapters(g, 4, 8.0, b_std=0.05)
    mg = load(ctx, g, lora, monkeypatch, graph=True)
    me = load(ctx, g, lora, monkeypatch, graph=False)
    for m in (mg, me):
        m.checkpointing = ckpt
    for seed in range(1, 7):
        toks, pos, tok = sequence(spec.n_vocab, 320, 64, seed)
        tg = [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)]
        w = np.linspace(0.5, 1.5, 64).astype(np.float32) * seed
        out = []
        for m in (mg, me):
            m.zero_grad()
            out.append(m.forward_backward(toks, tg, w))
        assert rel(out[0][0], out[1][0]) <= 1e-4 and out[0][1] == out[1][1]
        for a, b in zip(grads(mg), grads(me)):
            assert rel(a, b) <= 1e-4
    assert mg.checkpointing is ckpt and mg.graph_replays >= 3 and me.graph_replays == 0
    mg.close()
    me.close()
