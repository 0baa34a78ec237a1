"""Precision of the device's attention backward (Attention::backward, src/attention.rs:246-367,
f32 in the reference) against a float64 backward computed from the device's own q, k, v and dO.

One block's tensors are captured during a step (rtq_model_debug_capture) of an F32-weight model
whose loss weights cycle through 1e-6, 1 and 1e3 over the target positions, so the captured last
block's dO rows span nine orders of magnitude (rows without a target: dO = 0).  The float64
reference recomputes P = softmax((q scale) k^T) (causal), dP = dO v^T, dS = P (dP - rowsum(P dP)),
dq = dS k scale, dk = dS^T q scale, dv = P^T dO from the captured operands.

Each product of the device's backward runs on 16-bit MFMA with both operands split into bf16 hi /
lo parts, each rounded to nearest (hi + lo within 2^-17 of the operand), f32 accumulation, so a
product carries a relative error near 2^-16 (1.5e-5) whatever its magnitude (bf16 keeps f32's
exponent range: no row scaling is needed).  Errors are measured per row relative to that row's
largest |value| (dq rows: query positions, dk / dv rows: key positions), so a row of 1e-6 is held
to its own scale, not to the 1e3 rows'.  Measured: 1.1e-5 .. 2.2e-5 (truncated splits: up to
9.2e-5).  Bar: 4e-5 per row, on both attention paths and both head sizes; rows whose reference is
exactly zero must be zero on the device.
"""
import numpy as np
import pytest

import oracle as O
import rust_trainer_amd as rt
from model_cases import adapters, sequence, tiny_spec
from rust_trainer_amd import gguf as G

pytestmark = pytest.mark.gpu

NAMES = O.LINEARS


def f64_backward(q, k, v, dO, nh, nkv, hd):
    t = q.shape[0]
    grp = nh // nkv
    q = q.reshape(t, nh, hd).astype(np.float64)
    k = k.reshape(t, nkv, hd).astype(np.float64)
    v = v.reshape(t, nkv, hd).astype(np.float64)
    dO = dO.reshape(t, nh, hd).astype(np.float64)
    scale = 1.0 / np.sqrt(hd)
    mask = np.tril(np.ones((t, t), bool))
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for h in range(nh):
        g = h // grp
        s = np.where(mask, (q[:, h] * scale) @ k[:, g].T, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        dp = dO[:, h] @ v[:, g].T
        ds = p * (dp - (p * dp).sum(axis=1, keepdims=True))
        dq[:, h] = ds @ k[:, g] * scale
        dk[:, g] += ds.T @ q[:, h] * scale
        dv[:, g] += p.T @ dO[:, h]
    return dq.reshape(t, -1), dk.reshape(t, -1), dv.reshape(t, -1)


def row_err(got, want):
    """largest per-row error relative to the row's largest |want| (rows of zeros excluded); and
    whether the rows that are zero in want are zero in got"""
    got = got.astype(np.float64)
    scale = np.abs(want).max(axis=1)
    nz = scale > 0
    err = (np.abs(got - want).max(axis=1)[nz] / scale[nz]).max()
    return float(err), bool(not got[~nz].any())


@pytest.mark.parametrize("fused", [True, False])
@pytest.mark.parametrize("hd", [64, 128])
def test_attention_backward_precision_mixed_row_magnitudes(ctx, hd, fused):
    spec = tiny_spec(O.F32, n_layer=2, n_head=4, n_head_kv=2, head_dim=hd, rope_dim=hd)
    g = G.GgufFile.from_bytes(spec.build())
    model = rt.GpuModel.from_gguf(g, ctx=ctx)
    model.fused_attention = fused
    model.attach_lora(4, 8.0, seed=1)
    lora = adapters(g, 4, 8.0)
    for i in range(model.lora_count()):
        inf = model.lora_info(i)
        model.set_lora(i, *lora[(inf["layer"], NAMES[inf["which"]])])
    t, n = 300, 240
    toks, pos, tok = sequence(spec.n_vocab, t, n, 5)
    wts = np.array([(1e-6, 1.0, 1e3)[i % 3] for i in range(n)], np.float32)
    model.debug_capture(1)
    model.zero_grad()
    model.forward_backward(toks, [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)], wts)
    c = model.config
    nh, nkv = c["n_head"], c["n_head_kv"]
    qd, kd = nh * hd, nkv * hd
    T = {name: model.debug_tensor(name, (t, w)) for name, w in
         (("q", qd), ("k", kd), ("v", kd), ("d_o", qd), ("dq", qd), ("dk", kd), ("dv", kd))}
    mags = np.abs(T["d_o"]).max(axis=1)
    assert mags.max() / mags[mags > 0].min() > 1e6  # the rows do span the magnitudes
    dq, dk, dv = f64_backward(T["q"], T["k"], T["v"], T["d_o"], nh, nkv, hd)
    out = {}
    for name, want in (("dq", dq), ("dk", dk), ("dv", dv)):
        out[name] = row_err(T[name], want)
    print(f"hd {hd} fused {fused}: " + ", ".join(f"{k} {e:.2e}" for k, (e, _) in out.items()))
    for name, (err, zeros) in out.items():
        assert zeros, f"{name}: rows that are zero in the reference are not zero"
        assert err <= 4e-5, f"{name}: row-relative error {err:.2e}"
    model.close()
