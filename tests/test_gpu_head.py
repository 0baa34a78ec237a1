"""GPU parity of the LM head + cross-entropy (Model::head, src/model.rs:561-609) and the embedding
gather (src/model.rs:446-454) against the CPU oracle.

Bars: log-probs and dx within max |gpu - oracle| / max |oracle| <= 1e-3 (and per element
1e-3 * max(|oracle|, 1) for logp); greedy hits equal; gathered rows bit-exact (they are row()).
"""
import ctypes

import numpy as np
import pytest

import oracle as O
import rust_trainer_amd as rt
from rust_trainer_amd.head import head_d

pytestmark = pytest.mark.gpu

TOL = 1e-3


def rel_err(got, want):
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    assert got.shape == want.shape
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def case(wtype, V, d, t, n, seed=1):
    w = O.Rng(seed).vec_normal(V * d, 0.02).reshape(V, d)
    blocks = O.quantize(wtype, w) if wtype != O.F32 else w.astype(np.float32)
    x = O.Rng(seed + 1).vec_normal(t * d, 1.0).reshape(t, d)
    norm = (1.0 + O.Rng(seed + 2).vec_normal(d, 0.1)).astype(np.float32)
    rng = np.random.default_rng(seed)
    pos = rng.integers(0, t, n).astype(np.int32)
    tok = rng.integers(0, V, n).astype(np.int32)
    wts = rng.uniform(0.25, 2.0, n).astype(np.float32)
    return blocks, x, norm, pos, tok, wts


def oracle_blocks(wtype, blocks):
    return blocks if wtype != O.F32 else np.ascontiguousarray(blocks, np.float32).view(np.uint8)


@pytest.mark.parametrize("wtype,V,d,t,n", [
    (O.Q4_0, 700, 256, 11, 7), (O.Q8_0, 5001, 256, 40, 33), (O.Q4_K, 4096, 512, 20, 16),
    (O.Q6_K, 3000, 256, 9, 24), (O.Q4_0, 151936, 1024, 96, 64), (O.F32, 1000, 96, 7, 12)])
def test_head_matches_oracle(ctx, wtype, V, d, t, n):
    blocks, x, norm, pos, tok, wts = case(wtype, V, d, t, n)
    eps, off = 1e-6, 0.0
    f = rt.HipFrozen(wtype, blocks, V, d, ctx=ctx)
    targets = [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)]
    logp, dx, hits = rt.head(f, norm, x, targets, wts, eps=eps, offset=off)
    lp_o, hits_o, dx_o = O.lm_head(wtype, oracle_blocks(wtype, blocks), V, d, norm, x, pos, tok, wts, eps=eps,
                                   off=off, chunk=64, nthreads=16)
    assert rel_err(logp, lp_o) <= TOL
    assert np.all(np.abs(logp - lp_o) <= TOL * np.maximum(np.abs(lp_o), 1.0))
    assert hits == hits_o
    assert rel_err(dx, dx_o) <= TOL
    untouched = np.setdiff1d(np.arange(t), pos)
    assert not dx.reshape(t, d)[untouched].any()
    # log-probs only: same log-probs, no gradient
    lp2, dx2, h2 = rt.head(f, norm, x, targets, None, eps=eps, offset=off)
    np.testing.assert_array_equal(lp2, logp)
    assert h2 == hits and dx2.size == 0
    f.close()


def test_head_offset_norm_and_repeated_positions(ctx):
    """zero-centred norm (offset 1) and several targets on one position (their gradients add)"""
    wtype, V, d, t = O.Q8_0, 2048, 256, 5
    blocks, x, norm, _, _, _ = case(wtype, V, d, t, 1, seed=9)
    pos = np.array([2, 2, 0, 2, 4, 0], np.int32)
    tok = np.array([1, 2047, 5, 1, 900, 5], np.int32)
    wts = np.array([1.0, 0.5, 2.0, 1.0, 1.5, 0.75], np.float32)
    f = rt.HipFrozen(wtype, blocks, V, d, ctx=ctx)
    logp, dx, hits = rt.head(f, norm, x, [rt.Target(int(p), int(k)) for p, k in zip(pos, tok)], wts, eps=1e-5,
                             offset=1.0)
    lp_o, hits_o, dx_o = O.lm_head(wtype, blocks, V, d, norm, x, pos, tok, wts, eps=1e-5, off=1.0)
    assert rel_err(logp, lp_o) <= TOL and hits == hits_o and rel_err(dx, dx_o) <= TOL
    assert logp[0] == logp[3] and logp[2] == logp[5]  # same (pos, token): same log-prob
    f.close()


def test_head_rejects_bad_targets_and_handles_none(ctx):
    blocks, x, norm, _, _, _ = case(O.Q4_0, 256, 64, 3, 1)
    f = rt.HipFrozen(O.Q4_0, blocks, 256, 64, ctx=ctx)
    with pytest.raises(rt.RtqError):
        rt.head(f, norm, x, [rt.Target(3, 0)], [1.0])
    with pytest.raises(rt.RtqError):
        rt.head(f, norm, x, [rt.Target(0, 256)], [1.0])
    logp, dx, hits = rt.head(f, norm, x, [], [])
    assert logp.size == 0 and hits == 0 and dx.size == 3 * 64 and not dx.any()
    f.close()


def test_head_device_api_marks_invalid_targets(ctx):
    """rtq_lm_head_d: out-of-range targets read nothing (logp NaN, hit 0, no gradient); the
    valid targets match the host API.  The host call has 2 targets and the device call 5, so their
    logit products run on different kernels (t <= 4: rtq_gemvq4_*, whose Q4_0 sums add the
    k-groups' scaled shares in another order): equal to 1e-5, not bit for bit."""
    import torch

    wtype, V, d, t = O.Q4_0, 4096, 256, 6
    blocks, x, norm, _, _, _ = case(wtype, V, d, t, 1, seed=4)
    pos = np.array([1, 6, 3, -1, 5], np.int32)
    tok = np.array([7, 0, V, 2, 4095], np.int32)
    wts = np.ones(5, np.float32)
    f = rt.HipFrozen(wtype, blocks, V, d, ctx=ctx)
    dev = torch.device("cuda", 0)
    xd, nd = torch.from_numpy(x).to(dev), torch.from_numpy(norm).to(dev)
    pd, kd, wd = (torch.from_numpy(a).to(dev) for a in (pos, tok, wts))
    lp = torch.empty(5, device=dev)
    hit = torch.empty(5, dtype=torch.int32, device=dev)
    dxd = torch.full((t, d), 7.0, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    head_d(f, nd.data_ptr(), xd.data_ptr(), t, pd.data_ptr(), kd.data_ptr(), wd.data_ptr(), 5, lp.data_ptr(),
           hit.data_ptr(), dxd.data_ptr(), stream=st)
    torch.cuda.synchronize()
    lp, hit, dxd = lp.cpu().numpy(), hit.cpu().numpy(), dxd.cpu().numpy()
    assert np.isnan(lp[[1, 2, 3]]).all() and not hit[[1, 2, 3]].any()
    good = [0, 4]
    lp_h, dx_h, _ = rt.head(f, norm, x, [rt.Target(int(pos[i]), int(tok[i])) for i in good], wts[good])
    np.testing.assert_allclose(lp[good], lp_h, rtol=1e-5, atol=0)
    np.testing.assert_allclose(dxd.reshape(-1), dx_h, rtol=1e-5, atol=1e-5 * np.abs(dx_h).max())
    assert not dxd.reshape(t, d)[[0, 2, 3, 4]].any()  # the rows without a valid target are cleared
    f.close()


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0, O.Q4_K, O.Q6_K, O.F32])
def test_embed_tokens_gathers_rows(ctx, wtype):
    V, d = 1000, 256
    blocks, _, _, _, _, _ = case(wtype, V, d, 1, 1, seed=3)
    f = rt.HipFrozen(wtype, blocks, V, d, ctx=ctx)
    toks = np.array([0, 999, 5, 5, 123, 998, 1], np.int32)
    x = rt.embed_tokens(f, toks).reshape(-1, d)
    for i, k in enumerate(toks):
        np.testing.assert_array_equal(x[i], O.frozen_row(wtype, oracle_blocks(wtype, blocks), V, d, int(k)))
    with pytest.raises(rt.RtqError):
        rt.embed_tokens(f, [1000])
    # device gather: an id out of range gives a NaN row and reads nothing
    import torch

    ids = torch.tensor([5, 1000, -3, 998], dtype=torch.int32, device="cuda")
    out = torch.empty(4, d, device="cuda")
    rt.lib().rtq_frozen_gather_d(ctx.handle, f.handle, ids.data_ptr(), 4, out.data_ptr(),
                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    o = out.cpu().numpy()
    assert np.isnan(o[1]).all() and np.isnan(o[2]).all()
    np.testing.assert_array_equal(o[[0, 3]], x[[2, 5]])
    f.close()
