"""GPU: frozen weights uploaded straight from a GGUF image (rtq_weight_from_gguf, the loader's
``fz(&l.wq)``, src/rie.rs:183, :218-231) behave exactly like weights created from the same bytes,
and agree with the oracle."""
import ctypes

import numpy as np
import pytest

import oracle as O
import rust_trainer_amd as rt
from rust_trainer_amd import gguf as G

pytestmark = pytest.mark.gpu

TOL = 1e-3


def rel_err(got, want):
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0, O.Q4_K, O.Q6_K])
@pytest.mark.parametrize("mapped", [False, True])
def test_weight_from_gguf_matches_direct_create(ctx, tmp_path, wtype, mapped):
    s = G.SyntheticSpec.tiny("qwen3", wtype)
    s.n_layer, s.tied_output = 1, False
    if mapped:
        path = tmp_path / "m.gguf"
        w = s.writer()
        w.write(path)
        w.close()
        g = G.GgufFile.open(path)
    else:
        g = G.GgufFile.from_bytes(s.build())
    t = 5
    for name in ["blk.0.attn_q.weight", "blk.0.ffn_down.weight", "output.weight", "token_embd.weight"]:
        info = g.tensor(name)
        n, k = info.n_rows(), info.row_len()
        raw = np.array(g.tensor_data(info))
        a = rt.HipFrozen.from_gguf(g, name, ctx=ctx)
        b = rt.HipFrozen(info.ty, raw, n, k, ctx=ctx)
        assert (a.out_dim(), a.in_dim(), a.nbytes(), a.ggml_type) == (n, k, raw.nbytes, wtype)
        x = O.Rng(2).vec_normal(t * k, 1.0)
        ya, yb = a.forward(x, t), b.forward(x, t)
        np.testing.assert_array_equal(ya, yb, err_msg=name)
        assert rel_err(ya, O.frozen_forward(wtype, raw, n, k, x.reshape(t, k))) <= TOL, name
        dy = O.Rng(3).vec_normal(t * n, 1.0)
        da, db = np.zeros(t * k, np.float32), np.zeros(t * k, np.float32)
        a.backward_input(dy, t, da)
        b.backward_input(dy, t, db)
        np.testing.assert_array_equal(da, db, err_msg=name)
        ra = np.empty(k, np.float32)
        a.row(n - 1, ra)
        np.testing.assert_array_equal(ra, O.frozen_row(wtype, raw, n, k, n - 1))
        a.close()
        b.close()
    h = ctypes.c_void_p()
    assert rt.lib().rtq_weight_from_gguf(ctx.handle, g.handle, b"absent.weight", ctypes.byref(h)) == 1
    assert b"absent.weight" in rt.lib().rtq_last_error()
    g.close()
