"""GPU parity: the gfx950 path through the C ABI against the CPU oracle on identical seeded inputs.

Bars (from the hot-path contract):
  * activation quantisation (Q8_0 / Q8_K blocks) and the integer block sums: bit-exact;
  * row() dequantisation: bit-exact;
  * f32 outputs and gradients: max |gpu - oracle| / max |oracle| <= 1e-3 per tensor (TOL);
    the reference's own per-element check 1e-3 * max(|want|, 1) (tests/engine.rs:115) is also
    applied to dx against the dense dequantised product.
Inputs follow the benchmark recipe: W ~ N(0, 0.02) seed 1, X ~ N(0, 1) seed 2, dy ~ N(0, 1)
seed 3, A ~ N(0, 1/1024) (std 1/32) seed 4, B ~ N(0, 0.01) seed 5, all from the reference Rng.
"""
import numpy as np
import pytest

import oracle as O
import rust_trainer_amd as rt

pytestmark = pytest.mark.gpu

TOL = 1e-3
FORMATS = [O.Q4_0, O.Q8_0, O.Q4_K, O.Q6_K]
BLOCK = {O.Q4_0: 32, O.Q8_0: 32, O.Q4_K: 256, O.Q6_K: 256}


def cases(shapes, formats=FORMATS):
    """(format, *shape) for every shape whose K is a whole number of the format's blocks."""
    return [(f, *sh) for f in formats for sh in shapes if sh[1] % BLOCK[f] == 0]


def rel_err(got, want):
    got = np.asarray(got, np.float64).reshape(-1)
    want = np.asarray(want, np.float64).reshape(-1)
    assert got.shape == want.shape
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def make(wtype, n, k, t, seed=1):
    w = O.Rng(seed).vec_normal(n * k, 0.02).reshape(n, k)
    blocks = O.quantize(wtype, w)
    x = O.Rng(seed + 1).vec_normal(t * k, 1.0).reshape(t, k)
    dy = O.Rng(seed + 2).vec_normal(t * n, 1.0).reshape(t, n)
    return blocks, x, dy


def lora(n, k, r):
    A = O.Rng(4).vec_normal(r * k, 1.0 / 32.0).reshape(r, k)
    B = O.Rng(5).vec_normal(n * r, 0.01).reshape(n, r)
    return A, B


def hip(ctx, wtype, blocks, n, k):
    return rt.HipFrozen(wtype, blocks, n, k, ctx=ctx)


# ---------------------------------------------------------------- bit-exact parts
@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
def test_activation_quantisation_bit_exact(ctx, wtype):
    n, k, t = 64, 1024, 37
    blocks, x, _ = make(wtype, n, k, t)
    # tie cases: a block whose amax is 127 has id = 1, so x = m + 0.5 must round away from zero
    x[0, :32] = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5] + [j - 11.5 for j in range(24)], np.float32)
    x[1, 32:64] = 0.0  # all-zero block: d = 0, codes 0
    x[2, :32] *= np.float32(1e-6)  # tiny scale: fp16 subnormal d
    w = hip(ctx, wtype, blocks, n, k)
    got = w.debug_quantize_acts(x, t)
    want = O.quantize_acts(wtype, x)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("wtype", [O.Q4_K, O.Q6_K])
def test_activation_quantisation_q8_k_bit_exact(ctx, wtype):
    n, k, t = 64, 1024, 21
    blocks, x, _ = make(wtype, n, k, t)
    # first element of largest |x| wins, across the 16-column segments of a super-block too
    x[0, :256] *= np.float32(0.01)
    x[0, 40], x[0, 200] = -7.0, 7.0
    x[1, 256:512] *= np.float32(0.01)
    x[1, 300], x[1, 301] = 5.0, -5.0
    x[2, 512:768] *= np.float32(0.01)
    x[2, 520], x[2, 515] = -3.0, 3.0  # lower column, later segment order does not matter
    # max = -127: iscale = 1, so x = m + 0.5 rounds to even
    x[3, :8] = np.array([-127.0, 2.5, -2.5, 0.5, -0.5, 1.5, 126.5, -126.5], np.float32)
    x[3, 8:256] = np.float32(0.25)
    x[4, 768:1024] = 0.0  # all-zero super-block: d = 0, codes 0
    x[5, :256] *= np.float32(1e-6)
    w = hip(ctx, wtype, blocks, n, k)
    got = w.debug_quantize_acts(x, t)
    want = O.quantize_acts(wtype, x)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("wtype,n,k,t", cases([(80, 256, 20), (64, 96, 3), (128, 1024, 65), (48, 512, 3)]))
def test_block_isums_bit_exact(ctx, wtype, n, k, t):
    blocks, x, _ = make(wtype, n, k, t)
    w = hip(ctx, wtype, blocks, n, k)
    got = w.debug_block_isums(x, t)
    want = O.block_isums(wtype, blocks, O.quantize_acts(wtype, x), k)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("wtype", FORMATS)
def test_row_dequant_bit_exact(ctx, wtype):
    n, k = 200, 384 if BLOCK[wtype] == 32 else 512
    blocks, _, _ = make(wtype, n, k, 1)
    w = hip(ctx, wtype, blocks, n, k)
    out = np.empty(k, np.float32)
    for r in (0, 1, 15, 16, 63, 64, 127, 199):
        w.row(r, out)
        assert np.array_equal(out, O.frozen_row(wtype, blocks, n, k, r)), r


# ---------------------------------------------------------------- FrozenMatmul
SHAPES = [(64, 128, 1), (100, 96, 5), (256, 512, 37), (3072, 1024, 16), (3072, 1024, 256), (1024, 3072, 64),
          (2048, 1024, 1), (1024, 1024, 16), (80, 2048, 130)]


@pytest.mark.parametrize("wtype,n,k,t", cases(SHAPES))
def test_forward_matches_oracle(ctx, wtype, n, k, t):
    blocks, x, _ = make(wtype, n, k, t)
    w = hip(ctx, wtype, blocks, n, k)
    y = w.forward(x, t)
    assert y.shape == (t * n,)
    want = O.frozen_forward(wtype, blocks, n, k, x, nthreads=8)
    assert rel_err(y, want) <= TOL


@pytest.mark.parametrize("wtype,n,k,t", cases(SHAPES))
def test_backward_input_matches_oracle(ctx, wtype, n, k, t):
    blocks, _, dy = make(wtype, n, k, t)
    w = hip(ctx, wtype, blocks, n, k)
    dx0 = O.Rng(7).vec_normal(t * k, 1.0)
    dx = dx0.copy()
    w.backward_input(dy, t, dx)  # accumulates
    want = O.frozen_backward_input(wtype, blocks, n, k, dy, dx=np.zeros((t, k), np.float32), nthreads=8)
    assert rel_err(dx - dx0, want) <= TOL
    # tests/engine.rs:96-120: equals the dense dy . W built from row(), 1e-3 * max(|want|, 1)
    W = np.stack([O.frozen_row(wtype, blocks, n, k, r) for r in range(n)]).astype(np.float64)
    dense = dy.astype(np.float64) @ W
    got = (dx - dx0).reshape(t, k)
    assert (np.abs(got - dense) < 1e-3 * np.maximum(np.abs(dense), 1.0)).all()


def test_empty_token_count(ctx):
    blocks, _, _ = make(O.Q4_0, 64, 128, 1)
    w = hip(ctx, O.Q4_0, blocks, 64, 128)
    assert w.forward(np.zeros(0, np.float32), 0).size == 0
    dx = np.zeros(0, np.float32)
    w.backward_input(np.zeros(0, np.float32), 0, dx)


def test_nbytes_and_dims(ctx):
    blocks, _, _ = make(O.Q4_0, 3072, 1024, 1)
    w = hip(ctx, O.Q4_0, blocks, 3072, 1024)
    assert w.nbytes() == 3072 * 1024 // 32 * 18 == blocks.nbytes
    assert (w.out_dim(), w.in_dim()) == (3072, 1024)


def test_errors_are_status_codes(ctx):
    blocks, _, _ = make(O.Q4_0, 64, 128, 1)
    with pytest.raises(rt.RtqError) as e:
        rt.HipFrozen(O.Q4_0, blocks[:, :-1], 64, 128, ctx=ctx)  # wrong byte count
    assert e.value.status == 1
    with pytest.raises(rt.RtqError) as e:
        rt.HipFrozen(3, blocks, 64, 128, ctx=ctx)  # Q4_1: not a supported format
    assert e.value.status == 2
    w = hip(ctx, O.Q4_0, blocks, 64, 128)
    with pytest.raises(rt.RtqError):
        w.row(64, np.empty(128, np.float32))


# ---------------------------------------------------------------- Linear + LoRA
@pytest.mark.parametrize("wtype,n,k,t,r", cases([(3072, 1024, 256, 16), (256, 512, 37, 2), (100, 96, 5, 16),
                                                 (512, 256, 70, 64), (512, 2048, 9, 16), (1024, 3072, 130, 8)]))
def test_linear_lora_matches_oracle(ctx, wtype, n, k, t, r):
    alpha = 2.0 * r
    blocks, x, dy = make(wtype, n, k, t)
    A, B = lora(n, k, r)
    bias = O.Rng(6).vec_normal(n, 0.1)
    lin = rt.Linear("blk.0.ffn_gate", hip(ctx, wtype, blocks, n, k), bias=bias)
    lin.lora = rt.Lora(r, alpha, A, B)
    y = lin.forward(x, t)
    want = O.linear_forward(wtype, blocks, n, k, x, bias=bias, A=A, B=B, alpha=alpha, nthreads=8)
    assert rel_err(y, want) <= TOL
    ga0 = O.Rng(8).vec_normal(r * k, 0.01)
    gb0 = O.Rng(9).vec_normal(n * r, 0.01)
    lin.lora.ga[...] = ga0
    lin.lora.gb[...] = gb0
    dx = lin.backward(x, dy, t)
    wdx, wga, wgb = O.linear_backward(wtype, blocks, n, k, x, dy, A=A, B=B, alpha=alpha, nthreads=8)
    assert rel_err(dx, wdx) <= TOL
    assert rel_err(lin.lora.ga - ga0, wga) <= TOL
    assert rel_err(lin.lora.gb - gb0, wgb) <= TOL


@pytest.mark.parametrize("wtype", FORMATS)
@pytest.mark.parametrize("t", [1, 7, 16])
def test_linear_lora_large_n(ctx, wtype, t):
    # N = 65536 takes the T <= 16 GEMV kernel with K split across workgroups (atomics), plus the
    # LoRA up-projection and bias in its epilogue
    n, k, r = 65536, 1024, 16
    alpha = 32.0
    blocks, x, dy = make(wtype, n, k, t)
    A, B = lora(n, k, r)
    bias = O.Rng(6).vec_normal(n, 0.1)
    lin = rt.Linear("blk.0.ffn_up", hip(ctx, wtype, blocks, n, k), bias=bias)
    lin.lora = rt.Lora(r, alpha, A, B)
    y = lin.forward(x, t)
    want = O.linear_forward(wtype, blocks, n, k, x, bias=bias, A=A, B=B, alpha=alpha, nthreads=8)
    assert rel_err(y, want) <= TOL
    dx = lin.backward(x, dy, t)
    wdx, wga, wgb = O.linear_backward(wtype, blocks, n, k, x, dy, A=A, B=B, alpha=alpha, nthreads=8)
    assert rel_err(dx, wdx) <= TOL
    assert rel_err(lin.lora.ga, wga) <= TOL
    assert rel_err(lin.lora.gb, wgb) <= TOL


def test_linear_disabled_adapter_and_no_bias(ctx):
    n, k, t, r = 256, 256, 9, 4
    blocks, x, dy = make(O.Q4_0, n, k, t)
    A, B = lora(n, k, r)
    lin = rt.Linear("blk.0.attn_q", hip(ctx, O.Q4_0, blocks, n, k))
    lin.lora = rt.Lora(r, 8.0, A, B)
    lin.lora_enabled = False
    y = lin.forward(x, t)
    assert rel_err(y, O.frozen_forward(O.Q4_0, blocks, n, k, x)) <= TOL
    dx = lin.backward(x, dy, t)
    assert rel_err(dx, O.frozen_backward_input(O.Q4_0, blocks, n, k, dy)) <= TOL
    assert not lin.lora.ga.any() and not lin.lora.gb.any()


# ---------------------------------------------------------------- device-pointer API
def test_device_pointer_api_matches_host_api(ctx):
    import torch

    n, k, t, r = 3072, 1024, 256, 16
    blocks, x, dy = make(O.Q4_0, n, k, t)
    A, B = lora(n, k, r)
    w = hip(ctx, O.Q4_0, blocks, n, k)
    dev = torch.device("cuda", 0)
    X = torch.from_numpy(x).to(dev)
    DY = torch.from_numpy(dy).to(dev)
    At, Bt = torch.from_numpy(A).to(dev), torch.from_numpy(B).to(dev)
    Y = torch.empty(t, n, device=dev)
    DX = torch.empty(t, k, device=dev)
    GA = torch.zeros(r, k, device=dev)
    GB = torch.zeros(n, r, device=dev)
    from rust_trainer_amd import _ffi
    import ctypes

    lv = _ffi.RtqLora(r, 32.0, At.data_ptr(), Bt.data_ptr(), 1)
    s = torch.cuda.current_stream().cuda_stream
    _ffi.check(_ffi.lib().rtq_linear_forward_d(ctx.handle, w.handle, None, ctypes.byref(lv), X.data_ptr(), t,
                                               Y.data_ptr(), s), "fwd_d")
    _ffi.check(_ffi.lib().rtq_linear_backward_d(ctx.handle, w.handle, ctypes.byref(lv), X.data_ptr(), DY.data_ptr(), t,
                                                DX.data_ptr(), GA.data_ptr(), GB.data_ptr(), s), "bwd_d")
    torch.cuda.synchronize()
    lin = rt.Linear("x", w)
    lin.lora = rt.Lora(r, 32.0, A, B)
    assert rel_err(Y.cpu().numpy(), lin.forward(x, t)) <= 1e-6
    dx = lin.backward(x, dy, t)
    assert rel_err(DX.cpu().numpy(), dx) <= 1e-5
    assert rel_err(GA.cpu().numpy(), lin.lora.ga) <= 1e-5
    assert rel_err(GB.cpu().numpy(), lin.lora.gb) <= 1e-5


# ---------------------------------------------------------------- maximum size
@pytest.mark.parametrize("wtype", FORMATS)
def test_lm_head_shape_t1(ctx, wtype):
    # tied LM head of Qwen3-0.6B: 151936 x 1024, one token (decode-shaped GEMV)
    n, k, t = 151936, 1024, 1
    blocks, x, dy = make(wtype, n, k, t)
    w = hip(ctx, wtype, blocks, n, k)
    y = w.forward(x, t)
    assert rel_err(y, O.frozen_forward(wtype, blocks, n, k, x, nthreads=16)) <= TOL
    dx = np.zeros(t * k, np.float32)
    w.backward_input(dy, t, dx)
    assert rel_err(dx, O.frozen_backward_input(wtype, blocks, n, k, dy, nthreads=16)) <= TOL


# ---------------------------------------------------------------- configs[1] sweep points
def _dense_dx_check(wtype, blocks, n, k, dy, got):
    """tests/engine.rs:96-120: dx equals the dense dy . W of the dequantised rows, per element
    within 1e-3 * max(|want|, 1)"""
    W = O.dequantize(wtype, blocks, k).reshape(n, k).astype(np.float64)
    dense = dy.astype(np.float64) @ W
    bad = np.abs(got.reshape(dense.shape) - dense) >= 1e-3 * np.maximum(np.abs(dense), 1.0)
    assert not bad.any(), f"{int(bad.sum())} dx elements off"


@pytest.mark.parametrize("wtype", [O.Q8_0, O.Q4_K, O.Q6_K])
@pytest.mark.parametrize("shape", ["q_proj", "kv_proj", "down_proj"])
def test_config1_sweep_t2048_matches_oracle(ctx, wtype, shape):
    """configs[1] at T = 2048 (Linear forward with LoRA r = 16, Linear backward: dx, dA, dB)"""
    import time

    n, k = {"q_proj": (2048, 1024), "kv_proj": (1024, 1024), "down_proj": (1024, 3072)}[shape]
    t, r = 2048, 16
    blocks, x, dy = make(wtype, n, k, t)
    A, B = lora(n, k, r)
    lin = rt.Linear(shape, hip(ctx, wtype, blocks, n, k))
    lin.lora = rt.Lora(r, 32.0, A, B)
    y = lin.forward(x, t)
    dx = lin.backward(x, dy, t)
    t0 = time.perf_counter()
    wy = O.linear_forward(wtype, blocks, n, k, x, A=A, B=B, alpha=32.0, nthreads=16)
    wdx, wga, wgb = O.linear_backward(wtype, blocks, n, k, x, dy, A=A, B=B, alpha=32.0, nthreads=16)
    print(f"oracle (16 threads): {time.perf_counter() - t0:.1f} s")
    errs = rel_err(y, wy), rel_err(dx, wdx), rel_err(lin.lora.ga, wga), rel_err(lin.lora.gb, wgb)
    print("y, dx, dA, dB rel err", " ".join(f"{e:.1e}" for e in errs))
    assert max(errs) <= TOL
    # the frozen part alone against the dense product (FrozenMatmul::backward_input)
    dxf = np.zeros(t * k, np.float32)
    lin.w.backward_input(dy, t, dxf)
    _dense_dx_check(wtype, blocks, n, k, dy, dxf)


@pytest.mark.parametrize("wtype,t", [(f, 16) for f in FORMATS] + [(O.Q4_K, 256), (O.Q8_0, 256), (O.Q6_K, 256)] +
                         [(f, 2048) for f in FORMATS])
def test_config1_lm_head_matches_oracle(ctx, wtype, t):
    """configs[1]'s tied LM head 151936 x 1024 (no adapter) at T = 16 and 2048 in every format and
    T = 256 (Q4_K, Q8_0, Q6_K): forward and FrozenMatmul::backward_input against the oracle and, per
    element, against the dense product"""
    import time

    n, k = 151936, 1024
    blocks, x, dy = make(wtype, n, k, t)
    w = hip(ctx, wtype, blocks, n, k)
    y = w.forward(x, t)
    dx = np.zeros(t * k, np.float32)
    w.backward_input(dy, t, dx)
    t0 = time.perf_counter()
    wy = O.frozen_forward(wtype, blocks, n, k, x, nthreads=16)
    wdx = O.frozen_backward_input(wtype, blocks, n, k, dy, nthreads=16)
    print(f"oracle (16 threads): {time.perf_counter() - t0:.1f} s; y {rel_err(y, wy):.1e} dx {rel_err(dx, wdx):.1e}")
    assert rel_err(y, wy) <= TOL and rel_err(dx, wdx) <= TOL
    _dense_dx_check(wtype, blocks, n, k, dy, dx)


# ---------------------------------------------------------------- large-grid forward (rtq_mm_*)
@pytest.fixture(scope="module", params=["1", "2", "3"], ids=["mm128", "mm64", "mm32"])
def ctx_mm(request):
    """A context that sends every wide Q4_0 / Q8_0 forward through the 128 x 128-tile kernel
    (RTQ_FWD_MM=1) or its 128 x 64- or 128 x 32-tile variant (RTQ_FWD_MM=2, 3), so small shapes
    cover their padding and epilogue cases."""
    import os

    old = os.environ.get("RTQ_FWD_MM")
    os.environ["RTQ_FWD_MM"] = request.param
    try:
        c = rt.Context(0)
    finally:
        if old is None:
            del os.environ["RTQ_FWD_MM"]
        else:
            os.environ["RTQ_FWD_MM"] = old
    yield c
    c.close()


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
@pytest.mark.parametrize("n,k,t,r", [(200, 256, 130, 16), (320, 512, 256, 0), (1000, 1024, 300, 80), (130, 128, 129, 16),
                                     (64, 128, 17, 4)])
def test_linear_forward_mm_matches_oracle(ctx_mm, wtype, n, k, t, r):
    # partial row groups and row blocks (N = 130, 200), N % 4 != 0 (scalar stores), token padding
    # inside a 128-token block, no LoRA, LoRA rank above the LDS staging limit (80)
    blocks, x, _ = make(wtype, n, k, t)
    bias = O.Rng(6).vec_normal(n, 0.1)
    lin = rt.Linear("blk.0.attn_q", hip(ctx_mm, wtype, blocks, n, k), bias=bias)
    kw = {}
    if r:
        A, B = lora(n, k, r)
        lin.lora = rt.Lora(r, 2.0 * r, A, B)
        kw = dict(A=A, B=B, alpha=2.0 * r)
    y = lin.forward(x, t)
    want = O.linear_forward(wtype, blocks, n, k, x, bias=bias, nthreads=8, **kw)
    assert rel_err(y, want) <= TOL


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
def test_forward_mm_selected_by_grid_size(ctx, wtype):
    # 4096 rows x 1024 tokens: 32 x 8 tiles of 128 x 128, a workgroup per CU, so the default
    # context picks rtq_mm_* by itself
    n, k, t = 4096, 256, 1024
    blocks, x, _ = make(wtype, n, k, t)
    w = hip(ctx, wtype, blocks, n, k)
    y = w.forward(x, t)
    assert rel_err(y, O.frozen_forward(wtype, blocks, n, k, x, nthreads=8)) <= TOL


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
@pytest.mark.parametrize("r", [0, 48])
def test_forward_mm32_selected_by_grid_size(ctx, wtype, r):
    # the fused q|k|v shape of the configs[2] step: 4096 rows x 512 tokens is 128 tiles of 128 x
    # 128 (half the CUs) but 256 of 128 x 64, so the default context picks the 128 x 32 tiles
    # (rtq_mm32_*, two workgroups per CU)
    n, k, t = 4096, 1024, 512
    blocks, x, _ = make(wtype, n, k, t)
    lin = rt.Linear("blk.0.attn_qkv", hip(ctx, wtype, blocks, n, k))
    kw = {}
    if r:
        A, B = lora(n, k, r)
        lin.lora = rt.Lora(r, 2.0 * r, A, B)
        kw = dict(A=A, B=B, alpha=2.0 * r)
    ctx.set_timing(True)
    ctx.reset_timing()
    y = lin.forward(x, t)
    ran = ctx.timing()
    ctx.set_timing(False)
    assert any(name.startswith("rtq_mm32_") for name in ran), ran
    want = O.linear_forward(wtype, blocks, n, k, x, nthreads=16, **kw)
    assert rel_err(y, want) <= TOL


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
@pytest.mark.parametrize("r", [0, 16, 80])
def test_forward_mm_many_tiles(ctx, wtype, r):
    # 64 row blocks x 10 token blocks = 640 workgroups, more than two per CU; LoRA staged in LDS
    # (r = 16) or read from global memory (r = 80); T = 1250 pads the last token block
    n, k, t = 8192, 256, 1250
    blocks, x, _ = make(wtype, n, k, t)
    bias = O.Rng(6).vec_normal(n, 0.1)
    lin = rt.Linear("blk.0.ffn_up", hip(ctx, wtype, blocks, n, k), bias=bias)
    kw = {}
    if r:
        A, B = lora(n, k, r)
        lin.lora = rt.Lora(r, 2.0 * r, A, B)
        kw = dict(A=A, B=B, alpha=2.0 * r)
    y = lin.forward(x, t)
    want = O.linear_forward(wtype, blocks, n, k, x, bias=bias, nthreads=8, **kw)
    assert rel_err(y, want) <= TOL


# ---------------------------------------------------------------- int8-MFMA forward (rtq_mmi8_*)
def _context(env):
    import os

    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        return rt.Context(0)
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


@pytest.fixture(scope="module")
def ctx_i8_pair():
    """Two contexts forcing the 128 x 64 tiles (RTQ_FWD_MM=2): one on the f16 MFMA kernels
    (rtq_mm64_*), one on their int8-MFMA variants for both formats (RTQ_FWD_I8=1, rtq_mmi8_64_*)"""
    f16 = _context({"RTQ_FWD_MM": "2", "RTQ_FWD_I8": "0"})
    i8 = _context({"RTQ_FWD_MM": "2", "RTQ_FWD_I8": "1"})
    yield f16, i8
    i8.close()
    f16.close()


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
@pytest.mark.parametrize("n,k,t,r", [(200, 256, 130, 16), (320, 512, 256, 0), (1000, 1024, 300, 80), (130, 128, 129, 16),
                                     (64, 128, 17, 4), (4096, 1024, 512, 64)])
def test_linear_forward_int8_mfma_matches_oracle(ctx_i8_pair, wtype, n, k, t, r):
    """Forward with the block sums on v_mfma_i32_32x32x32_i8: against the oracle (1e-3), and
    against the f16-MFMA kernel of the same tiles - the integer block sums, scale products and the
    epilogue's FMA order are the same, so without an adapter y is bit-identical; with one, the
    LoRA up-projection sums its ranks in another MFMA shape (f32 rounding)"""
    c16, c8 = ctx_i8_pair
    blocks, x, _ = make(wtype, n, k, t)
    bias = O.Rng(6).vec_normal(n, 0.1)
    out = []
    for c in (c16, c8):
        lin = rt.Linear("blk.0.attn_q", hip(c, wtype, blocks, n, k), bias=bias)
        if r:
            A, B = lora(n, k, r)
            lin.lora = rt.Lora(r, 2.0 * r, A, B)
        c.set_timing(True)
        c.reset_timing()
        out.append(lin.forward(x, t))
        ran = c.timing()
        c.set_timing(False)
        assert any(name.startswith("rtq_mmi8") == (c is c8) and name.startswith("rtq_mm") for name in ran), ran
    kw = dict(A=A, B=B, alpha=2.0 * r) if r else {}
    want = O.linear_forward(wtype, blocks, n, k, x, bias=bias, nthreads=8, **kw)
    assert rel_err(out[1], want) <= TOL
    if r == 0:
        np.testing.assert_array_equal(out[1], out[0])
    else:
        assert rel_err(out[1], out[0]) <= 1e-6


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
def test_frozen_forward_int8_mfma_block_sums_bit_identical(ctx_i8_pair, wtype):
    """FrozenMatmul::forward of the LM-head-like shape 8192 x 1024 at T = 384 (several token blocks,
    padding in the last): the int8 and f16 kernels return the same bits"""
    c16, c8 = ctx_i8_pair
    n, k, t = 8192, 1024, 384
    blocks, x, _ = make(wtype, n, k, t)
    y16 = hip(c16, wtype, blocks, n, k).forward(x, t)
    y8 = hip(c8, wtype, blocks, n, k).forward(x, t)
    np.testing.assert_array_equal(y8, y16)
    assert rel_err(y8, O.frozen_forward(wtype, blocks, n, k, x, nthreads=16)) <= TOL


def test_forward_int8_mfma_is_the_q8_0_default(ctx):
    """the default context runs a Q8_0 weight's large-grid forward on int8 MFMA (the 128 x 128 choice
    taken as 128 x 64 int8 tiles) and a Q4_0 weight's on the f16 kernel"""
    n, k, t = 4096, 256, 1024
    for wtype, prefix in ((O.Q8_0, "rtq_mmi8_64_q8_0"), (O.Q4_0, "rtq_mm_q4_0")):
        blocks, x, _ = make(wtype, n, k, t)
        w = hip(ctx, wtype, blocks, n, k)
        ctx.set_timing(True)
        ctx.reset_timing()
        y = w.forward(x, t)
        ran = ctx.timing()
        ctx.set_timing(False)
        assert prefix in ran, ran
        assert rel_err(y, O.frozen_forward(wtype, blocks, n, k, x, nthreads=8)) <= TOL


# ---------------------------------------------------------------- K-quant LDS-ring forward (rtq_mmk*)
@pytest.fixture(scope="module", params=["1", "2"], ids=["mmk64", "mmk32"])
def ctx_mmk(request):
    """A context that sends every wide K-quant forward through the LDS-ring kernel's 64-token
    (RTQ_FWD_MMK=1) or 32-token (2) tiles"""
    c = _context({"RTQ_FWD_MMK": request.param})
    yield c
    c.close()


@pytest.mark.parametrize("wtype", [O.Q4_K, O.Q6_K])
@pytest.mark.parametrize("n,k,t,r", [(200, 256, 130, 16), (320, 512, 256, 0), (1000, 1024, 300, 80), (130, 256, 129, 16),
                                     (64, 512, 17, 4), (2560, 2560, 192, 16)])
def test_linear_forward_kquant_ring_matches_oracle(ctx_mmk, wtype, n, k, t, r):
    """K-quant forward on the LDS-ring kernel (super-block sums of f16 MFMAs on scale-folded
    fragments, one f32 epilogue per super-block): partial row groups and blocks, token padding,
    no LoRA, LoRA above the LDS staging limit (80), the configs[3] o_proj-like shape"""
    blocks, x, _ = make(wtype, n, k, t)
    bias = O.Rng(6).vec_normal(n, 0.1)
    lin = rt.Linear("blk.0.attn_q", hip(ctx_mmk, wtype, blocks, n, k), bias=bias)
    kw = {}
    if r:
        A, B = lora(n, k, r)
        lin.lora = rt.Lora(r, 2.0 * r, A, B)
        kw = dict(A=A, B=B, alpha=2.0 * r)
    ctx_mmk.set_timing(True)
    ctx_mmk.reset_timing()
    y = lin.forward(x, t)
    ran = ctx_mmk.timing()
    ctx_mmk.set_timing(False)
    assert any(name.startswith("rtq_mmk") for name in ran), ran
    want = O.linear_forward(wtype, blocks, n, k, x, bias=bias, nthreads=8, **kw)
    assert rel_err(y, want) <= TOL


@pytest.mark.parametrize("wtype", [O.Q4_K, O.Q6_K])
def test_forward_kquant_ring_selected_and_equal_to_tile_kernel(ctx, wtype):
    """at 6144 x 2560 and 1024 tokens the default context picks the ring kernel by itself; its
    super-block sums are the tile kernel's (RTQ_FWD_MMK=0), so y agrees to f32 rounding of the same
    per-super-block epilogue (bitwise where the sums are exact)"""
    n, k, t = 6144, 2560, 1024
    blocks, x, _ = make(wtype, n, k, t)
    ctx.set_timing(True)
    ctx.reset_timing()
    y = hip(ctx, wtype, blocks, n, k).forward(x, t)
    ran = ctx.timing()
    ctx.set_timing(False)
    assert any(name.startswith("rtq_mmk64") for name in ran), ran
    c0 = _context({"RTQ_FWD_MMK": "0"})
    y0 = hip(c0, wtype, blocks, n, k).forward(x, t)
    c0.close()
    assert rel_err(y, y0) <= 1e-6
    assert rel_err(y, O.frozen_forward(wtype, blocks, n, k, x, nthreads=16)) <= TOL


# ---------------------------------------------------------------- eight-wave forward, 32- and 16-row tiles
@pytest.fixture(scope="module", params=[1, 2])
def ctx_rg(request):
    """A context that sends every eight-wave Q4_0 / Q8_0 forward through its 16- or 32-row-tile
    variant (RTQ_FWD_RG=1 / 2) and never through rtq_mm_* (RTQ_FWD_MM=0), so small shapes cover its
    padding."""
    c = _context({"RTQ_FWD_RG": str(request.param), "RTQ_FWD_MM": "0"})
    yield request.param, c
    c.close()


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
@pytest.mark.parametrize("n,k,t,r", [(200, 256, 130, 16), (1000, 1024, 300, 80), (130, 128, 17, 4), (1024, 2048, 512, 16)])
def test_linear_forward_rg_matches_oracle(ctx_rg, wtype, n, k, t, r):
    # partial 16- / 32-row tiles (N = 130, 200, 1000), token padding, LoRA ranks 4 / 16 / 80, the
    # o_proj shape of the configs[2] step
    rg, c = ctx_rg
    blocks, x, _ = make(wtype, n, k, t)
    bias = O.Rng(6).vec_normal(n, 0.1)
    lin = rt.Linear("blk.0.attn_output", hip(c, wtype, blocks, n, k), bias=bias)
    A, B = lora(n, k, r)
    lin.lora = rt.Lora(r, 2.0 * r, A, B)
    y, ran = _ran(c, lambda: lin.forward(x, t))
    assert any(name.endswith(f"_w8r{rg}") for name in ran), ran
    want = O.linear_forward(wtype, blocks, n, k, x, bias=bias, A=A, B=B, alpha=2.0 * r, nthreads=16)
    assert rel_err(y, want) <= TOL


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
def test_forward_rg1_selected_by_grid_size(ctx, wtype):
    # the kv_proj shape of configs[1] at 256 tokens: 64 row groups x 4 token tiles is 128 tiles of
    # 32 rows (fewer than the CUs) but 256 of 16, so the default context picks the 16-row tiles
    n, k, t = 1024, 1024, 256
    blocks, x, _ = make(wtype, n, k, t)
    w = hip(ctx, wtype, blocks, n, k)
    y, ran = _ran(ctx, lambda: w.forward(x, t))
    assert any(name.endswith("_w8r1") for name in ran), ran
    assert rel_err(y, O.frozen_forward(wtype, blocks, n, k, x, nthreads=16)) <= TOL


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
def test_forward_rg2_selected_by_grid_size(ctx, wtype):
    # the down_proj shape of the configs[2] step: 64 row groups x 8 token tiles is 176 tiles of 48
    # rows (fewer than the CUs) but 256 of 32, so the default context picks the 32-row tiles
    n, k, t = 1024, 3072, 512
    blocks, x, _ = make(wtype, n, k, t)
    w = hip(ctx, wtype, blocks, n, k)
    ctx.set_timing(True)
    ctx.reset_timing()
    y = w.forward(x, t)
    ran = ctx.timing()
    ctx.set_timing(False)
    assert any(name.endswith("_w8r2") for name in ran), ran
    assert rel_err(y, O.frozen_forward(wtype, blocks, n, k, x, nthreads=16)) <= TOL


# ---------------------------------------------------------------- dx with 256-token tiles (rtq_dxw_*)
@pytest.fixture(scope="module")
def ctx_dxw():
    """A context that sends every t > 16 dx through the 256-token-tile kernel (RTQ_DX_WIDE=1), so
    small shapes cover its token padding and partial-layout mapping."""
    import os

    old = os.environ.get("RTQ_DX_WIDE")
    os.environ["RTQ_DX_WIDE"] = "1"
    try:
        c = rt.Context(0)
    finally:
        if old is None:
            del os.environ["RTQ_DX_WIDE"]
        else:
            os.environ["RTQ_DX_WIDE"] = old
    yield c
    c.close()


@pytest.fixture(scope="module")
def ctx_dx32():
    """A context that sends every t > 16 dx through the 32-token-tile kernel (RTQ_DX_32=1,
    rtq_dx32_*, four-wave workgroups writing the 64-token kernel's partial layout)."""
    c = _context({"RTQ_DX_32": "1"})
    yield c
    c.close()


@pytest.mark.parametrize("which", ["ctx_dxw", "ctx_dx32"])
@pytest.mark.parametrize("wtype,n,k,t", cases([(256, 512, 37), (100, 256, 300), (80, 2048, 130), (3072, 1024, 256),
                                               (1024, 3072, 64), (512, 1024, 20)]))
def test_backward_input_dxw_matches_oracle(request, which, wtype, n, k, t):
    # the 256- and 32-token-tile dx kernels: token padding inside a tile (37, 130, 20: half of a
    # 64-token fragment never written by the 32-token kernel), ragged N, several splits
    c = request.getfixturevalue(which)
    blocks, _, dy = make(wtype, n, k, t)
    w = hip(c, wtype, blocks, n, k)
    dx0 = O.Rng(7).vec_normal(t * k, 1.0)
    dx = dx0.copy()
    w.backward_input(dy, t, dx)
    want = O.frozen_backward_input(wtype, blocks, n, k, dy, dx=np.zeros((t, k), np.float32), nthreads=8)
    assert rel_err(dx - dx0, want) <= TOL
    W = np.stack([O.frozen_row(wtype, blocks, n, k, r) for r in range(n)]).astype(np.float64)
    dense = dy.astype(np.float64) @ W
    got = (dx - dx0).reshape(t, k)
    assert (np.abs(got - dense) < 1e-3 * np.maximum(np.abs(dense), 1.0)).all()


def _dense(wtype, blocks, n, k):
    return np.stack([O.frozen_row(wtype, blocks, n, k, r) for r in range(n)]).astype(np.float64)


@pytest.mark.parametrize("which", ["ctx", "ctx_dxw", "ctx_dx32"])
@pytest.mark.parametrize("wtype", FORMATS)
@pytest.mark.parametrize("t", [1, 7, 16, 64, 300])
def test_backward_input_precision(request, which, wtype, t):
    """dx on f16 hi / lo operands with each dy row scaled into the f16 range (t <= 16: rtq_dx16_*,
    its scale per token from the split's rows; t > 16: rtq_dx_* / rtq_dxw_*, from the row maxima of
    256-row slices): every row within 2e-6 of the f64 product of the dequantised weight, relative to
    the row's largest |dx|, for rows of magnitudes 1e-6, 1 and 1e3 and a zero row (the reference's
    f32 axpy, src/rie.rs:99-107, is good to about 1e-7 here).  A lost lo part (error near 2^-11),
    bf16-level splits (2^-16) or one scale for all rows (rows 1e9 below the largest in f16
    subnormals) fail it."""
    c = request.getfixturevalue(which)
    n, k = 1024, 512
    blocks, _, dy = make(wtype, n, k, t)
    dy = dy.copy()
    dy[0::3] *= np.float32(1e-6)
    dy[1::3] *= np.float32(1e3)
    if t > 5:
        dy[5] = 0.0
    w = hip(c, wtype, blocks, n, k)
    dx = np.zeros(t * k, np.float32)
    w.backward_input(dy, t, dx)
    dense = dy.astype(np.float64) @ _dense(wtype, blocks, n, k)
    got = dx.reshape(t, k).astype(np.float64)
    assert t <= 5 or not got[5].any()
    scale = np.maximum(np.abs(dense).max(axis=1, keepdims=True), 1e-300)
    assert (np.abs(got - dense) / scale).max() <= 2e-6


@pytest.mark.parametrize("t", [7, 100])
@pytest.mark.parametrize("wtype,std", [(O.Q4_0, 1e5), (O.Q8_0, 3e5)])
def test_backward_input_huge_weight_scales(ctx, wtype, std, t):
    # fp16 block scales near 1e4: dequantised values far beyond the f16 range, so the dx kernels
    # pre-scale W by a power of two and scale the partials back
    n, k = 256, 512
    w64 = O.Rng(1).vec_normal(n * k, std).reshape(n, k)
    blocks = O.quantize(wtype, w64)
    dy = O.Rng(3).vec_normal(t * n, 1.0).reshape(t, n)
    w = hip(ctx, wtype, blocks, n, k)
    dx = np.zeros(t * k, np.float32)
    w.backward_input(dy, t, dx)
    dense = dy.astype(np.float64) @ _dense(wtype, blocks, n, k)
    assert np.isfinite(dx).all()
    assert rel_err(dx, dense) <= 2e-6


@pytest.mark.parametrize("which", ["ctx_dxw", "ctx_dx32"])
@pytest.mark.parametrize("wtype", FORMATS)
def test_linear_backward_dxw_lora(request, which, wtype):
    n, k, t, r = 512, 1024 if BLOCK[wtype] == 256 else 768, 300, 16
    blocks, x, dy = make(wtype, n, k, t)
    A, B = lora(n, k, r)
    lin = rt.Linear("blk.0.attn_v", hip(request.getfixturevalue(which), wtype, blocks, n, k))
    lin.lora = rt.Lora(r, 32.0, A, B)
    dx = lin.backward(x, dy, t)
    wdx, wga, wgb = O.linear_backward(wtype, blocks, n, k, x, dy, A=A, B=B, alpha=32.0, nthreads=8)
    assert rel_err(dx, wdx) <= TOL
    assert rel_err(lin.lora.ga, wga) <= TOL
    assert rel_err(lin.lora.gb, wgb) <= TOL


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q6_K])
def test_backward_input_dxw_selected_by_grid(ctx, wtype):
    # 4 token groups x 8 K chunks x 8 row splits of 16 steps: the default context picks the
    # 256-token tiles by itself
    n, k, t = 4096, 1024, 1000
    blocks, _, dy = make(wtype, n, k, t)
    w = hip(ctx, wtype, blocks, n, k)
    dx = np.zeros(t * k, np.float32)
    w.backward_input(dy, t, dx)
    assert rel_err(dx, O.frozen_backward_input(wtype, blocks, n, k, dy, nthreads=8)) <= TOL


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q6_K])
@pytest.mark.parametrize("t", [512, 700])
def test_linear_backward_long_token_range(ctx, wtype, t):
    # t >= 512 with LoRA: the 16-wave finish reduces dA / dB over the tokens (t = 700: ragged
    # last wave range)
    n, k, r = 640, 1024, 16
    blocks, x, dy = make(wtype, n, k, t)
    A, B = lora(n, k, r)
    lin = rt.Linear("blk.0.ffn_down", hip(ctx, wtype, blocks, n, k))
    lin.lora = rt.Lora(r, 32.0, A, B)
    ga0 = O.Rng(8).vec_normal(r * k, 0.01)
    gb0 = O.Rng(9).vec_normal(n * r, 0.01)
    lin.lora.ga[...] = ga0
    lin.lora.gb[...] = gb0
    dx = lin.backward(x, dy, t)
    wdx, wga, wgb = O.linear_backward(wtype, blocks, n, k, x, dy, A=A, B=B, alpha=32.0, nthreads=8)
    assert rel_err(dx, wdx) <= TOL
    assert rel_err(lin.lora.ga - ga0, wga) <= TOL
    assert rel_err(lin.lora.gb - gb0, wgb) <= TOL


# ---------------------------------------------------------------- trainer-native FrozenWeight (F32, Q8_0 f32-scale)
def _trainer_weight(ctx, kind, n, k):
    w = O.Rng(1).vec_normal(n * k, 0.02).reshape(n, k)
    if kind == "f32":
        return rt.HipFrozen.f32(w, n, k, ctx=ctx), O.F32, w.astype(np.float32).view(np.uint8)
    return rt.HipFrozen.q8_0(w, n, k, ctx=ctx), O.TQ8_0, O.quantize(O.TQ8_0, w)


@pytest.mark.parametrize("kind", ["f32", "tq8"])
@pytest.mark.parametrize("n,k,t", [(64, 128, 1), (200, 256, 37), (37, 96, 5), (3072, 1024, 256), (1000, 2048, 600)])
def test_trainer_native_frozen_matches_oracle(ctx, kind, n, k, t):
    hw, otype, ob = _trainer_weight(ctx, kind, n, k)
    assert hw.nbytes() == (n * k * 4 if kind == "f32" else n * (k // 32) * 4 + n * k)  # src/frozen.rs:180-185
    x = O.Rng(2).vec_normal(t * k, 1.0).reshape(t, k)
    dy = O.Rng(3).vec_normal(t * n, 1.0).reshape(t, n)
    assert rel_err(hw.forward(x, t), O.frozen_forward(otype, ob, n, k, x, nthreads=8)) <= TOL
    dx0 = O.Rng(7).vec_normal(t * k, 1.0)
    dx = dx0.copy()
    hw.backward_input(dy, t, dx)  # accumulates
    want = O.frozen_backward_input(otype, ob, n, k, dy, nthreads=8)
    assert rel_err(dx - dx0, want) <= TOL
    out = np.empty(k, np.float32)
    for r in (0, n // 2, n - 1):  # row(): copy / 0 + d * q, bit-exact
        hw.row(r, out)
        assert np.array_equal(out, O.frozen_row(otype, ob, n, k, r)), r


@pytest.mark.parametrize("kind", ["f32", "tq8"])
def test_trainer_native_linear_lora_matches_oracle(ctx, kind):
    n, k, t, r = 512, 256, 70, 16
    hw, otype, ob = _trainer_weight(ctx, kind, n, k)
    _, x, dy = make(O.Q4_0, n, k, t)
    A, B = lora(n, k, r)
    bias = O.Rng(6).vec_normal(n, 0.1)
    lin = rt.Linear("blk.0.attn_o", hw, bias=bias)
    lin.lora = rt.Lora(r, 2.0 * r, A, B)
    y = lin.forward(x, t)
    assert rel_err(y, O.linear_forward(otype, ob, n, k, x, bias=bias, A=A, B=B, alpha=2.0 * r, nthreads=8)) <= TOL
    ga0 = O.Rng(8).vec_normal(r * k, 0.01)
    gb0 = O.Rng(9).vec_normal(n * r, 0.01)
    lin.lora.ga[...] = ga0
    lin.lora.gb[...] = gb0
    dx = lin.backward(x, dy, t)
    wdx, wga, wgb = O.linear_backward(otype, ob, n, k, x, dy, A=A, B=B, alpha=2.0 * r, nthreads=8)
    assert rel_err(dx, wdx) <= TOL
    assert rel_err(lin.lora.ga - ga0, wga) <= TOL
    assert rel_err(lin.lora.gb - gb0, wgb) <= TOL


def test_trainer_q8_0_falls_back_to_f32(ctx):
    # FrozenWeight::q8_0 keeps f32 when the row length is not a whole number of blocks
    # (src/frozen.rs:55-57)
    w = O.Rng(1).vec_normal(8 * 40, 0.02).reshape(8, 40)
    hw = rt.HipFrozen.q8_0(w, 8, 40, ctx=ctx)
    assert hw.ggml_type == rt.TYPE_F32 and hw.nbytes() == 8 * 40 * 4
    x = O.Rng(2).vec_normal(3 * 40, 1.0).reshape(3, 40)
    assert rel_err(hw.forward(x, 3), x.astype(np.float64) @ w.T.astype(np.float64)) <= 1e-5


# ---------------------------------------------------------------- one-launch GEMV (t <= 4)
@pytest.fixture(scope="module")
def ctx_no_gemvq():
    """A context without the one-launch GEMV (RTQ_GEMVQ=0): activation kernel + rtq_gemv_* / rtq_fwd_*_s"""
    c = _context({"RTQ_GEMVQ": "0"})
    yield c
    c.close()


def _ran(c, fn):
    c.set_timing(True)
    c.reset_timing()
    out = fn()
    names = c.timing()
    c.set_timing(False)
    return out, names


@pytest.mark.parametrize("r", [0, 16])
@pytest.mark.parametrize("wtype,n,k,t", cases([(64, 128, 1), (100, 96, 3), (2048, 1024, 1), (1024, 3072, 4),
                                               (300, 512, 2), (1000, 256, 4), (4100, 768, 1)]))
def test_gemvq_matches_oracle(ctx, wtype, n, k, t, r):
    """rtq_gemvq*_* (t <= 4: activation codes formed in the kernel, integer block sums by
    v_dot4_i32_i8) against the oracle: ragged N (100, 300, 1000, 4100 rows), K padded to a chunk
    (96, 768), a bias, tokens 2 and 3 of the four-token kernel.  With a LoRA (r=16) the forward
    takes the two-launch path (h = x A^T formed once, not in every workgroup): checked against
    the oracle too"""
    blocks, x, _ = make(wtype, n, k, t)
    bias = O.Rng(6).vec_normal(n, 0.1)
    lin = rt.Linear("blk.0.attn_q", hip(ctx, wtype, blocks, n, k), bias=bias)
    if r:
        A, B = lora(n, k, r)
        lin.lora = rt.Lora(r, 2.0 * r, A, B)
    y, names = _ran(ctx, lambda: lin.forward(x, t))
    if r:
        assert names and not any(nm.startswith("rtq_gemvq") for nm in names), names
    else:
        assert names and all(nm.startswith("rtq_gemvq") for nm in names), names
    kw = dict(A=A, B=B, alpha=2.0 * r) if r else {}
    want = O.linear_forward(wtype, blocks, n, k, x, bias=bias, nthreads=8, **kw)
    assert rel_err(y, want) <= TOL


@pytest.mark.parametrize("wtype", FORMATS)
@pytest.mark.parametrize("t", [1, 3, 4])
def test_gemvq_against_mfma_gemv(ctx, ctx_no_gemvq, wtype, t):
    """The one-launch kernel against the MFMA GEMV (rtq_gemv_*: the same activation codes and
    exact integer sums), on a weight tall enough for the MFMA GEMV to run without splitting K
    (131072 rows: its split adds chunk partials with atomics).  K-quants without an adapter: the
    same bits (the same super-block sums and epilogue operations); Q4_0 / Q8_0 (k-group shares
    scaled before they are added): within 1e-6; with a LoRA both contexts take the two-launch
    path"""
    n, k = 131072, 256
    blocks, x, _ = make(wtype, n, k, t)
    outs = []
    for c, pre in ((ctx, "rtq_gemvq"), (ctx_no_gemvq, "rtq_gemv_")):
        lin = rt.Linear("output", hip(c, wtype, blocks, n, k))
        y, names = _ran(c, lambda: lin.forward(x, t))
        assert any(nm.startswith(pre) for nm in names), names
        A, B = lora(n, k, 16)
        lin.lora = rt.Lora(16, 32.0, A, B)
        outs.append((y, lin.forward(x, t)))
    if BLOCK[wtype] == 256:
        np.testing.assert_array_equal(outs[0][0], outs[1][0])
    else:
        assert rel_err(outs[0][0], outs[1][0]) <= 1e-6
    assert rel_err(outs[0][1], outs[1][1]) <= 1e-6
    assert rel_err(outs[0][0], O.frozen_forward(wtype, blocks, n, k, x, nthreads=16)) <= TOL


@pytest.mark.parametrize("wtype", FORMATS)
def test_gemvq_lm_head_t1(ctx, wtype):
    """The LM head shape at t = 1 (151936 x 1024): tiles spread over every CU, several per wave"""
    n, k, t = 151936, 1024, 1
    blocks, x, _ = make(wtype, n, k, t)
    w = hip(ctx, wtype, blocks, n, k)
    y, names = _ran(ctx, lambda: w.forward(x, t))
    assert all(nm.startswith("rtq_gemvq1") for nm in names), names
    assert rel_err(y, O.frozen_forward(wtype, blocks, n, k, x, nthreads=16)) <= TOL


# ---------------------------------------------------------------- t = 1 dx on f32 FMAs
@pytest.mark.parametrize("wtype,n,k", cases([(64, 128), (100, 96), (2048, 1024), (1000, 256), (4100, 768),
                                             (151936, 1024)]))
def test_dxv1_matches_oracle(ctx, wtype, n, k):
    """rtq_dxv1_* (t = 1: codes as exact f16 values into f32 mixed-precision FMAs, k-group rows
    added by DPP steps): against the oracle and, per element, the dense dy . W (1e-6 of the largest
    |dx|); ragged N, K padded to a chunk, the LM head shape"""
    blocks, _, dy = make(wtype, n, k, 1)
    w = hip(ctx, wtype, blocks, n, k)
    dx = np.zeros(k, np.float32)
    _, names = _ran(ctx, lambda: w.backward_input(dy, 1, dx))
    assert any(nm.startswith("rtq_dxv1") for nm in names), names
    if n >= 4100:  # 33 and 128 row splits: the workgroup-per-(token, 64 columns) finish
        assert "rtq_bwd_finish_rows" in names, names
    want = O.frozen_backward_input(wtype, blocks, n, k, dy, dx=np.zeros((1, k), np.float32), nthreads=16)
    assert rel_err(dx, want) <= TOL
    if n <= 4100:
        dense = dy.astype(np.float64) @ _dense(wtype, blocks, n, k)
        assert np.abs(dx - dense.reshape(-1)).max() <= 1e-6 * np.abs(dense).max()
    # accumulation onto a non-zero dx: one f32 add of the same sum, bit for bit
    dx0 = O.Rng(7).vec_normal(k, 1.0).astype(np.float32)
    acc = dx0.copy()
    w.backward_input(dy, 1, acc)
    assert np.array_equal(acc, dx0 + dx)


@pytest.mark.parametrize("wtype", FORMATS)
def test_dxv1_lora_backward(ctx, wtype):
    """Linear::backward at t = 1 through rtq_dxv1_* with LoRA r=16 (g . A added by the finish)"""
    n, k, r = 512, 1024 if BLOCK[wtype] == 256 else 768, 16
    blocks, x, dy = make(wtype, n, k, 1)
    A, B = lora(n, k, r)
    lin = rt.Linear("blk.0.attn_v", hip(ctx, wtype, blocks, n, k))
    lin.lora = rt.Lora(r, 2.0 * r, A, B)
    dx = lin.backward(x, dy, 1)
    wdx, wga, wgb = O.linear_backward(wtype, blocks, n, k, x, dy, A=A, B=B, alpha=2.0 * r, nthreads=8)
    assert rel_err(dx, wdx) <= TOL
    assert rel_err(lin.lora.ga, wga) <= TOL
    assert rel_err(lin.lora.gb, wgb) <= TOL


@pytest.mark.parametrize("t", [1, 5, 16])
@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
def test_many_split_finish_ragged_columns(ctx, wtype, t):
    """FrozenMatmul::backward_input at T <= 16 over 8192 rows and K = 160 (two and a half 64-column
    segments): 64 row splits, summed by the workgroup-per-(token, 64 columns) finish with its last
    segment half outside K; accumulated onto a non-zero dx, against the oracle and the dense dy . W"""
    n, k = 8192, 160
    blocks, _, dy = make(wtype, n, k, t)
    w = hip(ctx, wtype, blocks, n, k)
    dx0 = O.Rng(7).vec_normal(t * k, 1.0).astype(np.float32)
    dx = dx0.copy()
    _, names = _ran(ctx, lambda: w.backward_input(dy, t, dx))
    assert "rtq_bwd_finish_rows" in names, names
    want = O.frozen_backward_input(wtype, blocks, n, k, dy, dx=np.zeros((t, k), np.float32), nthreads=16)
    assert rel_err(dx - dx0, want) <= TOL
    _dense_dx_check(wtype, blocks, n, k, dy, (dx - dx0).astype(np.float32))


# ---------------------------------------------------------------- g partials: 64 / 32 / 16 tokens per workgroup
@pytest.fixture(scope="module", params=[16, 32, 64])
def ctx_gtok(request):
    """A context whose LoRA g partials (g = s dy.B per 256-row slice) run on one workgroup form
    (RTQ_GTOK): 64 tokens (a wave per 16 tokens), 32 (two waves per 16 tokens, 128 rows each, summed
    through LDS) or 16 (four waves per 64 rows)"""
    c = _context({"RTQ_GTOK": str(request.param)})
    yield request.param, c
    c.close()


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q6_K])
@pytest.mark.parametrize("t,r", [(100, 48), (512, 16), (45, 40)])
def test_g_partial_forms_match_oracle(ctx_gtok, wtype, t, r):
    """Linear::backward with LoRA on each g-partial form against the oracle: ragged tokens (45, 100),
    rank tiles 1-3 with a ragged last one (r = 40), a ragged last slice of B (N = 1000)"""
    gtok, c = ctx_gtok
    n, k = 1000, 512 if BLOCK[wtype] == 256 else 384
    if BLOCK[wtype] == 256:
        n = 1024
    blocks, x, dy = make(wtype, n, k, t)
    A, B = lora(n, k, r)
    lin = rt.Linear("blk.0.attn_q", hip(c, wtype, blocks, n, k))
    lin.lora = rt.Lora(r, 2.0 * r, A, B)
    dx = lin.backward(x, dy, t)
    wdx, wga, wgb = O.linear_backward(wtype, blocks, n, k, x, dy, A=A, B=B, alpha=2.0 * r, nthreads=8)
    assert rel_err(dx, wdx) <= TOL, gtok
    assert rel_err(lin.lora.ga, wga) <= TOL, gtok
    assert rel_err(lin.lora.gb, wgb) <= TOL, gtok
