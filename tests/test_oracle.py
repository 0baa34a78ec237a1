"""Pins the CPU oracle (oracle/rtq_oracle.c) before it is trusted as the GPU path's checker.

Every oracle function is checked against something it does not compute itself: committed
known-answer vectors (tests/golden/known_answers.json, written by make_golden.py from the
format definitions), numpy's IEEE half conversion, brute-force integer sums, float64 closed
forms, and the reference's own invariants (tests/engine.rs:96-120 dense-dequant dx,
src/frozen.rs:218-227 adjoint identity, src/tensor.rs:205-238 matmul layouts agree).
"""
import json
import math
import os

import numpy as np
import pytest

import oracle as O

GOLD = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


# ---------------------------------------------------------------- Rng (src/tensor.rs:155-199)
@pytest.mark.parametrize("seed", ["1", "2", "3", "9"])
def test_rng_matches_splitmix_definition(seed):
    r = O.Rng(int(seed))
    assert [str(r.next_u64()) for _ in range(6)] == GOLD["rng"][seed]["u64"]
    r = O.Rng(int(seed))
    assert [r.uniform() for _ in range(6)] == GOLD["rng"][seed]["uniform"]


def test_rng_normal_is_box_muller():
    # normal() = sqrt(-2 ln u1) cos(2 pi u2) over consecutive uniforms (u1 clamped at 1e-12)
    a, b = O.Rng(11), O.Rng(11)
    for _ in range(200):
        u1 = max(b.uniform(), 1e-12)
        u2 = b.uniform()
        want = math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * math.pi * u2)
        assert abs(a.normal() - want) < 1e-5 * max(1.0, abs(want))
    v = O.Rng(3).vec_normal(200000, 0.02)
    assert abs(v.mean()) < 2e-4 and abs(v.std() - 0.02) < 2e-4


# ---------------------------------------------------------------- IEEE half
def test_fp16_to_fp32_all_halves():
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    ours = np.array([O.fp16_bits_to_fp32(int(x)) for x in h], dtype=np.float32)
    ok = ~np.isnan(ref)
    assert np.array_equal(ours[ok].view(np.uint32), ref[ok].view(np.uint32))
    assert np.isnan(ours[~ok]).all()


def test_fp32_to_fp16_round_to_nearest_even():
    r = np.random.default_rng(0)
    xs = (r.standard_normal(20000) * 10.0 ** r.integers(-9, 5, 20000)).astype(np.float32)
    # exact ties between adjacent halves, subnormal halves, overflow boundary
    ties = np.array([1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 2 ** -24 * 1.5, 2 ** -24 * 2.5, 65504.0, 65519.0, 65520.0,
                     -65520.0, 2 ** -25, 2 ** -26, 0.0, -0.0], dtype=np.float32)
    xs = np.concatenate([xs, ties])
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    ours = np.array([O.fp32_to_fp16_bits(float(x)) for x in xs], dtype=np.uint16)
    assert np.array_equal(ours, ref)


# ---------------------------------------------------------------- block formats
@pytest.mark.parametrize("case", range(len(GOLD["dequant"])))
def test_dequant_known_answers(case):
    c = GOLD["dequant"][case]
    blocks = np.frombuffer(bytes.fromhex(c["blocks"]), dtype=np.uint8)
    got = O.dequantize(c["type"], blocks, c["k"]).reshape(-1)
    assert np.array_equal(got, np.array(c["values"], dtype=np.float32)), O.TYPE_NAMES[c["type"]]


def test_quantiser_known_answers():
    for c in GOLD["quantise"]:
        x = np.array(c["x"], dtype=np.float32)
        if c["kind"] == "q8_0":
            b = O.quantize_acts(O.Q8_0, x[None, :])[0]
            assert int(b[0]) | (int(b[1]) << 8) == c["d_bits"]
            assert b[2:].view(np.int8).tolist() == c["q"]
            # the weight quantiser uses the same reference rule
            w = O.quantize(O.Q8_0, x[None, :])[0]
            assert np.array_equal(w, b)
        elif c["kind"] == "q8_k":
            b = O.quantize_acts(O.Q4_K, x[None, :])[0]
            assert b[:4].view(np.float32)[0] == np.float32(c["d"])
            assert b[4:260].view(np.int8).tolist() == c["q"]
            assert b[260:292].view(np.int16).tolist() == c["bsums"]
        elif c["kind"] == "q4_0":
            b = O.quantize(O.Q4_0, x[None, :])[0]
            assert int(b[0]) | (int(b[1]) << 8) == c["d_bits"]
            codes = [int(b[2 + j]) & 0xF for j in range(16)] + [int(b[2 + j]) >> 4 for j in range(16)]
            assert codes == c["q"]


@pytest.mark.parametrize("wtype,bound", [(O.Q4_0, None), (O.Q8_0, 0.5), (O.Q4_K, None), (O.Q6_K, None)])
def test_quantise_roundtrip(wtype, bound):
    w = O.Rng(1).vec_normal(64 * 512, 0.02).reshape(64, 512)
    b = O.quantize(wtype, w)
    assert b.shape == (64, O.row_bytes(wtype, 512))
    d = O.dequantize(wtype, b, 512)
    err = np.abs(d - w)
    if wtype == O.Q8_0:
        # |x - q d16| <= d/2 + |q| |d - d16| <= d16 (1/2 + 127 * 2^-11) (codes use the unrounded d)
        dd = np.array([O.fp16_bits_to_fp32(int(r[i]) | (int(r[i + 1]) << 8))
                       for r in b for i in range(0, b.shape[1], 34)]).reshape(64, 16)
        assert (err.reshape(64, 16, 32) <= dd[..., None] * (0.5 + 127 * 2 ** -11) * (1 + 2 ** -10)).all()
    rel = np.sqrt((err ** 2).mean()) / 0.02
    assert rel < {O.Q4_0: 0.12, O.Q8_0: 0.01, O.Q4_K: 0.12, O.Q6_K: 0.03}[wtype]


def test_q4_0_quantiser_is_ggml_reference():
    # independent numpy restatement of ggml's quantize_row_q4_0_ref on random blocks
    x = O.Rng(5).vec_normal(40 * 32, 1.0).reshape(40, 32)
    b = O.quantize(O.Q4_0, x.reshape(1, -1))[0].reshape(40, 18)
    for i in range(40):
        blk = x[i]
        j = int(np.argmax(np.abs(blk)))  # first index of the largest |x|
        d = np.float32(blk[j]) / np.float32(-8.0)
        idv = np.float32(1.0) / d if d != 0 else np.float32(0.0)
        codes = [min(15, int(np.float32(v) * idv + np.float32(8.5))) for v in blk]
        got = [int(b[i, 2 + k]) & 0xF for k in range(16)] + [int(b[i, 2 + k]) >> 4 for k in range(16)]
        assert got == codes
        assert int(b[i, 0]) | (int(b[i, 1]) << 8) == int(np.array([d], np.float16).view(np.uint16)[0])


def test_q8_k_acts_numpy_restatement():
    x = O.Rng(6).vec_normal(3 * 256, 1.0).reshape(3, 256)
    b = O.quantize_acts(O.Q6_K, x)
    for i in range(3):
        blk = x[i]
        j = int(np.argmax(np.abs(blk)))
        iscale = np.float32(-127.0) / np.float32(blk[j])
        q = np.minimum(127, np.rint(iscale * blk)).astype(np.int64)  # rint: half to even
        assert b[i, 4:260].view(np.int8).tolist() == q.tolist()
        assert b[i, :4].view(np.float32)[0] == np.float32(1.0) / iscale
        assert b[i, 260:].view(np.int16).tolist() == [int(q[16 * g:16 * g + 16].sum()) for g in range(16)]


# ---------------------------------------------------------------- integer block dots
def test_isum_known_answer():
    c = GOLD["isum_q4_0"]
    w = np.frombuffer(bytes.fromhex(c["w"]), np.uint8)[None, :]
    a = np.frombuffer(bytes.fromhex(c["a"]), np.uint8)[None, :]
    assert O.block_isums(O.Q4_0, w, a, 32)[0, 0, 0] == c["isum"]


def _codes(wtype, blocks, k):
    """Integer codes and per-element integer multipliers from dequantising with unit scales."""
    b = blocks.copy()
    n = b.shape[0]
    if wtype in (O.Q4_0, O.Q8_0):
        bb = 18 if wtype == O.Q4_0 else 34
        for i in range(0, b.shape[1], bb):
            b[:, i:i + 2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        return np.rint(O.dequantize(wtype, b, k)).astype(np.int64).reshape(n, k)
    raise NotImplementedError


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0])
def test_block_isums_brute_force(wtype):
    k, n, t = 128, 5, 3
    w = O.Rng(1).vec_normal(n * k, 0.02).reshape(n, k)
    x = O.Rng(2).vec_normal(t * k, 1.0).reshape(t, k)
    blocks = O.quantize(wtype, w)
    acts = O.quantize_acts(wtype, x)
    isums = O.block_isums(wtype, blocks, acts, k)
    wc = _codes(wtype, blocks, k)
    ac = acts.reshape(t, k // 32, 34)[:, :, 2:].view(np.int8).reshape(t, k).astype(np.int64)
    want = np.einsum("tbk,nbk->tnb", ac.reshape(t, k // 32, 32), wc.reshape(n, k // 32, 32))
    assert np.array_equal(isums, want)


@pytest.mark.parametrize("wtype", [O.Q4_K, O.Q6_K])
def test_kquant_isums_brute_force(wtype):
    k, n, t = 512, 3, 2
    w = O.Rng(1).vec_normal(n * k, 0.02).reshape(n, k)
    x = O.Rng(2).vec_normal(t * k, 1.0).reshape(t, k)
    blocks = O.quantize(wtype, w)
    acts = O.quantize_acts(wtype, x)
    isums = O.block_isums(wtype, blocks, acts, k)
    ac = np.stack([acts[i].reshape(k // 256, 292)[:, 4:260].view(np.int8).reshape(k) for i in range(t)]).astype(
        np.int64)
    bb = O.BLOCK_BYTES[wtype]
    for o in range(n):
        row = blocks[o].reshape(k // 256, bb)
        for sb in range(k // 256):
            blk = row[sb]
            if wtype == O.Q4_K:
                # decode codes, scales and mins from dequant with d = 1, dmin = 0 and d = 0, dmin = 1
                b1 = blk.copy()
                b1[0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
                b1[2:4] = 0
                scq = np.rint(O.dequantize(O.Q4_K, b1, 256)[0]).astype(np.int64)   # sc_j * q
                b2 = blk.copy()
                b2[0:2] = 0
                b2[2:4] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
                mins = -np.rint(O.dequantize(O.Q4_K, b2, 256)[0]).astype(np.int64)  # m_j per element
                for i in range(t):
                    a = ac[i, 256 * sb:256 * sb + 256]
                    s1 = int((scq * a).sum())
                    s2 = int(sum(mins[32 * j] * a[32 * j:32 * j + 32].sum() for j in range(8)))
                    assert isums[i, o, 2 * sb] == s1 and isums[i, o, 2 * sb + 1] == s2
            else:
                b1 = blk.copy()
                b1[208:210] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
                scq = np.rint(O.dequantize(O.Q6_K, b1, 256)[0]).astype(np.int64)   # sc_s * q
                for i in range(t):
                    a = ac[i, 256 * sb:256 * sb + 256]
                    assert isums[i, o, sb] == int((scq * a).sum())


# ---------------------------------------------------------------- FrozenMatmul
FORMATS = [O.Q4_0, O.Q8_0, O.Q4_K, O.Q6_K]


def _setup(wtype, n, k, t, seed=1):
    w = O.Rng(seed).vec_normal(n * k, 0.02).reshape(n, k)
    blocks = O.quantize(wtype, w)
    x = O.Rng(seed + 1).vec_normal(t * k, 1.0).reshape(t, k)
    dy = O.Rng(seed + 2).vec_normal(t * n, 1.0).reshape(t, n)
    return blocks, x, dy


@pytest.mark.parametrize("wtype", FORMATS)
def test_forward_matches_f64_of_same_operands(wtype):
    n, k, t = 48, 512, 5
    blocks, x, _ = _setup(wtype, n, k, t)
    y = O.frozen_forward(wtype, blocks, n, k, x, nthreads=3)
    y64 = O.frozen_forward_f64(wtype, blocks, n, k, x)
    assert np.abs(y - y64).max() <= 1e-5 * np.abs(y64).max()
    # and it is the dense product of dequantised weights and dequantised activations
    deq_w = O.dequantize(wtype, blocks, k).astype(np.float64)
    acts = O.quantize_acts(wtype, x)
    if wtype in (O.Q4_0, O.Q8_0):
        a = acts.reshape(t, k // 32, 34)
        dx = np.array([[O.fp16_bits_to_fp32(int(a[i, b, 0]) | (int(a[i, b, 1]) << 8)) for b in range(k // 32)]
                       for i in range(t)])
        deq_x = (a[:, :, 2:].view(np.int8).astype(np.float64) * dx[..., None]).reshape(t, k)
    else:
        a = acts.reshape(t, k // 256, 292)
        deq_x = (a[:, :, 4:260].view(np.int8).astype(np.float64) *
                 a[:, :, :4].copy().view(np.float32).astype(np.float64)).reshape(t, k)
    assert np.abs(deq_x @ deq_w.T - y64).max() <= 1e-9 * np.abs(y64).max()


@pytest.mark.parametrize("wtype", FORMATS)
def test_backward_input_matches_dense_and_adjoint(wtype):
    # tests/engine.rs:96-120 (dense dy.W from row()) and src/frozen.rs:218-227 (adjoint identity)
    n, k, t = 70, 256, 3
    blocks, x, dy = _setup(wtype, n, k, t)
    W = np.stack([O.frozen_row(wtype, blocks, n, k, r) for r in range(n)]).astype(np.float64)
    dx = O.frozen_backward_input(wtype, blocks, n, k, dy, nthreads=4)
    want = dy.astype(np.float64) @ W
    assert (np.abs(dx - want) < 1e-3 * np.maximum(np.abs(want), 1.0)).all()
    # accumulates into an existing dx
    dx2 = O.frozen_backward_input(wtype, blocks, n, k, dy, dx=np.ones((t, k), np.float32))
    assert np.abs(dx2 - 1.0 - want).max() < 1e-5
    # adjoint with the dequantised weight: <dy, x W^T> == <dy W, x>
    lhs = float((dy.astype(np.float64) * (x.astype(np.float64) @ W.T)).sum())
    rhs = float((dx.astype(np.float64) * x).sum())
    assert abs(lhs - rhs) < 1e-3 * max(abs(lhs), 1.0)


def test_backward_thread_count_only_changes_rounding():
    n, k, t = 200, 256, 4
    blocks, _, dy = _setup(O.Q4_0, n, k, t)
    a = O.frozen_backward_input(O.Q4_0, blocks, n, k, dy, nthreads=1)
    b = O.frozen_backward_input(O.Q4_0, blocks, n, k, dy, nthreads=7)
    assert np.abs(a - b).max() <= 1e-5 * np.abs(a).max()


# ---------------------------------------------------------------- dense primitives + Linear
def test_matmul_layouts_agree():
    # src/tensor.rs:205-238
    r = O.Rng(1)
    m, k, n = 5, 7, 3
    a = r.vec_normal(m * k, 1.0).reshape(m, k)
    b = r.vec_normal(n * k, 1.0).reshape(n, k)
    c = O.matmul_nt(a, b)
    c2 = O.matmul_nn(a, np.ascontiguousarray(b.T))
    assert np.abs(c - c2).max() < 1e-5
    c3 = O.matmul_tn_acc(np.zeros((k, n), np.float32), a, c)
    assert np.abs(c3 - a.T.astype(np.float64) @ c).max() < 1e-4
    assert abs(O.dot(a[0], b[0]) - float(a[0].astype(np.float64) @ b[0])) < 1e-5


def _lora(n, k, r, seed=4):
    A = O.Rng(seed).vec_normal(r * k, 1.0 / 32.0).reshape(r, k)
    B = O.Rng(seed + 1).vec_normal(n * r, 0.01).reshape(n, r)
    return A, B


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q4_K])
def test_linear_closed_forms_f64(wtype):
    n, k, t, r, alpha = 64, 256, 6, 4, 8.0
    blocks, x, dy = _setup(wtype, n, k, t)
    A, B = _lora(n, k, r)
    bias = O.Rng(7).vec_normal(n, 0.1)
    s = alpha / r
    y = O.linear_forward(wtype, blocks, n, k, x, bias=bias, A=A, B=B, alpha=alpha)
    base = O.frozen_forward_f64(wtype, blocks, n, k, x)
    x64, A64, B64, dy64 = (v.astype(np.float64) for v in (x, A, B, dy))
    want = base + bias + s * (x64 @ A64.T) @ B64.T
    assert np.abs(y - want).max() <= 1e-5 * np.abs(want).max()
    # disabled adapter is bypassed (Linear::lora_enabled)
    y0 = O.linear_forward(wtype, blocks, n, k, x, bias=bias, A=A, B=B, alpha=alpha, lora_enabled=False)
    assert np.abs(y0 - (base + bias)).max() <= 1e-5 * np.abs(want).max()
    ga0 = O.Rng(9).vec_normal(r * k, 0.1).reshape(r, k)
    dx, ga, gb = O.linear_backward(wtype, blocks, n, k, x, dy, A=A, B=B, alpha=alpha, ga=ga0)
    W = O.dequantize(wtype, blocks, k).astype(np.float64)
    h = x64 @ A64.T
    g = s * dy64 @ B64
    assert np.abs(dx - (dy64 @ W + g @ A64)).max() <= 1e-5 * np.abs(dy64 @ W).max()
    assert np.abs(ga - (ga0 + g.T @ x64)).max() <= 1e-5 * np.abs(g.T @ x64).max()
    assert np.abs(gb - s * dy64.T @ h).max() <= 1e-5 * np.abs(s * dy64.T @ h).max()


def test_lora_grads_finite_differences():
    # tests/engine.rs:125-183 style: loss = sum(y * c) is linear in B and quadratic-free in A,
    # so central differences are exact up to rounding
    wtype, n, k, t, r, alpha = O.Q8_0, 32, 64, 3, 2, 4.0
    blocks, x, _ = _setup(wtype, n, k, t)
    A, B = _lora(n, k, r)
    c = O.Rng(8).vec_normal(t * n, 1.0).reshape(t, n)
    _, ga, gb = O.linear_backward(wtype, blocks, n, k, x, c, A=A, B=B, alpha=alpha)

    def loss(A_, B_):
        return float((O.linear_forward(wtype, blocks, n, k, x, A=A_, B=B_, alpha=alpha).astype(np.float64) * c).sum())

    rng = np.random.default_rng(0)
    for _ in range(6):
        i, j = rng.integers(0, r), rng.integers(0, k)
        e = 1e-2
        Ap, Am = A.copy(), A.copy()
        Ap[i, j] += e
        Am[i, j] -= e
        num = (loss(Ap, B) - loss(Am, B)) / (2 * e)
        assert abs(num - ga[i, j]) <= 3e-2 * max(abs(num), abs(ga[i, j])) + 2e-3
        o, q = rng.integers(0, n), rng.integers(0, r)
        Bp, Bm = B.copy(), B.copy()
        Bp[o, q] += e
        Bm[o, q] -= e
        num = (loss(A, Bp) - loss(A, Bm)) / (2 * e)
        assert abs(num - gb[o, q]) <= 3e-2 * max(abs(num), abs(gb[o, q])) + 2e-3


def test_oracle_rejects_bad_shapes():
    with pytest.raises(ValueError):
        O.frozen_forward(O.Q4_0, np.zeros((2, 18), np.uint8), 2, 48, np.zeros((1, 48), np.float32))


# ---------------------------------------------------------------- trainer-native FrozenWeight (src/frozen.rs)
def _tq8_views(b, n, k):
    sc = b[: n * (k // 32) * 4].view(np.float32).reshape(n, k // 32)
    qs = b[n * (k // 32) * 4:].view(np.int8).reshape(n, k)
    return sc, qs


def test_tq8_quantiser_known_answers():
    # src/frozen.rs:59-70: d = amax / 127, q = round(x / d) with halves away from zero; amax 127
    # gives d = 1, so x = m + 0.5 must round away from zero
    w = np.zeros((3, 32), np.float32)
    w[0, :8] = [127.0, 2.5, -2.5, 0.5, -0.5, 1.49, -126.5, 3.0]
    w[2, :] = np.float32(1e-30) * np.arange(32, dtype=np.float32)  # tiny but non-zero
    sc, qs = _tq8_views(O.quantize(O.TQ8_0, w), 3, 32)
    assert sc[0, 0] == 1.0 and list(qs[0, :8]) == [127, 3, -3, 1, -1, 1, -127, 3]
    assert sc[1, 0] == 0.0 and not qs[1].any()  # all-zero block: d = 0, id = 0, codes 0
    assert qs[2, 31] == 127 and sc[2, 0] == np.float32(np.float32(31e-30) / np.float32(127.0))


def test_tq8_round_trip_bound():
    n, k = 40, 256
    w = O.Rng(11).vec_normal(n * k, 0.02).reshape(n, k)
    sc, qs = _tq8_views(O.quantize(O.TQ8_0, w), n, k)
    deq = (qs.astype(np.float64).reshape(n, k // 32, 32) * sc[:, :, None]).reshape(n, k)
    assert (np.abs(deq - w) <= sc.repeat(32, axis=1) * 0.5 * (1 + 1e-6)).all()


def test_tq8_forward_backward_row_match_dense_products():
    # q8_dot / q8_axpy / row (src/frozen.rs:80-108,113-177) against float64 products of the
    # dequantised matrix, and the adjoint identity <dy, x W^T> = <dy W, x> (src/frozen.rs:218-227)
    n, k, t = 48, 128, 5
    w = O.Rng(1).vec_normal(n * k, 0.02).reshape(n, k)
    b = O.quantize(O.TQ8_0, w)
    sc, qs = _tq8_views(b, n, k)
    W = (qs.astype(np.float64).reshape(n, k // 32, 32) * sc[:, :, None]).reshape(n, k)
    x = O.Rng(2).vec_normal(t * k, 1.0).reshape(t, k)
    dy = O.Rng(3).vec_normal(t * n, 1.0).reshape(t, n)
    y = O.frozen_forward(O.TQ8_0, b, n, k, x)
    assert np.abs(y - x.astype(np.float64) @ W.T).max() <= 1e-5 * np.abs(x @ W.T).max()
    assert np.allclose(O.frozen_forward_f64(O.TQ8_0, b, n, k, x), x.astype(np.float64) @ W.T, rtol=1e-12, atol=1e-12)
    dx = O.frozen_backward_input(O.TQ8_0, b, n, k, dy)
    assert np.abs(dx - dy.astype(np.float64) @ W).max() <= 1e-5 * np.abs(dy @ W).max()
    assert abs(float((dy * y).sum()) - float((dx * x).sum())) <= 1e-4 * float(np.abs(dy * y).sum())
    for r in (0, 17, n - 1):
        assert np.array_equal(O.frozen_row(O.TQ8_0, b, n, k, r), (np.float32(0) + sc[r].repeat(32) * qs[r].astype(np.float32)))


# ---------------------------------------------------------------- LM head + cross-entropy
def _head_case(wtype, V, d, t, seed=1):
    w = O.Rng(seed).vec_normal(V * d, 0.3).reshape(V, d)
    blocks = O.quantize(wtype, w) if wtype != O.F32 else w.astype(np.float32).view(np.uint8).reshape(V, -1)
    x = O.Rng(seed + 1).vec_normal(t * d, 1.0).reshape(t, d)
    norm = (1.0 + O.Rng(seed + 2).vec_normal(d, 0.1)).astype(np.float32)
    return blocks, x, norm


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0, O.Q6_K])
def test_lm_head_closed_forms_f64(wtype):
    """Model::head (src/model.rs:561-609) against f64 closed forms over the same operands: the
    log-softmax of the oracle's logits, the argmax hits, and dx = rmsnorm_backward(dequant(W)^T
    w (softmax - onehot)) scattered to the target positions (repeated positions add)."""
    V, d, t = 700, 256, 11
    blocks, x, norm = _head_case(wtype, V, d, t)
    pos = np.array([0, 4, 10, 4, 7, 2, 9], np.int32)
    tok = np.array([3, 699, 0, 17, 350, 5, 698], np.int32)
    wts = np.array([1.0, 0.5, 2.0, 1.0, 0.25, 1.5, 1.0], np.float32)
    eps, off = 1e-6, 0.0
    logp, hits, dx = O.lm_head(wtype, blocks, V, d, norm, x, pos, tok, wts, eps=eps, off=off, chunk=3)
    # f64 restatement
    xs = x[pos].astype(np.float64)
    ir = 1.0 / np.sqrt((xs * xs).sum(1) / d + eps)
    ns = (xs * ir[:, None] * (norm.astype(np.float64) + off)).astype(np.float32)
    logits = O.frozen_forward(wtype, blocks, V, d, ns).astype(np.float64)
    m = logits.max(1, keepdims=True)
    lse = (m + np.log(np.exp(logits - m).sum(1, keepdims=True)))[:, 0]
    want = logits[np.arange(pos.size), tok] - lse
    np.testing.assert_allclose(logp, want, rtol=0, atol=2e-5 * np.abs(want).max())
    assert hits == int((logits.argmax(1) == tok).sum())
    p = np.exp(logits - lse[:, None])
    dl = wts[:, None].astype(np.float64) * p
    dl[np.arange(pos.size), tok] -= wts
    Wd = O.dequantize(wtype, blocks, d).astype(np.float64).reshape(V, d)
    dns = dl @ Wd
    g = dns * (norm.astype(np.float64) + off)
    c = (g * xs).sum(1) * ir ** 3 / d
    dxs = g * ir[:, None] - xs * c[:, None]
    want_dx = np.zeros((t, d))
    for i, p_ in enumerate(pos):
        want_dx[p_] += dxs[i]
    assert np.abs(dx - want_dx).max() <= 1e-4 * np.abs(want_dx).max()
    assert not dx[[1, 3, 5, 6, 8]].any()  # rows without targets stay zero
    # without weights: log-probs only, same values
    lp2, h2, dx2 = O.lm_head(wtype, blocks, V, d, norm, x, pos, tok, None, eps=eps, off=off, chunk=64)
    np.testing.assert_array_equal(lp2, logp)
    assert h2 == hits and dx2 is None


def test_lm_head_gradient_finite_differences():
    """dL/dx of L = -sum w_i logp_i by central differences in x (F32 head: no activation
    quantisation, so L is smooth), norm offset 1 as in the zero-centred norm."""
    V, d, t = 60, 32, 4
    blocks, x, norm = _head_case(O.F32, V, d, t, seed=7)
    x = x.astype(np.float64)
    pos = np.array([1, 3, 0], np.int32)
    tok = np.array([2, 59, 30], np.int32)
    wts = np.array([1.0, 0.5, 2.0], np.float32)
    eps, off = 1e-5, 1.0

    def loss(xx):
        lp, _, _ = O.lm_head(O.F32, blocks, V, d, norm, xx.astype(np.float32), pos, tok, None, eps=eps, off=off)
        return -float((wts.astype(np.float64) * lp).sum())

    _, _, dx = O.lm_head(O.F32, blocks, V, d, norm, x.astype(np.float32), pos, tok, wts, eps=eps, off=off)
    h = 1e-2
    rng = np.random.default_rng(0)
    for _ in range(12):
        r, k = int(rng.choice(pos)), int(rng.integers(0, d))
        xp, xm = x.copy(), x.copy()
        xp[r, k] += h
        xm[r, k] -= h
        fd = (loss(xp) - loss(xm)) / (2 * h)
        assert abs(fd - dx[r, k]) <= 2e-2 * max(1.0, abs(fd)), (r, k, fd, dx[r, k])


def test_lm_head_rejects_out_of_range_targets():
    blocks, x, norm = _head_case(O.Q8_0, 64, 32, 3)
    with pytest.raises(Exception):
        O.lm_head(O.Q8_0, blocks, 64, 32, norm, x, [3], [0])
    with pytest.raises(Exception):
        O.lm_head(O.Q8_0, blocks, 64, 32, norm, x, [0], [64])
