"""rtq_linear_forward_noalloc_d: the Linear forward that allocates nothing (its workspace is the
library's file-scope device array) against rtq_linear_forward_d on the same inputs.

* three calls in a row on one fresh context, each smaller than or different from the one before
  (config 1 with LoRA and bias; the same weight at 37 tokens without LoRA; a Q6_K weight at 5
  tokens, the skinny path), so stale scratch contents from the previous call must not leak in:
  every output equals the allocating entry point's within 1e-5 (the kernels are the same);
* the device's free memory does not move across the no-allocation calls;
* a forward whose workspace exceeds the array is refused before any launch, naming the maximum;
* trainer-native (F32, TQ8_0) weights allocate nothing either and give the allocating path's output.
"""
import ctypes

import numpy as np
import pytest

import oracle as O
import rust_trainer_amd as rt
from rust_trainer_amd import _ffi

pytestmark = pytest.mark.gpu


def rel(a, b):
    a, b = np.asarray(a, np.float64).ravel(), np.asarray(b, np.float64).ravel()
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def weight(ctx, wtype, n, k, seed):
    blocks = O.quantize(wtype, O.Rng(seed).vec_normal(n * k, 0.02).reshape(n, k))
    return rt.HipFrozen(wtype, blocks, n, k, ctx=ctx)


def test_noalloc_forward_matches_allocating_forward():
    import torch

    dev = torch.device("cuda", 0)
    ctx = rt.Context(0)  # fresh: no workspace allocated yet
    cases = []
    w1 = weight(ctx, O.Q4_0, 3072, 1024, 1)
    w2 = weight(ctx, O.Q6_K, 512, 1024, 2)
    for w, n, k, t, r, bias in ((w1, 3072, 1024, 256, 16, True), (w1, 3072, 1024, 37, 0, False),
                                (w2, 512, 1024, 5, 8, True)):
        x = torch.from_numpy(O.Rng(10 + t).vec_normal(t * k, 1.0).reshape(t, k)).to(dev)
        A = torch.from_numpy(O.Rng(20 + t).vec_normal(max(r, 1) * k, 1.0 / 32).reshape(max(r, 1), k)).to(dev)
        B = torch.from_numpy(O.Rng(30 + t).vec_normal(n * max(r, 1), 0.01).reshape(n, max(r, 1))).to(dev)
        b = torch.from_numpy(O.Rng(40 + t).vec_normal(n, 0.1)).to(dev) if bias else None
        y_na = torch.full((t, n), float("nan"), device=dev)
        y_ref = torch.empty(t, n, device=dev)
        lv = _ffi.RtqLora(r, 2.0 * r, A.data_ptr(), B.data_ptr(), 1) if r else None
        cases.append((w, t, x, b, lv, y_na, y_ref))
    stream = torch.cuda.current_stream().cuda_stream
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info(0)[0]
    for w, t, x, b, lv, y_na, _ in cases:
        print(f"[no-alloc] {w.out_dim()}x{w.in_dim()} t={t} lora={'yes' if lv else 'no'}", flush=True)
        _ffi.check(_ffi.lib().rtq_linear_forward_noalloc_d(ctx.handle, w.handle, b.data_ptr() if b is not None else None,
                                                           ctypes.byref(lv) if lv else None, x.data_ptr(), t,
                                                           y_na.data_ptr(), stream), "rtq_linear_forward_noalloc_d")
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(0)[0] == free0, "the no-allocation forward changed the device's free memory"
    for w, t, x, b, lv, y_na, y_ref in cases:
        _ffi.check(_ffi.lib().rtq_linear_forward_d(ctx.handle, w.handle, b.data_ptr() if b is not None else None,
                                                   ctypes.byref(lv) if lv else None, x.data_ptr(), t,
                                                   y_ref.data_ptr(), stream), "rtq_linear_forward_d")
    torch.cuda.synchronize()
    for w, t, x, b, lv, y_na, y_ref in cases:
        got, want = y_na.cpu().numpy(), y_ref.cpu().numpy()
        assert np.isfinite(got).all()
        assert rel(got, want) <= 1e-5, (w.out_dim(), t)
    # and once more, the second call smaller than the first, after the allocating calls
    w, t, x, b, lv, y_na, y_ref = cases[1]
    y_na.fill_(float("nan"))
    _ffi.check(_ffi.lib().rtq_linear_forward_noalloc_d(ctx.handle, w.handle, None, None, x.data_ptr(), t,
                                                       y_na.data_ptr(), stream), "rtq_linear_forward_noalloc_d")
    torch.cuda.synchronize()
    assert rel(y_na.cpu().numpy(), y_ref.cpu().numpy()) <= 1e-5
    ctx.close()


def test_noalloc_forward_refuses_what_it_cannot_serve():
    import torch

    dev = torch.device("cuda", 0)
    ctx = rt.Context(0)
    n, k, t = 64, 8192, 4096  # the activation fragments alone take t * k * 2 = 64 MiB
    w = weight(ctx, O.Q4_0, n, k, 3)
    x = torch.zeros(t, k, device=dev)
    y = torch.full((t, n), 5.0, device=dev)
    rc = _ffi.lib().rtq_linear_forward_noalloc_d(ctx.handle, w.handle, None, None, x.data_ptr(), t, y.data_ptr(), None)
    assert rc == 1 and b"maximum" in _ffi.lib().rtq_last_error()
    torch.cuda.synchronize()
    assert bool((y == 5.0).all()), "a refused call wrote its output"
    # trainer-native weights run on the f32 GEMM and allocate nothing either: same output as the
    # allocating entry point
    stream = torch.cuda.current_stream().cuda_stream
    for wf in (rt.HipFrozen.f32(O.Rng(5).vec_normal(96 * 256, 0.02), 96, 256, ctx=ctx),
               rt.HipFrozen.q8_0(O.Rng(6).vec_normal(96 * 256, 0.02), 96, 256, ctx=ctx)):
        xs = torch.from_numpy(O.Rng(7).vec_normal(9 * 256, 1.0).reshape(9, 256)).to(dev)
        y1, y2 = torch.empty(9, 96, device=dev), torch.empty(9, 96, device=dev)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info(0)[0]
        _ffi.check(_ffi.lib().rtq_linear_forward_noalloc_d(ctx.handle, wf.handle, None, None, xs.data_ptr(), 9,
                                                           y1.data_ptr(), stream), "rtq_linear_forward_noalloc_d")
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info(0)[0] == free0
        _ffi.check(_ffi.lib().rtq_linear_forward_d(ctx.handle, wf.handle, None, None, xs.data_ptr(), 9, y2.data_ptr(),
                                                   stream), "rtq_linear_forward_d")
        torch.cuda.synchronize()
        assert torch.equal(y1, y2)
    ctx.close()
