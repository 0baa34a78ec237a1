"""Benchmark of the frozen quantised-matmul hot path on one MI355X.

Default workload (the configuration the metric names): one LoRA training
step of a Qwen3-0.6B-shaped synthetic Q4_0 GGUF model (28 layers, hidden 1024, FFN 3072, 16 / 8
heads of 128, QK-norm, NEOX RoPE, vocabulary 151936 tied; random N(0, 0.02) weights, norms 1) with
LoRA r=16 alpha=32 on q, k, v, o, gate, up, down, on 512 uniform-random token ids with cross-entropy
on the last 256 positions.  One step = zero_grad + Model::forward_backward through
rtq_model_forward_backward: 196 frozen-linear calls fused into 112 (q | k | v, gate | up), the
attention and norms around them, the LM head + cross-entropy, and the backward of all of it, every
tensor resident in HBM.  ``value`` = 512 tokens / step time (the reference's tok/s definition,
examples/bench_train.rs:57-61); the K timed steps run back to back between two synchronisations.
``roofline`` is that of the dominant quantised-matmul kernel of the step (its algorithmic bytes and
flops over its event-timed total; see ``step_roofline``), ``cpu_baseline`` the oracle's whole step
(all 28 blocks) on the host cores, threads pinned, median of 3 after a warm-up (see
``model_cpu_baseline``).

``--linear`` measures configs[0] instead: one Qwen3-0.6B gate_proj frozen linear, Q4_0 W 3072x1024
(N(0, 0.02), ggml reference quantiser), X 256x1024 and dy 256x3072 ~ N(0, 1), LoRA r=16 alpha=32
(A ~ N(0, 1/1024), B ~ N(0, 0.01)); seeds 1..5 of the reference Rng.  One step = Linear forward (y)
and Linear backward (dx, dA, dB), device-resident inputs, through the C ABI's device-pointer entry
points on torch's current stream.  Operand sets rotate over >256 MB so neither L2 nor the Infinity
Cache holds a step's inputs.  The timed region is one replay of a HIP graph (torch.cuda.CUDAGraph
over the library's device-pointer calls on one stream) of exactly K steps, with no events inside.
Per-kernel durations come from an eager pass of the same steps with HIP events recorded by the
library around each launch on the launch stream; these intervals include the dispatch of the kernel
packet and so read a few microseconds longer than the kernel-trace durations of rocprofv3.

``--sweep`` measures BASELINE configs[1] instead: Q8_0, Q4_K, Q6_K (and Q4_0) at the Qwen3-0.6B
shapes q_proj 2048x1024, k/v_proj 1024x1024, down_proj 1024x3072 and the tied LM head 151936x1024,
T in {1, 16, 256, 2048}, LoRA r=16 except on the LM head.  Per case it times a graph of calls
(Linear forward; Linear backward, or FrozenMatmul::backward_input for the LM head) rotating over
operand sets of at least 512 MB in total, and prints one JSON line with the per-call time and the
call's roofline fraction (algorithmic bytes and flops, each operand touched once).  ``--case
FMT:SHAPE:T`` runs one of those cases (for a kernel trace of it).

``--traffic`` runs 24 eager config-1 steps and then three 64 MiB device copies, for two
``rocprofv3 --pmc`` passes (FETCH_SIZE, then WRITE_SIZE); ``--traffic-report FETCH_DIR WRITE_DIR``
turns the two passes into HBM bytes per launch of each library kernel (each counter scaled so that
the copies read and write 64 MiB), writes ``profiles/traffic_<kernel>_configs0.json`` (read by the
``--linear`` run for ``roofline.traffic``) and prints a table.  ``--traffic-step`` does the same for
two configs[2] training steps; ``--traffic-report F W --traffic-step`` writes
``profiles/traffic_<kernel>_configs2.json`` for the block-linear kernels (read by the default run).

``--head`` measures the LM head + cross-entropy of configs[2] (``Model::head``: tied Q4_0 head
151936 x 1024, 512 positions, loss on the last 256) through ``rtq_lm_head_d``, one JSON line with
the per-call time, per-kernel times, the softmax kernels' HBM fraction and the CPU oracle's rate.

``--config 3`` / ``--config 4`` measure BASELINE configs[3] (Qwen3-4B-shaped Q4_K/Q6_K model, a
packed batch of 8 x 1024 tokens sharing a 200-token prefix) and configs[4] (Llama-3-8B-shaped Q8_0
model, 2048 tokens, LoRA r=64, activations recomputed): one JSON line each with tokens/s, the
per-kernel breakdown and the dominant quantised-matmul kernel's roofline (work recorded by the
runtime per launch).  Their weights are drawn from numpy's PCG64 in parallel worker processes.

``--gguf-load PRESET[:WTYPE]`` builds a synthetic GGUF model (``SyntheticSpec``), writes it to a
temporary file, maps and parses it and uploads every frozen tensor to the GPU, and prints one JSON
line with the load throughput (frozen-tensor bytes over map + parse + upload time).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "trained tokens/s fwd+bwd, Qwen3-0.6B Q4_0 LoRA r16; quant-matmul % roofline"
N, K, T, R, ALPHA = 3072, 1024, 256, 16, 32.0
HBM_PEAK_GBS = 8000.0
# the arithmetic each part of the path computes in (the bench records' "dtype")
ARITH_FWD = ("Q8 activation codes x weight codes: exact integer block sums on f16 MFMA 16x16x32, f32 scale "
             "epilogue (frozen forward)")
ARITH_DX = ("f16 MFMA on f16 hi / lo splits of dy 2^e (per token row) and of W, about 2^-21 per product, "
            "f32 accumulation (frozen dx)")
ARITH_ATTN = ("attention forward on f16 MFMA over f16 hi / lo splits (22 bits), backward on bf16 MFMA over "
              "bf16 hi / lo splits rounded to nearest (about 2^-16 per product)")
ARITH_REST = "f32 MFMA (LoRA), f32 (norms, RoPE, SwiGLU), f32 / f64 softmax (LM head)"
F16_PEAK_TFLOPS = 2500.0  # dense f16/bf16 MFMA (the forward's integer block dots and dx run on it)


def kernel_work(name: str) -> tuple[float, float] | None:
    """(algorithmic bytes, flops) of one launch of a kernel at the bench shape."""
    w_bytes = N * K // 32 * 18
    if name.startswith("rtq_fwd_"):
        acts = T * K + T * (K // 32) * 2  # int8 codes + fp16 scales
        return float(w_bytes + acts + T * N * 4 + N * R * 4 + T * R * 4), float(2 * T * N * K + 2 * T * N * R)
    if name.startswith("rtq_dx"):  # rtq_dx_*, rtq_dx2_*, rtq_dx16_*
        return float(w_bytes + T * N * 4 + T * K * 4), float(2 * T * N * K)
    if name == "rtq_act_prep_q8_0":  # quantise x, h = x.A^T
        return float(T * K * 4 + T * K + T * (K // 32) * 4 + R * K * 4 + T * R * 4), float(2 * T * K * R)
    if name == "rtq_bwd_prep":  # partials of h = x.A^T and g = dy.B
        return float(T * K * 4 + T * N * 4 + (R * K + N * R) * 4 + 2 * T * R * 4), float(2 * T * R * (K + N))
    if name == "rtq_bwd_finish":  # dB, dA, dx = sum of split partials + g.A
        return float(T * N * 4 + T * K * 4 + 2 * T * R * 4 + 2 * (N * R + R * K) * 4 + 2 * T * K * 4), \
            float(2 * T * R * (N + 2 * K))
    return None


def roofline(name: str, avg_ms: float) -> dict | None:
    work = kernel_work(name)
    if work is None:
        return None
    bytes_, flops = work
    ai = flops / bytes_ if bytes_ else 0.0
    ridge = F16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)
    sec = avg_ms * 1e-3
    if ai < ridge:
        ach = bytes_ / sec / 1e9
        out = {"bound": "hbm", "achieved": round(ach, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
               "frac": round(ach / HBM_PEAK_GBS, 4)}
    else:
        ach = flops / sec / 1e12
        out = {"bound": "mfma", "achieved": round(ach, 2), "peak": F16_PEAK_TFLOPS, "unit": "TFLOP/s",
               "frac": round(ach / F16_PEAK_TFLOPS, 4)}
    out["kernel"] = name
    out["algorithmic_bytes"] = int(bytes_)
    out["flops"] = int(flops)
    out["avg_us"] = round(avg_ms * 1e3, 3)
    out["traffic"] = measured_traffic(name)
    return out


def measured_traffic(name: str):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary, if any."""
    p = os.path.join(ROOT, "profiles", f"traffic_{name}_configs0.json")
    if os.path.exists(p):
        try:
            return json.load(open(p)).get("bytes_per_launch")
        except Exception:
            return None
    return None


# ---------------------------------------------------------------- configs[1] sweep
SWEEP_SHAPES = {"q_proj": (2048, 1024), "kv_proj": (1024, 1024), "down_proj": (1024, 3072), "lm_head": (151936, 1024)}
# the merged projections of the configs[2] / configs[3] / configs[4] blocks (q|k|v and gate|up are one
# launch in the step; one plain adapter here), for --case runs only: (rows, cols, LoRA rank)
BLOCK_SHAPES = {"qwen06_qkv": (4096, 1024, 16), "qwen06_gate_up": (6144, 1024, 16), "qwen06_o": (1024, 2048, 16),
                "qwen06_down": (1024, 3072, 16), "llama_qkv": (6144, 4096, 64), "llama_o": (4096, 4096, 64), "llama_gate_up": (28672, 4096, 64),
                "llama_down": (4096, 14336, 64), "llama_head": (128256, 4096, 0), "qwen4b_qkv": (6144, 2560, 16),
                "qwen4b_gate_up": (19456, 2560, 16), "qwen4b_down": (2560, 9728, 16)}
SWEEP_TYPES = {"Q8_0": 8, "Q4_K": 12, "Q6_K": 14, "Q4_0": 2}
SWEEP_T = (1, 16, 256, 2048)
BLOCK = {2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210)}


def call_work(wtype: int, n: int, k: int, t: int, r: int, backward: bool) -> tuple[float, float]:
    """(algorithmic bytes, flops) of one Linear call, each operand touched once."""
    be, bb = BLOCK[wtype]
    wb = n * k // be * bb
    if not backward:  # y = x W^T + s (x A^T) B^T
        return float(wb + t * k * 4 + t * n * 4 + r * (k + n) * 4), float(2 * t * n * k + 2 * t * r * (k + n))
    # dx = dy W (+ g A), g = s dy B, h = x A^T, dA += g^T x, dB += (s dy)^T h
    lora_bytes = (t * k * 4 + 2 * (r * k + n * r) * 4 + (r * k + n * r) * 4) if r else 0
    return float(wb + t * n * 4 + t * k * 4 + lora_bytes), float(2 * t * n * k + (6 * t * r * k + 4 * t * n * r if r else 0))


def call_roofline(bytes_: float, flops: float, sec: float) -> dict:
    t_hbm, t_mfma = bytes_ / (HBM_PEAK_GBS * 1e9), flops / (F16_PEAK_TFLOPS * 1e12)
    if t_hbm >= t_mfma:
        return {"bound": "hbm", "achieved": round(bytes_ / sec / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(t_hbm / sec, 4)}
    return {"bound": "mfma", "achieved": round(flops / sec / 1e12, 2), "peak": F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(t_mfma / sec, 4)}


def sweep(cases: list[tuple[str, str, int]], calls_min: int) -> None:
    import torch

    import rust_trainer_amd as rt
    from rust_trainer_amd import _ffi, synth

    dev = torch.device("cuda", 0)
    L = _ffi.lib()
    ctx = rt.Context(0)
    side = torch.cuda.Stream()
    weights_cache: dict = {}
    for fmt, shape, t in cases:
        wtype = SWEEP_TYPES[fmt]
        if shape in BLOCK_SHAPES:
            n, k, r = BLOCK_SHAPES[shape]
        else:
            n, k = SWEEP_SHAPES[shape]
            r = 0 if shape == "lm_head" else R
        key = (fmt, shape)
        # N(0, 0.02) weights, N(0, 1) activations and gradients from torch's generators (seeded):
        # the reference Rng's stream is not needed for timing, and is slow at the LM head's sizes
        if key not in weights_cache:
            weights_cache.clear()
            gen = torch.Generator().manual_seed(1)
            w = (torch.randn(n, k, generator=gen) * 0.02).numpy()
            weights_cache[key] = synth.QUANTIZERS[wtype](w)
            del w
        blocks = weights_cache[key]
        gd = torch.Generator(device=dev).manual_seed(2)
        x = torch.randn(t, k, device=dev, generator=gd)
        dy = torch.randn(t, n, device=dev, generator=gd)
        A = torch.randn(max(r, 1), k, device=dev, generator=gd) / 32.0
        B = torch.randn(n, max(r, 1), device=dev, generator=gd) * 0.01
        set_bytes = blocks.nbytes + 4 * (2 * t * k + 2 * t * n)
        nsets = int(min(1024, max(2, -(-512 * 2**20 // set_bytes))))
        sets = []
        for _ in range(nsets):
            sset = {"w": rt.HipFrozen(wtype, blocks, n, k, ctx=ctx), "x": x.clone(), "dy": dy.clone(),
                    "y": torch.empty(t, n, device=dev), "dx": torch.zeros(t, k, device=dev),
                    "a": A.clone(), "b": B.clone(), "ga": torch.zeros(max(r, 1), k, device=dev),
                    "gb": torch.zeros(n, max(r, 1), device=dev)}
            sset["lora"] = _ffi.RtqLora(r, 2.0 * r, sset["a"].data_ptr(), sset["b"].data_ptr(), 1) if r else None
            sets.append(sset)
        ctx.reserve(t, n, k, r)
        torch.cuda.synchronize()

        def fwd(i: int, st: int) -> None:
            ss = sets[i % nsets]
            lp = ctypes.byref(ss["lora"]) if r else None
            _ffi.check(L.rtq_linear_forward_d(ctx.handle, ss["w"].handle, None, lp, ss["x"].data_ptr(), t,
                                              ss["y"].data_ptr(), st), "forward")

        def bwd(i: int, st: int) -> None:
            ss = sets[i % nsets]
            if r:
                _ffi.check(L.rtq_linear_backward_d(ctx.handle, ss["w"].handle, ctypes.byref(ss["lora"]),
                                                   ss["x"].data_ptr(), ss["dy"].data_ptr(), t, ss["dx"].data_ptr(),
                                                   ss["ga"].data_ptr(), ss["gb"].data_ptr(), st), "backward")
            else:
                _ffi.check(L.rtq_frozen_backward_input_d(ctx.handle, ss["w"].handle, ss["dy"].data_ptr(), t,
                                                         ss["dx"].data_ptr(), st), "backward_input")

        ncalls = max(calls_min, nsets)
        out = {"sweep": "configs[1]" if shape in SWEEP_SHAPES else "block", "format": fmt, "shape": shape, "rows": n, "cols": k, "tokens": t,
               "lora_rank": r, "operand_sets": nsets, "calls": ncalls}
        for name, fn in (("forward", fwd), ("backward", bwd)):
            with torch.cuda.stream(side):
                st = torch.cuda.current_stream().cuda_stream
                for i in range(min(ncalls, 2 * nsets)):
                    fn(i, st)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                st = torch.cuda.current_stream().cuda_stream
                for i in range(ncalls):
                    fn(i, st)
            g.replay()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            g.replay()
            torch.cuda.synchronize()
            sec = (time.perf_counter() - t0) / ncalls
            bytes_, flops = call_work(wtype, n, k, t, r, name == "backward")
            out[name] = {"us_per_call": round(sec * 1e6, 3), "tokens_per_s": round(t / sec, 1),
                         "gflops": round(flops / sec / 1e9, 1), "algorithmic_bytes": int(bytes_),
                         "roofline": call_roofline(bytes_, flops, sec)}
            del g
        print(json.dumps(out), flush=True)
        for sset in sets:
            sset["w"].close()
        del sets, x, dy, A, B
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    ctx.close()


# ---------------------------------------------------------------- HBM traffic (rocprofv3 --pmc)
COPY_MIB = 64


def traffic_run() -> None:
    import torch

    import rust_trainer_amd as rt
    from rust_trainer_amd import _ffi, synth

    dev = torch.device("cuda", 0)
    ctx = rt.Context(0)
    ctx.reserve(T, N, K, R)
    L = _ffi.lib()
    blocks = synth.quantize_q4_0(synth.Rng(1).vec_normal(N * K, 0.02).reshape(N, K))
    sets = []
    for _ in range(8):
        s = {"w": rt.HipFrozen(rt.TYPE_Q4_0, blocks, N, K, ctx=ctx), "x": torch.randn(T, K, device=dev),
             "dy": torch.randn(T, N, device=dev), "y": torch.empty(T, N, device=dev), "dx": torch.empty(T, K, device=dev),
             "a": torch.randn(R, K, device=dev) / 32.0, "b": torch.randn(N, R, device=dev) * 0.01,
             "ga": torch.zeros(R, K, device=dev), "gb": torch.zeros(N, R, device=dev)}
        s["lora"] = _ffi.RtqLora(R, ALPHA, s["a"].data_ptr(), s["b"].data_ptr(), 1)
        sets.append(s)
    st = torch.cuda.current_stream().cuda_stream
    for i in range(24):
        s = sets[i % len(sets)]
        lp = ctypes.byref(s["lora"])
        _ffi.check(L.rtq_linear_forward_d(ctx.handle, s["w"].handle, None, lp, s["x"].data_ptr(), T, s["y"].data_ptr(),
                                          st), "forward")
        _ffi.check(L.rtq_linear_backward_d(ctx.handle, s["w"].handle, lp, s["x"].data_ptr(), s["dy"].data_ptr(), T,
                                           s["dx"].data_ptr(), s["ga"].data_ptr(), s["gb"].data_ptr(), st), "backward")
    torch.cuda.synchronize()
    src = torch.empty(COPY_MIB * 2**20 // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    for s in sets:
        s["w"].close()
    ctx.close()
    print("traffic run done", flush=True)


def traffic_run_step() -> None:
    """Two configs[2] training steps, then the three 64 MiB calibration copies (for --pmc passes)."""
    import numpy as np
    import torch

    import rust_trainer_amd as rt
    from rust_trainer_amd import gguf as G, synth

    g = G.GgufFile.from_bytes(G.SyntheticSpec.preset("qwen3-0.6b", G.GGML_Q4_0).build())
    ctx = rt.Context(0)
    model = rt.GpuModel.from_gguf(g, ctx=ctx)
    model.attach_lora(STEP_R, STEP_ALPHA, seed=1)
    tokens = (synth.Rng(7).next_u64(STEP_T) % np.uint64(model.config["n_vocab"])).astype(np.int32)
    targets = rt.answer_targets(tokens, STEP_T - STEP_N)
    wts = np.full(len(targets), 1.0 / len(targets), np.float32)
    for _ in range(2):
        model.zero_grad()
        model.forward_backward(tokens, targets, wts)
    src = torch.empty(COPY_MIB * 2**20 // 4, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    model.close()
    ctx.close()
    print("traffic step run done", flush=True)


def step_kernel_work(name: str) -> tuple[float, float] | None:
    """Average algorithmic (bytes, flops) per launch of a block-linear kernel of the configs[2] step."""
    cfg = {"n_embd": 1024, "n_head": 16, "n_head_kv": 8, "head_dim": 128, "n_ff": 3072}
    calls, backward = step_calls_for(name, cfg)
    if calls is None:
        return None
    if backward:
        w = [(float(n * k // 32 * 18 + STEP_T * (n + k) * 4), float(2 * STEP_T * n * k)) for n, k, _ in calls]
    else:
        w = [call_work(2, n, k, STEP_T, r, False) for n, k, r in calls]
    return sum(b for b, _ in w) / len(w), sum(f for _, f in w) / len(w)


def traffic_report(fetch_dir: str, write_dir: str, step: bool = False) -> None:
    """Counter CSVs of the two --pmc passes -> profiles/traffic_<kernel>_configs0.json (configs2 for
    the training step) and a table."""
    import csv
    import glob

    def read(d: str, counter: str) -> tuple[dict, float]:
        per: dict = {}
        copies = []
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] != counter:
                    continue
                v, name = float(r["Counter_Value"]), r["Kernel_Name"]
                dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3
                if name.startswith("rtq_"):
                    per.setdefault(name, []).append((v, dur))
                elif "copy" in name.lower():
                    copies.append(v)
        copies.sort()
        return per, (sum(copies[-3:]) / len(copies[-3:]) if copies else 0.0)

    fetch, fcopy = read(fetch_dir, "FETCH_SIZE")
    write, wcopy = read(write_dir, "WRITE_SIZE")
    ff = COPY_MIB * 1024 / fcopy if fcopy else None  # KiB the copy moves / KiB the counter reads
    wf = COPY_MIB * 1024 / wcopy if wcopy else None
    rows = []
    for name in sorted(set(fetch) & set(write)):
        fk = sum(v for v, _ in fetch[name]) / len(fetch[name])
        wk = sum(v for v, _ in write[name]) / len(write[name])
        total = (fk * ff + wk * wf) * 1024 if ff and wf else None
        algo = step_kernel_work(name) if step else kernel_work(name)
        out = {"kernel": name, "workload": "configs[2] training step (average launch over the block linears it serves)" if step
               else "configs[0] (Q4_0 3072x1024, T=256, LoRA r=16)",
               "fetch_kib_raw": round(fk, 1), "write_kib_raw": round(wk, 1),
               "fetch_scale": round(ff, 4) if ff else None, "write_scale": round(wf, 4) if wf else None,
               "bytes_per_launch": round(total) if total else None,
               "algorithmic_bytes": int(algo[0]) if algo else None, "launches": len(fetch[name])}
        if step and algo is None:
            continue
        tag = "configs2" if step else "configs0"
        json.dump(out, open(os.path.join(ROOT, "profiles", f"traffic_{name}_{tag}.json"), "w"), indent=1)
        rows.append(out)
    print(f"calibration: {COPY_MIB} MiB copies read {fcopy:.0f} KiB (FETCH_SIZE) and write {wcopy:.0f} KiB "
          f"(WRITE_SIZE) -> scales {ff:.4f} / {wf:.4f}")
    print("| kernel | launches | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes/launch (scaled) | algorithmic bytes |")
    print("|---|---|---|---|---|---|")
    for o in rows:
        print(f"| {o['kernel']} | {o['launches']} | {o['fetch_kib_raw']} | {o['write_kib_raw']} | "
              f"{o['bytes_per_launch']} | {o['algorithmic_bytes']} |")


SQ_COUNTERS = ("SQ_VALU_MFMA_BUSY_CYCLES SQ_ACTIVE_INST_VALU SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS "
               "SQ_LDS_BANK_CONFLICT SQ_WAIT_INST_LDS SQ_WAVE_CYCLES GRBM_GUI_ACTIVE")
SIMD_NUM, CU_NUM = 1024, 256


def counters_report(sq_dir: str, fetch_dir: str | None, write_dir: str | None, title: str, out_md: str) -> None:
    """Per-kernel summary of one rocprofv3 --pmc pass of SQ_COUNTERS (and, if given, the FETCH_SIZE /
    WRITE_SIZE passes with the copy calibration of --traffic-report) -> a markdown table in
    profiles/<out_md>, kernels ordered by their share of the profiled run's kernel time.
    MFMA busy % = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x 1024 SIMDs); VALU busy % =
    SQ_ACTIVE_INST_VALU / (GRBM_GUI_ACTIVE per XCD x 256 CUs); LDS bank-conflict % = conflict cycles /
    (GRBM_GUI_ACTIVE per XCD x 256 CUs) (the formulas of rocprofiler-sdk's MfmaUtil, VALUBusy and
    LDSBankConflict; GRBM_GUI_ACTIVE in the CSV is the sum over the 8 XCDs)."""
    import csv
    import glob

    def per_kernel(d: str) -> dict:
        agg: dict = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                name = r["Kernel_Name"]
                k = agg.setdefault(name, {"disp": {}, "sum": {}, "each": []})
                k["disp"][r["Dispatch_Id"]] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3
                k["sum"][r["Counter_Name"]] = k["sum"].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
                k["each"].append(float(r["Counter_Value"]))
        return agg

    sq = per_kernel(sq_dir)
    fetch = per_kernel(fetch_dir) if fetch_dir else {}
    write = per_kernel(write_dir) if write_dir else {}

    def copy_scale(agg: dict) -> float | None:  # the three largest copy dispatches are the calibration copies
        vals = sorted(x for n, v in agg.items() if "copy" in n.lower() for x in v["each"])
        return COPY_MIB * 1024 / (sum(vals[-3:]) / len(vals[-3:])) if vals else None

    fs, ws = copy_scale(fetch), copy_scale(write)
    total_us = sum(sum(v["disp"].values()) for n, v in sq.items() if n.startswith("rtq_"))
    rows = []
    for name, v in sq.items():
        if not name.startswith("rtq_"):
            continue
        n = len(v["disp"])
        c = {k: x / n for k, x in v["sum"].items()}
        gui = c.get("GRBM_GUI_ACTIVE", 0.0) / 8.0
        row = {"kernel": name, "dispatches": n, "avg_us": sum(v["disp"].values()) / n,
               "share": sum(v["disp"].values()) / total_us if total_us else 0.0,
               "mfma_busy": 100.0 * c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (gui * SIMD_NUM) if gui else None,
               "valu_busy": 100.0 * c.get("SQ_ACTIVE_INST_VALU", 0.0) / (gui * CU_NUM) if gui else None,
               "lds_conflict": 100.0 * c.get("SQ_LDS_BANK_CONFLICT", 0.0) / (gui * CU_NUM) if gui else None,
               "valu": c.get("SQ_INSTS_VALU"), "mfma": c.get("SQ_INSTS_MFMA"), "lds": c.get("SQ_INSTS_LDS"),
               "wait_lds": c.get("SQ_WAIT_INST_LDS")}
        if name in fetch and fs:
            row["fetch_mb"] = fetch[name]["sum"]["FETCH_SIZE"] / len(fetch[name]["disp"]) * fs * 1024 / 1e6
        if name in write and ws:
            row["write_mb"] = write[name]["sum"]["WRITE_SIZE"] / len(write[name]["disp"]) * ws * 1024 / 1e6
        rows.append(row)
    rows.sort(key=lambda r: -r["share"])

    def f(x, fmt):
        return "-" if x is None else format(x, fmt)

    lines = [f"# {title}", "",
             "| kernel | dispatches | avg us (under counters) | share | MFMA busy % | VALU busy % | LDS bank-conflict % | "
             "VALU insts | MFMA insts | LDS insts | HBM read MB | HBM write MB |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for r in rows:
        lines.append(f"| {r['kernel']} | {r['dispatches']} | {r['avg_us']:.1f} | {r['share']:.3f} | {f(r['mfma_busy'], '.1f')} | "
                     f"{f(r['valu_busy'], '.1f')} | {f(r['lds_conflict'], '.1f')} | {f(r['valu'], '.0f')} | "
                     f"{f(r['mfma'], '.0f')} | {f(r['lds'], '.0f')} | {f(r.get('fetch_mb'), '.2f')} | "
                     f"{f(r.get('write_mb'), '.2f')} |")
    if fs and ws:
        lines += ["", f"HBM bytes: FETCH_SIZE x {fs:.4f} and WRITE_SIZE x {ws:.4f} (the {COPY_MIB} MiB calibration copies' "
                  "counter readings against the bytes they move)."]
    text = "\n".join(lines) + "\n"
    path = os.path.join(ROOT, "profiles", out_md)
    head = ""
    if os.path.exists(path):  # keep a hand-written preamble (commands) above the generated table
        old = open(path).read()
        cut = old.find("<!-- generated -->")
        head = old[:cut] if cut >= 0 else ""
    open(path, "w").write((head or "") + "<!-- generated -->\n" + text)
    print(text)


def host_threads() -> int:
    """Host threads the CPU baselines use: the CPUs of this process's affinity mask, at most 16 (one
    GPU's share of the GPU box's host cores, whatever the machine's total)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def host_info() -> dict:
    """The host the CPU baseline ran on: the machine's CPU count (nproc), this process's affinity
    mask, and why the threads stop at 16 (a GPU box runs one GPU's share of its host cores)."""
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = os.cpu_count() or 1
    return {"nproc": os.cpu_count(), "affinity_cpus": aff, "threads_cap": 16,
            "cap": "worker pools on a GPU box stay within one GPU's share of its host cores (16)"}


def timed_runs(fn, warmup: int, runs: int, threads: int) -> list[float]:
    """Seconds of each of ``runs`` calls of fn after ``warmup`` untimed ones, with an OpenMP team of
    ``threads`` pinned one per CPU (the calling thread's affinity is restored afterwards)."""
    import oracle as O

    saved = os.sched_getaffinity(0)
    try:
        O.pin_threads(threads)
        for _ in range(warmup):
            fn()
        out = []
        for _ in range(runs):
            t0 = time.perf_counter()
            fn()
            out.append(time.perf_counter() - t0)
        return out
    finally:
        os.sched_setaffinity(0, saved)


def cpu_baseline(inputs, seconds: float) -> dict:
    """configs[0] on the host cores: the oracle's Linear forward + backward (C restatement of
    RieFrozen / Linear, AVX2 + FMA, OpenMP), threads pinned, 2 warm-up calls then the median of 10,
    at nproc (at most 16), 4 and 1 threads.  ``seconds`` is unused (the sample is fixed)."""
    import statistics

    import oracle as O

    blocks, x, dy, A, B = inputs

    def step():
        O.linear_forward(O.Q4_0, blocks, N, K, x, A=A, B=B, alpha=ALPHA, nthreads=threads)
        O.linear_backward(O.Q4_0, blocks, N, K, x, dy, A=A, B=B, alpha=ALPHA, nthreads=threads)

    fb, ff = call_work(2, N, K, T, R, False)
    bb, bf = call_work(2, N, K, T, R, True)
    nproc = host_threads()
    by = {}
    for threads in sorted({nproc, 4, 1}, reverse=True):
        ts = timed_runs(step, 2, 10, threads)
        med = statistics.median(ts)
        by[str(threads)] = {"tokens_per_s": round(T / med, 1), "median_ms": round(med * 1e3, 3),
                            "gflops": round((ff + bf) / med / 1e9, 2), "gb_per_s": round((fb + bb) / med / 1e9, 3),
                            "runs_ms": [round(t * 1e3, 3) for t in ts]}
    return {"value": by[str(nproc)]["tokens_per_s"], "unit": "tokens/s", "cores": nproc, "kind": "port",
            "cpu_model": O.cpu_model(), "host": host_info(), "by_threads": by,
            "method": "threads pinned one per CPU (sched_setaffinity), AVX2 + FMA build (-march=x86-64-v3), "
                      "2 warm-up calls then the median of 10",
            "sample": f"configs[0] whole: Linear forward + backward (y, dx, dA, dB), Q4_0 {N}x{K}, T={T}, "
                      f"LoRA r={R}; C restatement of RieFrozen/Linear (oracle/rtq_oracle.c, -O3, OpenMP)"}


# ---------------------------------------------------------------- LM head + cross-entropy
HEAD_V, HEAD_D, HEAD_T, HEAD_N = 151936, 1024, 512, 256


def head_bench(steps: int, warmup: int, cpu_seconds: float, no_cpu: bool) -> None:
    """Model::head of configs[2]: Qwen3-0.6B tied LM head (Q4_0 151936 x 1024), 512 positions,
    cross-entropy on the last 256 (answer_targets), weights 1/256; one call = final RMSNorm +
    logits + log-softmax + dlogits + lm_head backward_input + RMSNorm backward (rtq_lm_head_d)."""
    import numpy as np
    import torch

    import rust_trainer_amd as rt
    from rust_trainer_amd import _ffi, synth

    V, D, T_, N_ = HEAD_V, HEAD_D, HEAD_T, HEAD_N
    blocks = synth.quantize_q4_0(synth.Rng(1).vec_normal(V * D, 0.02).reshape(V, D))
    X = synth.Rng(2).vec_normal(T_ * D, 1.0).reshape(T_, D)
    tokens = (synth.Rng(3).next_u64(T_) % np.uint64(V)).astype(np.int32)
    targets = rt.answer_targets(tokens, T_ - N_)
    pos = np.array([tg.pos for tg in targets], np.int32)
    tok = np.array([tg.token for tg in targets], np.int32)
    wts = np.full(N_, 1.0 / N_, np.float32)
    norm = np.ones(D, np.float32)
    dev = torch.device("cuda", 0)
    ctx = rt.Context(0)
    f = rt.HipFrozen(rt.TYPE_Q4_0, blocks, V, D, ctx=ctx)
    xd, nd = torch.from_numpy(X).to(dev), torch.from_numpy(norm).to(dev)
    pd, kd, wd = (torch.from_numpy(a).to(dev) for a in (pos, tok, wts))
    lp = torch.empty(N_, device=dev)
    hit = torch.empty(N_, dtype=torch.int32, device=dev)
    dx = torch.empty(T_, D, device=dev)
    L = _ffi.lib()
    side = torch.cuda.Stream()

    def call(st: int) -> None:
        _ffi.check(L.rtq_lm_head_d(ctx.handle, f.handle, nd.data_ptr(), 1e-6, 0.0, xd.data_ptr(), T_, pd.data_ptr(),
                                   kd.data_ptr(), wd.data_ptr(), N_, lp.data_ptr(), hit.data_ptr(), dx.data_ptr(),
                                   st), "rtq_lm_head_d")

    def eager(k: int) -> None:
        with torch.cuda.stream(side):
            st = torch.cuda.current_stream().cuda_stream
            for _ in range(k):
                call(st)
        torch.cuda.synchronize()

    eager(warmup)
    ctx.set_timing(True)
    ctx.reset_timing()
    eager(steps)
    per = ctx.timing()
    ctx.set_timing(False)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        st = torch.cuda.current_stream().cuda_stream
        for _ in range(steps):
            call(st)
    g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    logits_bytes = N_ * V * 4
    ce = [k for k in per if k.startswith("rtq_head_") and k != "rtq_head_norm" and k != "rtq_head_norm_bwd"]
    ce_ms = sum(per[k][1] / per[k][0] for k in ce)
    ce_bytes = 4 * logits_bytes  # max, sum and grad read the logits, grad writes dlogits over them
    wbytes = V * D // 32 * 18
    bytes_, flops = 2 * wbytes + (T_ * D + 2 * N_ * D) * 4 + T_ * D * 4, 4.0 * N_ * V * D
    result = {
        "metric": "LM head + cross-entropy fwd+bwd (Model::head), targets/s", "value": round(N_ / (ms * 1e-3), 1),
        "unit": "targets/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "data": "synthetic",
        "dtype": f"{ARITH_FWD.replace('frozen forward', 'logits')}; f32 / f64 softmax; "
                 f"{ARITH_DX.replace('frozen dx', 'dlogits . W')}",
        "config": {"workload": "configs[2] head: tied LM head Q4_0 151936x1024, 512 positions, loss on the "
                               "last 256 (answer_targets), weights 1/256",
                   "vocab": V, "hidden": D, "positions": T_, "targets": N_},
        "call_roofline": call_roofline(bytes_, flops, ms * 1e-3),
        "softmax_roofline": {"bound": "hbm", "achieved": round(ce_bytes / (ce_ms * 1e-3) / 1e9, 1),
                             "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(ce_bytes / (ce_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                             "kernels": ce, "algorithmic_bytes": ce_bytes},
        "kernels": {k: {"avg_us": round(m * 1e3 / c, 3), "launches": c} for k, (c, m) in sorted(per.items())},
    }
    if not no_cpu:
        import oracle as O

        threads = host_threads()
        n_s, calls, t0 = 16, 0, time.perf_counter()
        while True:
            O.lm_head(O.Q4_0, blocks, V, D, norm, X, pos[:n_s], tok[:n_s], wts[:n_s], nthreads=threads)
            calls += 1
            el = time.perf_counter() - t0
            if el >= cpu_seconds:
                break
        result["cpu_baseline"] = {"value": round(n_s * calls / el, 1), "unit": "targets/s", "cores": threads,
                                  "kind": "port", "host": host_info(),
                                  "sample": f"{calls} calls of Model::head on {n_s} targets in {el:.1f} s "
                                            f"(oracle/rtq_oracle.c or_lm_head, -O3 AVX2, OpenMP)"}
    f.close()
    ctx.close()
    print(json.dumps(result), flush=True)


# ---------------------------------------------------------------- full training step
STEP_T, STEP_N, STEP_R, STEP_ALPHA = 512, 256, 16, 32.0


def model_flops(cfg: dict, t: int, n: int) -> tuple[float, dict]:
    """Flops of one training step (forward + backward, activations kept): per block 2 t (params) for
    each linear pass (forward, dx), the LoRA products, attention's causal products; the head's
    forward and dx on the n target rows."""
    d, nh, nkv, hd, ff, L, V = (cfg[k] for k in ("n_embd", "n_head", "n_head_kv", "head_dim", "n_ff", "n_layer",
                                                  "n_vocab"))
    lin = d * nh * hd + 2 * d * nkv * hd + nh * hd * d + 3 * d * ff
    r = STEP_R
    lora_dims = [(d, nh * hd), (d, nkv * hd), (d, nkv * hd), (nh * hd, d), (d, ff), (d, ff), (ff, d)]
    lora = sum(2 * t * r * (k + n_) + 2 * t * r * (3 * k + 2 * n_) for k, n_ in lora_dims)
    att_fwd = 2 * 2 * nh * (t * (t + 1) / 2) * hd  # S and O over the causal half
    att_bwd = 4 * 2 * nh * (t * (t + 1) / 2) * hd  # dP, dV, dQ, dK
    per_block = 2 * t * lin * 2 + lora + att_fwd + att_bwd
    head = 2 * n * V * d * 2
    parts = {"linears_fwd_dx": 4.0 * t * lin * L, "lora": float(lora * L), "attention": (att_fwd + att_bwd) * L,
             "head": float(head)}
    return per_block * L + head, parts


def model_bench(steps: int, warmup: int, cpu_seconds: float, no_cpu: bool) -> dict:
    """Qwen3-0.6B-shaped synthetic Q4_0 GGUF, LoRA r=16 alpha=32 on q,k,v,o,gate,up,down,
    512 uniform-random tokens, cross-entropy on the last 256 (answer_targets, weights 1/256); one
    step = zero_grad + Model::forward_backward (rtq_model_forward_backward)."""
    import numpy as np
    import torch

    import rust_trainer_amd as rt
    from rust_trainer_amd import gguf as G, synth

    t0 = time.perf_counter()
    spec = G.SyntheticSpec.preset("qwen3-0.6b", G.GGML_Q4_0)
    image = spec.build(workers=max(1, min(16, os.cpu_count() or 1)))
    print(f"[model] built the synthetic GGUF in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    g = G.GgufFile.from_bytes(image)
    ctx = rt.Context(0)
    model = rt.GpuModel.from_gguf(g, ctx=ctx)
    n_params = model.attach_lora(STEP_R, STEP_ALPHA, seed=1)
    if ATTENTION_MODE is not None:  # --attention: force the fused or the unfused kernels
        model.fused_attention = ATTENTION_MODE
    cfg = model.config
    tokens = (synth.Rng(7).next_u64(STEP_T) % np.uint64(cfg["n_vocab"])).astype(np.int32)
    targets = rt.answer_targets(tokens, STEP_T - STEP_N)
    wts = np.full(len(targets), 1.0 / len(targets), np.float32)

    def step() -> np.ndarray:
        model.zero_grad()
        return model.forward_backward(tokens, targets, wts)[0]

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    ctx.set_timing(True)
    ctx.reset_timing()
    step()
    per = ctx.timing()
    ctx.set_timing(False)
    t0 = time.perf_counter()
    for _ in range(steps):
        lp = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    flops, parts = model_flops(cfg, STEP_T, len(targets))
    total_k = sum(m for _, m in per.values())
    result = {
        "value": round(STEP_T / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 3),
        "mean_loss": float(-lp.mean()),
        "config": {"workload": "configs[2]: Qwen3-0.6B-shaped synthetic Q4_0 GGUF (28 layers, hidden 1024, FFN "
                               "3072, 16/8 heads of 128, QK-norm, NEOX RoPE 1e6, vocab 151936 tied), LoRA r=16 "
                               "alpha=32 on q,k,v,o,gate,up,down, 512 random tokens, loss on the last 256",
                   "tokens": STEP_T, "targets": len(targets), "rank": STEP_R, "lora_params": n_params},
        "step_flops": flops, "step_flops_parts": parts,
        "step_roofline": {"bound": "mfma", "achieved": round(flops / (ms * 1e-3) / 1e12, 2), "peak": F16_PEAK_TFLOPS,
                          "unit": "TFLOP/s", "frac": round(flops / (ms * 1e-3) / 1e12 / F16_PEAK_TFLOPS, 4)},
        "kernels": {k: {"launches": c, "total_us": round(m * 1e3, 1), "share": round(m / total_k, 4)}
                    for k, (c, m) in sorted(per.items(), key=lambda kv: -kv[1][1])},
    }
    if not no_cpu:
        result["cpu_baseline"] = model_cpu_baseline(spec, g, cpu_seconds)
    model.close()
    ctx.close()
    return result


def step_layer_calls(cfg: dict, t: int) -> list[tuple[int, int, int]]:
    """(rows, cols, adapter rank) of the frozen linear calls of one block: q | k | v, o, gate | up,
    down (the fused groups of rtq_model_*)."""
    d, nh, nkv, hd, ff = (cfg[k] for k in ("n_embd", "n_head", "n_head_kv", "head_dim", "n_ff"))
    return [(nh * hd + 2 * nkv * hd, d, 3 * STEP_R), (d, nh * hd, STEP_R), (2 * ff, d, 2 * STEP_R), (d, ff, STEP_R)]


def step_calls_for(name: str, cfg: dict):
    """(calls, backward) of the block linears a kernel serves in the step, by the runtime's choice at
    T = 512: rtq_mm32_* the wide fused forwards (q | k | v, gate | up), rtq_fwd_*_w8 the others (o,
    down), rtq_dx_* every input gradient."""
    qkv, o, gu, down = step_layer_calls(cfg, STEP_T)
    if name.startswith("rtq_dx_"):
        return [qkv, o, gu, down], True
    if name.startswith("rtq_mm32_"):
        return [qkv, gu], False
    if name.startswith("rtq_fwd_"):
        return [o, down], False
    return None, False


def step_roofline(cfg: dict, kernels: dict) -> dict | None:
    """Roofline of the dominant quantised-matmul kernel of the step: the algorithmic bytes and flops
    of the block linears it ran (forward: W + x + y + adapter, 2 T N K + LoRA; dx: W + dy + dx,
    2 T N K) over its total time in the step."""
    qmm = {k: v for k, v in kernels.items() if k.startswith(("rtq_fwd_", "rtq_mm_", "rtq_gemv_", "rtq_dx"))}
    if not qmm:
        return None
    name = max(qmm, key=lambda k: qmm[k]["total_us"])
    per_layer, backward = step_calls_for(name, cfg)
    if per_layer is None:
        return None
    calls = per_layer * cfg["n_layer"]
    if qmm[name]["launches"] != len(calls):
        return None  # the kernel also served other shapes: no per-call attribution
    bytes_ = flops = 0.0
    for n, k, r in calls:
        b, f = call_work(2, n, k, STEP_T, 0 if backward else r, False)
        if backward:  # dx = dy . W: W + dy + dx
            b, f = float(n * k // 32 * 18 + STEP_T * n * 4 + STEP_T * k * 4), float(2 * STEP_T * n * k)
        bytes_ += b
        flops += f
    sec = qmm[name]["total_us"] * 1e-6
    out = call_roofline(bytes_, flops, sec)
    out.update({"kernel": name, "launches": len(calls), "avg_us": round(qmm[name]["total_us"] / len(calls), 3),
                "algorithmic_bytes": int(bytes_ / len(calls)), "flops": int(flops / len(calls)),
                "traffic": measured_traffic_step(name)})
    return out


def measured_traffic_step(name: str):
    p = os.path.join(ROOT, "profiles", f"traffic_{name}_configs2.json")
    if os.path.exists(p):
        try:
            return json.load(open(p)).get("bytes_per_launch")
        except Exception:
            return None
    return None


def step_line(args) -> dict:
    """The contract line: configs[2]'s full training step."""
    r = model_bench(args.steps, args.warmup, args.cpu_seconds, args.no_cpu)
    cfg = {"n_embd": 1024, "n_head": 16, "n_head_kv": 8, "head_dim": 128, "n_ff": 3072, "n_layer": 28}
    line = {
        "metric": METRIC, "value": r["value"], "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": r["ms_per_step"], "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{ARITH_FWD}; {ARITH_DX}; {ARITH_ATTN}; {ARITH_REST}",
        "data": "synthetic",
        "config": r["config"],
        "roofline": step_roofline(cfg, r["kernels"]),
        "step_roofline": r["step_roofline"],
        "kernels": r["kernels"],
    }
    if "cpu_baseline" in r:
        line["cpu_baseline"] = r["cpu_baseline"]
    return line


ATTENTION_MODE = None  # bench.py --attention fused|unfused (None: the library's choice)


# ---------------------------------------------------------------- configs[3] and configs[4]
def config_workload(idx: int):
    """(spec, description, build_batch) of BASELINE.json configs[3] / configs[4]; build_batch(model)
    returns (one step's callable, sequence tokens per step, extra config fields)."""
    import numpy as np

    import rust_trainer_amd as rt
    from rust_trainer_amd import gguf as G, synth
    from rust_trainer_amd.packing import answer_targets, pack

    if idx == 3:
        spec = G.SyntheticSpec.preset("qwen3-4b", G.GGML_Q4_K)
        desc = ("configs[3]: Qwen3-4B-shaped synthetic GGUF (36 layers, hidden 2560, FFN 9728, 32/8 heads of 128, "
                "QK-norm, NEOX RoPE 1e6, vocab 151936 tied), Q4_K attention/gate/up, Q6_K down and embedding/output, "
                "LoRA r=16 alpha=32 on every projection; 8 sequences x 1024 random tokens sharing a 200-token prefix, "
                "packed (shared prompt computed once, 6792 tokens), answer-token loss on the final 300 positions of "
                "each sequence")
        rank, alpha = 16, 32.0

        def batch(model):
            V = model.config["n_vocab"]
            r = synth.Rng(11).next_u64(200 + 8 * 824) % np.uint64(V)
            prefix = [int(v) for v in r[:200]]
            seqs = [prefix + [int(v) for v in r[200 + 824 * k: 200 + 824 * (k + 1)]] for k in range(8)]
            p = pack(seqs)
            targets = []
            for k, sq in enumerate(seqs):
                targets += p.map_targets(k, answer_targets(sq, 1024 - 300))
            wts = np.full(len(targets), 1.0 / len(targets), np.float32)

            def step():
                model.zero_grad()
                return model.forward_backward_packed(p, targets, wts)[0]

            return step, 8 * 1024, {"packed_tokens": len(p.tokens), "sequences": 8, "targets": len(targets),
                                    "rank": rank}
    elif idx == 4:
        spec = G.SyntheticSpec.preset("llama3-8b", G.GGML_Q8_0)
        desc = ("configs[4]: Llama-3-8B-shaped synthetic GGUF (32 layers, hidden 4096, FFN 14336, 32/8 heads of 128, "
                "adjacent-pair RoPE 5e5, vocab 128256 untied), every linear Q8_0, LoRA r=64 alpha=128 on every "
                "projection; 2048 random tokens, activations recomputed in the backward (checkpointing), loss on "
                "the last 1024 positions")
        rank, alpha = 64, 128.0

        def batch(model):
            V = model.config["n_vocab"]
            tokens = (synth.Rng(7).next_u64(2048) % np.uint64(V)).astype(np.int32)
            targets = rt.answer_targets(tokens, 2048 - 1024)
            wts = np.full(len(targets), 1.0 / len(targets), np.float32)
            model.checkpointing = True

            def step():
                model.zero_grad()
                return model.forward_backward(tokens, targets, wts)[0]

            return step, 2048, {"tokens": 2048, "targets": len(targets), "rank": rank, "checkpointing": True}
    else:
        raise SystemExit(f"--config {idx}: use 3 or 4 (configs[0] is --linear, configs[1] --sweep, configs[2] the "
                         f"default line)")
    spec.fast = True
    return spec, desc, rank, alpha, batch


def config_bench(idx: int, steps: int, warmup: int) -> dict:
    """One JSON line for configs[3] / configs[4]: tokens/s of the whole training step (sequence
    tokens / step time), per-kernel event times, the dominant quantised-matmul kernel's roofline from
    the algorithmic work the runtime records per launch."""
    import numpy as np
    import torch

    import rust_trainer_amd as rt
    from rust_trainer_amd import gguf as G

    spec, desc, rank, alpha, batch = config_workload(idx)
    t0 = time.perf_counter()
    workers = max(1, min(16, os.cpu_count() or 1))
    image = spec.build(workers=workers)
    print(f"[config {idx}] built the synthetic GGUF ({len(image) / 1e9:.2f} GB) in {time.perf_counter() - t0:.1f} s "
          f"with {workers} workers", file=sys.stderr, flush=True)
    g = G.GgufFile.from_bytes(image)
    ctx = rt.Context(0)
    t0 = time.perf_counter()
    model = rt.GpuModel.from_gguf(g, ctx=ctx)
    print(f"[config {idx}] loaded in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
    n_params = model.attach_lora(rank, alpha, seed=1)
    if ATTENTION_MODE is not None:
        model.fused_attention = ATTENTION_MODE
    step, seq_tokens, extra = batch(model)
    for i in range(warmup):
        step()
        print(f"[config {idx}] warmup step {i + 1} done", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    ctx.set_timing(True)
    ctx.reset_timing()
    step()
    per = ctx.timing()
    work = ctx.timing_work()
    ctx.set_timing(False)
    t0 = time.perf_counter()
    for _ in range(steps):
        lp = step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    total_k = sum(m for _, m in per.values())
    qmm = {k: v for k, v in per.items() if k in work}
    dom = max(qmm, key=lambda k: qmm[k][1]) if qmm else None
    roof = None
    if dom:
        cnt, kms = per[dom]
        fl, by = work[dom]
        roof = call_roofline(by / cnt, fl / cnt, kms * 1e-3 / cnt)
        roof.update({"kernel": dom, "launches": cnt, "avg_us": round(kms * 1e3 / cnt, 3),
                     "algorithmic_bytes": int(by / cnt), "flops": int(fl / cnt), "traffic": None,
                     "timing": "HIP events on the launch stream (a few us above kernel-trace durations)"})
    linear_fl = sum(f for f, _ in work.values())
    linear_ms = sum(per[k][1] for k in work)
    return {
        "metric": f"trained tokens/s fwd+bwd, BASELINE configs[{idx}]", "value": round(seq_tokens / (ms * 1e-3), 1),
        "unit": "tokens/s", "n_gpus": 1, "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": f"{ARITH_FWD}; {ARITH_DX}; {ARITH_ATTN}; {ARITH_REST}",
        "data": "synthetic (weights N(0, 0.02) from numpy PCG64, quantised with the synthetic encoders)",
        "config": dict({"workload": desc, "lora_params": n_params}, **extra),
        "mean_loss": float(-lp.mean()),
        "roofline": roof,
        "frozen_linear_kernels": {"tflops_achieved": round(linear_fl / (linear_ms * 1e-3) / 1e12, 2),
                                  "share_of_kernel_time": round(linear_ms / total_k, 4)},
        "kernels": {k: {"launches": c, "total_us": round(m * 1e3, 1), "share": round(m / total_k, 4)}
                    for k, (c, m) in sorted(per.items(), key=lambda kv: -kv[1][1])[:24]},
    }


def model_cpu_baseline(spec, g, seconds: float) -> dict:
    """configs[2]'s training step on the host cores: the oracle's Model::forward_backward (C
    restatement, AVX2 + FMA, OpenMP) over the whole 28-block model, threads pinned at nproc (at most
    16), one warm-up step of a 2-block cut of the same model (same shapes: thread pool, first-touch
    pages), then the median of 3 full steps.  ``seconds`` is unused (the sample is fixed)."""
    import statistics

    import numpy as np

    import oracle as O
    from rust_trainer_amd import gguf as G, synth

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from model_cases import adapters, oracle_model

    threads = host_threads()
    tokens = (synth.Rng(7).next_u64(STEP_T) % np.uint64(spec.n_vocab)).astype(np.int32)
    pos = np.arange(STEP_T - STEP_N - 1, STEP_T - 1, dtype=np.int32)
    tok = tokens[STEP_T - STEP_N:].copy()
    wts = np.full(STEP_N, 1.0 / STEP_N, np.float32)

    def model_of(n_layer: int):
        sp = G.SyntheticSpec.preset("qwen3-0.6b", G.GGML_Q4_0)
        sp.n_layer = n_layer
        g = G.GgufFile.from_bytes(sp.build(workers=threads))
        return oracle_model(g, adapters(g, STEP_R, STEP_ALPHA), STEP_ALPHA), g

    small, gs = model_of(2)
    timed_runs(lambda: O.model_forward_backward(small, tokens, pos, tok, wts, nthreads=threads), 1, 0, threads)
    del small, gs
    full = oracle_model(g, adapters(g, STEP_R, STEP_ALPHA), STEP_ALPHA)  # the GPU step's own GGUF image
    ts = timed_runs(lambda: O.model_forward_backward(full, tokens, pos, tok, wts, nthreads=threads), 0, 3, threads)
    med = statistics.median(ts)
    return {"value": round(STEP_T / med, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": O.cpu_model(), "host": host_info(),
            "method": "threads pinned one per CPU (sched_setaffinity), AVX2 + FMA build (-march=x86-64-v3), one "
                      "warm-up step of a 2-block cut of the model, then the median of 3 full steps",
            "runs_s": [round(t, 2) for t in ts],
            "sample": f"configs[2] whole: the oracle's Model::forward_backward over all {spec.n_layer} blocks and the "
                      f"head, {STEP_T} tokens, loss on the last {STEP_N}, LoRA r={STEP_R} on every projection "
                      f"(oracle/rtq_oracle*.c, -O3, OpenMP): {med:.1f} s per step"}


def gguf_load(arg: str) -> None:
    """Load throughput of a synthetic GGUF model: write the file, map and parse it, upload every
    frozen tensor (the loader's ``fz``, src/rie.rs:183, :218-231) with rtq_weight_from_gguf."""
    import tempfile

    import torch

    import rust_trainer_amd as rt
    from rust_trainer_amd import gguf as G

    preset, _, wt = arg.partition(":")
    spec = G.SyntheticSpec.preset(preset, G.GGML_NAMES[wt or "Q4_0"])
    assert spec is not None, f"unknown preset {preset}; one of {list(G.SyntheticSpec.PRESETS)}"
    t0 = time.perf_counter()
    w = spec.writer()
    build_s = time.perf_counter() - t0
    print(f"[gguf-load] built {preset} in {build_s:.1f} s", file=sys.stderr, flush=True)
    ctx = rt.Context(0)
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "model.gguf")
        t0 = time.perf_counter()
        w.write(path)
        write_s = time.perf_counter() - t0
        w.close()
        size = os.path.getsize(path)
        t0 = time.perf_counter()
        g = G.GgufFile.open(path)
        open_s = time.perf_counter() - t0
        frozen = [t for t in g.tensors() if not t.name.endswith("norm.weight")]
        per_type: dict = {}
        weights = []
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for t in frozen:
            weights.append(rt.HipFrozen.from_gguf(g, t.name, ctx=ctx))
            per_type[t.ty] = per_type.get(t.ty, 0) + t.nbytes
        torch.cuda.synchronize()
        upload_s = time.perf_counter() - t0
        fbytes = sum(t.nbytes for t in frozen)
        for x in weights:
            x.close()
        g.close()
    ctx.close()
    print(json.dumps({
        "metric": "GGUF load: frozen-tensor bytes uploaded per second (map + parse + repack + host-to-device)",
        "value": round(fbytes / (open_s + upload_s) / 1e9, 3), "unit": "GB/s", "higher_is_better": True,
        "n_gpus": 1, "data": "synthetic",
        "config": {"workload": f"SyntheticSpec::preset({preset}, {wt or 'Q4_0'}) (configs[2] shapes for qwen3-0.6b)",
                   "file_bytes": size, "frozen_tensors": len(frozen), "frozen_bytes": fbytes,
                   "bytes_by_type": {str(k): v for k, v in per_type.items()}},
        "open_ms": round(open_s * 1e3, 3), "upload_ms": round(upload_s * 1e3, 1),
        "write_GBps": round(size / write_s / 1e9, 3), "build_s": round(build_s, 1),
    }), flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 20; --linear 200)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (default 3; --linear 20)")
    ap.add_argument("--sets", type=int, default=40, help="rotating operand sets (~10 MB each)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--title", default=None, help="--counters-report: the table's title")
    ap.add_argument("--sweep", action="store_true", help="configs[1] sweep: one JSON line per case")
    ap.add_argument("--case", default=None, help="one sweep case FMT:SHAPE:T, e.g. Q4_K:lm_head:1")
    ap.add_argument("--calls", type=int, default=50, help="sweep: calls per timed graph (at least the sets)")
    ap.add_argument("--traffic", action="store_true", help="config-1 steps + calibration copies for --pmc passes")
    ap.add_argument("--traffic-report", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"))
    ap.add_argument("--counters-report", nargs=4, metavar=("SQ_DIR", "FETCH_DIR", "WRITE_DIR", "OUT_MD"),
                    help="per-kernel counter table (SQ pass + traffic passes) -> profiles/OUT_MD")
    ap.add_argument("--attention", choices=("fused", "unfused"), default=None,
                    help="training-step benches: force the fused or the unfused attention kernels")
    ap.add_argument("--traffic-step", action="store_true",
                    help="configs[2] steps + calibration copies for --pmc passes (with --traffic-report: the step)")
    ap.add_argument("--head", action="store_true", help="configs[2] LM head + cross-entropy (Model::head)")
    ap.add_argument("--model", action="store_true", help="configs[2] step details only (no contract fields)")
    ap.add_argument("--linear", action="store_true", help="configs[0]: one frozen linear, forward + backward")
    ap.add_argument("--config", type=int, default=None, metavar="I",
                    help="BASELINE.json configs[I] for I = 3 (Qwen3-4B packed) or 4 (Llama-3-8B, recomputed): one "
                         "JSON line (configs[0] is --linear, configs[1] --sweep, configs[2] the default line)")
    ap.add_argument("--gguf-load", default=None, metavar="PRESET[:WTYPE]",
                    help="GGUF load throughput of a synthetic model, e.g. qwen3-0.6b:Q4_0")
    args = ap.parse_args()
    linear_mode = args.linear or args.traffic or args.sweep or bool(args.case) or args.head
    big = args.config in (3, 4)
    if args.steps is None:
        args.steps = 200 if linear_mode else (3 if big else 20)
    if args.warmup is None:
        args.warmup = 20 if linear_mode else (1 if big else 3)
    global ATTENTION_MODE
    if args.attention:
        ATTENTION_MODE = args.attention == "fused"
    if args.counters_report:
        sq_d, f_d, w_d, out_md = args.counters_report
        title = args.title or ("configs[2] training step: counters per kernel" if args.traffic_step
                               else "configs[0] Linear forward + backward: counters per kernel")
        counters_report(sq_d, None if f_d == "-" else f_d, None if w_d == "-" else w_d, title, out_md)
        return 0
    if args.traffic_report:
        traffic_report(*args.traffic_report, step=args.traffic_step)
        return 0
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build runs the hot path on one GPU only; --gpus {args.gpus} "
              f"(WORLD_SIZE={world}) is not supported (the multi-GPU sharding is design-only)", file=sys.stderr)
        return 2
    if args.traffic:
        traffic_run()
        return 0
    if args.traffic_step:
        traffic_run_step()
        return 0
    if args.gguf_load:
        gguf_load(args.gguf_load)
        return 0
    if args.config is not None:
        if args.config == 2:
            print(json.dumps(step_line(args)), flush=True)
        else:
            print(json.dumps(config_bench(args.config, args.steps, args.warmup)), flush=True)
        return 0
    if args.head:
        head_bench(args.steps, args.warmup, args.cpu_seconds, args.no_cpu)
        return 0
    if args.model:
        print(json.dumps(model_bench(args.steps, args.warmup, args.cpu_seconds, args.no_cpu)), flush=True)
        return 0
    if not args.linear and not args.sweep and not args.case:
        print(json.dumps(step_line(args)), flush=True)
        return 0
    if args.sweep or args.case:
        if args.case:
            fmt, shape, t = args.case.split(":")
            cases = [(fmt, shape, int(t))]
        else:
            cases = [(f, s, t) for f in ("Q8_0", "Q4_K", "Q6_K", "Q4_0") for s in SWEEP_SHAPES for t in SWEEP_T]
        sweep(cases, args.calls)
        return 0

    import numpy as np
    import torch

    import rust_trainer_amd as rt
    from rust_trainer_amd import _ffi, synth

    W = synth.Rng(1).vec_normal(N * K, 0.02).reshape(N, K)
    X = synth.Rng(2).vec_normal(T * K, 1.0).reshape(T, K)
    DY = synth.Rng(3).vec_normal(T * N, 1.0).reshape(T, N)
    A = synth.Rng(4).vec_normal(R * K, 1.0 / 32.0).reshape(R, K)
    B = synth.Rng(5).vec_normal(N * R, 0.01).reshape(N, R)
    blocks = synth.quantize_q4_0(W)

    dev = torch.device("cuda", 0)
    ctx = rt.Context(0)
    ctx.reserve(T, N, K, R)
    sets = []
    for _ in range(args.sets):
        s = {
            "w": rt.HipFrozen(rt.TYPE_Q4_0, blocks, N, K, ctx=ctx),
            "x": torch.from_numpy(X).to(dev), "dy": torch.from_numpy(DY).to(dev),
            "y": torch.empty(T, N, device=dev), "dx": torch.empty(T, K, device=dev),
            "a": torch.from_numpy(A).to(dev), "b": torch.from_numpy(B).to(dev),
            "ga": torch.zeros(R, K, device=dev), "gb": torch.zeros(N, R, device=dev),
        }
        s["lora"] = _ffi.RtqLora(R, ALPHA, s["a"].data_ptr(), s["b"].data_ptr(), 1)
        sets.append(s)
    torch.cuda.synchronize()
    L = _ffi.lib()
    # all work goes to one side stream, captured into HIP graphs (torch.cuda.CUDAGraph): the step's
    # five kernels are launched back to back by the GPU, without host launch gaps
    side = torch.cuda.Stream()

    def step(i: int, stream: int) -> None:
        s = sets[i % len(sets)]
        lp = ctypes.byref(s["lora"])
        _ffi.check(L.rtq_linear_forward_d(ctx.handle, s["w"].handle, None, lp, s["x"].data_ptr(), T,
                                          s["y"].data_ptr(), stream), "forward")
        _ffi.check(L.rtq_linear_backward_d(ctx.handle, s["w"].handle, lp, s["x"].data_ptr(), s["dy"].data_ptr(), T,
                                           s["dx"].data_ptr(), s["ga"].data_ptr(), s["gb"].data_ptr(), stream),
                   "backward")

    def capture(nsteps: int) -> "torch.cuda.CUDAGraph":
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            st = torch.cuda.current_stream().cuda_stream
            for i in range(nsteps):
                step(i, st)
        return g

    with torch.cuda.stream(side):
        st = torch.cuda.current_stream().cuda_stream
        for i in range(args.warmup):
            step(i, st)
    torch.cuda.synchronize()

    # per-kernel durations: HIP events recorded by the library around every launch, on the launch
    # stream, in an eager pass (event records are not captured into graphs); then the dominant
    # kernel alone, with events around its launches only
    def eager(nsteps: int) -> None:
        with torch.cuda.stream(side):
            st = torch.cuda.current_stream().cuda_stream
            for i in range(nsteps):
                step(i, st)
        torch.cuda.synchronize()

    ctx.set_timing(True)
    ctx.reset_timing()
    eager(args.steps)
    per = {name: (cnt, ms) for name, (cnt, ms) in ctx.timing().items()}
    dominant = max(per, key=lambda k: per[k][1])
    ctx.set_timing(True, dominant)
    ctx.reset_timing()
    eager(args.steps)
    dom_cnt, dom_ms = ctx.timing()[dominant]
    ctx.set_timing(False)

    # timed region: exactly K steps, one graph replay, no events inside
    g = capture(args.steps)
    g.replay()  # warm replay
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    ms_per_step = elapsed * 1e3 / args.steps

    result = {
        "metric": METRIC,
        "value": round(T / (ms_per_step * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{ARITH_FWD}; {ARITH_DX}; f32 MFMA (LoRA)",
        "data": "synthetic",
        "config": {"workload": "configs[0]: Qwen3-0.6B gate_proj frozen linear, Q4_0 W 3072x1024, T=256, "
                               "LoRA r=16 alpha=32; Linear forward (y) + backward (dx, dA, dB)",
                   "rows": N, "cols": K, "tokens": T, "rank": R, "operand_sets": args.sets},
        "roofline": roofline(dominant, dom_ms / dom_cnt),
        "kernels": {k: {"avg_us": round(ms * 1e3 / c, 3),
                        "frac": roofline(k, ms / c)["frac"] if kernel_work(k) else None}
                    for k, (c, ms) in sorted(per.items())},
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline((blocks, X, DY, A, B), args.cpu_seconds)
    for s in sets:
        s["w"].close()
    ctx.close()
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
