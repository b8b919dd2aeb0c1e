"""Benchmark of the matmul hot path on one MI355X.

Workload: every contraction of one TINY training step, forward and backward,
FP32 (4 layers, hidden 256, 4 heads x 64, SwiGLU FFN 688, untied vocab 16384, batch 16 x seq 256):
115 dense-equivalent GEMMs = 195.82 GFLOP, issued by irontensor_amd.step.GemmStep as 51 GEMMs
(fused QKV and gate|up) in 39 launches (each layer's four weight-gradient GEMMs as one grouped
launch, it_gemm_group) plus the fused attention kernels (forward, and the one-kernel dQ + dK/dV
backward after its row pass, per layer), captured once into a HIP graph and replayed on one
stream. A "step" is one replay; inputs are
resident in HBM before timing starts. The same step with the weight gradients on a second stream
is timed beside it (config.ms_per_step_side_stream).

Prints ONE JSON line (rank 0 = this process). Extra figures (configs 1, 3, 4 and 5: the FP32 QKV
projection, BF16 attention, the medium BF16 step, the BF16 square and decode GEMMs) go under
"extra". The CPU baseline is the oracle's reference loop on host cores over a bounded sample of the
same workload.

`--kernel-only` runs just a calibration copy (f32 -> bf16 conversion of a known size) and the
dominant TINY kernel, for `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE` runs that give the
`roofline.traffic` figure (read back from profiles/tiny_dominant_kernel_traffic.md).
"""
from __future__ import annotations

import argparse
import ctypes as C
import hashlib
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_TFLOPS = {"f32": 157.3, "bf16": 2500.0}
PEAK_HBM_GBS = 8000.0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def parse_key_flops(key: str) -> float:
    """FLOPs of one launch from a profiler key '...|tag[M,N,K]xB s..' (x2 for the SwiGLU dual-B); a
    grouped launch's key lists every call, '...|tag[M,N,K]+[M,N,K]+...x1 s..', and counts their sum."""
    body = key.split("|", 1)[-1]
    m = re.search(r"\]x(\d+)", body)
    trips = re.findall(r"\[(\d+),(\d+),(\d+)\]", body)
    if not m or not trips:
        return 0.0
    B = int(m.group(1))
    total = sum(2.0 * int(M) * int(N) * int(K) for M, N, K in trips)
    return total * B * (2 if "_swiglu" in key else 1)


def profiler_stats(ctx) -> dict:
    from irontensor_amd import profiler
    return profiler.stats(ctx)


class Timer:
    """hipEvents on the library's stream (the stream every kernel is launched on)."""

    def __init__(self, ctx):
        self.ctx = ctx
        self.a, self.b = C.c_void_p(), C.c_void_p()
        ctx.lib.it_event_create(ctx.handle, C.byref(self.a))
        ctx.lib.it_event_create(ctx.handle, C.byref(self.b))

    def start(self):
        self.ctx.lib.it_event_record(self.ctx.handle, self.a)

    def stop_ms(self) -> float:
        self.ctx.lib.it_event_record(self.ctx.handle, self.b)
        self.ctx.lib.it_event_sync(self.b)
        ms = C.c_float()
        self.ctx.lib.it_event_elapsed_ms(self.a, self.b, C.byref(ms))
        return float(ms.value)


class StepEvents:
    """One hipEvent before each of `n` steps and one after the last, on the library's stream: the
    per-step durations of a timed run without extra synchronisation inside it."""

    def __init__(self, ctx, n: int):
        self.ctx = ctx
        self.ev = [C.c_void_p() for _ in range(n + 1)]
        for e in self.ev:
            ctx.lib.it_event_create(ctx.handle, C.byref(e))

    def mark(self, i: int) -> None:
        self.ctx.lib.it_event_record(self.ctx.handle, self.ev[i])

    def durations_ms(self) -> list:
        self.ctx.lib.it_event_sync(self.ev[-1])
        out = []
        for a, b in zip(self.ev, self.ev[1:]):
            ms = C.c_float()
            self.ctx.lib.it_event_elapsed_ms(a, b, C.byref(ms))
            out.append(float(ms.value))
        return out

    def close(self) -> None:
        for e in self.ev:
            self.ctx.lib.it_event_destroy(e)


def time_gemm(it, timer, a, b, out, trans_a, trans_b, iters, warm=3) -> float:
    for _ in range(warm):
        it.gemm(a, b, trans_a=trans_a, trans_b=trans_b, out=out)
    it.Context.global_().sync()
    timer.start()
    for _ in range(iters):
        it.gemm(a, b, trans_a=trans_a, trans_b=trans_b, out=out)
    return timer.stop_ms() / iters


def _bf16(it, x):
    return it.Tensor.from_f32_as_bf16(x, list(x.shape))


def _dev(it, seed, shape, std=1.0, prec=None):
    """Seeded N(0, std^2) device tensor (synth.normal's stream, drawn on the GPU)."""
    from irontensor_amd import synth
    return synth.normal_tensor(seed, list(shape), std=std, precision=prec if prec is not None else it.Precision.FP32)


def extra_config1(it, timer) -> dict:
    """Config 1: the FP32 QKV projection Y = X.W^T, X [4096,256], W [768,256]."""
    from irontensor_amd import synth
    x = it.Tensor.from_f32_slice(synth.normal(1, (4096, 256)), [4096, 256])
    w = it.Tensor.from_f32_slice(synth.normal(2, (768, 256), std=0.02), [768, 256])
    y = it.Tensor.empty([4096, 768])
    ms = time_gemm(it, timer, x, w, y, False, True, 50)
    tf = 2 * 4096 * 768 * 256 / (ms * 1e-3) / 1e12
    return {"config1_fp32_qkv_4096x768x256_NT": {"ms": round(ms, 5), "tflops": round(tf, 2),
                                                 "frac_fp32_peak": round(tf / PEAK_TFLOPS["f32"], 4)}}


def extra_attention(it, timer) -> dict:
    """Config 3: BF16 attention, Q, K, V, dO [16,8,1024,64], causal, scale 1/8. The fused kernels
    (forward; backward from the saved O and row log-sum-exp) next to the materialised five-GEMM
    form. FLOPs are dense-equivalent (2 GEMMs forward, 5 backward, 2*BH*S*S*D each); the causal
    useful fraction is (S+1)/(2S)."""
    from irontensor_amd import synth
    b, h, s, d = 16, 8, 1024, 64
    q, k, v, do = (_dev(it, 30 + i, (b, h, s, d), prec=it.Precision.BF16) for i in range(4))
    ctx = it.Context.global_()

    def run(fn, iters):
        fn()
        ctx.sync()
        timer.start()
        for _ in range(iters):
            fn()
        return timer.stop_ms() / iters

    o, lse = it.flash_attention_forward_bhsd(q, k, v, causal=True, scale=0.125)
    f_ms = run(lambda: it.flash_attention_forward_bhsd(q, k, v, causal=True, scale=0.125), 10)
    b_ms = run(lambda: it.flash_attention_backward(do, q, k, v, causal=True, scale=0.125, o=o, lse=lse), 5)
    mf_ms = run(lambda: it.attention_forward_bhsd(q, k, v, causal=True, scale=0.125), 3)
    mb_ms = run(lambda: it.attention_backward_recompute(do, q, k, v, causal=True, scale=0.125), 3)
    unit = 2.0 * b * h * s * s * d
    useful = (s + 1) / (2 * s)
    res = {}
    for name, ms, n in (("fused_forward", f_ms, 2), ("fused_backward", b_ms, 5),
                        ("materialised_forward", mf_ms, 2), ("materialised_backward_recompute", mb_ms, 7)):
        tf = n * unit / (ms * 1e-3) / 1e12
        res[name] = {"ms": round(ms, 4), "tflops_dense_equiv": round(tf, 1),
                     "tflops_useful": round(tf * useful, 1),
                     "frac_bf16_peak_useful": round(tf * useful / PEAK_TFLOPS["bf16"], 4)}
    res["useful_fraction"] = round(useful, 5)
    res["torch_sdpa_same_run"] = (sdpa_library(b, h, s, d, unit * useful) if TORCH_STATE["ready"]
                                  else {"skipped": TORCH_STATE["error"] or "torch not initialised first"})
    return {"config3_bf16_attention_16x8x1024x64_causal": res}


def sdpa_library(b: int, h: int, s: int, d: int, useful_unit: float) -> dict:
    """PyTorch's fused attention on the same box and in the same process, for comparison: causal
    scaled_dot_product_attention (scale 1/8) on BF16 [b, h, s, d] with the flash and the
    memory-efficient backends only (the math backend, batched BF16 products on a transposed K, is
    never selected). Forward timed alone, backward as forward + backward minus forward; TFLOP/s on
    the same useful-FLOP count as the fused kernels (2 and 5 GEMMs of 2*B*H*S*S*D times the
    causal fraction)."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    g = torch.Generator(device="cuda:0")
    g.manual_seed(0)
    q, k, v, do = (torch.randn(b, h, s, d, device="cuda:0", dtype=torch.bfloat16, generator=g) for _ in range(4))
    for t in (q, k, v):
        t.requires_grad_(True)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, iters):
        fn()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / iters

    out = {}
    for name, backend in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel([backend]):
                fwd = lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=0.125)  # noqa: E731

                def fwd_bwd():
                    q.grad = k.grad = v.grad = None
                    fwd().backward(do)

                f_ms = timed(fwd, 10)
                b_ms = timed(fwd_bwd, 5) - f_ms
            out[name] = {"forward_ms": round(f_ms, 4), "forward_tflops_useful": round(2 * useful_unit / f_ms / 1e9, 1),
                         "backward_ms": round(b_ms, 4),
                         "backward_tflops_useful": round(5 * useful_unit / b_ms / 1e9, 1)}
        except RuntimeError as e:  # the backend is not built for this device
            out[name] = f"unavailable: {str(e)[:160]}"
    del q, k, v, do
    torch.cuda.empty_cache()
    return out


def attention_only(it, timer, reps: int) -> dict:
    """The fused attention kernels alone: config 3 (BF16 [16,8,1024,64]) and the TINY step's FP32
    shape ([16,4,256,64]), causal, forward then backward from the saved O and LSE, `reps` times."""
    P = it.Precision
    out = {}
    for (b, h, s, prec) in ((16, 8, 1024, P.BF16), (16, 4, 256, P.FP32)):
        q, k, v, do = (_dev(it, 30 + i, (b, h, s, 64), prec=prec) for i in range(4))
        it.Context.global_().sync()
        timer.start()
        for _ in range(reps):
            o, lse = it.flash_attention_forward_bhsd(q, k, v, causal=True, scale=0.125)
            it.flash_attention_backward(do, q, k, v, causal=True, scale=0.125, o=o, lse=lse)
        out[f"{prec.name.lower()}_{b}x{h}x{s}x64_fwd_bwd_ms"] = round(timer.stop_ms() / max(1, reps), 4)
    return out


def extra_med_step(it, timer, steps=5, warmup=2) -> dict:
    """Config 4: the medium BF16 step (12 layers, hidden 1024, 16 x 64 heads, SwiGLU FFN 2816 with
    the fused bias + SwiGLU epilogue, vocab 32768, batch 8 x seq 1024): every contraction forward
    and backward, graph-replayed on one stream (each layer's weight gradients as one grouped
    launch), and the same step with the weight gradients on a second stream. Per-kernel times come
    from one eager step on one stream."""
    from irontensor_amd.step import MEDIUM, GemmStep
    ctx = it.Context.global_()
    step = GemmStep(MEDIUM, it.Precision.BF16, ctx, ffn_bias=True)

    def timed(overlap: bool) -> float:
        step.close()
        step.overlap = overlap
        step.enqueue()
        step.capture()
        for _ in range(warmup):
            step.replay()
        ctx.sync()
        timer.start()
        for _ in range(steps):
            step.replay()
        return timer.stop_ms() / steps

    try:
        step.enqueue()
        ctx.sync()
        flops = step.flops()
        ms2 = timed(True)
        ms = timed(False)
        ctx.lib.it_profiler_reset(ctx.handle)
        ctx.lib.it_profiler_enable(ctx.handle, 1)
        step.enqueue()
        stats = profiler_stats(ctx)
        ctx.lib.it_profiler_enable(ctx.handle, 0)
    finally:
        step.close()
    top = sorted(stats.items(), key=lambda kv: -kv[1]["total_ms"])[:10]
    tf = flops / (ms * 1e-3) / 1e12
    return {"config4_bf16_medium_step": {
        "ms_per_step": round(ms, 3), "ms_per_step_side_stream": round(ms2, 3), "streams": 1,
        "gflop_per_step": round(flops / 1e9, 1), "tflops": round(tf, 1),
        "frac_bf16_peak": round(tf / PEAK_TFLOPS["bf16"], 4), "steps": steps,
        "eager_single_stream_kernel_ms": round(sum(v["total_ms"] for v in stats.values()), 3),
        "top_kernels": [{"key": k, "ms_per_step": round(v["total_ms"], 3), "calls": v["calls"]} for k, v in top]}}


def bf16_square(it, timer, sizes) -> dict:
    """BF16 n^3 GEMMs, NN/NT/TN, BF16 out: the median of three batches of `iters` timed launches
    each ((n, iters) in `sizes`); single batches moved by up to 15% with the clock."""
    from irontensor_amd import synth
    P = it.Precision
    out = {}
    for n, iters in sizes:
        a = _dev(it, 3, (n, n), prec=P.BF16)
        b = _dev(it, 4, (n, n), prec=P.BF16)
        c = it.Tensor.empty([n, n], P.BF16)
        for lay, (ta, tb) in (("NN", (False, False)), ("NT", (False, True)), ("TN", (True, False))):
            ms = sorted(time_gemm(it, timer, a, b, c, ta, tb, iters, warm=2) for _ in range(3))[1]
            tf = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
            out[f"bf16_square_{n}_{lay}"] = {"ms": round(ms, 4), "tflops": round(tf, 1),
                                             "frac_bf16_peak": round(tf / PEAK_TFLOPS["bf16"], 4)}
        del a, b, c
    return out


def vs_library(it, timer, sizes=((1024, 50), (2048, 30), (4096, 20), (8192, 6))) -> dict:
    """The BF16 n^3 GEMM against AMD's library in the same process: torch.mm on BF16 [n, n] tensors
    (served by hipBLASLt) in the NN, NT and TN layouts (the transposed operand a 2-D transposed view,
    which the library reads in place), then this library's NN, NT and TN forms on its own seeded
    operands; three batches of `iters` launches each, TFLOP/s per batch. BF16 out."""
    import torch
    dev = torch.device("cuda:0")
    P = it.Precision
    res = {}
    for n, iters in sizes:
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        a = torch.randn(n, n, device=dev, dtype=torch.bfloat16, generator=g)
        b = torch.randn(n, n, device=dev, dtype=torch.bfloat16, generator=g)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        tf = lambda ms: round(2.0 * n ** 3 / (ms * 1e-3) / 1e12, 1)  # noqa: E731
        out = {}
        for lay, (x, y) in (("NN", (a, b)), ("NT", (a, b.t())), ("TN", (a.t(), b))):
            for _ in range(3):
                torch.mm(x, y)
            torch.cuda.synchronize()
            out[f"hipblaslt_torch_mm_{lay}"] = []
            for _ in range(3):
                e0.record()
                for _ in range(iters):
                    torch.mm(x, y)
                e1.record()
                torch.cuda.synchronize()
                out[f"hipblaslt_torch_mm_{lay}"].append(tf(e0.elapsed_time(e1) / iters))
        del a, b
        torch.cuda.empty_cache()
        A, B = _dev(it, 3, (n, n), prec=P.BF16), _dev(it, 4, (n, n), prec=P.BF16)
        Cm = it.Tensor.empty([n, n], P.BF16)
        for lay, (ta, tb) in (("NN", (False, False)), ("NT", (False, True)), ("TN", (True, False))):
            out[f"this_{lay}"] = [tf(time_gemm(it, timer, A, B, Cm, ta, tb, iters, warm=3)) for _ in range(3)]
        del A, B, Cm
        res[f"bf16_{n}_vs_library_tflops"] = out
    return res


F32_LM_HEAD = (("forward_NT", 4096, 16384, 256, False, True), ("data_grad_NN", 4096, 256, 16384, False, False),
               ("weight_grad_TN", 16384, 256, 4096, True, False))


def vs_library_f32(it, timer, iters: int = 10) -> dict:
    """The TINY step's three FP32 LM-head GEMMs against AMD's library in the same process: torch.mm
    on FP32 tensors (hipBLASLt; the transposed operand a 2-D transposed view, TF32 off), then this
    library's own GEMM on seeded operands of the same layout; three batches of `iters` launches each,
    microseconds per launch per batch."""
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    dev = torch.device("cuda:0")
    res = {}
    for name, m, n, k, ta, tb in F32_LM_HEAD:
        g = torch.Generator(device=dev)
        g.manual_seed(0)
        a = torch.randn(*((k, m) if ta else (m, k)), device=dev, generator=g)
        b = torch.randn(*((n, k) if tb else (k, n)), device=dev, generator=g)
        x, y = (a.t() if ta else a), (b.t() if tb else b)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(3):
            torch.mm(x, y)
        torch.cuda.synchronize()
        lib_us = []
        for _ in range(3):
            e0.record()
            for _ in range(iters):
                torch.mm(x, y)
            e1.record()
            torch.cuda.synchronize()
            lib_us.append(round(e0.elapsed_time(e1) / iters * 1e3, 1))
        del a, b, x, y
        torch.cuda.empty_cache()
        A = _dev(it, 3, (k, m) if ta else (m, k))
        B = _dev(it, 4, (n, k) if tb else (k, n))
        Cm = it.Tensor.empty([m, n])
        this_us = [round(time_gemm(it, timer, A, B, Cm, ta, tb, iters) * 1e3, 1) for _ in range(3)]
        del A, B, Cm
        fl = 2.0 * m * n * k
        res[f"f32_lm_head_{name}_{m}x{n}x{k}"] = {
            "hipblaslt_torch_mm_us": lib_us, "this_us": this_us,
            "hipblaslt_tflops_best": round(fl / (min(lib_us) * 1e-6) / 1e12, 1),
            "this_tflops_best": round(fl / (min(this_us) * 1e-6) / 1e12, 1)}
    return res


def extra_sweep(it, timer) -> dict:
    """Config 5: BF16 square GEMMs n^3, n in {1024 .. 16384}, NN/NT/TN, BF16 out; and the decode
    shapes (decode_shapes)."""
    out = bf16_square(it, timer, ((1024, 50), (2048, 30), (4096, 20), (8192, 8), (16384, 3)))
    out.update(decode_shapes(it, timer))
    return out


def decode_shapes(it, timer, rounds: int = 4) -> dict:
    """Config 5b: the decode shapes M in {1, 4, 16}, K 4096, N 11008 in the NT (W [N, K]), NN and TN
    (W [K, N]) layouts, BF16 in and out (HBM-bound: bytes / time against 8 TB/s). The timing rotates
    over DECODE_COPIES distinct weight copies (8 x 90 MB, more than the 256 MB Infinity Cache), so
    every call streams its weight from HBM; `rounds` passes over the copies are timed. Operands
    are seeded N(0,1)."""
    P = it.Precision
    out = {}
    k, n = 4096, 11008
    copies = DECODE_COPIES
    w_nk = [_dev(it, 500 + c, (n, k), prec=P.BF16) for c in range(copies)]
    w_kn = [_dev(it, 600 + c, (k, n), prec=P.BF16) for c in range(copies)]
    ctx = it.Context.global_()
    for m in (1, 4, 16):
        xa = _dev(it, 6, (m, k), prec=P.BF16)
        xt = _dev(it, 8, (k, m), prec=P.BF16)
        yo = it.Tensor.empty([m, n], P.BF16)
        for lay, (A, Bs, ta, tb) in (("NT", (xa, w_nk, False, True)), ("NN", (xa, w_kn, False, False)),
                                     ("TN", (xt, w_kn, True, False))):
            for c in range(copies):
                it.gemm(A, Bs[c], trans_a=ta, trans_b=tb, out=yo)
            ctx.sync()
            iters = rounds * copies
            timer.start()
            for i in range(iters):
                it.gemm(A, Bs[i % copies], trans_a=ta, trans_b=tb, out=yo)
            ms = timer.stop_ms() / iters
            gbs = (n * k * 2 + m * k * 2 + m * n * 2) / (ms * 1e-3) / 1e9
            out[f"bf16_decode_m{m}_k4096_n11008_{lay}"] = {"ms": round(ms, 5), "GBps": round(gbs, 1),
                                                           "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4),
                                                           "weights": f"{copies} copies rotated (cold in L2/MALL)"}
    return out


DECODE_COPIES = 8


def train_step_figures(it, timer, steps: int, warmup: int) -> dict:
    """The complete TINY training step (irontensor_amd.train.TrainStep): embedding, 4 layers with
    RMSNorm, RoPE and fused attention, final norm, LM head, fused cross entropy, the backward pass,
    the global-norm clip and Lion, graph-replayed. Per-kernel shares from one eager profiled step."""
    from irontensor_amd.step import TINY
    from irontensor_amd.train import TrainStep
    ctx = it.Context.global_()
    st = TrainStep(TINY, ctx)
    try:
        st.step()
        ctx.sync()
        loss0 = st.loss_value()
        st.capture()
        for _ in range(warmup):
            st.step()
        ctx.sync()
        t0 = time.perf_counter()
        timer.start()
        for _ in range(steps):
            st.step()
        ev_ms = timer.stop_ms() / steps
        ctx.sync()
        wall_ms = (time.perf_counter() - t0) * 1e3 / steps
        loss1, gnorm = st.loss_value(), st.grad_norm()
        ctx.lib.it_profiler_reset(ctx.handle)
        ctx.lib.it_profiler_enable(ctx.handle, 1)
        st.enqueue()
        stats = profiler_stats(ctx)
        ctx.lib.it_profiler_enable(ctx.handle, 0)
    finally:
        st.close()
    total = sum(v["total_ms"] for v in stats.values())
    groups = {}
    for k, v in stats.items():
        g = k.split("|")[0].split("[")[0]
        g = "gemm" if g.startswith("gemm") or g.startswith("gemv") else g
        groups[g] = groups.get(g, 0.0) + v["total_ms"]
    return {"ms_per_step": round(wall_ms, 4), "ms_per_step_events": round(ev_ms, 4),
            "tokens_per_s": round(TINY.tokens / (wall_ms * 1e-3), 0), "steps": steps, "warmup": warmup,
            "loss_first": round(loss0, 4), "loss_last": round(loss1, 4), "grad_norm_last": round(gnorm, 4),
            "gemm_tflops_in_step": round(st.gemm_flops() / (wall_ms * 1e-3) / 1e12, 2),
            "eager_kernel_ms_by_group": {k: round(v, 4) for k, v in sorted(groups.items(), key=lambda kv: -kv[1])},
            "eager_kernel_ms_total": round(total, 4),
            "optimizer": "Lion lr 3e-4 betas (0.9, 0.99) wd 0.1, clip 1.0 (src/bin/benchmark.rs:124-129)",
            "execution": "one hipGraph per step on one stream; each layer's weight gradients as one grouped launch; "
                         "loss, norm and clip stay on the GPU"}


def extra_fusions(it, timer, iters: int = 10) -> dict:
    """The reference's GEMM prologue/epilogue fusions against the unfused ops, at the TINY step's
    shapes: RMSNorm -> Q|K|V projection ([4096, 256] -> 768) and the LM head with cross entropy
    ([4096, 256] x [16384, 256]^T, loss + grad_hidden + grad_weight), one vocabulary chunk (the
    default 256 MiB budget) and four (64 MiB)."""
    from irontensor_amd import synth, train_ops as T
    P = it.Precision
    out = {}

    def run(fn):
        fn()
        it.Context.global_().sync()
        timer.start()
        for _ in range(iters):
            fn()
        return timer.stop_ms() / iters

    x = _dev(it, 1, (4096, 256))
    g = it.Tensor.from_f32_slice(1 + synth.normal(2, (256,), std=0.1), [256])
    w = _dev(it, 3, (768, 256), std=0.02)
    xn = it.Tensor.empty([4096, 256])
    y = it.Tensor.empty([4096, 768])
    lib, h = it.Context.global_().lib, it.Context.global_().handle

    def unfused():
        lib.it_rmsnorm_forward(h, 0, 4096, 256, 1e-5, C.c_void_p(x.ptr), None, C.c_void_p(g.ptr), None,
                               C.c_void_p(xn.ptr))
        it.gemm(xn, w, trans_b=True, out=y)

    def fused():
        lib.it_fused_rmsnorm_linear(h, 4096, 256, 768, 1e-5, C.c_void_p(x.ptr), C.c_void_p(g.ptr), C.c_void_p(w.ptr),
                                    C.c_void_p(y.ptr))

    out["rmsnorm_qkv_4096x256x768"] = {"unfused_us": round(run(unfused) * 1e3, 2), "fused_us": round(run(fused) * 1e3, 2)}
    hs = _dev(it, 4, (4096, 256))
    E = _dev(it, 5, (16384, 256), std=0.02)
    tg = synth.tokens(6, 4096, 16384)
    t32 = it.Tensor.from_f32_slice(tg.astype(np.int32).view(np.float32), [4096])
    tu = T.upload_ids(tg, 16384)
    logits, dlog = it.Tensor.empty([4096, 16384]), it.Tensor.empty([4096, 16384])
    dh, dw, mean = it.Tensor.empty([4096, 256]), it.Tensor.empty([16384, 256]), it.Tensor.empty([1])

    def lm_unfused():
        it.gemm(hs, E, trans_b=True, out=logits)
        lib.it_cross_entropy_fused(h, 0, 4096, 16384, C.c_void_p(logits.ptr), C.c_void_p(tu.ptr), None,
                                   C.c_void_p(dlog.ptr), C.c_void_p(mean.ptr))
        it.gemm(dlog, hs, trans_a=True, out=dw)
        it.gemm(dlog, E, out=dh)

    def lm_fused(budget):
        def f():
            lib.it_fused_linear_cross_entropy(h, 4096, 256, 16384, C.c_void_p(hs.ptr), C.c_void_p(E.ptr),
                                              C.c_void_p(t32.ptr), None, C.c_void_p(mean.ptr), C.c_void_p(dh.ptr),
                                              C.c_void_p(dw.ptr), budget)
        return f

    out["lm_head_ce_4096x256x16384"] = {
        "unfused_us": round(run(lm_unfused) * 1e3, 1),
        "fused_1chunk_us": round(run(lm_fused(256 << 20)) * 1e3, 1),
        "fused_4chunks_us": round(run(lm_fused(64 << 20)) * 1e3, 1),
        "logits_bytes_unfused": 2 * 4096 * 16384 * 4, "logits_bytes_fused_4chunks": 4096 * 4096 * 4,
        "note": "unfused: logits GEMM, cross entropy, dW and dX GEMMs (logits and dlogits buffers); fused: "
                "chunk GEMM + stats, gradient in place, dW/dX GEMMs per chunk (chunks but the last one recomputed)"}
    return {"fusions": out}


TORCH_STATE = {"ready": False, "error": None}


def init_torch_first() -> None:
    """Lets torch's HIP runtime take the device before this library's context does (the other order
    leaves torch without a visible device), for the same-process library comparison; a failure is
    recorded and the comparison skipped."""
    try:
        import torch
        torch.empty(1, device="cuda:0")
        TORCH_STATE["ready"] = True
    except Exception as e:  # noqa: BLE001 - recorded in the line, the bench goes on without it
        TORCH_STATE["error"] = f"{type(e).__name__}: {e}"[:200]


def extras(it, timer) -> dict:
    out = {}
    for fn in (extra_config1, extra_attention, extra_fusions, extra_sweep, extra_med_step):
        log(f"[bench] extra: {fn.__name__}")
        out.update(fn(it, timer))
    if TORCH_STATE["ready"]:
        log("[bench] extra: vs_library")
        out.update(vs_library(it, timer))
    else:
        out["bf16_4096_vs_library_tflops"] = {"skipped": TORCH_STATE["error"] or "torch not initialised first"}
    return out


TRAFFIC_FILE = ROOT / "profiles" / "tiny_dominant_kernel_traffic.md"


def committed_traffic(key: str):
    """HBM bytes per launch of `key` from the committed rocprofv3 --pmc summary, or None. The file
    holds a line 'traffic_bytes_per_launch <key> = <bytes>'."""
    if not TRAFFIC_FILE.exists():
        return None
    for line in TRAFFIC_FILE.read_text().splitlines():
        m = re.match(r"\s*traffic_bytes_per_launch (.+) = (\d+)\s*$", line)
        if m and m.group(1) == key:
            return int(m.group(2))
    return None


def kernel_only(it, ctx, step, iters: int) -> int:
    """Calibration copy, then each of the step's largest GEMMs (the LM-head forward, dX and dW) and
    the first layer's grouped weight gradients (any of which can be the dominant kernel) `iters`
    times in a row, for rocprofv3 --pmc passes. Prints the order of the groups with their profiler
    keys, to map dispatches back to keys."""
    from irontensor_amd import synth
    n = 1 << 26  # 256 MiB read, 128 MiB written
    src = _dev(it, 9, (n,))
    dst = it.Tensor.empty([n], it.Precision.BF16)
    ctx.sync()
    for _ in range(5):
        if ctx.lib.it_f32_to_bf16(ctx.handle, C.c_void_p(src.ptr), C.c_void_p(dst.ptr), n) != 0:
            raise RuntimeError("conversion failed")
    ctx.sync()
    biggest = max(2.0 * M * N * K for (_, _, M, N, K) in step._calls)
    groups = []
    for (ta, tb, M, N, K) in list(step._calls):
        if 2.0 * M * N * K < 0.9 * biggest:
            continue
        ctx.lib.it_profiler_reset(ctx.handle)
        ctx.lib.it_profiler_enable(ctx.handle, 1)
        for _ in range(iters):
            name = step.reissue(ta, tb, M, N, K)
        stats = profiler_stats(ctx)
        ctx.lib.it_profiler_enable(ctx.handle, 0)
        (key, st), = stats.items()
        groups.append({"key": key, "step_gemm": name, "launches": iters,
                       "avg_us_events": round(st["total_ms"] / st["calls"] * 1e3, 2)})
    # The first layer's weight gradients as the step groups them (one it_gemm_group call).
    ctx.lib.it_profiler_reset(ctx.handle)
    ctx.lib.it_profiler_enable(ctx.handle, 1)
    for _ in range(iters):
        names = step.reissue_group()
    stats = profiler_stats(ctx)
    ctx.lib.it_profiler_enable(ctx.handle, 0)
    for key, st in stats.items():
        groups.append({"key": key, "step_gemm": "+".join(names), "launches": st["calls"],
                       "avg_us_events": round(st["total_ms"] / st["calls"] * 1e3, 2)})
    print(json.dumps({"calibration": {"kernel": "f32_to_bf16_kernel", "elements": n, "read_bytes": 4 * n,
                                      "write_bytes": 2 * n, "launches": 5},
                      "groups": groups}), flush=True)
    return 0


def cpu_baseline(step) -> dict:
    """One complete TINY training step on the oracle (oracle/train_step.py: embedding, layers, final
    norm, LM head, cross entropy, backward, clip, Lion) on host cores; its contractions are the
    reference's sequential f32 loop (oracle/ref.c), row-parallel over all host threads. `value` is
    the contractions' FLOPs over the time spent in them (timed call by call inside the step);
    `train_step_ms` is the whole step. Config 1 is also timed on one thread."""
    import oracle
    from oracle import train_step as ots
    from irontensor_amd import synth
    s = step.s
    H, F, V, L = s.hidden, s.ffn, s.vocab, s.layers
    thr = oracle.default_threads()
    w = lambda sh, seed: synth.normal(seed, sh, std=0.02)  # noqa: E731
    acc = {"t": 0.0, "flops": 0.0}

    def timed(fn, flops_of):
        def run(*a, **k):
            t = time.perf_counter()
            out = fn(*a, **k)
            acc["t"] += time.perf_counter() - t
            acc["flops"] += flops_of(*a, **k)
            return out
        return run

    def gemm_flops(a, b, trans_a=False, trans_b=False, threads=None):
        m, kk = (a.shape[1], a.shape[0]) if trans_a else a.shape
        n = b.shape[0] if trans_b else b.shape[1]
        return 2.0 * m * n * kk

    def attn_flops(n_gemms):
        def f(*a, **k):
            q = a[1] if n_gemms == 5 else a[0]
            bh, sq, d = q.shape
            return n_gemms * 2.0 * bh * sq * sq * d
        return f

    prm = {"emb": w((V, H), 40), "E": w((V, H), 41), "final_norm": np.ones(H, np.float32),
           "attn_norm": [np.ones(H, np.float32)] * L, "ffn_norm": [np.ones(H, np.float32)] * L,
           "Wqkv": [w((3 * H, H), 42 + l) for l in range(L)], "Wo": [w((H, H), 50 + l) for l in range(L)],
           "Wgu": [w((2 * F, H), 60 + l) for l in range(L)], "Wd": [w((H, F), 70 + l) for l in range(L)]}
    mom = [np.zeros_like(x) for x in ots.param_list(prm)]
    stream = synth.tokens(99, s.batch * (s.seq + 1), V).reshape(s.batch, s.seq + 1)
    saved = (ots.gemm_f32, ots.attention_fwd_bhsd, ots.attention_bwd_bhsd)
    ots.gemm_f32 = timed(saved[0], gemm_flops)
    ots.attention_fwd_bhsd = timed(saved[1], attn_flops(2))
    ots.attention_bwd_bhsd = timed(saved[2], attn_flops(5))
    try:
        t0 = time.perf_counter()
        ots.train_step(prm, mom, stream[:, :-1].ravel(), stream[:, 1:].ravel(), s, threads=thr)
        dt = time.perf_counter() - t0
    finally:
        ots.gemm_f32, ots.attention_fwd_bhsd, ots.attention_bwd_bhsd = saved
    # config 1 on one thread, for the per-core figure
    a = lambda sh, seed: synth.normal(seed, sh)  # noqa: E731
    x1, w1 = a((4096, 256), 30), w((768, 256), 31)
    t1 = time.perf_counter()
    oracle.gemm_f32(x1, w1, False, True, threads=1)
    dt1 = time.perf_counter() - t1
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(acc["flops"] / acc["t"] / 1e12, 5), "unit": "TFLOP/s", "cores": thr,
            "host_cpus": os.cpu_count(), "cpu_model": model,
            "config1_one_thread_ms": round(dt1 * 1e3, 1),
            "config1_one_thread_gflops": round(2 * 4096 * 768 * 256 / dt1 / 1e9, 3),
            "kind": "port",
            "sample": (f"one complete TINY training step on the oracle: {acc['flops'] / 1e9:.1f} GFLOP of "
                       f"contractions (linear GEMMs, attention forward and backward, LM head) in "
                       f"{acc['t']:.2f} s of a {dt:.2f} s step; oracle/ref.c sequential f32 loop (no FMA "
                       f"contraction), {thr} threads"),
            "seconds": round(dt, 2),
            "contraction_seconds": round(acc["t"], 2),
            "train_step_ms": round(dt * 1e3, 1)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip the extra GEMM figures")
    ap.add_argument("--kernel-only", action="store_true",
                    help="run only a calibration copy and the dominant kernel (for rocprofv3 --pmc)")
    ap.add_argument("--train-only", action="store_true",
                    help="run only the complete TINY training step, graph-replayed (for kernel traces)")
    ap.add_argument("--bf16-square", action="store_true",
                    help="run only the BF16 4096^3, 8192^3 and 16384^3 GEMMs, NN/NT/TN (for rocprofv3 --pmc)")
    ap.add_argument("--medium-step", action="store_true",
                    help="run only config 4, the medium BF16 step (graph replay, single stream, and one "
                         "profiled eager step; for rocprofv3)")
    ap.add_argument("--vs-library", action="store_true",
                    help="time the BF16 4096^3 GEMM through torch.mm (hipBLASLt) and through this library, "
                         "in one process (for same-box A/B traces and counters)")
    ap.add_argument("--vs-library-f32", action="store_true",
                    help="time the TINY step's three FP32 LM-head GEMMs through torch.mm (hipBLASLt) and through "
                         "this library, in one process, --steps launches per batch (for same-box traces and counters)")
    ap.add_argument("--decode", action="store_true",
                    help="run only the BF16 decode shapes (M 1/4/16, K 4096, N 11008; NT, NN, TN) with cold "
                         "weights, --steps passes over the rotated copies (for rocprofv3)")
    ap.add_argument("--attention", action="store_true",
                    help="run only the fused attention forward + backward, config 3 BF16 [16,8,1024,64] and the "
                         "TINY FP32 shape [16,4,256,64], causal, --steps times each (for rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the kernels run one GPU's shard; sharding across GPUs is not built)", file=sys.stderr)
        return 2
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: launched with WORLD_SIZE > 1; this build runs on one GPU only", file=sys.stderr)
        return 2
    if os.environ.get("IRONTENSOR_LIB") and not (args.attention or args.medium_step or args.bf16_square or args.decode
                                                 or args.vs_library or args.vs_library_f32):
        print("bench.py: IRONTENSOR_LIB is set; the bench times only the in-tree library "
              "(irontensor_amd/libirontensor_hip.so), unset it", file=sys.stderr)
        return 2

    if args.vs_library or args.vs_library_f32 or args.attention or not (
            args.no_extra or args.kernel_only or args.train_only or args.bf16_square or args.medium_step or args.decode):
        init_torch_first()
        if (args.vs_library or args.vs_library_f32) and not TORCH_STATE["ready"]:
            print(f"bench.py: torch could not take the device: {TORCH_STATE['error']}", file=sys.stderr)
            return 1
    import irontensor_amd as it
    from irontensor_amd.step import TINY, GemmStep

    if it.device_count() == 0:
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    ctx = it.Context.global_()
    info = ctx.info()
    log(f"[bench] device {info}")
    from irontensor_amd import _lib
    lib_path = Path(_lib.LIB_PATH).resolve()
    lib_info = {"path": str(lib_path.relative_to(ROOT)) if lib_path.is_relative_to(ROOT) else str(lib_path),
                "sha256": hashlib.sha256(lib_path.read_bytes()).hexdigest()}
    log(f"[bench] library {lib_info}")
    if args.bf16_square:
        print(json.dumps(bf16_square(it, Timer(ctx), ((4096, args.steps), (8192, max(1, args.steps // 4)),
                                                      (16384, max(1, args.steps // 16))))), flush=True)
        return 0
    if args.attention:
        out = attention_only(it, Timer(ctx), args.steps)
        if TORCH_STATE["ready"]:
            out["torch_sdpa_bf16_16x8x1024x64_causal"] = sdpa_library(16, 8, 1024, 64,
                                                                      2.0 * 16 * 8 * 1024 ** 2 * 64 * 1025 / 2048)
        print(json.dumps(out), flush=True)
        return 0
    if args.vs_library:
        print(json.dumps(vs_library(it, Timer(ctx), sizes=((1024, 2 * args.steps), (2048, args.steps), (4096, args.steps),
                                                            (8192, max(2, args.steps // 4))))), flush=True)
        return 0
    if args.vs_library_f32:
        print(json.dumps(vs_library_f32(it, Timer(ctx), iters=args.steps)), flush=True)
        return 0
    if args.decode:
        print(json.dumps(decode_shapes(it, Timer(ctx), rounds=max(1, args.steps))), flush=True)
        return 0
    if args.medium_step:
        print(json.dumps(extra_med_step(it, Timer(ctx), steps=args.steps, warmup=args.warmup)), flush=True)
        return 0
    if args.train_only:
        print(json.dumps({"train_step": train_step_figures(it, Timer(ctx), args.steps, args.warmup)}), flush=True)
        return 0
    step = GemmStep(TINY, it.Precision.FP32, ctx)
    step.enqueue()                      # eager once: records the launch list, sizes scratch
    ctx.sync()
    total_flops = step.flops()
    log(f"[bench] TINY step: {len(step.launches)} contractions, {total_flops / 1e9:.2f} GFLOP")
    if args.kernel_only:
        return kernel_only(it, ctx, step, args.steps)
    step.capture()
    for _ in range(args.warmup):
        step.replay()
    ctx.sync()
    timer = Timer(ctx)
    marks = StepEvents(ctx, args.steps)
    t0 = time.perf_counter()
    timer.start()
    for i in range(args.steps):
        marks.mark(i)
        step.replay()
    marks.mark(args.steps)
    gpu_ms = timer.stop_ms()
    ctx.sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    step_ms = marks.durations_ms()
    marks.close()
    ms_median = float(np.median(step_ms))
    log(f"[bench] timed {args.steps} steps: wall {ms_per_step:.3f} ms/step, events "
        f"{gpu_ms / args.steps:.3f} ms/step, median step {ms_median:.3f} ms")

    # Per-kernel durations: the same steps run eagerly on the same one stream with hipEvents around
    # every launch.
    ctx.lib.it_profiler_reset(ctx.handle)
    ctx.lib.it_profiler_enable(ctx.handle, 1)
    for _ in range(args.steps):
        step.enqueue()
    stats = profiler_stats(ctx)
    ctx.lib.it_profiler_enable(ctx.handle, 0)
    # The same step with each layer's weight-gradient group on the context's side stream, beside
    # the data-gradient chain, graph-replayed and timed the same way.
    step.close()
    step.overlap = True
    step.enqueue()
    step.capture()
    for _ in range(args.warmup):
        step.replay()
    ctx.sync()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step.replay()
    ctx.sync()
    ms_side = (time.perf_counter() - t1) * 1e3 / args.steps
    log(f"[bench] side-stream replay {ms_side:.3f} ms/step")
    step.close()
    step.overlap = False
    gemm_ms = sum(v["total_ms"] for v in stats.values()) / args.steps
    dom_key, dom = max(stats.items(), key=lambda kv: kv[1]["total_ms"])
    avg_ms = dom["total_ms"] / dom["calls"]
    dom_flops = parse_key_flops(dom_key)
    achieved = dom_flops / (avg_ms * 1e-3) / 1e12
    log(f"[bench] dominant kernel {dom_key}: {dom['calls']} calls, avg {avg_ms * 1e3:.1f} us, "
        f"{achieved:.1f} TFLOP/s; sum of GEMM launches {gemm_ms:.3f} ms/step")
    per_kernel = sorted(((k, v["total_ms"] / v["calls"], v["calls"] // args.steps) for k, v in stats.items()),
                        key=lambda x: -x[1] * x[2])
    s_ = TINY
    attn_unit = 2.0 * s_.batch * s_.heads * s_.seq * s_.seq * s_.head_dim
    attn_flops = sum(x.flops for x in step.launches if x.name.startswith("attn."))
    attn_skipped = attn_flops * (1.0 - (s_.seq + 1) / (2.0 * s_.seq))
    assert abs(attn_flops - 7 * s_.layers * attn_unit) < 1.0

    result = {
        "metric": "GEMM TFLOP/s (% of MFMA peak) + TINY train-step ms, FP32 and BF16, 1 GPU",
        "value": round(total_flops / (ms_per_step * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "ms_per_step_median": round(ms_median, 4),
        "ms_per_step_min_max": [round(min(step_ms), 4), round(max(step_ms), 4)],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded SplitMix64/Box-Muller: activations and upstream grads N(0,1), weights N(0,0.02))",
        "config": {
            "workload": "TINY training step, all contractions fwd+bwd (BASELINE configs[1])",
            "layers": 4, "hidden": 256, "heads": 4, "head_dim": 64, "ffn": 688, "vocab": 16384,
            "tied_lm_head": False, "batch": 16, "seq": 256, "gflop_per_step": round(total_flops / 1e9, 2),
            "gemm_launches": len(step.launches),
            "execution": "hipGraph replay on one stream; each layer's weight gradients as one grouped launch",
            "frac_fp32_mfma_peak": round(total_flops / (ms_per_step * 1e-3) / 1e12 / PEAK_TFLOPS["f32"], 4),
            "ms_per_step_side_stream": round(ms_side, 4),
            "tflops_side_stream": round(total_flops / (ms_side * 1e-3) / 1e12, 3),
            "attention_gflop_dense_equiv": round(attn_flops / 1e9, 2),
            "attention_gflop_skipped_by_causal": round(attn_skipped / 1e9, 2),
            "note_flops": "value counts attention as dense-equivalent GEMMs (BASELINE's definition); the causal "
                          "kernels skip the masked half, attention_gflop_skipped_by_causal of gflop_per_step",
        },
        "library": lib_info,
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_TFLOPS["f32"],
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_TFLOPS["f32"], 4),
            "traffic": committed_traffic(dom_key),
            "kernel": dom_key,
            "avg_us": round(avg_ms * 1e3, 2),
            "flops_per_launch": dom_flops,
        },
        "gemm_kernel_ms_per_step": round(gemm_ms, 4),
        "top_kernels": [{"key": k, "avg_us": round(a * 1e3, 2), "per_step": c} for k, a, c in per_kernel[:8]],
    }
    log("[bench] complete TINY training step")
    result["train_step"] = train_step_figures(it, timer, args.steps, args.warmup)
    log(f"[bench] train step {result['train_step']['ms_per_step']} ms")
    if not args.no_extra:
        log("[bench] extra GEMM figures")
        result["extra"] = extras(it, timer)
    if not args.no_cpu:
        log("[bench] CPU baseline (oracle on host cores)")
        result["cpu_baseline"] = cpu_baseline(step)
    print(json.dumps(result), flush=True)
    step.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
