"""Benchmark of the matmul hot path on one MI355X.

Workload: every contraction of one TINY training step, forward and backward,
FP32 (4 layers, hidden 256, 4 heads x 64, SwiGLU FFN 688, untied vocab 16384, batch 16 x seq 256):
115 dense-equivalent GEMMs = 195.82 GFLOP, issued by irontensor_amd.step.GemmStep as 75 GEMM
launches (fused QKV and gate|up) plus the attention softmax / softmax-backward, captured once into
a HIP graph and replayed. A "step" is one replay; inputs are resident in HBM before timing starts.

Prints ONE JSON line (rank 0 = this process). Extra figures (config 1, the BF16 square and decode
GEMMs) go under "extra". The CPU baseline is the oracle's reference loop on host cores over a
bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes as C
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
    """FLOPs of one launch from a profiler key '...|tag[M,N,K]xB s..' (x2 for the SwiGLU dual-B)."""
    m = re.search(r"\[(\d+),(\d+),(\d+)\]x(\d+)", key)
    if not m:
        return 0.0
    M, N, K, B = (int(g) for g in m.groups())
    return 2.0 * M * N * K * B * (2 if "_swiglu" in key else 1)


def profiler_stats(ctx) -> dict:
    lib = ctx.lib
    need = C.c_size_t(0)
    lib.it_profiler_report(ctx.handle, None, 0, C.byref(need))
    buf = C.create_string_buffer(need.value + 16)
    st = lib.it_profiler_report(ctx.handle, buf, need.value + 16, C.byref(need))
    if st != 0:
        raise RuntimeError("profiler report failed")
    return json.loads(buf.value.decode())


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


def time_gemm(it, timer, a, b, out, trans_a, trans_b, iters, warm=3) -> float:
    for _ in range(warm):
        it.gemm(a, b, trans_a=trans_a, trans_b=trans_b, out=out)
    it.Context.global_().sync()
    timer.start()
    for _ in range(iters):
        it.gemm(a, b, trans_a=trans_a, trans_b=trans_b, out=out)
    return timer.stop_ms() / iters


def extras(it, timer) -> dict:
    """Config 1 (FP32 QKV projection) and the BF16 square / decode GEMMs, timed with hipEvents."""
    from irontensor_amd import synth
    P = it.Precision
    out = {}
    x = it.Tensor.from_f32_slice(synth.normal(1, (4096, 256)), [4096, 256])
    w = it.Tensor.from_f32_slice(synth.normal(2, (768, 256), std=0.02), [768, 256])
    y = it.Tensor.empty([4096, 768])
    ms = time_gemm(it, timer, x, w, y, False, True, 50)
    tf = 2 * 4096 * 768 * 256 / (ms * 1e-3) / 1e12
    out["config1_fp32_qkv_4096x768x256_NT"] = {"ms": round(ms, 5), "tflops": round(tf, 2),
                                               "frac_fp32_peak": round(tf / PEAK_TFLOPS["f32"], 4)}
    for n in (4096, 8192):
        a = it.Tensor.from_f32_as_bf16(synth.normal(3, (n, n)), [n, n])
        b = it.Tensor.from_f32_as_bf16(synth.normal(4, (n, n)), [n, n])
        c = it.Tensor.empty([n, n], P.BF16)
        for lay, (ta, tb) in (("NN", (False, False)), ("NT", (False, True)), ("TN", (True, False))):
            ms = time_gemm(it, timer, a, b, c, ta, tb, 10 if n == 4096 else 4)
            tf = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
            out[f"bf16_square_{n}_{lay}"] = {"ms": round(ms, 4), "tflops": round(tf, 1),
                                             "frac_bf16_peak": round(tf / PEAK_TFLOPS["bf16"], 4)}
        del a, b, c
    k, n = 4096, 11008
    wt = it.Tensor.from_f32_as_bf16(synth.normal(5, (n, k)), [n, k])
    for m in (1, 4, 16):
        xa = it.Tensor.from_f32_as_bf16(synth.normal(6, (m, k)), [m, k])
        yo = it.Tensor.empty([m, n], P.BF16)
        ms = time_gemm(it, timer, xa, wt, yo, False, True, 20)
        gbs = (n * k * 2 + m * k * 2 + m * n * 2) / (ms * 1e-3) / 1e9
        out[f"bf16_decode_m{m}_k4096_n11008_NT"] = {"ms": round(ms, 5), "GBps": round(gbs, 1),
                                                    "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    return out


def cpu_baseline(step) -> dict:
    """The oracle's sequential f32 loop (the reference's CPU matmul), row-parallel over host cores,
    on a bounded sample of the workload: layer 0's forward and backward GEMMs plus the LM-head
    forward GEMM, at the step's real shapes."""
    import oracle
    from irontensor_amd import synth
    s = step.s
    T, H, F, V = s.tokens, s.hidden, s.ffn, s.vocab
    thr = oracle.default_threads()
    w = lambda sh, seed: synth.normal(seed, sh, std=0.02)  # noqa: E731
    a = lambda sh, seed: synth.normal(seed, sh)  # noqa: E731
    X, X2, Hh, O = a((T, H), 1), a((T, H), 2), a((T, F), 3), a((T, H), 4)
    Wqkv, Wo, Wg, Wd, E = w((3 * H, H), 5), w((H, H), 6), w((2 * F, H), 7), w((H, F), 8), w((V, H), 9)
    dZ, dGU, dY, dQKV = a((T, H), 10), a((T, 2 * F), 11), a((T, H), 12), a((T, 3 * H), 13)
    calls = [
        (X, Wqkv, False, True), (O, Wo, False, True), (X2, Wg, False, True), (Hh, Wd, False, True),
        (dZ, Wd, False, False), (dZ, Hh, True, False), (dGU, Wg, False, False), (dGU, X2, True, False),
        (dY, Wo, False, False), (dY, O, True, False), (dQKV, Wqkv, False, False), (dQKV, X, True, False),
        (a((T, H), 14), E, False, True),
    ]
    flops = 0.0
    t0 = time.perf_counter()
    for A, B, ta, tb in calls:
        r = oracle.gemm_f32(A, B, ta, tb, threads=thr)
        flops += 2.0 * A.shape[0] * A.shape[1] * (B.shape[0] if tb else B.shape[1])
        del r
    bh = s.batch * s.heads
    q, k, v, do = (a((bh, s.seq, s.head_dim), 20 + i) for i in range(4))
    oracle.attention_fwd_bhsd(q, k, v, 0.125, True, threads=thr)
    oracle.attention_bwd_bhsd(do, q, k, v, 0.125, True, threads=thr)
    flops += 7 * 2.0 * bh * s.seq * s.seq * s.head_dim
    dt = time.perf_counter() - t0
    return {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": thr,
            "kind": "port",
            "sample": (f"layer 0 forward+backward contractions (12 linear GEMMs, 7 attention GEMMs) "
                       f"+ LM-head forward GEMM of the TINY step, {flops / 1e9:.1f} GFLOP in "
                       f"{dt:.2f} s; oracle/ref.c sequential f32 loop, {thr} threads"),
            "seconds": round(dt, 2),
            "ms_per_step_extrapolated": round(step.flops() / (flops / dt) * 1e3, 1)}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip the extra GEMM figures")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is design-only, see DESIGN.md)", file=sys.stderr)
        return 2
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: launched with WORLD_SIZE > 1; this build runs on one GPU only", file=sys.stderr)
        return 2

    import irontensor_amd as it
    from irontensor_amd.step import TINY, GemmStep

    if it.device_count() == 0:
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1
    ctx = it.Context.global_()
    info = ctx.info()
    log(f"[bench] device {info}")
    step = GemmStep(TINY, it.Precision.FP32, ctx)
    step.enqueue()                      # eager once: records the launch list, sizes scratch
    ctx.sync()
    total_flops = step.flops()
    log(f"[bench] TINY step: {len(step.launches)} contractions, {total_flops / 1e9:.2f} GFLOP")
    step.capture()
    for _ in range(args.warmup):
        step.replay()
    ctx.sync()
    timer = Timer(ctx)
    t0 = time.perf_counter()
    timer.start()
    for _ in range(args.steps):
        step.replay()
    gpu_ms = timer.stop_ms()
    ctx.sync()
    wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    log(f"[bench] timed {args.steps} steps: wall {ms_per_step:.3f} ms/step, events "
        f"{gpu_ms / args.steps:.3f} ms/step")

    # Per-kernel durations: the same steps run eagerly with hipEvents around every launch.
    ctx.lib.it_profiler_reset(ctx.handle)
    ctx.lib.it_profiler_enable(ctx.handle, 1)
    for _ in range(args.steps):
        step.enqueue()
    stats = profiler_stats(ctx)
    ctx.lib.it_profiler_enable(ctx.handle, 0)
    gemm_ms = sum(v["total_ms"] for v in stats.values()) / args.steps
    dom_key, dom = max(stats.items(), key=lambda kv: kv[1]["total_ms"])
    avg_ms = dom["total_ms"] / dom["calls"]
    dom_flops = parse_key_flops(dom_key)
    achieved = dom_flops / (avg_ms * 1e-3) / 1e12
    log(f"[bench] dominant kernel {dom_key}: {dom['calls']} calls, avg {avg_ms * 1e3:.1f} us, "
        f"{achieved:.1f} TFLOP/s; sum of GEMM launches {gemm_ms:.3f} ms/step")
    per_kernel = sorted(((k, v["total_ms"] / v["calls"], v["calls"] // args.steps) for k, v in stats.items()),
                        key=lambda x: -x[1] * x[2])

    result = {
        "metric": "GEMM TFLOP/s (% of MFMA peak) + TINY train-step ms, FP32 and BF16, 1 GPU",
        "value": round(total_flops / (ms_per_step * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded SplitMix64/Box-Muller: activations and upstream grads N(0,1), weights N(0,0.02))",
        "config": {
            "workload": "TINY training step, all contractions fwd+bwd (BASELINE configs[1])",
            "layers": 4, "hidden": 256, "heads": 4, "head_dim": 64, "ffn": 688, "vocab": 16384,
            "tied_lm_head": False, "batch": 16, "seq": 256, "gflop_per_step": round(total_flops / 1e9, 2),
            "gemm_launches": len(step.launches), "execution": "hipGraph replay, one stream",
            "frac_fp32_mfma_peak": round(total_flops / (ms_per_step * 1e-3) / 1e12 / PEAK_TFLOPS["f32"], 4),
        },
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_TFLOPS["f32"],
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_TFLOPS["f32"], 4),
            "traffic": None,
            "kernel": dom_key,
            "avg_us": round(avg_ms * 1e3, 2),
            "flops_per_launch": dom_flops,
        },
        "gemm_kernel_ms_per_step": round(gemm_ms, 4),
        "top_kernels": [{"key": k, "avg_us": round(a * 1e3, 2), "per_step": c} for k, a, c in per_kernel[:8]],
    }
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
