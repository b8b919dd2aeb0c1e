"""Writes tests/golden/oracle_vectors.json: seeded tiny cases and the oracle's exact outputs.

These pin the oracle against silent change (its outputs are stored bit-exactly as uint32/uint16).
The attention case uses the input formulas of the reference's test_attention_simple
(src/ops/attention.rs:623-651). Re-run only when the oracle is deliberately changed:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from irontensor_amd import synth  # noqa: E402


def f32_bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32).ravel().tolist()


def main():
    out = {"gemm_f32": [], "gemm_bf16": [], "attention_bshd": []}
    m, n, k = 5, 7, 9
    for i, (ta, tb) in enumerate([(0, 0), (0, 1), (1, 0), (1, 1)]):
        a_shape = [k, m] if ta else [m, k]
        b_shape = [n, k] if tb else [k, n]
        a = synth.normal(100 + i, a_shape)
        b = synth.normal(200 + i, b_shape, std=0.02)
        c = oracle.gemm_f32(a, b, bool(ta), bool(tb), threads=1)
        out["gemm_f32"].append({"name": f"f32_{'NT'[ta]}{'NT'[tb]}", "trans_a": ta, "trans_b": tb,
                                "a_shape": a_shape, "b_shape": b_shape, "a": f32_bits(a),
                                "b": f32_bits(b), "out": f32_bits(c)})
        ab, bb = oracle.f32_to_bf16(a), oracle.f32_to_bf16(b)
        c16 = oracle.gemm_bf16(ab, bb, bool(ta), bool(tb), out_bf16=True, threads=1)
        out["gemm_bf16"].append({"name": f"bf16_{'NT'[ta]}{'NT'[tb]}", "trans_a": ta, "trans_b": tb,
                                 "a_shape": a_shape, "b_shape": b_shape, "a": ab.ravel().tolist(),
                                 "b": bb.ravel().tolist(), "out": c16.ravel().tolist()})
    shape = [1, 4, 2, 8]
    numel = int(np.prod(shape))
    idx = np.arange(numel, dtype=np.float32)
    q = idx * np.float32(0.1) - np.float32(3.0)
    kk = idx * np.float32(0.1) - np.float32(2.0)
    v = idx * np.float32(0.1) - np.float32(1.0)
    for causal in (False, True):
        o = oracle.attention_bshd(q.reshape(shape), kk.reshape(shape), v.reshape(shape), causal, threads=1)
        out["attention_bshd"].append({"name": f"attention_simple_causal{int(causal)}", "shape": shape,
                                      "causal": causal, "q": f32_bits(q), "k": f32_bits(kk),
                                      "v": f32_bits(v), "out": f32_bits(o)})
    path = Path(__file__).resolve().parent / "oracle_vectors.json"
    path.write_text(json.dumps(out, separators=(",", ":")) + "\n")
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
