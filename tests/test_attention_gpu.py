"""GPU parity of the batched attention contractions against the oracle's reference_attention and
attention_backward_recompute restatements (src/ops/attention.rs:544-621, src/train/helpers.rs:120-193).
Tolerances as in test_gemm_gpu: FP32 normwise 1e-5 (plus the reference tests' absolute bounds);
BF16 relative Frobenius 1e-2 against the f32 oracle on the unrounded inputs."""
from __future__ import annotations

import numpy as np
import pytest

from irontensor_amd import synth
from tests.numerics import BF16_FROB_TOL, FP32_TOL, frob_rel, normwise_rel

pytestmark = pytest.mark.gpu


def _bshd(it, x):
    return it.Tensor.from_f32_slice(x, x.shape)


@pytest.mark.parametrize("name,b,s,h,d,causal,fill,tol", [
    # src/ops/attention.rs:623-651, :653-679, :681-711
    ("simple", 1, 4, 2, 8, False, "simple", 1e-3),
    ("causal", 1, 4, 1, 4, True, "causal", 1e-3),
    ("larger", 2, 16, 4, 32, True, "larger", 1e-2),
])
def test_reference_attention_cases(it, oracle, name, b, s, h, d, causal, fill, tol):
    n = b * s * h * d
    i = np.arange(n, dtype=np.float32)
    if fill == "simple":
        q, k, v = i * np.float32(0.1) - 3, i * np.float32(0.1) - 2, i * np.float32(0.1) - 1
    elif fill == "causal":
        q = k = v = (i + 1) * np.float32(0.1)
    else:
        q = k = v = ((np.arange(n) % 100).astype(np.float32) - 50) * np.float32(0.01)
    shape = (b, s, h, d)
    q, k, v = (x.reshape(shape).astype(np.float32) for x in (q, k, v))
    out = it.attention(_bshd(it, q), _bshd(it, k), _bshd(it, v), causal).numpy()
    ref = oracle.attention_bshd(q, k, v, causal)
    assert np.max(np.abs(out - ref)) < tol
    assert normwise_rel(out, ref) <= FP32_TOL


def test_attention_kv_length_differs(it, oracle):
    b, sq, skv, h, d = 2, 24, 40, 3, 16
    q = synth.normal(1, (b, sq, h, d))
    k = synth.normal(2, (b, skv, h, d))
    v = synth.normal(3, (b, skv, h, d))
    out = it.attention(_bshd(it, q), _bshd(it, k), _bshd(it, v), False).numpy()
    t = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3)).astype(np.float64)  # noqa: E731
    s = t(q) @ np.swapaxes(t(k), -1, -2) / np.sqrt(d)
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ref = (p @ t(v)).transpose(0, 2, 1, 3)
    assert normwise_rel(out, ref) <= FP32_TOL


def test_attention_empty_returns_zeros(it):
    z = it.Tensor.zeros([1, 0, 2, 4])
    out = it.attention(z, z, z, False)
    assert out.shape() == [1, 0, 2, 4]


@pytest.mark.parametrize("b,h,s,d", [(2, 4, 16, 8), (4, 4, 256, 64)])
def test_attention_backward_recompute_f32(it, oracle, b, h, s, d):
    """(2,4,16,8) is the shape of test_attention_backward_pipelined_correctness
    (src/train/helpers.rs:435-494); (4,4,256,64) is a quarter of one TINY layer."""
    print(f"[attn bwd f32] {b}x{h}x{s}x{d}", flush=True)
    q, k, v, do = (synth.normal(10 + i, (b, h, s, d)) for i in range(4))
    dq, dk, dv = it.attention_backward_recompute(*(it.Tensor.from_f32_slice(x, x.shape) for x in (do, q, k, v)))
    rq, rk, rv = oracle.attention_bwd_bhsd(do, q, k, v, 1 / np.sqrt(d), True)
    for got, ref in ((dq, rq), (dk, rk), (dv, rv)):
        g = got.numpy()
        assert np.max(np.abs(g - ref)) < 1e-3
        assert normwise_rel(g, ref) <= FP32_TOL


@pytest.mark.parametrize("causal", [True, False])
def test_attention_forward_bhsd_f32(it, oracle, causal):
    b, h, s, d = 2, 4, 256, 64
    q, k, v = (synth.normal(20 + i, (b, h, s, d)) for i in range(3))
    o, p = it.attention_forward_bhsd(*(it.Tensor.from_f32_slice(x, x.shape) for x in (q, k, v)), causal=causal)
    ro, rp = oracle.attention_fwd_bhsd(q, k, v, 1 / np.sqrt(d), causal)
    assert normwise_rel(o.numpy(), ro) <= FP32_TOL
    pp = p.numpy()
    assert normwise_rel(pp, rp.reshape(pp.shape)) <= FP32_TOL
    if causal:
        assert np.all(pp[:, np.triu(np.ones((s, s), bool), 1)] == 0)


def test_attention_bf16_forward_backward(it, oracle):
    """BASELINE config 3 at 1/16 of the batch (1 x 8 heads x 1024 x 64); the full size is in the
    property test below."""
    b, h, s, d = 1, 8, 1024, 64
    q, k, v, do = (synth.normal(30 + i, (b, h, s, d)) for i in range(4))
    tq, tk, tv, tdo = (it.Tensor.from_f32_as_bf16(x, x.shape) for x in (q, k, v, do))
    o, _ = it.attention_forward_bhsd(tq, tk, tv, causal=True, scale=0.125)
    ro, _ = oracle.attention_fwd_bhsd(q, k, v, 0.125, True)
    err_o = frob_rel(o.numpy(), ro)
    dq, dk, dv = it.attention_backward_recompute(tdo, tq, tk, tv, causal=True, scale=0.125)
    rq, rk, rv = oracle.attention_bwd_bhsd(do, q, k, v, 0.125, True)
    errs = [frob_rel(x.numpy(), r) for x, r in ((dq, rq), (dk, rk), (dv, rv))]
    print(f"[attn bf16] frob O {err_o:.3e} dQ {errs[0]:.3e} dK {errs[1]:.3e} dV {errs[2]:.3e}", flush=True)
    assert err_o <= BF16_FROB_TOL
    assert max(errs) <= BF16_FROB_TOL


def test_attention_bf16_full_size_properties(it):
    """Config 3 at full size [16,8,1024,64]: causal P rows sum to 1 with exact zeros above the
    diagonal, and O = P.V checked by a float64 Freivalds product on one head group."""
    b, h, s, d = 16, 8, 1024, 64
    q, k, v = (synth.normal(40 + i, (b, h, s, d)) for i in range(3))
    tq, tk, tv = (it.Tensor.from_f32_as_bf16(x, x.shape) for x in (q, k, v))
    o, p = it.attention_forward_bhsd(tq, tk, tv, causal=True, scale=0.125)
    pp = it.bf16_to_f32(p.as_bf16_slice()).reshape(b * h, s, s)
    rows = pp.astype(np.float64).sum(-1)
    assert np.max(np.abs(rows - 1.0)) < 1e-2  # BF16 P: each entry carries <= 2^-9 relative error
    assert np.all(pp[:, np.triu(np.ones((s, s), bool), 1)] == 0)
    oo = o.numpy().reshape(b * h, s, d).astype(np.float64)
    vv = it.bf16_to_f32(tv.as_bf16_slice()).reshape(b * h, s, d).astype(np.float64)
    x = synth.normal(44, (d,)).astype(np.float64)
    for g in (0, 77, 127):
        lhs = oo[g] @ x
        rhs = pp[g].astype(np.float64) @ (vv[g] @ x)
        scale = np.abs(pp[g]) @ (np.abs(vv[g]) @ np.abs(x))
        assert np.max(np.abs(lhs - rhs) / scale) < 1e-5
