"""The GEMM prologue/epilogue fusions on the GPU against the oracle: RMSNorm -> projection (gamma
folded into the A-tile load, 1/rms into the epilogue) and the chunked linear + cross entropy (no
[rows, vocab] logits). FP32 within the normwise 1e-5 contract; chunking changes nothing beyond
rounding; ignored targets give zero rows."""
from __future__ import annotations

import numpy as np
import pytest

from irontensor_amd import synth
from tests.numerics import FP32_TOL, normwise_rel

pytestmark = pytest.mark.gpu


def _t(it, a):
    return it.Tensor.from_f32_slice(np.ascontiguousarray(a, np.float32), list(np.shape(a)))


@pytest.mark.parametrize("rows,hidden,out_f", [(4096, 256, 768), (4096, 256, 1376), (37, 100, 50), (5, 64, 32),
                                               (1024, 1024, 3072)])
def test_fused_rmsnorm_linear(it, oracle, rows, hidden, out_f):
    from irontensor_amd import train_ops as T
    print(f"[case] fused_rmsnorm_linear {rows}x{hidden} -> {out_f}", flush=True)
    x = synth.normal(1, (rows, hidden))
    g = (1 + synth.normal(2, (hidden,), std=0.1)).astype(np.float32)
    w = synth.normal(3, (out_f, hidden), std=0.02)
    got = T.fused_rmsnorm_linear(_t(it, x), _t(it, g), _t(it, w), 1e-5).numpy()
    assert normwise_rel(got, oracle.fused_rmsnorm_linear(x, g, w, 1e-5)) <= FP32_TOL
    # same as the unfused path (normalize, then X.W^T) on the GPU
    xn = T.rmsnorm(_t(it, x), _t(it, g), 1e-5)
    assert normwise_rel(got, it.linear_forward(xn, _t(it, w)).numpy()) <= FP32_TOL


def test_fused_rmsnorm_linear_reference_case(it, oracle):
    """src/ops/fused_rmsnorm_linear.rs:244-276 inputs (the reference allows 1e-3 there)."""
    from irontensor_amd import train_ops as T
    rows, hidden, out_f = 4, 64, 32
    x = ((np.arange(rows * hidden) % 100) - 50.0).astype(np.float32).reshape(rows, hidden) * np.float32(0.01)
    g = (1.0 + np.sin(np.arange(hidden, dtype=np.float64)) * 0.1).astype(np.float32)
    w = ((np.arange(out_f * hidden) % 200) - 100.0).astype(np.float32).reshape(out_f, hidden) * np.float32(0.001)
    got = T.fused_rmsnorm_linear(_t(it, x), _t(it, g), _t(it, w), 1e-5).numpy()
    assert normwise_rel(got, oracle.fused_rmsnorm_linear(x, g, w, 1e-5)) <= FP32_TOL


@pytest.mark.parametrize("rows,hidden,vocab,chunk", [(256, 128, 1000, 0), (256, 128, 1000, 256 * 4 * 256),
                                                     (64, 32, 333, 64 * 4 * 128), (7, 16, 40, 0)])
def test_fused_linear_cross_entropy(it, oracle, rows, hidden, vocab, chunk):
    from irontensor_amd import train_ops as T
    print(f"[case] fused_linear_cross_entropy {rows}x{hidden}, vocab {vocab}, chunk bytes {chunk}", flush=True)
    h = synth.normal(4, (rows, hidden))
    w = synth.normal(5, (vocab, hidden), std=0.2)
    t = synth.tokens(6, rows, vocab).astype(np.int32)
    t[::5] = -100
    loss, gh, gw = T.fused_linear_cross_entropy(_t(it, h), _t(it, w), t, chunk_bytes=chunk)
    rm, _, rgh, rgw = oracle.fused_linear_cross_entropy(h, w, t)
    assert abs(loss - rm) <= FP32_TOL * abs(rm)
    assert normwise_rel(gh.numpy(), rgh) <= FP32_TOL
    assert normwise_rel(gw.numpy(), rgw) <= FP32_TOL
    assert not gh.numpy()[::5].any()
    loss2, gh2 = T.fused_linear_cross_entropy(_t(it, h), _t(it, w), t, chunk_bytes=chunk, forward_only=True)
    assert loss2 == loss and np.array_equal(gh2.numpy(), gh.numpy())


def test_fused_linear_cross_entropy_tiny_lm_head(it):
    """The TINY LM head ([4096, 256] x [16384, 256]^T) in 4 chunks against the unfused GPU path
    (logits GEMM, fused cross entropy, dlogits.E and dlogits^T.H; the weight gradient unscaled)."""
    from irontensor_amd import train_ops as T
    rows, hidden, vocab = 4096, 256, 16384
    h, w = synth.normal(7, (rows, hidden)), synth.normal(8, (vocab, hidden), std=0.02)
    t = synth.tokens(9, rows, vocab).astype(np.int32)
    H, W = _t(it, h), _t(it, w)
    loss, gh, gw = T.fused_linear_cross_entropy(H, W, t, chunk_bytes=rows * 4 * 4096)
    logits = it.matmul_mps_nt(H, W)
    mean, _, dlog = T.cross_entropy_fused(logits, t.astype(np.uint32))
    assert abs(loss - mean) <= FP32_TOL * abs(mean)
    assert normwise_rel(gh.numpy(), it.matmul(dlog, W).numpy()) <= FP32_TOL
    assert normwise_rel(gw.numpy() / rows, it.matmul_tn(dlog, H).numpy()) <= FP32_TOL
