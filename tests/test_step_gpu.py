"""The TINY step driver on the GPU: one eager step checked against the oracle
at layer 0 (QKV projection, fused attention forward, fused attention backward into dQKV), and the
HIP-graph replay bit-identical to the eager step (every kernel on the path is deterministic)."""
from __future__ import annotations

import numpy as np
import pytest

from irontensor_amd.step import TINY, GemmStep
from tests.numerics import FP32_TOL, normwise_rel
from tests.stepcheck import StepChecker

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def step(it):
    st = GemmStep(TINY, it.Precision.FP32)
    assert st.fused  # head_dim 64 takes the fused attention kernels
    st.enqueue()
    it.Context.global_().sync()
    return st


def _heads(x, s):
    """[T, 3H] or [T, H] -> per-part [B, H, S, D] (float32)."""
    b, n, h, d = s.batch, s.seq, s.heads, s.head_dim
    parts = x.shape[1] // (h * d)
    y = x.reshape(b, n, parts, h, d).transpose(2, 0, 3, 1, 4)
    return [np.ascontiguousarray(p) for p in y]


def test_step_layer0_against_oracle(it, oracle, step):
    s = step.s
    x, wqkv = step.X[0].numpy(), step.Wqkv[0].numpy()
    qkv = step.QKV[0].numpy()
    assert normwise_rel(qkv, oracle.gemm_f32(x, wqkv, trans_b=True)) <= FP32_TOL
    q, k, v = _heads(qkv, s)
    ro, _ = oracle.attention_fwd_bhsd(q, k, v, 1 / np.sqrt(s.head_dim), True)
    (o,) = _heads(step.O[0].numpy(), s)
    assert normwise_rel(o, ro) <= FP32_TOL
    # layer 0's backward runs last, so dQKV holds its attention gradients
    (do,) = _heads(step.dO.numpy(), s)
    refs = oracle.attention_bwd_bhsd(do, q, k, v, 1 / np.sqrt(s.head_dim), True)
    got = _heads(step.dQKV.numpy(), s)
    for name, g, r in zip("QKV", got, refs):
        assert normwise_rel(g, r) <= FP32_TOL, name


def test_step_lm_head_gemms_against_oracle(it, oracle, step):
    """The three LM-head GEMMs at [4096,16384,256] (forward NT, dE TN, dHf NN) in the plans the
    step uses, on 64+ sampled output rows against the oracle's FP32 loop (normwise 1e-5)."""
    s = step.s
    T, H, V = s.tokens, s.hidden, s.vocab
    chk = StepChecker(it, oracle, step, rows=64, log=lambda m: print(m, flush=True))
    for key in ((False, True, T, V, H), (True, False, V, H, T), (False, False, T, H, V)):
        chk.check_call(key)


def test_tiny_every_gemm_plan(it, oracle, step):
    """Every distinct GEMM of the TINY step at its step shape and in the plan
    the step runs it with, on 64+ sampled output rows against the oracle's FP32 loop (normwise 1e-5):
    the fused QKV projection with its RoPE epilogue input, Wo, the SwiGLU up-projection, down, the
    four data gradients, the four weight gradients and the three LM-head GEMMs."""
    chk = StepChecker(it, oracle, step, rows=64, log=lambda m: print(m, flush=True))
    plans = {key: chk.check_call(key) for key in list(step._calls)}
    print(f"[tiny] {len(plans)} distinct GEMMs, plans: {sorted(set(plans.values()))}", flush=True)
    assert len(plans) == 15
    # The reissued calls overwrote shared buffers: leave the module's step as a whole step left it.
    step.enqueue()
    it.Context.global_().sync()


def test_step_graph_replay_matches_eager(it, step):
    names = ["logits", "dE", "dHf", "dQKV", "dX"]
    eager = {n: getattr(step, n).numpy() for n in names}
    eager["dWqkv0"] = step.dWqkv[0].numpy()
    eager["Z3"] = step.Z[3].numpy()
    step.capture()
    for _ in range(3):
        step.replay()
        it.Context.global_().sync()
        for n in names:
            assert np.array_equal(getattr(step, n).numpy(), eager[n]), n
        assert np.array_equal(step.dWqkv[0].numpy(), eager["dWqkv0"])
        assert np.array_equal(step.Z[3].numpy(), eager["Z3"])


def test_step_fused_matches_materialised(it):
    a = GemmStep(TINY, it.Precision.FP32, seed=99, fused_attention=True)
    b = GemmStep(TINY, it.Precision.FP32, seed=99, fused_attention=False)
    a.enqueue()
    b.enqueue()
    it.Context.global_().sync()
    for l in range(TINY.layers):
        assert normwise_rel(a.O[l].numpy(), b.O[l].numpy()) <= FP32_TOL
    assert normwise_rel(a.dQKV.numpy(), b.dQKV.numpy()) <= FP32_TOL
    assert normwise_rel(a.dX.numpy(), b.dX.numpy()) <= FP32_TOL


def test_step_side_stream_matches_single_stream(it):
    """Weight gradients on the side stream (the default) give bit-identical results to the same
    step issued on one stream, eagerly and through a captured graph."""
    a = GemmStep(TINY, it.Precision.FP32, seed=7, overlap_weight_grads=True)
    b = GemmStep(TINY, it.Precision.FP32, seed=7, overlap_weight_grads=False)
    for st in (a, b):
        st.enqueue()
    it.Context.global_().sync()

    def grads(st):
        return [x.numpy() for x in (st.dE, st.dHf, st.dX, *st.dWqkv, *st.dWo, *st.dWgu, *st.dWd)]

    ga, gb = grads(a), grads(b)
    for x, y in zip(ga, gb):
        assert np.array_equal(x, y)
    a.capture()
    for _ in range(2):
        a.replay()
        it.Context.global_().sync()
        for x, y in zip(grads(a), gb):
            assert np.array_equal(x, y)
