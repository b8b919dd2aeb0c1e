"""BASELINE config 4 on the GPU: the medium BF16 training step's contractions
(GemmStep(MEDIUM, BF16, ffn_bias=True): 12 layers, hidden 1024, 16 heads x 64, SwiGLU FFN 2816 with
the fused bias + SwiGLU epilogue, vocab 32768, batch 8 x seq 1024), in the reference trainer's call
order (src/train/trainer/train_step.rs:39-236).

* Graph replay of the whole step equals the eager step bit for bit (every kernel is deterministic).
* The in-step fused attention (B8 x H16 x S1024, causal, read in place from the fused QKV buffer) on
  three sampled heads of the first and last layer, forward O and backward dQ/dK/dV, against
  oracle.attention_{fwd,bwd}_bhsd on the same BF16 values: relative Frobenius 1e-2.
* Every distinct GEMM of the step (shape, layout, epilogue, and the plan the library picks for it,
  recorded by the profiler) on 64+ sampled output rows: against the oracle on the same BF16
  operands (FP32 normwise 1e-5, or half a BF16 ulp + 1e-5 for BF16 outputs) and against the f32
  oracle on the unrounded seeded inputs (relative Frobenius 1e-2). tests/stepcheck.py does it.
* A layer's four weight gradients, which the step issues as one it_gemm_group launch: each within
  FP32 normwise 1e-5 of the same GEMM issued alone (the call the previous check verifies).
"""
from __future__ import annotations

import hashlib

import numpy as np
import pytest

from irontensor_amd.step import MEDIUM, GemmStep
from tests.numerics import BF16_FROB_TOL, FP32_TOL, frob_rel, normwise_rel
from tests.stepcheck import StepChecker

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def med(it):
    _log("[medium] building GemmStep(MEDIUM, BF16, ffn_bias=True)")
    st = GemmStep(MEDIUM, it.Precision.BF16, ffn_bias=True)
    st.enqueue()
    it.Context.global_().sync()
    _log("[medium] eager step done")
    yield st
    st.close()


def _digest(t) -> str:
    raw = t.as_bf16_slice() if t.is_bf16() else t.as_f32_slice()
    return hashlib.sha256(raw.tobytes()).hexdigest()


def test_medium_graph_replay_matches_eager(it, med):
    st = med
    picks = {"logits": st.logits, "dE": st.dE, "dHf": st.dHf, "dX": st.dX, "Hh0": st.Hh[0], "Z11": st.Z[11],
             "G5": st.G[5], "O5": st.O[5], "lse5": st.lse[5], "dQKV3": st.dQKV_layers[3],
             "dWqkv0": st.dWqkv[0], "dWgu6": st.dWgu[6], "dWd11": st.dWd[11], "dWo2": st.dWo[2]}
    eager = {k: _digest(t) for k, t in picks.items()}
    st.capture()
    for rep in range(2):
        st.replay()
        it.Context.global_().sync()
        for k, t in picks.items():
            assert _digest(t) == eager[k], (rep, k)
    _log(f"[medium] graph replay x2 == eager on {len(picks)} outputs")


def _heads(x, s, part, picks):
    """[T, parts*H] rows of the step -> [len(picks), S, D] for bh in picks (b = bh // heads)."""
    b, n, h, d = s.batch, s.seq, s.heads, s.head_dim
    parts = x.shape[1] // (h * d)
    y = x.reshape(b, n, parts, h, d)
    return np.stack([y[bh // h, :, part, bh % h, :] for bh in picks]).astype(np.float32)


@pytest.mark.parametrize("layer", [0, 11])
def test_medium_in_step_attention(it, oracle, med, layer):
    st, s = med, med.s
    picks = [0, 77, 127]
    qkv = st.QKV[layer].numpy()
    q, k, v = (_heads(qkv, s, i, picks) for i in range(3))
    scale = 1.0 / np.sqrt(s.head_dim)
    ro, _ = oracle.attention_fwd_bhsd(q, k, v, scale, True)
    o = _heads(st.O[layer].numpy(), s, 0, picks)
    err_o = frob_rel(o, ro)
    do = _heads(st.dO.numpy(), s, 0, picks)
    refs = oracle.attention_bwd_bhsd(do, q, k, v, scale, True)
    got = [_heads(st.dQKV_layers[layer].numpy(), s, i, picks) for i in range(3)]
    errs = [frob_rel(g, r) for g, r in zip(got, refs)]
    _log(f"[medium attention L{layer}] heads {picks}: frob O {err_o:.2e} dQ {errs[0]:.2e} "
         f"dK {errs[1]:.2e} dV {errs[2]:.2e}")
    assert err_o <= BF16_FROB_TOL
    assert max(errs) <= BF16_FROB_TOL


def test_medium_every_gemm_plan(it, oracle, med):
    chk = StepChecker(it, oracle, med, rows=64, log=_log)
    plans = {}
    for key in list(med._calls):
        plans[key] = chk.check_call(key)
    _log(f"[medium] {len(plans)} distinct GEMMs, plans: {sorted(set(plans.values()))}")
    assert len(plans) == 15


def test_medium_grouped_weight_gradients(it, med):
    st = med
    ctx = it.Context.global_()
    from irontensor_amd import profiler
    profiler.reset(ctx)
    profiler.enable(ctx)
    st.enqueue()
    ctx.sync()
    keys = [k for k in profiler.stats(ctx) if "_dtl_group" in k]
    profiler.enable(ctx, False)
    _log(f"[medium] grouped weight-gradient launches: {keys}")
    assert keys, "the step's weight gradients did not run as a group"
    s, l = st.s, st.s.layers - 1  # the reissued calls are the first of each shape: the last layer's
    T, H, F = s.tokens, s.hidden, s.ffn
    outs = {(True, False, H, F, T): st.dWd[l], (True, False, 2 * F, H, T): st.dWgu[l],
            (True, False, H, H, T): st.dWo[l], (True, False, 3 * H, H, T): st.dWqkv[l]}
    grouped = {k: t.numpy() for k, t in outs.items()}
    for k, t in outs.items():
        st.reissue(*k)
        ctx.sync()
        err = normwise_rel(grouped[k], t.numpy())
        _log(f"[medium] grouped vs single {k[2:]}: normwise {err:.2e}")
        assert err <= FP32_TOL, k
    # On the side stream (overlap_weight_grads) the group is the same kernel, so the same bits.
    st.overlap = True
    try:
        st.enqueue()
        ctx.sync()
        for k, t in outs.items():
            assert np.array_equal(t.numpy(), grouped[k]), k
    finally:
        st.overlap = False
