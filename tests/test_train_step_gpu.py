"""The full training step on the GPU (irontensor_amd.train.TrainStep: embedding, layers, final norm,
LM head, fused cross entropy, backward, clip, Lion) against the oracle's step (oracle/train_step.py)
on the same parameters and batch, and its determinism: graph replay and the side stream give
bit-identical parameters to eager single-stream steps.

Tolerances: every gradient within normwise 1e-4 of the oracle's (each contraction meets the 1e-5
contract; the chain through two layers compounds it), the loss within 1e-5 relative, the global
norm within 1e-5 relative; Lion inside the step is bit-exact given the step's own gradients."""
from __future__ import annotations

import numpy as np
import pytest

from irontensor_amd.step import TINY, ModelShape
from tests.numerics import FP32_TOL, normwise_rel

pytestmark = pytest.mark.gpu

SMALL64 = ModelShape("small64", 2, 128, 2, 64, 176, 1000, 2, 128)
GRAD_TOL = 1e-4


def _oracle_params(st):
    from oracle.train_step import LAYER_KEYS
    arrs = [t.numpy() for t in st.params]
    p = {"emb": arrs[0], "final_norm": arrs[1], "E": arrs[2]}
    L = st.s.layers
    for j, k in enumerate(LAYER_KEYS):
        p[k] = [arrs[3 + 6 * l + j] for l in range(L)]
    return p


@pytest.mark.parametrize("fused,xent", [(True, False), (False, False), (True, True)])
def test_train_step_matches_oracle(it, oracle, fused, xent):
    """xent: the LM-head backward GEMMs rebuild the cross-entropy gradient from the logits
    (IT_EPI_XENT_A) instead of reading a stored gradient."""
    from irontensor_amd.train import TrainStep
    from oracle import train_step as ts
    print(f"[case] train step vs oracle, fused attention={fused}, xent operand={xent}", flush=True)
    st = TrainStep(SMALL64, seed=5, fused_attention=fused, max_grad_norm=1e-3, xent_operand=xent)
    p0 = _oracle_params(st)
    m0 = [m.numpy() for m in st.momentum]
    st.step()
    it.Context.global_().sync()
    hp = ts.Hyper(max_grad_norm=1e-3)
    ref = ts.train_step(p0, m0, st.ids_host, st.targets_host, SMALL64, hp)
    assert abs(st.loss_value() - ref["loss"]) <= 1e-5 * abs(ref["loss"])
    got = [g.numpy() for g in st.grads]
    for i, (g, r) in enumerate(zip(got, ref["grads"])):
        assert normwise_rel(g, r) <= GRAD_TOL, i
    norm, clip = st.norm_clip.numpy()
    assert abs(norm - ref["norm"]) <= 1e-5 * ref["norm"]
    assert ref["clip"] < 1.0  # the clip is active in this case
    # Lion inside the step, given the step's own gradients and clip factor: bit-exact
    for w0, m, g, w1, m1 in zip(ts.param_list(p0), m0, got, st.params, st.momentum):
        rw, rm = oracle.lion(w0, m, g, st.lr, st.beta1, st.beta2, st.wd, scale=float(clip))
        assert np.array_equal(w1.numpy(), rw)
        assert np.array_equal(m1.numpy(), rm)


def test_train_step_tiny_matches_oracle(it, oracle):
    """One complete TrainStep at the TINY shape (4 layers, H 256, 4 x 64,
    F 688, vocab 16384, 16 x 256 tokens) against the oracle's step on the same parameters and batch:
    loss within 1e-5 relative, every gradient within normwise 1e-4, the global norm within 1e-5.
    The oracle step runs the restated reference loops on the host's threads (about 20 s)."""
    from irontensor_amd.train import TrainStep
    from oracle import train_step as ts
    print("[case] TINY train step vs oracle", flush=True)
    st = TrainStep(TINY, seed=9)
    p0 = _oracle_params(st)
    st.step()
    it.Context.global_().sync()
    loss, grads, _ = ts.gradients(p0, st.ids_host, st.targets_host, TINY)
    print(f"[tiny step] loss {st.loss_value():.6f} oracle {loss:.6f}", flush=True)
    assert abs(st.loss_value() - loss) <= 1e-5 * abs(loss)
    worst = 0.0
    for i, (g, r) in enumerate(zip(st.grads, ts.param_list(grads))):
        err = normwise_rel(g.numpy(), r)
        worst = max(worst, err)
        assert err <= GRAD_TOL, i
    ref_norm = float(np.sqrt(sum(float(np.sum(r.astype(np.float64) ** 2)) for r in ts.param_list(grads))))
    norm, _ = st.norm_clip.numpy()
    print(f"[tiny step] worst gradient normwise {worst:.2e}; norm {norm:.6f} oracle {ref_norm:.6f}", flush=True)
    assert abs(norm - ref_norm) <= 1e-5 * ref_norm


def test_train_step_graph_and_side_stream_bit_identical(it):
    """Two steps: eager on one stream vs eager then graph replay with the side stream."""
    from irontensor_amd.train import TrainStep
    a = TrainStep(TINY, seed=11, overlap_weight_grads=False)
    b = TrainStep(TINY, seed=11, overlap_weight_grads=True)
    a.step()
    a.step()
    b.step()
    b.capture()
    b.step()  # replay
    it.Context.global_().sync()
    for x, y in zip(a.params, b.params):
        assert np.array_equal(x.numpy(), y.numpy())
    assert a.loss_value() == b.loss_value()
    b.close()


def test_train_step_dw_fork_modes_bit_identical(it):
    """Weight gradients issued one by one and forked to the side stream per GEMM or per layer: the
    same parameters after two graph-replayed steps, bit for bit."""
    from irontensor_amd.train import TrainStep
    a = TrainStep(TINY, seed=17, dw_fork="gemm", overlap_weight_grads=True, group_weight_grads=False)
    b = TrainStep(TINY, seed=17, dw_fork="layer", overlap_weight_grads=True, group_weight_grads=False)
    for st in (a, b):
        st.step()
        st.capture()
        st.step()
    it.Context.global_().sync()
    for x, y in zip(a.params, b.params):
        assert np.array_equal(x.numpy(), y.numpy())
    a.close()
    b.close()


def test_train_step_grouped_weight_gradients(it):
    """TINY: each layer's weight gradients as one grouped launch (the default) against the same
    GEMMs issued one by one: the same loss and data gradients bit for bit (the grouping touches only
    the weight-gradient GEMMs), weight gradients within the FP32 GEMM contract (normwise 1e-5: the
    group's split-K changes the summation order over K = 4096; measured 1.05e-6)."""
    from irontensor_amd import profiler
    from irontensor_amd.train import TrainStep
    ctx = it.Context.global_()
    a = TrainStep(TINY, seed=19, group_weight_grads=False)
    b = TrainStep(TINY, seed=19)
    a.step()
    profiler.reset(ctx)
    profiler.enable(ctx)
    b.step()
    ctx.sync()
    keys = [k for k in profiler.stats(ctx) if "_group" in k]
    profiler.enable(ctx, False)
    print(f"[tiny] grouped launches: {keys}", flush=True)
    assert len(keys) == 1 and keys[0].startswith("gemm_f32_TN_64x64_group")
    assert a.loss_value() == b.loss_value()
    L = TINY.layers
    dw = {id(t) for l in range(L) for t in (a.dWqkv[l], a.dWo[l], a.dWgu[l], a.dWd[l])}
    for i, (x, y) in enumerate(zip(a.grads, b.grads)):
        if id(x) in dw:
            assert normwise_rel(y.numpy(), x.numpy()) <= FP32_TOL, i
        else:
            assert np.array_equal(y.numpy(), x.numpy()), i


def test_train_step_xent_operand_matches_stored_gradient(it):
    """TINY: one step with the cross-entropy operand against one with the stored gradient: the
    same loss, and gradients equal to FP32 rounding (the rebuilt gradient is the stored one element
    for element; only the GEMMs' summation order differs: the LM-head data gradient runs on 256 x 128
    tiles with eight k splits from the stored gradient, on 64 x 64 tiles with two from the logits)."""
    from irontensor_amd.train import TrainStep
    a = TrainStep(TINY, seed=13, xent_operand=False)
    b = TrainStep(TINY, seed=13, xent_operand=True)
    a.step()
    b.step()
    it.Context.global_().sync()
    assert a.loss_value() == b.loss_value()
    for i, (x, y) in enumerate(zip(a.grads, b.grads)):
        assert normwise_rel(y.numpy(), x.numpy()) <= FP32_TOL, i


def test_train_step_tiny_loss_decreases(it):
    """TINY learns its fixed batch: the loss starts near log(vocab) and falls."""
    from irontensor_amd.train import TrainStep
    st = TrainStep(TINY, seed=3)
    st.step()
    st.capture()
    losses = [st.loss_value()]
    for _ in range(15):
        st.step()
        losses.append(st.loss_value())
    print(f"[tiny] losses {losses[0]:.4f} -> {losses[-1]:.4f}, grad norm {st.grad_norm():.4f}", flush=True)
    assert abs(losses[0] - np.log(TINY.vocab)) < 0.1
    assert losses[-1] < losses[0] - 0.2
    assert all(np.isfinite(losses))
    st.close()
