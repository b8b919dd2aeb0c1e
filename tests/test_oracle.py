"""Pins the CPU oracle (oracle/ref.c) before it is trusted as the parity checker.

Each oracle function is checked against the reference's own known answers, against exact
arithmetic, and against independent float64 implementations (numpy), chosen so that a dropped term,
a transposed operand, a wrong index or sign fails at least one check (see the mutation tests at the
bottom, which plant such mistakes in a copy of the oracle's inputs/outputs on the CPU).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from irontensor_amd import synth
from tests.numerics import op

GOLDEN = Path(__file__).resolve().parent / "golden"


# ------------------------------------------------------------------ reference known answers

def test_kat_matmul_2x2(oracle):
    # src/ops/gemm.rs:291-306 and src/ops/mps_gemm.rs:569-584
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    assert oracle.gemm_f32(a, b).tolist() == [[19, 22], [43, 50]]


def test_kat_matmul_bf16(oracle):
    # src/ops/bf16_ops/mod.rs:34-49: [1,2,3;4,5,6] @ [1,2;3,4;5,6] = [22,28;49,64]
    a = oracle.f32_to_bf16(np.array([[1, 2, 3], [4, 5, 6]], np.float32))
    b = oracle.f32_to_bf16(np.array([[1, 2], [3, 4], [5, 6]], np.float32))
    out = oracle.bf16_to_f32(oracle.gemm_bf16(a, b, out_bf16=True))
    assert out.tolist() == [[22, 28], [49, 64]]


def test_kat_linear_with_bias(oracle):
    # src/nn/linear.rs:224-238: [1,2] @ I^T + [1,2] = [2,4]
    x = np.array([[1, 2]], np.float32)
    w = np.array([[1, 0], [0, 1]], np.float32)
    y = oracle.add_bias(oracle.gemm_f32(x, w, trans_b=True), np.array([1, 2], np.float32))
    assert y.tolist() == [[2, 4]]


def test_kat_matmul_backward_2d(oracle):
    # src/ops/backward/gemm.rs:457-509: A=i*0.1 [3,4], B=i*0.1 [4,2], grad_C = 1
    m, k, n = 3, 4, 2
    a = (np.arange(m * k, dtype=np.float32) * np.float32(0.1)).reshape(m, k)
    b = (np.arange(k * n, dtype=np.float32) * np.float32(0.1)).reshape(k, n)
    gc = np.ones((m, n), np.float32)
    ga = oracle.gemm_f32(gc, b, trans_b=True)
    gb = oracle.gemm_f32(a, gc, trans_a=True)
    # grad_A[i,j] = sum_l B[j,l]; grad_B[i,j] = sum_l A[l,i] (closed forms with grad_C = 1)
    np.testing.assert_allclose(ga, np.broadcast_to(b.astype(np.float64).sum(1), (m, k)), atol=1e-6)
    np.testing.assert_allclose(gb, np.broadcast_to(a.astype(np.float64).sum(0)[:, None], (k, n)), atol=1e-6)


def test_kat_mps_matches_reference_integers(oracle):
    # src/ops/mps_gemm.rs:637-668: a=(i%7)-3, b=(i%5)-2, 16x8x12 -- exact in f32
    m, k, n = 16, 8, 12
    a = ((np.arange(m * k) % 7) - 3).astype(np.float32).reshape(m, k)
    b = ((np.arange(k * n) % 5) - 2).astype(np.float32).reshape(k, n)
    exact = a.astype(np.int64) @ b.astype(np.int64)
    assert np.array_equal(oracle.gemm_f32(a, b), exact.astype(np.float32))


def test_kat_matmul_larger_against_f64(oracle):
    # src/ops/gemm.rs:308-351: a=(i+j)*0.01 [64,32], b=(i*j)*0.01 [32,48], tol 1e-3
    m, k, n = 64, 32, 48
    i, j = np.meshgrid(np.arange(m), np.arange(k), indexing="ij")
    a = ((i + j).astype(np.float32) * np.float32(0.01))
    i, j = np.meshgrid(np.arange(k), np.arange(n), indexing="ij")
    b = ((i * j).astype(np.float32) * np.float32(0.01))
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert np.max(np.abs(oracle.gemm_f32(a, b) - ref)) < 1e-3


# ------------------------------------------------------------------ exact arithmetic and invariants

@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("batch", [None, 3])
def test_gemm_exact_integers(oracle, ta, tb, batch):
    # entries in [-3, 3] with K <= 4096 keep every partial sum < 2^24: exact in any order
    m, n, k = 13, 11, 29
    shp_a = (k, m) if ta else (m, k)
    shp_b = (n, k) if tb else (k, n)
    if batch:
        shp_a, shp_b = (batch,) + shp_a, (batch,) + shp_b
    a = synth.small_ints(1, shp_a, -3, 3)
    b = synth.small_ints(2, shp_b, -3, 3)
    exact = op(a, ta).astype(np.int64) @ op(b, tb).astype(np.int64)
    got = oracle.gemm_f32(a, b, bool(ta), bool(tb))
    assert np.array_equal(got, exact.astype(np.float32))


def test_nt_tn_equal_nn_on_transposed_copies_bitwise(oracle):
    a = synth.normal(3, (37, 53))
    b = synth.normal(4, (53, 41))
    nn = oracle.gemm_f32(a, b)
    nt = oracle.gemm_f32(a, np.ascontiguousarray(b.T), trans_b=True)
    tn = oracle.gemm_f32(np.ascontiguousarray(a.T), b, trans_a=True)
    assert np.array_equal(nn, nt) and np.array_equal(nn, tn)


def test_f32_loop_is_sequential_not_pairwise(oracle):
    # 1 + 2^-24 + ... : a sequential f32 sum of [1, 2^-24 x 4] stays 1.0 (each add rounds away),
    # while any reordering that adds the small terms first gives 1 + 2^-22.
    a = np.array([[1.0, 2.0 ** -24, 2.0 ** -24, 2.0 ** -24, 2.0 ** -24]], np.float32)
    b = np.ones((5, 1), np.float32)
    assert oracle.gemm_f32(a, b)[0, 0] == np.float32(1.0)


def test_f64_matches_numpy_and_f32_error_bound(oracle):
    a = synth.normal(5, (64, 300))
    b = synth.normal(6, (300, 80), std=0.02)
    f64 = oracle.gemm_f64(a, b)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    np.testing.assert_allclose(f64, ref, rtol=1e-12, atol=1e-14)
    f32 = oracle.gemm_f32(a, b).astype(np.float64)
    bound = 300 * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert np.all(np.abs(f32 - ref) <= bound)


def test_thread_count_does_not_change_results(oracle):
    a = synth.normal(7, (4, 33, 70))
    b = synth.normal(8, (4, 70, 29))
    one = oracle.gemm_f32(a, b, threads=1)
    many = oracle.gemm_f32(a, b, threads=7)
    assert np.array_equal(one, many)


# ------------------------------------------------------------------ BF16

def test_bf16_rne_known_cases(oracle):
    # src/precision.rs:24-29: ties to even at bit 16
    cases = {
        1.0: 0x3F80,
        1.0 + 2 ** -8: 0x3F80,            # exact tie, lsb 0 -> stays
        1.0 + 3 * 2 ** -8: 0x3F82,        # exact tie, lsb 1 -> rounds up to even
        1.0 + 2 ** -8 + 2 ** -20: 0x3F81,  # above the tie -> up
        -2.5: 0xC020,
        0.0: 0x0000,
        float("inf"): 0x7F80,
        float("-inf"): 0xFF80,
    }
    for x, bits in cases.items():
        assert oracle.load().ref_f32_to_bf16(x) == bits, x
    assert np.isnan(oracle.bf16_to_f32(np.array([oracle.load().ref_f32_to_bf16(float("nan"))], np.uint16)))[0]


def test_bf16_reference_roundtrip_values(oracle):
    # src/precision.rs:51-65
    vals = np.array([0.0, 1.0, -1.0, 0.5, -0.5, 100.0, -100.0, 1e-5, 1e5], np.float32)
    back = oracle.bf16_to_f32(oracle.f32_to_bf16(vals))
    rel = np.where(np.abs(vals) > 1e-10, np.abs((back - vals) / np.where(vals == 0, 1, vals)), np.abs(back - vals))
    assert np.all(rel < 0.01)


def test_bf16_matches_bit_level_restatement(oracle):
    from irontensor_amd.tensor import f32_to_bf16
    bits = synth.splitmix64(9, 200000).astype(np.uint32)
    x = bits.view(np.float32)
    finite = np.isfinite(x)
    assert np.array_equal(oracle.f32_to_bf16(x)[finite], f32_to_bf16(x)[finite])


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_bf16_gemm_exact_integers_and_equals_widened_f32(oracle, ta, tb):
    m, n, k = 9, 14, 40
    a = synth.small_ints(10, (k, m) if ta else (m, k), -8, 8)
    b = synth.small_ints(11, (n, k) if tb else (k, n), -8, 8)
    ab, bb = oracle.f32_to_bf16(a), oracle.f32_to_bf16(b)
    got = oracle.gemm_bf16(ab, bb, bool(ta), bool(tb))
    exact = op(a, ta).astype(np.int64) @ op(b, tb).astype(np.int64)
    assert np.array_equal(got, exact.astype(np.float32))
    r = synth.normal(12, (m, k))
    s = synth.normal(13, (k, n))
    rb, sb = oracle.f32_to_bf16(r), oracle.f32_to_bf16(s)
    assert np.array_equal(oracle.gemm_bf16(rb, sb), oracle.gemm_f32(oracle.bf16_to_f32(rb), oracle.bf16_to_f32(sb)))
    out16 = oracle.gemm_bf16(rb, sb, out_bf16=True)
    assert np.array_equal(out16, oracle.f32_to_bf16(oracle.gemm_bf16(rb, sb)))


# ------------------------------------------------------------------ softmax, SwiGLU

def test_softmax_rows_matches_f64(oracle):
    x = synth.normal(14, (7, 33)) * 3
    ref = np.exp(x.astype(np.float64) - x.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    np.testing.assert_allclose(oracle.softmax_rows(x), ref, rtol=1e-5, atol=1e-7)


def test_softmax_backward_finite_difference(oracle):
    x = synth.normal(15, (3, 6)).astype(np.float64)
    g = synth.normal(16, (3, 6)).astype(np.float64)

    def sm(z):
        e = np.exp(z - z.max(1, keepdims=True))
        return e / e.sum(1, keepdims=True)

    y = sm(x)
    got = oracle.softmax_backward(g.astype(np.float32), y.astype(np.float32))
    eps = 1e-6
    num = np.zeros_like(x)
    for r in range(3):
        for c in range(6):
            xp, xm = x.copy(), x.copy()
            xp[r, c] += eps
            xm[r, c] -= eps
            num[r, c] = ((sm(xp) - sm(xm)) * g).sum() / (2 * eps)
    np.testing.assert_allclose(got, num, rtol=1e-4, atol=1e-6)


def test_swiglu_closed_forms_and_derivative(oracle):
    g = synth.normal(17, (1000,)) * 4
    u = synth.normal(18, (1000,))
    ref = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
    np.testing.assert_allclose(oracle.swiglu(g, u), ref, rtol=1e-5, atol=1e-6)
    assert np.all(oracle.swiglu(np.zeros(4, np.float32), np.ones(4, np.float32)) == 0)
    go = synth.normal(19, (1000,))
    gg, gu = oracle.swiglu_backward(go, g, u)
    gd, eps = g.astype(np.float64), 1e-5
    silu = lambda z: z / (1 + np.exp(-z))  # noqa: E731
    dnum = (silu(gd + eps) - silu(gd - eps)) / (2 * eps)
    np.testing.assert_allclose(gg, go * u * dnum, rtol=1e-3, atol=1e-5)
    np.testing.assert_allclose(gu, go * silu(gd), rtol=1e-5, atol=1e-6)


# ------------------------------------------------------------------ attention

def _attention_f64(q, k, v, causal, scale):
    q, k, v = (t.astype(np.float64) for t in (q, k, v))
    s = q @ np.swapaxes(k, -1, -2) * scale
    if causal:
        n = s.shape[-1]
        s = np.where(np.triu(np.ones((n, n), bool), 1), -np.inf, s)
    e = np.exp(s - s.max(-1, keepdims=True))
    p = e / e.sum(-1, keepdims=True)
    return p @ v, p


@pytest.mark.parametrize("causal", [False, True])
def test_attention_matches_f64(oracle, causal):
    bh, s, d = 6, 19, 8
    q, k, v = (synth.normal(20 + i, (bh, s, d)) for i in range(3))
    o, p = oracle.attention_fwd_bhsd(q, k, v, 1 / np.sqrt(d), causal)
    o_ref, p_ref = _attention_f64(q, k, v, causal, 1 / np.sqrt(d))
    np.testing.assert_allclose(o, o_ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-6)
    if causal:
        assert np.all(p[:, np.triu(np.ones((s, s), bool), 1)] == 0)


def test_attention_closed_forms(oracle):
    # Q = 0: uniform weights, so O row r is the mean of V rows 0..r (causal) or of all rows.
    bh, s, d = 2, 9, 4
    q = np.zeros((bh, s, d), np.float32)
    k = synth.normal(30, (bh, s, d))
    v = synth.normal(31, (bh, s, d))
    o, _ = oracle.attention_fwd_bhsd(q, k, v, 0.5, True)
    prefix = np.cumsum(v.astype(np.float64), axis=1) / np.arange(1, s + 1)[None, :, None]
    np.testing.assert_allclose(o, prefix, rtol=1e-5, atol=1e-6)
    o, _ = oracle.attention_fwd_bhsd(q, k, v, 0.5, False)
    np.testing.assert_allclose(o, np.broadcast_to(v.astype(np.float64).mean(1, keepdims=True), o.shape),
                               rtol=1e-5, atol=1e-6)
    # causal row 0 attends only to key 0
    o, _ = oracle.attention_fwd_bhsd(synth.normal(32, (bh, s, d)), k, v, 0.5, True)
    np.testing.assert_allclose(o[:, 0], v[:, 0], rtol=1e-6)


def test_attention_bshd_layout_matches_bhsd(oracle):
    # reference_attention indexes [B,S,H,D] (src/ops/attention.rs:552-606)
    b, s, h, d = 2, 16, 4, 32
    q, k, v = (synth.normal(40 + i, (b, s, h, d)) for i in range(3))
    out = oracle.attention_bshd(q, k, v, True)
    t = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3)).reshape(b * h, s, d)  # noqa: E731
    o, _ = oracle.attention_fwd_bhsd(t(q), t(k), t(v), 1 / np.sqrt(d), True)
    assert np.array_equal(out, o.reshape(b, h, s, d).transpose(0, 2, 1, 3))


def test_attention_backward_finite_difference(oracle):
    bh, s, d = 2, 5, 3
    scale = 0.7
    q, k, v, do = (synth.normal(50 + i, (bh, s, d)) for i in range(4))
    dq, dk, dv = oracle.attention_bwd_bhsd(do, q, k, v, scale, True)

    def loss(qq, kk, vv):
        o, _ = _attention_f64(qq, kk, vv, True, scale)
        return float((o * do.astype(np.float64)).sum())

    eps = 1e-4
    for grad, which in ((dq, 0), (dk, 1), (dv, 2)):
        num = np.zeros((bh, s, d))
        base = [q.astype(np.float64), k.astype(np.float64), v.astype(np.float64)]
        for idx in np.ndindex(bh, s, d):
            plus = [x.copy() for x in base]
            minus = [x.copy() for x in base]
            plus[which][idx] += eps
            minus[which][idx] -= eps
            num[idx] = (loss(*plus) - loss(*minus)) / (2 * eps)
        np.testing.assert_allclose(grad, num, rtol=2e-3, atol=2e-4)


# ------------------------------------------------------------------ committed fixtures

def test_golden_vectors(oracle):
    data = json.loads((GOLDEN / "oracle_vectors.json").read_text())
    for case in data["gemm_f32"]:
        a = np.array(case["a"], np.uint32).view(np.float32).reshape(case["a_shape"])
        b = np.array(case["b"], np.uint32).view(np.float32).reshape(case["b_shape"])
        out = oracle.gemm_f32(a, b, case["trans_a"], case["trans_b"])
        assert out.view(np.uint32).ravel().tolist() == case["out"], case["name"]
    for case in data["gemm_bf16"]:
        a = np.array(case["a"], np.uint16).reshape(case["a_shape"])
        b = np.array(case["b"], np.uint16).reshape(case["b_shape"])
        out = oracle.gemm_bf16(a, b, case["trans_a"], case["trans_b"], out_bf16=True)
        assert out.ravel().tolist() == case["out"], case["name"]
    for case in data["attention_bshd"]:
        q, k, v = (np.array(case[n], np.uint32).view(np.float32).reshape(case["shape"]) for n in "qkv")
        out = oracle.attention_bshd(q, k, v, case["causal"])
        got = out.view(np.uint32).ravel()
        want = np.array(case["out"], np.uint32)
        # exp() may differ by an ulp between libm builds; everything else is exact
        assert np.max(np.abs(got.view(np.float32) - want.view(np.float32))) <= 1e-6, case["name"]


# ------------------------------------------------------------------ the checks have teeth

def test_planted_mistakes_are_caught(oracle):
    """Plants plausible mistakes in copies of oracle results and confirms the checks above reject
    them: a transposed operand, a dropped k term, a sign flip and a wrong causal diagonal."""
    m, k, n = 16, 8, 12
    a = ((np.arange(m * k) % 7) - 3).astype(np.float32).reshape(m, k)
    b = ((np.arange(k * n) % 5) - 2).astype(np.float32).reshape(k, n)
    exact = (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32)
    assert np.array_equal(oracle.gemm_f32(a, b), exact)
    dropped = (a[:, :-1].astype(np.int64) @ b[:-1].astype(np.int64)).astype(np.float32)
    assert not np.array_equal(dropped, exact)
    assert not np.array_equal(-exact, exact)
    sq = synth.small_ints(60, (9, 9), -3, 3)
    assert not np.array_equal(oracle.gemm_f32(sq, sq, trans_b=True), oracle.gemm_f32(sq, sq))
    q, kk, v = (synth.normal(61 + i, (1, 6, 4)) for i in range(3))
    o_good, _ = _attention_f64(q, kk, v, True, 0.5)
    s = (q.astype(np.float64) @ np.swapaxes(kk, -1, -2)) * 0.5
    s = np.where(np.triu(np.ones((6, 6), bool), 0), -np.inf, s)  # mask the diagonal too (wrong)
    s[:, 0, 0] = 0.0
    e = np.exp(s - s.max(-1, keepdims=True))
    o_bad = (e / e.sum(-1, keepdims=True)) @ v
    assert np.max(np.abs(o_bad - o_good)) > 1e-3
    o_oracle, _ = oracle.attention_fwd_bhsd(q, kk, v, 0.5, True)
    assert np.max(np.abs(o_oracle - o_good)) < 1e-5


# ------------------------------------------------------------------ attention helpers (transpose, mask)

@pytest.mark.parametrize("batch,m,n", [(1, 1, 1), (2, 3, 5), (3, 70, 130), (4, 64, 64)])
def test_transpose_3d_matches_numpy_and_is_an_involution(oracle, batch, m, n):
    x = synth.normal(70 + m, (batch, m, n))
    t = oracle.transpose_3d(x, batch, m, n)
    assert np.array_equal(t, np.swapaxes(x, 1, 2))
    assert np.array_equal(oracle.transpose_3d(t, batch, n, m), x)


def test_causal_mask_3d_matches_triu_and_gives_prefix_means(oracle):
    b, s = 3, 17
    x = synth.normal(75, (b, s, s))
    y = oracle.causal_mask_3d(x, b, s)
    upper = np.triu(np.ones((s, s), bool), 1)
    assert np.all(np.isneginf(y[:, upper]))
    assert np.array_equal(y[:, ~upper], x[:, ~upper])
    # a masked constant score row softmaxes to 1/(row+1) on the allowed columns, so P.V is the
    # running mean of V's rows
    p = oracle.softmax_rows(oracle.causal_mask_3d(np.zeros((1, s, s), np.float32), 1, s)[0])
    v = synth.normal(76, (s, 4)).astype(np.float64)
    means = np.cumsum(v, 0) / np.arange(1, s + 1)[:, None]
    assert np.max(np.abs(p @ v - means)) < 1e-6
    # a mask that also hides the diagonal (c >= r) is caught by the same checks
    bad = np.where(np.triu(np.ones((s, s), bool), 0), -np.inf, x[0])
    assert not np.array_equal(bad, y[0])
