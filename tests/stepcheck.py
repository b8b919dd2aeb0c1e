"""Sampled-row parity of one GEMM of a GemmStep against the oracle (a helper of the step tests).

A recorded call (GemmStep._calls) is launched again alone with the library profiler on, so its
plan (kernel, tile, split-K) is known; then `rows` sampled output rows are compared with the oracle
on the same operands read back from the device:

* FP32 operands: normwise FP32_TOL against oracle.gemm_f32;
* BF16 operands: against oracle.gemm_bf16 (FP32 sums of the same BF16 values) normwise FP32_TOL for
  an FP32 output, and within half a BF16 ulp plus FP32_TOL for a BF16 output; and relative
  Frobenius BF16_FROB_TOL against oracle.gemm_f32 on the unrounded seeded inputs (regenerated on
  the host from the step's seeds; an operand that a GEMM wrote has no unrounded form and enters
  as its BF16 value).
The fused SwiGLU call (bias + dual B) is checked on gate, up and h = silu(gate) * up.
"""
from __future__ import annotations

import numpy as np

from irontensor_amd import _lib, profiler, synth
from irontensor_amd.tensor import Precision
from tests.numerics import BF16_FROB_TOL, FP32_TOL, bf16_out_excess, frob_rel, normwise_rel


def sample_rows(m: int, count: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    rows = set(rng.choice(m, size=min(count, m), replace=False).tolist()) | {0, m - 1}
    return np.array(sorted(rows), dtype=np.int64)


class StepChecker:
    def __init__(self, it, oracle, step, rows: int = 64, log=print):
        self.it, self.oracle, self.st, self.nrows, self.log = it, oracle, step, rows, log
        self._f32_cache = {}

    # -------------------------------------------------------------- operands
    def _host(self, t):
        """Device tensor -> host array in its own dtype (uint16 for BF16)."""
        if t.precision() is Precision.BF16:
            return t.as_bf16_slice().reshape(t.shape())
        return t.as_f32_slice().reshape(t.shape())

    def _unrounded(self, t, idx2d):
        """f32 values of seeded tensor t at [rows, cols] index arrays (np.ix_ style), regenerated
        on the host; None when t was not seeded (a GEMM or kernel wrote it)."""
        info = self.st.seed_of.get(t.ptr)
        if info is None:
            return None
        seed, std = info
        cols = t.shape()[-1]
        r, c = idx2d
        flat = np.asarray(r)[:, None] * cols + np.asarray(c)[None, :]
        return synth.normal_at(seed, flat, std=std)

    def _full_unrounded(self, t):
        if t.ptr not in self._f32_cache:
            info = self.st.seed_of.get(t.ptr)
            self._f32_cache[t.ptr] = None if info is None else synth.normal(info[0], t.shape(), std=info[1])
        return self._f32_cache[t.ptr]

    # -------------------------------------------------------------- one call
    def check_call(self, key) -> str:
        it, oracle, st = self.it, self.oracle, self.st
        name, A, B, Cout, ta, tb, M, N, K, alpha, epi, a_off, lda = st._calls[key]
        assert a_off == 0 and lda == A.shape()[-1], name
        ctx = st.ctx
        profiler.reset(ctx)
        profiler.enable(ctx)
        st.reissue(*key)
        plans = list(profiler.stats(ctx))
        profiler.enable(ctx, False)
        ctx.sync()
        assert len(plans) == 1, plans
        plan = plans[0]
        rows = sample_rows(M, self.nrows, seed=M * 31 + N * 7 + K)
        a = self._host(A)
        b = self._host(B)
        a_rows = a[:, rows] if ta else a[rows, :]
        bf16 = A.precision() is Precision.BF16
        dual = epi is not None and epi.flags & _lib.IT_EPI_SWIGLU
        has_bias = epi is not None and epi.flags & _lib.IT_EPI_BIAS
        if dual:
            F = N
            wg, wu = b[:F], b[F:2 * F]
            bias = st.bgu[st.Wgu.index(B)].numpy() if has_bias else np.zeros(2 * F, np.float32)
            refs = self._products(A, B, a_rows, rows, (wg, wu), ta, tb, bf16, split_b=F)
            g_ref = [oracle.add_bias(r, bias[:F]) for r in refs["g"]]
            u_ref = [oracle.add_bias(r, bias[F:]) for r in refs["u"]]
            li = st.Wgu.index(B)
            outs = {"gate": (st.G[li], g_ref), "up": (st.U[li], u_ref),
                    "h": (Cout, [oracle.swiglu(g, u) for g, u in zip(g_ref, u_ref)])}
        else:
            assert not has_bias
            refs = self._products(A, B, a_rows, rows, (b,), ta, tb, bf16)
            outs = {"out": (Cout, [r * np.float32(alpha) for r in refs["g"]])}
        msgs = []
        for what, (t, (ref_same, ref_unrounded)) in outs.items():
            got = t.numpy().reshape(M, -1)[rows]
            if t.precision() is Precision.BF16:
                e1 = bf16_out_excess(got, ref_same)
            else:
                e1 = normwise_rel(got, ref_same)
            assert e1 <= FP32_TOL, (name, plan, what, e1)
            msg = f"{what}: same-operand {e1:.2e}"
            if bf16:
                e2 = frob_rel(got, ref_unrounded)
                assert e2 <= BF16_FROB_TOL, (name, plan, what, e2)
                msg += f", frob vs unrounded {e2:.2e}"
            msgs.append(msg)
        line = f"[{name}] {plan}: {len(rows)} rows; " + "; ".join(msgs)
        self.log(line)
        return plan

    def _products(self, A, B, a_rows, rows, bparts, ta, tb, bf16, split_b=None):
        """{"g": (same-operand product, unrounded product)} and, for two B parts, "u" too."""
        oracle = self.oracle
        out = {}
        for tag, bp in zip(("g", "u"), bparts):
            if bf16:
                same = oracle.gemm_bf16(np.ascontiguousarray(a_rows), np.ascontiguousarray(bp), ta, tb)
                ka = A.shape()[0] if ta else A.shape()[1]
                idx = (np.arange(ka), rows) if ta else (rows, np.arange(ka))
                a32 = self._unrounded(A, idx)
                if a32 is None:
                    a32 = self.it.bf16_to_f32(a_rows)
                b32 = self._full_unrounded(B)
                if b32 is None:
                    b32 = self.it.bf16_to_f32(np.asarray(self._host(B)))
                if split_b is not None:
                    off = 0 if tag == "g" else split_b
                    b32 = b32[off:off + split_b]
                unr = oracle.gemm_f32(np.ascontiguousarray(a32, np.float32), np.ascontiguousarray(b32, np.float32),
                                      ta, tb)
            else:
                same = oracle.gemm_f32(np.ascontiguousarray(a_rows), np.ascontiguousarray(bp), ta, tb)
                unr = same
            out[tag] = (same, unr)
        # regroup as {"g": [same, unrounded], "u": [...]}
        return {k: list(v) for k, v in out.items()}
