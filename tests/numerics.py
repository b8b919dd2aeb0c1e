"""Error metrics used by the parity tests (fixed here so every test states the same contract).

FP32 parity: normwise max relative error  max|x - ref| / max|ref|  <= 1e-5, against the oracle's
sequential f32 loop on the same inputs. A per-element relative error is ill-conditioned where
sums cancel to near zero (inputs are zero-mean), so the normwise form is the contract; the
per-element bound |x - ref| <= tol * (|A|.|B|)_ij is checked alongside where cheap.
BF16 parity: relative Frobenius error  ||x - ref||_F / ||ref||_F  <= 1e-2 against the f32 oracle
on the unrounded f32 inputs.
"""
from __future__ import annotations

import numpy as np

FP32_TOL = 1e-5
BF16_FROB_TOL = 1e-2


def normwise_rel(x, ref) -> float:
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.max(np.abs(ref)) if ref.size else 0.0
    diff = np.max(np.abs(x - ref)) if ref.size else 0.0
    return float(diff / denom) if denom > 0 else float(diff)


def frob_rel(x, ref) -> float:
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    denom = np.linalg.norm(ref)
    diff = np.linalg.norm(x - ref)
    return float(diff / denom) if denom > 0 else float(diff)


def op(a, trans):
    return np.swapaxes(a, -1, -2) if trans else a


# A BF16 output is the round-to-nearest-even of an FP32 sum, and RNE moves a value by at most half a
# BF16 ulp, 2^-8 of its magnitude. Against the oracle's FP32 sum on the same operands, a BF16 output
# may therefore differ by 2^-8 |ref| plus the summation-order difference of the FP32 sums, which is
# held to the FP32 contract (FP32_TOL of the largest reference magnitude).
BF16_HALF_ULP = 2.0 ** -8


def bf16_out_excess(x, ref) -> float:
    """max over elements of (|x - ref| - 2^-8 |ref|) / max|ref|: <= FP32_TOL when x is a BF16
    rounding of an FP32 result that meets the FP32 contract against ref."""
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if not ref.size:
        return 0.0
    denom = np.max(np.abs(ref)) or 1.0
    return float(np.max(np.abs(x - ref) - BF16_HALF_ULP * np.abs(ref)) / denom)
