"""GPU conversions to_bf16_gpu / to_f32_gpu (src/ops/bf16_ops/precision.rs:15-78) against the oracle's
restatement of the reference's RNE formula (src/precision.rs:24-29): bit-exact for every non-NaN
input, NaN stays NaN; widening is exact for all 65536 BF16 patterns."""
from __future__ import annotations

import numpy as np
import pytest

from irontensor_amd import synth

pytestmark = pytest.mark.gpu


def _specials() -> np.ndarray:
    f32 = np.float32
    vals = [0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 100.0, -100.0, 1e-5, 1e5, -2.5,   # src/precision.rs:51-95
            1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20,         # ties and near-ties
            float("inf"), float("-inf"),
            float(np.finfo(f32).max), float(-np.finfo(f32).max),                # rounds to inf
            float(np.finfo(f32).tiny), 2 ** -127, 2 ** -130, 2 ** -149, -2 ** -149,  # denormals
            3.0 * 2 ** -135, 2 ** -133 + 2 ** -141]
    return np.array(vals, dtype=f32)


@pytest.mark.parametrize("n", [len(_specials()), 1 << 20, (1 << 20) + 5])
def test_to_bf16_gpu_bit_exact(it, oracle, n):
    base = _specials()
    x = np.concatenate([base, synth.normal(90, (n,)) * np.float32(37.0)])[:n] if n > len(base) else base
    # every 7th value scaled into the denormal range
    if n > len(base):
        x[::7] *= np.float32(2.0 ** -130)
    got = it.to_bf16_gpu(it.Tensor.from_f32_slice(x, [n])).as_bf16_slice()
    ref = oracle.f32_to_bf16(x)
    assert np.array_equal(got, ref)


def test_to_bf16_gpu_nan_stays_nan(it):
    x = np.array([np.nan, -np.nan, 1.0], np.float32)
    x[1] = np.frombuffer(np.uint32(0x7FA00001).tobytes(), np.float32)[0]  # signalling NaN payload
    got = it.to_bf16_gpu(it.Tensor.from_f32_slice(x, [3])).as_bf16_slice()
    back = it.bf16_to_f32(got)
    assert np.isnan(back[0]) and np.isnan(back[1]) and back[2] == 1.0
    assert (got[1] & 0x7F80) == 0x7F80 and (got[1] & 0x0040)  # quiet


def test_to_f32_gpu_all_patterns(it, oracle):
    pats = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = it.to_f32_gpu(it.Tensor.from_bf16_slice(pats, [1 << 16])).numpy()
    ref = oracle.bf16_to_f32(pats)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
