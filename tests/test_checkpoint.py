"""The IRON v2 checkpoint format (irontensor_amd/checkpoint.py) against the byte layout the
reference writes (src/train/checkpoint.rs:52-181,318-334; optimizer state src/nn/model.rs:462-487),
round trips, the reference's error cases, and (GPU) a TrainStep saved and restored bit-exactly."""
from __future__ import annotations

import io
import struct

import numpy as np
import pytest

from irontensor_amd import checkpoint as ck
from irontensor_amd import synth


def _tiny(seed=1, layers=2, h=8, f=12, v=11):
    rng = np.random.default_rng(seed)
    r = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    lay = [{"wq": r(h, h), "wk": r(h, h), "wv": r(h, h), "wo": r(h, h), "w_gate": r(f, h), "w_up": r(f, h),
            "w_down": r(h, f), "attn_norm": r(h), "ffn_norm": r(h)} for _ in range(layers)]
    w = ck.Weights(r(v, h), lay, r(h))
    cfg = ck.ModelConfig(v, h, layers, 2, 2, f, 1e-5, 10000.0, 64, True, 0)
    return w, cfg


def test_save_load_tensor_reference_case():
    """test_save_load_tensor (src/train/checkpoint.rs:341-353) plus the exact bytes."""
    t = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    buf = io.BytesIO()
    ck.save_tensor(buf, t)
    raw = buf.getvalue()
    assert raw == struct.pack("<IQQ6f", 2, 2, 3, 1, 2, 3, 4, 5, 6)
    back = ck.load_tensor(io.BytesIO(raw))
    assert back.shape == (2, 3) and np.array_equal(back, t)


def test_header_and_config_bytes():
    w, cfg = _tiny()
    meta = ck.Checkpoint(cfg, step=7, epoch=3, best_val_loss=1.5, learning_rate=3e-4)
    raw = ck.to_bytes(w, meta)
    assert raw[:4] == b"NORI"  # 0x49524F4E little endian
    assert struct.unpack_from("<II", raw, 0) == (0x49524F4E, 2)
    assert struct.unpack_from("<QQff", raw, 8) == (7, 3, 1.5, np.float32(3e-4))
    off = 8 + 24
    assert struct.unpack_from("<QQQQQQ", raw, off) == (11, 8, 2, 2, 2, 12)
    assert struct.unpack_from("<ffQBB", raw, off + 48) == (np.float32(1e-5), 10000.0, 64, 1, 0)
    off += 48 + 18
    assert struct.unpack_from("<IQQ", raw, off) == (2, 11, 8)  # embed_tokens first
    # then per layer wq, wk, wv, wo, w_gate, w_up, w_down, attn_norm, ffn_norm
    off += 4 + 16 + 11 * 8 * 4
    assert struct.unpack_from("<IQQ", raw, off) == (2, 8, 8)
    assert np.array_equal(np.frombuffer(raw, "<f4", 64, off + 20).reshape(8, 8), w.layers[0]["wq"])
    # tail: final norm, tie flag 1, no optimizer state
    assert raw[-2:] == b"\x01\x00"


def test_round_trip_with_optimizer_and_untied_head():
    w, cfg = _tiny(seed=2)
    cfg.tie_weights = False
    w.output_weight = synth.normal(3, (11, 8))
    _, mcfg = _tiny(seed=4)
    mw, _ = _tiny(seed=5)
    opt = ck.OptimizerState(mw.embed_tokens, mw.layers, mw.final_norm, synth.normal(6, (11, 8)))
    raw = ck.to_bytes(w, ck.Checkpoint(cfg, 1, 2, 0.5, 1e-3), opt)
    w2, meta, opt2 = ck.load_model_weights(io.BytesIO(raw))
    assert meta.step == 1 and meta.epoch == 2 and meta.has_optimizer_state and not meta.config.tie_weights
    assert np.array_equal(w2.embed_tokens, w.embed_tokens) and np.array_equal(w2.output_weight, w.output_weight)
    for a, b in zip(w2.layers, w.layers):
        assert all(np.array_equal(a[k], b[k]) for k in ck.LAYER_KEYS)
    assert np.array_equal(opt2.output_weight, opt.output_weight)
    assert all(np.array_equal(opt2.layers[1][k], opt.layers[1][k]) for k in ck.LAYER_KEYS)
    # a reader that stops where the reference's reader stops still gets a whole v2 file
    tail = raw.index(ck.EXT_TAG)
    w3, meta3, opt3 = ck.load_model_weights(io.BytesIO(raw[:tail]))
    assert w3.output_weight is None and opt3 is not None


def test_version1_and_errors():
    w, cfg = _tiny(seed=7)
    raw = bytearray(ck.to_bytes(w, ck.Checkpoint(cfg)))
    v1 = bytearray(raw[:-1])  # version 1 files end after the tie flag
    struct.pack_into("<I", v1, 4, 1)
    w1, meta1, opt1 = ck.load_model_weights(io.BytesIO(bytes(v1)))
    assert opt1 is None and np.array_equal(w1.final_norm, w.final_norm)
    bad = bytearray(raw)
    struct.pack_into("<I", bad, 0, 0x12345678)
    with pytest.raises(ValueError, match="bad magic"):
        ck.load_model_weights(io.BytesIO(bytes(bad)))
    bad = bytearray(raw)
    struct.pack_into("<I", bad, 4, 3)
    with pytest.raises(ValueError, match="Unsupported checkpoint version: 3"):
        ck.load_model_weights(io.BytesIO(bytes(bad)))
    with pytest.raises(EOFError):
        ck.load_model_weights(io.BytesIO(bytes(raw[:200])))


@pytest.mark.gpu
def test_train_step_checkpoint_round_trip(it, tmp_path):
    """A TrainStep after two steps, saved and loaded into a fresh one: parameters and momenta
    bit-identical, and the next step identical in both."""
    from irontensor_amd.step import ModelShape
    from irontensor_amd.train import TrainStep
    shape = ModelShape("ck", 2, 128, 2, 64, 176, 1000, 2, 64)
    a = TrainStep(shape, seed=1)
    a.step()
    a.step()
    path = tmp_path / "step.iron"
    a.save_checkpoint(path, step=2)
    b = TrainStep(shape, seed=99)
    b.set_batch(a.ids_host, a.targets_host)
    meta = b.load_checkpoint(path)
    assert meta.step == 2 and meta.has_optimizer_state
    for x, y in zip(a.params + a.momentum, b.params + b.momentum):
        assert np.array_equal(x.numpy(), y.numpy())
    a.step()
    b.step()
    it.Context.global_().sync()
    assert a.loss_value() == b.loss_value()
    for x, y in zip(a.params, b.params):
        assert np.array_equal(x.numpy(), y.numpy())
