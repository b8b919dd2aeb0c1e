"""IronTensor's "IRON" checkpoint format (version 2), read and written on the host.

Byte layout (little endian), as src/train/checkpoint.rs:11-17,52-104,137-181,318-334 writes it:

    u32 magic 0x49524F4E ("IRON"), u32 version (2; version 1 is read too)
    u64 step, u64 epoch, f32 best_val_loss, f32 learning_rate
    config: u64 vocab_size, hidden_dim, num_layers, num_heads, num_kv_heads, intermediate_dim;
            f32 norm_eps, rope_base; u64 max_seq_len; u8 tie_weights; u8 precision (0 FP32, 1 FP16, 2 BF16)
    tensors, each u32 ndim, ndim x u64 dims, f32 data (BF16 is widened to FP32 on save):
            embed_tokens; per layer wq, wk, wv, wo, w_gate, w_up, w_down, attn_norm, ffn_norm;
            final_norm
    u8 tie_weights
    u8 has_optimizer_state, then (src/nn/model.rs:462-487) the Lion momenta as tensors:
            embed; u32 num_layers; per layer wq, wk, wv, wo, w_gate, w_up, w_down, attn_norm,
            ffn_norm (src/nn/transformer.rs:120-126, attention.rs:296-302, ffn.rs:121-126);
            final_norm; u8 has_output_state [+ output weight momentum]

The reference does not store an untied output projection's weights (its trainer multiplies by
embed_tokens, src/train/trainer/mod.rs:228-235). A file written here for an untied model appends
that matrix after the reference's last field as an extension block (b"IRTX", u32 1, the tensor);
the reference's reader stops before it, so the file stays loadable there.
"""
from __future__ import annotations

import io
import struct
from dataclasses import dataclass, field
from typing import BinaryIO, Dict, List, Optional, Tuple

import numpy as np

MAGIC = 0x49524F4E
VERSION = 2
MIN_VERSION = 1
EXT_TAG = b"IRTX"
LAYER_KEYS = ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down", "attn_norm", "ffn_norm")


@dataclass
class ModelConfig:
    """ModelConfig fields stored in a checkpoint (src/train/checkpoint.rs:318-334)."""
    vocab_size: int
    hidden_dim: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    intermediate_dim: int
    norm_eps: float = 1e-5
    rope_base: float = 10000.0
    max_seq_len: int = 512
    tie_weights: bool = True
    precision: int = 0  # 0 FP32, 1 FP16, 2 BF16


@dataclass
class Checkpoint:
    """Checkpoint metadata (src/train/checkpoint.rs:19-47)."""
    config: ModelConfig
    step: int = 0
    epoch: int = 0
    best_val_loss: float = float("inf")
    learning_rate: float = 0.0
    has_optimizer_state: bool = False


@dataclass
class Weights:
    """Model tensors by the reference's names: embed_tokens, final_norm, layers[i][key] for
    key in LAYER_KEYS, and the untied output projection when there is one."""
    embed_tokens: np.ndarray
    layers: List[Dict[str, np.ndarray]]
    final_norm: np.ndarray
    output_weight: Optional[np.ndarray] = None


@dataclass
class OptimizerState:
    """Lion momenta with the same structure as Weights (GPTModelState, src/nn/model.rs:440-520)."""
    embed: np.ndarray
    layers: List[Dict[str, np.ndarray]]
    final_norm: np.ndarray
    output_weight: Optional[np.ndarray] = None


def _w(f: BinaryIO, fmt: str, *v) -> None:
    f.write(struct.pack("<" + fmt, *v))


def _r(f: BinaryIO, fmt: str):
    n = struct.calcsize("<" + fmt)
    b = f.read(n)
    if len(b) != n:
        raise EOFError("unexpected end of checkpoint")
    return struct.unpack("<" + fmt, b)


def save_tensor(f: BinaryIO, a: np.ndarray) -> None:
    """src/train/checkpoint.rs:52-73: u32 ndim, u64 dims, f32 values."""
    a = np.ascontiguousarray(a, dtype="<f4")
    _w(f, "I", a.ndim)
    for d in a.shape:
        _w(f, "Q", d)
    f.write(a.tobytes())


def load_tensor(f: BinaryIO) -> np.ndarray:
    """src/train/checkpoint.rs:75-98."""
    (ndim,) = _r(f, "I")
    shape = tuple(_r(f, "Q")[0] for _ in range(ndim))
    n = int(np.prod(shape)) if shape else 1
    b = f.read(4 * n)
    if len(b) != 4 * n:
        raise EOFError("unexpected end of checkpoint tensor data")
    return np.frombuffer(b, dtype="<f4").astype(np.float32).reshape(shape)


def _write_config(f: BinaryIO, c: ModelConfig) -> None:
    _w(f, "QQQQQQ", c.vocab_size, c.hidden_dim, c.num_layers, c.num_heads, c.num_kv_heads, c.intermediate_dim)
    _w(f, "ff", c.norm_eps, c.rope_base)
    _w(f, "Q", c.max_seq_len)
    _w(f, "BB", 1 if c.tie_weights else 0, int(c.precision))


def _read_config(f: BinaryIO) -> ModelConfig:
    v, h, l, nh, nkv, ffn = _r(f, "QQQQQQ")
    eps, base = _r(f, "ff")
    (msl,) = _r(f, "Q")
    (tie,) = _r(f, "B")
    b = f.read(1)  # precision byte; absent in old files (FP32)
    prec = {1: 1, 2: 2}.get(b[0], 0) if b else 0
    return ModelConfig(v, h, l, nh, nkv, ffn, eps, base, msl, tie == 1, prec)


def save_model_weights(path_or_file, weights: Weights, checkpoint: Checkpoint,
                       optimizer_state: Optional[OptimizerState] = None) -> None:
    """save_model_weights / save_model_weights_with_optimizer (src/train/checkpoint.rs:100-181)."""
    own = isinstance(path_or_file, (str, bytes)) or hasattr(path_or_file, "__fspath__")
    f = open(path_or_file, "wb") if own else path_or_file
    try:
        _w(f, "II", MAGIC, VERSION)
        _w(f, "QQff", checkpoint.step, checkpoint.epoch, checkpoint.best_val_loss, checkpoint.learning_rate)
        _write_config(f, checkpoint.config)
        save_tensor(f, weights.embed_tokens)
        for layer in weights.layers:
            for k in LAYER_KEYS:
                save_tensor(f, layer[k])
        save_tensor(f, weights.final_norm)
        _w(f, "B", 1 if checkpoint.config.tie_weights else 0)
        _w(f, "B", 1 if optimizer_state is not None else 0)
        if optimizer_state is not None:
            save_tensor(f, optimizer_state.embed)
            _w(f, "I", len(optimizer_state.layers))
            for layer in optimizer_state.layers:
                for k in LAYER_KEYS:
                    save_tensor(f, layer[k])
            save_tensor(f, optimizer_state.final_norm)
            _w(f, "B", 1 if optimizer_state.output_weight is not None else 0)
            if optimizer_state.output_weight is not None:
                save_tensor(f, optimizer_state.output_weight)
        if weights.output_weight is not None and not checkpoint.config.tie_weights:
            f.write(EXT_TAG)
            _w(f, "I", 1)
            save_tensor(f, weights.output_weight)
    finally:
        if own:
            f.close()


def load_model_weights(path_or_file) -> Tuple[Weights, Checkpoint, Optional[OptimizerState]]:
    """load_model_weights_with_optimizer (src/train/checkpoint.rs:183-316): errors on a bad magic
    number or an unsupported version, as the reference does."""
    own = isinstance(path_or_file, (str, bytes)) or hasattr(path_or_file, "__fspath__")
    f = open(path_or_file, "rb") if own else path_or_file
    try:
        magic, version = _r(f, "II")
        if magic != MAGIC:
            raise ValueError("Invalid checkpoint file (bad magic number)")
        if not MIN_VERSION <= version <= VERSION:
            raise ValueError(f"Unsupported checkpoint version: {version} (supported: {MIN_VERSION}-{VERSION})")
        step, epoch, best, lr = _r(f, "QQff")
        cfg = _read_config(f)
        embed = load_tensor(f)
        layers = [{k: load_tensor(f) for k in LAYER_KEYS} for _ in range(cfg.num_layers)]
        final_norm = load_tensor(f)
        _r(f, "B")  # tie flag (already in the config)
        opt = None
        if version >= 2:
            b = f.read(1)
            if b and b[0] == 1:
                o_embed = load_tensor(f)
                (nl,) = _r(f, "I")
                o_layers = [{k: load_tensor(f) for k in LAYER_KEYS} for _ in range(nl)]
                o_final = load_tensor(f)
                (has_out,) = _r(f, "B")
                o_out = load_tensor(f) if has_out == 1 else None
                opt = OptimizerState(o_embed, o_layers, o_final, o_out)
        out_w = None
        tag = f.read(4)
        if tag == EXT_TAG:
            _r(f, "I")
            out_w = load_tensor(f)
        w = Weights(embed, layers, final_norm, out_w)
        ck = Checkpoint(cfg, step, epoch, best, lr, opt is not None)
        return w, ck, opt
    finally:
        if own:
            f.close()


def to_bytes(weights: Weights, checkpoint: Checkpoint, optimizer_state: Optional[OptimizerState] = None) -> bytes:
    buf = io.BytesIO()
    save_model_weights(buf, weights, checkpoint, optimizer_state)
    return buf.getvalue()
