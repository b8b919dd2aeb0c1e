"""IronTensor's matrix-multiplication path, MI355X-native (gfx950 MFMA kernels behind a C ABI).

Python mirror of the reference's Rust ops/Tensor API for this path; every op runs the hand-written
HIP kernels in libirontensor_hip.so (built by irontensor_amd.build).
"""
from .errors import (DeviceError, EmptyTensor, InnerDimensionMismatch, InvalidValue, Panic,
                     PrecisionMismatch, ShapeMismatch, TensorError, UnsupportedDimensions)
from .tensor import Context, Precision, Tensor, bf16_to_f32, device_count, f32_to_bf16
from .ops import (Linear, attention, attention_backward_recompute, attention_forward_bhsd,
                  ensure_fp32, flash_attention, flash_attention_backward, flash_attention_bshd,
                  flash_attention_forward_bhsd, gemm, gemm_group, linear, linear_backward, linear_forward, matmul,
                  matmul_backward, matmul_backward_a, matmul_backward_b, matmul_bf16,
                  matmul_bf16_batched, matmul_custom, matmul_mps, matmul_mps_nt, matmul_mps_tn,
                  matmul_tn, softmax_backward, softmax_rows, swiglu_up, to_bf16_gpu, to_f32_gpu,
                  causal_mask_3d_gpu, transpose_3d_gpu)

__all__ = [name for name in dir() if not name.startswith("_")]
