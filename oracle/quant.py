"""Upstream activation quantisation in numpy (oracle; test infrastructure only).

  hidden_values    exact fp32 values of bf16 (uint16 bits), fp16 or fp32 hidden states
  quantize_hidden  x [T, 7168] -> (q uint8 e4m3fn codes [T, 7168], scale fp32 [56, T]):
                   per token and 128 columns scale = max(amax / 448, 1e-12),
                   q = e4m3(x / scale) rounded to nearest even -- the in-path
                   requantisation of kernel.py:131-135 applied to the layer input, whose
                   contract (e4m3fn [T, 7168], scales [56, T]) is kernel.py:600-603

Only tests/, __graft_entry__.smoke() and bench.py's CPU baseline use this package, and
only as the checker of the HIP library.
"""
from __future__ import annotations

import numpy as np

from . import fp8
from .experts import requant_rows


def hidden_values(x: np.ndarray, dtype: str) -> np.ndarray:
    """float32 values of hidden states given as bf16 bit patterns (uint16), fp16 or fp32."""
    if dtype == "bf16":
        return fp8.bf16_to_f32(np.asarray(x, dtype=np.uint16))
    if dtype == "fp16":
        return np.asarray(x, dtype=np.float16).astype(np.float32)
    return np.asarray(x, dtype=np.float32)


def quantize_hidden(x: np.ndarray, block: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """x float32 [T, H] -> (e4m3fn codes uint8 [T, H], scales float32 [H/block, T])."""
    x = np.asarray(x, dtype=np.float32)
    q, scale_tb = requant_rows(x, block)
    return q, np.ascontiguousarray(scale_tb.T)
