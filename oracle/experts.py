"""Per-expert math of the layer in numpy (oracle; test infrastructure only).

  dequant_rows     a[t, k] = e4m3(q[t, k]) * s[k // 128, t]          kernel.py:104-108, :123
  dequant_blocks   w[r, c] = e4m3(q[r, c]) * s[r // 128, c // 128]   kernel.py:111-120, :228-232
  gemm             x @ w.T in fp32                                    kernel.py:123-124, :234
  swiglu           silu(X2) * X1, X1 = first `inter` columns, X2 = the rest,
                   silu(x) = x / (1 + exp(-x))                        kernel.py:126-129
  requant_rows     per row and `block` columns: scale = max(amax / 448, 1e-12),
                   q = e4m3(c / scale)                                kernel.py:131-135
"""
from __future__ import annotations

import numpy as np

from . import fp8

F32 = np.float32


def dequant_rows(q: np.ndarray, scale_kt: np.ndarray, block: int = 128) -> np.ndarray:
    """q uint8 [n, K], scale_kt fp32 [K/block, n] -> fp32 [n, K]."""
    n, K = q.shape
    a = fp8.decode(q).reshape(n, K // block, block)
    return (a * np.asarray(scale_kt, dtype=F32).T[:, :, None]).reshape(n, K).astype(F32)


def dequant_rows_rowmajor(q: np.ndarray, scale_tk: np.ndarray, block: int = 128) -> np.ndarray:
    """q uint8 [n, K], scale_tk fp32 [n, K/block] -> fp32 [n, K]."""
    return dequant_rows(q, np.asarray(scale_tk).T, block)


def dequant_blocks(q: np.ndarray, scale: np.ndarray, block: int = 128) -> np.ndarray:
    """q uint8 [R, C], scale fp32 [R/block, C/block] -> fp32 [R, C]."""
    R, C = q.shape
    w = fp8.decode(q).reshape(R // block, block, C // block, block)
    return (w * np.asarray(scale, dtype=F32)[:, None, :, None]).reshape(R, C).astype(F32)


def gemm(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """x [n, K] @ w[R, K].T in fp32 -> [n, R]."""
    return np.matmul(np.asarray(x, dtype=F32), np.asarray(w, dtype=F32).T).astype(F32)


def silu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, dtype=F32)
    with np.errstate(over="ignore"):
        return (x / (F32(1.0) + np.exp(-x))).astype(F32)


def swiglu(g: np.ndarray, inter: int) -> np.ndarray:
    """silu of the second half times the first half of g [n, 2*inter]."""
    g = np.asarray(g, dtype=F32)
    return (silu(g[:, inter:]) * g[:, :inter]).astype(F32)


def requant_rows(c: np.ndarray, block: int = 128):
    """c fp32 [n, I] -> (q uint8 [n, I], scale fp32 [n, I/block])."""
    c = np.asarray(c, dtype=F32)
    n, I = c.shape
    cb = c.reshape(n, I // block, block)
    amax = np.abs(cb).max(axis=-1)
    scale = np.maximum((amax / F32(448.0)).astype(F32), F32(1e-12)).astype(F32)
    q = fp8.encode((cb / scale[..., None]).astype(F32)).reshape(n, I)
    return q, scale


def dequant_requant(q: np.ndarray, scale: np.ndarray, block: int = 128) -> np.ndarray:
    """Inverse of requant_rows: uint8 [n, I] with scales [n, I/block] -> fp32 [n, I]."""
    return dequant_rows_rowmajor(q, scale, block)
