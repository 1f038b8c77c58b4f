"""DeepSeek-V3 no-aux grouped routing in numpy (oracle; test infrastructure only).

Restates moe_routing_kernel (kernel.py:428-542) operation by operation in IEEE fp32:
  s = sigmoid(logit)                                  kernel.py:466
  b = s + bias                                        kernel.py:467 (bias as fp32, :616, :626)
  group score = largest + second largest b of the group (the first occurrence of the
    maximum is masked, so a repeated maximum counts twice)          kernel.py:479-488
  keep TOPK_GROUP groups: rounds of "max over the scores, first unselected group equal
    to it"                                                          kernel.py:495-501
  top-k experts: rounds of "first index of the max of b over kept groups (-inf
    elsewhere and for already chosen experts)"                      kernel.py:515-534
  weights = s_k / (sum s + 1e-20) * routed_scaling_factor, sum in selection order
                                                                    kernel.py:537-538
The sigmoid is the fixed fp32 operation sequence of the HIP kernel (Cody-Waite e^y with
a degree-7 Taylor polynomial, y clamped to [-80, 80]); numpy's fp32 element-wise
operations are correctly rounded and never fused, so the two agree bit for bit.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
LOG2E = F32(1.44269502162933349609375)      # 0x3fb8aa3b
LN2_HI = F32(0.693359375)                   # 0x3f318000
LN2_LO = F32(-2.12194440e-4)                # 0xb95e8083
TAYLOR = [F32(1.0), F32(1.0), F32(0.5), F32(1.66666672e-1), F32(4.16666679e-2),
          F32(8.33333377e-3), F32(1.38888892e-3), F32(1.98412701e-4)]   # 1/k!, k = 0..7
CLAMP = F32(80.0)


def sigmoid_f32(x: np.ndarray) -> np.ndarray:
    """1 / (1 + e^-x) in the exact fp32 operation order of the HIP routing kernel."""
    x = np.asarray(x, dtype=F32)
    y = -x
    y = np.where(y > CLAMP, CLAMP, y).astype(F32)
    y = np.where(y < -CLAMP, -CLAMP, y).astype(F32)
    n = np.rint(y * LOG2E).astype(F32)
    r = ((y - n * LN2_HI) - n * LN2_LO).astype(F32)
    p = TAYLOR[7]
    for c in TAYLOR[6::-1]:
        p = (p * r + c).astype(F32)
    with np.errstate(invalid="ignore"):
        ni = np.where(np.isnan(n), 0, n).astype(np.int32)
    e = np.ldexp(p, ni).astype(F32)
    return (F32(1.0) / (F32(1.0) + e)).astype(F32)


def route(logits: np.ndarray, bias: np.ndarray, routed_scaling_factor: float,
          n_group: int = 8, topk_group: int = 4, top_k: int = 8):
    """Returns (topk_ids int32 [T, top_k] in selection order, topk_weights fp32 [T, top_k])."""
    logits = np.asarray(logits, dtype=F32)
    bias = np.asarray(bias, dtype=F32).reshape(-1)
    T, E = logits.shape
    gsz = E // n_group
    rows = np.arange(T)
    s = sigmoid_f32(logits)
    b = (s + bias[None, :]).astype(F32)

    srt = np.sort(b.reshape(T, n_group, gsz), axis=-1)
    group_scores = (srt[..., -1] + srt[..., -2]).astype(F32)

    selected = np.zeros((T, n_group), dtype=bool)
    for _ in range(topk_group):
        tmp = np.where(selected, F32(-np.inf), group_scores)
        best = tmp.max(axis=1, keepdims=True)
        is_best = (tmp == best) & ~selected
        has = is_best.any(axis=1)
        g = np.argmax(is_best, axis=1)
        selected[rows[has], g[has]] = True

    pruned = np.where(np.repeat(selected, gsz, axis=1), b, F32(-np.inf)).astype(F32)
    ids = np.zeros((T, top_k), dtype=np.int32)
    svals = np.zeros((T, top_k), dtype=F32)
    for k in range(top_k):
        j = np.argmax(pruned, axis=1)      # first index of the maximum
        ids[:, k] = j
        svals[:, k] = s[rows, j]
        pruned[rows, j] = F32(-np.inf)
    total = svals[:, 0].copy()
    for k in range(1, top_k):
        total = (total + svals[:, k]).astype(F32)
    total = (total + F32(1e-20)).astype(F32)
    weights = ((svals / total[:, None]).astype(F32) * F32(routed_scaling_factor)).astype(F32)
    return ids, weights

