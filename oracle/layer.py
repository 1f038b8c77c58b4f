"""The whole fused MoE layer in numpy (oracle; test infrastructure only).

layer_forward() composes routing -> dispatch -> per-expert GEMM1 + SwiGLU -> GEMM2 ->
weighted combine -> bf16, following run() (kernel.py:562-729) and the competition
definition (writeup.pdf p.1 s.1.2: a loop over local experts of dequantise, matmul,
SwiGLU, matmul, weighted accumulate).

mode="definition": the intermediate C stays fp32 (the definition's math); each token's
  output sums its experts' weighted rows in ascending expert order, as the definition's
  loop over experts does.
mode="emulated":   C is requantised to e4m3 with one scale per row per `requant_block`
  columns before GEMM2 (kernel.py:131-135 uses 64; the HIP kernels use 64 below 4096 tokens
  and 128 from 4096 on), and each token sums its weighted rows in top-k slot order starting from
  0, as the HIP combine does; a token with one local assignment gets exactly that row.
  With `act_override` = (act uint8 [N, I], act_scale fp32 [N, I/requant_block]) in
  bucket-row order, GEMM1 is skipped and GEMM2 + combine run on that intermediate instead
  of the oracle's own: a check of the second half of the layer on exactly the
  intermediate a kernel produced.
Weights are dequantised one touched expert at a time (kept in `dequant_cache`, a dict the
caller owns, when given, so that several calls on one weight set dequantise each expert
once); `tokens` restricts the GEMMs and the output to a subset of tokens (routing still
runs for all of them).
"""
from __future__ import annotations

import numpy as np

from . import dispatch as dsp
from . import experts as ex
from . import fp8
from . import routing

F32 = np.float32


def _expert_weights(e, w13q, s13, w2q, s2, block, cache):
    """fp32 W13[e] and W2[e], dequantised (kernel.py:111-120, :228-232), from `cache` if there."""
    if cache is not None and e in cache:
        return cache[e]
    w = (ex.dequant_blocks(w13q[e], s13[e], block), ex.dequant_blocks(w2q[e], s2[e], block))
    if cache is not None:
        cache[e] = w
    return w


def layer_forward(routing_logits, routing_bias, hidden_states, hidden_states_scale, gemm1_weights,
                  gemm1_weights_scale, gemm2_weights, gemm2_weights_scale, local_expert_offset,
                  routed_scaling_factor, mode: str = "definition", requant_block: int = 128,
                  topk=None, tokens=None, block: int = 128, dequant_cache: dict | None = None,
                  act_override=None):
    """All arrays are numpy: logits fp32 [T, E], bias fp32 [E], hidden uint8 [T, H],
    hidden scale fp32 [H/128, T], W13 uint8 [E_l, 2I, H], S13 fp32 [E_l, 2I/128, H/128],
    W2 uint8 [E_l, H, I], S2 fp32 [E_l, H/128, I/128]. Returns a dict of intermediates
    and "output" (fp32 values rounded to bf16) / "output_f32" for the rows of `tokens`
    (all tokens when None)."""
    if mode not in ("definition", "emulated"):
        raise ValueError(mode)
    if act_override is not None and mode != "emulated":
        raise ValueError("act_override needs mode='emulated'")
    hidden = np.asarray(hidden_states, dtype=np.uint8)
    T, H = hidden.shape
    e_local, two_i, _ = gemm1_weights.shape
    inter = two_i // 2
    if topk is None:
        ids, wts = routing.route(routing_logits, routing_bias, routed_scaling_factor)
    else:
        ids, wts = (np.asarray(topk[0], dtype=np.int32), np.asarray(topk[1], dtype=F32))
    top_k = ids.shape[1]
    d = dsp.dispatch(ids, wts, local_expert_offset, e_local)
    n = len(d["sorted_slot"])
    tok_sel = np.arange(T) if tokens is None else np.asarray(tokens, dtype=np.int64)
    want = np.zeros(T, dtype=bool)
    want[tok_sel] = True

    act = np.zeros((n, inter), dtype=np.uint8) if mode == "emulated" else None
    act_scale = np.zeros((n, inter // requant_block), dtype=F32) if mode == "emulated" else None
    swiglu = np.zeros((n, inter), dtype=F32)  # fp32 SwiGLU row of each assignment
    y = np.zeros((n, H), dtype=F32)          # weighted GEMM2 row of each assignment
    done = np.zeros(n, dtype=bool)
    for e in range(e_local):
        lo, hi = int(d["expert_start"][e]), int(d["expert_start"][e + 1])
        if hi == lo:
            continue
        rows = np.arange(lo, hi)
        rows = rows[want[d["sorted_token"][rows]]]
        if len(rows) == 0:
            continue
        tok = d["sorted_token"][rows]
        a = ex.dequant_rows(hidden[tok], np.asarray(hidden_states_scale)[:, tok], block)
        w13, w2 = _expert_weights(e, gemm1_weights, gemm1_weights_scale, gemm2_weights,
                                  gemm2_weights_scale, block, dequant_cache)
        if act_override is None:
            c = ex.swiglu(ex.gemm(a, w13), inter)
            swiglu[rows] = c
        del w13
        if mode == "emulated":
            if act_override is None:
                q, sc = ex.requant_rows(c, requant_block)
            else:
                q, sc = act_override[0][rows], act_override[1][rows]
            act[rows], act_scale[rows] = q, sc
            c = ex.dequant_requant(q, sc, requant_block)
        o = ex.gemm(c, w2)
        del w2
        y[rows] = (o * d["sorted_weight"][rows][:, None]).astype(F32)
        done[rows] = True

    out = np.zeros((len(tok_sel), H), dtype=F32)
    pos = np.full(T, -1, dtype=np.int64)
    pos[tok_sel] = np.arange(len(tok_sel))
    if mode == "emulated":
        inv = np.full(T * top_k, -1, dtype=np.int64)
        inv[d["sorted_slot"]] = np.arange(n)
        for k in range(top_k):
            slots = np.arange(T) * top_k + k
            sel = (inv[slots] >= 0) & want
            out[pos[sel]] += y[inv[slots[sel]]]
    else:
        for e in range(e_local):
            lo, hi = int(d["expert_start"][e]), int(d["expert_start"][e + 1])
            rows = np.arange(lo, hi)
            rows = rows[done[rows]]
            # a token that names expert e more than once (kernel.py:522-534 can repeat an id)
            # has several rows here: add each of them, in bucket (slot) order
            np.add.at(out, pos[d["sorted_token"][rows]], y[rows])
    return {
        "topk_ids": ids,
        "topk_weights": wts,
        **d,
        "swiglu": swiglu,
        "act": act,
        "act_scale": act_scale,
        "rows": y,
        "tokens": tok_sel,
        "output_f32": out,
        "output": fp8.bf16_round(out),
    }
