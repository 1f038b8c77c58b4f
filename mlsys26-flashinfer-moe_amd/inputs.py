"""Seeded synthetic inputs for the layer's benchmark and parity workloads.

Shapes and distributions (all five workloads share them; only T, the local expert
offset and the router bias differ):
  hidden states  bf16 N(0,1) [T, 7168] quantised to e4m3fn with one scale per token per
                 128 columns (scale = amax/448), stored [56, T] as in kernel.py:603;
  W13 [32, 4096, 7168] and W2 [32, 7168, 2048]  N(0, 0.02) quantised to e4m3fn with one
                 fp32 scale per 128x128 block (scale = amax/448);
  router logits  fp32 N(0,1) [T, 256]; router bias bf16 N(0, 0.1) [256];
  routed_scaling_factor = 2.5.
Tensors are generated on `device` with a torch.Generator seeded per workload, so one
seed gives one set of inputs on one device type.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from ._lib import BLOCK, EXPERTS_GLOBAL, EXPERTS_LOCAL, HIDDEN, INTER

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0
ROUTED_SCALING_FACTOR = 2.5


@dataclass(frozen=True)
class Workload:
    name: str
    num_tokens: int
    local_expert_offset: int
    seed: int
    boosted_local_experts: tuple = field(default_factory=tuple)  # local ids whose bias is +3.0
    description: str = ""


WORKLOADS = {
    "t16": Workload("t16", 16, 0, 1000, (), "plumbing: 16 tokens, local experts 0..31"),
    "t64": Workload("t64", 64, 0, 1001, (), "decode: 64 tokens, local experts 0..31"),
    "t1024_off64": Workload("t1024_off64", 1024, 64, 1002, (), "mid batch: 1024 tokens, local experts 64..95"),
    "t8192": Workload("t8192", 8192, 0, 1003, (), "prefill: 8192 tokens, local experts 0..31"),
    "t4096_skew": Workload("t4096_skew", 4096, 0, 1004, (3, 11, 19, 27),
                           "skewed: 4096 tokens, bias +3.0 on local experts 3, 11, 19, 27"),
}


def quantize_rows_1x128(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[T, H] float -> e4m3fn [T, H] and scales [H/128, T]: max(amax/448, 1e-12) per token
    per block, the formula of quantize_hidden (computed here with torch, independently)."""
    T, H = x.shape
    xb = x.float().reshape(T, H // BLOCK, BLOCK)
    scale = (xb.abs().amax(dim=-1) / FP8_MAX).clamp_min(1e-12)
    q = (xb / scale[..., None]).to(FP8).reshape(T, H)
    return q, scale.t().contiguous()


def quantize_blocks_128x128(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[R, C] float -> e4m3fn [R, C] and scales [R/128, C/128] (amax/448 per block)."""
    R, C = w.shape
    wb = w.float().reshape(R // BLOCK, BLOCK, C // BLOCK, BLOCK)
    amax = wb.abs().amax(dim=(1, 3)).clamp_min(1e-12)
    scale = amax / FP8_MAX
    q = (wb / scale[:, None, :, None]).to(FP8).reshape(R, C)
    return q, scale


def make_weights(seed: int, device, experts: int = EXPERTS_LOCAL):
    """W13, S13, W2, S2 for `experts` local experts (generated one expert at a time)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    w13 = torch.empty((experts, 2 * INTER, HIDDEN), dtype=FP8, device=device)
    s13 = torch.empty((experts, 2 * INTER // BLOCK, HIDDEN // BLOCK), dtype=torch.float32, device=device)
    w2 = torch.empty((experts, HIDDEN, INTER), dtype=FP8, device=device)
    s2 = torch.empty((experts, HIDDEN // BLOCK, INTER // BLOCK), dtype=torch.float32, device=device)
    for e in range(experts):
        w = torch.randn((2 * INTER, HIDDEN), generator=gen, device=device, dtype=torch.float32) * 0.02
        w13[e], s13[e] = quantize_blocks_128x128(w)
        w = torch.randn((HIDDEN, INTER), generator=gen, device=device, dtype=torch.float32) * 0.02
        w2[e], s2[e] = quantize_blocks_128x128(w)
        del w
    return w13, s13, w2, s2


def make_activations(num_tokens: int, seed: int, device, local_expert_offset: int = 0,
                     boosted_local_experts=()):
    """routing_logits, routing_bias (bf16), hidden_states (e4m3fn), hidden_states_scale."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    logits = torch.randn((num_tokens, EXPERTS_GLOBAL), generator=gen, device=device, dtype=torch.float32)
    bias = (torch.randn((EXPERTS_GLOBAL,), generator=gen, device=device, dtype=torch.float32) * 0.1)
    for le in boosted_local_experts:
        bias[local_expert_offset + le] = 3.0
    bias = bias.to(torch.bfloat16)
    hidden = torch.randn((num_tokens, HIDDEN), generator=gen, device=device, dtype=torch.float32)
    hidden = hidden.to(torch.bfloat16)
    hq, hs = quantize_rows_1x128(hidden)
    return logits, bias, hq, hs


def make_workload(name: str, device, weights=None):
    """All inputs of a named workload as a dict of keyword arguments of `run` (minus output)."""
    wl = WORKLOADS[name]
    logits, bias, hq, hs = make_activations(wl.num_tokens, wl.seed, device, wl.local_expert_offset,
                                            wl.boosted_local_experts)
    if weights is None:
        weights = make_weights(wl.seed + 7919, device)
    w13, s13, w2, s2 = weights
    return dict(routing_logits=logits, routing_bias=bias, hidden_states=hq, hidden_states_scale=hs,
                gemm1_weights=w13, gemm1_weights_scale=s13, gemm2_weights=w2, gemm2_weights_scale=s2,
                local_expert_offset=wl.local_expert_offset, routed_scaling_factor=ROUTED_SCALING_FACTOR)
