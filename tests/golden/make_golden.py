"""Writes the golden fixtures that pin the CPU oracle to independent library routines.

  fp8_e4m3fn_golden.npz  torch's CPU float8_e4m3fn cast: the decode table of all 256 codes
                         and the codes of ~60k float32 inputs (every fp8 value, every
                         midpoint between neighbours and its fp32 neighbours, the overflow
                         region, subnormals, random values), plus torch's bf16 rounding of
                         random and tie values.
  routing_golden.npz     transformers' DeepseekV3TopkRouter (sigmoid + bias, top-2 group
                         score, top-4 of 8 groups, top-8 experts, renormalised weights times
                         routed_scaling_factor) on seeded logits: 256 rows N(0,1) with bias
                         N(0,0.1) in bf16, 128 rows with +3.0 bias on 4 experts, 128 rows
                         N(0,3). Ids are stored sorted per row (the router's topk is unsorted).

Run from the repository root: python tests/golden/make_golden.py
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent


def fp8_fixture():
    codes = torch.arange(256, dtype=torch.uint8)
    table = codes.view(torch.float8_e4m3fn).float().numpy()
    finite = np.sort(np.unique(table[np.isfinite(table)]))
    mids = ((finite[:-1].astype(np.float64) + finite[1:]) / 2).astype(np.float32)
    up = np.nextafter(mids, np.float32(np.inf))
    down = np.nextafter(mids, np.float32(-np.inf))
    rng = np.random.default_rng(7)
    rand = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 50,
        rng.uniform(-2.0 ** -5, 2.0 ** -5, 8000).astype(np.float32),
        rng.uniform(440, 500, 2000).astype(np.float32) * rng.choice([-1, 1], 2000).astype(np.float32),
    ])
    special = np.array([0.0, -0.0, 448.0, -448.0, 460.0, 464.0, 464.00003, 465.0, 479.9, 480.0, 1e6,
                        np.inf, -np.inf, 2.0 ** -9, 2.0 ** -10, 3 * 2.0 ** -11, 1e-30], dtype=np.float32)
    values = np.concatenate([finite, mids, up, down, rand, special]).astype(np.float32)
    got = torch.from_numpy(values).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    bf_vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32),
        # exact bf16 ties: low 16 bits 0x8000 with odd and even kept parts
        (rng.integers(0x3f000000, 0x40000000, 4000, dtype=np.uint32) & 0xFFFF0000 | 0x8000).view(np.float32),
        np.array([0.0, -0.0, 3.0e38, 1e-40, np.inf], dtype=np.float32),
    ]).astype(np.float32)
    bf_bits = torch.from_numpy(bf_vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.savez_compressed(OUT / "fp8_e4m3fn_golden.npz", decode_table=table, values=values, codes=got,
                        bf16_values=bf_vals, bf16_bits=bf_bits)


def routing_fixture():
    from transformers.models.deepseek_v3.configuration_deepseek_v3 import DeepseekV3Config
    from transformers.models.deepseek_v3.modeling_deepseek_v3 import DeepseekV3TopkRouter

    cfg = DeepseekV3Config(hidden_size=256, n_routed_experts=256, num_experts_per_tok=8, n_group=8,
                           topk_group=4, routed_scaling_factor=2.5, norm_topk_prob=True)
    router = DeepseekV3TopkRouter(cfg)
    with torch.no_grad():
        router.weight.copy_(torch.eye(256))           # router logits = input exactly
    g = torch.Generator().manual_seed(11)
    parts = []
    for rows, scale, boost in ((256, 1.0, False), (128, 1.0, True), (128, 3.0, False)):
        logits = torch.randn(rows, 256, generator=g) * scale
        bias = (torch.randn(256, generator=g) * 0.1)
        if boost:
            bias[[3, 11, 19, 27]] = 3.0
        bias = bias.to(torch.bfloat16).float()
        router.e_score_correction_bias.copy_(bias)
        with torch.no_grad():
            lg, w, idx = router(logits)
        assert torch.equal(lg, logits)
        order = torch.argsort(idx, dim=1)
        parts.append((logits.numpy(), np.full(rows, len(parts), dtype=np.int32), bias.numpy(),
                      torch.gather(idx, 1, order).numpy().astype(np.int32),
                      torch.gather(w, 1, order).numpy().astype(np.float32)))
    logits, bias_index, ids, w = (np.concatenate([p[i] for p in parts]) for i in (0, 1, 3, 4))
    bias_sets = np.stack([p[2] for p in parts]).astype(np.float32)
    np.savez_compressed(OUT / "routing_golden.npz", logits=logits, bias_sets=bias_sets,
                        bias_index=bias_index, ids_sorted=ids, weights_sorted=w,
                        routed_scaling_factor=np.float32(2.5))


if __name__ == "__main__":
    fp8_fixture()
    routing_fixture()
    for f in sorted(OUT.glob("*.npz")):
        print(f.name, f.stat().st_size)
