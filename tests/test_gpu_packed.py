"""The packed copy of the expert weights (moe_fp8_pack_weights, run_packed) on the GPU.

* Layout: blocks of the packed copy against the layout stated in include/moe_fp8.h, restated
  here with numpy index arithmetic on the row-major weights (first and last blocks, blocks in
  the middle, both halves of a W13 block), and the whole copy as a permutation of the weights'
  bytes (equal byte sums and byte histograms of the W13 and W2 parts).
* Results: run_packed is bit-identical to moe_fp8_run on the row-major weights up to 256 tokens,
  where the streaming GEMMs read the packed copy (16-row items: T = 1, 16, 40, 64, other expert
  offsets, fp32 output; 32-row items: T = 65, 200, 256), and above 256 tokens, where the copy
  is not read (T = 257, 600).
* run() builds the copy of a weight set on its first call of up to 256 tokens, reuses it, gives
  the row-major result bit for bit, rebuilds it after an in-place change of the weights, and
  streams the row-major weights when the cache is off.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

_STATE = {}
W13_BYTES = 32 * 4096 * 7168


def _gh():
    import gpu_helpers
    return gpu_helpers


def _weights_and_packed():
    gh = _gh()
    if "w" not in _STATE:
        dev = torch.device("cuda:0")
        print("generating weights and their packed copy on cuda:0", flush=True)
        w = gh.inputs.make_weights(515, dev)
        packed = gh.pkg.pack_weights(w[0], w[2])
        torch.cuda.synchronize()
        _STATE["w"], _STATE["p"] = w, packed
    return _STATE["w"], _STATE["p"]


def _expected_fragment(rows: np.ndarray, k: int) -> np.ndarray:
    """The 2 KB fragment of 16 rows (uint8 [16, K]) for K-step k: lane l holds bytes
    [16(l/16), +16) and [64 + 16(l/16), +16) of K block k of row l%16."""
    out = np.empty((64, 32), np.uint8)
    for lane in range(64):
        r, g = lane % 16, lane // 16
        base = 128 * k
        out[lane, :16] = rows[r, base + 16 * g: base + 16 * g + 16]
        out[lane, 16:] = rows[r, base + 64 + 16 * g: base + 64 + 16 * g + 16]
    return out.reshape(-1)


@pytest.mark.parametrize("e,s,k", [(0, 0, 0), (0, 0, 1), (3, 17, 55), (12, 64, 27), (31, 127, 0), (31, 127, 55)])
def test_packed_w13_blocks(e, s, k):
    (w13, _, _, _), packed = _weights_and_packed()
    off = ((e * 128 + s) * 56 + k) * 4096
    got = packed[off: off + 4096].cpu().numpy()
    gate = w13[e, 16 * s: 16 * s + 16].view(torch.uint8).cpu().numpy()
    up = w13[e, 2048 + 16 * s: 2048 + 16 * s + 16].view(torch.uint8).cpu().numpy()
    assert np.array_equal(got[:2048], _expected_fragment(gate, k))
    assert np.array_equal(got[2048:], _expected_fragment(up, k))


@pytest.mark.parametrize("e,h,k", [(0, 0, 0), (0, 1, 0), (5, 447, 15), (31, 200, 7), (31, 447, 15)])
def test_packed_w2_blocks(e, h, k):
    (_, _, w2, _), packed = _weights_and_packed()
    off = W13_BYTES + ((e * 448 + h) * 16 + k) * 2048
    got = packed[off: off + 2048].cpu().numpy()
    rows = w2[e, 16 * h: 16 * h + 16].view(torch.uint8).cpu().numpy()
    assert np.array_equal(got, _expected_fragment(rows, k))


def test_packed_copy_is_a_permutation_of_the_weights():
    (w13, _, w2, _), packed = _weights_and_packed()
    assert packed.numel() == W13_BYTES + 32 * 7168 * 2048
    for part, src in ((packed[:W13_BYTES], w13), (packed[W13_BYTES:], w2)):
        s = src.view(torch.uint8).reshape(-1)
        assert int(part.sum(dtype=torch.int64)) == int(s.sum(dtype=torch.int64))
        assert torch.equal(torch.bincount(part.int(), minlength=256), torch.bincount(s.int(), minlength=256))


@pytest.mark.parametrize("T,offset,out_dtype", [(1, 0, torch.bfloat16), (2, 32, torch.bfloat16), (3, 0, torch.bfloat16),
                                                (4, 224, torch.float32), (8, 0, torch.bfloat16),
                                                (9, 0, torch.bfloat16), (16, 0, torch.bfloat16),
                                                (64, 0, torch.bfloat16), (64, 96, torch.bfloat16),
                                                (40, 224, torch.float32), (65, 0, torch.bfloat16),
                                                (200, 32, torch.bfloat16), (256, 0, torch.float32), (257, 0, torch.bfloat16),
                                                (600, 0, torch.bfloat16)])
def test_run_packed_is_bit_identical_to_run(T, offset, out_dtype):
    gh = _gh()
    dev = torch.device("cuda:0")
    w, packed = _weights_and_packed()
    print(f"run_packed against run: T={T} offset={offset} {out_dtype}", flush=True)
    # up to 8 tokens GEMM1 runs its deep-ring instances (6 slots up to 2 tokens, 4 up to 8); a few
    # boosted local experts make sure these batches have local work
    boosted = (1, 7, 12, 30) if T <= 9 else ()
    logits, bias, hq, hs = gh.inputs.make_activations(T, 6100 + T + offset, dev, local_expert_offset=offset,
                                                      boosted_local_experts=boosted)
    kw = dict(routing_logits=logits, routing_bias=bias, hidden_states=hq, hidden_states_scale=hs,
              gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2], gemm2_weights_scale=w[3],
              local_expert_offset=offset, routed_scaling_factor=2.5)
    ref = torch.full((T, 7168), float("nan"), dtype=out_dtype, device=dev)
    got = torch.full((T, 7168), float("nan"), dtype=out_dtype, device=dev)
    gh.run_layer(gh.make_args(**kw, output=ref), gh.new_workspace(T, dev))   # moe_fp8_run, row-major
    gh.pkg.run_packed(**kw, output=got, packed_weights=packed)
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()
    if boosted:
        assert ref.float().abs().amax() > 0
    assert torch.equal(ref.view(torch.int16) if out_dtype == torch.bfloat16 else ref.view(torch.int32),
                       got.view(torch.int16) if out_dtype == torch.bfloat16 else got.view(torch.int32))


def test_run_keeps_a_packed_copy_per_weight_set():
    gh = _gh()
    moe = gh.pkg.moe
    dev = torch.device("cuda:0")
    w = gh.inputs.make_weights(516, dev, experts=32)
    T = 24
    logits, bias, hq, hs = gh.inputs.make_activations(T, 6200, dev)
    kw = dict(routing_logits=logits, routing_bias=bias, hidden_states=hq, hidden_states_scale=hs,
              gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2], gemm2_weights_scale=w[3],
              local_expert_offset=0, routed_scaling_factor=2.5)
    ref = torch.empty((T, 7168), dtype=torch.bfloat16, device=dev)
    gh.run_layer(gh.make_args(**kw, output=ref), gh.new_workspace(T, dev))
    cache = moe.PackedWeightCache()
    saved = moe._packed_weights
    moe._packed_weights = cache
    try:
        out = torch.empty_like(ref)
        gh.pkg.run(**kw, output=out)
        assert len(cache) == 1
        first = cache.get(w[0], w[2])
        gh.pkg.run(**kw, output=out)
        torch.cuda.synchronize()
        assert len(cache) == 1 and cache.get(w[0], w[2]) is first
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        # an in-place change of W2 makes the copy stale: the next call repacks and follows it
        w[2].view(torch.uint8)[0, :16, :].zero_()
        gh.run_layer(gh.make_args(**kw, output=ref), gh.new_workspace(T, dev))
        gh.pkg.run(**kw, output=out)
        torch.cuda.synchronize()
        assert cache.get(w[0], w[2]) is not first
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        # off: the row-major weights, no new copy
        moe.set_packed_weight_sets(0)
        cache.clear()
        gh.pkg.run(**kw, output=out)
        torch.cuda.synchronize()
        assert len(cache) == 0
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    finally:
        moe._packed_weights = saved


def test_run_on_a_second_stream_uses_the_copy():
    """run() on a side stream with a copy built on another: the copy is recorded on the side stream
    (Tensor.record_stream), the side stream waits for the packing kernel through the cache's event
    (nothing else orders it: the inputs are ready before the first call and the side stream does
    not wait for the building stream), and the result is the row-major one, bit for bit."""
    gh = _gh()
    moe = gh.pkg.moe
    dev = torch.device("cuda:0")
    w = gh.inputs.make_weights(517, dev, experts=32)
    T = 20
    logits, bias, hq, hs = gh.inputs.make_activations(T, 6300, dev)
    kw = dict(routing_logits=logits, routing_bias=bias, hidden_states=hq, hidden_states_scale=hs,
              gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2], gemm2_weights_scale=w[3],
              local_expert_offset=0, routed_scaling_factor=2.5)
    ref = torch.empty((T, 7168), dtype=torch.bfloat16, device=dev)
    gh.run_layer(gh.make_args(**kw, output=ref), gh.new_workspace(T, dev))
    cache = moe.PackedWeightCache()
    saved = moe._packed_weights
    moe._packed_weights = cache
    try:
        out = torch.empty_like(ref)
        out2 = torch.empty_like(ref)
        side = torch.cuda.Stream(device=dev)
        torch.cuda.synchronize()                          # inputs, ref and outputs are ready
        gh.pkg.run(**kw, output=out)                      # builds the copy on the current stream
        with torch.cuda.stream(side):
            gh.pkg.run(**kw, output=out2)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize()
        ent = next(iter(cache._entries.values()))
        assert len(ent["streams"]) == 2
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
        assert torch.equal(out2.view(torch.int16), ref.view(torch.int16))
    finally:
        moe._packed_weights = saved
