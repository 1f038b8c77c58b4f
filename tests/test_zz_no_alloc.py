"""moe_fp8_run_static: the whole layer on the library's own device workspace (a static device
array of MOE_FP8_STATIC_SCRATCH_BYTES, up to MOE_FP8_STATIC_MAX_TOKENS tokens), for callers
that cannot allocate. Its output must be bit-identical to moe_fp8_run's with a caller
workspace: the same kernels run in the same order, and the array's contents left by an
earlier, larger call must not leak into a later one."""
import ctypes

import numpy as np
import pytest
import torch



def _gh():
    import gpu_helpers
    return gpu_helpers


def test_static_entry_rejects_before_any_launch(pkg):
    """Argument checks: on the CPU and on the GPU alike nothing is launched for these."""
    L = pkg._lib
    lib = L.load()
    assert L.workspace_bytes(L.STATIC_MAX_TOKENS) <= L.STATIC_SCRATCH_BYTES
    assert L.workspace_bytes(L.STATIC_MAX_TOKENS + 1) > 0
    a = L.MoeFp8Args()
    assert lib.moe_fp8_run_static(None, None) == L.EINVAL_POINTER
    a.num_tokens = -1
    assert lib.moe_fp8_run_static(ctypes.byref(a), None) == L.EINVAL_TOKENS
    a.num_tokens = L.STATIC_MAX_TOKENS + 1
    assert lib.moe_fp8_run_static(ctypes.byref(a), None) == L.ESTATIC_TOKENS
    assert "MOE_FP8_STATIC_MAX_TOKENS" in L.strerror(L.ESTATIC_TOKENS)
    a.num_tokens = 0
    assert lib.moe_fp8_run_static(ctypes.byref(a), None) == L.OK
    # the pointers are checked before the device (and before the first call's clear kernel)
    a.num_tokens = 4
    assert lib.moe_fp8_run_static(ctypes.byref(a), None) == L.EINVAL_POINTER


@pytest.mark.gpu
def test_static_matches_run_on_successive_calls():
    """Two calls in a row, the second with fewer tokens (and another offset and bias dtype),
    each bit-equal to moe_fp8_run on a fresh caller workspace; then the first again."""
    gh = _gh()
    _lib = gh._lib
    dev = torch.device("cuda:0")
    lib = _lib.load()
    w = gh.inputs.make_weights(6060, dev)
    cases = [(64, 0, 6061, torch.bfloat16), (23, 96, 6062, torch.float32), (64, 0, 6061, torch.bfloat16)]
    for T, offset, seed, bias_dtype in cases:
        print(f"moe_fp8_run_static T={T} offset={offset}", flush=True)
        logits, bias, hq, hs = gh.inputs.make_activations(T, seed, dev, local_expert_offset=offset)
        kw = dict(routing_logits=logits, routing_bias=bias.to(bias_dtype), hidden_states=hq,
                  hidden_states_scale=hs, gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2],
                  gemm2_weights_scale=w[3], local_expert_offset=offset, routed_scaling_factor=2.5)
        ref = torch.full((T, 7168), float("nan"), dtype=torch.bfloat16, device=dev)
        ws = gh.new_workspace(T, dev)
        gh.run_layer(gh.make_args(**kw, output=ref), ws)
        got = torch.full((T, 7168), float("nan"), dtype=torch.bfloat16, device=dev)
        args = gh.make_args(**kw, output=got)
        _lib.check(lib.moe_fp8_run_static(args, gh.stream()), "moe_fp8_run_static")
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"T={T}: static and caller workspace differ"
        assert np.isfinite(got.float().cpu().numpy()).all()
