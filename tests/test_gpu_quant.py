"""The upstream activation quantiser (moe_fp8_quantize_hidden) on the GPU against the
oracle (oracle/quant.py), bit for bit: e4m3fn codes and fp32 scales, for bf16, fp16 and
fp32 inputs, ragged T, special values, and as the input of the layer."""
import numpy as np
import pytest
import torch

from oracle import quant

pytestmark = pytest.mark.gpu
H = 7168


def _gh():
    import gpu_helpers
    return gpu_helpers


def _hidden(T, seed, emin=-30, emax=30):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((T, H // 128, 128), generator=g)
    e = torch.randint(emin, emax + 1, (T, H // 128, 1), generator=g).float()
    return (x * torch.exp2(e)).reshape(T, H)


def _check(x_cpu, dtype):
    gh = _gh()
    x = x_cpu.to(dtype)
    q, s = gh.pkg.quantize_hidden(x.to("cuda"))
    torch.cuda.synchronize()
    q_ref, s_ref = quant.quantize_hidden(x.float().numpy())
    qg = q.view(torch.uint8).cpu().numpy()
    sg = s.cpu().numpy()
    bad = np.argwhere(qg != q_ref)
    assert bad.size == 0, f"{len(bad)} codes differ, first at {bad[0].tolist()}: {qg[tuple(bad[0])]} vs {q_ref[tuple(bad[0])]}"
    assert np.array_equal(sg.view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("T", [1, 15, 16, 17, 64, 1000])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_matches_oracle(T, dtype):
    print(f"quantize T={T} {dtype}", flush=True)
    # fp16 has a narrower exponent range: keep its blocks inside it
    lim = 12 if dtype == torch.float16 else 30
    _check(_hidden(T, 7 * T + 1, -lim, lim), dtype)


def test_prefill_size():
    print("quantize T=8192 bf16", flush=True)
    _check(_hidden(8192, 3, -8, 8), torch.bfloat16)


def test_special_values():
    print("quantize special values", flush=True)
    x = _hidden(6, 99, -4, 4)
    x[0, 0:128] = 0.0                                    # zero block: scale 1e-12, codes 0
    x[0, 128:256] = -0.0                                 # negative zeros keep their sign
    x[1, 0:128] = 0.0
    x[1, 5] = 3.0                                        # a single nonzero element
    x[2, 0:128] = torch.linspace(-1e-3, 1e-3, 128)       # outputs through the subnormal codes
    x[2, 7] = 1.0
    x[3, :] = 1e-30                                      # scale clamped to 1e-12
    x[4, 0:128] = 3.0e38                                 # near the bf16 and fp32 maximum
    x[5, 256:384] = -2.5                                 # constant block: every code -448
    _check(x, torch.bfloat16)
    _check(x, torch.float32)


def test_layer_on_quantized_input():
    """Quantising bf16 hidden states on the GPU and running the layer equals running it on
    the torch-quantised tensors (the same bits, so the same output)."""
    print("quantize -> layer T=48", flush=True)
    gh = _gh()
    dev = torch.device("cuda:0")
    T = 48
    w = gh.inputs.make_weights(5, dev)
    logits, bias, _, _ = gh.inputs.make_activations(T, 6, dev)
    x = torch.randn((T, H), generator=torch.Generator().manual_seed(8)).to(torch.bfloat16)
    hq_t, hs_t = gh.inputs.quantize_rows_1x128(x)
    hq, hs = gh.pkg.quantize_hidden(x.to(dev))
    assert torch.equal(hq.view(torch.uint8).cpu(), hq_t.view(torch.uint8))
    assert torch.equal(hs.cpu(), hs_t)
    kw = dict(routing_logits=logits, routing_bias=bias, gemm1_weights=w[0], gemm1_weights_scale=w[1],
              gemm2_weights=w[2], gemm2_weights_scale=w[3], local_expert_offset=0, routed_scaling_factor=2.5)
    out_a = torch.empty((T, H), dtype=torch.bfloat16, device=dev)
    out_b = torch.empty_like(out_a)
    gh.pkg.run(hidden_states=hq, hidden_states_scale=hs, output=out_a, **kw)
    gh.pkg.run(hidden_states=hq_t.to(dev), hidden_states_scale=hs_t.to(dev), output=out_b, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b)


def test_misaligned_buffers():
    """Input and output buffers off the kernel's access alignment (bf16 input 4 bytes off, fp8
    output 4 bytes off) give the aligned call's codes and scales."""
    gh = _gh()
    x = _hidden(37, 11).to(torch.bfloat16).to("cuda")
    q_ref, s_ref = gh.pkg.quantize_hidden(x)
    xb = torch.zeros(4 + x.numel() * 2, dtype=torch.uint8, device="cuda")
    xm = xb[4:].view(torch.bfloat16).view(x.shape)
    xm.copy_(x)
    ob = torch.zeros(4 + q_ref.numel(), dtype=torch.uint8, device="cuda")
    qm = ob[4:].view(torch.float8_e4m3fn).view(q_ref.shape)
    assert xm.data_ptr() % 16 != 0 and qm.data_ptr() % 8 != 0
    q, s = gh.pkg.quantize_hidden(xm, out=qm)
    torch.cuda.synchronize()
    assert q.data_ptr() == qm.data_ptr()
    assert torch.equal(q.view(torch.uint8), q_ref.view(torch.uint8)) and torch.equal(s, s_ref)


def test_validation():
    gh = _gh()
    with pytest.raises(AssertionError, match="hidden must be \\[T, 7168\\]"):
        gh.pkg.quantize_hidden(torch.zeros((4, 100), dtype=torch.bfloat16, device="cuda"))
    with pytest.raises(AssertionError, match="float32, bfloat16 or float16"):
        gh.pkg.quantize_hidden(torch.zeros((4, H), dtype=torch.int32, device="cuda"))
    q, s = gh.pkg.quantize_hidden(torch.zeros((0, H), dtype=torch.bfloat16, device="cuda"))
    assert q.shape == (0, H) and s.shape == (56, 0)
