"""CPU oracle of the fused FP8 block-scale MoE layer -- TEST INFRASTRUCTURE ONLY.

A restatement in numpy of the algorithm of nikhilnd/mlsys26-flashinfer-moe's `run`
(kernel.py:562-729) and of the competition definition's fp32 dequantise-and-matmul
math it is judged against (writeup.pdf p.1 s.1.2). Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import it, and only as the checker or as the timed
CPU baseline; the product path (the HIP library) never calls into it.

Modules:
  fp8       e4m3fn decode/encode and bf16 rounding          (kernel.py:135, 729)
  routing   DeepSeek-V3 no-aux grouped routing, bit-exact    (kernel.py:428-542)
  dispatch  local filter, histogram, CSR, stable buckets,
            tile schedule                                    (kernel.py:252-407)
  experts   block-scale dequantisation, GEMM1 + SwiGLU,
            fp8 requantisation, GEMM2, weighted combine      (kernel.py:7-250, 663-729)
  layer     the whole layer, in "definition" (fp32 intermediate) or "emulated"
            (fp8-requantised intermediate, as the kernels compute it) mode.
  quant     the step before the layer: hidden states -> e4m3fn + 1x128 scales [56, T]
                                                             (kernel.py:131-135, 600-603)

How each function is pinned (tests/test_oracle_*.py):
  fp8.decode/encode, bf16_round  exhaustive/edge comparison with torch's CPU casts
                                  (tests/golden/fp8_e4m3fn_golden.npz, bf16 cases)
  routing.sigmoid_f32            float64 bound (<= 3 ulp), monotonicity, symmetry, constants
  routing.route                  transformers' DeepseekV3TopkRouter (tests/golden/routing_golden.npz),
                                  invariants, closed-form special cases (ties, forced bias)
  dispatch.*                     brute-force bucket construction, invariants
  experts.*                      exact small-integer cases, one-hot rows, SwiGLU half
                                  convention (closed form), requant closed form,
                                  torch CPU matmul at small shapes
  layer.layer_forward            pure-Python brute force of the whole composition on
                                  tiny shapes
  quant.quantize_hidden          torch's CPU float8_e4m3fn cast of x / scale, block-max
                                  448 and zero-block closed forms, power-of-two scaling
                                  and sign symmetry, round-trip error bound
"""
