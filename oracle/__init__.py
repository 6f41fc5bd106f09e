"""CPU oracle for the quantized-linear hot path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's CPU dequantize-then-matmul path
(kairyu/quant/{awq,gptq,fp8,int8}.py, kairyu/quant/linear.py:401-553,
kairyu/models/moe.py:86-119,255-273, kairyu/models/grouped_moe.py:295-330).
It is the checker the HIP kernels are compared against.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the ``kairyu_amd`` package never does, and nothing here is ever the
thing measured or shipped.

Pinning (how each function is known to be right, see tests/test_oracle_*.py):
  numerics.e4m3_encode/decode  exhaustive vs torch.float8_e4m3fn casts
  numerics.bf16_round          vs torch.bfloat16 casts (RNE) on 1e6 values
  formats.awq_*                reference known answer (tests/unit/test_quant_compute.py:14-23)
                               + brute-force per-element decode of the GPU
                               kernel's closed-form shift (quant_gemm_gpu.py:259-261)
  formats.gptq_*               reference known answers (test_quant_compute.py:25-39)
                               + brute force
  formats.quantize_int8_*      reference fixture; torch.round half-even identity
  linear.int8_*                exactness proof: int64 matmul == fp64 BLAS matmul
  linear.fp8_*                 e4m3 products exact in fp64 (closed form)
  linear.swiglu_reference      torch's own fp16 / bf16 silu(g) * u on the CPU
                               (the reference MLP's operation, layers.py:243-244):
                               bf16 identical, fp16 within 2 ulp on a silu
                               rounding boundary (tests/test_parity_bounds.py)
  moe.route_*                  reference fixtures (test_moe_precision.py:97-154)
  moe.combine_*                reference fixtures (test_moe_precision.py:138-154,194-226)
  parity                       the device-output criteria (ulp bound with the
                               measured MFMA accumulation slack, relative RMSE,
                               the routed-expert statistics); pinned by planted
                               mistakes in tests/test_parity_bounds.py
  moe block-FP8 expert math    parity unpinned at the reference boundary (no
                               reference implementation or test exists); the
                               pieces are pinned individually as above
"""
