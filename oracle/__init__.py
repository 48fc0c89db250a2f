"""CPU oracle for the hybrid DiT block hot path. TEST INFRASTRUCTURE ONLY.

A plain restatement (numpy / torch-CPU, fp32-fp64) of the reference's algorithms,
each function citing the reference file:line it follows. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and
only as the checker or the timed CPU baseline, never as part of the product path.

Pinning (what independently checks each function, beyond the GPU comparison):
  mxfp8.e4m3fn_encode      torch.float8_e4m3fn cast, exhaustive over every bf16 pattern
                           times power-of-two scales; decode round trip
  mxfp8.e8m0_exponent      closed form max(ceil(log2(amax/448)), -127); reference KATs
                           [0,224,448,449,896] -> [0,126,127,128,128], [1,4,16] -> [119,121,123]
  mxfp8.swizzle_offset     reference swizzle KAT (test_rtx5090_mxfp8_capability.py:31-40),
                           bijection on [RP x KP/32]
  mxfp8.quantize           reconstruction bound |x - dq| <= 2^-4 |amax|, padding zeros,
                           chunk invariance (test_paper_stack_mxfp8_ops.py:49-64)
  mxfp8.gemm               float64 matmul of exact dequantized operands (closed form)
  mxfp8.prenorm/act        float64 evaluation of the stated formula, torch RMSNorm/GELU
                           cross-checks
Functions added for the VDA and window branches document their pins in their modules.
"""
