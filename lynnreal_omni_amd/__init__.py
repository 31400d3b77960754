"""MI355X-native (gfx950) W8A8 DiT projection path of LynnReal-Omni.

Drop-in modules with the reference's call surface:
  int8_gemm           int8_matmul, _torch_matmul          (model/int8_gemm.py)
  int8                Int8Linear, quantize_transformer    (model/int8.py)
  kernels             quantize_rows, int8_epilogue, _rms_adaln(_quant_int8),
                      residual_rms_quant, _gated_residual, _swiglu(_quant_int8)
                                                          (model/kernels.py)
  elementwise_fusion  block_forward, enable_elementwise_fusion
                                                          (model/elementwise_fusion.py)
  fusion              projection_chain (the fused W8A8 block chain)
  acceleration        fastest_available, optional_kernel_failure
                                                          (model/acceleration.py)
  flash_int8          the Flash W8A8 shard format loader  (model/flash_int8.py)
All compute runs in liblynnreal_amd.so (hand-written HIP for gfx950, C ABI in
include/lynnreal_amd.h); there is no CPU or Triton fallback.
"""
__version__ = "0.1.0"
