"""CPU oracle of the W8A8 DiT projection path - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline),
never as the thing measured or shipped. The product path
(lynnreal_omni_amd) never imports it and has no CPU fallback.

  oracle.reference   numpy/ctypes wrappers of lr_oracle.c, the C restatement
                     of the reference's arithmetic (each function cites it)
  oracle.torch_path  the reference's torch path (model/int8.py:60-68,
                     model/int8_gemm.py:84-92, model/kernels.py semantics) in
                     torch CPU ops: an independent second restatement used to
                     pin the C one, and the CPU baseline of bench.py
  oracle.bf16        bfloat16 <-> float32 conversions on numpy arrays

The checks that pin each function (golden fixtures, closed forms, torch's
own library routines, brute force on small inputs) are in tests/test_oracle.py.
"""
