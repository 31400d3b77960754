"""A C++ host program drives the library through the C ABI alone.

tests/abi_host/c_abi_consumer.cpp (built by lynnreal_omni_amd.build next to
the library) allocates device memory with the HIP runtime, calls
lr_quantize_rows and lr_int8_gemm (bf16 + bias and raw int32 epilogues) as a
non-Python host would, and compares every output with its own C++ statement
of the reference arithmetic (model/int8.py:64-67, model/int8_gemm.py:84-92),
bit for bit. Without a GPU it stops at lr_device_supported with status 5.
"""
import subprocess

import pytest
import torch

from lynnreal_omni_amd import build

BINARY = build.ABI_CONSUMER


def _run():
    if not BINARY.exists():
        pytest.fail(f"{BINARY} is missing: build it with `python -m lynnreal_omni_amd.build`")
    return subprocess.run([str(BINARY)], capture_output=True, text=True, timeout=240)


@pytest.mark.gpu
def test_c_abi_consumer_bit_exact():
    proc = _run()
    print(proc.stdout, proc.stderr)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "c_abi_consumer ok" in proc.stdout


def test_c_abi_consumer_links_and_refuses_without_a_gpu():
    """The program loads the library through its rpath, checks the ABI
    version and refuses to run on a machine without a gfx950 GPU."""
    if torch.cuda.is_available():
        pytest.skip("a GPU is present: the GPU test runs the program")
    proc = _run()
    assert proc.returncode == 5 and "not a gfx950" in proc.stderr, proc.stdout + proc.stderr
