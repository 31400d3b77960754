"""The capability probe (model/acceleration.py:31-39) on gfx950: both exact
probes (the MFMA GEMM against the torch path, the fused residual + norm + quant
against the two-kernel sequence) pass, so the fused path is reported available."""
import pytest

from lynnreal_omni_amd import acceleration

pytestmark = pytest.mark.gpu


def test_fastest_available_reports_the_fused_path():
    report = acceleration.fastest_available()
    assert report["int8_gemm"] == "hip"
    assert report["fused"] is True
    assert report["fallbacks"] == []
