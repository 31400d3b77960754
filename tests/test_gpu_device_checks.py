"""Every wrapper refuses a tensor argument that is not on the device of its
first tensor, with a ValueError raised before any kernel launch.

The kernels take raw device pointers: a host tensor (for example adaLN
indices built on the CPU) reaching a kernel would be an invalid address. The
reference's Triton launches raise a Python error in that case, and the
fused-block guard (model/fusion.py:101-116) relies on getting one.
"""
import types

import pytest
import torch

from lynnreal_omni_amd import flash, int8_gemm, kernels

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _bf(shape, device=DEV):
    return torch.randn(*shape, device=device).bfloat16()


def _gemm_args():
    a = torch.randint(-127, 128, (32, 64), dtype=torch.int8, device=DEV)
    w = torch.randint(-127, 128, (48, 64), dtype=torch.int8, device=DEV)
    rs = torch.rand(32, device=DEV)
    cs = torch.rand(48, device=DEV)
    bias = _bf((48,))
    return dict(a=a, b=w.t(), row_scale=rs, column_scale=cs, bias=bias)


@pytest.mark.parametrize("name", ["b", "row_scale", "column_scale", "bias"])
def test_int8_matmul_refuses_host_operands(name):
    args = _gemm_args()
    args[name] = args[name].cpu()
    with pytest.raises(ValueError, match=name):
        int8_gemm.int8_matmul(**args)


@pytest.mark.parametrize("name", ["residual", "table", "indices"])
def test_gated_epilogue_refuses_host_operands(name):
    args = _gemm_args()
    extra = dict(residual=_bf((32, 48)), table=_bf((1, 6 * 48)),
                 indices=torch.zeros(32, dtype=torch.int64, device=DEV), gate_slot=2)
    extra[name] = extra[name].cpu()
    with pytest.raises(ValueError, match=name):
        int8_gemm.int8_matmul(**args, **extra)


def test_int32_gemm_refuses_host_weight():
    args = _gemm_args()
    with pytest.raises(ValueError, match="b is on cpu"):
        int8_gemm.int8_matmul_int32(args["a"], args["b"].cpu())


def test_epilogue_refuses_host_scales():
    acc = torch.randint(-1000, 1000, (8, 16), dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="weight_scale"):
        kernels.int8_epilogue(acc, torch.rand(8, device=DEV), torch.rand(16), None)
    with pytest.raises(ValueError, match="bias"):
        kernels.int8_epilogue(acc, torch.rand(8, device=DEV), torch.rand(16, device=DEV), _bf((16,), "cpu"))


@pytest.mark.parametrize("name", ["norm.weight", "table", "indices"])
def test_norm_refuses_host_operands(name):
    x = _bf((1, 8, 64))
    parts = {"norm.weight": _bf((64,)), "table": _bf((1, 6 * 64)),
             "indices": torch.zeros(8, dtype=torch.int64, device=DEV)}
    parts[name] = parts[name].cpu()
    norm = types.SimpleNamespace(weight=parts["norm.weight"], eps=1e-6)
    for fn in (kernels._rms_adaln, kernels._rms_adaln_quant_int8):
        with pytest.raises(ValueError, match=name.replace(".", r"\.")):
            fn(x, norm, parts["table"], parts["indices"], 0, 1)
    with pytest.raises(ValueError, match=name.replace(".", r"\.")):
        kernels.residual_rms_quant(x, _bf((1, 8, 64)), norm, parts["table"], parts["indices"])


def test_residual_norm_refuses_host_update():
    x = _bf((1, 8, 64))
    norm = types.SimpleNamespace(weight=_bf((64,)), eps=1e-6)
    with pytest.raises(ValueError, match="update"):
        kernels.residual_rms_quant(x, _bf((1, 8, 64), "cpu"), norm, _bf((1, 6 * 64)),
                                   torch.zeros(8, dtype=torch.int64, device=DEV))


@pytest.mark.parametrize("name", ["update", "table", "indices"])
def test_gated_residual_refuses_host_operands(name):
    parts = {"update": _bf((1, 8, 64)), "table": _bf((1, 6 * 64)),
             "indices": torch.zeros(8, dtype=torch.int64, device=DEV)}
    parts[name] = parts[name].cpu()
    with pytest.raises(ValueError, match=name):
        kernels._gated_residual(_bf((1, 8, 64)), parts["update"], parts["table"], parts["indices"], 2)


@pytest.mark.parametrize("name", ["key", "query_weight", "key_weight", "cos", "sin"])
def test_qk_norm_rope_refuses_host_operands(name):
    q = _bf((1, 4, 2, 64))
    parts = {"key": _bf((1, 4, 2, 64)), "query_weight": _bf((64,)), "key_weight": _bf((64,)),
             "cos": torch.rand(4, 64, device=DEV), "sin": torch.rand(4, 64, device=DEV)}
    parts[name] = parts[name].cpu()
    with pytest.raises(ValueError, match=name):
        kernels.qk_norm_rope(q, parts["key"], parts["query_weight"], parts["key_weight"],
                             (parts["cos"], parts["sin"]), 1e-6)


def test_qk_norm_rope_checks_the_norm_weight_length():
    q, k = _bf((1, 4, 2, 64)), _bf((1, 4, 2, 64))
    rot = (torch.rand(4, 64, device=DEV), torch.rand(4, 64, device=DEV))
    with pytest.raises(ValueError, match="head_dim=64"):
        kernels.qk_norm_rope(q, k, _bf((32,)), _bf((64,)), rot, 1e-6)
    with pytest.raises(ValueError, match="head_dim=64"):
        kernels.qk_norm_rope(q, k, _bf((64,)), _bf((128,)), rot, 1e-6)


def test_adaln_table_refuses_host_operands():
    w = _bf((96, 64))
    with pytest.raises(ValueError, match="temb"):
        kernels.adaln_table(torch.randn(2, 64), w)
    with pytest.raises(ValueError, match="bias"):
        kernels.adaln_table(torch.randn(2, 64, device=DEV), w, _bf((96,), "cpu"))


@pytest.mark.parametrize("name", ["current", "input"])
def test_flash_restore_refuses_host_operands(name):
    parts = {"current": _bf((1, 4, 32)), "input": _bf((1, 4, 32))}
    parts[name] = parts[name].cpu()
    with pytest.raises(ValueError, match=name):
        flash.restore(_bf((1, 8, 32)), parts["current"], parts["input"],
                      torch.arange(8, device=DEV) // 2)
