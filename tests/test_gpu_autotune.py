"""GPU checks of the opt-in tile autotuner of int8_matmul (LYNNREAL_AMD_AUTOTUNE=1).

The reference tunes its Triton tile per shape on first use and keeps the
choice in memory and in a JSON file (model/int8_gemm.py:53-81,124-151). Here
the candidates are the HIP tiles; each computes the same bits, so a tuned
call must equal the untuned one and the oracle bit for bit, and the recorded
choice must be read back instead of timing again.
"""
import json

import pytest
import torch

from lynnreal_omni_amd import int8_gemm
from oracle import torch_path as tp

pytestmark = pytest.mark.gpu


@pytest.fixture
def tuning(monkeypatch, tmp_path):
    # The switch is read at import (LYNNREAL_AMD_AUTOTUNE=1); set it as that would.
    monkeypatch.setattr(int8_gemm, "_AUTOTUNE", True)
    monkeypatch.setenv("LYNNREAL_AMD_CACHE_DIR", str(tmp_path))
    int8_gemm._selected.clear()
    yield tmp_path
    int8_gemm._selected.clear()


def _case(m, n, k, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-127, 128, (m, k), dtype=torch.int8, generator=g)
    w = torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=g)
    rs = torch.rand(m, generator=g) * 1e-2 + 1e-3
    cs = torch.rand(n, generator=g) * 4e-3 + 1e-3
    b = (0.02 * torch.randn(n, generator=g)).bfloat16()
    return (q, w, rs, cs, b), (q.cuda(), w.cuda().t(), rs.cuda(), cs.cuda(), b.cuda())


@pytest.mark.parametrize("m,n,k", [(512, 1024, 1024), (129, 520, 640), (2048, 2560, 1280)])
def test_tuned_call_equals_oracle_and_is_recorded(tuning, m, n, k):
    (q, w, rs, cs, b), args = _case(m, n, k, m + n + k)
    got = int8_gemm.int8_matmul(*args)
    assert torch.equal(got.cpu(), tp.epilogue(tp.int_mm(q, w), rs.reshape(-1, 1), cs.reshape(1, -1), b))
    files = list(tuning.glob("int8-*.json"))
    assert len(files) == 1
    choice = int8_gemm._decode(json.loads(files[0].read_text()))
    assert choice is not int8_gemm._MISSING
    assert list(int8_gemm._selected.values()) == [choice]
    # The untuned library choice and the tuned one give the same bits.
    assert torch.equal(got, int8_gemm.int8_matmul(*args, tile=choice if choice is not None else "auto"))


def test_recorded_choice_is_read_back(tuning, monkeypatch):
    """A cache file decides the tile without timing: the recorded (128, 128)
    is taken even where it is not the fastest, and the output is unchanged."""
    (q, w, rs, cs, b), args = _case(256, 512, 512, 11)
    first = int8_gemm.int8_matmul(*args)
    [path] = list(tuning.glob("int8-*.json"))
    path.write_text(json.dumps([128, 128]))
    int8_gemm._selected.clear()
    timed = []
    monkeypatch.setattr(torch.cuda, "Event", lambda **kw: timed.append(kw) or pytest.fail("timed again"))
    again = int8_gemm.int8_matmul(*args)
    assert not timed
    assert list(int8_gemm._selected.values()) == [(128, 128)]
    assert torch.equal(first, again)


def test_gated_and_gelu_epilogues_tune_separately(tuning):
    """The epilogue is part of the key, as the bias flag is in the reference's."""
    m, n, k = 256, 1024, 512
    (q, w, rs, cs, b), args = _case(m, n, k, 5)
    plain = int8_gemm.int8_matmul(*args)
    gelu = int8_gemm.int8_matmul(*args, activation="gelu_tanh")
    g = torch.Generator().manual_seed(6)
    residual = torch.randn(1, m, n, generator=g).bfloat16().cuda()
    table = (0.1 * torch.randn(1, 6 * n, generator=g)).bfloat16().cuda()
    idx = torch.zeros(m, dtype=torch.int64).cuda()
    gated = int8_gemm.int8_matmul(*args, residual=residual, table=table, indices=idx, gate_slot=2)
    assert len(list(tuning.glob("int8-*.json"))) == 3
    library = dict(tile="auto")
    assert torch.equal(plain, int8_gemm.int8_matmul(*args, **library))
    assert torch.equal(gelu, int8_gemm.int8_matmul(*args, activation="gelu_tanh", **library))
    assert torch.equal(gated, int8_gemm.int8_matmul(*args, residual=residual, table=table, indices=idx,
                                                    gate_slot=2, **library))


def test_capture_takes_the_library_choice(tuning):
    """Inside graph capture nothing is timed or recorded; the captured call
    runs the library's own tile and replays to the eager result."""
    (q, w, rs, cs, b), args = _case(256, 512, 512, 21)
    eager = int8_gemm.int8_matmul(*args, tile="auto")
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = int8_gemm.int8_matmul(*args)
    torch.cuda.current_stream().wait_stream(stream)
    assert not list(tuning.glob("int8-*.json")) and not int8_gemm._selected
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
