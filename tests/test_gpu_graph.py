"""The projection chain captured in a HIP graph (torch.cuda.CUDAGraph over the
library's launches on the capturing stream): the library allocates nothing,
synchronizes nothing and records no memset, so a captured chain replays to the
eager result. Each replay runs on new inputs copied into the captured buffers,
with eager work and synchronizations between the replays, and is checked bit
for bit against the eager chain on the same inputs."""
import types

import pytest
import torch

from helpers import bf16_randn
from lynnreal_omni_amd import fusion, kernels as k
from lynnreal_omni_amd.int8 import Int8Linear

pytestmark = pytest.mark.gpu

T, D, F = 300, 512, 1024      # 300 rows: a tail tile on every GEMM


def _layers(g, dev):
    def one(n, kk):
        w = torch.randint(-127, 128, (n, kk), dtype=torch.int8, generator=g)
        s = torch.rand(n, 1, generator=g) * 4e-3 + 1e-3
        b = (0.02 * torch.randn(n, generator=g)).bfloat16()
        return Int8Linear.from_packed(w.to(dev), s.to(dev), b.to(dev), gemm="hip")
    return fusion.ChainLayers(to_qkv=one(3 * D, D), to_out=one(D, D), up=one(F, D), down=one(D, F))


def _inputs(g, dev):
    x = bf16_randn((1, T, D), g, outliers=0.01).to(dev)
    attn = bf16_randn((1, T, D), g).to(dev)
    table = (0.1 * torch.randn(3, 6 * D, generator=g)).bfloat16().to(dev)
    idx = torch.randint(0, 3, (T,), generator=g).to(dev)
    return x, attn, table, idx


@torch.inference_mode()
def test_captured_chain_replays_match_eager():
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(77)
    layers = _layers(g, dev)
    norm = types.SimpleNamespace(weight=(1 + 0.05 * torch.randn(D, generator=g)).bfloat16().to(dev),
                                 eps=1e-6)
    static = _inputs(g, dev)

    def run(x, attn, table, idx):
        return fusion.projection_chain(x, layers, norm, norm, table, idx, attn)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(*static)                              # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run(*static)

    for replay in range(3):
        fresh = _inputs(g, dev)
        for dst, src in zip(static, fresh):
            dst.copy_(src)
        graph.replay()
        torch.cuda.synchronize()
        want = run(*fresh)                       # eager, on other buffers
        k.quantize_rows(fresh[1].reshape(T, D))   # unrelated eager work between replays
        torch.cuda.synchronize()
        for got, exp, name in zip(outs, want, ("qkv", "x1", "x2")):
            assert torch.equal(got, exp), (replay, name)
