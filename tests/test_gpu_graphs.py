"""HIP-graph capture of the widened paths (the decode step is replayed from a graph):
W8A8 (fused and separate activation quantization, prefill GEMM), the gate / up SiLU.mul
epilogue and paged attention. Each graph is replayed several times with eager work of the
same kernels in between, and every replay must equal the eager result bit for bit."""

import pytest
import torch
import torch.nn as nn

from localstrm_amd import Int8GEMMLinear, QuantizedLinear, fuse_linears, paged_attention_decode

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _check_graph(fn, eager_between):
    with torch.no_grad():
        ref = fn().clone()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(g, stream=stream):
                out = fn()
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
            eager_between()
            torch.cuda.synchronize()


@pytest.mark.parametrize("m,path", [(1, None), (4, "unfused"), (300, None)])
def test_w8a8_graph_replays(monkeypatch, m, path):
    print(f"w8a8 graph M={m} path={path}", flush=True)
    if path:
        monkeypatch.setenv("LSQ_W8A8_PATH", path)
    torch.manual_seed(m)
    layer = Int8GEMMLinear.from_float(nn.Linear(896, 4864, bias=True), dtype=torch.bfloat16).to(DEV)
    x = torch.randn(m, 896, device=DEV, dtype=torch.bfloat16)
    x2 = torch.randn(m, 896, device=DEV, dtype=torch.bfloat16)
    _check_graph(lambda: layer(x), lambda: layer(x2))


def test_silu_mul_graph_replays():
    print("silu_mul graph", flush=True)
    torch.manual_seed(1)
    gate = QuantizedLinear.from_float(nn.Linear(896, 4864, bias=False), "int4", group_size=128).to(DEV)
    up = QuantizedLinear.from_float(nn.Linear(896, 4864, bias=False), "int4", group_size=128).to(DEV)
    f = fuse_linears([gate, up], act="silu_mul")
    x = torch.randn(32, 896, device=DEV, dtype=torch.bfloat16)
    x2 = torch.randn(32, 896, device=DEV, dtype=torch.bfloat16)
    _check_graph(lambda: f(x), lambda: f(x2))


def test_paged_attention_graph_replays():
    print("paged attention graph", flush=True)
    g = torch.Generator().manual_seed(2)
    b, h, hkv, d, bs, seq = 4, 14, 2, 64, 16, 700
    nblk = -(-seq // bs)
    nb = b * nblk + 3
    kp = torch.randint(-128, 128, (nb, bs, hkv, d), generator=g, dtype=torch.int8).to(DEV)
    vp = torch.randint(-128, 128, (nb, bs, hkv, d), generator=g, dtype=torch.int8).to(DEV)
    ks = (torch.rand(nb, bs, hkv, 1, generator=g) * 0.02 + 0.002).half().to(DEV)
    vs = (torch.rand(nb, bs, hkv, 1, generator=g) * 0.02 + 0.002).half().to(DEV)
    bt = torch.randperm(nb, generator=g)[: b * nblk].reshape(b, nblk).to(DEV)
    sl = torch.tensor([700, 1, 333, 256], dtype=torch.int64, device=DEV)
    q = torch.randn(b, h, 1, d, generator=g).half().to(DEV)
    q2 = torch.randn(b, h, 1, d, generator=g).half().to(DEV)
    run = lambda qq: paged_attention_decode(qq, kp, vp, bt, sl, bs, ks, vs, max_sl=seq)
    _check_graph(lambda: run(q), lambda: run(q2))


@pytest.mark.parametrize("n,k,m", [(3584, 18944, 8), (896, 4864, 32), (896, 4864, 16)])
def test_split_k_graph_replays(n, k, m):
    """The split-K decode forms (16-token split at 3584 x 18944, the batched split at
    896 x 4864), whose workspace the module takes from torch's allocator inside forward:
    captured, replayed three times with eager calls of the same layer in between, every
    replay equal to the eager result bit for bit."""
    print(f"split-K graph N={n} K={k} M={m}", flush=True)
    torch.manual_seed(n + m)
    layer = QuantizedLinear.from_float(nn.Linear(k, n, bias=True), "int4", group_size=128).to(DEV)
    x = torch.randn(m, k, device=DEV).to(torch.bfloat16)
    _check_graph(lambda: layer(x), lambda: layer(x))
