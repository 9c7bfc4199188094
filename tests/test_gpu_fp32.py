"""GPU parity of the fp32-activation decode GEMV (lsq_gemv32.hip: 1..8 fp32 tokens per
launch, more in blocks of 8, on the tiled INT8 / INT4 layouts, each weight formed as
round_fp32(q * s) like the reference's dequantize(), products summed in fp32 on the VALU).
The reference's CPU path runs in fp32 (src/kernels/quantization.py:104-141), and the
single-layer INT8 4864 x 896 workload allows fp32 activations.

Bar: rel = max|y - y_ref| / max|y_ref| <= 1e-5 against the float64 oracle
(oracle.quant_oracle.linear_f64 on the oracle's fp32-dequantized weights), the bar the
fp32 case of the config-1 test holds. Shapes cover the workgroup partition edges (a partial
last row tile, few k tiles, 4 / 8 / 16 waves), group sizes, scale and bias types, strided
activations; the generic kernel (LSQ_GEMV32=0) serves as a second, independent GPU path.
"""

import numpy as np
import pytest
import torch

import bench
from localstrm_amd import QuantizedLinear
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TOL = 1e-5


def _say(msg):
    print(msg, flush=True)


def _layer(kind, n, k, group=128, seed=0, scale_dtype=None, bias=False):
    if kind == "int8":
        w, s, _ = bench.make_int8(n, k, 1, seed=seed)
        if scale_dtype is not None:
            s = s.to(scale_dtype)
        ql = QuantizedLinear.from_quantized(w.to(DEV), s.to(DEV), quant_type="int8")
    else:
        w, s, _ = bench.make_int4(n, k, 1, group, seed=seed)
        if group >= k:
            s = s.float()
        if scale_dtype is not None:
            s = s.to(scale_dtype)
        ql = QuantizedLinear.from_quantized(w.to(DEV), s.to(DEV), quant_type="int4", in_features=k,
                                            group_size=group)
    b = None
    if bias:
        b = torch.randn(n, generator=torch.Generator().manual_seed(seed + 7))
        ql.bias = torch.nn.Parameter(b.to(DEV), requires_grad=False)
    return ql, w, s, b


def _oracle(kind, w, s, b, x, k, group, rows):
    if kind == "int8":
        wd = qo.dequant_int8(w[rows].numpy(), s[rows].float().numpy(), "f32")
    else:
        wd = qo.dequant_int4(w[rows].numpy(), s[rows].float().numpy(), k, min(group, k), "f32")
    return qo.linear_f64(x.numpy(), wd, None if b is None else b[rows].numpy(), "f32")


def _check(kind, n, k, m, group=128, seed=0, scale_dtype=None, bias=False, ldx=None):
    ql, w, s, b = _layer(kind, n, k, group, seed, scale_dtype, bias)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(seed + 100))
    xd = x.to(DEV)
    if ldx is not None:
        big = torch.zeros(m, ldx, device=DEV)
        big[:, :k] = xd
        xd = big[:, :k]
    with torch.no_grad():
        y = ql(xd).cpu().numpy()
    assert y.dtype == np.float32
    rows = np.arange(n) if n <= 2048 else np.sort(np.random.default_rng(seed).choice(n, 640, replace=False))
    rows = np.unique(np.concatenate([rows, [n - 1]]))  # the partial last row tile
    err = qo.rel_err(y[:, rows], _oracle(kind, w, s, b, x, k, group, rows))
    _say(f"  {kind} {n}x{k} M={m} g={group} scale={scale_dtype} bias={bias} ldx={ldx}: rel_err={err:.3e}")
    assert np.isfinite(y).all()
    assert err <= TOL
    return ql, xd, y


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 16, 23, 64])
@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_fp32_decode_baseline_shape(kind, m):
    """18944 x 3584 (1184 row tiles: 237 workgroups of 16 waves), bias on even M; past 8
    tokens in blocks of 8 (23: two full blocks and one of 7)."""
    _check(kind, 18944, 3584, m, bias=(m % 2 == 0), seed=m)


@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_fp32_config1_shape(kind):
    """Qwen2.5-0.5B gate_proj 4864 x 896, the single-layer INT8 workload (152 workgroups of
    8 waves)."""
    for m in (1, 4, 8):
        _check(kind, 4864, 896, m, seed=11 + m)


@pytest.mark.parametrize("n,k", [(16390, 128), (16390, 384), (4090, 1152), (130, 2048), (16, 128)])
@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_fp32_partition_edges(kind, n, k):
    """A partial last row tile, one to three k tiles (runs shorter than the ring), a single
    row tile, layers of 1..1025 row tiles (4, 8 and 16 waves)."""
    _check(kind, n, k, 3, bias=True, seed=n + k)


@pytest.mark.parametrize("group", [128, 256, 1024, 2048])
def test_fp32_int4_groups(group):
    """Group sizes of 1, 2 and 8 k tiles, and per-channel INT4 (group = K)."""
    _check("int4", 16384, 2048, 2, group=group, bias=True, seed=group)


@pytest.mark.parametrize("kind,sdt", [("int8", torch.float16), ("int8", torch.bfloat16),
                                      ("int4", torch.float16), ("int4", torch.float32)])
def test_fp32_scale_dtypes(kind, sdt):
    _check(kind, 4864, 1024, 2, scale_dtype=sdt, seed=5)


def test_fp32_strided_activations():
    _check("int8", 4864, 1024, 3, ldx=1032, seed=6)
    _check("int4", 4864, 1024, 3, ldx=1028, seed=7)
    # a row stride that is not a multiple of 4 floats: the generic kernel takes it
    _check("int8", 4864, 1024, 2, ldx=1025, seed=8)


def test_fp32_deterministic_and_matches_generic_kernel(monkeypatch):
    """Bit-identical on a second call (fixed summation order); the generic kernel
    (LSQ_GEMV32=0, one wave per output row) within the bar; nine tokens (a block of 8 and
    one of 1) meet it too."""
    for kind in ("int8", "int4"):
        ql, xd, y1 = _check(kind, 18944, 3584, 4, bias=True, seed=21)
        with torch.no_grad():
            y2 = ql(xd).cpu().numpy()
            monkeypatch.setenv("LSQ_GEMV32", "0")
            y0 = ql(xd).cpu().numpy()
            monkeypatch.delenv("LSQ_GEMV32")
        assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
        err = qo.rel_err(y1, y0.astype(np.float64))
        _say(f"  {kind} fp32 GEMV vs generic kernel: rel={err:.3e}")
        assert err <= TOL
        _check(kind, 4864, 896, 9, seed=22)
