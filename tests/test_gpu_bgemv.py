"""GPU parity of the batched decode GEMV (lsq_bgemv.hip: 17..64 tokens, whole row tiles per
workgroup (1, 3 or 5 by layer size), K and the tokens split over its 8 waves, activations
DMA'd into per-wave LDS slabs, the phases' partial sums added in order). By default the
kernel serves INT4 at 33..64 tokens, INT4 at 17..32 tokens below 1000 row tiles and INT8
up to 256 row tiles; most tests force it for every shape it covers (LSQ_BGEMV=1) so that
every instantiation runs, and one runs the default dispatch on the Qwen2.5-0.5B shapes.

Bars as in test_gpu_parity.py: rel = max|y - y_ref| / max|y_ref| <= 1e-2 against the
float64 oracle (oracle.quant_oracle.linear_f64 on the oracle's dequantized weights,
src/kernels/quantization.py:104-141). Shapes cover the partition edges: a partial last row
tile, k-tile counts that leave waves with unequal runs or none (K = 384: 3 k tiles for 4
waves), token counts at the block edges (17, 32, 33, 64), strided activations.
"""

import numpy as np
import pytest
import torch

import bench
from localstrm_amd import QuantizedLinear
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _force_bgemv(monkeypatch):
    monkeypatch.setenv("LSQ_BGEMV", "1")

DEV = torch.device("cuda:0")
REL_TOL = 1e-2


def _say(msg):
    print(msg, flush=True)


def _dtn(dtype):
    return {torch.float16: "f16", torch.bfloat16: "bf16"}[dtype]


def _layer(kind, n, k, group=128, dtype=torch.bfloat16, bias=False, seed=0, scale_dtype=None):
    if kind == "int8":
        w, s, _ = bench.make_int8(n, k, 1, x_dtype=dtype, seed=seed)
        ql = QuantizedLinear.from_quantized(w.to(DEV), s.to(DEV), quant_type="int8")
    else:
        w, s, _ = bench.make_int4(n, k, 1, group, x_dtype=dtype, seed=seed)
        if group >= k:
            s = s.float()
        if scale_dtype is not None:
            s = s.to(scale_dtype)
        ql = QuantizedLinear.from_quantized(w.to(DEV), s.to(DEV), quant_type="int4", in_features=k,
                                            group_size=group)
    b = None
    if bias:
        b = torch.randn(n, generator=torch.Generator().manual_seed(seed + 7)).to(dtype)
        ql.bias = torch.nn.Parameter(b.to(DEV), requires_grad=False)
    return ql, w, s, b


def _oracle(kind, w, s, b, x, k, group, dt, rows):
    if kind == "int8":
        wd = qo.dequant_int8(w[rows].numpy(), s[rows].numpy(), dt)
    else:
        wd = qo.dequant_int4(w[rows].numpy(), s[rows].float().numpy(), k, min(group, k), dt)
    return qo.linear_f64(x.float().numpy(), wd, None if b is None else b[rows].float().numpy(), dt)


def _check(kind, n, k, m, group=128, dtype=torch.bfloat16, bias=False, seed=0, scale_dtype=None, ldx=None):
    ql, w, s, b = _layer(kind, n, k, group, dtype, bias, seed, scale_dtype)
    g = torch.Generator().manual_seed(seed + 100)
    x = torch.randn(m, k, generator=g).to(dtype)
    xd = x.to(DEV)
    if ldx is not None:
        big = torch.zeros(m, ldx, dtype=dtype, device=DEV)
        big[:, :k] = xd
        xd = big[:, :k]
    with torch.no_grad():
        y = ql(xd).float().cpu().numpy()
    rows = np.arange(n) if n <= 2048 else np.sort(np.random.default_rng(seed).choice(n, 640, replace=False))
    rows = np.unique(np.concatenate([rows, [n - 1]]))  # the partial last row tile
    err = qo.rel_err(y[:, rows], _oracle(kind, w, s, b, x, k, group, _dtn(dtype), rows))
    _say(f"  {kind} {n}x{k} M={m} g={group} {_dtn(dtype)} bias={bias} ldx={ldx}: rel_err={err:.3e}")
    assert np.isfinite(y).all()
    assert err <= REL_TOL
    return ql, xd, y


@pytest.mark.parametrize("m", [17, 24, 32, 33, 48, 64])
@pytest.mark.parametrize("kind", ["int4", "int8"])
def test_bgemv_decode_shape(kind, m):
    """The Qwen2.5-7B MLP's batched decode shape, 18944 x 3584 (1184 row tiles: 237
    workgroups), bias on odd M."""
    _check(kind, 18944, 3584, m, bias=(m % 2 == 1), seed=m)


@pytest.mark.parametrize("k", [384, 1152, 2048])
@pytest.mark.parametrize("kind", ["int4", "int8"])
def test_bgemv_partition_edges(kind, k):
    """16390 rows (1025 row tiles, the last partial; 205 workgroups of 5); K of 3 k tiles
    (one of the 4 waves has none), 9 (runs of 3, 2, 2, 2) and 16."""
    for m in (17, 64):
        _check(kind, 16390, k, m, bias=True, seed=k + m)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("group", [128, 256, 1024, 2048])
def test_bgemv_groups_and_dtypes(group, dtype):
    """Group sizes of 1, 2, 8 k tiles and per-channel INT4 (group = K), both activation types."""
    _check("int4", 16384, 2048, 40, group=group, dtype=dtype, bias=True, seed=group)


@pytest.mark.parametrize("sdt", [torch.float16, torch.float32])
def test_bgemv_scale_dtypes(sdt):
    _check("int4", 16384, 1024, 20, scale_dtype=sdt, seed=3)


def test_bgemv_strided_activations():
    _check("int4", 16384, 1024, 36, ldx=1536, seed=4)
    _check("int8", 16384, 1024, 36, ldx=1152, seed=5)


def test_bgemv_deterministic_and_matches_previous_kernel(monkeypatch):
    """Bit-identical on a second call (fixed reduction order); the chunked decode kernel
    (LSQ_BGEMV=0) agrees within the contract."""
    ql, xd, y1 = _check("int4", 18944, 3584, 64, seed=9)
    with torch.no_grad():
        y2 = ql(xd).float().cpu().numpy()
        monkeypatch.setenv("LSQ_BGEMV", "0")
        y_old = ql(xd).float().cpu().numpy()
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    err = qo.rel_err(y1, y_old.astype(np.float64))
    _say(f"  new vs chunked decode kernel: rel={err:.3e}")
    assert err <= REL_TOL


@pytest.mark.parametrize("m", [17, 32, 48, 64])
@pytest.mark.parametrize("kind", ["int4", "int8"])
def test_bgemv_small_layers(kind, m):
    """The one- and three-row-tile workgroups: the Qwen2.5-0.5B projections of the batched
    decode step (896 x 4864 down: 56 workgroups of one row tile; 4864 x 896 gate / up: 102
    of three; 1152 x 896 fused q/k/v: 72 of one; 128 x 896 k / v: 8 of one)."""
    for n, k in ((896, 4864), (4864, 896), (1152, 896), (128, 896)):
        _check(kind, n, k, m, bias=(n != 896), seed=n + k + m)


@pytest.mark.parametrize("n", [4090, 4096, 4112, 12288, 12304])
def test_bgemv_row_tile_bands(n):
    """Row-tile counts at the 1 / 3 / 5 boundaries: 256 (one each), 257 (86 workgroups of
    three or two), 768 (256 of three), 769 (154 of five or four); 4090 rows end in a
    partial tile."""
    for kind in ("int4", "int8"):
        _check(kind, n, 1024, 40, bias=True, seed=n)


@pytest.mark.parametrize("m", [20, 32, 64])
def test_bgemv_default_dispatch_qwen05b(m, monkeypatch):
    """The default policy (no LSQ_BGEMV) on the 0.5B shapes it now takes, INT4 and INT8."""
    monkeypatch.delenv("LSQ_BGEMV", raising=False)
    for kind in ("int4", "int8"):
        for n, k in ((896, 4864), (9728, 896), (896, 896)):
            _check(kind, n, k, m, seed=3 * n + k + m)


# ---- split-K form (at most 128 row tiles, 16+ k tiles, with the module's workspace):
# one row tile per workgroup times S K slices, the slices added in order by a merge kernel.

@pytest.mark.parametrize("m", [17, 32, 33, 64])
@pytest.mark.parametrize("kind", ["int4", "int8"])
def test_bgemv_split_k_down_proj(kind, m, monkeypatch):
    """Qwen2.5-0.5B down_proj 896 x 4864 (56 row tiles, 38 k tiles: 4 slices by default),
    bias on odd M; the split is the default here, so LSQ_BGEMV is left unset."""
    monkeypatch.delenv("LSQ_BGEMV", raising=False)
    _check(kind, 896, 4864, m, bias=(m % 2 == 1), seed=m)


@pytest.mark.parametrize("splits", ["2", "5", "16"])
def test_bgemv_split_k_forced(splits, monkeypatch):
    """Forced slice counts on 2000 x 8192 (125 row tiles, the last partial; 64 k tiles),
    INT4 group-wise and per-channel, INT8, fp16 activations."""
    monkeypatch.setenv("LSQ_SPLITK", splits)
    _check("int4", 2000, 8192, 40, bias=True, seed=int(splits))
    _check("int4", 2000, 8192, 24, group=8192, seed=int(splits) + 1)
    _check("int8", 2000, 8192, 64, bias=True, seed=int(splits) + 2)
    _check("int4", 2000, 8192, 48, dtype=torch.float16, group=256, seed=int(splits) + 3)


def test_bgemv_split_k_deterministic_and_matches_unsplit(monkeypatch):
    monkeypatch.delenv("LSQ_BGEMV", raising=False)
    ql, xd, y1 = _check("int4", 896, 4864, 32, seed=41)
    with torch.no_grad():
        y2 = ql(xd).float().cpu().numpy()
        monkeypatch.setenv("LSQ_SPLITK", "0")
        y0 = ql(xd).float().cpu().numpy()
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    err = qo.rel_err(y1, y0.astype(np.float64))
    _say(f"  split vs unsplit: rel={err:.3e}")
    assert err <= REL_TOL
