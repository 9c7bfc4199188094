"""GPU parity of the decode GEMV kernel (lsq_gemv.hip: 1..16 tokens, tiled layouts, whole
row tiles per workgroup, last-arriving wave reduces a row tile in wave order).

Bars as in test_gpu_parity.py: rel = max|y - y_ref| / max|y_ref| <= 1e-2 against the
float64 oracle (oracle.quant_oracle.linear_f64 on the oracle's dequantized weights,
src/kernels/quantization.py:104-141). LSQ_GEMV_CFG="rpw,w,d" forces a configuration
(row tiles per workgroup, waves per workgroup, ring depth), so that every compiled
instantiation and partition edge runs: runs crossing a row-tile boundary, workgroups of
unequal size, a partial last row tile, fewer k tiles than waves per row tile.
"""

import numpy as np
import pytest
import torch

import bench
from localstrm_amd import QuantizedLinear
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
REL_TOL = 1e-2


def _say(msg):
    print(msg, flush=True)


def _dtn(dtype):
    return {torch.float16: "f16", torch.bfloat16: "bf16"}[dtype]


def _run(kind, n, k, m, group=128, dtype=torch.bfloat16, bias=False, seed=0, scale_dtype=None, rows=None):
    """Layer output on the GPU and the float64 oracle on the same (sampled) rows."""
    if kind == "int8":
        w, s, x = bench.make_int8(n, k, m, x_dtype=dtype, seed=seed)
        ql = QuantizedLinear.from_quantized(w.to(DEV), s.to(DEV), quant_type="int8")
    else:
        w, s, x = bench.make_int4(n, k, m, group, x_dtype=dtype, seed=seed)
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
    if rows is None:
        rows = np.arange(n) if n <= 2048 else np.sort(np.random.default_rng(seed).choice(n, 512, replace=False))
    with torch.no_grad():
        y = ql(x.to(DEV)).float().cpu().numpy()
    dt = _dtn(dtype)
    if kind == "int8":
        wd = qo.dequant_int8(w[rows].numpy(), s[rows].numpy(), dt)
    else:
        wd = qo.dequant_int4(w[rows].numpy(), s[rows].float().numpy(), k, min(group, k), dt)
    ref = qo.linear_f64(x.float().numpy(), wd, None if b is None else b[rows].float().numpy(), dt)
    return ql, x, y, y[:, rows], ref


def _check(kind, n, k, m, cfg=None, monkeypatch=None, **kw):
    if cfg is not None:
        monkeypatch.setenv("LSQ_GEMV_CFG", cfg)
    _, _, y, got, ref = _run(kind, n, k, m, **kw)
    err = qo.rel_err(got, ref)
    _say(f"  {kind} {n}x{k} M={m} cfg={cfg} {kw}: rel_err={err:.3e}")
    assert np.isfinite(y).all()
    assert err <= REL_TOL
    return y


@pytest.mark.parametrize("m", [1, 2, 4, 5, 16])
@pytest.mark.parametrize("kind", ["int4", "int8"])
def test_gemv_default_large_n(kind, m):
    """18944 x 3584 (1184 row tiles: the default configuration, 237 workgroups of 4-5 row
    tiles, runs crossing row tiles), bias on odd M."""
    _check(kind, 18944, 3584, m, bias=(m % 2 == 1), seed=m)


@pytest.mark.parametrize("cfg", ["1,16,2", "2,16,3", "3,8,2", "5,16,3", "5,8,3", "8,16,2", "16,16,3",
                                 "4,4,3", "1,4,2"])
@pytest.mark.parametrize("kind", ["int4", "int8"])
def test_gemv_forced_configs(kind, cfg, monkeypatch):
    """Every compiled (waves, ring depth) and several row-tile splits, at 1, 4 and 16 tokens,
    on a layer whose 1025 row tiles (N = 16390: the last tile partial) do not divide the
    grid evenly; 16 k tiles, so 16 waves still get one unit each at one row tile."""
    for m in (1, 4, 16):
        _check(kind, 16390, 2048, m, cfg=cfg, monkeypatch=monkeypatch, bias=True, seed=m + len(cfg))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("group", [128, 256, 512, 1024])
def test_gemv_groups_and_dtypes(group, dtype, monkeypatch):
    """Group sizes of 1, 2 and 4 k tiles and per-channel INT4 (group = K), both activation
    types; the small layer is forced onto this kernel."""
    _check("int4", 1040, 1024, 3, cfg="1,8,3", monkeypatch=monkeypatch, group=group, dtype=dtype,
           bias=True, seed=group)


@pytest.mark.parametrize("sdt", [torch.float16, torch.float32])
def test_gemv_scale_dtypes(sdt, monkeypatch):
    """Group scales stored as fp16 / fp32 (rounded to the activation type while staged)."""
    _check("int4", 2048, 1024, 2, cfg="2,8,2", monkeypatch=monkeypatch, scale_dtype=sdt, seed=11)


def test_gemv_non_power_of_two_groups_fall_back(monkeypatch):
    """Group 384 (3 k tiles) is not served by this kernel: the launcher declines and the
    LDS-staged decode kernel computes the layer."""
    _check("int4", 16384, 1536, 2, cfg="4,16,3", monkeypatch=monkeypatch, group=384, seed=5)


def test_gemv_matches_previous_kernel_and_is_deterministic(monkeypatch):
    """Same layer through this kernel twice (bit-identical: fixed reduction order) and
    through the LDS-staged decode kernel (LSQ_GEMV=0; same result within the contract)."""
    ql, x, y1, _, _ = _run("int4", 18944, 3584, 4, seed=21)
    xd = x.to(DEV)
    with torch.no_grad():
        y2 = ql(xd).float().cpu().numpy()
        monkeypatch.setenv("LSQ_GEMV", "0")
        y_old = ql(xd).float().cpu().numpy()
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    err = qo.rel_err(y1, y_old.astype(np.float64))
    _say(f"  new vs LDS-staged decode kernel: rel={err:.3e}")
    assert err <= REL_TOL


# ---- split-K form (layers of fewer than 1024 row tiles, 8+ k tiles, 1-16 tokens): the
# forward passes a workspace (lsq_linear_workspace_bytes), workgroups take (row-tile
# range, K slice) pairs, a second kernel adds the slices in order.

@pytest.mark.parametrize("m", [2, 3, 4, 8, 13, 16])
@pytest.mark.parametrize("kind", ["int4", "int8"])
def test_split_k_down_projection(kind, m, monkeypatch):
    """3584 x 18944 (224 row tiles, 148 k tiles; 3 to 10 slices by M; at 2 tokens, whose
    x the unsplit kernels serve by default, 3 slices forced), bias on odd M."""
    if m == 2:
        monkeypatch.setenv("LSQ_SPLITK", "3")
    rows = np.sort(np.random.default_rng(500 + m).choice(3584, 384, replace=False))
    _check(kind, 3584, 18944, m, bias=(m % 2 == 1), seed=m, rows=rows)


@pytest.mark.parametrize("m", [1, 5, 16])
@pytest.mark.parametrize("kind", ["int4", "int8"])
def test_split_k_small_layers(kind, m, monkeypatch):
    """896 x 4864 (Qwen2.5-0.5B down_proj: 56 row tiles, 38 k tiles in 4 slices of 9-10)
    and 3590 x 8192 (a partial last row tile; 2-4 slices); the split is forced where the
    default leaves these small activations to the unsplit kernels."""
    if m < 16:
        monkeypatch.setenv("LSQ_SPLITK", "4")
    _check(kind, 896, 4864, m, bias=True, seed=m)
    if m < 16:
        monkeypatch.setenv("LSQ_SPLITK", "2")
    rows = np.unique(np.concatenate([np.sort(np.random.default_rng(m).choice(3590, 256, replace=False)), [3589]]))
    _check(kind, 3590, 8192, m, bias=(m != 5), seed=m + 1, rows=rows)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("group", [128, 256, 1024, 8192])
def test_split_k_groups_and_dtypes(group, dtype):
    """1040 x 8192 at 6 tokens (65 row tiles, 3 slices of 21-22 k tiles: slices straddle
    group boundaries for groups of 2 and 8 k tiles), per-channel INT4 at group = K."""
    _check("int4", 1040, 8192, 6, group=group, dtype=dtype, bias=True, seed=group)


@pytest.mark.parametrize("sdt", [torch.float16, torch.float32])
def test_split_k_scale_dtypes(sdt):
    _check("int4", 1040, 8192, 7, scale_dtype=sdt, seed=13)


def test_split_k_workspace_contract():
    """Through the C ABI: the workspace size query, the split result bit-identical on a
    repeat, a too-small or NULL workspace giving the unsplit kernels' result (the plain
    entry point's, bit for bit), both within the contract of each other."""
    from localstrm_amd import _lib
    n, k, m = 3584, 18944, 8
    w, s, x = bench.make_int4(n, k, m, 128, seed=31)
    ql = QuantizedLinear.from_quantized(w.to(DEV), s.to(DEV), quant_type="int4", in_features=k,
                                        group_size=128)
    lib = _lib.load()
    nws = lib.lsq_linear_workspace_bytes(m, n, k)
    assert nws >= 4 * m * n * 2 and nws % 256 == 0
    assert lib.lsq_linear_workspace_bytes(m, 18944, 3584) == 0   # 1184 row tiles: no split
    assert lib.lsq_linear_workspace_bytes(20, n, k) == 0         # 17-23 tokens here: no split
    # 24-64 tokens on this long-K layer: the split-K GEMM's slices (up to 16 of [M][N] fp32)
    assert lib.lsq_linear_workspace_bytes(32, n, k) >= 2 * 32 * n * 4
    xd = x.to(DEV)
    tiled = ql.weight_tiled
    stream = _lib.stream_handle(DEV)

    def call(ws, nbytes):
        y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
        args = (xd.data_ptr(), k, None, tiled.data_ptr(), ql.scale.data_ptr(),
                _lib.dtype_code(ql.scale.dtype), 128, None, 0, y.data_ptr(), n,
                _lib.dtype_code(torch.bfloat16), m, n, k)
        if ws is False:
            rc = lib.lsq_w4_linear(*args, stream)
        else:
            rc = lib.lsq_w4_linear_ws(*args, _lib.ptr(ws), nbytes, stream)
        _lib.check(rc, "lsq_w4_linear(_ws)")
        return y.float().cpu().numpy()

    ws = torch.empty(nws, dtype=torch.uint8, device=DEV)
    ys1, ys2 = call(ws, nws), call(ws, nws)
    y_small = call(ws, nws - 256)
    y_null = call(None, 0)
    y_plain = call(False, 0)
    assert np.array_equal(ys1.view(np.uint32), ys2.view(np.uint32))
    assert np.array_equal(y_small.view(np.uint32), y_plain.view(np.uint32))
    assert np.array_equal(y_null.view(np.uint32), y_plain.view(np.uint32))
    err = qo.rel_err(ys1, y_plain.astype(np.float64))
    _say(f"  split vs unsplit: rel={err:.3e}")
    assert err <= REL_TOL
    with torch.no_grad():
        y_mod = ql(xd).float().cpu().numpy()   # the module passes a workspace
    assert np.array_equal(y_mod.view(np.uint32), ys1.view(np.uint32))
