"""GPU parity for the W8A8 path (Int8GEMMLinear, src/kernels/quantization.py:287-459).

The bar is bit-exactness: the int32 GEMM is exact and every other step is an IEEE
elementwise operation, so the kernels' x_q, scale_x and y must equal the oracle's
(oracle/quant_oracle.py act_quant_i8 / w8a8_linear) bit for bit. The scale's evaluation
order on the device is pinned against torch itself on the GPU. Every call goes through
the C ABI (directly, or via Int8GEMMLinear -> ctypes).
"""

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from localstrm_amd import CachedQuantizedLinear, Int8GEMMLinear, QuantizedLinear, _lib
from localstrm_amd import apply_optional_quantization
from oracle import quant_oracle as qo
from tests.synthetic import seeded_model

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _say(msg):
    print(msg, flush=True)


def _pad_k(k):
    return -(-k // 128) * 128


def _bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def _act_quant(x2, k, ldq=None):
    """liblsq act quant of x2 [M, >=K] (GPU, any row stride)."""
    m = x2.shape[0]
    ldq = ldq or _pad_k(k)
    xq = torch.full((m, ldq), 99, dtype=torch.int8, device=DEV)
    sx = torch.empty(m, dtype=torch.float32, device=DEV)
    rc = _lib.load().lsq_act_quant_i8(x2.data_ptr(), x2.stride(0), _lib.dtype_code(x2.dtype), m, k,
                                      xq.data_ptr(), ldq, sx.data_ptr(), _lib.stream_handle(DEV))
    _lib.check(rc, "lsq_act_quant_i8")
    torch.cuda.synchronize()
    return xq, sx


def _linear(x2, wq, sw, bias, monkeypatch=None, path=None):
    """liblsq W8A8 linear: x2 [M, K] (GPU), wq int8 [N, K], sw fp32 [N], bias or None."""
    m, k = x2.shape
    n = wq.shape[0]
    lib = _lib.load()
    wt = wq.t().contiguous().to(DEV)
    tiled = torch.empty(lib.lsq_w8a8_tiled_bytes(n, k), dtype=torch.int8, device=DEV)
    _lib.check(lib.lsq_w8a8_retile(wt.data_ptr(), tiled.data_ptr(), n, k, _lib.stream_handle(DEV)), "retile")
    y = torch.empty((m, n), dtype=x2.dtype, device=DEV)
    xq = torch.empty((m, _pad_k(k)), dtype=torch.int8, device=DEV)
    sx = torch.empty(m, dtype=torch.float32, device=DEV)
    swd = sw.to(DEV).contiguous()
    b = bias.to(DEV).contiguous() if bias is not None else None
    if path is not None:
        monkeypatch.setenv("LSQ_W8A8_PATH", path)
    rc = lib.lsq_w8a8_linear(x2.data_ptr(), x2.stride(0), tiled.data_ptr(), swd.data_ptr(),
                             _lib.dtype_code(swd.dtype), _lib.ptr(b),
                             _lib.dtype_code(b.dtype) if b is not None else 0, y.data_ptr(), n,
                             _lib.dtype_code(x2.dtype), m, n, k, xq.data_ptr(), sx.data_ptr(),
                             _lib.stream_handle(DEV))
    if path is not None:
        monkeypatch.delenv("LSQ_W8A8_PATH")
    _lib.check(rc, "lsq_w8a8_linear")
    torch.cuda.synchronize()
    return y, xq, sx


# ----------------------------------------------------------------------------- scale


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_act_scale_matches_torch_on_the_device(dt):
    """The oracle's scale (product with fp32 1/127, then round_T, then the clamp) equals
    torch's own `max|x| / 127.0` clamp on the GPU, over every positive finite bf16 / fp16
    value and 300k random fp32 magnitudes; liblsq's scale equals both."""
    _say(f"act scale {dt}")
    if dt == "bf16":
        bits = np.arange(1, 0x7F80, dtype=np.uint32) << 16
        vals = bits.view(np.float32)
    elif dt == "f16":
        vals = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    else:
        rng = np.random.default_rng(0)
        vals = (rng.uniform(0.5, 1.0, 300000) * 2.0 ** rng.integers(-40, 40, 300000)).astype(np.float32)
    sign = np.where(np.arange(vals.size) % 2 == 0, 1.0, -1.0).astype(np.float32)
    x = torch.from_numpy((vals * sign).reshape(-1, 1)).to(TDT[dt]).to(DEV)
    x2 = torch.cat([x, x * 0.5], dim=1).contiguous()  # max|row| is the first column
    dev = torch.clamp(torch.max(torch.abs(x2), dim=-1, keepdim=True)[0] / 127.0, min=1e-8).float()
    ref = qo.act_scale_i8(x2.float().cpu().numpy(), dt)
    _, sx = _act_quant(x2, 2)
    assert np.array_equal(_bits(dev.cpu().numpy()), _bits(ref))
    assert np.array_equal(_bits(sx.cpu().numpy().reshape(-1, 1)), _bits(ref))
    if dt == "f32":  # the sample tells the two division orders apart
        true_div = (np.abs(x2.float().cpu().numpy()).max(axis=1) / np.float32(127.0)).astype(np.float32)
        assert np.count_nonzero(true_div != ref[:, 0]) > 1000


# ----------------------------------------------------------------------------- x_q


ACT_CASES = [(1, 896, 896), (7, 100, 100), (64, 3584, 3584), (300, 1024, 1024), (5, 8, 8),
             (9, 72, 200), (3, 9000, 9000), (520, 8300, 8300)]  # long rows: 1024 / 256 threads


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("m,k,ldx", ACT_CASES)
def test_act_quant_bit_exact(dt, m, k, ldx):
    _say(f"act quant {dt} M={m} K={k} ldx={ldx}")
    g = torch.Generator().manual_seed(m * 7 + k)
    x = (torch.randn(m, ldx, generator=g) * torch.rand(m, 1, generator=g) * 8).to(TDT[dt])
    if m >= 5:
        x[1] = 0                       # zero row
        x[2, : min(k, 4)] = 3e-7 if dt != "f16" else 6e-8  # tiny row
        x[2, min(k, 4):] = 0
        x[3, 0] = 250.0                # one large value
    xd = x.to(DEV)
    x2 = xd[:, :k]
    xq, sx = _act_quant(x2, k)
    ref_q, ref_s = qo.act_quant_i8(x[:, :k].float().numpy(), dt)
    xq = xq.cpu().numpy()
    assert np.array_equal(_bits(sx.cpu().numpy()), _bits(ref_s[:, 0]))
    assert np.array_equal(xq[:, :k], ref_q)
    assert (xq[:, k:_pad_k(k)] == 0).all()  # padding columns


def _near_tie_rows(dt, m, k, seed):
    """Rows whose values sit on or next to half-integer multiples of the row's scale
    (the cases where rint(v * rcp(s)) and rint(v / s) could part ways)."""
    rng = np.random.default_rng(seed)
    rows = []
    for i in range(m):
        mx = np.float32(rng.uniform(0.05, 300.0))
        s = qo.act_scale_i8(np.array([[mx]], np.float32), dt)[0, 0]
        kk = rng.integers(-127, 127, size=k).astype(np.float32)
        d = rng.choice(np.array([0.0, 2.0 ** -12, -2.0 ** -12, 2.0 ** -20, -2.0 ** -20, 0.25], np.float32), size=k)
        v = qo.round_to((kk + np.float32(0.5) + d) * s, dt)
        v[0] = qo.round_to(np.array([mx], np.float32), dt)[0]
        v = np.where(np.abs(v) > np.abs(v[0]), np.float32(0.0), v)  # keep v[0] the row max
        rows.append(v)
    return np.stack(rows).astype(np.float32)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_act_quant_near_ties_bit_exact(dt):
    _say(f"act quant near ties {dt}")
    x32 = _near_tie_rows(dt, 64, 512, 1)
    xq, sx = _act_quant(torch.from_numpy(x32).to(TDT[dt]).to(DEV), 512)
    ref_q, ref_s = qo.act_quant_i8(x32, dt)
    assert np.array_equal(_bits(sx.cpu().numpy()), _bits(ref_s[:, 0]))
    assert np.array_equal(xq.cpu().numpy()[:, :512], ref_q)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("m", [1, 4, 16])
def test_w8a8_fused_quant_near_ties_bit_exact(monkeypatch, dt, m):
    # the decode kernel's own quantization on the same near-tie rows
    _say(f"w8a8 fused near ties {dt} M={m}")
    k, n = 512, 272
    x32 = _near_tie_rows(dt, m, k, 2 + m)
    g = torch.Generator().manual_seed(m)
    wq = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    sw = torch.rand(n, generator=g) * 0.02 + 1e-3
    y, _, _ = _linear(torch.from_numpy(x32).to(TDT[dt]).to(DEV), wq, sw, None, monkeypatch, "fused")
    ref = qo.w8a8_linear(x32, wq.numpy(), sw.numpy(), None, dt)
    assert np.array_equal(_bits(y.float().cpu().numpy()), _bits(ref))


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("m,n,k", [(8, 272, 896), (16, 1000, 3584), (64, 272, 896)])
def test_w8a8_forced_fused_decode_bit_exact(monkeypatch, dt, m, n, k):
    # the in-kernel quantization on inputs the heuristic would send to the separate kernel
    _say(f"w8a8 fused-forced {dt} M={m} N={n} K={k}")
    x, wq, sw, bias = _lin_inputs(dt, m, n, k)
    y, _, _ = _linear(x.to(DEV), wq, sw, bias, monkeypatch, "fused")
    ref = qo.w8a8_linear(x.float().numpy(), wq.numpy(), sw.numpy(),
                         None if bias is None else bias.float().numpy(), dt)
    assert np.array_equal(_bits(y.float().cpu().numpy()), _bits(ref))


# ----------------------------------------------------------------------------- linear


LIN_CASES = [
    # (M, N, K): decode-shaped (M <= 64) then GEMM-shaped
    (1, 272, 896), (5, 272, 896), (16, 1000, 896), (33, 272, 896), (64, 272, 896),
    (1, 128, 64), (17, 136, 200), (1, 4864, 896),
    (65, 520, 1024), (300, 264, 256), (257, 136, 64), (513, 1024, 384),
]


def _lin_inputs(dt, m, n, k):
    g = torch.Generator().manual_seed(m + n + k)
    x = (torch.randn(m, k, generator=g) * 2).to(TDT[dt])
    if m >= 3:
        x[1] = 0                                           # zero row: scale = clamp bound
        x[2] = 6e-8 if dt == "f16" else 3e-7               # fp16: scale rounds to 0
    wq = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    sw = torch.rand(n, generator=g) * 0.02 + 1e-3
    bias = (torch.randn(n, generator=g)).to(TDT[dt]) if (m + n) % 2 else None
    return x, wq, sw, bias


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("m,n,k", LIN_CASES)
def test_w8a8_linear_bit_exact(dt, m, n, k):
    # decode shapes with small x quantize inside the GEMV kernel (one launch)
    _say(f"w8a8 {dt} M={m} N={n} K={k}")
    x, wq, sw, bias = _lin_inputs(dt, m, n, k)
    y, _, _ = _linear(x.to(DEV), wq, sw, bias)
    ref = qo.w8a8_linear(x.float().numpy(), wq.numpy(), sw.numpy(),
                         None if bias is None else bias.float().numpy(), dt)
    got = y.float().cpu().numpy()
    mism = np.count_nonzero(_bits(got) != _bits(ref))
    assert mism == 0, f"{mism} of {got.size} outputs differ"


@pytest.mark.parametrize("m", [1, 8, 17, 33, 64])
def test_w8a8_linear_bit_exact_large_n(m):
    # N = 18944 (1184 row tiles) at K = 1024: the 6 x 2 workgroups of the decode kernel,
    # with the 17..64-token blocks
    n, k = 18944, 1024
    _say(f"w8a8 large N bf16 M={m} N={n} K={k}")
    x, wq, sw, bias = _lin_inputs("bf16", m, n, k)
    y, _, _ = _linear(x.to(DEV), wq, sw, bias)
    ref = qo.w8a8_linear(x.float().numpy(), wq.numpy(), sw.numpy(),
                         None if bias is None else bias.float().numpy(), "bf16")
    got = y.float().cpu().numpy()
    mism = np.count_nonzero(_bits(got) != _bits(ref))
    assert mism == 0, f"{mism} of {got.size} outputs differ"


@pytest.mark.parametrize("m,n,k", [(1, 3584, 18944), (2, 3584, 18944), (3, 3584, 18944),
                                   (8, 3584, 18944), (13, 3584, 18944),
                                   (16, 4096, 14336), (64, 4096, 14336)])
def test_w8a8_large_k_token_blocks(m, n, k):
    # 1-2 long rows: quantized inside the decode kernel; x_q of 8+ tokens at K = 18944
    # exceeds LDS: blocks of 4 (2 passes at M = 8, 4 at M = 13 with a ragged last
    # block), of 8 at K = 14336 (16 tokens); 64 tokens there: the GEMM's 64 x 128 tiles
    # (no workspace here: the unsplit GEMM)
    _say(f"w8a8 large K blocks bf16 M={m} N={n} K={k}")
    x, wq, sw, bias = _lin_inputs("bf16", m, n, k)
    y, _, _ = _linear(x.to(DEV), wq, sw, bias)
    ref = qo.w8a8_linear(x.float().numpy(), wq.numpy(), sw.numpy(),
                         None if bias is None else bias.float().numpy(), "bf16")
    got = y.float().cpu().numpy()
    mism = np.count_nonzero(_bits(got) != _bits(ref))
    assert mism == 0, f"{mism} of {got.size} outputs differ"


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("m", [1, 2])
def test_w8a8_long_rows_quantized_in_kernel_dtypes(dt, m):
    # one or two rows of 18944 activations (the decode kernel quantizes them itself) in
    # every activation type: fp32 at M=1 is 4736 16-byte chunks
    _say(f"w8a8 long rows {dt} M={m} N=3584 K=18944")
    x, wq, sw, bias = _lin_inputs(dt, m, 3584, 18944)
    y, _, _ = _linear(x.to(DEV), wq, sw, bias)
    ref = qo.w8a8_linear(x.float().numpy(), wq.numpy(), sw.numpy(),
                         None if bias is None else bias.float().numpy(), dt)
    got = y.float().cpu().numpy()
    mism = np.count_nonzero(_bits(got) != _bits(ref))
    assert mism == 0, f"{mism} of {got.size} outputs differ"


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("m,n,k", [(1, 272, 896), (5, 1000, 896), (16, 272, 2048), (64, 272, 896)])
def test_w8a8_unfused_decode_bit_exact(monkeypatch, dt, m, n, k):
    # the same shapes through act_quant_kernel + the decode kernel on x_q
    _say(f"w8a8 unfused {dt} M={m} N={n} K={k}")
    x, wq, sw, bias = _lin_inputs(dt, m, n, k)
    y, xq, sx = _linear(x.to(DEV), wq, sw, bias, monkeypatch, "unfused")
    ref_q, ref_s = qo.act_quant_i8(x.float().numpy(), dt)
    assert np.array_equal(xq.cpu().numpy()[:, :k], ref_q)
    assert np.array_equal(_bits(sx.cpu().numpy()), _bits(ref_s[:, 0]))
    ref = qo.w8a8_linear(x.float().numpy(), wq.numpy(), sw.numpy(),
                         None if bias is None else bias.float().numpy(), dt)
    assert np.array_equal(_bits(y.float().cpu().numpy()), _bits(ref))


@pytest.mark.parametrize("m,n,k", [(1, 272, 896), (33, 272, 896), (64, 520, 1024)])
def test_w8a8_gemm_kernel_on_decode_shapes(monkeypatch, m, n, k):
    # the prefill kernel must give the same bits as the decode kernel (and the oracle)
    _say(f"w8a8 gemm-forced M={m} N={n} K={k}")
    g = torch.Generator().manual_seed(3 * m + k)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(DEV)
    wq = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    sw = torch.rand(n, generator=g) * 0.02 + 1e-3
    bias = torch.randn(n, generator=g).to(torch.bfloat16)
    y_dec, _, _ = _linear(x, wq, sw, bias)
    y_gemm, _, _ = _linear(x, wq, sw, bias, monkeypatch, "gemm")
    assert torch.equal(y_dec.view(torch.int16), y_gemm.view(torch.int16))


@pytest.mark.parametrize("variant", ["1", "2", "3", "0"])
@pytest.mark.parametrize("m,n,k", [(65, 520, 1024), (257, 136, 64), (300, 264, 256), (1024, 2048, 640),
                                   (40, 1000, 1920)])
def test_w8a8_gemm_pipeline_depths(monkeypatch, variant, m, n, k):
    # The GEMM's tile, k step and LDS stages (LSQ_W8A8_GEMM: 1 = 256 x 256 tiles, 128
    # columns, 2 stages; 2 = 256 x 256, 64 columns, 3 stages; 3 = 64 x 128 tiles, 128
    # columns, 6 stages; 0 = 256 x 256, 64 columns, 4 stages), bit-exact against the
    # oracle: the XCD-blocked tile order (1024 x 2048) and the plain one, K of 1 to 15
    # k tiles (fewer steps than the pipeline holds at K = 64 and 256), partial tiles in M
    # and N.
    _say(f"w8a8 gemm pipeline {variant} M={m} N={n} K={k}")
    monkeypatch.setenv("LSQ_W8A8_GEMM", variant)
    x, wq, sw, bias = _lin_inputs("bf16", m, n, k)
    y, _, _ = _linear(x.to(DEV), wq, sw, bias, monkeypatch, "gemm")
    ref = qo.w8a8_linear(x.float().numpy(), wq.numpy(), sw.numpy(),
                         None if bias is None else bias.float().numpy(), "bf16")
    mism = np.count_nonzero(_bits(y.float().cpu().numpy()) != _bits(ref))
    assert mism == 0, f"{mism} of {y.numel()} outputs differ"


def _linear_ws(x2, wq, sw, bias, nws=None, misalign=False):
    """lsq_w8a8_linear_ws with lsq_w8a8_workspace_bytes of workspace (or nws bytes)."""
    m, k = x2.shape
    n = wq.shape[0]
    lib = _lib.load()
    wt = wq.t().contiguous().to(DEV)
    tiled = torch.empty(lib.lsq_w8a8_tiled_bytes(n, k), dtype=torch.int8, device=DEV)
    _lib.check(lib.lsq_w8a8_retile(wt.data_ptr(), tiled.data_ptr(), n, k, _lib.stream_handle(DEV)), "retile")
    y = torch.empty((m, n), dtype=x2.dtype, device=DEV)
    xq = torch.empty((m, _pad_k(k)), dtype=torch.int8, device=DEV)
    sx = torch.empty(m, dtype=torch.float32, device=DEV)
    swd = sw.to(DEV).contiguous()
    b = bias.to(DEV).contiguous() if bias is not None else None
    nws = lib.lsq_w8a8_workspace_bytes(m, n, k) if nws is None else nws
    ws = torch.full((nws + 16,), 0x7F, dtype=torch.uint8, device=DEV)  # stale contents
    wp = ws.data_ptr() + (4 if misalign else 0)
    rc = lib.lsq_w8a8_linear_ws(x2.data_ptr(), x2.stride(0), tiled.data_ptr(), swd.data_ptr(),
                                _lib.dtype_code(swd.dtype), _lib.ptr(b),
                                _lib.dtype_code(b.dtype) if b is not None else 0, y.data_ptr(), n,
                                _lib.dtype_code(x2.dtype), m, n, k, xq.data_ptr(), sx.data_ptr(),
                                wp if nws > 0 else None, nws, _lib.stream_handle(DEV))
    torch.cuda.synchronize()
    return rc, y


@pytest.mark.parametrize("m,n,k", [(64, 512, 18944), (33, 640, 4864), (16, 384, 18944), (8, 3584, 18944),
                                   (5, 256, 10240), (100, 520, 8192), (64, 3584, 18944),
                                   (256, 520, 8192), (600, 1000, 8192), (1024, 3584, 18944),
                                   (24, 1002, 8192)])
def test_w8a8_split_k_bit_exact(m, n, k):
    # The split-K GEMM (int32 slices in the workspace, exact merge, the GEMM's rescale):
    # bit-exact against the oracle and bit-identical to the workspace-free entry point.
    # Below 17 tokens the workspace also moves long rows from the decode kernel's token
    # blocks to the split GEMM (16 and 8 tokens at K = 18944); 5 x 10240 fits the decode
    # kernel and leaves the workspace unused. Past 192 tokens the 256 x 256 tiles split
    # (256 x 520 x 8192: 3 tiles, 16 slices; 1024 x 3584 x 18944: 56 tiles, 4 slices);
    # N = 1002: a partial last tile of output columns.
    _say(f"w8a8 split-K M={m} N={n} K={k}")
    x, wq, sw, bias = _lin_inputs("bf16", m, n, k)
    xd = x.to(DEV)
    nws = _lib.load().lsq_w8a8_workspace_bytes(m, n, k)
    assert nws > 0
    rc, y = _linear_ws(xd, wq, sw, bias)
    _lib.check(rc, "lsq_w8a8_linear_ws")
    plain, _, _ = _linear(xd, wq, sw, bias)
    ref = qo.w8a8_linear(x.float().numpy(), wq.numpy(), sw.numpy(),
                         None if bias is None else bias.float().numpy(), "bf16")
    got = y.float().cpu().numpy()
    mism = np.count_nonzero(_bits(got) != _bits(ref))
    assert mism == 0, f"{mism} of {got.size} outputs differ from the oracle"
    assert torch.equal(y.view(torch.int16), plain.view(torch.int16))


@pytest.mark.parametrize("forced", ["2", "7", "16"])
@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_w8a8_split_k_forced_slices_and_dtypes(monkeypatch, forced, dt):
    # LSQ_W8A8_SPLITK=n forces n slices (ragged: 32 k tiles over 7); every activation type
    m, n, k = 40, 1000, 4096
    monkeypatch.setenv("LSQ_W8A8_SPLITK", forced)
    _say(f"w8a8 split-K forced={forced} {dt} M={m} N={n} K={k}")
    x, wq, sw, bias = _lin_inputs(dt, m, n, k)
    nws = _lib.load().lsq_w8a8_workspace_bytes(m, n, k)
    assert nws >= int(forced) * m * n * 4
    rc, y = _linear_ws(x.to(DEV), wq, sw, bias)
    _lib.check(rc, "lsq_w8a8_linear_ws")
    ref = qo.w8a8_linear(x.float().numpy(), wq.numpy(), sw.numpy(),
                         None if bias is None else bias.float().numpy(), dt)
    assert np.array_equal(_bits(y.float().cpu().numpy()), _bits(ref))


def test_w8a8_workspace_contract(monkeypatch):
    lib = _lib.load()
    assert lib.lsq_w8a8_workspace_bytes(64, 3584, 18944) == 9 * 64 * 3584 * 4  # 28 tiles: 9 slices
    assert lib.lsq_w8a8_workspace_bytes(64, 18944, 3584) == 0   # 148 tiles: no split
    assert lib.lsq_w8a8_workspace_bytes(256, 3584, 18944) == 16 * 256 * 3584 * 4  # 14 large tiles
    assert lib.lsq_w8a8_workspace_bytes(2048, 14336, 4096) == 0  # 448 large tiles: no split
    assert lib.lsq_w8a8_workspace_bytes(64, 3584, 1024) == 0    # 8 k tiles: too short
    assert lib.lsq_w8a8_workspace_bytes(0, 3584, 18944) == 0
    monkeypatch.setenv("LSQ_W8A8_SPLITK", "0")
    assert lib.lsq_w8a8_workspace_bytes(64, 3584, 18944) == 0
    monkeypatch.delenv("LSQ_W8A8_SPLITK")
    # a misaligned workspace is refused; a short one runs the unsplit GEMM, same bits
    m, n, k = 33, 640, 4864
    x, wq, sw, bias = _lin_inputs("bf16", m, n, k)
    xd = x.to(DEV)
    rc, _ = _linear_ws(xd, wq, sw, bias, misalign=True)
    assert rc == -6  # LSQ_E_ALIGN
    rc, y_short = _linear_ws(xd, wq, sw, bias, nws=1024)
    _lib.check(rc, "lsq_w8a8_linear_ws")
    rc, y_split = _linear_ws(xd, wq, sw, bias)
    _lib.check(rc, "lsq_w8a8_linear_ws")
    assert torch.equal(y_short.view(torch.int16), y_split.view(torch.int16))


def test_w8a8_module_split_k_down_projection():
    # Int8GEMMLinear on a 3584 x 18944 down projection at 32 tokens: the module takes the
    # workspace from torch's allocator; two calls in a row give the same bits
    n, k, m = 3584, 18944, 32
    g = torch.Generator().manual_seed(5)
    lin = nn.Linear(k, n, bias=True)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(n, k, generator=g) * 0.02)
        lin.bias.copy_(torch.randn(n, generator=g) * 0.1)
    q = Int8GEMMLinear.from_float(lin.to(torch.bfloat16)).to(DEV)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        y1 = q(x)
        y2 = q(x)
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))
    wq = q.weight_q_t.t().contiguous().cpu()
    ref = qo.w8a8_linear(x.float().cpu().numpy(), wq.numpy(), q.scale_w_t.reshape(-1).float().cpu().numpy(),
                         q.bias.detach().float().cpu().numpy(), "bf16")
    assert np.array_equal(_bits(y1.float().cpu().numpy()), _bits(ref))


@pytest.mark.parametrize("m,n,k", [(64, 256, 4096), (40, 128, 10240)])
def test_w8a8_large_k_token_blocks_and_gemm(m, n, k):
    # 64 tokens x K = 4096 and 40 x 10240 do not fit the decode kernel's LDS: without a
    # workspace the GEMM's 64 x 128 tiles (past 32 tokens, or 16 on layers of 16+ tiles)
    _say(f"w8a8 large K M={m} N={n} K={k}")
    g = torch.Generator().manual_seed(k)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    wq = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    sw = torch.rand(n, generator=g) * 0.02 + 1e-3
    y, _, _ = _linear(x.to(DEV), wq, sw, None)
    ref = qo.w8a8_linear(x.float().numpy(), wq.numpy(), sw.numpy(), None, "bf16")
    assert np.array_equal(_bits(y.float().cpu().numpy()), _bits(ref))


def test_w8a8_strided_input_and_scale_dtypes():
    _say("w8a8 strided x, fp16 scale, fp32 bias")
    g = torch.Generator().manual_seed(9)
    m, n, k = 24, 200, 384
    big = torch.randn(m, k + 64, generator=g).to(torch.float16)
    x = big.to(DEV)[:, 32:32 + k]
    wq = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    sw = (torch.rand(n, generator=g) * 0.02 + 1e-3).to(torch.float16)
    bias = torch.randn(n, generator=g)
    y, _, _ = _linear(x, wq, sw, bias)
    ref = qo.w8a8_linear(big[:, 32:32 + k].float().numpy(), wq.numpy(), sw.float().numpy(),
                         bias.numpy(), "f16")
    assert np.array_equal(_bits(y.float().cpu().numpy()), _bits(ref))


def test_w8a8_retile_round_trip_and_shared_layout():
    lib = _lib.load()
    s = _lib.stream_handle(DEV)
    for n, k in ((50, 200), (272, 896), (16, 128)):
        wt = torch.randint(-128, 128, (k, n), dtype=torch.int8, device=DEV)
        tiled = torch.empty(lib.lsq_w8a8_tiled_bytes(n, k), dtype=torch.int8, device=DEV)
        _lib.check(lib.lsq_w8a8_retile(wt.data_ptr(), tiled.data_ptr(), n, k, s), "retile")
        back = torch.empty_like(wt)
        _lib.check(lib.lsq_w8a8_untile(tiled.data_ptr(), back.data_ptr(), n, k, s), "untile")
        torch.cuda.synchronize()
        assert torch.equal(back, wt)
        if k % 128 == 0:  # same bytes as the weight-only INT8 tiled layout of W = wt^T
            t8 = torch.empty(lib.lsq_w8_tiled_bytes(n, k), dtype=torch.int8, device=DEV)
            _lib.check(lib.lsq_w8_retile(wt.t().contiguous().data_ptr(), t8.data_ptr(), n, k, s), "w8")
            torch.cuda.synchronize()
            assert torch.equal(t8, tiled)


# ----------------------------------------------------------------------------- module


def test_int8_gemm_linear_module_reference_shapes():
    # tests/test_hybrid_int8.py:256-280 of the reference: fp16, M % 32 != 0 shapes
    _say("Int8GEMMLinear module shapes")
    torch.manual_seed(0)
    lin = nn.Linear(64, 128, bias=True, device=DEV, dtype=torch.float16)
    layer = Int8GEMMLinear.from_float(lin, dtype=torch.float16).to(DEV)
    wq = layer.weight_q_t.t().cpu().numpy()
    sw = layer.scale_w_t.reshape(-1).cpu().numpy()
    b = layer.bias.detach().float().cpu().numpy()
    for shape in [(1, 1, 64), (4, 1, 64), (1, 37, 64), (2, 32, 64)]:
        x = torch.randn(shape, device=DEV, dtype=torch.float16)
        with torch.no_grad():
            ref_out = lin(x)
            out = layer(x)
        assert out.shape == (*shape[:-1], 128) and out.dtype == torch.float16
        cos = F.cosine_similarity(ref_out.float().flatten(), out.float().flatten(), dim=0).item()
        assert cos > 0.99, (shape, cos)
        exact = qo.w8a8_linear(x.reshape(-1, 64).float().cpu().numpy(), wq, sw, b, "f16")
        assert np.array_equal(_bits(out.reshape(-1, 128).float().cpu().numpy()), _bits(exact))
    with pytest.raises(ValueError, match="does not match layer in_features"):
        layer(torch.randn(2, 63, device=DEV, dtype=torch.float16))


def test_int8_gemm_linear_fallbacks(monkeypatch):
    # kill switch (test_hybrid_int8.py:285-296) and K % 8 != 0: the weight-only INT8
    # kernels, against the oracle's dequantized linear
    _say("Int8GEMMLinear fallbacks")
    torch.manual_seed(1)
    for k, n in ((64, 128), (63, 127)):
        lin = nn.Linear(k, n, bias=True, device=DEV)
        layer = Int8GEMMLinear.from_float(lin, dtype=torch.bfloat16)
        x = torch.randn(3, 5, k, device=DEV, dtype=torch.bfloat16)
        if k % 8 == 0:
            monkeypatch.setenv("MINIVLLM_DISABLE_INT8_GEMM", "1")
        with torch.no_grad():
            y = layer(x)
        monkeypatch.delenv("MINIVLLM_DISABLE_INT8_GEMM", raising=False)
        assert layer._warned_fallback and y.shape == (3, 5, n)
        w = qo.dequant_int8(layer.weight_q_t.t().cpu().numpy(), layer.scale_w_t.reshape(-1, 1).cpu().numpy(), "bf16")
        ref = qo.linear(x.reshape(-1, k).float().cpu().numpy(), w, layer.bias.detach().float().cpu().numpy(), "bf16")
        assert qo.rel_err(y.reshape(-1, n).float().cpu().numpy(), ref) <= 1e-2


def test_hybrid_int8_model_forward():
    # the whole synthetic decoder in hybrid_int8 on the GPU against the float model
    _say("hybrid_int8 model forward")
    ref_model = seeded_model().to(DEV).half()
    model = seeded_model()
    apply_optional_quantization(model, quant_type="hybrid_int8")
    model = model.to(DEV).half()
    assert isinstance(model.model.layers[0].mlp.up_proj, Int8GEMMLinear)
    assert isinstance(model.model.layers[0].self_attn.k_proj, CachedQuantizedLinear)
    x = torch.randn(2, 9, 64, device=DEV, dtype=torch.float16)
    with torch.no_grad():
        ref = ref_model(x).float()
        out = model(x).float()
    cos = F.cosine_similarity(ref.flatten(), out.flatten(), dim=0).item()
    _say(f"  cos={cos:.5f}")
    assert cos > 0.99
