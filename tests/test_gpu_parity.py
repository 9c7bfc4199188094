"""GPU parity: the HIP kernels in liblsq.so against the pinned CPU oracle.

Bars (from the reference's contract, src/kernels/quantization.py:104-141):
  * unpacked INT4 nibbles and dequantized weights: bit-exact (torch.equal);
  * layer outputs: rel = max|y - y_ref| / max|y_ref| <= 1e-2 (the reference's own
    convention, tests/test_int8_multi_step.py:184-188), where y_ref is the float64
    oracle on identical inputs. The kernels accumulate in fp32, so the observed error is
    far below the bar; tests also report it.
Every call goes through localstrm_amd.QuantizedLinear -> ctypes -> the C ABI.
"""

import os

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import bench
from localstrm_amd import QuantizedLinear, _lib
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
REL_TOL = 1e-2
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz")
GOLDEN_CASES = ["int8_pc", "int4_pc_oddk", "int4_g16", "int4_g128", "int8_k256", "int4_pc_k128"]


def _say(msg):
    print(msg, flush=True)


def _layer(kind, w, s, k=None, group=None, bias=None):
    if kind == "int8":
        return QuantizedLinear.from_quantized(w.to(DEV), s.to(DEV), bias=None if bias is None else bias.to(DEV),
                                              quant_type="int8")
    return QuantizedLinear.from_quantized(w.to(DEV), s.to(DEV), bias=None if bias is None else bias.to(DEV),
                                          quant_type="int4", in_features=k, group_size=group)


def _oracle_deq(kind, w, s, k, group, dt):
    if kind == "int8":
        return qo.dequant_int8(w.numpy(), s.float().numpy(), dt)
    return qo.dequant_int4(w.numpy(), s.float().numpy(), k, group, dt)


def _dt_name(dtype):
    return {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[dtype]


# ----------------------------------------------------------------------------- golden


@pytest.mark.parametrize("name", GOLDEN_CASES)
@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_golden_dequant_bit_exact_and_output(name, dt):
    _say(f"golden {name} {dt}")
    z = np.load(GOLDEN, allow_pickle=False)
    n, k, g = (int(v) for v in z[f"{name}/meta"])
    g = None if g < 0 else g
    q = torch.from_numpy(z[f"{name}/q"])
    s = torch.from_numpy(z[f"{name}/scale"])
    bias = torch.from_numpy(z[f"{name}/bias"])
    if name.startswith("int8"):
        ql = _layer("int8", q, s, bias=bias)
    else:
        if g is not None:
            s = s.to(torch.bfloat16)  # golden group scales are bf16 values
        ql = _layer("int4", torch.from_numpy(qo.pack_int4(z[f"{name}/q"])), s, k, g, bias)
    w = ql.dequantize(TDT[dt]).float().cpu().numpy()
    assert np.array_equal(w.view(np.uint32), z[f"{name}/w_{dt}"].view(np.uint32))
    x = torch.from_numpy(z[f"{name}/x_{dt}"]).to(TDT[dt]).to(DEV)
    with torch.no_grad():
        y = ql(x).float().cpu().numpy()
    err = qo.rel_err(y, z[f"{name}/y_{dt}_exact"])
    _say(f"  rel_err={err:.3e}")
    assert err <= REL_TOL
    # fp32 accumulation of the exact T-valued products: far tighter than the contract
    assert err <= {"f32": 1e-5, "f16": 2e-3, "bf16": 1e-2}[dt]


# ----------------------------------------------------------------------------- unpack / dequant


@pytest.mark.parametrize("k", [32, 33, 128, 1536])
def test_int4_unpack_and_dequant_bit_exact(k):
    """GPU form of the reference regression tests/test_quantized_loader.py:438-463."""
    _say(f"unpack k={k}")
    torch.manual_seed(k)
    ql = QuantizedLinear.from_float(nn.Linear(k, 64, bias=False), "int4").to(DEV)
    packed = ql.weight_packed.cpu()
    q_ref = qo.unpack_int4(packed.numpy(), k)
    assert torch.equal(ql.unpack_int4().cpu(), torch.from_numpy(q_ref))
    w_ref = torch.from_numpy(q_ref).float() * ql.scale.cpu()
    assert torch.equal(ql.dequantize().cpu(), w_ref)
    w16 = ql.dequantize(torch.float16)
    assert w16.dtype == torch.float16
    assert (w16.float().cpu() - w_ref).abs().max().item() <= 1e-3


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_full_size_dequant_bit_exact(dt):
    """The Qwen2.5-7B MLP shapes: INT8 18944x3584 per-channel and INT4 group-128 18944x3584."""
    _say(f"full-size dequant {dt}")
    w, s, _ = bench.make_int8(18944, 3584, 1)
    ql = _layer("int8", w, s)
    got = ql.dequantize(TDT[dt]).float().cpu().numpy()
    assert np.array_equal(got.view(np.uint32), _oracle_deq("int8", w, s, 3584, None, dt).view(np.uint32))
    p, s4, _ = bench.make_int4(18944, 3584, 1)
    ql4 = _layer("int4", p, s4, 3584, 128)
    got4 = ql4.dequantize(TDT[dt]).float().cpu().numpy()
    assert np.array_equal(got4.view(np.uint32), _oracle_deq("int4", p, s4, 3584, 128, dt).view(np.uint32))


def test_retile_w8_round_trip():
    _say("retile w8 round trip")
    lib = _lib.load()
    for n, k in [(16, 128), (17, 256), (18944, 3584), (100, 896)]:
        w, _, _ = bench.make_int8(n, k, 1, seed=n)
        w = w.to(DEV)
        tiled = torch.empty(lib.lsq_w8_tiled_bytes(n, k), dtype=torch.int8, device=DEV)
        back = torch.zeros_like(w)
        st = _lib.stream_handle(DEV)
        _lib.check(lib.lsq_w8_retile(w.data_ptr(), tiled.data_ptr(), n, k, st), "retile")
        _lib.check(lib.lsq_w8_untile(tiled.data_ptr(), back.data_ptr(), n, k, st), "untile")
        assert torch.equal(back, w)
        # layout: byte j*1024 + 16*l + b of tile (rt, kt) = W[16 rt + l%16, 128 kt + 32 (l//16) + 16 j + b]
        t = tiled.view(-1, k // 128, 2, 64, 16).cpu()
        wc = w.cpu()
        for rt, kt, j, l, b in [(0, 0, 0, 0, 0), (0, 0, 1, 63, 15), ((n - 1) // 16, k // 128 - 1, 1, 17, 3)]:
            r = 16 * rt + l % 16
            if r < n:
                assert t[rt, kt, j, l, b] == wc[r, 128 * kt + 32 * (l // 16) + 16 * j + b]
        if n % 16:
            lanes = torch.arange(64) % 16
            assert int(t[-1][:, :, lanes >= n % 16].abs().sum()) == 0


def test_retile_round_trip():
    _say("retile round trip")
    lib = _lib.load()
    for n, k in [(16, 128), (17, 256), (18944, 3584), (128, 896)]:
        p, _, _ = bench.make_int4(n, k, 1, seed=n)
        p = p.to(DEV)
        nbytes = lib.lsq_w4_tiled_bytes(n, k)
        tiled = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        back = torch.zeros_like(p)
        st = _lib.stream_handle(DEV)
        _lib.check(lib.lsq_w4_retile(p.data_ptr(), tiled.data_ptr(), n, k, st), "retile")
        _lib.check(lib.lsq_w4_untile(tiled.data_ptr(), back.data_ptr(), n, k, st), "untile")
        assert torch.equal(back, p)
        # padded rows of the last tile are zero
        if n % 16:
            t = tiled.view(-1, k // 128, 64, 16)[-1]
            lanes = torch.arange(64, device=DEV) % 16
            assert int(t[:, lanes >= n % 16].abs().sum()) == 0


# ----------------------------------------------------------------------------- layer outputs


def _check_layer(kind, n, k, m, group=128, dtype=torch.bfloat16, bias=False, seed=0, rows=None):
    if kind == "int8":
        w, s, x = bench.make_int8(n, k, m, x_dtype=dtype, seed=seed)
    else:
        w, s, x = bench.make_int4(n, k, m, group, x_dtype=dtype, seed=seed)
    b = torch.randn(n, generator=torch.Generator().manual_seed(seed + 1)) if bias else None
    ql = _layer(kind, w, s, k, group, b)
    with torch.no_grad():
        y = ql(x.to(DEV)).float().cpu().numpy()
    dt = _dt_name(dtype)
    sel = slice(None) if rows is None else rows
    wd = _oracle_deq(kind, w[sel] if rows is not None else w, s[sel] if rows is not None else s, k, group, dt)
    ref = qo.linear_f64(x.float().numpy(), wd, None if b is None else b[sel].numpy(), dt)
    got = y[:, sel]
    err = qo.rel_err(got, ref)
    _say(f"  {kind} N={n} K={k} M={m} g={group} {dt} bias={bias}: rel_err={err:.3e}")
    assert err <= REL_TOL
    return err


@pytest.mark.parametrize("m", [1, 8, 32, 64])
@pytest.mark.parametrize("layout", ["tiled", "canonical"])
def test_int8_decode_config_shape(m, layout, monkeypatch):
    """INT8 per-channel decode at 18944x3584, M in {1, 8, 32, 64}, both weight layouts;
    oracle on 512 rows."""
    monkeypatch.setenv("LSQ_WEIGHT_LAYOUT", layout)
    rows = np.sort(np.random.default_rng(m).choice(18944, 512, replace=False))
    _check_layer("int8", 18944, 3584, m, rows=rows)


@pytest.mark.parametrize("m", [1, 16, 17, 32, 64])
@pytest.mark.parametrize("layout", ["tiled", "canonical"])
def test_int4_g128_decode_config_shape(m, layout, monkeypatch):
    """INT4 group-128 decode at 18944x3584, M in {1, 16, 64} and the chunked kernel's
    6 x 2 workgroups at 17 and 32 tokens, both weight layouts."""
    monkeypatch.setenv("LSQ_WEIGHT_LAYOUT", layout)
    rows = np.sort(np.random.default_rng(m).choice(18944, 512, replace=False))
    _check_layer("int4", 18944, 3584, m, rows=rows)


@pytest.mark.parametrize("m", [17, 33, 64])
@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_decode_large_n_small_k_token_blocks(kind, m):
    """18944 x 1024: 1184 row tiles over 8 k tiles take the 6 x 2 workgroups, here with
    the 17..64-token blocks (activations resident in LDS); oracle on 512 rows."""
    rows = np.sort(np.random.default_rng(100 + m).choice(18944, 512, replace=False))
    _check_layer(kind, 18944, 1024, m, rows=rows, bias=(m % 2 == 1))


@pytest.mark.parametrize("m", [2, 4, 8, 16, 24, 33, 64])
@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_decode_large_k_small_n(kind, m):
    """Down-projection shape 3584 x 18944: x of 4+ tokens exceeds LDS, so the chunked decode
    serves every M here (with fewer K slices when the staged group scales need the room);
    oracle on 256 rows."""
    rows = np.sort(np.random.default_rng(200 + m).choice(3584, 256, replace=False))
    _check_layer(kind, 3584, 18944, m, rows=rows, bias=(m % 2 == 0), seed=m)


@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_chunked_decode_6x2_one_block(kind):
    """16384 x 16384 at 8 tokens: x (256 KB) exceeds LDS, so the chunked decode runs its
    6 x 2 workgroups with one 16-token block; oracle on 256 rows."""
    rows = np.sort(np.random.default_rng(300).choice(16384, 256, replace=False))
    _check_layer(kind, 16384, 16384, 8, rows=rows, bias=True, seed=11)


@pytest.mark.parametrize("rg", ["4", "8"])
@pytest.mark.parametrize("m", [4, 16])
def test_chunked_decode_waves_per_workgroup(m, rg, monkeypatch):
    """3584 x 18944 with LSQ_DECODE_MB_RG forcing 4 or 8 waves per workgroup (the 2 x 2
    and 4 x 1 fallbacks of the one-block path); oracle on 256 rows."""
    monkeypatch.setenv("LSQ_DECODE_MB_RG", rg)
    monkeypatch.setenv("LSQ_GEMV", "0")  # (its split-K form takes these shapes by default)
    rows = np.sort(np.random.default_rng(400 + m).choice(3584, 256, replace=False))
    for kind in ("int4", "int8"):
        _check_layer(kind, 3584, 18944, m, rows=rows, bias=(m == 4), seed=m + 1)


@pytest.mark.parametrize("m", [9, 16])
def test_decode_qwen05b_down_proj_16_tokens(m):
    """896 x 4864 (Qwen2.5-0.5B down_proj) at 9 and 16 tokens: chunked decode."""
    _check_layer("int4", 896, 4864, m, bias=True, seed=m)


@pytest.mark.parametrize("m", [256, 2048, 8192])
@pytest.mark.parametrize("layout", ["tiled", "canonical"])
def test_int4_g128_prefill_config_shape(m, layout, monkeypatch):
    """INT4 group-128 prefill GEMM at the Llama-3-8B MLP shape 14336x4096, M in
    {256, 2048, 8192}; oracle on 256 sampled output columns and (for M > 256) 256 sampled
    rows."""
    monkeypatch.setenv("LSQ_WEIGHT_LAYOUT", layout)
    n, k = 14336, 4096
    p, s, x = bench.make_int4(n, k, m, 128, seed=m)
    ql = _layer("int4", p, s, k, 128)
    with torch.no_grad():
        y = ql(x.to(DEV)).float().cpu().numpy()
    rng = np.random.default_rng(m)
    cols = np.sort(rng.choice(n, 256, replace=False))
    rows = np.arange(m) if m <= 256 else np.sort(rng.choice(m, 256, replace=False))
    wd = qo.dequant_int4(p[cols].numpy(), s[cols].float().numpy(), k, 128, "bf16")
    ref = qo.linear_f64(x[rows].float().numpy(), wd, None, "bf16")
    err = qo.rel_err(y[np.ix_(rows, cols)], ref)
    _say(f"  int4 prefill M={m} {layout}: rel_err={err:.3e}")
    assert err <= REL_TOL


@pytest.mark.parametrize("variant", ["reg", "wide", "mid", "small", "lds"])
@pytest.mark.parametrize("kind", ["int8", "int4"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_gemm_edges_bias_and_dtypes(kind, dtype, variant, monkeypatch):
    """Every prefill kernel (register weights with 128 x 128, 256 x 256, 64 x 128 and
    64 x 64 tiles, LDS weights) on ragged M and N edges (M=300, N=272 = 256 + 16), bias,
    both dtypes, per-channel INT8, group-128 INT4, and per-channel INT4."""
    monkeypatch.setenv("LSQ_GEMM", variant)
    _check_layer(kind, 272, 512, 300, group=128, dtype=dtype, bias=True, seed=7)
    if kind == "int4":
        _check_layer("int4", 272, 512, 300, group=512, dtype=dtype, bias=True, seed=8)


@pytest.mark.parametrize("layout", ["tiled", "canonical"])
@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_gemm_tile_choice_small_n_layers(kind, layout, monkeypatch):
    """The default tile choice on layers where 128 x 128 tiles leave most CUs idle (64-row
    tiles: 128 or, for INT4 with few tiles, 64 weight rows wide; 256 x 256 only when it
    still gives 112+ workgroups), against the oracle on sampled columns: Qwen2.5-0.5B
    down_proj 896 x 4864 and gate_proj 4864 x 896, Qwen2.5-7B down_proj 3584 x 18944, and
    14336 x 4096 at 96 tokens."""
    monkeypatch.setenv("LSQ_WEIGHT_LAYOUT", layout)
    for n, k, m in ((896, 4864, 65), (896, 4864, 1024), (4864, 896, 128), (4864, 896, 256),
                    (3584, 18944, 128), (14336, 4096, 96)):
        cols = np.arange(n) if n <= 1024 else np.sort(np.random.default_rng(n + m).choice(n, 512, replace=False))
        _check_layer(kind, n, k, m, bias=(m % 2 == 1), seed=n + k + m, rows=cols)


@pytest.mark.parametrize("splits", ["2", "5", "16"])
@pytest.mark.parametrize("variant", ["reg", "wide", "mid", "small"])
@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_gemm_split_k_forced(kind, variant, splits, monkeypatch):
    """The prefill GEMM's split-K form (K slices over workgroups, fp32 partial sums in the
    module's workspace, ordered merge with the bias) with forced slice counts on every
    tile shape it serves: ragged M and N (M=300, N=272), bias, group-128 and per-channel
    INT4, per-channel INT8, both activation types; 16 slices of K = 8192 leave 8 steps
    each."""
    monkeypatch.setenv("LSQ_GEMM", variant)
    monkeypatch.setenv("LSQ_GEMM_SPLITK", splits)
    for dtype in (torch.bfloat16, torch.float16):
        _check_layer(kind, 272, 8192, 300, group=128, dtype=dtype, bias=True, seed=int(splits))
    if kind == "int4":
        _check_layer("int4", 272, 8192, 300, group=8192, bias=True, seed=3)


@pytest.mark.parametrize("m", [128, 2048])
def test_gemm_split_k_deterministic_and_matches_unsplit(m, monkeypatch):
    """Qwen2.5-7B down_proj 3584 x 18944 (split by default: 64 x 64 tiles at 128 tokens,
    256 x 256 at 2048): bit-identical on a second call; the unsplit kernel
    (LSQ_GEMM_SPLITK=0) within the contract (the slices' sums are added in another order);
    the oracle on sampled columns and rows."""
    w, s, x = bench.make_int4(3584, 18944, m, 128, seed=5)
    ql = _layer("int4", w, s, 18944, 128)
    xd = x.to(DEV)
    with torch.no_grad():
        y1 = ql(xd).float().cpu().numpy()
        y2 = ql(xd).float().cpu().numpy()
        monkeypatch.setenv("LSQ_GEMM_SPLITK", "0")
        y0 = ql(xd).float().cpu().numpy()
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
    err = qo.rel_err(y1, y0.astype(np.float64))
    _say(f"  split vs unsplit GEMM M={m}: rel={err:.3e}")
    assert err <= REL_TOL
    rng = np.random.default_rng(m)
    cols = np.sort(rng.choice(3584, 128, replace=False))
    rows = np.arange(m) if m <= 256 else np.sort(rng.choice(m, 128, replace=False))
    wd = qo.dequant_int4(w[cols].numpy(), s[cols].float().numpy(), 18944, 128, "bf16")
    ref = qo.linear_f64(x[rows].float().numpy(), wd, None, "bf16")
    assert qo.rel_err(y1[np.ix_(rows, cols)], ref) <= REL_TOL


@pytest.mark.parametrize("m", [24, 33, 64])
@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_batched_decode_through_split_gemm(kind, m, monkeypatch):
    """24-64 tokens on long-K, small-N layers (Qwen2.5-7B down_proj 3584 x 18944, Llama-3-8B
    down_proj 4096 x 14336) run the split-K GEMM with 64 x 128 tiles: against the oracle on
    sampled columns, and against the decode kernels (LSQ_BATCH_GEMM=0) within the
    contract; without a workspace (the plain C entry point) the decode kernels serve the
    call unchanged."""
    from localstrm_amd import _lib
    for n, k in ((3584, 18944), (4096, 14336)):
        cols = np.sort(np.random.default_rng(n + m).choice(n, 384, replace=False))
        _check_layer(kind, n, k, m, bias=(m % 2 == 1), seed=n + m, rows=cols)
    n, k = 3584, 18944
    if kind == "int8":
        w, s, x = bench.make_int8(n, k, m, seed=m)
    else:
        w, s, x = bench.make_int4(n, k, m, 128, seed=m)
    ql = _layer(kind, w, s, k, 128)
    xd = x.to(DEV)
    with torch.no_grad():
        y_gemm = ql(xd).float().cpu().numpy()
        monkeypatch.setenv("LSQ_BATCH_GEMM", "0")
        y_dec = ql(xd).float().cpu().numpy()
    err = qo.rel_err(y_gemm, y_dec.astype(np.float64))
    _say(f"  {kind} M={m}: split GEMM vs decode kernels rel={err:.3e}")
    assert err <= REL_TOL


@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_gemm_split_k_canonical_layout_through_c_abi(kind, monkeypatch):
    """The split-K GEMM reading the canonical layouts (int8 [N, K], packed INT4 [N, K/2]:
    what a C caller passes without building the tiled copy) with a workspace, forced and by
    default (896 x 4864 at 256 tokens splits), against the oracle and against the plain
    entry point (no workspace: unsplit)."""
    from localstrm_amd import _lib
    lib = _lib.load()
    n, k, m = 896, 4864, 256
    if kind == "int8":
        w, s, x = bench.make_int8(n, k, m, seed=3)
    else:
        w, s, x = bench.make_int4(n, k, m, 128, seed=3)
    wd_, sd, xd = w.to(DEV), s.to(DEV), x.to(DEV)
    b = torch.randn(n, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    bd = b.to(DEV)
    stream = _lib.stream_handle(DEV)

    def call(ws, nbytes):
        y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
        if kind == "int8":
            args = (xd.data_ptr(), k, wd_.data_ptr(), None, sd.data_ptr(), _lib.dtype_code(sd.dtype),
                    bd.data_ptr(), _lib.dtype_code(bd.dtype), y.data_ptr(), n, _lib.dtype_code(torch.bfloat16), m, n, k)
            rc = lib.lsq_w8_linear_ws(*args, _lib.ptr(ws), nbytes, stream) if ws is not False else lib.lsq_w8_linear(*args, stream)
        else:
            args = (xd.data_ptr(), k, wd_.data_ptr(), None, sd.data_ptr(), _lib.dtype_code(sd.dtype), 128,
                    bd.data_ptr(), _lib.dtype_code(bd.dtype), y.data_ptr(), n, _lib.dtype_code(torch.bfloat16), m, n, k)
            rc = lib.lsq_w4_linear_ws(*args, _lib.ptr(ws), nbytes, stream) if ws is not False else lib.lsq_w4_linear(*args, stream)
        _lib.check(rc, "linear_ws")
        return y.float().cpu().numpy()

    wdq = qo.dequant_int8(w.numpy(), s.numpy(), "bf16") if kind == "int8" else qo.dequant_int4(w.numpy(), s.float().numpy(), k, 128, "bf16")
    ref = qo.linear_f64(x.float().numpy(), wdq, b.float().numpy(), "bf16")
    plain = call(False, 0)
    assert qo.rel_err(plain, ref) <= REL_TOL
    for forced in (None, "3", "9"):
        if forced:
            monkeypatch.setenv("LSQ_GEMM_SPLITK", forced)
        nws = lib.lsq_linear_workspace_bytes(m, n, k)
        assert nws > 0
        ws = torch.empty(nws, dtype=torch.uint8, device=DEV)
        got = call(ws, nws)
        err = qo.rel_err(got, ref)
        _say(f"  {kind} canonical split={forced or 'default'}: rel_err={err:.3e}")
        assert err <= REL_TOL
        assert qo.rel_err(got, plain.astype(np.float64)) <= REL_TOL


def test_int8_single_linear_config():
    """Qwen2.5-0.5B gate_proj: W int8 [4864, 896], fp32 scale, x fp32 and bf16 [1, 896]."""
    for dtype in (torch.float32, torch.bfloat16):
        w, s, x = bench.make_int8(4864, 896, 1, x_dtype=torch.float32)
        ql = _layer("int8", w, s)
        xt = x.to(dtype)
        with torch.no_grad():
            y = ql(xt.to(DEV)).float().cpu().numpy()
        dt = _dt_name(dtype)
        ref = qo.linear_f64(xt.float().numpy(), qo.dequant_int8(w.numpy(), s.numpy(), dt), None, dt)
        err = qo.rel_err(y, ref)
        _say(f"  config-1 {dt}: rel_err={err:.3e}")
        assert err <= (1e-5 if dtype == torch.float32 else REL_TOL)


@pytest.mark.parametrize("kind", ["int8", "int4"])
@pytest.mark.parametrize("m", [1, 3, 16, 17, 33, 63, 64, 65, 100, 256])
def test_ragged_m_with_bias(kind, m):
    _check_layer(kind, 256, 512, m, group=128, bias=True, seed=m)


@pytest.mark.parametrize("kind,n,k,group", [
    ("int8", 100, 384, None),     # N not a multiple of 16
    ("int4", 100, 384, 128),
    ("int4", 64, 384, 64),        # group below the 128-column tile: generic kernel
    ("int4", 64, 200, 128),       # K not a multiple of 128
    ("int4", 48, 256, None),      # per-channel (reference) INT4
    ("int8", 24, 100, None),      # K not a multiple of 128
])
def test_odd_shapes(kind, n, k, group):
    g = (group if group is not None else k) if kind == "int4" else 128
    for dtype in (torch.bfloat16, torch.float16):
        _check_layer(kind, n, k, 5, group=g, dtype=dtype, seed=n + k)


@pytest.mark.parametrize("layout", ["tiled", "canonical"])
@pytest.mark.parametrize("kind,group", [("int8", None), ("int4", 128), ("int4", 896)])
def test_batched_decode_edges(layout, kind, group, monkeypatch):
    """Batched decode (17..64 tokens): a partial last workgroup (N = 272 = 17 row tiles),
    an odd number of k tiles (K = 896, so the last activation chunk is half empty), a
    single k tile (K = 128), bias, both activation types, group-128 and per-channel INT4."""
    monkeypatch.setenv("LSQ_WEIGHT_LAYOUT", layout)
    g = group if group is not None else 128
    for m in (17, 40, 64):
        for dtype in (torch.bfloat16, torch.float16):
            _check_layer(kind, 272, 896, m, group=g, dtype=dtype, bias=True, seed=m)
    _check_layer(kind, 80, 128, 33, group=128, bias=True, seed=3)


@pytest.mark.parametrize("kind,group", [("int8", None), ("int4", 128), ("int4", 256), ("int4", 384),
                                        ("int4", 4864)])
def test_chunked_decode_large_k(kind, group):
    """17..64 tokens with activations too large for LDS (K = 4864, the Qwen2.5-0.5B down
    projection): the chunked decode kernel, partial last workgroup, bias, both dtypes;
    groups of 1, 2 and 3 k tiles (384: the last group is partial) and per-channel."""
    g = group if group is not None else 128
    for m in (17, 48):
        for dtype in (torch.bfloat16, torch.float16):
            _check_layer(kind, 272, 4864, m, group=g, dtype=dtype, bias=True, seed=m + 1)


def test_batched_decode_strided_x():
    p, s, _ = bench.make_int4(256, 512, 40)
    ql = _layer("int4", p, s, 512, 128)
    wide = torch.randn(40, 640, dtype=torch.bfloat16, device=DEV)
    with torch.no_grad():
        y1 = ql(wide[:, :512])
        y2 = ql(wide[:, :512].contiguous())
    assert torch.equal(y1, y2)


def test_fp16_decode_paths():
    for kind in ("int8", "int4"):
        for m in (1, 16, 40):
            _check_layer(kind, 512, 1024, m, dtype=torch.float16, seed=m)


def test_empty_input_and_strided_x():
    p, s, x = bench.make_int4(64, 256, 8)
    ql = _layer("int4", p, s, 256, 128)
    with torch.no_grad():
        y0 = ql(torch.empty(0, 256, dtype=torch.bfloat16, device=DEV))
        assert y0.shape == (0, 64)
        wide = torch.randn(8, 384, dtype=torch.bfloat16, device=DEV)
        y1 = ql(wide[:, :256])
        y2 = ql(wide[:, :256].contiguous())
    assert torch.equal(y1, y2)


def test_shape_mismatch_raises():
    p, s, _ = bench.make_int4(64, 256, 1)
    ql = _layer("int4", p, s, 256, 128)
    with pytest.raises(RuntimeError):
        ql(torch.randn(2, 128, dtype=torch.bfloat16, device=DEV))


# ----------------------------------------------------------------------------- reference-style


def test_output_dtype_device_and_shapes():
    """tests/test_quantized_loader.py:211-223 and :311-333 on the GPU."""
    lin = nn.Linear(64, 32, bias=True)
    for mode in ("int8", "int4"):
        ql = QuantizedLinear.from_float(lin, mode).to(DEV)
        for dtype in (torch.float32, torch.float16, torch.bfloat16):
            for shape in [(1, 64), (4, 64), (1, 1, 64), (4, 1, 64), (2, 16, 64), (8, 32, 64)]:
                x = torch.randn(*shape, dtype=dtype, device=DEV)
                with torch.no_grad():
                    out = ql(x)
                assert out.dtype == dtype and out.device == x.device
                assert out.shape == shape[:-1] + (32,)
                assert torch.isfinite(out).all()


@pytest.mark.parametrize("mode,cos_min,max_abs,mean_abs,seed", [
    ("int8", 0.999, 0.05, 0.01, 12345), ("int4", 0.99, 0.35, 0.08, 54321)])
def test_accuracy_vs_float_linear(mode, cos_min, max_abs, mean_abs, seed):
    """tests/test_quantized_loader.py:228-306: quantized vs the float layer, fp32 x."""
    torch.manual_seed(seed)
    for in_f, out_f in [(32, 32), (64, 32), (32, 64), (128, 64), (64, 128)]:
        ref = nn.Linear(in_f, out_f, bias=True)
        ql = QuantizedLinear.from_float(ref, mode).to(DEV)
        x = torch.randn(8, in_f)
        with torch.no_grad():
            r = ref(x)
            o = ql(x.to(DEV)).cpu()
        cos = F.cosine_similarity(r.flatten(), o.flatten(), dim=0).item()
        err = (r - o).abs()
        assert cos >= cos_min and err.max().item() <= max_abs and err.mean().item() <= mean_abs


def test_bias_and_no_bias():
    for mode in ("int8", "int4"):
        qb = QuantizedLinear.from_float(nn.Linear(32, 16, bias=True), mode).to(DEV)
        qn = QuantizedLinear.from_float(nn.Linear(32, 16, bias=False), mode).to(DEV)
        assert qb.bias is not None and qn.bias is None
        x = torch.randn(2, 32, device=DEV)
        assert qb(x).shape == (2, 16) and qn(x).shape == (2, 16)


def test_loader_moves_to_gpu_and_builds_tiled_layout():
    from localstrm_amd import load_and_quantize_model
    from tests.synthetic import seeded_model

    model, _, _ = load_and_quantize_model(seeded_model(h=128), device=DEV, quantization="int4",
                                          dtype=torch.bfloat16)
    q = model.model.layers[0].self_attn.q_proj
    assert all(b.device.type == "cuda" for b in model.buffers())
    assert q.weight_tiled.numel() == 128 * 128 // 2
    x = torch.randn(3, 5, 128, device=DEV)
    with torch.no_grad():
        y = model.model(x)
    assert torch.isfinite(y).all()
    # an in-place update of weight_packed (load_state_dict) is picked up by the tiled copy
    sd = {k: v.clone() for k, v in q.state_dict().items()}
    sd["weight_packed"] = torch.full_like(sd["weight_packed"], 0x88)  # all q = 0
    q.load_state_dict(sd)
    with torch.no_grad():
        out = q(torch.randn(2, 128, device=DEV, dtype=torch.bfloat16))
    assert torch.allclose(out.float(), q.bias.detach().to(torch.bfloat16).float().expand_as(out))


def test_autograd_grad_wrt_input():
    lin = nn.Linear(64, 32, bias=True)
    ql = QuantizedLinear.from_float(lin, "int8").to(DEV)
    x = torch.randn(4, 64, device=DEV, requires_grad=True)
    y = ql(x)
    y.sum().backward()
    w = ql.dequantize(torch.float32)
    assert torch.allclose(x.grad, torch.ones(4, 32, device=DEV) @ w, atol=1e-5)
    assert torch.allclose(ql.bias.grad, torch.full((32,), 4.0, device=DEV))


def test_graph_capture_replays_match_eager():
    p, s, x = bench.make_int4(512, 1024, 4)
    ql = _layer("int4", p, s, 1024, 128)
    x = x.to(DEV)
    with torch.no_grad():
        ref = ql(x).clone()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(g, stream=stream):
                out = ql(x)
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
            _ = ql(x)  # eager work between replays


@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_fused_linears_match_separate_layers(kind):
    """fuse_linears (q/k/v-shaped: 896, 128, 128 rows with bias; and gate/up-shaped: two
    4864-row layers without bias) against the layers run one by one and the oracle."""
    from localstrm_amd import fuse_linears

    for shapes, bias in (([896, 128, 128], True), ([4864, 4864], False)):
        layers, wds = [], []
        for i, n in enumerate(shapes):
            if kind == "int8":
                w, s, _ = bench.make_int8(n, 896, 1, seed=10 + i)
            else:
                w, s, _ = bench.make_int4(n, 896, 1, 128, seed=10 + i)
            b = torch.randn(n, generator=torch.Generator().manual_seed(20 + i)) if bias else None
            layers.append(_layer(kind, w, s, 896, 128, b))
            wds.append((_oracle_deq(kind, w, s, 896, 128, "bf16"), None if b is None else b.numpy()))
        fused = fuse_linears(layers)
        for m in (1, 32, 300):
            x = torch.randn(m, 896, generator=torch.Generator().manual_seed(m)).to(torch.bfloat16)
            with torch.no_grad():
                outs = fused(x.to(DEV))
                sep = [l(x.to(DEV)) for l in layers]
            assert len(outs) == len(shapes)
            for o, s_, (wd, bd), n in zip(outs, sep, wds, shapes):
                assert o.shape == (m, n) and o.dtype == torch.bfloat16
                ref = qo.linear_f64(x.float().numpy(), wd, bd, "bf16")
                err = qo.rel_err(o.float().cpu().numpy(), ref)
                assert err <= REL_TOL
                assert qo.rel_err(o.float().cpu().numpy(), s_.float().cpu().numpy()) <= REL_TOL
            _say(f"  fused {kind} {shapes} M={m}: ok")
