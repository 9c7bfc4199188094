"""GPU checks of the weight quantizer (lsq_quantize_w8 / lsq_quantize_w4, csrc/lsq_quantize.hip)
against the oracle's quantizers (oracle.quant_oracle.quantize_int8 / quantize_int4, the CPU
restatement of src/kernels/quantization.py:72-94): q, packed nibbles, tiled layouts and
scales bit for bit, at the 18944 x 3584 layer shape, on constructed round-half-to-even
ties, on odd and non-multiple-of-128 K, with strided rows; and from_float on a GPU layer
against from_float on the CPU (the reference's CPU staging, quantization.py:593-610).
"""

import numpy as np
import pytest
import torch
import torch.nn as nn

from localstrm_amd import Int8GEMMLinear, QuantizedLinear, _lib
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
SDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


def _say(msg):
    print(msg, flush=True)


def _weights(n, k, dt, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(n, k, generator=g) * 0.02
    w[:, 0] *= 40  # a few large columns, so the row and group maxima vary
    return w.to(TDT[dt])


def _q8(w, tiled=False):
    """(q, tiled or None, scale) from lsq_quantize_w8 on the GPU."""
    n, k = w.shape
    wd = w.to(DEV)
    ld = wd.stride(0)
    lib = _lib.load()
    scale = torch.empty(n, dtype=torch.float32, device=DEV)
    q = torch.full((n, k), 99, dtype=torch.int8, device=DEV)
    t = torch.full((lib.lsq_w8_tiled_bytes(n, k),), 99, dtype=torch.int8, device=DEV) if tiled else None
    rc = lib.lsq_quantize_w8(wd.data_ptr(), _lib.dtype_code(wd.dtype), ld, n, k, scale.data_ptr(), q.data_ptr(),
                             _lib.ptr(t), _lib.stream_handle(DEV))
    _lib.check(rc, "lsq_quantize_w8")
    torch.cuda.synchronize()
    return q, t, scale


def _untile8(t, n, k):
    out = torch.empty((n, k), dtype=torch.int8, device=DEV)
    lib = _lib.load()
    _lib.check(lib.lsq_w8_untile(t.data_ptr(), out.data_ptr(), n, k, _lib.stream_handle(DEV)), "untile")
    return out


def _q4(w, group, sdt, tiled=False):
    n, k = w.shape
    wd = w.to(DEV)
    lib = _lib.load()
    per_channel = group is None or group >= k
    ng = 1 if per_channel else -(-k // group)
    scale = torch.empty((n, ng), dtype=torch.float32 if per_channel else SDT[sdt], device=DEV)
    p = torch.full((n, (k + 1) // 2), 0x5A, dtype=torch.uint8, device=DEV)
    t = torch.full((lib.lsq_w4_tiled_bytes(n, k),), 0x5A, dtype=torch.uint8, device=DEV) if tiled else None
    rc = lib.lsq_quantize_w4(wd.data_ptr(), _lib.dtype_code(wd.dtype), wd.stride(0), n, k, 0 if per_channel else group,
                             scale.data_ptr(), _lib.dtype_code(scale.dtype), p.data_ptr(), _lib.ptr(t),
                             _lib.stream_handle(DEV))
    _lib.check(rc, "lsq_quantize_w4")
    torch.cuda.synchronize()
    return p, t, scale


def _untile4(t, n, k):
    out = torch.empty((n, (k + 1) // 2), dtype=torch.uint8, device=DEV)
    lib = _lib.load()
    _lib.check(lib.lsq_w4_untile(t.data_ptr(), out.data_ptr(), n, k, _lib.stream_handle(DEV)), "untile")
    return out


def _f32(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_quantize_w8_full_size(dt):
    n, k = 18944, 3584
    w = _weights(n, k, dt, seed=1)
    _say(f"  quantize_w8 {dt} {n}x{k}")
    q, t, s = _q8(w, tiled=True)
    q_ref, s_ref = qo.quantize_int8(_f32(w))
    assert np.array_equal(s.cpu().numpy().view(np.uint32), s_ref.reshape(-1).view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert torch.equal(_untile8(t, n, k).cpu(), torch.from_numpy(q_ref))


@pytest.mark.parametrize("group,sdt", [(128, "bf16"), (64, "f16"), (256, "f32"), (None, "f32")])
def test_quantize_w4_full_size(group, sdt):
    n, k = 18944, 3584
    w = _weights(n, k, "bf16", seed=2)
    _say(f"  quantize_w4 {n}x{k} group={group} scale {sdt}")
    p, t, s = _q4(w, group, sdt, tiled=True)
    p_ref, s_ref = qo.quantize_int4(_f32(w), group_size=group, scale_dt=sdt)
    assert np.array_equal(_f32(s).view(np.uint32), np.asarray(s_ref, np.float32).view(np.uint32))
    assert np.array_equal(p.cpu().numpy(), p_ref)
    assert np.array_equal(_untile4(t, n, k).cpu().numpy(), p_ref)


def test_quantize_ties_round_half_to_even():
    """Rows whose max is exactly 127 (INT8) / 7 (INT4) have scale 1.0, so w / s is w and
    every x.5 is a tie: round half to even, as torch.round."""
    row8 = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -127.5 + 0.5, 3.5, -3.5, 0.0]
    w8 = torch.tensor([row8 + [0.0] * (128 - len(row8))] * 16, dtype=torch.float32)
    q, t, s = _q8(w8, tiled=True)
    assert torch.equal(s.cpu(), torch.ones(16))
    expect = [127, 0, 2, 2, 0, -2, -2, 126, -127, 4, -4, 0]
    assert q.cpu()[0, :12].tolist() == expect
    assert torch.equal(_untile8(t, 16, 128).cpu(), q.cpu())
    row4 = [7.0, 0.5, 1.5, 2.5, 3.5, -3.5, -0.5, 6.5, -6.5, -7.5 + 0.5, 5.5, -2.5]
    w4 = torch.tensor([row4 + [0.0] * (128 - len(row4))] * 16, dtype=torch.float32)
    p, t4, s4 = _q4(w4, None, "f32", tiled=True)
    assert torch.equal(s4.cpu(), torch.ones(16, 1))
    got = qo.unpack_int4(p.cpu().numpy(), 128)[0, :12].tolist()
    assert got == [7, 0, 2, 2, 4, -4, 0, 6, -6, -7, 6, -2]
    assert torch.equal(_untile4(t4, 16, 128).cpu(), p.cpu())


def test_quantize_w4_group_uses_the_stored_scale():
    """The hand-worked group of the oracle's test (max / 7 = 1 + 2^-9: stored as 1.0 in
    bf16, exactly in fp16) on the GPU: q = 4 against the bf16 scale, 3 against fp16."""
    w = torch.tensor([[7.013671875, 3.50390625, -7.0, 2.5]], dtype=torch.float32)
    p, _, s = _q4(w, 2, "bf16")
    assert s.float().cpu().tolist() == [[1.0, 1.0]] and p.cpu().tolist() == [[0xCF, 0xA1]]
    p16, _, s16 = _q4(w, 2, "f16")
    assert s16.float().cpu().tolist() == [[1.001953125, 1.0]]
    assert qo.unpack_int4(p16.cpu().numpy(), 4).tolist() == [[7, 3, -7, 2]]


@pytest.mark.parametrize("n,k", [(5, 33), (17, 100), (33, 1000), (3, 1)])
def test_quantize_odd_shapes_canonical(n, k):
    """K odd (the last high nibble stays 0), K not a multiple of 128, K = 1."""
    w = _weights(n, k, "f16", seed=n + k)
    q, _, s = _q8(w)
    q_ref, s_ref = qo.quantize_int8(_f32(w))
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(s.cpu().numpy(), s_ref.reshape(-1))
    for group, sdt in ((None, "f32"), (16, "bf16"), (7, "f16")):
        p, _, s4 = _q4(w, group, sdt)
        p_ref, s4_ref = qo.quantize_int4(_f32(w), group_size=group, scale_dt=sdt)
        assert np.array_equal(p.cpu().numpy(), p_ref), (group, sdt)
        assert np.array_equal(_f32(s4), np.asarray(s4_ref, np.float32))


def test_quantize_strided_rows_and_zero_rows():
    """Rows read with a stride larger than K (a column slice); an all-zero row takes the
    1e-8 clamp and quantizes to 0."""
    big = _weights(64, 384, "bf16", seed=9)
    big[3] = 0
    w = big[:, :256]
    lib = _lib.load()
    wd = big.to(DEV)
    scale = torch.empty(64, dtype=torch.float32, device=DEV)
    q = torch.empty((64, 256), dtype=torch.int8, device=DEV)
    rc = lib.lsq_quantize_w8(wd.data_ptr(), _lib.dtype_code(wd.dtype), 384, 64, 256, scale.data_ptr(),
                             q.data_ptr(), None, _lib.stream_handle(DEV))
    _lib.check(rc, "lsq_quantize_w8")
    q_ref, s_ref = qo.quantize_int8(_f32(w))
    assert np.array_equal(q.cpu().numpy(), q_ref) and np.array_equal(scale.cpu().numpy(), s_ref.reshape(-1))
    assert scale[3].item() == np.float32(1e-8) and not q[3].any()


@pytest.mark.parametrize("mode,group", [("int8", None), ("int4", None), ("int4", 128)])
def test_from_float_on_gpu_matches_cpu_staging(mode, group):
    """QuantizedLinear.from_float on a GPU layer (this quantizer, tiled copy written
    directly) holds what from_float on the CPU layer (the reference's staging) holds."""
    torch.manual_seed(4)
    lin = nn.Linear(1024, 528, bias=True).to(torch.bfloat16)
    cpu = QuantizedLinear.from_float(lin, mode, group_size=group)
    gpu = QuantizedLinear.from_float(lin.to(DEV), mode, group_size=group)
    assert gpu.weight_tiled.numel() > 0 and gpu._buffers[gpu._cname()].numel() == 0
    cname = "weight_q" if mode == "int8" else "weight_packed"
    assert torch.equal(getattr(gpu, cname).cpu(), getattr(cpu, cname))
    assert gpu.scale.dtype == cpu.scale.dtype and torch.equal(gpu.scale.cpu(), cpu.scale)
    assert torch.equal(gpu.bias.detach().cpu(), cpu.bias.detach())
    cpu_on_gpu = cpu.to(DEV)
    assert torch.equal(gpu.weight_tiled, cpu_on_gpu.weight_tiled)
    x = torch.randn(3, 1024, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        assert torch.equal(gpu(x), cpu_on_gpu(x))


@pytest.mark.parametrize("k", [896, 1000])
def test_int8_gemm_from_float_on_gpu_matches_cpu(k):
    """Int8GEMMLinear.from_float on a GPU layer: the W8A8 tiled copy written directly
    (K % 128 == 0) or through weight_q_t and the W8A8 re-tile (K = 1000)."""
    torch.manual_seed(5)
    lin = nn.Linear(k, 264, bias=True).to(torch.float16)
    cpu = Int8GEMMLinear.from_float(lin)
    gpu = Int8GEMMLinear.from_float(lin.to(DEV))
    assert gpu.weight_tiled.numel() > 0 and gpu._buffers["weight_q_t"].numel() == 0
    assert torch.equal(gpu.weight_q_t.cpu(), cpu.weight_q_t)
    assert torch.equal(gpu.scale_w_t.cpu(), cpu.scale_w_t)
    x = torch.randn(5, k, device=DEV, dtype=torch.float16)
    with torch.no_grad():
        assert torch.equal(gpu(x), cpu.to(DEV)(x))
