"""Pins the CPU oracle (oracle/quant_oracle.py) before anything is checked against it.

Every oracle function is checked against something other than its own formula:
exact-rational golden vectors, torch's dtype casts and ops, hand-computed known answers,
brute force over every q value / byte value, and mathematical special cases. A planted
mistake (wrong nibble order, truncation instead of RNE, dropped round_T of the scale,
a transposed operand, a missing bias) fails at least one test here.
"""

import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import quant_oracle as qo
from oracle import torch_ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz")
TORCH_DT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


# ----------------------------------------------------------------------------- rounding


def test_round_bf16_matches_torch_on_boundaries():
    rng = np.random.default_rng(0)
    bits = np.concatenate([
        rng.integers(0, 2**32, size=200000, dtype=np.uint64).astype(np.uint32),
        # exact ties (low half = 0x8000) with even and odd kept lsb, and near-ties
        (rng.integers(0, 2**16, size=5000, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000,
        (rng.integers(0, 2**16, size=5000, dtype=np.uint64).astype(np.uint32) << 16) | 0x7FFF,
        (rng.integers(0, 2**16, size=5000, dtype=np.uint64).astype(np.uint32) << 16) | 0x8001,
        np.array([0x7F7FFFFF, 0xFF7FFFFF, 0x00000001, 0x80000001, 0x007FFFFF, 0x7F800000,
                  0xFF800000, 0x00000000, 0x80000000], dtype=np.uint32),
    ])
    f = bits.view(np.float32)
    f = f[~np.isnan(f)]
    ours = qo.round_bf16(f)
    theirs = torch.from_numpy(f.copy()).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


def test_round_bf16_known_ties():
    # 1 + 2^-8 is the exact midpoint of 1 and 1 + 2^-7: ties to the even mantissa (1.0)
    assert qo.round_bf16(np.float32(1.0 + 2**-8))[()] == 1.0
    # 1 + 3*2^-8 lies between 1 + 2^-7 (odd) and 1 + 2^-6 (even): rounds up
    assert qo.round_bf16(np.float32(1.0 + 3 * 2**-8))[()] == np.float32(1.0 + 2**-6)
    assert np.isnan(qo.round_bf16(np.float32("nan"))[()])
    assert qo.round_bf16(np.float32(3.4e38))[()] == np.inf


def test_round_f16_matches_torch():
    rng = np.random.default_rng(1)
    f = np.concatenate([rng.standard_normal(100000) * 100, rng.standard_normal(10000) * 1e-5]).astype(np.float32)
    ours = qo.round_f16(f)
    theirs = torch.from_numpy(f).to(torch.float16).float().numpy()
    assert np.array_equal(ours, theirs)


# ----------------------------------------------------------------------------- pack / unpack


def test_pack_known_answer():
    # byte j = (q[2j]+8) | (q[2j+1]+8) << 4; odd K pads the high nibble with 0
    q = np.array([[-8, 7, 0, 1, -1]], dtype=np.int8)
    assert qo.pack_int4(q).tolist() == [[0xF0, 0x98, 0x07]]


def test_unpack_every_byte_value():
    packed = np.arange(256, dtype=np.uint8).reshape(1, 256)
    q = qo.unpack_int4(packed, 512)
    b = np.arange(256)
    assert np.array_equal(q[0, 0::2], (b % 16) - 8)
    assert np.array_equal(q[0, 1::2], (b // 16) - 8)


@pytest.mark.parametrize("k", [32, 33, 128, 1536])
def test_pack_unpack_round_trip_and_torch(k):
    # the reference's own regression widths (tests/test_quantized_loader.py:442)
    rng = np.random.default_rng(k)
    q = rng.integers(-8, 8, size=(64, k)).astype(np.int8)
    p = qo.pack_int4(q)
    assert p.shape == (64, (k + 1) // 2) and p.dtype == np.uint8
    assert np.array_equal(qo.unpack_int4(p, k), q)
    assert np.array_equal(torch_ref.unpack_int4(torch.from_numpy(p), k).numpy(), q)


# ----------------------------------------------------------------------------- quantizers


def test_quantize_int8_known_answer():
    # max|w| = 254 -> scale 2; q = round(w / 2)
    w = np.array([[254.0, -128.0, 0.0, 2.0, 5.2, -3.0]], dtype=np.float32)
    q, s = qo.quantize_int8(w)
    assert s[0, 0] == 2.0
    assert q.tolist() == [[127, -64, 0, 1, 3, -2]]
    p, s4 = qo.quantize_int4(np.array([[14.0, -6.0, 1.0, 0.0]], np.float32))
    assert s4[0, 0] == 2.0
    assert qo.unpack_int4(p, 4).tolist() == [[7, -3, 0, 0]]


def test_quantize_round_half_even_ties():
    # scale = 7/7 = 1 exactly; w = k + 0.5 are exact ties and must go to the even integer
    w = np.array([[7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5]], dtype=np.float32)
    p, s = qo.quantize_int4(w)
    assert s[0, 0] == 1.0
    assert qo.unpack_int4(p, 8).tolist() == [[7, 0, 2, 2, 0, -2, -2, 4]]
    w8 = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -126.5, 125.5]], dtype=np.float32)
    q8, s8 = qo.quantize_int8(w8)
    assert s8[0, 0] == 1.0
    assert q8.tolist() == [[127, 0, 2, 2, 0, -2, -126, 126]]


def test_quantize_zero_row_clamps_scale():
    q, s = qo.quantize_int8(np.zeros((2, 8), np.float32))
    assert np.all(s == np.float32(1e-8)) and np.all(q == 0)


def test_quantizers_match_torch_op_sequence():
    g = torch.Generator().manual_seed(5)
    w = torch.randn(64, 96, generator=g) * 0.05
    q, s = qo.quantize_int8(w.numpy())
    ts = torch.clamp(w.abs().max(dim=-1, keepdim=True)[0] / 127.0, min=1e-8)
    tq = torch.clamp(torch.round(w / ts), -128, 127).to(torch.int8)
    assert np.array_equal(q, tq.numpy()) and np.array_equal(s, ts.numpy())
    p, s4 = qo.quantize_int4(w.numpy())
    ts4 = torch.clamp(w.abs().max(dim=-1, keepdim=True)[0] / 7.0, min=1e-8)
    tq4 = torch.clamp(torch.round(w / ts4), -8, 7).to(torch.int8)
    assert np.array_equal(qo.unpack_int4(p, 96), tq4.numpy()) and np.array_equal(s4, ts4.numpy())


def test_group_quantizer_reduces_to_per_channel():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((16, 256)) * 0.02).astype(np.float32)
    p1, s1 = qo.quantize_int4(w, group_size=None)
    p2, s2 = qo.quantize_int4(w, group_size=256, scale_dt="f32")
    assert np.array_equal(p1, p2) and np.array_equal(s1, s2)
    # a group quantizer on a matrix whose groups are row-constant copies is per-channel
    wg = np.tile(w[:, :64], (1, 4))
    pg, sg = qo.quantize_int4(wg, group_size=64, scale_dt="f32")
    assert np.all(sg == sg[:, :1])
    pc, sc = qo.quantize_int4(wg)
    assert np.array_equal(pg, pc)


def test_group_quantizer_uses_the_stored_scale_known_answer():
    """Group-wise INT4 quantizes against the scale as stored (rounded to its dtype), worked
    by hand. Group 0 = [7.013671875, 3.50390625]: max / 7 = 1 + 2^-9 exactly in fp32. bf16
    keeps 7 mantissa bits, so 1 + 2^-9 (a quarter ulp above 1.0) is stored as 1.0 and
    3.50390625 / 1.0 rounds to 4; fp16 keeps 10 bits, stores 1 + 2^-9 exactly, and
    3.50390625 / 1.001953125 = 3.4970... rounds to 3. Group 1 = [-7.0, 2.5]: scale 1.0,
    2.5 is a tie and rounds to the even 2. A quantizer using the unrounded fp32 scale would
    give 3 for bf16 too; one rounding ties away from zero would give 3 for 2.5."""
    w = np.array([[7.013671875, 3.50390625, -7.0, 2.5]], np.float32)
    p, s = qo.quantize_int4(w, group_size=2, scale_dt="bf16")
    assert s.tolist() == [[1.0, 1.0]]
    assert qo.unpack_int4(p, 4).tolist() == [[7, 4, -7, 2]]
    assert p.tolist() == [[0xCF, 0xA1]]  # q + 8 = 15, 12 | 1, 10; low nibble = even column
    p16, s16 = qo.quantize_int4(w, group_size=2, scale_dt="f16")
    assert s16.tolist() == [[1.001953125, 1.0]]
    assert qo.unpack_int4(p16, 4).tolist() == [[7, 3, -7, 2]]


# ----------------------------------------------------------------------------- dequant


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_dequant_int8_exhaustive_vs_torch(dt):
    rng = np.random.default_rng(11)
    q = np.tile(np.arange(-128, 128, dtype=np.int8), (300, 1))
    s = rng.uniform(1e-8, 0.5, size=(300, 1)).astype(np.float32)
    ours = qo.dequant_int8(q, s, dt)
    theirs = torch_ref.dequant_int8(torch.from_numpy(q), torch.from_numpy(s), TORCH_DT[dt]).float().numpy()
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("scale_dt", ["f32", "bf16"])
def test_dequant_int4_grouped_exhaustive_vs_torch(dt, scale_dt):
    rng = np.random.default_rng(12)
    k, g = 64, 16
    q = np.tile(np.arange(-8, 8, dtype=np.int8), (200, k // 16))
    p = qo.pack_int4(q)
    s = qo.round_to(rng.uniform(0.001, 0.05, size=(200, k // g)), scale_dt)
    ours = qo.dequant_int4(p, s, k, g, dt)
    ts = torch.from_numpy(s)
    if scale_dt == "bf16":
        ts = ts.to(torch.bfloat16)
    theirs = torch_ref.dequant_int4(torch.from_numpy(p), ts, k, g, TORCH_DT[dt]).float().numpy()
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))


def test_dequant_scale_is_rounded_before_the_product():
    # a scale that is not bf16-representable: round_bf16(q*s) != round_bf16(q*round_bf16(s))
    s = np.array([[np.float32(0.0123456)]], np.float32)
    q = np.arange(-128, 128, dtype=np.int8).reshape(1, -1)
    ours = qo.dequant_int8(q, s, "bf16")
    wrong = qo.round_bf16(q.astype(np.float32) * s)
    assert not np.array_equal(ours, wrong)
    assert np.array_equal(ours, qo.round_bf16(q.astype(np.float32) * qo.round_bf16(s)))


def test_group_dequant_reduces_to_per_channel():
    rng = np.random.default_rng(13)
    q = rng.integers(-8, 8, size=(8, 256)).astype(np.int8)
    p = qo.pack_int4(q)
    s = rng.uniform(0.001, 0.05, size=(8, 1)).astype(np.float32)
    a = qo.dequant_int4(p, s, 256, None, "bf16")
    b = qo.dequant_int4(p, np.repeat(s, 2, axis=1), 256, 128, "bf16")
    assert np.array_equal(a, b)


# ----------------------------------------------------------------------------- linear


def test_linear_closed_forms():
    rng = np.random.default_rng(14)
    w = qo.round_bf16(rng.standard_normal((24, 40)).astype(np.float32))
    # one-hot rows of x pick out columns of W^T exactly
    x = np.eye(40, dtype=np.float32)[:5]
    y = qo.linear(x, w, None, "f32")
    assert np.array_equal(y, w[:, :5].T)
    # identity weight returns x (+ bias); bias is rounded to T first
    xi = qo.round_bf16(rng.standard_normal((3, 40)).astype(np.float32))
    b = np.full(40, 0.1, np.float32)
    y2 = qo.linear(xi, np.eye(40, dtype=np.float32), b, "bf16")
    assert np.array_equal(y2, qo.round_bf16(xi.astype(np.float64) + float(qo.round_bf16(b)[0])))


def test_linear_vs_torch_cpu_gemm():
    g = torch.Generator().manual_seed(15)
    x = torch.randn(7, 96, generator=g)
    w = torch.randn(33, 96, generator=g)
    b = torch.randn(33, generator=g)
    ours = qo.linear(x.numpy(), w.numpy(), b.numpy(), "f32")
    theirs = F.linear(x.double(), w.double(), b.double()).float().numpy()
    assert qo.rel_err(ours, theirs) < 1e-6
    # a transposed operand is caught
    bad = qo.linear(x.numpy(), w.numpy()[::-1], b.numpy(), "f32")
    assert qo.rel_err(bad, theirs) > 1e-2


def test_rel_err_convention():
    assert qo.rel_err([1.0, 2.0], [1.0, 2.0]) == 0.0
    assert qo.rel_err([1.0, 2.1], [1.0, 2.0]) == pytest.approx(0.05)


# ----------------------------------------------------------------------------- golden


def _golden():
    return np.load(GOLDEN, allow_pickle=False)


GOLDEN_CASES = ["int8_pc", "int4_pc_oddk", "int4_g16", "int4_g128", "int8_k256", "int4_pc_k128"]


@pytest.mark.parametrize("name", GOLDEN_CASES)
@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
def test_oracle_matches_exact_golden(name, dt):
    z = _golden()
    n, k, g = (int(v) for v in z[f"{name}/meta"])
    g = None if g < 0 else g
    q = z[f"{name}/q"]
    s = z[f"{name}/scale"]
    if name.startswith("int8"):
        w = qo.dequant_int8(q, s, dt)
    else:
        w = qo.dequant_int4(qo.pack_int4(q), s, k, g, dt)
    assert np.array_equal(w.view(np.uint32), z[f"{name}/w_{dt}"].view(np.uint32))
    x_t = qo.round_to(z[f"{name}/x"], dt)
    assert np.array_equal(x_t, z[f"{name}/x_{dt}"])
    y = qo.linear_f64(x_t, w, z[f"{name}/bias"], dt)
    assert np.max(np.abs(y - z[f"{name}/y_{dt}_exact"])) < 1e-9
    yr = qo.linear(x_t, w, z[f"{name}/bias"], dt)
    # float64 sums can straddle a rounding boundary of T only at exact-ties; none here
    assert np.array_equal(yr, z[f"{name}/y_{dt}"])


# ----------------------------------------------------------------------------- W8A8


def test_act_quant_known_answers():
    # a row whose max|x| is 127 has scale 1 in every type, so x_q = round_half_even(x)
    x = np.array([[127.0, 2.5, -2.5, 3.5, -0.5, 0.5, 1.5, -126.5]], np.float32)
    for dt in ("bf16", "f16", "f32"):
        q, s = qo.act_quant_i8(x, dt)
        assert s[0, 0] == 1.0
        assert q[0].tolist() == [127, 2, -2, 4, 0, 0, 2, -126]
    # zero rows take the clamp bound 1e-8 converted to T; fp16 has none (0), so x_q is
    # 0 / 0 -> 0
    z = np.zeros((2, 5), np.float32)
    assert qo.act_scale_i8(z, "bf16")[0, 0] == torch.tensor(1e-8, dtype=torch.bfloat16).float().item()
    assert qo.act_scale_i8(z, "f32")[0, 0] == np.float32(1e-8)
    assert qo.act_scale_i8(z, "f16")[0, 0] == 0.0
    assert (qo.act_quant_i8(z, "f16")[0] == 0).all()
    # a fp16 row too small for a nonzero scale: nonzero x -> +-inf -> clamped
    t = np.array([[6e-8, -6e-8, 0.0]], np.float32)
    q, s = qo.act_quant_i8(qo.round_f16(t), "f16")
    assert s[0, 0] == 0.0 and q[0].tolist() == [127, -128, 0]


def test_act_scale_uses_the_fp32_reciprocal():
    # 1/127 rounded to fp32 and the product rounded to fp32, then to T (known answers
    # worked in exact rational arithmetic)
    from fractions import Fraction

    rcp = np.float32(1.0) / np.float32(127.0)
    assert Fraction(float(rcp)) != Fraction(1, 127)
    rng = np.random.default_rng(11)
    mx = rng.uniform(1e-3, 1e3, size=2000).astype(np.float32)
    got = qo.act_scale_i8(mx.reshape(-1, 1), "f32")[:, 0]
    for m, g in zip(mx[:200], got[:200]):
        exact = Fraction(float(m)) * Fraction(float(rcp))
        assert Fraction(float(g)) == Fraction(float(np.float32(float(exact))))  # nearest fp32
    # the two evaluation orders differ on a visible share of fp32 inputs
    div = (mx / np.float32(127.0)).astype(np.float32)
    assert np.count_nonzero(div != got) > 20


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_act_quant_matches_torch_ops_given_the_scale(dt):
    # :413-414 with torch's own CPU ops: max|x| and the quantization step from the scale
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal((37, 300)).astype(np.float32) * 3).to(TORCH_DT[dt])
    x32 = x.float().numpy()
    xq, s = qo.act_quant_i8(x32, dt)
    mx = torch.max(torch.abs(x), dim=-1, keepdim=True)[0].float().numpy()
    np.testing.assert_array_equal(np.max(np.abs(x32), axis=-1, keepdims=True), mx)
    ref = torch.clamp(torch.round(x.float() / torch.from_numpy(s)), -128, 127).to(torch.int8)
    np.testing.assert_array_equal(xq, ref.numpy())
    # torch's CPU division by the scalar is a true division; on this sample it gives the
    # same scales as the GPU's reciprocal product (the order is pinned on the GPU)
    if dt != "f32":
        st = torch.clamp(torch.max(torch.abs(x), dim=-1, keepdim=True)[0] / 127.0, min=1e-8).float()
        np.testing.assert_array_equal(s, st.numpy())


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("with_bias", [False, True])
def test_w8a8_linear_matches_int_mm_and_torch_epilogue(dt, with_bias):
    # steps 6-11 of Int8GEMMLinear.forward (quantization.py:416-447) with torch's CPU
    # torch._int_mm and elementwise ops, from the oracle's x_q / scale_x
    rng = np.random.default_rng(5)
    m, k, n = 37, 96, 40
    x = qo.round_to(rng.standard_normal((m, k)).astype(np.float32) * 2, dt)
    w = rng.integers(-128, 128, size=(n, k)).astype(np.int8)
    sw = rng.uniform(1e-3, 2e-2, size=n).astype(np.float32)
    bias = qo.round_to(rng.standard_normal(n).astype(np.float32), dt) if with_bias else None
    y = qo.w8a8_linear(x, w, sw, bias, dt)
    xq, sx = qo.act_quant_i8(x, dt)
    xp = torch.nn.functional.pad(torch.from_numpy(xq), (0, 0, 0, 32 - m % 32))
    acc = torch._int_mm(xp, torch.from_numpy(np.ascontiguousarray(w.T)))[:m]
    out = acc.float() * (torch.from_numpy(sx) * torch.from_numpy(sw).reshape(1, -1))
    if with_bias:
        out = out + torch.from_numpy(bias).to(TORCH_DT[dt]).float()
    ref = out.to(TORCH_DT[dt]).float().numpy()
    np.testing.assert_array_equal(y, ref)


def test_w8a8_linear_closed_form():
    # w = 3 I, scale_w = 0.5, rows with max|x| = 127 (scale 1): y = round_T(3 x_q * 0.5 + b)
    k = 16
    x = np.tile(np.arange(-7, 9, dtype=np.float32) * 15.875, (3, 1))
    x[:, 0] = 127.0
    w = (3 * np.eye(k)).astype(np.int8)
    b = np.linspace(-1, 1, k).astype(np.float32)
    y = qo.w8a8_linear(x, w, np.full(k, 0.5, np.float32), qo.round_bf16(b), "bf16")
    xq = np.rint(x).clip(-128, 127)
    np.testing.assert_array_equal(y, qo.round_bf16(xq * 1.5 + qo.round_bf16(b)))


# ----------------------------------------------------------------------------- SiLU.mul


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_silu_mul_matches_torch_ops(dt):
    rng = np.random.default_rng(8)
    g = qo.round_to(rng.standard_normal(20000).astype(np.float32) * 4, dt)
    u = qo.round_to(rng.standard_normal(20000).astype(np.float32) * 2, dt)
    ours = qo.silu_mul(g, u, dt)
    gt = torch.from_numpy(g).to(TORCH_DT[dt])
    ut = torch.from_numpy(u).to(TORCH_DT[dt])
    ref = (F.silu(gt) * ut).float().numpy()
    # exp is correctly rounded in neither library: a rare last-place difference in fp32 may
    # move a T rounding; everything else is the same op order
    rel = np.abs(ours - ref) / np.maximum(np.abs(ref), 1e-6)
    if dt == "f32":
        assert np.max(rel) < 2.0 ** -20  # a few fp32 ulps
    else:
        assert np.mean(ours == ref) > 0.999
        assert np.max(rel) < 2.0 ** -7   # at most one ulp of T
    # closed forms: silu(0) = 0, silu(g) -> g for large g, -> -0 for very negative g
    assert qo.silu_mul(np.float32([0.0]), np.float32([3.0]), dt)[0] == 0.0
    assert qo.silu_mul(np.float32([60.0]), np.float32([0.5]), dt)[0] == 30.0
    assert qo.silu_mul(np.float32([-200.0]), np.float32([1.0]), dt)[0] == 0.0


# ----------------------------------------------------------------------------- paged attention


def _paged_case(rng, b, h, hkv, d, bs, nblk, seqs, int8):
    nb = b * nblk + 3
    perm = rng.permutation(nb)[: b * nblk].reshape(b, nblk)  # scattered physical blocks
    if int8:
        kp = rng.integers(-128, 128, size=(nb, bs, hkv, d)).astype(np.int8)
        vp = rng.integers(-128, 128, size=(nb, bs, hkv, d)).astype(np.int8)
        ks = qo.round_f16(rng.uniform(0.002, 0.02, size=(nb, bs, hkv)).astype(np.float32))
        vs = qo.round_f16(rng.uniform(0.002, 0.02, size=(nb, bs, hkv)).astype(np.float32))
    else:
        kp = qo.round_f16(rng.standard_normal((nb, bs, hkv, d)).astype(np.float32))
        vp = qo.round_f16(rng.standard_normal((nb, bs, hkv, d)).astype(np.float32))
        ks = vs = None
    q = qo.round_f16(rng.standard_normal((b, h, d)).astype(np.float32))
    return q, kp, vp, ks, vs, perm, np.array(seqs, dtype=np.int64)


@pytest.mark.parametrize("int8", [False, True])
@pytest.mark.parametrize("mapping", ["contiguous", "interleaved"])
def test_paged_attention_matches_torch_sdpa_on_gathered_tensors(int8, mapping):
    # the reference's ground truth: gather the blocks, dequantize, expand heads, SDPA
    rng = np.random.default_rng(4)
    b, h, hkv, d, bs = 3, 6, 2, 64, 16
    q, kp, vp, ks, vs, bt, seqs = _paged_case(rng, b, h, hkv, d, bs, 5, [38, 80, 1], int8)
    ours = qo.paged_attention(q, kp, vp, bt, seqs, bs, "f16", ks, vs, mapping)
    g = h // hkv
    for bb in range(b):
        n = int(seqs[bb])
        blk, off = bt[bb][np.arange(n) // bs], np.arange(n) % bs
        k = torch.from_numpy(kp[blk, off].astype(np.float32))
        v = torch.from_numpy(vp[blk, off].astype(np.float32))
        if int8:
            k = (k.half() * torch.from_numpy(ks[blk, off])[..., None].half()).float()
            v = (v.half() * torch.from_numpy(vs[blk, off])[..., None].half()).float()
        for hh in range(h):
            kvh = hh // g if mapping == "contiguous" else hh % hkv
            qq = torch.from_numpy(q[bb, hh]).view(1, 1, 1, d)
            ref = F.scaled_dot_product_attention(qq, k[:, kvh].view(1, 1, n, d), v[:, kvh].view(1, 1, n, d))
            ref = ref.half().float().view(d).numpy()
            assert np.max(np.abs(ours[bb, hh] - ref)) <= 2e-3 * max(1.0, np.max(np.abs(ref)))


def test_paged_attention_closed_forms():
    rng = np.random.default_rng(5)
    b, h, hkv, d, bs = 1, 2, 1, 64, 4
    q, kp, vp, _, _, bt, _ = _paged_case(rng, b, h, hkv, d, bs, 3, [10], False)
    kp[:] = qo.round_f16(np.float32(0.25))  # equal scores: output = mean of the values
    out = qo.paged_attention(q, kp, vp, bt, np.array([10]), bs, "f32")
    ts = np.arange(10)
    vals = vp[bt[0][ts // bs], ts % bs, 0].astype(np.float64)
    np.testing.assert_allclose(out[0, 0], vals.mean(axis=0), rtol=1e-5, atol=1e-6)
    # one key aligned with q and large: the output is that token's value
    kp[:] = 0
    kp[bt[0][1], 3, 0] = q[0, 1] * 50
    out = qo.paged_attention(q, kp, vp, bt, np.array([10]), bs, "f32")
    np.testing.assert_allclose(out[0, 1], vp[bt[0][1], 3, 0], rtol=1e-4, atol=1e-5)
    # a mask that hides everything past token 4 equals seq_len 5
    mask = np.zeros((1, 10), dtype=bool)
    mask[0, :5] = True
    a = qo.paged_attention(q, kp, vp, bt, np.array([10]), bs, "f32", mask=mask, max_sl=10)
    bb = qo.paged_attention(q, kp, vp, bt, np.array([5]), bs, "f32", max_sl=5)
    np.testing.assert_array_equal(a, bb)
