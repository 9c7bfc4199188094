"""Host-side tests (no GPU): loader routing and accounting, quantizer parity with the
oracle, error behaviour, and the C ABI of liblsq.so (loads, exports every declared
symbol, rejects bad arguments before touching the GPU).

Mirrors the offline tier of the reference's tests/test_quantized_loader.py (routing
:125-180, placement :185-206, invalid modes :360-372, failure cleanup :377-388, 'none'
mode :393-407, mocked from_pretrained :412-433, unsupported architecture :468-486,
trust_remote_code :491-507).
"""

import ctypes
import os
import re
from unittest.mock import MagicMock, patch

import numpy as np
import pytest
import torch
import torch.nn as nn

from localstrm_amd import (
    CachedQuantizedLinear,
    Int8GEMMLinear,
    QuantizedLinear,
    apply_optional_quantization,
    can_use_int8_gemm,
    load_and_quantize_model,
)
from localstrm_amd import _lib
from oracle import quant_oracle as qo
from tests.synthetic import seeded_model

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "localstrm_amd.h")
PROJS = ("q_proj", "k_proj", "v_proj", "o_proj")
MLPS = ("gate_proj", "up_proj", "down_proj")


# ----------------------------------------------------------------------------- loader


@pytest.mark.parametrize("mode,min_savings", [("int8", 30.0), ("int4", 50.0)])
def test_cpu_staged_loading_routes_all_projections(mode, min_savings):
    model, orig, quant = load_and_quantize_model(seeded_model(), device="cpu", quantization=mode)
    for layer in model.model.layers:
        for p in PROJS:
            m = getattr(layer.self_attn, p)
            assert isinstance(m, QuantizedLinear) and m.quant_type == mode
        for p in MLPS:
            assert isinstance(getattr(layer.mlp, p), QuantizedLinear)
        q = layer.self_attn.q_proj
        if mode == "int8":
            assert q.weight_q.dtype == torch.int8 and q.weight_q.shape == (64, 64)
        else:
            assert q.weight_packed.dtype == torch.uint8
            assert q.weight_packed.shape == (q.out_features, (q.in_features + 1) // 2)
    assert not isinstance(model.lm_head, QuantizedLinear)
    assert (1.0 - quant / orig) * 100 > min_savings


def test_group_wise_loading_and_accounting():
    model, orig, quant = load_and_quantize_model(
        seeded_model(), device="cpu", quantization="int4", group_size=32
    )
    q = model.model.layers[0].mlp.down_proj  # in_features 128 -> 4 groups
    assert q.group_size == 32 and q.scale.shape == (64, 4) and q.scale.dtype == torch.bfloat16
    assert quant < orig


def test_cpu_device_placement():
    model, _, _ = load_and_quantize_model(seeded_model(), device="cpu", quantization="int8")
    assert all(p.device.type == "cpu" for p in model.parameters())
    assert all(b.device.type == "cpu" for b in model.buffers())


def test_invalid_modes():
    model = seeded_model()
    for mode in ["int16", "fp8", "awq", "gptq", "unknown_mode", "123"]:
        with pytest.raises(ValueError, match="Invalid quantization mode"):
            load_and_quantize_model(model, device="cpu", quantization=mode)
        with pytest.raises(ValueError, match="Invalid quantization type"):
            apply_optional_quantization(model, quant_type=mode)


def test_failure_cleanup():
    model = seeded_model()
    with patch("localstrm_amd.quantization.apply_optional_quantization",
               side_effect=RuntimeError("Simulated OOM")):
        with patch("torch.cuda.empty_cache") as empty:
            with pytest.raises(RuntimeError, match="Simulated OOM"):
                load_and_quantize_model(model, device="cpu", quantization="int8")
            if torch.cuda.is_available():
                empty.assert_called()


def test_none_mode_unchanged():
    model, orig, quant = load_and_quantize_model(seeded_model(), device="cpu", quantization="none")
    assert orig == quant
    assert type(model.model.layers[0].self_attn.q_proj) is nn.Linear


def test_mocked_from_pretrained_stages_on_cpu():
    mock_model = seeded_model()
    mock_model.to = MagicMock(return_value=mock_model)
    with patch("transformers.AutoModelForCausalLM.from_pretrained", return_value=mock_model) as fp:
        target = torch.device("cuda")
        load_and_quantize_model("mock/model", device=target, quantization="int8")
        fp.assert_called_once()
        mock_model.to.assert_any_call("cpu")
        mock_model.to.assert_any_call(target)


@pytest.mark.parametrize("mode", ["int8", "int4", "hybrid_int8"])
def test_unsupported_architecture(mode):
    seq = nn.Sequential(nn.Linear(64, 128), nn.ReLU(), nn.Linear(128, 64))
    with pytest.raises(ValueError) as ei:
        apply_optional_quantization(seq, quant_type=mode)
    msg = str(ei.value)
    assert f"Quantization '{mode}' failed" in msg
    assert "no compatible linear layers found" in msg
    assert "Supported architectures require transformer blocks" in msg


def test_hybrid_int8_routing_and_accounting():
    # tests/test_hybrid_int8.py:170-192 of the reference
    model = seeded_model()
    orig, quant = apply_optional_quantization(model, quant_type="hybrid_int8")
    for layer in model.model.layers:
        for p in PROJS:
            m = getattr(layer.self_attn, p)
            assert isinstance(m, CachedQuantizedLinear) and m.weight.dtype == torch.float32
        for p in MLPS:
            m = getattr(layer.mlp, p)
            assert isinstance(m, Int8GEMMLinear)
            assert m.weight_q_t.shape == (m.in_features, m.out_features)
            assert m.scale_w_t.shape == (1, m.out_features)
    assert quant < orig and 0.40 < quant / orig < 0.70


def test_hybrid_int8_unaligned_mlp_falls_back_to_int8(caplog):
    # tests/test_hybrid_int8.py:197-225: MLP dims not divisible by 8 -> QuantizedLinear int8
    class OddMlp(nn.Module):
        def __init__(self):
            super().__init__()
            self.gate_proj = nn.Linear(63, 127)
            self.up_proj = nn.Linear(63, 127)
            self.down_proj = nn.Linear(127, 63)

    class OddLayer(nn.Module):
        def __init__(self):
            super().__init__()
            self.self_attn = seeded_model().model.layers[0].self_attn
            self.mlp = OddMlp()

    class OddModel(nn.Module):
        def __init__(self):
            super().__init__()
            self.layers = nn.ModuleList([OddLayer()])

    m = OddModel()
    with caplog.at_level("WARNING", logger="mini_vllm.quantization"):
        apply_optional_quantization(m, quant_type="hybrid_int8")
    assert isinstance(m.layers[0].self_attn.q_proj, CachedQuantizedLinear)
    g = m.layers[0].mlp.gate_proj
    assert isinstance(g, QuantizedLinear) and g.quant_type == "int8"
    assert "not divisible by 8" in caplog.text


def test_cached_quantized_linear_matches_reference_steps():
    # quantization.py:212-240 and :264-276, a dense layer once built (runs on the CPU)
    lin = _linear(128, 64, 3)
    c = CachedQuantizedLinear.from_float(lin, dtype=torch.float32)
    q, s = qo.quantize_int8(lin.weight.detach().numpy())
    np.testing.assert_array_equal(c.weight.numpy(), q.astype(np.float32) * s)
    x = torch.randn(4, 16, 64)
    ref = lin(x)
    out = c(x)
    cos = torch.nn.functional.cosine_similarity(ref.flatten(), out.flatten(), dim=0).item()
    assert cos > 0.99
    assert c.memory_footprint_bytes() == 128 * 64 * 4 + 128 * 4
    c16 = CachedQuantizedLinear.from_quantized(torch.from_numpy(q), torch.from_numpy(s), lin.bias.detach())
    assert c16.weight.dtype == torch.float16
    np.testing.assert_array_equal(c16.weight.float().numpy(), qo.round_f16(q.astype(np.float32) * s))


def test_int8_gemm_linear_buffers_and_no_cpu_path(monkeypatch):
    lin = _linear(48, 64, 4)
    m = Int8GEMMLinear.from_float(lin, dtype=torch.float32)
    assert set(m.state_dict().keys()) == {"weight_q_t", "scale_w_t", "bias"}
    q, s = qo.quantize_int8(lin.weight.detach().numpy())
    np.testing.assert_array_equal(m.weight_q_t.numpy(), q.T)
    np.testing.assert_array_equal(m.scale_w_t.numpy(), s.T)
    assert m.dequantize().dtype == torch.float32
    with pytest.raises(RuntimeError, match="Int8GEMMLinear.forward: .* GPU only"):
        m(torch.randn(2, 64))
    # the kill switch takes the fallback (which, like every path here, needs a GPU)
    monkeypatch.setenv("MINIVLLM_DISABLE_INT8_GEMM", "1")
    ok, why = can_use_int8_gemm()
    assert not ok and "MINIVLLM_DISABLE_INT8_GEMM" in why
    with pytest.raises(RuntimeError, match="GPU only"):
        m(torch.randn(1, 1, 64))
    assert m._warned_fallback
    monkeypatch.delenv("MINIVLLM_DISABLE_INT8_GEMM")
    if not torch.cuda.is_available():
        assert can_use_int8_gemm()[0] is False
    assert can_use_int8_gemm("cpu")[0] is False or not torch.cuda.is_available()
    mq = Int8GEMMLinear.from_quantized(torch.from_numpy(q), torch.from_numpy(s), dtype=torch.bfloat16)
    np.testing.assert_array_equal(mq.weight_q_t.numpy(), q.T)
    assert mq.bias is None and mq.output_dtype == torch.bfloat16


def test_load_and_quantize_synthetic_hybrid():
    # tests/test_hybrid_int8.py:339-352
    model, orig, quant = load_and_quantize_model(seeded_model(), device="cpu", quantization="hybrid_int8")
    assert isinstance(model.model.layers[0].self_attn.q_proj, CachedQuantizedLinear)
    assert isinstance(model.model.layers[0].mlp.gate_proj, Int8GEMMLinear)
    assert quant < orig


@pytest.mark.parametrize("flag", [True, False])
def test_trust_remote_code_pass_through(flag):
    with patch("transformers.AutoModelForCausalLM.from_pretrained", return_value=seeded_model()) as fp:
        load_and_quantize_model("custom/model-id", device="cpu", quantization="none",
                                trust_remote_code=flag)
        fp.assert_called_once()
        assert fp.call_args[1].get("trust_remote_code") is flag


# ----------------------------------------------------------------------------- quantizer parity


def _linear(n, k, seed, bias=True):
    torch.manual_seed(seed)
    return nn.Linear(k, n, bias=bias)


@pytest.mark.parametrize("k", [32, 33, 128, 1536])
def test_from_float_int4_matches_oracle(k):
    lin = _linear(64, k, k)
    ql = QuantizedLinear.from_float(lin, "int4")
    p, s = qo.quantize_int4(lin.weight.detach().numpy())
    assert np.array_equal(ql.weight_packed.numpy(), p)
    assert np.array_equal(ql.scale.numpy(), s)
    assert ql.weight_packed.shape == (64, (k + 1) // 2)


@pytest.mark.parametrize("shape", [(32, 32), (64, 32), (32, 64), (128, 64), (64, 128), (4864, 896)])
def test_from_float_int8_matches_oracle(shape):
    n, k = shape
    lin = _linear(n, k, n + k)
    ql = QuantizedLinear.from_float(lin, "int8")
    q, s = qo.quantize_int8(lin.weight.detach().numpy())
    assert np.array_equal(ql.weight_q.numpy(), q) and np.array_equal(ql.scale.numpy(), s)


@pytest.mark.parametrize("group,sdt", [(128, torch.bfloat16), (64, torch.float32), (100, torch.bfloat16)])
def test_from_float_int4_grouped_matches_oracle(group, sdt):
    lin = _linear(48, 384, group)
    ql = QuantizedLinear.from_float(lin, "int4", group_size=group, scale_dtype=sdt)
    p, s = qo.quantize_int4(lin.weight.detach().numpy(), group_size=group,
                            scale_dt="bf16" if sdt == torch.bfloat16 else "f32")
    assert ql.scale.dtype == sdt
    assert np.array_equal(ql.weight_packed.numpy(), p)
    assert np.array_equal(ql.scale.float().numpy(), s)


def test_from_quantized_validates_shapes():
    w = torch.zeros(8, 16, dtype=torch.uint8)
    ql = QuantizedLinear.from_quantized(w, torch.ones(8, 1), quant_type="int4")
    assert ql.in_features == 32 and ql.scale.shape == (8, 1)
    ql = QuantizedLinear.from_quantized(w, torch.ones(8, 2, dtype=torch.bfloat16), quant_type="int4",
                                        in_features=31, group_size=16)
    assert ql.in_features == 31 and ql.group_size == 16
    with pytest.raises(ValueError):
        QuantizedLinear.from_quantized(w, torch.ones(8, 3), quant_type="int4", group_size=16)
    with pytest.raises(ValueError):
        QuantizedLinear.from_quantized(w, torch.ones(8, 1), quant_type="int4", in_features=40)
    q8 = QuantizedLinear.from_quantized(torch.zeros(8, 16, dtype=torch.int8), torch.ones(8),
                                        bias=torch.zeros(8), quant_type="int8")
    assert q8.scale.shape == (8, 1) and q8.bias is not None


def test_state_dict_matches_reference_buffers():
    ql = QuantizedLinear.from_float(_linear(16, 64, 0), "int4")
    assert set(ql.state_dict().keys()) == {"weight_packed", "scale", "bias"}
    q8 = QuantizedLinear.from_float(_linear(16, 64, 0, bias=False), "int8")
    assert set(q8.state_dict().keys()) == {"weight_q", "scale"}


def test_unknown_quant_type_is_float_layer():
    ql = QuantizedLinear(8, 4, quant_type="fp8")
    assert isinstance(ql.weight, nn.Parameter) and ql.weight.shape == (4, 8)


# ----------------------------------------------------------------------------- no CPU path


def test_cpu_forward_and_dequantize_raise():
    for mode in ("int8", "int4"):
        ql = QuantizedLinear.from_float(_linear(16, 32, 1), mode)
        with pytest.raises(RuntimeError, match="GPU only"):
            ql(torch.randn(2, 32))
        with pytest.raises(RuntimeError, match="GPU only"):
            ql.dequantize()


# ----------------------------------------------------------------------------- C ABI


def _declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(lsq_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_what_the_binding_binds():
    assert _declared_symbols() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_symbols():
        assert hasattr(lib, name), name
    assert lib.lsq_version() >= 100


def test_library_rejects_bad_arguments_without_gpu():
    lib = _lib.load()
    # NULL pointers and bad shapes/dtypes are rejected before any HIP call
    assert lib.lsq_w8_linear(None, 16, None, None, None, 0, None, 0, None, 16, 2, 1, 16, 16, None) == -1
    assert lib.lsq_w4_linear(1 << 20, 8, 1 << 20, None, 1 << 20, 0, 128, None, 0, 1 << 20, 16, 2,
                             1, 16, 16, None) == -2  # ldx < K
    assert lib.lsq_w4_linear(1 << 20, 16, 1 << 20, None, 1 << 20, 0, 0, None, 0, 1 << 20, 16, 2,
                             1, 16, 16, None) == -4  # group_size 0
    assert lib.lsq_w4_linear(1 << 20, 16, 1 << 20, None, 1 << 20, 0, 16, None, 0, 1 << 20, 16, 7,
                             1, 16, 16, None) == -3  # dtype 7
    assert lib.lsq_w4_retile(1 << 20, 1 << 20, 16, 100, None) == -5  # K % 128 != 0
    # an empty batch (M = 0) may carry NULL x / y, as torch gives for zero-element tensors
    assert lib.lsq_w4_linear(None, 16, 1 << 20, None, 1 << 20, 0, 16, None, 0, None, 16, 2,
                             0, 16, 16, None) == 0
    assert lib.lsq_w8_linear(None, 16, 1 << 20, None, 1 << 20, 0, None, 0, None, 16, 2, 0, 16,
                             16, None) == 0
    assert lib.lsq_w8_linear(None, 16, 1 << 20, None, 1 << 20, 0, None, 0, 1 << 20, 16, 2, 1, 16,
                             16, None) == -1  # M > 0 needs x
    assert lib.lsq_w8_linear(1 << 20, 128, 1 << 20, (1 << 20) + 8, 1 << 20, 0, None, 0, 1 << 20,
                             16, 2, 1, 16, 128, None) == -6  # tiled copy not 16-byte aligned
    # the quantizer: shapes, dtypes, missing outputs and layouts before any HIP call
    assert lib.lsq_quantize_w8(1 << 20, 2, 8, 16, 16, 1 << 20, 1 << 20, None, None) == -2  # ldw < K
    assert lib.lsq_quantize_w8(1 << 20, 3, 16, 16, 16, 1 << 20, 1 << 20, None, None) == -3  # int8 input
    assert lib.lsq_quantize_w8(1 << 20, 2, 16, 16, 16, 1 << 20, None, None, None) == -1  # no output
    assert lib.lsq_quantize_w8(1 << 20, 2, 100, 16, 100, 1 << 20, None, 1 << 20, None) == -5  # tiled, K % 128
    assert lib.lsq_quantize_w4(1 << 20, 2, 16, 16, 16, -1, 1 << 20, 0, 1 << 20, None, None) == -4
    assert lib.lsq_quantize_w4(1 << 20, 2, 16, 16, 16, 0, 1 << 20, 2, 1 << 20, None, None) == -3  # per channel: fp32
    assert lib.lsq_quantize_w4(1 << 20, 2, 256, 16, 256, 12, 1 << 20, 2, None, 1 << 20, None) == -5  # group % 8
    assert lib.lsq_quantize_w4(None, 2, 16, 0, 16, 0, None, 0, None, None, None) == 0  # N = 0: nothing to do
    # measurement probes: sizes and launch shapes are checked before any HIP call
    assert lib.lsq_probe_read(1 << 20, 0, 1 << 20, 256, 512, None) == -2
    assert lib.lsq_probe_read(1 << 20, 1 << 31, 1 << 20, 256, 512, None) == -2
    assert lib.lsq_probe_read(1 << 20, 4096, 1 << 20, 256, 96, None) == -2
    assert lib.lsq_probe_read(None, 4096, 1 << 20, 256, 512, None) == -1
    # the allocation-free W8A8 entry point refuses what its fixed scratch cannot hold
    # (2047 rows x 4096 int8 + 2047 fp32 scales > 8 MiB), before any HIP call
    assert lib.lsq_w8a8_linear_noalloc(None, 4096, None, None, 0, None, 0, None, 64, 2, 2047, 64,
                                       4096, None) == -7
    assert lib.lsq_w8a8_linear_noalloc(None, 4096, None, None, 0, None, 0, None, 64, 2, 2046, 64,
                                       4096, None) == -1  # fits: then the NULL pointers
    assert lib.lsq_w8_retile(1 << 20, 1 << 20, 16, 100, None) == -5
    assert lib.lsq_w8_tiled_bytes(18944, 3584) == 18944 * 3584
    assert lib.lsq_w8_tiled_bytes(17, 128) == 2 * 2048
    assert lib.lsq_w4_tiled_bytes(18944, 3584) == 18944 * 3584 // 2
    assert lib.lsq_w4_tiled_bytes(17, 128) == 2 * 1024  # rows padded to 16
    assert lib.lsq_w4_tiled_bytes(16, 100) == 0
    # W8A8 entry points
    assert lib.lsq_w8a8_tiled_bytes(18944, 3584) == 18944 * 3584
    assert lib.lsq_w8a8_tiled_bytes(17, 64) == 32 * 128  # rows to 16, K to 128
    assert lib.lsq_w8a8_tiled_bytes(0, 64) == 0
    assert lib.lsq_act_quant_i8(1 << 20, 16, 2, 1, 32, 1 << 20, 32, 1 << 20, None) == -2  # ldx < K
    assert lib.lsq_act_quant_i8(1 << 20, 32, 5, 1, 32, 1 << 20, 32, 1 << 20, None) == -3
    assert lib.lsq_act_quant_i8(None, 32, 2, 1, 32, 1 << 20, 32, 1 << 20, None) == -1
    assert lib.lsq_act_quant_i8(None, 32, 2, 0, 32, None, 32, None, None) == 0  # M = 0
    args = [1 << 20, 64, 1 << 20, 1 << 20, 0, None, 0, 1 << 20, 64, 2, 1, 64, 64, 1 << 20, 1 << 20, None]
    assert lib.lsq_w8a8_linear(*args[:12], 0, *args[13:]) == -2  # K = 0
    bad = list(args)
    bad[13] = (1 << 20) + 8
    assert lib.lsq_w8a8_linear(*bad) == -6  # x_q workspace not 16-byte aligned
    bad = list(args)
    bad[14] = None
    assert lib.lsq_w8a8_linear(*bad) == -1
    bad = list(args)
    bad[4] = 9
    assert lib.lsq_w8a8_linear(*bad) == -3
    assert lib.lsq_w8a8_linear(*args[:10], 0, *args[11:]) == 0  # M = 0
    # the workspace form: a misaligned workspace is refused before any HIP call; its size
    # (host arithmetic only): S x M x N int32 sums where the 64 x 128 tiles are few and K long
    assert lib.lsq_w8a8_linear_ws(*args[:15], (1 << 20) + 4, 4096, None) == -6
    assert lib.lsq_w8a8_linear_ws(*args[:10], 0, *args[11:15], None, 0, None) == 0  # M = 0
    assert lib.lsq_w8a8_workspace_bytes(64, 3584, 18944) == 9 * 64 * 3584 * 4
    assert lib.lsq_w8a8_workspace_bytes(16, 384, 18944) == 16 * 16 * 384 * 4
    assert lib.lsq_w8a8_workspace_bytes(64, 18944, 3584) == 0  # 148 tiles
    assert lib.lsq_w8a8_workspace_bytes(256, 3584, 18944) == 16 * 256 * 3584 * 4  # 14 large tiles
    assert lib.lsq_w8a8_workspace_bytes(2048, 3584, 18944) == 2 * 2048 * 3584 * 4  # 112 large tiles
    assert lib.lsq_w8a8_workspace_bytes(2048, 14336, 4096) == 0  # 448 large tiles
    assert lib.lsq_w8a8_workspace_bytes(64, 3584, 1024) == 0  # 8 k tiles
    assert lib.lsq_w8a8_workspace_bytes(0, 3584, 18944) == 0
    for code in (-1, -2, -3, -4, -5, -6):
        assert lib.lsq_status_string(code).startswith(b"lsq:")
    with pytest.raises(_lib.LsqError, match="group_size"):
        _lib.check(-4, "probe")


def test_fuse_linears_silu_mul_interleaves_gate_and_up():
    from localstrm_amd import fuse_linears

    gate = QuantizedLinear.from_float(_linear(48, 64, 11, bias=False), "int8")
    up = QuantizedLinear.from_float(_linear(48, 64, 12, bias=True), "int8")
    f = fuse_linears([gate, up], act="silu_mul")
    assert f.out_features == 48 and f.fused.out_features == 96 and f.act == "silu_mul"
    w = f.fused.weight_q
    for t in range(3):
        assert torch.equal(w[32 * t:32 * t + 16], gate.weight_q[16 * t:16 * t + 16])
        assert torch.equal(w[32 * t + 16:32 * t + 32], up.weight_q[16 * t:16 * t + 16])
    assert torch.equal(f.fused.bias.detach()[16:32], up.bias.detach()[:16])
    assert (f.fused.bias.detach()[:16] == 0).all()
    with pytest.raises(ValueError, match="gate_proj, up_proj"):
        fuse_linears([gate, up, up], act="silu_mul")
    odd = QuantizedLinear.from_float(_linear(40, 64, 13), "int8")
    with pytest.raises(ValueError, match="% 16"):
        fuse_linears([odd, odd], act="silu_mul")
    with pytest.raises(ValueError, match="act"):
        fuse_linears([gate, up], act="gelu")


def test_fuse_linears_concatenates_and_validates():
    """fuse_linears builds one layer whose rows are the layers' rows in order (CPU side:
    construction only, no kernel call)."""
    import torch.nn as nn
    from localstrm_amd import QuantizedLinear, fuse_linears

    torch.manual_seed(0)
    q = QuantizedLinear.from_float(nn.Linear(256, 64, bias=True), "int4", group_size=128)
    k = QuantizedLinear.from_float(nn.Linear(256, 16, bias=True), "int4", group_size=128)
    o = QuantizedLinear.from_float(nn.Linear(256, 32, bias=False), "int4", group_size=128)
    f = fuse_linears([q, k, o])
    assert f.splits == [64, 16, 32] and f.out_features == 112 and f.in_features == 256
    assert torch.equal(f.fused.weight_packed, torch.cat([q.weight_packed, k.weight_packed, o.weight_packed]))
    assert torch.equal(f.fused.scale, torch.cat([q.scale, k.scale, o.scale]))
    assert torch.equal(f.fused.bias.detach(), torch.cat([q.bias.detach(), k.bias.detach(), torch.zeros(32)]))
    w8 = [QuantizedLinear.from_float(nn.Linear(64, n), "int8") for n in (8, 24)]
    f8 = fuse_linears(w8)
    assert torch.equal(f8.fused.weight_q, torch.cat([w.weight_q for w in w8]))
    with pytest.raises(ValueError):
        fuse_linears([q, QuantizedLinear.from_float(nn.Linear(128, 8), "int4", group_size=64)])
    with pytest.raises(ValueError):
        fuse_linears([q, w8[0]])
    with pytest.raises(ValueError):
        fuse_linears([])


# ----------------------------------------------------------------------------- packed checkpoints


@pytest.mark.parametrize("mode,group", [("int8", None), ("int4", None), ("int4", 32), ("hybrid_int8", None)])
def test_packed_checkpoint_round_trip_cpu(tmp_path, mode, group):
    from localstrm_amd import load_packed, save_packed

    model = seeded_model()
    apply_optional_quantization(model, quant_type=mode, group_size=group)
    path = str(tmp_path / "packed.safetensors")
    n = save_packed(model, path)
    assert n == 2 * 7
    fresh = seeded_model(seed=7)  # float skeleton with other weights
    assert load_packed(fresh, path) == n
    sd_a, sd_b = model.state_dict(), fresh.state_dict()
    quant_keys = [k for k in sd_a if ".self_attn." in k or ".mlp." in k]
    for k in quant_keys:
        assert sd_a[k].dtype == sd_b[k].dtype and torch.equal(sd_a[k], sd_b[k]), k
    for la, lb in zip(model.model.layers, fresh.model.layers):
        for p in PROJS:
            assert type(getattr(la.self_attn, p)) is type(getattr(lb.self_attn, p))
        for p in MLPS:
            a, b = getattr(la.mlp, p), getattr(lb.mlp, p)
            assert type(a) is type(b)
            if isinstance(a, QuantizedLinear):
                assert (a.quant_type, a.group_size) == (b.quant_type, b.group_size)


def test_packed_checkpoint_rejects_foreign_files(tmp_path):
    from safetensors.torch import save_file

    from localstrm_amd import load_packed, save_packed

    path = str(tmp_path / "other.safetensors")
    save_file({"a": torch.zeros(2)}, path, metadata={"format": "something-else"})
    with pytest.raises(ValueError, match="not a localstrm_amd.packed file"):
        load_packed(seeded_model(), path)
    with pytest.raises(ValueError, match="no quantized layers"):
        save_packed(seeded_model(), str(tmp_path / "none.safetensors"))
    model = seeded_model()
    apply_optional_quantization(model, quant_type="int8")
    good = str(tmp_path / "good.safetensors")
    save_packed(model, good)
    with pytest.raises(ValueError, match="no module named"):
        load_packed(nn.Sequential(nn.Linear(4, 4)), good)


def _rewrite_packed(src, dst, edit):
    """Copy a packed file, passing its tensors through edit(dict) (header kept)."""
    from safetensors import safe_open
    from safetensors.torch import save_file

    with safe_open(src, framework="pt") as f:
        meta = f.metadata()
        tensors = {k: f.get_tensor(k) for k in f.keys()}
    edit(tensors)
    save_file(tensors, dst, metadata=meta)


@pytest.mark.parametrize("case", ["short_packed", "wide_scale", "wrong_dtype", "missing", "extra",
                                  "tiled_bytes"])
def test_packed_checkpoint_rejects_mismatched_tensors(tmp_path, case):
    """A tensor whose shape, dtype or byte count disagrees with the layer's metadata (a
    truncated or mixed-up file) raises ValueError before anything is installed; the kernels
    size their buffer descriptors from N and K, so such a tensor must never reach them."""
    from safetensors import safe_open

    from localstrm_amd import load_packed, save_packed

    model = seeded_model()
    apply_optional_quantization(model, quant_type="int4", group_size=32)
    good = str(tmp_path / "good.safetensors")
    save_packed(model, good)
    key = "model.layers.0.mlp.down_proj"

    def edit(t):
        if case == "short_packed":
            t[f"{key}.weight_packed"] = t[f"{key}.weight_packed"][:-1].clone()
        elif case == "wide_scale":
            s = t[f"{key}.scale"]
            t[f"{key}.scale"] = torch.cat([s, s[:, :1]], dim=1)
        elif case == "wrong_dtype":
            t[f"{key}.weight_packed"] = t[f"{key}.weight_packed"].to(torch.int8)
        elif case == "missing":
            del t[f"{key}.scale"]
        elif case == "extra":
            t[f"{key}.extra"] = torch.zeros(3)
        elif case == "tiled_bytes":
            t[f"{key}.weight_tiled"] = torch.zeros(17, dtype=torch.uint8)

    bad = str(tmp_path / "bad.safetensors")
    if case in ("extra", "tiled_bytes"):
        # the header lists the layer's tensors: add the name there too
        import json
        from safetensors.torch import save_file

        with safe_open(good, framework="pt") as f:
            meta = dict(f.metadata())
            tensors = {k: f.get_tensor(k) for k in f.keys()}
        layers = json.loads(meta["layers"])
        layers[key]["tensors"].append("extra" if case == "extra" else "weight_tiled")
        meta["layers"] = json.dumps(layers)
        edit(tensors)
        save_file(tensors, bad, metadata=meta)
    else:
        _rewrite_packed(good, bad, edit)
    fresh = seeded_model(seed=7)
    before = {k: v.clone() for k, v in fresh.state_dict().items()}
    with pytest.raises(ValueError, match="load_packed"):
        load_packed(fresh, bad)
    if case != "missing":  # layers before the bad one are installed; the bad one never is
        assert isinstance(fresh.model.layers[0].mlp.down_proj, nn.Linear)
    assert load_packed(seeded_model(seed=7), good) == 14
