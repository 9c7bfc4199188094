"""GPU checks of the layers' device memory: one quantized weight copy on the GPU, as the
reference holds one (src/kernels/quantization.py:44-51, footprint :143-149; its preflight
budgets INT8 at 0.50 and INT4 at 0.25 of fp16, src/memory/preflight.py:462-471).

On a GPU a layer keeps only the tiled copy its kernels read; weight_q / weight_packed /
weight_q_t, state_dict() and .to("cpu") give the reference's canonical tensors, untiled on
demand, bit-identical to what was installed.
"""

import numpy as np
import pytest
import torch
import torch.nn as nn

import bench
from localstrm_amd import Int8GEMMLinear, QuantizedLinear
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
N, K = 18944, 3584


def _say(msg):
    print(msg, flush=True)


def _alloc_growth(make):
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(DEV)
    layer = make()
    torch.cuda.synchronize()
    return layer, torch.cuda.memory_allocated(DEV) - before


@pytest.mark.parametrize("kind", ["int8", "int4", "w8a8"])
def test_one_weight_copy_on_the_gpu(kind):
    """Allocation growth of one 18944 x 3584 layer: N*K (INT8, W8A8) or N*K/2 (INT4) bytes
    of weights plus the scales (within 1 %), not two copies."""
    if kind == "int4":
        p, s, x = bench.make_int4(N, K, 4)
        layer, grew = _alloc_growth(lambda: QuantizedLinear.from_quantized(
            p.to(DEV), s.to(DEV), quant_type="int4", in_features=K, group_size=128))
        expect = N * K // 2 + s.numel() * 2
    else:
        w, s, x = bench.make_int8(N, K, 4)
        if kind == "int8":
            layer, grew = _alloc_growth(lambda: QuantizedLinear.from_quantized(w.to(DEV), s.to(DEV),
                                                                               quant_type="int8"))
        else:
            layer, grew = _alloc_growth(lambda: Int8GEMMLinear.from_quantized(w.to(DEV), s.to(DEV),
                                                                              dtype=torch.bfloat16))
        expect = N * K + N * 4
    _say(f"  {kind}: allocated {grew} B for {expect} B of weights + scales "
         f"(footprint {layer.memory_footprint_bytes()} B)")
    assert abs(grew - expect) <= 0.01 * expect
    assert abs(layer.memory_footprint_bytes() - expect) <= 0.01 * expect
    with torch.no_grad():
        y = layer(x.to(DEV))
    assert torch.isfinite(y.float()).all()


@pytest.mark.parametrize("kind", ["int8", "int4"])
def test_canonical_views_state_dict_and_moves(kind):
    """weight_q / weight_packed, state_dict(), .to('cpu') and back, load_state_dict: the
    canonical tensors come back bit-identical and the layer keeps computing the same."""
    if kind == "int4":
        w, s, x = bench.make_int4(1040, 1024, 3)
        ql = QuantizedLinear.from_quantized(w.to(DEV), s.to(DEV), quant_type="int4", in_features=1024,
                                            group_size=128)
        cname = "weight_packed"
    else:
        w, s, x = bench.make_int8(1040, 1024, 3)
        ql = QuantizedLinear.from_quantized(w.to(DEV), s.to(DEV), quant_type="int8")
        cname = "weight_q"
    assert ql._buffers[cname].numel() == 0 and ql.weight_tiled.numel() > 0
    assert torch.equal(getattr(ql, cname).cpu(), w)
    sd = ql.state_dict()
    assert set(sd) == {cname, "scale"} and torch.equal(sd[cname].cpu(), w)
    xd = x.to(DEV)
    with torch.no_grad():
        y0 = ql(xd)
    ql.to("cpu")
    assert ql.weight_tiled.numel() == 0 and torch.equal(ql._buffers[cname], w)
    ql.to(DEV)
    assert ql._buffers[cname].numel() == 0
    with torch.no_grad():
        assert torch.equal(ql(xd), y0)
    # load_state_dict installs new weights into the tiled copy
    w2 = torch.zeros_like(w) if kind == "int8" else torch.full_like(w, 0x88)  # all q = 0
    ql.load_state_dict({cname: w2, "scale": s})
    assert torch.equal(getattr(ql, cname).cpu(), w2)
    with torch.no_grad():
        # exact zero for INT8; INT4 sums x * (128 + u) and removes 136 * sum(x) afterwards,
        # so zero weights leave an fp32 cancellation residue (~1e-5 here, on outputs of ~30)
        assert ql(xd).abs().max().item() <= (0.0 if kind == "int8" else 1e-4)
    # dequantize reads the tiled copy's weights
    ql.load_state_dict({cname: w, "scale": s})
    wd = ql.dequantize(torch.bfloat16).float().cpu().numpy()
    ref = (qo.dequant_int8(w.numpy(), s.numpy(), "bf16") if kind == "int8"
           else qo.dequant_int4(w.numpy(), s.float().numpy(), 1024, 128, "bf16"))
    assert np.array_equal(wd.view(np.uint32), ref.view(np.uint32))


def test_fp32_activations_read_the_tiled_copy():
    """fp32 activations run the generic kernel, which reads the tiled copy (there is no
    other copy on the GPU): the single-layer INT8 workload (4864 x 896, x fp32 [1, 896])."""
    w, s, x = bench.make_int8(4864, 896, 1, x_dtype=torch.float32)
    ql = QuantizedLinear.from_quantized(w.to(DEV), s.to(DEV), quant_type="int8")
    assert ql._buffers["weight_q"].numel() == 0
    with torch.no_grad():
        y = ql(x.to(DEV)).cpu().numpy()
    ref = qo.linear_f64(x.numpy(), qo.dequant_int8(w.numpy(), s.numpy(), "f32"), None, "f32")
    assert qo.rel_err(y, ref) <= 1e-5
    p, s4, x4 = bench.make_int4(272, 512, 5, x_dtype=torch.float32)
    q4 = QuantizedLinear.from_quantized(p.to(DEV), s4.to(DEV), quant_type="int4", in_features=512,
                                        group_size=128)
    with torch.no_grad():
        y4 = q4(x4.to(DEV)).cpu().numpy()
    ref4 = qo.linear_f64(x4.numpy(), qo.dequant_int4(p.numpy(), s4.float().numpy(), 512, 128, "f32"), None, "f32")
    assert qo.rel_err(y4, ref4) <= 1e-5


def test_w8a8_weight_view_and_fallback(monkeypatch):
    """Int8GEMMLinear: weight_q_t is untiled on demand, and the kill-switch fallback reads
    the W8A8 tiled copy as the INT8 layout (same bytes at K % 128 == 0)."""
    w, s, x = bench.make_int8(512, 1024, 4)
    layer = Int8GEMMLinear.from_quantized(w.to(DEV), s.to(DEV), dtype=torch.bfloat16)
    assert layer._buffers["weight_q_t"].numel() == 0
    assert torch.equal(layer.weight_q_t.cpu(), w.t())
    assert set(layer.state_dict()) == {"weight_q_t", "scale_w_t"}
    monkeypatch.setenv("MINIVLLM_DISABLE_INT8_GEMM", "1")
    with torch.no_grad():
        y = layer(x.to(DEV)).float().cpu().numpy()
    ref = qo.linear_f64(x.float().numpy(), qo.dequant_int8(w.numpy(), s.numpy(), "bf16"), None, "bf16")
    assert qo.rel_err(y, ref) <= 1e-2


def test_loader_footprint_matches_the_gpu():
    """load_and_quantize_model's reported quantized bytes match what the layers hold on the
    GPU (within the 16-row tile padding)."""
    from localstrm_amd import load_and_quantize_model
    from tests.synthetic import seeded_model

    model, orig, quant = load_and_quantize_model(seeded_model(h=128), device=DEV, quantization="int4",
                                                 dtype=torch.bfloat16)
    on_gpu = sum(b.numel() * b.element_size() for b in model.buffers()) + \
        sum(p.numel() * p.element_size() for p in model.parameters())
    _say(f"  reported {quant} B, on the GPU {on_gpu} B (float model {orig} B)")
    assert abs(on_gpu - quant) <= 0.02 * quant
