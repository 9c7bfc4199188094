"""GPU checks of pre-packed checkpoints (localstrm_amd/checkpoint.py): layers loaded from
a save_packed file onto the GPU use the saved tiled copies without re-tiling, and give
bit-identical outputs to the layers that were saved."""

import pytest
import torch

from localstrm_amd import (CachedQuantizedLinear, Int8GEMMLinear, QuantizedLinear,
                           apply_optional_quantization, load_packed, save_packed)
from tests.synthetic import seeded_model

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("mode,group", [("int8", None), ("int4", 32), ("hybrid_int8", None)])
def test_packed_load_on_gpu_skips_retile_and_matches(tmp_path, monkeypatch, mode, group):
    print(f"packed {mode} g={group}", flush=True)
    model = seeded_model(h=128)
    apply_optional_quantization(model, quant_type=mode, group_size=group)
    model = model.to(DEV).half()
    path = str(tmp_path / "m.safetensors")
    save_packed(model, path)

    def no_retile(self):
        raise AssertionError("re-tiled at load")

    fresh = seeded_model(h=128, seed=3)
    monkeypatch.setattr(QuantizedLinear, "_refresh_tiled", no_retile)
    monkeypatch.setattr(Int8GEMMLinear, "_refresh_tiled", no_retile)
    load_packed(fresh, path, device=DEV)
    monkeypatch.undo()
    x = torch.randn(3, 7, 128, device=DEV, dtype=torch.float16)
    pairs = [(a, b) for a, b in zip(model.modules(), fresh.modules())
             if isinstance(a, (QuantizedLinear, Int8GEMMLinear, CachedQuantizedLinear))]
    assert len(pairs) == 14
    with torch.no_grad():
        for a, b in pairs:
            assert type(a) is type(b)
            if not isinstance(a, CachedQuantizedLinear):
                assert torch.equal(a.weight_tiled, b.weight_tiled)
            xin = x if a.in_features == 128 else torch.randn(3, 7, a.in_features, device=DEV,
                                                             dtype=torch.float16)
            assert torch.equal(a(xin), b(xin))
