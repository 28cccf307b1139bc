"""Whole-network conversion, ``model.to(dtype=trit)``, and the patched ``nn.Linear.forward``
(t81/torch/__init__.py:136-164, 307-335) on the GPU path, against the oracle."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch
from torch import nn

from t81lib_amd import nn as t8nn, tensor as tt
from t81lib_amd.tensor import TernaryTensor, trit
from conftest import accum_rtol, fp_tolerance_ok

pytestmark = pytest.mark.gpu


def announce(case: str) -> None:
    sys.__stderr__.write(f"[gpu case] {case}\n")
    sys.__stderr__.flush()


class Mlp(nn.Module):
    def __init__(self):
        super().__init__()
        self.emb = nn.Embedding(50, 96)
        self.fc1 = nn.Linear(96, 130)
        self.norm = nn.LayerNorm(130)
        self.fc2 = nn.Linear(130, 70, bias=False)

    def forward(self, ids):
        h = self.emb(ids)
        return self.fc2(self.norm(self.fc1(h)))


def _linear_ref(orc, layer: nn.Linear, x: torch.Tensor, threshold: float = 0.5):
    """Oracle y = x T^T (+ bias), T the torch-form ternarization of the float weight."""
    w = layer.weight.detach().float().cpu().numpy()
    wp = orc.pack_rows(w, np.float32(orc.torch_threshold(threshold)), 1)
    xd = x.detach().reshape(-1, x.shape[-1]).double().cpu().numpy()
    ref = orc.trit_matmul_f64(xd, wp, w.shape[1])
    scale = orc.trit_matmul_abs_f64(xd, wp, w.shape[1])
    if layer.bias is not None:
        b = layer.bias.detach().double().cpu().numpy()
        ref, scale = ref + b, scale + np.abs(b)
    return ref, scale


def test_module_to_trit_converts_and_linear_runs_packed(gpu, orc):
    announce("convert model.to(dtype=trit)")
    torch.manual_seed(0)
    model = Mlp().to(gpu)
    with torch.no_grad():
        for lin in (model.fc1, model.fc2):
            lin.weight.normal_()                    # ~1/3 zero trits at 0.5
    out_model = model.to(dtype=trit)
    assert out_model is model
    for name in ("emb", "fc1", "fc2"):
        cache = getattr(model, name)._t81_ternary_cache
        assert list(cache) == ["weight"] and isinstance(cache["weight"], TernaryTensor)
    assert not hasattr(model.norm, "_t81_ternary_cache")        # no 2-D parameter
    # the cached limbs are the torch-form 0.5 packing of the float weight
    want = orc.pack_rows(model.fc1.weight.detach().cpu().numpy(),
                         np.float32(orc.torch_threshold(0.5)), 1)
    np.testing.assert_array_equal(model.fc1._t81_ternary_cache["weight"].packed.cpu().numpy(),
                                  want)
    x = torch.randn(7, 96, device=gpu)
    with torch.no_grad():
        y = model.fc1(x)
    ref, scale = _linear_ref(orc, model.fc1, x)
    ok, worst, nbad = fp_tolerance_ok(y.cpu().numpy(), ref, scale, accum_rtol(96, "f32"))
    assert ok, f"fc1: {nbad} outside, worst {worst:.3g}"
    # 3-D activations are flattened; gradients reach the input and the bias
    x3 = torch.randn(2, 5, 96, device=gpu, requires_grad=True)
    y3 = model.fc1(x3)
    assert y3.shape == (2, 5, 130)
    ref3, scale3 = _linear_ref(orc, model.fc1, x3)
    ok, worst, nbad = fp_tolerance_ok(y3.detach().reshape(-1, 130).cpu().numpy(), ref3, scale3,
                                      accum_rtol(96, "f32"))
    assert ok, f"3-D: {nbad} outside, worst {worst:.3g}"
    g = torch.randn_like(y3)
    (y3 * g).sum().backward()
    trits = model.fc1._t81_ternary_cache["weight"].trits().float()
    torch.testing.assert_close(x3.grad, (g.reshape(-1, 130) @ trits).reshape(2, 5, 96),
                               rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(model.fc1.bias.grad, g.reshape(-1, 130).sum(0), rtol=1e-5,
                               atol=1e-4)
    assert model.fc1.weight.grad is None                        # no weight gradient
    # the whole model runs; the unconverted layers are untouched
    ids = torch.randint(0, 50, (3, 4), device=gpu)
    with torch.no_grad():
        out = model(ids)
    assert out.shape == (3, 4, 70) and bool(torch.isfinite(out).all())


def test_cached_weights_repack_only_when_changed(gpu, orc, monkeypatch):
    announce("convert repack on change")
    torch.manual_seed(1)
    layer = nn.Linear(64, 33).to(gpu)
    with torch.no_grad():
        layer.weight.normal_()
    layer.to(dtype=trit)
    calls = []
    real = TernaryTensor.update_from_float
    monkeypatch.setattr(TernaryTensor, "update_from_float",
                        lambda self, src: (calls.append(1), real(self, src))[1])
    x = torch.randn(4, 64, device=gpu)
    with torch.no_grad():
        y0 = layer(x)
        layer(x)
    assert calls == [], "unchanged weights must not be re-packed"
    opt = torch.optim.SGD(layer.parameters(), lr=0.5)
    layer.weight.grad = torch.randn_like(layer.weight)
    opt.step()                                                  # in-place update
    with torch.no_grad():
        y1 = layer(x)
    assert len(calls) == 1, "an optimizer step must trigger exactly one re-pack"
    ref, scale = _linear_ref(orc, layer, x)
    ok, worst, nbad = fp_tolerance_ok(y1.cpu().numpy(), ref, scale, accum_rtol(64, "f32"))
    assert ok, f"after step: {nbad} outside"
    assert not torch.equal(y0, y1)
    # writes through .data bypass the version counter: refresh_ternary_weights re-packs
    with torch.no_grad():
        layer.weight.data.mul_(-1.0)
    tt.refresh_ternary_weights(layer)
    with torch.no_grad():
        y2 = layer(x)
    ref, scale = _linear_ref(orc, layer, x)
    ok, _, nbad = fp_tolerance_ok(y2.cpu().numpy(), ref, scale, accum_rtol(64, "f32"))
    assert ok, f"after refresh: {nbad} outside"


def test_t8_linear_threshold_and_to_device_args(gpu):
    """A t8.nn.Linear converts with its own ternary_threshold; .to(device, dtype=trit)
    applies the move before converting; a plain dtype call is untouched."""
    announce("convert t8.nn.Linear + args")
    layer = t8nn.Linear(48, 8, threshold=0.7)
    layer.to("cuda", dtype=trit)
    assert layer.weight.device.type == "cuda"
    assert layer._t81_ternary_cache["weight"]._threshold == pytest.approx(0.7)
    plain = nn.Linear(4, 2).to(torch.float16)
    assert plain.weight.dtype == torch.float16 and not hasattr(plain, "_t81_ternary_cache")
