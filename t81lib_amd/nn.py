"""``Linear``: the reference's ``t8.nn.Linear`` (t81/nn/linear.py:18-125) on the GPU path.

Eval mode packs the weight once (K1, threshold 0.45 by default, cached until
``train()`` or ``load_state_dict``) and runs the packed matmul (K2 for <= 16
tokens, K3 above), with the bias fused into the kernel's epilogue when no
gradient is needed and added by autograd otherwise (so ``bias.grad`` is filled,
as in the reference).  Train mode keeps the reference's quantization-aware
forward, ``F.linear(x, ternary(w / s) * s, b)`` with ``s`` an EMA(0.99) of max |w|
(t81/nn/linear.py:72-99): the weight gradient flows through the dorso_round
surrogate of :func:`t81lib_amd.qat.ternary`, and ``configure_qat`` switches on
stochastic ternarization (t81/nn/linear.py:124-125, t81/qat.py:12-25).  Training
is plain torch code.
"""

from __future__ import annotations

from collections import OrderedDict
from typing import Optional

import torch
from torch import nn
from torch.nn import functional as F

from .qat import ternary
from .tensor import TernaryTensor

_DEFAULT_THRESHOLD = 0.45


class Linear(nn.Linear):
    """Balanced-ternary ``nn.Linear`` whose inference path runs on packed limbs."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 device: Optional[torch.device] = None, dtype: Optional[torch.dtype] = None,
                 threshold: float = _DEFAULT_THRESHOLD, semantics: str = "trit_dot") -> None:
        super().__init__(in_features, out_features, bias=bias, device=device, dtype=dtype)
        self.ternary_threshold = threshold
        self.semantics = semantics
        self.ternary_weight: Optional[TernaryTensor] = None
        self.register_buffer("training_scale", None)
        self._stochastic_rounding = False

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.training:
            return F.linear(x, self._quantize_training_weight(), self.bias)
        if self.ternary_weight is None:
            self.ternary_weight = TernaryTensor.from_float(
                self.weight.detach(), threshold=self.ternary_threshold, semantics=self.semantics)
        return self._packed_linear(x)

    def _packed_linear(self, x: torch.Tensor) -> torch.Tensor:
        # t81/nn/linear.py:53-70: 3-D inputs are flattened to (batch*seq, features)
        if x.ndim == 3:
            batch, seq, features = x.shape
            return self._packed_linear(x.reshape(batch * seq, features)).reshape(batch, seq, -1)
        if x.ndim != 2:
            raise ValueError("t81.nn.Linear expects 2D or 3D inputs")
        bias = self.bias
        if torch.is_grad_enabled() and (x.requires_grad or (bias is not None and bias.requires_grad)):
            # autograd: dx through the transposed limbs, dbias through the addition
            out = self.ternary_weight.matmul_input(x)
            return out + bias if bias is not None else out
        return self.ternary_weight.linear(x, bias=bias.detach() if bias is not None else None)

    def _quantize_training_weight(self) -> torch.Tensor:
        scale = self._update_training_scale()
        quantized = ternary(self.weight / scale, threshold=self.ternary_threshold,
                            stochastic=self._stochastic_rounding)
        return quantized * scale

    def _update_training_scale(self) -> torch.Tensor:
        candidate = self.weight.detach().abs().amax().clamp(min=1e-6).to(torch.float32)
        existing = self.training_scale
        if existing is None or existing.device != candidate.device:
            self.training_scale = candidate
            return self.training_scale
        combined = (existing.to(torch.float32) * 0.99 + candidate * 0.01).clamp(min=1e-6)
        self.training_scale = combined.detach()
        return self.training_scale

    def extra_repr(self) -> str:
        base = super().extra_repr()
        if self.ternary_threshold != _DEFAULT_THRESHOLD:
            return f"{base}, threshold={self.ternary_threshold}"
        return base

    def train(self, mode: bool = True) -> "Linear":
        if mode:
            self.ternary_weight = None
        return super().train(mode)

    def load_state_dict(self, state_dict, strict: bool = True, assign: bool = False):
        normalized = OrderedDict()
        for key, value in state_dict.items():
            if key in {"weight", "bias"} and value.is_floating_point() and value.dtype in {
                    torch.bfloat16, torch.float16}:
                value = value.to(torch.float32)
            normalized[key] = value
        result = super().load_state_dict(normalized, strict=strict, assign=assign)
        self.ternary_weight = None
        self.training_scale = None
        return result

    def configure_qat(self, *, stochastic_rounding: bool) -> None:
        """t81/nn/linear.py:124-125: stochastic ternarization of the training weights."""
        self._stochastic_rounding = stochastic_rounding


__all__ = ["Linear"]
