"""Quantization-aware training helpers: the ``t81.qat`` surface ``t8.nn.Linear`` trains with.

``ternary(x, threshold, stochastic)`` (t81/qat.py:49-57) returns balanced-ternary
values in the forward pass and back-propagates through the ``dorso_round``
surrogate (t81/qat.py:28-35): the gradient reaching ``x`` is 2 where |x| < 0.5 and
0 elsewhere (|x| = 0.5 included), not the identity of a plain straight-through
estimator.  Forward values (t81/qat.py:12-25): x is clamped to [-1, 1]; entries
with |x| >= threshold take sign(x), the rest 0; with ``stochastic=True`` each such
entry is kept with probability (|x| - threshold) / (1 - threshold) (clamped to
[0, 1], the denominator floored at 1e-6), drawing one ``torch.rand_like`` sample
per entry from torch's global generator -- the same draw as the reference, so a
seeded run repeats.  Plain torch code (training runs on whatever device the
weights are on); the packed GPU kernels serve the eval path.
"""

from __future__ import annotations

import torch


def _clamp_threshold(threshold: float) -> float:
    """t81/qat.py:8-9: thresholds are clipped to [0, 1]."""
    return float(max(0.0, min(threshold, 1.0)))


def quantize(x: torch.Tensor, threshold: float, stochastic: bool = False) -> torch.Tensor:
    """The forward value of ``ternary`` (no gradient), t81/qat.py:12-25."""
    c = x.detach().clamp(-1.0, 1.0)
    mag = c.abs()
    keep = mag >= threshold
    if stochastic:
        prob = ((mag - threshold) / max(1.0 - threshold, 1e-6)).clamp(0.0, 1.0)
        keep = keep & (torch.rand_like(prob) < prob)
    return torch.where(keep, torch.sign(c), torch.zeros_like(c))


def dorso_round(x: torch.Tensor) -> torch.Tensor:
    """t81/qat.py:28-35: 1 for x >= 0.5, -1 for x <= -0.5, 2x between (so the gradient is
    2 inside (-0.5, 0.5) and 0 outside)."""
    one = torch.ones_like(x)
    return torch.where(x >= 0.5, one, torch.where(x <= -0.5, -one, 2.0 * x))


class _SurrogateGradient(torch.autograd.Function):
    """Value of ``quantized``, gradient of ``surrogate`` (t81/qat.py:38-46)."""

    @staticmethod
    def forward(ctx, surrogate: torch.Tensor, quantized: torch.Tensor) -> torch.Tensor:
        return quantized.clone()

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor):
        return grad_output, None


def ternary(x: torch.Tensor, threshold: float = 0.45, stochastic: bool = False) -> torch.Tensor:
    """Balanced-ternary quantization of ``x`` for training (t81/qat.py:49-57)."""
    threshold = _clamp_threshold(threshold)
    return _SurrogateGradient.apply(dorso_round(x), quantize(x, threshold, stochastic))


__all__ = ["ternary", "dorso_round", "quantize"]
