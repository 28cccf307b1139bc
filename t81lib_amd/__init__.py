"""t81lib_amd -- MI355X (gfx950) backend of t81lib's packed-ternary GEMM path.

Layers, bottom up:

* ``libt81_hip.so`` (``csrc/``): hand-written HIP kernels behind the C ABI of
  ``include/t81_hip.h`` -- K1 quantize+pack, K2 decode GEMV, K3 prefill GEMM,
  K4 the reference's limb-integer ``gemm_ternary``.
* :mod:`t81lib_amd.ops` -- torch device tensors over that ABI.
* :mod:`t81lib_amd.t81lib` -- the reference extension module's surface
  (``gemm_ternary``, ``pack_dense_matrix``, ``quantize_to_trits``, ...).
* :mod:`t81lib_amd.tensor` -- ``TernaryTensor`` / ``trit`` (``t81.torch``).
* :mod:`t81lib_amd.nn` -- ``Linear`` (``t8.nn.Linear``).

Everything computes on the GPU; without the built library or a gfx950
device, calls raise instead of falling back to the CPU.
"""

from __future__ import annotations

from . import _lib
from ._lib import T81HipError, available

__all__ = ["T81HipError", "available", "ops", "t81lib", "tensor", "nn", "TernaryTensor",
           "trit", "Linear"]


def __getattr__(name: str):
    import importlib

    if name in ("ops", "t81lib", "tensor", "nn"):
        return importlib.import_module(f".{name}", __name__)
    if name in ("TernaryTensor", "trit"):
        return getattr(importlib.import_module(".tensor", __name__), name)
    if name == "Linear":
        return importlib.import_module(".nn", __name__).Linear
    raise AttributeError(f"module {__name__} has no attribute {name}")


del _lib
