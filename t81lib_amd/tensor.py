"""``TernaryTensor`` and the ``trit`` dtype marker, GPU-resident.

Mirrors t81/torch/__init__.py:115-304 (``trit``, ``TernaryTensor.from_float``,
``update_from_float``, ``matmul_input``, ``torch.matmul``/``torch.mm``
interception, autograd through ``_TernaryGemmFunction``), with the packed limbs
kept on the GPU and packed once by the K1 kernel instead of per call on the
host.  Two readings of ``matmul_input`` are available:

* ``semantics="trit_dot"`` (default) -- y = x @ T^T over the packed trits, the
  reading every other consumer of the packed weights uses (the reference's own
  backward, t81/torch/__init__.py:291-304; training forward
  t81/nn/linear.py:43-45).  Runs K2 (M <= 16) or K3.
* ``semantics="reference_limb"`` -- the reference's literal path
  (t81/torch/__init__.py:241-276): activations quantized at 0.5, packed
  column-wise, multiplied as limb integers by K4; bit-exact with the
  reference CPU ``gemm_ternary``, including its +-inf outputs.

Importing this module also installs the reference's two global patches
(t81/torch/__init__.py:307-335): ``nn.Module.to(dtype=trit)`` converts every 2-D
parameter of a network into a cached ``TernaryTensor`` with a forward pre-hook
that keeps it in step with the float weights, and ``nn.Linear.forward`` runs the
packed matmul for layers that carry such a cache.  Differences, each a fix of a
reference defect: the reference forwards ``dtype=trit`` to torch's own
``Module.to``, which rejects a non-``torch.dtype`` with a TypeError before any
conversion happens, so here the trit marker is taken out of the arguments
first; the reference re-packs every cached weight twice per forward (the hook
and the patched forward both call ``update_from_float``), here a weight is
re-packed only when its parameter changed (its version counter or storage), so
weights written through ``.data`` need ``refresh_ternary_weights(module)``; and
inputs with more than two dimensions are flattened to (rows, features), where
the reference's ``matmul_input`` raises.
"""

from __future__ import annotations

import warnings
from typing import Any, Callable, Dict, Mapping, Optional, Sequence

import torch
from torch import nn

from . import _lib, ops


class TritDtype:
    __slots__ = ()

    def __repr__(self) -> str:
        return "t81.trit"


trit = TritDtype()

SEMANTICS = ("trit_dot", "reference_limb")


def _to_gpu_float(tensor: torch.Tensor) -> torch.Tensor:
    """Counterpart of _to_cpu_float (t81/torch/__init__.py:53-65): this build keeps
    everything on the GPU, so host tensors are moved there (with a warning)."""
    if tensor.is_meta:
        raise NotImplementedError(
            "t81.trit does not support meta tensors; load weights on CPU or disable offload.")
    if tensor.device.type != "cuda":
        if not torch.cuda.is_available():
            raise _lib.T81HipError("t81lib_amd needs a gfx950 GPU; none is visible")
        warnings.warn(
            f"t81.trit runs on the GPU; moving tensor from {tensor.device} to cuda.",
            RuntimeWarning, stacklevel=3)
        tensor = tensor.detach().to(device="cuda")
    tensor = tensor.detach()
    if tensor.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        tensor = tensor.to(torch.float32)
    return tensor.contiguous()


class TernaryTensor(torch.Tensor):
    """A (rows, cols) ternary matrix held as packed limbs (rows, ceil(cols/48), 16) on the GPU."""

    @staticmethod
    def __new__(cls, packed: torch.Tensor, shape: tuple[int, int], *, k_actual: int,
                k_limbs: int, float_source: Optional[torch.Tensor] = None,
                threshold: float = 0.5, semantics: str = "trit_dot") -> "TernaryTensor":
        if semantics not in SEMANTICS:
            raise ValueError(f"semantics must be one of {SEMANTICS}")
        t = torch.Tensor._make_wrapper_subclass(cls, shape, dtype=torch.float32,
                                                device=packed.device, requires_grad=False)
        t._packed = packed
        t._rows = int(shape[0])
        t._k_actual = int(k_actual)
        t._k_limbs = int(k_limbs)
        t._float_source = float_source
        t._packed_t = None  # T^T limbs for the backward, built on first use
        t._threshold = ops.torch_threshold(threshold)
        t._semantics = semantics
        return t

    @property
    def dtype(self) -> TritDtype:  # type: ignore[override]
        return trit

    @property
    def packed(self) -> torch.Tensor:
        """The (rows, L, 16) uint8 limb buffer (reference layout)."""
        return self._packed

    def __repr__(self) -> str:  # type: ignore[override]
        return f"TernaryTensor(shape={tuple(self.shape)}, trits_per_row={self._k_actual})"

    @staticmethod
    def _ensure_2d(tensor: torch.Tensor) -> torch.Tensor:
        if tensor.ndim != 2:
            raise ValueError("t81.trit tensors currently only support 2D matrices")
        return tensor

    @classmethod
    def from_float(cls, source: torch.Tensor, quantize: bool = True, threshold: float = 0.5,
                   semantics: str = "trit_dot") -> "TernaryTensor":
        """t81/torch/__init__.py:214-231: clamp, threshold (torch form), pack row-wise."""
        src = _to_gpu_float(cls._ensure_2d(source))
        rows, cols = src.shape
        k_limbs = ops.limbs_for(cols)
        if quantize:
            packed = ops.quantize_pack(src, ops.torch_threshold(threshold), _lib.THR_TORCH)
        else:
            packed = _pack_exact_trits(src)
        return cls(packed, (rows, cols), k_actual=cols, k_limbs=k_limbs, float_source=src,
                   threshold=threshold, semantics=semantics)

    def update_from_float(self, source: torch.Tensor) -> None:
        """t81/torch/__init__.py:233-239: re-quantize into the existing buffer."""
        src = _to_gpu_float(self._ensure_2d(source))
        if tuple(src.shape) != (self._rows, self._k_actual):
            raise ValueError("source shape does not match the ternary tensor")
        ops.quantize_pack(src, self._threshold, _lib.THR_TORCH, out=self._packed)
        self._float_source = src
        self._packed_t = None

    def trits(self) -> torch.Tensor:
        """(rows, cols) int8 trits (GPU unpack kernel)."""
        return ops.unpack(self._packed, self._rows, self._k_actual)

    def transposed_packed(self) -> torch.Tensor:
        """(cols, ceil(rows / 48), 16) limbs of T^T (GPU transpose kernel), cached until the
        weights change."""
        if self._packed_t is None:
            self._packed_t = ops.transpose_packed(self._packed, self._rows, self._k_actual)
        return self._packed_t

    def grad_input(self, grad_output: torch.Tensor) -> torch.Tensor:
        """T^T @ grad_output for grad_output (rows, tokens) -> (cols, tokens), float32: the
        backward of the reference's _TernaryGemmFunction (t81/torch/__init__.py:291-304),
        run as the forward GEMM over the transposed limbs."""
        g = grad_output.to(device=self._packed.device)
        if g.dtype not in (torch.float32, torch.bfloat16):
            g = g.float()
        gt = g.transpose(0, 1).contiguous()  # (tokens, rows)
        return ops.ternary_matmul(gt, self.transposed_packed(), self._rows).transpose(0, 1)

    def matmul_input(self, input: torch.Tensor, bias: Optional[torch.Tensor] = None
                     ) -> torch.Tensor:
        """input (tokens, cols) -> (tokens, rows): input @ T^T (+ bias), float32."""
        if input.ndim != 2:
            raise ValueError("t81.trit linear helpers expect 2D activations")
        rhs = input.transpose(-2, -1)
        out = _TernaryGemmFunction.apply(self, rhs)
        out = out.transpose(-2, -1)
        if bias is not None:
            out = out + bias.to(device=out.device, dtype=torch.float32)
        return out

    def linear(self, x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Inference fast path: x (tokens, cols) -> (tokens, rows) with the bias fused."""
        if self._semantics != "trit_dot":
            return self.matmul_input(x, bias=bias)
        x = _activations(x)
        return ops.ternary_matmul(x, self._packed, self._k_actual, bias=bias)

    @classmethod
    def __torch_function__(cls, func: Callable, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        if func in (torch.matmul, torch.mm):
            lhs, rhs = args
            if isinstance(lhs, TernaryTensor):
                return _TernaryGemmFunction.apply(lhs, rhs)
        # metadata (shape, device, ...) falls through to the default; real compute on the
        # storage-less wrapper fails loudly in __torch_dispatch__.
        return super().__torch_function__(func, types, args, kwargs)

    @classmethod
    def __torch_dispatch__(cls, func, types, args=(), kwargs=None):
        raise NotImplementedError(
            f"TernaryTensor holds packed trits only; it supports matmul/mm/matmul_input, "
            f"not {func}")

    # -- the two forward readings; rhs is (cols, tokens), result (rows, tokens) --
    def _compute_gemm(self, rhs: torch.Tensor) -> torch.Tensor:
        if rhs.shape[0] != self._k_actual:
            raise ValueError("rhs dimension does not match ternary weight width")
        if self._semantics == "trit_dot":
            x = _activations(rhs.transpose(0, 1))
            return ops.ternary_matmul(x, self._packed, self._k_actual).transpose(0, 1)
        # reference_limb: t81/torch/__init__.py:257-276 (quantize 0.5, column pack, limb
        # GEMM) as one kernel
        return ops.matmul_input_reference(self._packed, rhs.transpose(0, 1).float(), 0.5)


def _activations(x: torch.Tensor) -> torch.Tensor:
    if x.device.type != "cuda":
        raise ValueError("activations must be on the GPU")
    if x.dtype not in (torch.float32, torch.bfloat16, torch.int8):
        x = x.float()
    return x.contiguous()


def _pack_exact_trits(src: torch.Tensor) -> torch.Tensor:
    """quantize=False (t81/torch/__init__.py:222): values are taken as int8 trits."""
    as_int = src.to(torch.int8)
    if bool(((as_int < -1) | (as_int > 1)).any()):
        raise ValueError("limb trits must be -1..1")
    return ops.quantize_pack(as_int.to(torch.float32), 0.5, _lib.THR_TORCH)


class _TernaryGemmFunction(torch.autograd.Function):
    """Forward T @ rhs; backward grad_rhs = T^T @ grad (t81/torch/__init__.py:279-304)."""

    @staticmethod
    def forward(ctx, ternary_weight: TernaryTensor, rhs: torch.Tensor) -> torch.Tensor:
        device = rhs.device
        if device.type != "cuda":
            rhs_gpu = _to_gpu_float(rhs)
        else:
            rhs_gpu = rhs
        ctx.ternary = ternary_weight
        ctx.rhs_device = device
        ctx.rhs_dtype = rhs.dtype
        out = ternary_weight._compute_gemm(rhs_gpu)
        if device.type != "cuda":
            out = out.to(device)
        return out

    @staticmethod
    def backward(ctx, grad_output: torch.Tensor) -> tuple[None, torch.Tensor]:
        t: TernaryTensor = ctx.ternary
        grad_rhs = t.grad_input(grad_output)
        if ctx.rhs_device.type != "cuda":
            grad_rhs = grad_rhs.to(ctx.rhs_device)
        return None, grad_rhs


# ------------------------------------------------- whole-network conversion --
# Semantics given to the TernaryTensors that model.to(dtype=trit) creates.
conversion_semantics = "trit_dot"


def _extract_dtype_arg(args: Sequence[Any], kwargs: Mapping[str, Any]) -> Any:
    """t81/torch/__init__.py:127-134, also accepting the trit marker positionally."""
    if kwargs.get("dtype") is not None:
        return kwargs["dtype"]
    for arg in args:
        if arg is trit or isinstance(arg, torch.dtype):
            return arg
    return None


def _param_key(param: torch.Tensor) -> tuple:
    return (param.data_ptr(), param._version, tuple(param.shape))


def _sync_ternary_weights(module: nn.Module, _inputs: Sequence[Any] = ()) -> None:
    """Forward pre-hook (t81/torch/__init__.py:136-141): re-pack each cached weight whose
    parameter changed since it was packed (version counter, storage or shape)."""
    cache: Dict[str, TernaryTensor] = getattr(module, "_t81_ternary_cache", {})
    keys: Dict[str, tuple] = module.__dict__.setdefault("_t81_ternary_keys", {})
    for name, ternary in cache.items():
        param = getattr(module, name)
        key = _param_key(param)
        if keys.get(name) != key:
            ternary.update_from_float(param.detach())
            keys[name] = key


def refresh_ternary_weights(module: nn.Module) -> None:
    """Re-packs every cached weight of ``module`` and its children unconditionally (for
    weights written through ``.data``, which leaves the version counter unchanged)."""
    for sub in module.modules():
        sub.__dict__.pop("_t81_ternary_keys", None)
        _sync_ternary_weights(sub)


def _apply_ternary_conversion(module: nn.Module) -> None:
    """t81/torch/__init__.py:144-164: every submodule with 2-D parameters gets a cache of
    TernaryTensors (threshold: ``ternary_threshold``, else ``threshold``, else 0.5) and
    the forward pre-hook."""
    for sub in module.modules():
        if hasattr(sub, "_t81_ternary_cache"):
            continue
        cache: Dict[str, TernaryTensor] = {}
        keys: Dict[str, tuple] = {}
        for name, param in sub.named_parameters(recurse=False):
            if param.ndim != 2:
                continue
            threshold = getattr(sub, "ternary_threshold", getattr(sub, "threshold", 0.5))
            cache[name] = TernaryTensor.from_float(param.detach(), threshold=threshold,
                                                   semantics=conversion_semantics)
            keys[name] = _param_key(param)
        if cache:
            sub._t81_ternary_cache = cache
            sub.__dict__["_t81_ternary_keys"] = keys
            if not hasattr(sub, "_t81_hook_handle"):
                sub._t81_hook_handle = sub.register_forward_pre_hook(_sync_ternary_weights)


_original_module_to = nn.Module.to


def _ternary_module_to(self: nn.Module, *args, **kwargs) -> nn.Module:
    """nn.Module.to (t81/torch/__init__.py:310-318): ``dtype=trit`` converts the network
    after the rest of the call (device moves, ...) has been applied."""
    if _extract_dtype_arg(args, kwargs) is not trit:
        return _original_module_to(self, *args, **kwargs)
    args = tuple(a for a in args if a is not trit)
    kwargs = {k: v for k, v in kwargs.items() if not (k == "dtype" and v is trit)}
    module = _original_module_to(self, *args, **kwargs) if (args or kwargs) else self
    _apply_ternary_conversion(module)
    return module


_original_linear_forward = nn.Linear.forward


def _ternary_linear_forward(self: nn.Linear, input: torch.Tensor) -> torch.Tensor:
    """nn.Linear.forward (t81/torch/__init__.py:323-333): layers with a cached ternary
    weight run the packed matmul; the bias is added in float32 (fused into the kernel
    when no gradient is needed)."""
    cache: Dict[str, TernaryTensor] = getattr(self, "_t81_ternary_cache", {})
    ternary = cache.get("weight")
    if ternary is None:
        return _original_linear_forward(self, input)
    _sync_ternary_weights(self)
    lead = input.shape[:-1]
    x = input.reshape(-1, input.shape[-1]) if input.ndim != 2 else input
    bias = self.bias
    grad = torch.is_grad_enabled() and (
        input.requires_grad or (bias is not None and bias.requires_grad))
    if grad or x.device.type != "cuda" or ternary._semantics != "trit_dot":
        out = ternary.matmul_input(x)
        if bias is not None:
            out = out + bias
    else:
        out = ternary.linear(x, bias=bias.detach() if bias is not None else None)
    return out.reshape(*lead, out.shape[-1]) if input.ndim != 2 else out


nn.Module.to = _ternary_module_to
nn.Linear.forward = _ternary_linear_forward

__all__ = ["trit", "TritDtype", "TernaryTensor", "SEMANTICS", "refresh_ternary_weights"]
