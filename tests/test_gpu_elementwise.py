"""GPU parity of the backend contract's elementwise ops (where / clamp / lerp /
addcmul, include/t81_hip.h) with the oracle, bit for bit, and of the C++ plugin
inside a T81LIB_USE_ROCM build of the reference's own dispatch."""

from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

from test_oracle import EW_CASES, _same_or_both_nan

pytestmark = pytest.mark.gpu

SPECIALS = np.array([np.nan, np.inf, -np.inf, -0.0, 0.0, 1e-45, 3e38, -3e38, 1.0, -1.0],
                    np.float32)


def _inputs(n: int, seed: int):
    rng = np.random.default_rng(seed)
    arrs = [(rng.standard_normal(n) * 2).astype(np.float32) for _ in range(3)]
    for i, arr in enumerate(arrs):
        k = min(n, SPECIALS.size)
        arr[:k] = np.roll(SPECIALS, 3 * i)[:k]
    arrs[0][::7] = 0.0
    return arrs


def _run(ops, op, a, b, c, kw, out=None):
    if op == "where":
        return ops.where(a, b, c, out=out)
    if op == "clamp":
        return ops.clamp(a, kw["p0"], kw["p1"], out=out)
    if op == "lerp":
        return ops.lerp(a, b, c, out=out)
    return ops.addcmul(a, b, c, kw["p0"], out=out)


# (1 << 20) + 3: the non-temporal vector path and its scalar tail
@pytest.mark.parametrize("n", [0, 1, 3, 4, 5, 257, 100003, (1 << 20) + 3])
def test_elementwise_vs_oracle(gpu, orc, n):
    import torch

    from t81lib_amd import ops

    a, b, c = _inputs(n, n)
    ta, tb, tc = (torch.from_numpy(v).to(gpu) for v in (a, b, c))
    for op, kw in EW_CASES:
        got = _run(ops, op, ta, tb, tc, kw).cpu().numpy()
        want = orc.elementwise(op, a, b, c, **kw)
        assert _same_or_both_nan(got, want), (op, n)


def test_elementwise_unaligned_and_in_place(gpu, orc):
    import torch

    from t81lib_amd import ops

    a, b, c = _inputs(1027, 5)
    base = [torch.from_numpy(np.concatenate([[0.0], v]).astype(np.float32)).to(gpu)
            for v in (a, b, c)]
    ta, tb, tc = (t[1:] for t in base)  # 4-byte aligned, not 16-byte aligned
    for op, kw in EW_CASES:
        want = orc.elementwise(op, a, b, c, **kw)
        assert _same_or_both_nan(_run(ops, op, ta, tb, tc, kw).cpu().numpy(), want), op
        inplace = ta.clone()
        _run(ops, op, inplace, tb, tc, kw, out=inplace)
        assert _same_or_both_nan(inplace.cpu().numpy(), want), (op, "in place")
    # in place on the non-temporal path
    a, b, c = _inputs(1 << 20, 6)
    for op, kw in EW_CASES:
        want = orc.elementwise(op, a, b, c, **kw)
        inplace, tb, tc = (torch.from_numpy(v).to(gpu) for v in (a, b, c))
        _run(ops, op, inplace, tb, tc, kw, out=inplace)
        assert _same_or_both_nan(inplace.cpu().numpy(), want), (op, "in place, 1 Mi")


def test_elementwise_argument_errors(gpu):
    import torch

    from t81lib_amd import ops

    x = torch.zeros(4, device=gpu)
    with pytest.raises(ValueError):
        ops.lerp(x, x, torch.zeros(5, device=gpu))
    with pytest.raises(ValueError):
        ops.clamp(x.double(), 0.0, 1.0)


def test_rocm_plugin_inside_reference_dispatch(gpu):
    """oracle/_ref/plugin_check: the reference's gemm_ternary / where / clamp / lerp /
    addcmul routed to Backend::ROCm (this package's plugin) equal Backend::CPU bit for
    bit.  Built where the reference sources exist (oracle/Makefile `plugin`)."""
    import oracle

    if not os.path.exists(oracle.PLUGIN_CHECK):
        pytest.skip("oracle/_ref/plugin_check not built (needs the reference sources)")
    res = subprocess.run([oracle.PLUGIN_CHECK], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "all bit-exact" in res.stdout
