"""spmm_simple on the GPU against the CPU oracle and the reference's own outputs.

Bit-exact: every output element is a chain of double roundings in the entries' list
order, which the device kernel replays; only NaN payloads may differ (a NaN an
operation creates has its sign bit set on x86 and clear on the GPU), so NaN compares
equal to NaN.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

import oracle
from t81lib_amd import sparse, t81lib

pytestmark = pytest.mark.gpu

GOLDEN = np.load(os.path.join(os.path.dirname(__file__), "golden", "ref_vectors.npz"))


def announce(case: str) -> None:
    sys.__stderr__.write(f"[gpu case] {case}\n")
    sys.__stderr__.flush()


def same(got: np.ndarray, want: np.ndarray) -> bool:
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    nan = np.isnan(want)
    return bool(got.shape == want.shape and np.array_equal(np.isnan(got), nan)
                and np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)))


def golden_case(i):
    rows, cols, N = (int(d) for d in GOLDEN[f"sp{i}_dims"])
    alpha, beta = (float(a) for a in GOLDEN[f"sp{i}_ab"])
    return (GOLDEN[f"sp{i}_values"], GOLDEN[f"sp{i}_rows"], GOLDEN[f"sp{i}_cols"], rows, cols,
            GOLDEN[f"sp{i}_B"], GOLDEN[f"sp{i}_C"], N, alpha, beta)


NAMES = [str(n) for n in GOLDEN["sp_names"]]


@pytest.mark.parametrize("i", range(len(NAMES)), ids=NAMES)
def test_binding_matches_reference_outputs(gpu, i):
    """t81lib.spmm_simple on NumPy buffers, in place, as the reference's example calls it."""
    announce(f"spmm golden {NAMES[i]}")
    vals, ri, ci, rows, cols, B, C, N, alpha, beta = golden_case(i)
    Bh = B.copy().reshape(-1)
    Ch = C.copy().reshape(-1)
    if int(GOLDEN[f"sp{i}_rc"]) == 0:
        t81lib.spmm_simple(vals.tolist(), ri.tolist(), ci.tolist(), rows, cols, Bh, Ch, N,
                           alpha, beta)
    else:
        with pytest.raises(ValueError, match="index out of bounds"):
            t81lib.spmm_simple(vals.tolist(), ri.tolist(), ci.tolist(), rows, cols, Bh, Ch, N,
                               alpha, beta)
    assert same(Ch.reshape(rows, N), GOLDEN[f"sp{i}_out"])


@pytest.mark.parametrize("i", range(len(NAMES)), ids=NAMES)
def test_plan_matches_reference_outputs(gpu, i):
    """The reusable device form on GPU tensors; a bad index refuses to build."""
    announce(f"spmm plan golden {NAMES[i]}")
    vals, ri, ci, rows, cols, B, C, N, alpha, beta = golden_case(i)
    if int(GOLDEN[f"sp{i}_rc"]) != 0:
        with pytest.raises(ValueError, match="index out of bounds"):
            sparse.SparseTernaryMatrix(vals, ri, ci, rows, cols)
        return
    A = sparse.SparseTernaryMatrix(torch.from_numpy(vals).to(gpu), torch.from_numpy(ri).to(gpu),
                                   torch.from_numpy(ci).to(gpu), rows, cols)
    Cd = torch.from_numpy(C.copy()).to(gpu)
    A.matmul(torch.from_numpy(B).to(gpu), Cd, alpha, beta)
    assert same(Cd.cpu().numpy(), GOLDEN[f"sp{i}_out"])
    A.close()


def make_case(rows, cols, N, nnz, seed, one_row=None, big=True):
    g = np.random.default_rng(seed)
    vals = g.integers(-1, 2, nnz).astype(np.int64)
    if big and nnz:
        sel = g.random(nnz) < 0.2
        vals[sel] = g.integers(-2**63, 2**63 - 1, int(sel.sum()), dtype=np.int64, endpoint=True)
    ri = (np.full(nnz, one_row, np.int32) if one_row is not None
          else g.integers(0, max(rows, 1), nnz).astype(np.int32))
    ci = g.integers(0, max(cols, 1), nnz).astype(np.int32)
    scale = 1e-19 if big else 1.0
    B = (g.standard_normal((cols, N)) * scale).astype(np.float32)
    C = g.standard_normal((rows, N)).astype(np.float32)
    return vals, ri, ci, B, C


RANDOM = [  # rows, cols, N, nnz  (N picks 1/2/4 features per lane and 1..64 lanes per row)
    (1000, 800, 64, 20000), (3000, 2000, 128, 100000), (500, 700, 256, 30000),
    (257, 300, 100, 5000), (4096, 4096, 1, 50000), (100, 100, 3, 1000), (33, 17, 1000, 2000),
    (70000, 50, 2, 100000),          # rows > 2^16: three radix passes
    (2**24 + 3, 10, 1, 30000),       # rows > 2^24: four radix passes
    (5, 5, 1000, 0), (10, 10, 33, 1), (1, 1, 7, 3000), (6, 9, 130, 777),
]


@pytest.mark.parametrize("rows,cols,N,nnz", RANDOM)
def test_random_vs_oracle(gpu, rows, cols, N, nnz):
    announce(f"spmm random rows={rows} cols={cols} N={N} nnz={nnz}")
    vals, ri, ci, B, C = make_case(rows, cols, N, nnz, seed=rows * 31 + N * 7 + nnz)
    A = sparse.SparseTernaryMatrix(torch.from_numpy(vals).to(gpu), torch.from_numpy(ri).to(gpu),
                                   torch.from_numpy(ci).to(gpu), rows, cols)
    assert A.nnz == nnz
    Bd = torch.from_numpy(B).to(gpu)
    for alpha, beta in ((1.0, 0.0), (-0.37, 1.25)):
        Cd = torch.from_numpy(C).to(gpu)
        A.matmul(Bd, Cd, alpha, beta)
        rc, want = oracle.spmm_simple(vals, ri, ci, rows, cols, B, C, N, alpha, beta)
        assert rc == 0
        assert same(Cd.cpu().numpy(), want), f"alpha={alpha} beta={beta}"
    A.close()


@pytest.mark.parametrize("N", [64, 128, 256])
def test_one_long_row_keeps_list_order(gpu, N):
    """150k entries in one row span ~150 sort tiles: the stable sort must keep their order."""
    announce(f"spmm one long row N={N}")
    rows, cols, nnz = 4, 1000, 150000
    vals, ri, ci, B, C = make_case(rows, cols, N, nnz, seed=N, one_row=1, big=False)
    ri[::7] = 3
    A = sparse.SparseTernaryMatrix(vals, ri, ci, rows, cols)
    Cd = torch.from_numpy(C).to(gpu)
    A.matmul(torch.from_numpy(B).to(gpu), Cd, 0.75, -1.0)
    _, want = oracle.spmm_simple(vals, ri, ci, rows, cols, B, C, N, 0.75, -1.0)
    assert same(Cd.cpu().numpy(), want)
    A.close()


def test_misaligned_operands_take_the_scalar_path(gpu):
    announce("spmm misaligned B and C")
    rows, cols, N, nnz = 300, 200, 256, 8000
    vals, ri, ci, B, C = make_case(rows, cols, N, nnz, seed=9)
    A = sparse.SparseTernaryMatrix(vals, ri, ci, rows, cols)
    Bbuf = torch.zeros(B.size + 1, device=gpu)
    Bbuf[1:] = torch.from_numpy(B.reshape(-1)).to(gpu)
    Cbuf = torch.zeros(C.size + 1, device=gpu)
    Cbuf[1:] = torch.from_numpy(C.reshape(-1)).to(gpu)
    Bv, Cv = Bbuf[1:].view(cols, N), Cbuf[1:].view(rows, N)  # 4-byte, not 16-byte aligned
    A.matmul(Bv, Cv, 1.5, 0.5)
    _, want = oracle.spmm_simple(vals, ri, ci, rows, cols, B, C, N, 1.5, 0.5)
    assert same(Cv.cpu().numpy(), want)
    A.close()


def test_binding_on_gpu_tensors_in_place(gpu):
    announce("spmm binding with GPU tensors")
    rows, cols, N, nnz = 64, 48, 40, 3000
    vals, ri, ci, B, C = make_case(rows, cols, N, nnz, seed=4)
    Cd = torch.from_numpy(C).to(gpu)
    t81lib.spmm_simple(torch.from_numpy(vals), torch.from_numpy(ri), torch.from_numpy(ci), rows,
                       cols, torch.from_numpy(B).to(gpu), Cd, N, 2.0, 1.0)
    _, want = oracle.spmm_simple(vals, ri, ci, rows, cols, B, C, N, 2.0, 1.0)
    assert same(Cd.cpu().numpy(), want)


def test_binding_argument_errors(gpu):
    """The binding's checks and messages, python/bindings.cpp:112-134, 900-908."""
    announce("spmm argument errors")
    B = np.ones(6, np.float32)
    C = np.zeros(4, np.float32)
    with pytest.raises(ValueError, match="Values and indices lengths must match"):
        t81lib.spmm_simple([1, 2], [0], [0, 1], 2, 3, B, C, 2)
    with pytest.raises(ValueError, match="Matrix dimensions must be non-negative"):
        t81lib.spmm_simple([1], [0], [0], -1, 3, B, C, 2)
    with pytest.raises(ValueError, match="Feature dimension N must be non-negative"):
        t81lib.spmm_simple([1], [0], [0], 2, 3, B, C, -2)
    with pytest.raises(ValueError, match="byte size mismatch"):
        t81lib.spmm_simple([1], [0], [0], 2, 3, B[:5], C, 2)
    with pytest.raises(ValueError, match="must store float32"):
        t81lib.spmm_simple([1], [0], [0], 2, 3, B, np.zeros(4, np.float64), 2)
    ro = B.copy()
    ro.setflags(write=False)
    with pytest.raises(ValueError, match="must be writable"):
        t81lib.spmm_simple([1], [0], [0], 2, 3, ro, C, 2)
    with pytest.raises(ValueError, match="contiguous"):
        t81lib.spmm_simple([1], [0], [0], 2, 3, B, np.zeros(8, np.float32)[::2], 2)
    with pytest.raises(TypeError):
        t81lib.spmm_simple([1.5], [0], [0], 2, 3, B, C, 2)
    with pytest.raises(TypeError):
        t81lib.spmm_simple([2**63], [0], [0], 2, 3, B, C, 2)
    # the column check follows the row check of the same entry (simple.hpp:79-84)
    with pytest.raises(ValueError, match="Row index out of bounds"):
        t81lib.spmm_simple([1], [2], [9], 2, 3, B, C, 2)
    with pytest.raises(ValueError, match="Column index out of bounds"):
        t81lib.spmm_simple([1], [1], [3], 2, 3, B, C, 2)
