"""Bit-exact pins of the float32-activation paths of K2 and K3.

float32 activations enter the kernels as a pair of bfloat16 planes, x = hi + lo.  With
x = a + b / 256 (|a| <= 7, or <= 3 at K = 14336; |b| <= 127; conftest's
fixed_point_activations) both planes are exact, every partial sum is a multiple of 2^-8
below 2^16, and float32 adds them without rounding in any order, so the kernels' output
must equal 256 (a T) + b T from the integer oracle, divided by 256, bit for bit.  A kernel
that drops the lo plane (float32 computed at bfloat16 precision) loses the b / 256 part
of most activations and fails on essentially every output (tests/test_tolerance.py
plants that mistake in the oracle and checks it is caught).  Integer C and bias with
alpha = 0.5 / -1.25, beta = 0.5 / 1 keep the epilogue exact as well.

Paths covered (the north-star fp32 tolerance of 1e-3 relative is met with room to spare
by a bit-exact result; float activations enter at t81/torch/__init__.py:241-246):
* K2 column-strip kernel (M <= 4) at 4096 -> 14336, 14336 -> 4096, 8192 -> 3072, with the
  two planes as separate MFMAs or (one token from 4096 rows, two tokens) as B columns;
* K2 at 5..8 tokens: the staged stream kernel with the planes as B columns, and (x off
  16-byte alignment) the wave / stream kernels;
* K2 tile kernel at 9..16 tokens over K >= 6144 with its split sum in the workspace,
  and the stream kernel for the wider shapes it leaves;
* K3 eight-wave kernel at 17..64 tokens, on aligned x (vector loads) and on x one element
  off 16-byte alignment (element loads), two or four limbs per k-step (four over a long
  K), with the K split over a workspace and without;
* K3 at M > 64, including the config-4 shape 4096 -> 6144 at M = 512, every output
  against a float64 product of the unpacked trits on the GPU (exact) and a sample
  against the C oracle; and the path that runs the activations as two bf16 launches of
  their planes, chunk by chunk, from the workspace.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from t81lib_amd import _lib, ops
from conftest import fixed_point_acc256, fixed_point_activations, fixed_point_expected

pytestmark = pytest.mark.gpu

EPILOGUES = ((1.0, 0.0, False), (0.5, 1.0, True), (-1.25, 0.5, True))


def announce(case: str) -> None:
    sys.__stderr__.write(f"[gpu case] {case}\n")
    sys.__stderr__.flush()


def amax_for(K: int) -> int:
    return 7 if (256 * 7 + 127) * K < 2 ** 24 else 3


def problem(M, N, K, seed):
    a, b, x = fixed_point_activations(M, K, amax_for(K), seed)
    g = torch.Generator("cpu").manual_seed(seed)
    w = torch.randn((N, K), generator=g)
    c = torch.randint(-1000, 1001, (M, N), generator=g).float()
    bias = torch.randint(-1000, 1001, (N,), generator=g).float()
    return w, a, b, torch.from_numpy(x), c, bias


def assert_bits(got: np.ndarray, want: np.ndarray, what: str) -> None:
    got = np.ascontiguousarray(got, np.float32)
    bad = got.view(np.uint32) != want.view(np.uint32)
    if bad.any():
        i = tuple(int(v) for v in np.argwhere(bad)[0])
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outputs differ; first at "
                             f"{i}: got {got[i]!r}, want {want[i]!r}")


def run_cases(gpu, orc, M, N, K, seed, kernel, what, offset=0):
    """offset: x starts that many float32 elements into its buffer (1 moves it off the
    16-byte alignment the staged kernels need)."""
    w, a, b, x, c, bias = problem(M, N, K, seed)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    acc = fixed_point_acc256(orc, a, b, packed.cpu().numpy(), K)
    store = torch.zeros(M * K + 4, dtype=torch.float32, device=gpu)
    xg = store[offset:offset + M * K].view(M, K)
    xg.copy_(x.to(gpu))
    assert xg.data_ptr() % 16 == 4 * offset
    cg, bg = c.to(gpu), bias.to(gpu)
    for alpha, beta, use_bias in EPILOGUES:
        out = ops.ternary_matmul(xg, packed, K, alpha=alpha, beta=beta,
                                 c=cg.clone() if beta else None,
                                 bias=bg if use_bias else None, kernel=kernel)
        want = fixed_point_expected(acc, alpha, beta, c.numpy() if beta else None,
                                    bias.numpy() if use_bias else None)
        assert_bits(out.cpu().numpy(), want, f"{what} alpha={alpha} beta={beta} bias={use_bias}")
    return packed, acc, xg, cg, bg, c, bias


# ------------------------------------------------------------------- K2 strip --
STRIP = [(M, K, N) for (K, N) in ((4096, 14336), (14336, 4096), (8192, 3072)) for M in (1, 2, 3, 4)]
# the hi / lo planes as B token columns (one token from 4096 rows, two tokens): ragged K
# (element loads), ragged N, a short K
STRIP += [(1, 1000, 4100), (2, 999, 37), (2, 3072, 3072), (1, 48, 5000)]


@pytest.mark.parametrize("M,K,N", STRIP)
def test_strip_f32_bit_exact(gpu, orc, M, K, N):
    announce(f"exact f32 strip M={M} K={K} N={N}")
    run_cases(gpu, orc, M, N, K, seed=M * 31 + K + N, kernel=2, what="strip")


# ------------------------------------------------------ K2 wave / stream, 5..8 --
# offset 0: the staged stream kernel with each token's planes as two B columns (16-byte
# aligned x, K % 4 == 0); offset 1: the wave / stream kernels' two MFMAs per operand
FEW = [(5, 8192, 3072, 0), (8, 4096, 14336, 0), (6, 14336, 4096, 0), (7, 3072, 3072, 0),
       (8, 3072, 9216, 0), (5, 1000, 333, 0), (8, 14336, 4096, 0), (7, 4100, 20000, 0),
       (5, 8192, 3072, 1), (8, 4096, 14336, 1), (6, 14336, 4096, 1), (7, 1000, 333, 1)]


@pytest.mark.parametrize("M,K,N,offset", FEW)
def test_gemv_few_tokens_f32_bit_exact(gpu, orc, M, K, N, offset):
    announce(f"exact f32 K2 M={M} K={K} N={N} offset={offset}")
    run_cases(gpu, orc, M, N, K, seed=M * 37 + K + N, kernel=2, what="K2", offset=offset)


# --------------------------------------------------- K2 tile kernel, 9..16 tokens --
TILE = [
    # M, K, N, split expected: the tile kernel and its split sum over the workspace
    (16, 14336, 4096, True), (9, 6200, 37, True), (13, 6144, 8192, True),
    (12, 8192, 3072, True), (16, 9001, 300, True),
    # wider than the tile kernel takes: the stream kernel
    (16, 4096, 14336, False), (10, 3072, 9216, False),
]


@pytest.mark.parametrize("M,K,N,split", TILE)
def test_gemv_tile_f32_bit_exact(gpu, orc, M, K, N, split):
    announce(f"exact f32 K2 tile M={M} K={K} N={N}")
    ws = _lib.lib().t81_hip_ternary_matmul_workspace_size(M, N, K, _lib.DTYPE_F32)
    assert (ws > 0) == split, f"workspace {ws} B"
    run_cases(gpu, orc, M, N, K, seed=M * 41 + K + N, kernel=2, what="K2 tile")


# ---------------------------------------------- K3 eight-wave, aligned x, 17..64 --
ALIGNED = [(17, 4100, 3000), (24, 3072, 3072), (32, 4096, 14336), (32, 14336, 4096),
           (33, 3072, 9216), (40, 8192, 3072), (32, 8192, 3072), (48, 4104, 1000),
           (49, 4096, 6144), (64, 14336, 4096), (64, 3072, 16384), (20, 1000, 37)]


@pytest.mark.parametrize("M,K,N", ALIGNED)
def test_k3_small_m_aligned_f32_bit_exact(gpu, orc, M, K, N):
    """17..64 tokens at a 16-byte aligned x: the eight-wave kernel's vector-load path, two
    limbs per k-step, four (and 128-row tiles below 16384 rows) over K > 8192, or at <= 32
    tokens over K >= 8192 or N >= 8192; split over the workspace."""
    announce(f"exact f32 K3 aligned M={M} K={K} N={N}")
    run_cases(gpu, orc, M, N, K, seed=M * 53 + K + N, kernel=3, what="aligned")


# ------------------------------------------------------ K3 eight-wave, 17..64 --
EIGHT = [(48, 4104, 1000), (32, 3000, 4096), (64, 4096, 6144), (17, 4100, 3000),
         (20, 14336, 4096), (33, 3072, 9216), (64, 8192, 3072), (17, 8192, 8192),
         (24, 3072, 9216)]


@pytest.mark.parametrize("M,K,N", EIGHT)
def test_k3_eight_wave_f32_bit_exact(gpu, orc, M, K, N):
    """17..64 tokens with x one element off 16-byte alignment (element loads): with the
    workspace (K split, partial sums added in split order by a second kernel) and without
    it (one launch over all of K)."""
    announce(f"exact f32 K3 eight-wave M={M} K={K} N={N}")
    lib = _lib.lib()
    assert lib.t81_hip_ternary_matmul_workspace_size(M, N, K, _lib.DTYPE_F32) > 0
    packed, acc, xg, cg, bg, c, bias = run_cases(gpu, orc, M, N, K, seed=M * 43 + K + N,
                                                 kernel=3, what="split-K", offset=1)
    s = torch.cuda.current_stream().cuda_stream
    for alpha, beta, use_bias in EPILOGUES:
        plain = cg.clone()
        _lib.check(lib.t81_hip_ternary_matmul(xg.data_ptr(), _lib.DTYPE_F32, packed.data_ptr(),
                                              plain.data_ptr(), M, N, K, alpha, beta,
                                              bg.data_ptr() if use_bias else None, s))
        want = fixed_point_expected(acc, alpha, beta, c.numpy() if beta else None,
                                    bias.numpy() if use_bias else None)
        assert_bits(plain.cpu().numpy(), want, f"no workspace alpha={alpha} beta={beta}")


# ------------------------------------------------------------------ K3, M > 64 --
BIG = [(300, 3000, 1500), (100, 4096, 2000), (65, 14336, 700)]


@pytest.mark.parametrize("M,K,N", BIG)
def test_k3_f32_bit_exact(gpu, orc, M, K, N):
    announce(f"exact f32 K3 M={M} K={K} N={N}")
    run_cases(gpu, orc, M, N, K, seed=M * 47 + K + N, kernel=3, what="K3")


def test_k3_config4_f32_sampled_and_full(gpu, orc):
    """Config 4's 4096 -> 6144 at M = 512 with float32 activations: every output against a
    float64 product of the unpacked trits on the GPU (exact: multiples of 2^-8 far below
    2^53), that product against the C oracle on a sample of tokens x rows."""
    M, K, N = 512, 4096, 6144
    announce(f"exact f32 K3 config-4 M={M} K={K} N={N}")
    _, a, b, x, c, bias = problem(M, N, K, seed=4)
    g = torch.Generator("cpu").manual_seed(5)
    w = torch.randn((N, K), generator=g)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    del w
    xg, cg, bg = x.to(gpu), c.to(gpu), bias.to(gpu)
    tt = ops.unpack(packed, N, K).to(torch.float64).t().contiguous()
    exact = torch.matmul(xg.double(), tt)
    del tt
    rng = np.random.default_rng(6)
    toks = np.unique(np.concatenate([[0, M - 1, 255, 256], rng.choice(M, 24, replace=False)]))
    rows = np.unique(np.concatenate([[0, N - 1], rng.choice(N, 64, replace=False)]))
    pk = packed.cpu().numpy()[rows]
    acc_s = fixed_point_acc256(orc, a[toks], b[toks], pk, K)
    tsel, rsel = torch.from_numpy(toks).to(gpu), torch.from_numpy(rows).to(gpu)
    np.testing.assert_array_equal(exact[tsel][:, rsel].cpu().numpy() * 256.0,
                                  acc_s.astype(np.float64), err_msg="GPU float64 vs oracle")
    for alpha, beta, use_bias in EPILOGUES:
        out = ops.ternary_matmul(xg, packed, K, alpha=alpha, beta=beta,
                                 c=cg.clone() if beta else None,
                                 bias=bg if use_bias else None, kernel=3)
        want = alpha * exact
        if beta:
            want = want + beta * cg.double()
        if use_bias:
            want = want + bg.double()
        assert float(want.abs().max()) < 2 ** 13, "epilogue must stay exact in float32"
        bad = int((out.double() != want).sum())
        assert bad == 0, f"alpha={alpha} beta={beta}: {bad} of {M * N} outputs differ"
        got_s = out[tsel][:, rsel].cpu().numpy()
        want_s = fixed_point_expected(acc_s, alpha, beta,
                                      c.numpy()[toks][:, rows] if beta else None,
                                      bias.numpy()[rows] if use_bias else None)
        assert_bits(got_s, want_s, f"sample alpha={alpha} beta={beta}")
    del exact
    torch.cuda.empty_cache()


# ------------------------------------------- K3 float32 as two bf16 launches --
PLANES = [
    # M, K, N, chunks: float32 activations past 64 tokens whose bf16 launches need no split
    # of their own run as the bf16 planes in the workspace, chunk by chunk (a chunk's two
    # planes within 64 MiB): one chunk, and three of 700 tokens over K = 16384
    (2048, 4096, 6144, 1), (700, 2048, 16384, 1), (2100, 16384, 14336, 3),
]


@pytest.mark.parametrize("M,K,N,chunks", PLANES)
def test_k3_f32_planes_bit_exact(gpu, orc, M, K, N, chunks):
    """Every output against a float64 product of the unpacked trits on the GPU (exact), that
    product against the C oracle on a sample, with the workspace (the planes path: beta and
    bias in the first launch, the lo plane added by the second) and without it (the
    eight-wave kernel)."""
    announce(f"exact f32 K3 planes M={M} K={K} N={N}")
    lib = _lib.lib()
    rows = -(-M // chunks)
    assert lib.t81_hip_ternary_matmul_workspace_size(M, N, K, _lib.DTYPE_F32) == 4 * rows * K
    _, a, b, x, c, bias = problem(M, N, K, seed=M + K + N)
    g = torch.Generator("cpu").manual_seed(7)
    w = torch.randn((N, K), generator=g)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    del w
    xg, cg, bg = x.to(gpu), c.to(gpu), bias.to(gpu)
    tt = ops.unpack(packed, N, K).to(torch.float64).t().contiguous()
    exact = torch.matmul(xg.double(), tt)
    del tt
    rng = np.random.default_rng(8)
    toks = np.unique(np.concatenate([[0, M - 1, rows - 1, min(rows, M - 1)],
                                     rng.choice(M, 12, replace=False)]))
    cols = np.unique(np.concatenate([[0, N - 1], rng.choice(N, 24, replace=False)]))
    acc_s = fixed_point_acc256(orc, a[toks], b[toks], packed.cpu().numpy()[cols], K)
    tsel, csel = torch.from_numpy(toks).to(gpu), torch.from_numpy(cols).to(gpu)
    np.testing.assert_array_equal(exact[tsel][:, csel].cpu().numpy() * 256.0,
                                  acc_s.astype(np.float64), err_msg="GPU float64 vs oracle")
    s = torch.cuda.current_stream().cuda_stream
    for alpha, beta, use_bias in EPILOGUES:
        want = alpha * exact
        if beta:
            want = want + beta * cg.double()
        if use_bias:
            want = want + bg.double()
        assert float(want.abs().max()) < 2 ** 13, "epilogue must stay exact in float32"
        out = ops.ternary_matmul(xg, packed, K, alpha=alpha, beta=beta,
                                 c=cg.clone() if beta else None,
                                 bias=bg if use_bias else None, kernel=3)
        bad = int((out.double() != want).sum())
        assert bad == 0, f"planes alpha={alpha} beta={beta}: {bad} of {M * N} outputs differ"
        plain = cg.clone()
        _lib.check(lib.t81_hip_ternary_matmul(xg.data_ptr(), _lib.DTYPE_F32, packed.data_ptr(),
                                              plain.data_ptr(), M, N, K, alpha, beta,
                                              bg.data_ptr() if use_bias else None, s))
        bad = int((plain.double() != want).sum())
        assert bad == 0, f"eight-wave alpha={alpha} beta={beta}: {bad} outputs differ"
    del exact
    torch.cuda.empty_cache()
