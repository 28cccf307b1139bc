"""K4 (the reference's literal limb-integer gemm_ternary) on the GPU: bit-exact with the
compiled reference's golden vectors and with the oracle, including +-inf and NaN."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from t81lib_amd import _lib, ops

pytestmark = pytest.mark.gpu


def announce(case: str) -> None:
    sys.__stderr__.write(f"[gpu case] {case}\n")
    sys.__stderr__.flush()


def k4(gpu, A, B, C, M, N, K, alpha, beta):
    c = torch.from_numpy(np.ascontiguousarray(C, np.float32)).to(gpu)
    ops.gemm_limb(torch.from_numpy(np.ascontiguousarray(A)).to(gpu),
                  torch.from_numpy(np.ascontiguousarray(B)).to(gpu), c, M, N, K, alpha, beta)
    return c.cpu().numpy()


def test_golden_cases_bit_exact(gpu, golden):
    for i, name in enumerate(golden["g_names"]):
        announce(f"K4 golden {name}")
        M, N, K = (int(v) for v in golden[f"g{i}_shape"])
        al, be = (float(v) for v in golden[f"g{i}_ab"])
        got = k4(gpu, golden[f"g{i}_A"], golden[f"g{i}_B"], golden[f"g{i}_C"], M, N, K, al, be)
        np.testing.assert_array_equal(got.view(np.uint32), golden[f"g{i}_out"].view(np.uint32),
                                      err_msg=str(name))


def test_mul_wide_pairs_bit_exact(gpu, golden):
    """Every mul_wide golden pair as a 1x1x1 GEMM with alpha = 1, beta = 0: the float of
    multiply_to_double (overflowing pairs give +-inf, the rest round identically)."""
    announce("K4 mul_wide pairs")
    a, b = golden["mw_a"], golden["mw_b"]
    n = len(a)
    # A: n x 1 limbs, B: 1 x n limbs, diagonal of the n x n result = the pair products
    A = a.reshape(n, 1, 16)
    B = b.reshape(1, n, 16)
    got = k4(gpu, A, B, np.zeros((n, n), np.float32), n, n, 48, 1.0, 0.0)
    want = golden["mw_prod"].astype(np.float32)
    np.testing.assert_array_equal(np.diag(got).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("M,N,KL,nz", [(1, 1, 1, 16), (33, 17, 5, 6), (64, 40, 22, 9),
                                        (7, 129, 3, 16), (16, 16, 0, 1),
                                        # lanes per output 16 / 32 / 64 at their edges, and
                                        # several passes of 64 limbs
                                        (4, 4, 16, 16), (9, 11, 17, 16), (5, 7, 33, 16),
                                        (3, 5, 100, 16), (2, 3, 130, 12)])
def test_random_vs_oracle(gpu, orc, M, N, KL, nz):
    announce(f"K4 random M={M} N={N} KL={KL} nz={nz}")
    rng = np.random.default_rng(M * N + KL)
    A = np.full((M, KL, 16), 13, np.uint8)
    B = np.full((KL, N, 16), 13, np.uint8)
    A[..., :nz] = rng.integers(0, 27, (M, KL, nz))
    B[..., :nz] = rng.integers(0, 27, (KL, N, nz))
    C = rng.standard_normal((M, N)).astype(np.float32)
    for alpha, beta in ((1.0, 0.0), (0.37, -0.7), (0.0, 0.5)):
        got = k4(gpu, A, B, C, M, N, KL * 48, alpha, beta)
        want = orc.gemm_limb(A, B, C, M, N, KL * 48, alpha, beta)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_config1_reference_path(gpu, orc):
    """Config 1 through the reference's literal matmul_input pipeline: W = N(0,0.02)
    1024x1024 ternarized at 0.45 (all-zero trits -> C = 0) and the effective W/0.02;
    X = N(0,1) 64x1024 quantized at 0.5 and packed column-wise; K4 vs oracle bit-exact."""
    announce("K4 config1")
    g = torch.Generator("cpu").manual_seed(0)
    w = torch.randn((1024, 1024), generator=g) * 0.02
    x = torch.randn((64, 1024), generator=g)
    xpack = orc.pack_cols(x.numpy(), np.float32(orc.torch_threshold(0.5)), 1)   # (22, 64, 16)
    for scale in (1.0, 1.0 / 0.02):
        wp = orc.pack_rows((w * scale).numpy(), np.float32(orc.torch_threshold(0.45)), 1)
        K = wp.shape[1] * 48
        got = k4(gpu, wp, xpack, np.zeros((1024, 64), np.float32), 1024, 64, K, 1.0, 0.0)
        rows = slice(0, 96)  # oracle on a band of output rows keeps the CPU time small
        want = orc.gemm_limb(wp[rows], xpack, np.zeros((96, 64), np.float32), 96, 64, K)
        np.testing.assert_array_equal(got[rows].view(np.uint32), want.view(np.uint32))
        if scale == 1.0:
            assert (got == 0).all()
        else:
            assert np.isinf(got).mean() > 0.9


@pytest.mark.parametrize("tokens,k,rows", [(6, 100, 40), (1, 48, 1), (17, 4097, 33), (33, 2000, 100),
                                           (16, 1536, 16), (5, 1, 3)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_fused_reference_matmul_input_matches_two_kernels(gpu, tokens, k, rows, dtype):
    """matmul_input_reference (quantize 0.5 + column pack inside the limb GEMM) equals
    pack_cols followed by gemm_limb bit for bit, for alpha / beta and ragged shapes."""
    announce(f"fused matmul_input {dtype} tokens={tokens} k={k} rows={rows}")
    g = torch.Generator("cpu").manual_seed(tokens * 131 + k + rows)
    w = torch.randn(rows, k, generator=g)
    x = (torch.randn(tokens, k, generator=g) * 0.8).to(dtype).to(gpu)
    wp = ops.quantize_pack(w.to(gpu), ops.torch_threshold(0.45), _lib.THR_TORCH)
    c0 = torch.randn(rows, tokens, generator=g).to(gpu)
    for alpha, beta in ((1.0, 0.0), (0.5, 1.5), (-2.0, 0.25)):
        want = c0.clone()
        ops.gemm_limb(wp, ops.pack_cols(x, 0.5, _lib.THR_TORCH), want, rows, tokens,
                      ops.limbs_for(k) * 48, alpha, beta)
        got = ops.matmul_input_reference(wp, x, 0.5, alpha, beta, c=c0.clone())
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32),
                                      want.cpu().numpy().view(np.uint32))


def test_fused_reference_config1_vs_oracle(gpu, orc):
    """BASELINE config 1 (effective W/0.02 variant): W 1024 x 1024 at 0.45, X 64 x 1024 at
    0.5, alpha 1 beta 0 -- the reference CPU gemm_ternary's output, bit-exact."""
    announce("fused matmul_input config 1")
    g = torch.Generator("cpu").manual_seed(0)
    w = torch.randn(1024, 1024, generator=g)
    x = torch.randn(64, 1024, generator=g)
    wp = orc.pack_rows(w.numpy(), np.float32(orc.torch_threshold(0.45)), 1)
    xp = orc.pack_cols(x.numpy(), np.float32(orc.torch_threshold(0.5)), 1)
    want = orc.gemm_limb(wp, xp, np.zeros((1024, 64), np.float32), 1024, 64, wp.shape[1] * 48)
    got = ops.matmul_input_reference(torch.from_numpy(wp).to(gpu), x.to(gpu), 0.5).cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
