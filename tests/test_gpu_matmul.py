"""K2 (GEMV, M <= 16) and K3 (GEMM) against the trit-dot oracle.

Integer activations: bit-exact int32.  Float activations: elementwise
|y - ref| <= rtol * (|alpha| sum_k |x_k t_k| + |beta c| + |bias|) + 1e-6 with rtol
the float32 summation bound of conftest.accum_rtol (about K * 2^-23; 4.9e-4 at
K = 4096 for bfloat16), capped by the north-star 1e-2 (bfloat16) / 1e-3 (float32).
Full-size configs are checked on a seeded sample of outputs plus linearity;
tests/test_gpu_exact.py pins the bfloat16 kernels bit for bit with integer-valued
activations.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from t81lib_amd import _lib, ops
from conftest import accum_rtol, fp_tolerance_ok

pytestmark = pytest.mark.gpu

def announce(case: str) -> None:
    sys.__stderr__.write(f"[gpu case] {case}\n")
    sys.__stderr__.flush()


def make_problem(M, N, K, dtype, seed, zeros=True):
    g = torch.Generator("cpu").manual_seed(seed)
    w = torch.randn((N, K), generator=g)            # effective weights W/0.02 ~ N(0,1)
    if not zeros:
        w = torch.sign(w) + (w == 0).float()
    if dtype == torch.int8:
        x = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    else:
        x = torch.randn((M, K), generator=g).to(dtype)
    c = torch.randn((M, N), generator=g)
    bias = torch.randn((N,), generator=g)
    return w, x, c, bias


def oracle_matmul(orc, x, packed_np, K, alpha, beta, c, bias, rows=None, cols=None):
    """Reference y (float64) and tolerance scale on the selected tokens/rows."""
    xs = x if rows is None else x[rows]
    pk = packed_np if cols is None else packed_np[cols]
    xd = xs.to(torch.float64).numpy()
    acc = orc.trit_matmul_f64(xd, pk, K)
    scale_acc = orc.trit_matmul_abs_f64(xd, pk, K)
    cc = c.to(torch.float64).numpy()
    bb = bias.to(torch.float64).numpy() if bias is not None else None
    if rows is not None:
        cc = cc[rows]
    if cols is not None:
        cc = cc[:, cols]
        bb = bb[cols] if bb is not None else None
    ref = alpha * acc + (beta * cc if beta != 0 else 0)
    scale = abs(alpha) * scale_acc + (abs(beta) * np.abs(cc) if beta != 0 else 0)
    if bb is not None:
        ref = ref + bb
        scale = scale + np.abs(bb)
    return ref, scale


def run(gpu, w, x, c, bias, K, alpha, beta, use_bias, kernel=None, thr=0.45):
    packed = ops.quantize_pack(w.to(gpu), thr, _lib.THR_CPP)
    cg = c.to(gpu).contiguous() if beta != 0 else None
    out = ops.ternary_matmul(x.to(gpu), packed, K, alpha=alpha, beta=beta, c=cg,
                             bias=bias.to(gpu) if use_bias else None, kernel=kernel)
    torch.cuda.synchronize()
    return packed.cpu().numpy(), out.cpu()


SMALL = [
    # M, N, K
    (1, 64, 48), (1, 100, 1024), (4, 33, 1000), (16, 257, 3072), (3, 16, 4096), (16, 48, 97),
    (1, 7, 1), (2, 5, 47),
    (17, 64, 96), (64, 96, 1024), (100, 200, 300), (128, 512, 4096), (37, 45, 4097),
    # 17..64 tokens, bf16: the column-block stream kernel, two and three blocks (one and two
    # row groups per workgroup), and two launches at 49..64
    (32, 300, 4104), (25, 6200, 1536), (40, 300, 4104), (48, 6200, 1536), (60, 300, 4104),
]


@pytest.mark.parametrize("M,N,K", SMALL)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_float_activations_vs_oracle(gpu, orc, M, N, K, dtype):
    announce(f"matmul {dtype} M={M} N={N} K={K}")
    w, x, c, bias = make_problem(M, N, K, dtype, seed=M * 1000 + N + K)
    for alpha, beta, use_bias in ((1.0, 0.0, False), (0.5, 1.0, True), (-2.0, 0.25, False)):
        packed, out = run(gpu, w, x, c, bias, K, alpha, beta, use_bias)
        ref, scale = oracle_matmul(orc, x, packed, K, alpha, beta, c, bias if use_bias else None)
        ok, worst, nbad = fp_tolerance_ok(out.numpy(), ref, scale, accum_rtol(K, dtype))
        assert ok, f"alpha={alpha} beta={beta}: {nbad} outside, worst rel {worst:.3g}"


@pytest.mark.parametrize("M,N,K", [(1, 64, 48), (4, 33, 1000), (16, 257, 3072), (17, 64, 96),
                                   (64, 96, 1024), (100, 200, 4097), (300, 128, 2048)])
def test_int8_activations_bit_exact(gpu, orc, M, N, K):
    announce(f"matmul int8 M={M} N={N} K={K}")
    w, x, c, bias = make_problem(M, N, K, torch.int8, seed=7 + M + N + K)
    packed, out = run(gpu, w, x, c, bias, K, 1.0, 0.0, False)
    want = orc.trit_matmul_i64(x.numpy(), packed, K)
    assert out.dtype == torch.int32
    np.testing.assert_array_equal(out.numpy().astype(np.int64), want)
    # beta = 1 accumulates into an int32 C exactly
    c0 = torch.randint(-1000, 1000, (M, N), dtype=torch.int32)
    packed_t = torch.from_numpy(packed).to(gpu)
    out2 = ops.ternary_matmul(x.to(gpu), packed_t, K, beta=1.0, c=c0.to(gpu))
    np.testing.assert_array_equal(out2.cpu().numpy().astype(np.int64), want + c0.numpy())


# M <= 4 decode shapes for the column-strip kernel: one row x 64 limbs per load (M = 1
# when that pads the row no more), 2 x 32 (M <= 2), 4 x 16 (M <= 4); several ranges per
# wave (K = 30000, 14336 at M = 2, 8192 at M = 3), workgroups cut off at N, partial
# last limbs, and K % 8 != 0 (element-wise activation loads).
STRIP = [
    (1, 77, 3072), (1, 50, 8192), (1, 33, 14336), (1, 40, 30000), (1, 300, 4096),
    (2, 45, 14336), (2, 129, 4096), (3, 31, 8192), (4, 70, 14336), (4, 1000, 3072),
    (3, 9, 100), (4, 18, 4100), (1, 5, 4100),
]


@pytest.mark.parametrize("M,N,K", STRIP)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.int8])
def test_decode_strip_shapes(gpu, orc, M, N, K, dtype):
    announce(f"strip {dtype} M={M} N={N} K={K}")
    w, x, c, bias = make_problem(M, N, K, dtype, seed=11 * M + N + K)
    if dtype == torch.int8:
        packed, out = run(gpu, w, x, c, bias, K, 1.0, 0.0, False, kernel=2)
        want = orc.trit_matmul_i64(x.numpy(), packed, K)
        np.testing.assert_array_equal(out.numpy().astype(np.int64), want)
        return
    for alpha, beta, use_bias in ((1.0, 0.0, False), (0.5, 1.0, True)):
        packed, out = run(gpu, w, x, c, bias, K, alpha, beta, use_bias, kernel=2)
        ref, scale = oracle_matmul(orc, x, packed, K, alpha, beta, c, bias if use_bias else None)
        ok, worst, nbad = fp_tolerance_ok(out.numpy(), ref, scale, accum_rtol(K, dtype))
        assert ok, f"alpha={alpha} beta={beta}: {nbad} outside, worst rel {worst:.3g}"


@pytest.mark.parametrize("M,N,K", [(1, 14336, 4096), (1, 14336, 6144), (2, 14336, 4096)])
def test_decode_strip_balanced_full_check(gpu, orc, M, N, K):
    """bf16 strip launches whose strip length is shortened by one load to even out the
    workgroups per CU (7 loads for 1 x 4096 x 14336, 14 for the other two): every
    output against the oracle, with alpha, beta and bias."""
    announce(f"strip balanced M={M} N={N} K={K}")
    w, x, c, bias = make_problem(M, N, K, torch.bfloat16, seed=3 * M + N + K)
    packed, out = run(gpu, w, x, c, bias, K, 0.75, 0.5, True, kernel=2)
    ref, scale = oracle_matmul(orc, x, packed, K, 0.75, 0.5, c, bias)
    ok, worst, nbad = fp_tolerance_ok(out.numpy(), ref, scale, accum_rtol(K, torch.bfloat16))
    assert ok, f"{nbad} outside, worst rel {worst:.3g}"


@pytest.mark.parametrize("M", [1, 8, 16])
def test_gemv_and_gemm_kernels_agree(gpu, orc, M):
    """M <= 16 is valid for both kernels: each must match the oracle on its own."""
    announce(f"K2 vs K3 M={M}")
    K = 2000
    w, x, c, bias = make_problem(M, 320, K, torch.bfloat16, seed=M)
    for kernel in (2, 3):
        packed, out = run(gpu, w, x, c, bias, K, 1.0, 0.0, True, kernel=kernel)
        ref, scale = oracle_matmul(orc, x, packed, K, 1.0, 0.0, c, bias)
        ok, worst, nbad = fp_tolerance_ok(out.numpy(), ref, scale, accum_rtol(K, torch.bfloat16))
        assert ok, f"kernel {kernel}: {nbad} outside, worst {worst:.3g}"


def test_unaligned_activations(gpu, orc):
    announce("matmul unaligned x view")
    M, N, K = 5, 70, 512
    w, x, c, bias = make_problem(M, N, K, torch.bfloat16, seed=3)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    big = torch.empty(M * K + 1, dtype=torch.bfloat16, device=gpu)
    big[1:] = x.to(gpu).reshape(-1)
    xv = big[1:].view(M, K)
    for kernel in (2, 3):
        out = ops.ternary_matmul(xv, packed, K, kernel=kernel).cpu()
        ref, scale = oracle_matmul(orc, x, packed.cpu().numpy(), K, 1.0, 0.0, c, None)
        ok, worst, nbad = fp_tolerance_ok(out.numpy(), ref, scale, accum_rtol(K, torch.bfloat16))
        assert ok, f"kernel {kernel}"


def test_empty_and_zero_k(gpu):
    announce("matmul empty / K=0")
    packed = torch.empty((4, 0, 16), dtype=torch.uint8, device=gpu)
    out = ops.ternary_matmul(torch.empty((3, 0), device=gpu), packed, 0,
                             bias=torch.arange(4.0, device=gpu))
    np.testing.assert_array_equal(out.cpu().numpy(), np.tile(np.arange(4.0), (3, 1)))
    out = ops.ternary_matmul(torch.empty((0, 48), device=gpu),
                             torch.empty((4, 1, 16), dtype=torch.uint8, device=gpu), 48)
    assert out.shape == (0, 4)


# ------------------------------------------------------------ full-size configs --
PHI3 = {"qkv": (3072, 9216), "o": (3072, 3072), "gate_up": (3072, 16384), "down": (8192, 3072)}


@pytest.mark.parametrize("layer", list(PHI3))
@pytest.mark.parametrize("M", [1, 4, 16])
def test_config3_phi3_decode(gpu, orc, layer, M):
    """Config 3: Phi-3-mini decode shapes, bf16 activations, fp32 bias, full oracle check."""
    K, N = PHI3[layer]
    announce(f"config3 {layer} M={M} K={K} N={N}")
    w, x, c, bias = make_problem(M, N, K, torch.bfloat16, seed=sum(map(ord, layer)) + M)
    packed, out = run(gpu, w, x, c, bias, K, 1.0, 0.0, True)
    ref, scale = oracle_matmul(orc, x, packed, K, 1.0, 0.0, c, bias)
    ok, worst, nbad = fp_tolerance_ok(out.numpy(), ref, scale, accum_rtol(K, torch.bfloat16))
    assert ok, f"{nbad} outside, worst {worst:.3g}"


LLAMA = {"qkv": (4096, 6144), "gate_up": (4096, 28672), "down": (14336, 4096)}


@pytest.mark.parametrize("layer", list(LLAMA))
@pytest.mark.parametrize("M", [512, 2048, 8192])
def test_config4_llama_prefill_sampled(gpu, orc, layer, M):
    """Config 4 at full size: a seeded sample of 48 tokens x 96 rows against the oracle for
    (alpha, beta) = (1, 0) and (0.5, 1), plus linearity in the activations."""
    K, N = LLAMA[layer]
    announce(f"config4 {layer} M={M} K={K} N={N}")
    g = torch.Generator("cpu").manual_seed(M + N)
    w = torch.randn((N, K), generator=g)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    gg = torch.Generator(gpu).manual_seed(M + N)
    cg_full = torch.randn((M, N), generator=gg, device=gpu)  # C is generated on the GPU
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    packed_np = packed.cpu().numpy()
    rows = np.sort(np.random.default_rng(M).choice(M, 48, replace=False))
    cols = np.sort(np.random.default_rng(N).choice(N, 96, replace=False))
    rows_t = torch.from_numpy(rows).to(gpu)
    cols_t = torch.from_numpy(cols).to(gpu)
    c_sample = cg_full[rows_t][:, cols_t].cpu().double().numpy()
    xd = x[torch.from_numpy(rows)].double().numpy()
    acc = orc.trit_matmul_f64(xd, packed_np[cols], K)
    acc_abs = orc.trit_matmul_abs_f64(xd, packed_np[cols], K)
    xg = x.to(gpu)
    for alpha, beta in ((1.0, 0.0), (0.5, 1.0)):
        cg = cg_full.clone() if beta else None
        out = ops.ternary_matmul(xg, packed, K, alpha=alpha, beta=beta, c=cg)
        got = out[rows_t][:, cols_t].cpu().numpy()
        ref = alpha * acc + beta * c_sample
        scale = abs(alpha) * acc_abs + abs(beta) * np.abs(c_sample)
        ok, worst, nbad = fp_tolerance_ok(got, ref, scale, accum_rtol(K, torch.bfloat16))
        assert ok, f"alpha={alpha}: {nbad} outside, worst {worst:.3g}"
        del cg, out
    # linearity: W(x1 + x2) == W x1 + W x2 (exact inputs in fp32, tolerance on the sums)
    x1 = x[:64].float().to(gpu)
    x2 = torch.randn((64, K), generator=g).to(gpu)
    y12 = ops.ternary_matmul(x1 + x2, packed, K, kernel=3)
    y1 = ops.ternary_matmul(x1, packed, K, kernel=3)
    y2 = ops.ternary_matmul(x2, packed, K, kernel=3)
    scale = (x1.abs() + x2.abs()).sum(1, keepdim=True)
    assert bool(((y12 - y1 - y2).abs() <= 2e-3 * scale + 1e-4).all())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.int8])
def test_k3_row_split_full_check(gpu, orc, dtype):
    """300 big tiles on 256 CUs: rows of whole rounds take 256 x 256 tiles and the rest
    256 x 128 tiles in a second launch (C row stride = N, bias offset).  Every output is
    checked, across the boundary, with ragged M and N."""
    M, N, K = 257, 256 * 150 + 13, 100
    announce(f"K3 row split {dtype} M={M} N={N} K={K}")
    w, x, c, bias = make_problem(M, N, K, dtype, seed=11)
    if dtype == torch.int8:
        packed, out = run(gpu, w, x, c, bias, K, 1.0, 0.0, False, kernel=3)
        want = orc.trit_matmul_i64(x.numpy(), packed, K)
        np.testing.assert_array_equal(out.numpy().astype(np.int64), want)
        return
    packed, out = run(gpu, w, x, c, bias, K, 0.75, 0.5, True, kernel=3)
    ref, scale = oracle_matmul(orc, x, packed, K, 0.75, 0.5, c, bias)
    ok, worst, nbad = fp_tolerance_ok(out.numpy(), ref, scale, accum_rtol(K, dtype))
    assert ok, f"{nbad} outside, worst {worst:.3g}"


@pytest.mark.parametrize("M,N,K", [(300, 256 * 160 + 13, 200), (512, 256 * 80, 192),
                                   (260, 256 * 81 + 7, 480), (512, 256 * 200 - 5, 96),
                                   (300, 192 * 128 - 5, 200)])
def test_k3_big_tile_full_check(gpu, orc, M, N, K):
    """bf16 activations with K % 8 == 0 and at least 160 tiles of 256 x 256: the
    one-wave-per-SIMD kernel (activation tile loaded straight into LDS, two k-steps per
    loop iteration plus a peeled odd step).  Every output is checked: odd and even step
    counts, K past the last whole step, ragged M and N, alpha/beta/bias, (first case)
    the rows past whole rounds as split-K items of the same launch, (fourth case)
    400 whole tiles on a grid of one workgroup per CU, so some workgroups take a second
    tile, and (last case) 192 tiles of 256 rows run as 256 tiles of 192 rows."""
    announce(f"K3 big tile M={M} N={N} K={K}")
    w, x, c, bias = make_problem(M, N, K, torch.bfloat16, seed=K)
    packed, out = run(gpu, w, x, c, bias, K, 0.75, 0.5, True, kernel=3)
    ref, scale = oracle_matmul(orc, x, packed, K, 0.75, 0.5, c, bias)
    ok, worst, nbad = fp_tolerance_ok(out.numpy(), ref, scale, accum_rtol(K, torch.bfloat16))
    assert ok, f"{nbad} outside, worst {worst:.3g}"
    packed, out = run(gpu, w, x, c, bias, K, 1.0, 0.0, False, kernel=3)
    ref, scale = oracle_matmul(orc, x, packed, K, 1.0, 0.0, c, None)
    ok, worst, nbad = fp_tolerance_ok(out.numpy(), ref, scale, accum_rtol(K, torch.bfloat16))
    assert ok, f"beta=0: {nbad} outside, worst {worst:.3g}"


@pytest.mark.parametrize("M,N,K", [(300, 1000, 4104), (260, 4096, 2000), (200, 700, 1536)])
def test_k3_split_k_full_check(gpu, orc, M, N, K):
    """Few output tiles (bf16, K % 8 == 0): K is split over several workgroups per tile,
    partial tiles go to a workspace and a second kernel sums them in split order.  Every
    output is checked against the oracle, with and without the workspace (the plain entry
    point does not split), and two runs of the split path are bit-identical."""
    announce(f"K3 split-K M={M} N={N} K={K}")
    lib = _lib.lib()
    ws_bytes = lib.t81_hip_ternary_matmul_workspace_size(M, N, K, _lib.DTYPE_BF16)
    assert ws_bytes > 0, "shape expected to split"
    w, x, c, bias = make_problem(M, N, K, torch.bfloat16, seed=M + K)
    packed, out = run(gpu, w, x, c, bias, K, 0.75, 0.5, True, kernel=3)
    ref, scale = oracle_matmul(orc, x, packed, K, 0.75, 0.5, c, bias)
    ok, worst, nbad = fp_tolerance_ok(out.numpy(), ref, scale, accum_rtol(K, torch.bfloat16))
    assert ok, f"split: {nbad} outside, worst {worst:.3g}"
    _, out2 = run(gpu, w, x, c, bias, K, 0.75, 0.5, True, kernel=3)
    assert torch.equal(out, out2), "split path is not deterministic"
    pg = torch.from_numpy(packed).to(gpu)
    xg = x.to(gpu)
    cg = c.to(gpu).contiguous()
    bg = bias.to(gpu)
    rc = lib.t81_hip_ternary_matmul(xg.data_ptr(), _lib.DTYPE_BF16, pg.data_ptr(), cg.data_ptr(),
                                    M, N, K, 0.75, 0.5, bg.data_ptr(),
                                    torch.cuda.current_stream().cuda_stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    ok, worst, nbad = fp_tolerance_ok(cg.cpu().numpy(), ref, scale, accum_rtol(K, torch.bfloat16))
    assert ok, f"no split: {nbad} outside, worst {worst:.3g}"


def test_k3_workspace_arguments(gpu):
    """The workspace entry point rejects a size without a pointer and a misaligned
    workspace, and runs without splitting when the workspace is too small."""
    lib = _lib.lib()
    M, N, K = 300, 1000, 4104
    x = torch.randn((M, K), device=gpu).to(torch.bfloat16)
    packed = ops.quantize_pack(torch.randn((N, K), device=gpu), 0.45, _lib.THR_CPP)
    c = torch.empty((M, N), device=gpu)
    s = torch.cuda.current_stream().cuda_stream
    args = (3, x.data_ptr(), _lib.DTYPE_BF16, packed.data_ptr(), c.data_ptr(), M, N, K, 1.0, 0.0,
            None)
    assert lib.t81_hip_ternary_matmul_ws(*args, None, 64, s) == _lib.EINVAL_POINTER
    buf = torch.empty(1 << 20, dtype=torch.uint8, device=gpu)
    assert lib.t81_hip_ternary_matmul_ws(*args, buf.data_ptr() + 4, 64, s) == _lib.EINVAL_POINTER
    assert lib.t81_hip_ternary_matmul_ws(*args, buf.data_ptr(), 1 << 20, s) == 0
    want = ops.ternary_matmul(x, packed, K, kernel=3)
    torch.cuda.synchronize()
    assert torch.allclose(c, want, rtol=1e-5, atol=1e-3)


def test_k3_remainder_split_k(gpu, orc):
    """320 big tiles on 256 CUs: whole rounds of big tiles for the first 32768 rows, and
    the remaining 8192 rows as split-K big tiles over the workspace (C written through a
    row stride, bias offset).  Sampled columns on both sides of the boundary against the
    oracle, and all outputs against the path without a workspace (eight-wave remainder)."""
    M, N, K = 300, 256 * 160, 1536
    announce(f"K3 remainder split-K M={M} N={N} K={K}")
    lib = _lib.lib()
    assert lib.t81_hip_ternary_matmul_workspace_size(M, N, K, _lib.DTYPE_BF16) > 0
    g = torch.Generator("cpu").manual_seed(21)
    w = torch.randn((N, K), generator=g)
    x = torch.randn((M, K), generator=g).to(torch.bfloat16)
    c = torch.randn((M, N), generator=g)
    bias = torch.randn((N,), generator=g)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    xg, cg, bg = x.to(gpu), c.to(gpu), bias.to(gpu)
    out = ops.ternary_matmul(xg, packed, K, alpha=0.75, beta=0.5, c=cg.clone(), bias=bg, kernel=3)
    plain = cg.clone()
    _lib.check(lib.t81_hip_ternary_matmul(xg.data_ptr(), _lib.DTYPE_BF16, packed.data_ptr(),
                                          plain.data_ptr(), M, N, K, 0.75, 0.5, bg.data_ptr(),
                                          torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    cols = np.sort(np.concatenate([np.random.default_rng(1).choice(32768, 64, replace=False),
                                   32768 + np.random.default_rng(2).choice(8192, 64, replace=False)]))
    packed_np = packed.cpu().numpy()
    ref, scale = oracle_matmul(orc, x, packed_np, K, 0.75, 0.5, c, bias, cols=cols)
    got = out.cpu().numpy()[:, cols]
    ok, worst, nbad = fp_tolerance_ok(got, ref, scale, accum_rtol(K, torch.bfloat16))
    assert ok, f"{nbad} outside, worst {worst:.3g}"
    assert torch.allclose(out, plain, rtol=1e-5, atol=1e-3)


@pytest.mark.parametrize("M,N,K,dtype", [(16, 4096, 14336, torch.bfloat16),
                                         (5, 1000, 14336, torch.float32),
                                         (9, 3000, 9000, torch.int8),
                                         (16, 300, 5767, torch.bfloat16),
                                         (12, 14336, 4096, torch.bfloat16)])
def test_k2_m5_to_16_full_check(gpu, orc, M, N, K, dtype):
    """5 <= M <= 16 decode shapes (long and short K, ragged K, few and many row blocks):
    every output against the oracle through the Python path and through the plain C
    entry point; int8 bit-exact."""
    announce(f"K2 M={M} N={N} K={K} {dtype}")
    w, x, c, bias = make_problem(M, N, K, dtype, seed=N + M)
    lib = _lib.lib()
    code = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32, torch.int8: _lib.DTYPE_I8}[dtype]
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    packed_np = packed.cpu().numpy()
    xg = x.to(gpu)
    s = torch.cuda.current_stream().cuda_stream
    if dtype == torch.int8:
        want = orc.trit_matmul_i64(x.numpy(), packed_np, K)
        out = ops.ternary_matmul(xg, packed, K)
        plain = torch.empty((M, N), dtype=torch.int32, device=gpu)
        _lib.check(lib.t81_hip_ternary_matmul(xg.data_ptr(), code, packed.data_ptr(),
                                              plain.data_ptr(), M, N, K, 1.0, 0.0, None, s))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), want)
        np.testing.assert_array_equal(plain.cpu().numpy().astype(np.int64), want)
        return
    cg, bg = c.to(gpu), bias.to(gpu)
    out = ops.ternary_matmul(xg, packed, K, alpha=0.75, beta=0.5, c=cg.clone(), bias=bg)
    plain = cg.clone()
    _lib.check(lib.t81_hip_ternary_matmul(xg.data_ptr(), code, packed.data_ptr(), plain.data_ptr(),
                                          M, N, K, 0.75, 0.5, bg.data_ptr(), s))
    torch.cuda.synchronize()
    ref, scale = oracle_matmul(orc, x, packed_np, K, 0.75, 0.5, c, bias)
    for name, got in (("workspace", out), ("plain", plain)):
        ok, worst, nbad = fp_tolerance_ok(got.cpu().numpy(), ref, scale, accum_rtol(K, dtype))
        assert ok, f"{name}: {nbad} outside, worst {worst:.3g}"


@pytest.mark.parametrize("M,N,K,dtype,splits", [
    (9, 37, 6200, torch.float32, 5),       # 33 sub-blocks: one active wave in the last split
    (16, 4096, 14336, torch.bfloat16, 0),  # aligned bf16: the staged stream kernel instead
    (11, 3000, 9001, torch.bfloat16, 6),   # K % 8 != 0 (element loads)
    (16, 4100, 14400, torch.int8, 0),      # int8, K % 16 == 0: the staged stream kernel
    (16, 4100, 14408, torch.int8, -1),     # rows past N in the last block (-1: any split)
    (13, 8192, 6144, torch.float32, 4),    # four row groups per workgroup
    (12, 8193, 6144, torch.bfloat16, 0),   # wider than the tile kernel takes
    (8, 3000, 9000, torch.bfloat16, 0),    # fewer tokens than it takes
    (16, 14336, 4096, torch.int8, 0)])     # short K: the stream kernel
def test_k2_tile_kernel_plans(gpu, orc, M, N, K, dtype, splits):
    """K2 for 9..16 tokens over a long K with a workspace (gemv_tile_kernel; splits == 0:
    a shape it leaves to the stream / wave kernels): every output against the oracle
    (int8 bit-exact), run twice with identical bits (fixed summation order), and the
    workspace size reported for its K splits."""
    announce(f"K2 tile M={M} N={N} K={K} {dtype}")
    lib = _lib.lib()
    code = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32, torch.int8: _lib.DTYPE_I8}[dtype]
    ws = lib.t81_hip_ternary_matmul_workspace_size(M, N, K, code)
    if splits >= 0:
        assert ws == (4 * splits * M * N if splits > 1 else 0)
    else:
        assert ws > 0 and ws % (4 * M * N) == 0, "shape expected to split K"
    w, x, c, bias = make_problem(M, N, K, dtype, seed=3 * N + K + M)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    packed_np = packed.cpu().numpy()
    xg = x.to(gpu)
    if dtype == torch.int8:
        want = orc.trit_matmul_i64(x.numpy(), packed_np, K)
        cg = torch.randint(-1000, 1000, (M, N), dtype=torch.int32, device=gpu)
        outs = [ops.ternary_matmul(xg, packed, K, beta=1.0, c=cg.clone(), kernel=2) for _ in range(2)]
        torch.cuda.synchronize()
        np.testing.assert_array_equal(outs[0].cpu().numpy().astype(np.int64),
                                      want + cg.cpu().numpy().astype(np.int64))
    else:
        cg, bg = c.to(gpu), bias.to(gpu)
        outs = [ops.ternary_matmul(xg, packed, K, alpha=-1.25, beta=0.5, c=cg.clone(), bias=bg,
                                   kernel=2) for _ in range(2)]
        torch.cuda.synchronize()
        ref, scale = oracle_matmul(orc, x, packed_np, K, -1.25, 0.5, c, bias)
        ok, worst, nbad = fp_tolerance_ok(outs[0].cpu().numpy(), ref, scale, accum_rtol(K, dtype))
        assert ok, f"{nbad} outside, worst {worst:.3g}"
    assert torch.equal(outs[0], outs[1]), "two runs of the same call differ"


@pytest.mark.parametrize("M,N,K,dtype", [(56, 4096, 14340, torch.bfloat16),
                                         (60, 4096, 14336, torch.bfloat16),
                                         (48, 1000, 4104, torch.float32),
                                         (20, 3000, 9000, torch.int8),
                                         (100, 2000, 4800, torch.int8),
                                         (64, 6144, 4100, torch.bfloat16),
                                         (300, 1500, 3000, torch.float32),
                                         (50, 16384, 3076, torch.bfloat16),
                                         (40, 1000, 4100, torch.bfloat16),
                                         (20, 20000, 2008, torch.int8)])
def test_k3_eight_wave_split_k_full_check(gpu, orc, M, N, K, dtype):
    """Launches of the eight-wave kernel with few tiles (17 <= M <= 64: fp32 activations,
    int8 with K % 16 != 0, bf16 with K % 8 != 0 or, past 48 tokens, K > 8192, past 32
    tokens, K >= 12288 for bf16) split K: each
    split writes its raw sums (int32 for int8, exact) as a row-major M x N matrix in the
    workspace and a second kernel adds them in split order.  Every output against the
    oracle, with and without the workspace; int8 bit-exact."""
    announce(f"K3 eight-wave split-K M={M} N={N} K={K} {dtype}")
    lib = _lib.lib()
    code = {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32, torch.int8: _lib.DTYPE_I8}[dtype]
    assert lib.t81_hip_ternary_matmul_workspace_size(M, N, K, code) > 0, "shape expected to split"
    w, x, c, bias = make_problem(M, N, K, dtype, seed=M * 7 + K)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    packed_np = packed.cpu().numpy()
    xg = x.to(gpu)
    s = torch.cuda.current_stream().cuda_stream
    if dtype == torch.int8:
        want = orc.trit_matmul_i64(x.numpy(), packed_np, K)
        cg = c.round().to(torch.int32).to(gpu)
        out = ops.ternary_matmul(xg, packed, K, beta=1.0, c=cg.clone())
        plain = cg.clone()
        _lib.check(lib.t81_hip_ternary_matmul(xg.data_ptr(), code, packed.data_ptr(),
                                              plain.data_ptr(), M, N, K, 1.0, 1.0, None, s))
        torch.cuda.synchronize()
        want = want + cg.cpu().numpy().astype(np.int64)
        np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), want)
        np.testing.assert_array_equal(plain.cpu().numpy().astype(np.int64), want)
        return
    cg, bg = c.to(gpu), bias.to(gpu)
    out = ops.ternary_matmul(xg, packed, K, alpha=0.75, beta=0.5, c=cg.clone(), bias=bg)
    plain = cg.clone()
    _lib.check(lib.t81_hip_ternary_matmul(xg.data_ptr(), code, packed.data_ptr(), plain.data_ptr(),
                                          M, N, K, 0.75, 0.5, bg.data_ptr(), s))
    torch.cuda.synchronize()
    ref, scale = oracle_matmul(orc, x, packed_np, K, 0.75, 0.5, c, bias)
    for name, got in (("workspace", out), ("plain", plain)):
        ok, worst, nbad = fp_tolerance_ok(got.cpu().numpy(), ref, scale, accum_rtol(K, dtype))
        assert ok, f"{name}: {nbad} outside, worst {worst:.3g}"
