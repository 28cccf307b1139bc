"""Bit-exact pins of the bfloat16 hot-path kernels (K2 decode GEMV, K3 prefill GEMM).

The activations are integers with |x| <= 127, which bfloat16 holds exactly.  Every
product x * t (t a trit) is then an integer, every partial sum stays below 2^24 in
magnitude, and float32 adds such integers without rounding in any order: the
kernel's float32 output must equal the int64 oracle bit for bit.  alpha = 0.5,
integer C and integer bias keep the epilogue exact too (alpha * acc has one
fractional bit).  A kernel that drops or repeats any limb, any trit, any split or
any tile fails these tests on essentially every output it touches.

Paths covered (shapes taken from the configs):
* K2 column-strip kernel, natural trit order: one token, 4096 -> 14336 (two 32-limb
  rows per load, seven loads per strip) and the 3072-wide Phi-3 shapes (one row x
  64 limbs per load);
* K2 column-strip kernel, padded order: one token at K = 8192 / 14336; 2 tokens
  (S = 8) and 3-4 tokens (S = 4);
* K2 gemv.hip: 8, 12 and 16 tokens (activations staged in LDS, or streamed with
  two or four row groups per fragment);
* K3 big-tile kernel (one wave per SIMD): config 4 at M = 2048 (gate_up: whole
  256 x 256 tiles for the first 24576 rows, half-width 256 x 128 tiles for the
  remaining 4096 in the same launch, an odd step count with the peeled last step),
  M = 512 (every tile split over the workspace) and M = 8192, plus small shapes with
  odd, even and single step counts, ragged M and N and K past the last whole step,
  for whole, half-width and split-K items.

Full-size K3 outputs are checked twice: a seeded sample of tokens x rows, drawn
from every region of the launch, against the C oracle on the packed bytes, and
every output against a float64 product of the unpacked trits on the GPU (exact:
integer sums far below 2^53).
"""

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


def int_problem(M, N, K, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    w = torch.randn((N, K), generator=g)                        # ~1/3 zero trits at 0.45
    x = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int32)
    x[:, ::97] = 0                                              # a few exact zeros
    c = torch.randint(-1000, 1001, (M, N), generator=g).float()
    bias = torch.randint(-1000, 1001, (N,), generator=g).float()
    return w, x, c, bias


def expected(acc: np.ndarray, alpha: float, beta: float, c: np.ndarray, bias) -> np.ndarray:
    """alpha * acc + beta * c + bias, exact in float64, then float32 (exact: < 2^24)."""
    y = alpha * acc.astype(np.float64)
    if beta != 0.0:
        y = y + beta * c.astype(np.float64)
    if bias is not None:
        y = y + bias.astype(np.float64)
    assert np.abs(y).max(initial=0.0) < 2 ** 23, "test values must stay exact in float32"
    return y.astype(np.float32)


def assert_bits(got: np.ndarray, want: np.ndarray, what: str) -> None:
    got = np.ascontiguousarray(got, np.float32)
    bad = got.view(np.uint32) != want.view(np.uint32)
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"{what}: {int(bad.sum())} of {bad.size} outputs differ; first at "
                             f"{tuple(int(v) for v in i)}: got {got[tuple(i)]!r}, "
                             f"want {want[tuple(i)]!r}")


# --------------------------------------------------------------------- K2 --
PHI3 = {"qkv": (3072, 9216), "o": (3072, 3072), "gate_up": (3072, 16384), "down": (8192, 3072)}
LLAMA = {"qkv": (4096, 6144), "gate": (4096, 14336), "down": (14336, 4096)}

K2_CASES = (
    [("phi3." + name, M, K, N) for name, (K, N) in PHI3.items() for M in (1, 4, 16)]
    + [("llama.gate", M, 4096, 14336) for M in (1, 2, 3, 8, 12, 16)]
    + [("llama.down", M, 14336, 4096) for M in (1, 2, 4, 5, 8, 16)]
    # staged activation pieces at few tokens (one row group per workgroup), and at
    # 9..16 tokens over two row groups per workgroup
    + [("phi3.down", 5, 8192, 3072), ("phi3.o", 12, 3072, 3072), ("wide", 10, 3072, 6144)]
    + [("llama.qkv", 1, 4096, 6144), ("ragged", 1, 4100, 77), ("ragged", 3, 1000, 333),
       ("ragged", 13, 5767, 300)]
    # the strip kernel at 5..8 tokens (S = 2, two kept entries per lane): >= 12288 rows and
    # K <= 4096, one range per wave or several (staged B), ragged N and K
    + [("phi3.gate_up", M, 3072, 16384) for M in (5, 6, 7)]
    + [("ragged", 7, 4000, 12300), ("ragged", 6, 1000, 13000), ("ragged", 5, 4099, 12289)]
)


@pytest.mark.parametrize("name,M,K,N", K2_CASES)
def test_k2_integer_bf16_bit_exact(gpu, orc, name, M, K, N):
    announce(f"exact K2 {name} M={M} K={K} N={N}")
    w, x, c, bias = int_problem(M, N, K, seed=M * 7919 + K + N)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    packed_np = packed.cpu().numpy()
    acc = orc.trit_matmul_i64(x.to(torch.int8).numpy(), packed_np, K) if K <= 131071 else None
    xg = x.to(torch.bfloat16).to(gpu)
    assert torch.equal(xg.float().cpu(), x.float()), "integers must be exact in bfloat16"
    cg = c.to(gpu)
    for alpha, beta, use_bias in ((1.0, 0.0, False), (0.5, 1.0, True), (-2.0, 0.5, True)):
        out = ops.ternary_matmul(xg, packed, K, alpha=alpha, beta=beta,
                                 c=cg.clone() if beta else None,
                                 bias=bias.to(gpu) if use_bias else None, kernel=2)
        want = expected(acc, alpha, beta, c.numpy(), bias.numpy() if use_bias else None)
        assert_bits(out.cpu().numpy(), want, f"alpha={alpha} beta={beta} bias={use_bias}")


TWO_BLOCK_CASES = [
    # 17..32 tokens through the K3 entry: the column-block stream kernel with two blocks (one
    # row group per workgroup up to 4096 rows, two below 9216, two with four waves above),
    # ragged N and a K that ends inside a sub-block
    ("llama.down", 17, 14336, 4096), ("llama.gate", 24, 4096, 14336), ("llama.qkv", 32, 4096, 6144),
    ("phi3.o", 32, 3072, 3072), ("phi3.down", 32, 8192, 3072), ("phi3.gate_up", 32, 3072, 16384),
    ("ragged", 29, 4104, 333),
    # 33..48 tokens below K = 12288: three blocks, eight waves (one row group per workgroup
    # up to 4096 rows, two above); a third block of one token, of 16, and ragged shapes
    ("llama2.down", 33, 11008, 4096), ("llama.gate", 48, 4096, 14336), ("llama.qkv", 40, 4096, 6144),
    ("phi3.o", 48, 3072, 3072), ("phi3.down", 45, 8192, 3072), ("ragged", 37, 4104, 4133),
    # 49..64 tokens: two launches (tokens 0..31, then the rest: 17..32 of them)
    ("llama.gate", 64, 4096, 14336), ("phi3.o", 49, 3072, 3072), ("ragged", 57, 4104, 4133),
]


@pytest.mark.parametrize("name,M,K,N", TWO_BLOCK_CASES)
def test_two_block_integer_bf16_bit_exact(gpu, orc, name, M, K, N):
    announce(f"exact column-block M={M} {name} K={K} N={N}")
    lib = _lib.lib()
    assert lib.t81_hip_ternary_matmul_workspace_size(M, N, K, _lib.DTYPE_BF16) == 0
    w, x, c, bias = int_problem(M, N, K, seed=M * 131 + K + N)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    acc = orc.trit_matmul_i64(x.to(torch.int8).numpy(), packed.cpu().numpy(), K)
    xg = x.to(torch.bfloat16).to(gpu)
    cg = c.to(gpu)
    for alpha, beta, use_bias in ((1.0, 0.0, False), (0.5, 1.0, True), (-2.0, 0.5, True)):
        out = ops.ternary_matmul(xg, packed, K, alpha=alpha, beta=beta,
                                 c=cg.clone() if beta else None,
                                 bias=bias.to(gpu) if use_bias else None, kernel=3)
        want = expected(acc, alpha, beta, c.numpy(), bias.numpy() if use_bias else None)
        assert_bits(out.cpu().numpy(), want, f"alpha={alpha} beta={beta} bias={use_bias}")


SMALL_LONG_K = [
    # M, K, N, dtypes: 49..64 tokens over K > 8192 (and bf16 33..48 over K >= 12288), which
    # the column-block kernel leaves to the eight-wave kernel: four limbs per k-step, 128-row
    # tiles two per CU below 16384 rows (256-row tiles from 16384), the K split over the
    # workspace; ragged K and N
    (49, 14336, 4096, "bf16"), (64, 11008, 4096, "bf16"), (64, 14336, 16384, "bf16"),
    (57, 9000, 1000, "bf16"), (33, 14336, 4096, "bf16"), (48, 12288, 8192, "bf16"),
    (40, 13000, 999, "bf16"),
    (49, 14336, 4096, "int8"), (64, 11008, 4096, "int8"), (64, 14336, 16384, "int8"),
    (57, 9000, 1000, "int8"),
]


@pytest.mark.parametrize("M,K,N,dt", SMALL_LONG_K)
def test_small_m_long_k_bit_exact(gpu, orc, M, K, N, dt):
    """bf16 (integer values) and int8 activations, with the workspace (split K) and without
    it (one launch over all of K): every output equals the int64 oracle."""
    announce(f"exact small-M long-K {dt} M={M} K={K} N={N}")
    lib = _lib.lib()
    code = _lib.DTYPE_BF16 if dt == "bf16" else _lib.DTYPE_I8
    assert lib.t81_hip_ternary_matmul_workspace_size(M, N, K, code) > 0
    w, x, c, bias = int_problem(M, N, K, seed=M * 7 + K + N)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    acc = orc.trit_matmul_i64(x.to(torch.int8).numpy(), packed.cpu().numpy(), K)
    xg = (x.to(torch.bfloat16) if dt == "bf16" else x.to(torch.int8)).to(gpu)
    s = torch.cuda.current_stream().cuda_stream
    if dt == "bf16":
        cg = c.to(gpu)
        for alpha, beta, use_bias in ((1.0, 0.0, False), (0.5, 1.0, True)):
            want = expected(acc, alpha, beta, c.numpy(), bias.numpy() if use_bias else None)
            out = ops.ternary_matmul(xg, packed, K, alpha=alpha, beta=beta,
                                     c=cg.clone() if beta else None,
                                     bias=bias.to(gpu) if use_bias else None, kernel=3)
            assert_bits(out.cpu().numpy(), want, f"split alpha={alpha} beta={beta}")
            plain = cg.clone()
            _lib.check(lib.t81_hip_ternary_matmul(
                xg.data_ptr(), code, packed.data_ptr(), plain.data_ptr(), M, N, K, alpha, beta,
                bias.to(gpu).data_ptr() if use_bias else None, s))
            assert_bits(plain.cpu().numpy(), want, f"no workspace alpha={alpha} beta={beta}")
    else:
        ci = torch.randint(-(1 << 20), 1 << 20, (M, N), dtype=torch.int32)
        out = ops.ternary_matmul(xg, packed, K, kernel=3)
        np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), acc)
        out = ops.ternary_matmul(xg, packed, K, beta=1.0, c=ci.to(gpu), kernel=3)
        np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), acc + ci.numpy())
        plain = ci.to(gpu)
        _lib.check(lib.t81_hip_ternary_matmul(xg.data_ptr(), code, packed.data_ptr(),
                                              plain.data_ptr(), M, N, K, 1.0, 1.0, None, s))
        np.testing.assert_array_equal(plain.cpu().numpy().astype(np.int64), acc + ci.numpy())


# --------------------------------------------------------------------- K3 --
def _sample(M, N, n1, seed, tokens=48, rows=96):
    """Tokens from every 256-token tile; rows from both the whole-tile region [0, n1)
    and the split region [n1, N), including each region's first and last row."""
    rng = np.random.default_rng(seed)
    toks = set(rng.choice(M, min(tokens, M), replace=False).tolist())
    toks.update({0, M - 1, min(M - 1, 255), min(M - 1, 256)})
    picks = {0, N - 1}
    if 0 < n1 < N:
        picks.update({n1 - 1, n1})
        picks.update(rng.choice(n1, rows // 2, replace=False).tolist())
        picks.update((n1 + rng.choice(N - n1, rows // 2, replace=False)).tolist())
    else:
        picks.update(rng.choice(N, min(rows, N), replace=False).tolist())
    return np.array(sorted(toks)), np.array(sorted(picks))


def whole_round_rows(M: int, N: int) -> int:
    """Weight rows the K3 launcher runs as whole 256 x 256 tiles (the rest, if any, as
    split-K items): whole rounds of one tile per CU when the last round would be at most
    half full, else all rows (the launcher's rule)."""
    tiles_m = -(-M // 256)
    tiles = -(-N // 256) * tiles_m
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    rem = tiles % cus
    n1 = (tiles - rem) // tiles_m * 256
    if tiles >= 160 and tiles > cus and rem != 0 and 2 * rem <= cus and 0 < n1 < N:
        return n1
    return N


def tall_rows(M: int, N: int, K: int):
    """Weight rows the K3 launcher runs as whole 512 x 128 tiles when it takes the tall
    form (the rest as one round of 512 x 64 half-width tiles), or None when it does not
    (the launcher's rule for aligned bf16 activations)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    tiles_m = -(-M // 128)
    tiles = -(-N // 512) * tiles_m
    L = -(-K // 48)
    if M <= 64 or tiles < cus or 512 * L * 16 >= 0x7FFFFFFF:
        return None
    rem = tiles % cus
    if rem == 0:
        return N
    n1 = (tiles - rem) // tiles_m * 512
    if not 0 < n1 < N:
        return None
    t = -(-(N - n1) // 512) * -(-M // 64)
    return n1 if 4 * t >= 3 * cus and t <= cus else None


def _gpu_exact_product(xg_f64: torch.Tensor, packed: torch.Tensor, N: int, K: int) -> torch.Tensor:
    """x @ T^T in float64 on the GPU from the unpacked trits (exact for these integers)."""
    tt = ops.unpack(packed, N, K).to(torch.float64).t().contiguous()   # (K, N)
    return torch.matmul(xg_f64, tt)


K3_FULL = [
    # name, M, K, N
    ("llama.gate_up", 2048, 4096, 28672),   # whole tiles + half-width tiles, odd steps
    ("llama.qkv", 2048, 4096, 6144),
    ("llama.down", 2048, 14336, 4096),      # every tile split over the workspace
    ("llama.qkv", 512, 4096, 6144),         # every tile split over the workspace
    ("llama.down", 512, 14336, 4096),
    ("llama.qkv", 8192, 4096, 6144),
]


@pytest.mark.parametrize("name,M,K,N", K3_FULL)
def test_k3_config4_integer_bf16_bit_exact(gpu, orc, name, M, K, N):
    announce(f"exact K3 {name} M={M} K={K} N={N}")
    g = torch.Generator("cpu").manual_seed(M + N + K)
    w = torch.randn((N, K), generator=g)
    x = torch.randint(-127, 128, (M, K), generator=g, dtype=torch.int32)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    del w
    xg = x.to(torch.bfloat16).to(gpu)
    gg = torch.Generator(gpu).manual_seed(M * 3 + N)
    cg = torch.randint(-1000, 1001, (M, N), generator=gg, device=gpu).float()
    bias = torch.randint(-1000, 1001, (N,), generator=gg, device=gpu).float()
    exact = _gpu_exact_product(x.to(torch.float64).to(gpu), packed, N, K)
    toks, rows = _sample(M, N, whole_round_rows(M, N), seed=M + K)
    packed_np = packed.cpu().numpy()
    acc_s = orc.trit_matmul_i64(x[torch.from_numpy(toks)].to(torch.int8).numpy(),
                                packed_np[rows], K)
    np.testing.assert_array_equal(
        exact[torch.from_numpy(toks).to(gpu)][:, torch.from_numpy(rows).to(gpu)]
        .cpu().numpy().astype(np.int64), acc_s, err_msg="float64 GPU product vs oracle")
    for alpha, beta, use_bias in ((1.0, 0.0, False), (0.5, 1.0, True)):
        out = ops.ternary_matmul(xg, packed, K, alpha=alpha, beta=beta,
                                 c=cg.clone() if beta else None,
                                 bias=bias if use_bias else None, kernel=3)
        want_full = alpha * exact
        if beta:
            want_full = want_full + beta * cg.double()
        if use_bias:
            want_full = want_full + bias.double()
        assert float(want_full.abs().max()) < 2 ** 23
        bad = int((out.double() != want_full).sum())
        assert bad == 0, f"alpha={alpha} beta={beta}: {bad} of {M * N} outputs differ"
        tsel = torch.from_numpy(toks).to(gpu)
        rsel = torch.from_numpy(rows).to(gpu)
        got_s = out[tsel][:, rsel].cpu().numpy()
        c_s = cg[tsel][:, rsel].cpu().numpy()
        want_s = expected(acc_s, alpha, beta, c_s, bias[rsel].cpu().numpy() if use_bias else None)
        assert_bits(got_s, want_s, f"sampled vs oracle alpha={alpha} beta={beta}")
        del out, want_full
    del exact
    torch.cuda.empty_cache()


K3_SMALL = [
    # M, N, K: >= 160 big tiles (whole-tile kernel), odd and even step counts, K past
    # the last whole step, ragged M / N, more tiles than CUs; then few tiles (split-K over
    # tall 512 x 128 tiles when the workspace is given, else the eight-wave kernel)
    (300, 256 * 160 + 13, 200), (512, 256 * 80, 192), (260, 256 * 81 + 7, 480),
    (512, 256 * 200 - 5, 96), (300, 1000, 4104), (260, 4096, 2000), (200, 700, 1536),
    (300, 256 * 160, 1536),
    # whole rounds of 256 x 256 tiles, the remaining rows as one round of half-width
    # 256 x 128 tiles (on 256 CUs: 192-256 of them), ragged M and N
    (1900, 256 * 44 + 13, 200),
    # whole rounds of 256 x 256 tiles for the first 32768 rows, the rest (88 half-width
    # tiles, too few for a round) as 2 x 2 split-K items over the workspace, where the tall
    # tiles' remainder fits neither (two splits of four k-steps)
    (512, 256 * 150, 768),
    # 160-255 tiles of 256 x 256 whose 384 x 128 tiles fit one round (on 256 CUs: 252 and
    # 192 of them): 384 x 128 tiles; a last tile of 7 rows (three steps), ragged M over
    # three token tiles (16 steps)
    (200, 192 * 250 + 7, 200), (300, 192 * 128 - 5, 1536),
]


@pytest.mark.parametrize("M,N,K", K3_SMALL)
def test_k3_big_tile_integer_bf16_bit_exact(gpu, orc, M, N, K):
    announce(f"exact K3 big tile M={M} N={N} K={K}")
    w, x, c, bias = int_problem(M, N, K, seed=M + N + K)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    acc = orc.trit_matmul_i64(x.to(torch.int8).numpy(), packed.cpu().numpy(), K)
    xg = x.to(torch.bfloat16).to(gpu)
    cg = c.to(gpu)
    for alpha, beta, use_bias in ((1.0, 0.0, False), (0.5, 1.0, True)):
        out = ops.ternary_matmul(xg, packed, K, alpha=alpha, beta=beta,
                                 c=cg.clone() if beta else None,
                                 bias=bias.to(gpu) if use_bias else None, kernel=3)
        want = expected(acc, alpha, beta, c.numpy(), bias.numpy() if use_bias else None)
        assert_bits(out.cpu().numpy(), want, f"alpha={alpha} beta={beta}")


K3_HALF = [
    # M, N, K: whole rounds of 256 x 256 tiles for the first 8192 rows, the rest as one
    # round of half-width 256 x 128 tiles (on 256 CUs: 195 of them) in the same launch,
    # where the tall tiles' remainder (180 of 512 x 64) would not fill a round; one and
    # four steps; ragged M and N
    (1900, 256 * 44 + 13, 96), (1900, 256 * 44 + 13, 384),
]
K3_TALL = [
    # M, N, K: tall 512 x 128 tiles (four waves along the rows).  Whole rounds only (on 256
    # CUs): one round with ragged M and N, two rounds with three steps (K past the last
    # whole step), one token in the last token tile; then whole rounds for the first 16384
    # rows and the rest as one round of 512 x 64 half-width tiles (208 / 192 / 192 of them):
    # one, three and four steps, ragged N
    (1000, 512 * 32 - 5, 96), (1000, 512 * 64, 200), (129, 512 * 128, 96),
    (1000, 256 * 88 + 7, 96), (1000, 256 * 88, 200), (1000, 256 * 88 - 5, 384),
]


@pytest.mark.parametrize("M,N,K,tall", [c + (False,) for c in K3_HALF] +
                         [c + (True,) for c in K3_TALL])
def test_k3_half_width_integer_bf16_bit_exact(gpu, orc, M, N, K, tall):
    """Every output against the float64 product of the unpacked trits on the GPU, a sample
    from both regions against the C oracle, alpha / beta / bias, and no workspace asked
    for (the half-width and tall tiles need none)."""
    announce(f"exact K3 {'tall' if tall else 'half-width'} M={M} N={N} K={K}")
    lib = _lib.lib()
    assert lib.t81_hip_ternary_matmul_workspace_size(M, N, K, _lib.DTYPE_BF16) == 0
    w, x, c, bias = int_problem(M, N, K, seed=M + N + K)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    exact = _gpu_exact_product(x.to(torch.float64).to(gpu), packed, N, K)
    if tall:
        n1 = tall_rows(M, N, K)
        assert n1 is not None, "shape expected to take the tall tiles"
    else:
        assert tall_rows(M, N, K) is None, "shape expected to keep the 256 x 256 tiles"
        n1 = whole_round_rows(M, N)
        assert 0 < n1 < N, "shape expected to leave rows past whole rounds"
    toks, rows = _sample(M, N, n1, seed=K)
    acc_s = orc.trit_matmul_i64(x[torch.from_numpy(toks)].to(torch.int8).numpy(),
                                packed.cpu().numpy()[rows], K)
    tsel = torch.from_numpy(toks).to(gpu)
    rsel = torch.from_numpy(rows).to(gpu)
    np.testing.assert_array_equal(exact[tsel][:, rsel].cpu().numpy().astype(np.int64), acc_s)
    xg, cg, bg = x.to(torch.bfloat16).to(gpu), c.to(gpu), bias.to(gpu)
    for alpha, beta, use_bias in ((1.0, 0.0, False), (0.5, 1.0, True)):
        out = ops.ternary_matmul(xg, packed, K, alpha=alpha, beta=beta,
                                 c=cg.clone() if beta else None,
                                 bias=bg if use_bias else None, kernel=3)
        want = alpha * exact
        if beta:
            want = want + beta * cg.double()
        if use_bias:
            want = want + bg.double()
        bad = int((out.double() != want).sum())
        assert bad == 0, f"alpha={alpha} beta={beta}: {bad} of {M * N} outputs differ"
        del out, want
    del exact
    torch.cuda.empty_cache()


# ------------------------------------------------------------ K3, int8 activations --
I8_FULL = [
    # name, M, K, N: whole tiles + a round of half-width tiles (gate_up), all split (M =
    # 512), odd step
    # counts (K = 4096: 43 steps), long K (down), M = 8192
    ("llama.gate_up", 2048, 4096, 28672),
    ("llama.down", 2048, 14336, 4096),
    ("llama.qkv", 512, 4096, 6144),
    ("llama.qkv", 8192, 4096, 6144),
]
I8_SMALL = [
    # M > 64 and K % 16 == 0 take the integer big-tile kernel: ragged M / N, K past the last
    # whole step, even and odd step counts, more tiles than CUs, few tiles (split-K)
    (300, 256 * 160 + 13, 208), (260, 256 * 81 + 7, 480), (512, 256 * 200 - 5, 96),
    (65, 1000, 4096), (300, 1000, 4112), (100, 2000, 4800), (257, 700, 16),
    # whole rounds of 256 x 256 tiles for the first 8192 rows, the rest as one round of
    # 256 x 128 half-width tiles (195 of them on 256 CUs, where the tall tiles' remainder
    # would not fill a round): one and three steps, ragged M and N
    (1900, 256 * 44 + 13, 96), (1900, 256 * 44 + 13, 208),
    # tall 512 x 128 tiles (on 256 CUs): one round with ragged M and N, two rounds, one
    # token in the last token tile; whole rounds for the first 16384 rows and the rest as
    # one round of 512 x 64 half-width tiles (208 / 192 of them): one and three steps
    (1000, 512 * 32 - 5, 96), (1000, 512 * 64, 208), (129, 512 * 128, 96),
    (1000, 256 * 88 + 7, 96), (1000, 256 * 88 - 5, 208),
]


def _int8_problem(M, N, K, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    w = torch.randn((N, K), generator=g)
    x = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    c = torch.randint(-(1 << 20), 1 << 20, (M, N), generator=g, dtype=torch.int32)
    return w, x, c


@pytest.mark.parametrize("M,N,K", I8_SMALL)
def test_k3_int8_big_tile_bit_exact(gpu, orc, M, N, K):
    """int32 results of the integer-MFMA kernel equal the int64 oracle, with beta = 0 and
    beta = 1 (C accumulated exactly)."""
    announce(f"exact K3 int8 M={M} N={N} K={K}")
    w, x, c = _int8_problem(M, N, K, seed=M * 3 + N + K)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    want = orc.trit_matmul_i64(x.numpy(), packed.cpu().numpy(), K)
    xg = x.to(gpu)
    out = ops.ternary_matmul(xg, packed, K, kernel=3)
    assert out.dtype == torch.int32
    np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), want)
    out = ops.ternary_matmul(xg, packed, K, beta=1.0, c=c.to(gpu), kernel=3)
    np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), want + c.numpy())


I8_COLUMN_BLOCK_CASES = [
    # M, N, K: int8 activations at 17..64 tokens (K % 16 == 0) through the K3 entry: the
    # column-block stream kernel with int8 widened to bf16 in LDS (two blocks, three, two
    # launches at 49..64), one and two row groups per workgroup, ragged N, |x| up to 128
    (17, 4096, 14336), (32, 14336, 4096), (40, 3072, 3072), (48, 3072, 8192), (64, 6144, 4096),
    (57, 1000, 4112),
]


@pytest.mark.parametrize("M,N,K", I8_COLUMN_BLOCK_CASES)
def test_column_block_int8_bit_exact(gpu, orc, M, N, K):
    """int32 results equal the int64 oracle with beta = 0 and 1; no workspace asked for."""
    announce(f"exact column-block int8 M={M} N={N} K={K}")
    lib = _lib.lib()
    assert lib.t81_hip_ternary_matmul_workspace_size(M, N, K, _lib.DTYPE_I8) == 0
    w, x, c = _int8_problem(M, N, K, seed=M * 5 + N + K)
    x[0, :16] = -128                      # the int8 extreme widens exactly too
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    want = orc.trit_matmul_i64(x.numpy(), packed.cpu().numpy(), K)
    xg = x.to(gpu)
    out = ops.ternary_matmul(xg, packed, K, kernel=3)
    assert out.dtype == torch.int32
    np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), want)
    out = ops.ternary_matmul(xg, packed, K, beta=1.0, c=c.to(gpu), kernel=3)
    np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), want + c.numpy())


@pytest.mark.parametrize("name,M,K,N", I8_FULL)
def test_k3_int8_config4_bit_exact(gpu, orc, name, M, K, N):
    """Config-4 shapes with int8 activations: every output against a float64 product of the
    unpacked trits on the GPU (exact), and a sample from every region against the oracle."""
    announce(f"exact K3 int8 {name} M={M} K={K} N={N}")
    g = torch.Generator("cpu").manual_seed(M + N + K + 1)
    w = torch.randn((N, K), generator=g)
    x = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    del w
    xg = x.to(gpu)
    exact = _gpu_exact_product(xg.to(torch.float64), packed, N, K)
    gg = torch.Generator(gpu).manual_seed(M * 5 + N)
    cg = torch.randint(-(1 << 20), 1 << 20, (M, N), generator=gg, device=gpu, dtype=torch.int32)
    toks, rows = _sample(M, N, whole_round_rows(M, N), seed=M + K + 1)
    acc_s = orc.trit_matmul_i64(x[torch.from_numpy(toks)].numpy(), packed.cpu().numpy()[rows], K)
    tsel = torch.from_numpy(toks).to(gpu)
    rsel = torch.from_numpy(rows).to(gpu)
    for beta in (0.0, 1.0):
        out = ops.ternary_matmul(xg, packed, K, beta=beta, c=cg.clone() if beta else None,
                                 kernel=3)
        want = exact + (cg.double() if beta else 0)
        bad = int((out.double() != want).sum())
        assert bad == 0, f"beta={beta}: {bad} of {M * N} outputs differ"
        got_s = out[tsel][:, rsel].cpu().numpy().astype(np.int64)
        want_s = acc_s + (cg[tsel][:, rsel].cpu().numpy().astype(np.int64) if beta else 0)
        np.testing.assert_array_equal(got_s, want_s)
        del out, want
    del exact
    torch.cuda.empty_cache()


I8_STREAM_CASES = [
    # M, N, K: int8 activations at 5..16 tokens through K2 (K % 16 == 0, 16-byte aligned x:
    # the staged stream kernel; the strip kernel at 5..8 over >= 12288 rows and K <= 4096),
    # at the 5-token switch-over and at 6..15 tokens with masked token columns, for one,
    # two and four row groups per workgroup; K = 14400 ends inside a sub-block
    (8, 14336, 4096), (8, 4096, 14336), (12, 4100, 3072), (9, 257, 14400), (15, 9216, 3072),
    (11, 3072, 8192), (5, 4096, 14336), (6, 9216, 3072), (7, 3072, 8192), (5, 16384, 3072),
    (7, 12300, 4000),
]


@pytest.mark.parametrize("M,N,K,offset", [c + (0,) for c in I8_STREAM_CASES]
                         + [(8, 14336, 4096, 1), (8, 4096, 14336, 1)])
def test_k2_int8_stream_bit_exact(gpu, orc, M, N, K, offset):
    """int32 results equal the int64 oracle with beta = 0 and 1, with |x| up to 128; offset 1
    puts x one byte past a 16-byte boundary at the 8-token switch-over (no staging: element
    loads)."""
    announce(f"exact K2 int8 M={M} N={N} K={K} offset={offset}")
    w, x, c = _int8_problem(M, N, K, seed=M * 11 + N + K)
    x[0, :16] = -128
    packed = ops.quantize_pack(w.to(gpu), 0.45, _lib.THR_CPP)
    want = orc.trit_matmul_i64(x.numpy(), packed.cpu().numpy(), K)
    store = torch.zeros(M * K + 16, dtype=torch.int8, device=gpu)
    xg = store[offset:offset + M * K].view(M, K)
    xg.copy_(x.to(gpu))
    assert xg.data_ptr() % 16 == offset
    out = ops.ternary_matmul(xg, packed, K, kernel=2)
    assert out.dtype == torch.int32
    np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), want)
    out = ops.ternary_matmul(xg, packed, K, beta=1.0, c=c.to(gpu), kernel=2)
    np.testing.assert_array_equal(out.cpu().numpy().astype(np.int64), want + c.numpy())
