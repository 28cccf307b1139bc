"""t81_hip_ternary_matmul_noalloc: the trit-dot matmul with its split-K workspace in the
library's static device scratch, called through the C ABI and compared with
t81_hip_ternary_matmul_ws given a workspace of exactly the size it asks for -- same
kernels and split plan, so the outputs must agree bit for bit -- on two calls in a row,
the second on a smaller input, for each activation type that splits."""

from __future__ import annotations

import sys

import pytest
import torch

from t81lib_amd import _lib, ops

pytestmark = pytest.mark.gpu

SCRATCH = 64 << 20


def announce(case: str) -> None:
    sys.__stderr__.write(f"[gpu case] {case}\n")
    sys.__stderr__.flush()


def _problem(gpu, M, N, K, dtype, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    packed = ops.quantize_pack(torch.randn((N, K), generator=g).to(gpu), 0.45, _lib.THR_CPP)
    if dtype == torch.int8:
        x = torch.randint(-128, 128, (M, K), generator=g, dtype=torch.int8)
        c = torch.randint(-1000, 1000, (M, N), generator=g, dtype=torch.int32)
        bias, alpha, beta = None, 1.0, 1.0
    else:
        x = torch.randn((M, K), generator=g).to(dtype)
        c = torch.randn((M, N), generator=g)
        bias, alpha, beta = torch.randn((N,), generator=g).to(gpu), 0.75, 0.5
    return x.to(gpu), packed, c.to(gpu), bias, alpha, beta


def _code(dtype):
    return {torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32,
            torch.int8: _lib.DTYPE_I8}[dtype]


def _run_pair(gpu, M, N, K, dtype, seed):
    """(noalloc output, _ws output, workspace bytes) for one problem."""
    lib = _lib.lib()
    x, packed, c, bias, alpha, beta = _problem(gpu, M, N, K, dtype, seed)
    code = _code(dtype)
    need = lib.t81_hip_ternary_matmul_workspace_size(M, N, K, code)
    s = torch.cuda.current_stream().cuda_stream
    bptr = bias.data_ptr() if bias is not None else None
    c_ws = c.clone()
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=gpu)
    _lib.check(lib.t81_hip_ternary_matmul_ws(0, x.data_ptr(), code, packed.data_ptr(),
                                             c_ws.data_ptr(), M, N, K, alpha, beta, bptr,
                                             ws.data_ptr() if need > 0 else None, need, s))
    c_na = c.clone()
    _lib.check(lib.t81_hip_ternary_matmul_noalloc(0, x.data_ptr(), code, packed.data_ptr(),
                                                  c_na.data_ptr(), M, N, K, alpha, beta, bptr, s))
    torch.cuda.synchronize()
    return c_na, c_ws, need


@pytest.mark.parametrize("dtype,shapes", [
    # bf16: whole big tiles + split-K items in one launch (the rows past whole rounds too
    # few for a round of half-width tiles; 32 MiB), then every tile split (qkv at
    # M = 512), then a smaller split shape
    (torch.bfloat16, [(300, 36864, 1536), (512, 6144, 4096), (300, 1000, 4104)]),
    # int8 and float32: eight-wave splits of few tiles (int32 partials exact for int8)
    (torch.int8, [(20, 3000, 9000), (20, 1200, 4008)]),
    (torch.float32, [(48, 1000, 4104), (40, 700, 2000)]),
    # float32 past 64 tokens as the bf16 planes in the scratch, two bf16 launches per chunk
    (torch.float32, [(2048, 6144, 4096), (700, 16384, 2048)]),
    # K2 with 9..16 tokens over a long K (float32 and int8 activations; aligned bf16 runs
    # in one launch, as does int8 with K % 16 == 0): K split over workgroups, partials summed
    # in split order
    (torch.float32, [(16, 4096, 14336), (9, 3000, 9000)]),
    (torch.int8, [(12, 3072, 8200), (10, 2000, 7000)]),
])
def test_noalloc_matches_workspace_entry_point(gpu, dtype, shapes):
    for i, (M, N, K) in enumerate(shapes):
        announce(f"noalloc {dtype} call {i + 1} M={M} N={N} K={K}")
        c_na, c_ws, need = _run_pair(gpu, M, N, K, dtype, seed=M + N + K)
        assert 0 < need <= SCRATCH, f"shape expected to split within the scratch ({need} B)"
        assert torch.equal(c_na.view(torch.int32), c_ws.view(torch.int32)), \
            f"call {i + 1}: {int((c_na != c_ws).sum())} outputs differ"


def test_noalloc_without_split_and_rejection(gpu):
    lib = _lib.lib()
    announce("noalloc K2 and unsplit K3")
    # K2 at 4 and 16 tokens; whole big tiles; whole big tiles + a round of half-width
    # tiles (Llama gate_up at M = 2048)
    for M, N, K in ((4, 300, 4096), (16, 4096, 14336), (2048, 8192, 1024), (2048, 28672, 4096)):
        c_na, c_ws, need = _run_pair(gpu, M, N, K, torch.bfloat16, seed=M)
        assert need == 0
        assert torch.equal(c_na, c_ws)
    # a shape whose split needs more than the scratch is refused before any launch
    announce("noalloc rejection")
    M, K = 512, 4096
    N = next(n for n in range(6144, 256 * 160, 256)
             if lib.t81_hip_ternary_matmul_workspace_size(M, n, K, _lib.DTYPE_BF16) > SCRATCH)
    x, packed, c, bias, alpha, beta = _problem(gpu, M, N, K, torch.bfloat16, seed=5)
    before = c.clone()
    rc = lib.t81_hip_ternary_matmul_noalloc(0, x.data_ptr(), _lib.DTYPE_BF16, packed.data_ptr(),
                                            c.data_ptr(), M, N, K, alpha, beta, bias.data_ptr(),
                                            torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.EINVAL_SHAPE
    assert "static scratch" in _lib.last_error()
    torch.cuda.synchronize()
    assert torch.equal(c, before)


def test_noalloc_bad_arguments_before_scratch_check(gpu):
    """Argument errors are reported as t81_hip_ternary_matmul_ws reports them, before the
    scratch-size check."""
    lib = _lib.lib()
    s = torch.cuda.current_stream().cuda_stream
    rc = lib.t81_hip_ternary_matmul_noalloc(0, None, 9, None, None, 1, 1, 48, 1.0, 0.0, None, s)
    assert rc == _lib.EINVAL_DTYPE and "activations must be" in _lib.last_error()
    x = torch.zeros((17, 48), dtype=torch.bfloat16, device=gpu)
    w = torch.full((8, 1, 16), 13, dtype=torch.uint8, device=gpu)
    c = torch.zeros((17, 8), device=gpu)
    rc = lib.t81_hip_ternary_matmul_noalloc(2, x.data_ptr(), _lib.DTYPE_BF16, w.data_ptr(),
                                            c.data_ptr(), 17, 8, 48, 1.0, 0.0, None, s)
    assert rc == _lib.EINVAL_SHAPE and "M <= 16" in _lib.last_error()
    rc = lib.t81_hip_ternary_matmul_noalloc(2, None, _lib.DTYPE_BF16, None, None, 17, 8, 48, 1.0,
                                            0.0, None, s)
    assert rc == _lib.EINVAL_POINTER   # the pointer checks come first, as in the _ws form


@pytest.mark.parametrize("dtype,M,N,K", [(torch.float32, 48, 1000, 4104),
                                         (torch.bfloat16, 512, 6144, 4096),
                                         (torch.float32, 16, 4096, 14336)])
def test_noalloc_under_graph_capture(gpu, dtype, M, N, K):
    """A split shape captured in a HIP graph through the no-allocation entry point: every
    replay equals the workspace entry point's eager result bit for bit, with eager calls
    on other shapes (which overwrite the shared scratch) and synchronisations between the
    replays."""
    announce(f"noalloc graph capture {dtype} M={M} N={N} K={K}")
    lib = _lib.lib()
    x, packed, c, bias, alpha, beta = _problem(gpu, M, N, K, dtype, seed=M * 3 + K)
    code = _code(dtype)
    need = lib.t81_hip_ternary_matmul_workspace_size(M, N, K, code)
    assert 0 < need <= SCRATCH
    c_na, c_ws, _ = _run_pair(gpu, M, N, K, dtype, seed=M * 3 + K)   # eager, same inputs
    assert torch.equal(c_na.view(torch.int32), c_ws.view(torch.int32))
    bptr = bias.data_ptr() if bias is not None else None
    c_g = c.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.t81_hip_ternary_matmul_noalloc(0, x.data_ptr(), code, packed.data_ptr(),
                                                c_g.data_ptr(), M, N, K, alpha, beta, bptr,
                                                torch.cuda.current_stream().cuda_stream)
    _lib.check(rc)
    for i in range(3):
        c_g.copy_(c)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(c_g.view(torch.int32), c_ws.view(torch.int32)), \
            f"replay {i + 1}: {int((c_g != c_ws).sum())} outputs differ"
        # an eager split call on another shape reuses (overwrites) the scratch in between
        other = _run_pair(gpu, 40, 700, 2000, torch.float32, seed=i)
        assert torch.equal(other[0].view(torch.int32), other[1].view(torch.int32))
    del graph
