"""The reference's own TQ1_0 row codec on the GPU (src/t81/core/gguf_quants.h:14-168) and
the tensor payloads of its dequant_tq1_0 / dequant_tq2_0 bindings
(python/bindings.cpp:519-638, 961-995), against tests/golden/tq1_row_vectors.npz (written
by the compiled header, tests/golden/make_golden.py) and the oracle's restatement.

Words must match bit for bit; float outputs match bit for bit except that a NaN is
compared as a NaN (its payload is not part of the contract)."""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

import oracle
from t81lib_amd import gguf, t81lib

pytestmark = pytest.mark.gpu

VECTORS = os.path.join(os.path.dirname(__file__), "golden", "tq1_row_vectors.npz")


def announce(case: str) -> None:
    sys.__stderr__.write(f"[gpu case] {case}\n")
    sys.__stderr__.flush()


@pytest.fixture(scope="module")
def g():
    return np.load(VECTORS)


def _cases(d, prefix, key, okey):
    offs = d[f"{prefix}_{okey}"]
    arr = d[f"{prefix}_{key}"]
    return [arr[offs[i]:offs[i + 1]] for i in range(offs.size - 1)]


def same_bits(a, b, what=""):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    assert a.shape == b.shape, what
    bad = ~((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b)))
    if bad.any():
        i = np.argwhere(bad)[0]
        raise AssertionError(f"{what}: {int(bad.sum())} differ; first at {tuple(i)}: "
                             f"{a[tuple(i)]!r} vs {b[tuple(i)]!r}")


def test_constants():
    assert t81lib.TQ1_TRITS_PER_BLOCK == 8 and t81lib.TQ1_BLOCK_ROWS == 32


def test_quantize_row_golden(gpu, g):
    announce("tq1 row quantize golden")
    vals = _cases(g, "q", "values", "offsets")
    words = _cases(g, "q", "words", "word_offsets")
    for i, (v, w) in enumerate(zip(vals, words)):
        thr, sc = float(g["q_threshold"][i]), float(g["q_scale"][i])
        ret, got = t81lib.quantize_row_tq1_0(v, thr, sc)
        assert isinstance(got, np.ndarray) and got.dtype == np.uint16
        np.testing.assert_array_equal(got, w, err_msg=f"case {i} thr={thr} scale={sc}")
        same_bits(np.float32(ret), g["q_returned_scale"][i], f"scale of case {i}")
        # the same row as a GPU tensor: words stay on the GPU
        ret_d, got_d = t81lib.quantize_row_tq1_0(torch.from_numpy(v).to(gpu), thr, sc)
        assert got_d.is_cuda
        np.testing.assert_array_equal(got_d.cpu().numpy(), w)


def test_dequant_row_golden(gpu, g):
    announce("tq1 row dequantize golden")
    words = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    trits = t81lib.dequant_row_tq1_0(words, 8 * 65536, 1.0)
    np.testing.assert_array_equal(trits.astype(np.int8), g["d_trits"])
    for s_, want in zip(g["d_scales"], g["d_values"]):
        got = t81lib.dequant_row_tq1_0(g["d_words"], 8 * g["d_words"].size, float(s_))
        same_bits(got, want, f"scale {s_}")
    ragged = [t81lib.dequant_row_tq1_0(words[:64], n, 1.25) for n in (0, 1, 5, 8, 13, 100)]
    np.testing.assert_array_equal(np.concatenate(ragged), g["d_ragged"])
    # forcecast: an int64 array wraps to uint16 as numpy's unsafe cast does
    wide = words[:16].astype(np.int64) + 65536
    np.testing.assert_array_equal(t81lib.dequant_row_tq1_0(wide, 128, 1.0),
                                  t81lib.dequant_row_tq1_0(words[:16], 128, 1.0))


def test_row_errors(gpu):
    with pytest.raises(ValueError, match="requires a 1-D float array"):
        t81lib.quantize_row_tq1_0(np.zeros((2, 3), np.float32))
    with pytest.raises(ValueError, match="cols must be non-negative"):
        t81lib.dequant_row_tq1_0(np.zeros(2, np.uint16), -1, 1.0)
    with pytest.raises(ValueError, match="packed buffer too small"):
        t81lib.dequant_row_tq1_0(np.zeros(2, np.uint16), 17, 1.0)
    ret, w = t81lib.quantize_row_tq1_0(np.zeros(0, np.float32))
    assert ret == 0.0 and w.size == 0
    assert t81lib.quantize_row_tq1_0(np.zeros(0, np.float32), scale=2.0)[0] == 2.0


def _payloads(d):
    pays = _cases(d, "p", "bytes", "offsets")
    vals = _cases(d, "p", "values", "value_offsets")
    return [(tuple(int(v) for v in m), p, v) for m, p, v in zip(d["p_meta"], pays, vals)]


def test_dequant_tensor_golden(gpu, g):
    announce("tq1 payload dequantize golden")
    for (rows, cols, block_rows, refine), pay, want in _payloads(g):
        fn = t81lib.dequant_tq2_0 if refine else t81lib.dequant_tq1_0
        got = fn(pay.tobytes(), rows, cols, block_rows)
        assert got.shape == (rows, cols) and got.dtype == np.float32
        same_bits(got.reshape(-1), want, f"{(rows, cols, block_rows, refine)}")
        # device bytes, and an odd start address
        dev = torch.zeros(pay.size + 1, dtype=torch.uint8, device=gpu)
        dev[1:].copy_(torch.from_numpy(pay.copy()))
        got_d = fn(dev[1:], rows, cols, block_rows)
        assert got_d.is_cuda
        same_bits(got_d.cpu().numpy().reshape(-1), want, "device payload")


def test_dequant_tensor_truncation_messages(gpu, g):
    announce("tq1 payload truncation")
    msgs = {1: "buffer truncated while reading scale",
            2: "buffer truncated while skipping refinement bytes",
            3: "buffer truncated while reading quantized rows"}
    cases = _payloads(g)
    for ci, cut, rc in g["p_cuts"]:
        (rows, cols, block_rows, refine), pay, _ = cases[ci]
        fn = t81lib.dequant_tq2_0 if refine else t81lib.dequant_tq1_0
        with pytest.raises(ValueError, match=msgs[int(rc)]):
            fn(pay[:cut].tobytes(), rows, cols, block_rows)
    with pytest.raises(ValueError, match="rows and cols must be non-negative"):
        t81lib.dequant_tq1_0(b"\0\0", -1, 4)
    with pytest.raises(ValueError, match="buffer must be observed as bytes"):
        t81lib.dequant_tq1_0(np.zeros(8, np.uint16), 1, 8)


@pytest.mark.parametrize("rows,cols", [(1, 1), (37, 100), (300, 4096), (64, 14336), (1000, 9),
                                       (5, 2052), (3, 1028), (8, 8192), (4, 8196)])
def test_quantize_rows_vs_oracle(gpu, rows, cols):
    announce(f"tq1 rows {rows}x{cols}")
    rng = np.random.default_rng(rows + cols)
    m = rng.standard_normal((rows, cols)).astype(np.float32)
    m[0, :min(cols, 3)] = [np.nan, np.inf, -0.0][:min(cols, 3)]
    if rows > 2:
        m[2] = 0.0
    supplied = np.where(rng.random(rows) < 0.5, rng.random(rows) * 3, 0.0).astype(np.float32)
    for scales in (None, supplied):
        s_used, words = gguf.quantize_rows_tq1_0(torch.from_numpy(m).to(gpu), 0.45,
                                                 None if scales is None else
                                                 torch.from_numpy(scales).to(gpu))
        s_used, words = s_used.cpu().numpy(), words.cpu().numpy()
        for r in range(rows):
            sc = 0.0 if scales is None else float(scales[r])
            used, want = oracle.tq1r_quantize_row(m[r], 0.45, sc)
            np.testing.assert_array_equal(words[r], want, err_msg=f"row {r}")
            same_bits(s_used[r], used, f"scale row {r}")
        back = gguf.dequant_rows_tq1_0(torch.from_numpy(words).to(gpu), cols,
                                       torch.from_numpy(s_used).to(gpu)).cpu().numpy()
        for r in range(0, rows, max(1, rows // 17)):
            same_bits(back[r], oracle.tq1r_dequantize_row(words[r], cols, float(s_used[r])),
                      f"dequant row {r}")


@pytest.mark.parametrize("rows,cols,block_rows,refine", [
    (70, 100, 32, False), (70, 100, 32, True), (33, 8, 7, False), (9, 1, 1, True),
    (6, 40, -5, True), (3, 24, 1000, False), (0, 10, 32, False), (4, 0, 2, True),
    (4096, 4096, 32, True)])
def test_payload_writer_vs_oracle(gpu, rows, cols, block_rows, refine):
    announce(f"tq1 payload writer {rows}x{cols} block_rows={block_rows} refine={refine}")
    rng = np.random.default_rng(rows * 3 + cols)
    m = rng.standard_normal((rows, cols)).astype(np.float32)
    if rows > 5 and cols:
        m[5] *= 1e-9
    pay = gguf.quantize_tq1_0_payload(torch.from_numpy(m).to(gpu), block_rows, refine)
    assert pay.numel() == gguf.tq1_payload_bytes(rows, cols, block_rows, refine)
    sub = m if rows <= 300 else m[:96]
    want = oracle.tq1r_payload(sub, block_rows, refine)
    np.testing.assert_array_equal(pay.cpu().numpy()[:len(want)], np.frombuffer(want, np.uint8))
    fn = t81lib.dequant_tq2_0 if refine else t81lib.dequant_tq1_0
    back = fn(pay, rows, cols, block_rows)
    if rows <= 300:
        rc, ref_back = oracle.tq1r_dequant_tensor(pay.cpu().numpy().tobytes(), rows, cols,
                                                  block_rows, refine)
        assert rc == 0
        same_bits(back.cpu().numpy(), ref_back, "decode")
    else:
        # decode = trit * float(h) of the group, trits of m / float(h) at 0.45
        group = max(1, block_rows)
        assert group == 32
        mg = torch.from_numpy(m).to(gpu).reshape(rows // group, group, cols)
        h_np = np.abs(m.reshape(rows // group, -1)).max(1).astype(np.float16).astype(np.float32)
        inv = torch.from_numpy(np.float32(1.0) / h_np).to(gpu)[:, None, None]
        h = torch.from_numpy(h_np).to(gpu)[:, None, None]
        t = torch.clamp(mg * inv, -1.0, 1.0)
        trit = (t >= 0.45).float() - (t <= -0.45).float()
        want_d = (trit * h).reshape(rows, cols)
        assert torch.equal(back, want_d)
