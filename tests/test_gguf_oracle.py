"""Pins the CPU oracle for the GGUF ternary block codecs (TQ1_0, TQ2_0).

The formats are llama.cpp's ggml block_tq1_0 / block_tq2_0, written and read by
the reference with numpy (t81/gguf.py:518-663, 1020-1069).  The reference module
imports t81lib, whose pybind11 build is unavailable here, so it cannot be run for
vectors; the oracle is pinned by:
  * numpy's own float16 conversion (all 65536 halfs, 800k floats);
  * known-answer blocks worked out by hand from the ggml layouts (element order);
  * a round trip over every base-3 digit pattern (the fixed-point byte encoding
    (v * 256 + 242) // 243 and its digit extraction are independent formulas);
  * closed forms of the two trit rules (threshold, round half away from zero);
  * the reference's own round-trip cases (tests/python/test_gguf.py:68-99).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle

TQ1, TQ2 = oracle.TQ1_0, oracle.TQ2_0


def test_block_bytes():
    assert oracle.tq_block_bytes(TQ1) == 54   # t81/gguf.py:1047 (48 + 4 + fp16)
    assert oracle.tq_block_bytes(TQ2) == 66   # t81/gguf.py:1051 (64 + fp16)
    assert oracle.tq_block_bytes(0) == -1


def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(0)
    vals = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s
                           for s in (1e-8, 1e-6, 1e-5, 1e-3, 1.0, 100.0, 1e4, 6e4)])
    vals = np.concatenate([vals, np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, np.inf,
                                           -np.inf, np.nan, 2.0**-24, 2.0**-25, 2.0**-14],
                                          np.float32)])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16_bits(v) for v in vals], np.uint16)
    np.testing.assert_array_equal(got, want)
    halfs = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    back = np.array([oracle.f16_bits_to_f32(h) for h in halfs], np.float32)
    ref = halfs.view(np.float16).astype(np.float32)
    same = (back.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(back) & np.isnan(ref))
    assert same.all()


def _trit_block(trits: np.ndarray) -> np.ndarray:
    """A 256-value row whose quantization at threshold 0.5 (d = 1) is exactly `trits`."""
    v = trits.astype(np.float32).copy()
    assert np.abs(v).max() == 1.0
    return v[None, :]


def test_tq2_known_answer_element_order():
    # ggml dequantize_row_tq2_0: byte j + m (j in {0, 32}), shift 2l -> element
    # (j / 32) * 128 + l * 32 + m.  Element 37 = (a 0, l 1, m 5); element 200 =
    # (a 1, l 2, m 8).  Digit q = trit + 1, so an all-zero block is 0x55 everywhere.
    t = np.zeros(256, np.int8)
    t[37], t[200], t[0] = 1, -1, 1
    blk = oracle.tq_quantize(_trit_block(t), 0.5, TQ2)[0]
    want = np.full(64, 0x55, np.uint8)
    want[5] = 0b01_01_10_01                       # element 37 -> +1 at bits 2..3
    want[32 + 8] = 0b01_00_01_01                  # element 200 -> -1 at bits 4..5
    want[0] = 0b01_01_01_10                       # element 0 -> +1 at bits 0..1
    np.testing.assert_array_equal(blk[:64], want)
    assert blk[64] == 0x00 and blk[65] == 0x3C    # float16(1.0) = 0x3C00
    back = oracle.tq_dequantize(blk[None, :], 1, 256, TQ2)[0]
    np.testing.assert_array_equal(back, t.astype(np.float32))


def test_tq1_known_answer_element_order():
    # ggml block_tq1_0: qs[0:32] hold elements n*32 + m (n < 5, digit n weighted
    # 3^(4-n)), qs[32:48] elements 160 + n*16 + m, qh[0:4] elements 240 + n*4 + m
    # (four digits weighted 81, 27, 9, 3); a number v < 243 is stored as
    # (v * 256 + 242) // 243.  All digits 1 (zero trits): 121 -> 128, 120 -> 127.
    t = np.zeros(256, np.int8)
    t[161] = 1    # qs1 group, n = 0, m = 1 -> byte 33, digits 2,1,1,1,1 = 202 -> 213
    t[96 + 3] = -1  # qs0 group, n = 3, m = 3 -> byte 3, digits 1,1,1,0,1 = 118 -> 125
    t[240 + 2 * 4 + 1] = 1  # qh group, n = 2, m = 1 -> byte 49, 1,1,2,1 -> 129 -> 136
    t[255] = -1   # qh group, n = 3, m = 3 -> byte 51, 1,1,1,0 -> 117 -> 124
    blk = oracle.tq_quantize(_trit_block(t), 0.5, TQ1)[0]
    want = np.array([128] * 32 + [128] * 16 + [127] * 4, np.uint8)
    want[33], want[3], want[49], want[51] = 213, 125, 136, 124
    np.testing.assert_array_equal(blk[:52], want)
    back = oracle.tq_dequantize(blk[None, :], 1, 256, TQ1)[0]
    np.testing.assert_array_equal(back, t.astype(np.float32))


@pytest.mark.parametrize("quant", [TQ1, TQ2])
def test_round_trip_every_digit_pattern(quant):
    """All 3^5 five-digit patterns in every position group, d = 1: exact round trip."""
    pats = np.array(np.meshgrid(*[[-1, 0, 1]] * 5, indexing="ij")).reshape(5, -1).T  # 243 x 5
    trits = np.concatenate([pats.reshape(-1), np.array([1, -1] * 2, np.int64)])
    nblk = -(-trits.size // 256)
    trits = np.pad(trits, (0, nblk * 256 - trits.size)).reshape(nblk, 256)
    trits[:, 0] = 1  # every block has max |value| 1
    rows = trits.astype(np.float32)
    packed = oracle.tq_quantize(rows, 0.5, quant)
    back = oracle.tq_dequantize(packed, nblk, 256, quant)
    np.testing.assert_array_equal(back, rows)


def test_threshold_and_rounding_rules():
    # threshold form: |v / d| >= thr -> sign; d = max |v| = 2; d stored as fp16.
    row = np.zeros((1, 300), np.float32)
    row[0, :6] = [2.0, -0.9, 0.9, -1.0, 0.89, 0.0]
    back = oracle.tq_dequantize(oracle.tq_quantize(row, 0.45, TQ2), 1, 300, TQ2)[0]
    np.testing.assert_array_equal(back[:6], [2.0, -2.0, 2.0, -2.0, 0.0, 0.0])
    assert (back[256:] == 0).all()  # second block all zero: d = 0
    # rounding form (threshold 0): floor(v + 0.5) / ceil(v - 0.5) in float32, then
    # clip.  0.49999997 + 0.5 = 1 - 2^-25 rounds to 1.0 in float32, so it becomes 1,
    # as numpy computes it.
    row = np.zeros((1, 256), np.float32)
    row[0, :8] = [1.0, 0.5, -0.5, 0.49, -0.49, 0.49999997, -0.49999997, -1.0]
    back = oracle.tq_dequantize(oracle.tq_quantize(row, 0.0, TQ1), 1, 256, TQ1)[0]
    np.testing.assert_array_equal(back[:8], [1.0, 1.0, -1.0, 0.0, 0.0, 1.0, -1.0, -1.0])
    v = row[0, :8]
    np.testing.assert_array_equal(np.where(v >= 0, np.floor(v + 0.5), np.ceil(v - 0.5)),
                                  back[:8])
    # thresholds are clipped to [0, 1]: 7 behaves as 1, -3 as the rounding form
    same = oracle.tq_quantize(row, 1.0, TQ2)
    np.testing.assert_array_equal(oracle.tq_quantize(row, 7.0, TQ2), same)
    np.testing.assert_array_equal(oracle.tq_quantize(row, -3.0, TQ2),
                                  oracle.tq_quantize(row, 0.0, TQ2))


def test_scale_overflow_follows_float16():
    row = np.zeros((1, 256), np.float32)
    row[0, :3] = [1e6, -1e6, 0.0]
    back = oracle.tq_dequantize(oracle.tq_quantize(row, 0.5, TQ2), 1, 256, TQ2)[0]
    assert back[0] == np.inf and back[1] == -np.inf and np.isnan(back[2])  # inf * 0


@pytest.mark.parametrize("quant,thr,lo,hi,shape", [
    (TQ1, 0.45, -1.0, 0.8, (3, 4)),     # tests/python/test_gguf.py:68-75 (_DummyModel)
    (TQ2, 0.25, -0.9, 0.9, (3, 4)),
    (TQ2, 0.45, -0.9, 0.9, (3, 4)),     # test_roundtrip_gguf_tq2
    (TQ1, 0.45, -5.0, 5.0, (64, 128)),  # test_roundtrip_large_linear (_LargeDummyModel)
])
def test_reference_roundtrip_cases(quant, thr, lo, hi, shape):
    """The reference's GGUF round-trip fills: torch.linspace(lo, hi) over the weight.
    Closed form per row: d = max|row| (one block), trits |v / d| >= thr -> sign."""
    w = np.linspace(lo, hi, int(np.prod(shape)), dtype=np.float32).reshape(shape)
    back = oracle.tq_dequantize(oracle.tq_quantize(w, thr, quant), shape[0], shape[1], quant)
    assert back.shape == shape and np.isfinite(back).all()
    d = np.abs(w).max(axis=1, keepdims=True)
    t = np.where(np.abs(w * (np.float32(1) / d)) >= np.float32(thr), np.sign(w), 0)
    want = d.astype(np.float16).astype(np.float32) * t.astype(np.float32)
    np.testing.assert_array_equal(back, want)


def test_tq2_matmul_closed_form():
    rng = np.random.default_rng(3)
    w = rng.standard_normal((7, 600)).astype(np.float32)
    packed = oracle.tq_quantize(w, 0.3, TQ2)
    dense = oracle.tq_dequantize(packed, 7, 600, TQ2).astype(np.float64)
    x = rng.standard_normal((3, 600))
    y, scale = oracle.tq2_matmul_f64(x, packed, 600)
    np.testing.assert_allclose(y, x @ dense.T, rtol=1e-12, atol=1e-9)
    np.testing.assert_allclose(scale, np.abs(x) @ np.abs(dense).T, rtol=1e-12)
