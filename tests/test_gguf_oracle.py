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


# ---------------------------------------------- TQ1_0 row codec (gguf_quants.h) --
TQ1R = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                  "tq1_row_vectors.npz")


@pytest.fixture(scope="module")
def tq1g():
    return np.load(TQ1R)


def _cases(g, prefix, key, okey):
    offs = g[f"{prefix}_{okey}"]
    arr = g[f"{prefix}_{key}"]
    return [arr[offs[i]:offs[i + 1]] for i in range(offs.size - 1)]


def _same_bits(a, b) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))).all())


def test_tq1r_constants():
    assert oracle.TQ1_TRITS_PER_BLOCK == 8 and oracle.TQ1_BLOCK_ROWS == 32  # gguf_quants.h:14-15
    assert oracle.tq1r_words(0) == 0 and oracle.tq1r_words(8) == 1 and oracle.tq1r_words(9) == 2


def test_tq1r_quantize_golden(tq1g):
    vals = _cases(tq1g, "q", "values", "offsets")
    words = _cases(tq1g, "q", "words", "word_offsets")
    for i, (v, w) in enumerate(zip(vals, words)):
        thr, sc = float(tq1g["q_threshold"][i]), float(tq1g["q_scale"][i])
        used, got = oracle.tq1r_quantize_row(v, thr, sc)
        np.testing.assert_array_equal(got, w, err_msg=f"case {i} thr={thr} scale={sc}")
        # the binding returns the argument unless it is <= 0 (NaN is returned as given)
        s32 = np.float32(sc)
        ret = s32 if not s32 <= 0 else np.float32(oracle.tq1r_scale(v))
        assert _same_bits(ret, tq1g["q_returned_scale"][i])
        if s32 <= 0 or np.isnan(s32):
            assert _same_bits(used, oracle.tq1r_scale(v))


def test_tq1r_dequantize_golden(tq1g):
    words = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    trits = oracle.tq1r_dequantize_row(words, 8 * 65536, 1.0)
    np.testing.assert_array_equal(trits.astype(np.int8), tq1g["d_trits"])
    for s_, want in zip(tq1g["d_scales"], tq1g["d_values"]):
        got = oracle.tq1r_dequantize_row(tq1g["d_words"], 8 * tq1g["d_words"].size, float(s_))
        assert _same_bits(got, want), f"scale {s_}"
    ragged = [oracle.tq1r_dequantize_row(words[:64], n, 1.25) for n in (0, 1, 5, 8, 13, 100)]
    np.testing.assert_array_equal(np.concatenate(ragged), tq1g["d_ragged"])


def test_tq1r_half_to_float_golden_and_numpy(tq1g):
    halfs = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = np.array([oracle.f16_bits_to_f32(h) for h in halfs], np.float32)
    # (NaN compared as NaN: a float returned through ctypes passes a double, which quiets
    # a signalling NaN on the way)
    assert _same_bits(got, tq1g["h_values"])
    fin = ~np.isnan(got)
    np.testing.assert_array_equal(got[fin], halfs.view(np.float16).astype(np.float32)[fin])


def _payload_cases(g):
    pays = _cases(g, "p", "bytes", "offsets")
    vals = _cases(g, "p", "values", "value_offsets")
    return [(tuple(int(v) for v in m), p, v) for m, p, v in zip(g["p_meta"], pays, vals)]


def test_tq1r_payload_golden(tq1g):
    for (rows, cols, block_rows, refine), pay, want in _payload_cases(tq1g):
        rc, got = oracle.tq1r_dequant_tensor(pay.tobytes(), rows, cols, block_rows, bool(refine))
        assert rc == 0
        assert _same_bits(got.reshape(-1), want), (rows, cols, block_rows, refine)
    cases = _payload_cases(tq1g)
    for ci, cut, rc_want in tq1g["p_cuts"]:
        (rows, cols, block_rows, refine), pay, _ = cases[ci]
        rc, _ = oracle.tq1r_dequant_tensor(pay[:cut].tobytes(), rows, cols, block_rows,
                                           bool(refine))
        assert rc == rc_want, (ci, cut)


class _ShortRead(Exception):
    pass


def _stream_decode(buf: bytes, rows: int, cols: int, block_rows: int, refine: bool) -> int:
    """A brute-force reader that consumes the payload field by field, in the order the
    binding's loop reads it (python/bindings.cpp:596-635), and reports the kind of the
    first field it cannot read in full: 1 scale, 2 reserved bytes, 3 a row."""
    import io

    f = io.BytesIO(buf)

    def take(n, kind):
        if len(f.read(n)) != n:
            raise _ShortRead(kind)

    group = max(1, block_rows)
    done = 0
    try:
        while done < rows:
            take(2, 1)
            if refine:
                take(8, 2)
            for _ in range(min(group, rows - done)):
                take(2 * ((cols + 7) // 8), 3)
                done += 1
    except _ShortRead as e:
        return int(e.args[0])
    return 0


@pytest.mark.parametrize("rows,cols,block_rows,refine", [
    (5, 13, 32, 0), (70, 100, 32, 1), (33, 8, 7, 0), (9, 1, 1, 1), (4, 0, 2, 1), (6, 40, -5, 1),
    (3, 24, 1000, 0), (1, 17, 32, 1)])
def test_tq1r_truncation_every_cut(rows, cols, block_rows, refine):
    m = np.random.default_rng(rows * cols + 1).standard_normal((rows, cols)).astype(np.float32)
    pay = oracle.tq1r_payload(m, block_rows, bool(refine))
    for cut in range(len(pay) + 1):
        rc, _ = oracle.tq1r_dequant_tensor(pay[:cut], rows, cols, block_rows, bool(refine))
        assert rc == _stream_decode(pay[:cut], rows, cols, block_rows, bool(refine)), cut
    assert oracle.tq1r_dequant_tensor(b"", -1, 3)[0] == -1


def test_tq1r_word_code_closed_form():
    """Every digit pattern of 8 trits round-trips, the word equals sum_i d_i 3^i with
    d = {+1: 0, 0: 1, -1: 2}, and the 6561 valid words are a bijection."""
    digits = np.array(np.meshgrid(*[np.arange(3)] * 8, indexing="ij")).reshape(8, -1).T
    trits = np.where(digits == 0, 1, np.where(digits == 2, -1, 0)).astype(np.float32)
    words = np.empty(len(trits), np.uint16)
    for i, t in enumerate(trits):
        used, w = oracle.tq1r_quantize_row(t, 0.45, 1.0)
        words[i] = w[0]
    np.testing.assert_array_equal(words, (digits * 3 ** np.arange(8)).sum(1))
    assert np.unique(words).size == 6561 and words.max() == 6560
    back = oracle.tq1r_dequantize_row(words, 8 * words.size, 1.0).reshape(-1, 8)
    np.testing.assert_array_equal(back, trits)


@pytest.mark.skipif("not __import__('oracle').ref()", reason="oracle/_ref not built here")
def test_tq1r_matches_compiled_reference_live():
    ref = oracle.ref()
    g = np.random.default_rng(7)
    specials = np.array([np.nan, np.inf, -np.inf, -0.0, 1e-45, -1e-40, 3e38], np.float32)
    for i in range(300):
        n = int(g.integers(0, 90))
        v = (g.standard_normal(n) * 10.0 ** g.integers(-6, 3)).astype(np.float32)
        if n and i % 3 == 0:
            v[g.integers(0, n, 3)] = g.choice(specials, 3)
        thr = float(g.choice([0.45, 0.5, 0.0, 1.2, -0.1, np.nan, g.random()]))
        sc = float(g.choice([0.0, -1.0, np.nan, np.inf, 1e-40, g.random() * 3]))
        np.testing.assert_array_equal(oracle.tq1r_quantize_row(v, thr, sc)[1],
                                      ref.tq1_quantize_row(v, thr, sc), err_msg=f"case {i}")
        assert _same_bits(oracle.tq1r_scale(v), ref.tq1_compute_scale(v))
        w = g.integers(0, 65536, oracle.tq1r_words(n)).astype(np.uint16)
        s_ = float(g.choice([0.0, -0.0, 1.0, -2.5, np.inf, np.nan, 1e-42, g.standard_normal()]))
        assert _same_bits(oracle.tq1r_dequantize_row(w, n, s_), ref.tq1_dequantize_row(w, n, s_))
