"""Pins the oracle's scatter-mean (PATCH:151-215) and Q8_0 quantiser
(cpp_ggml/scripts/gguf_schema.py:14-24) with cases whose results IEEE
arithmetic fixes by hand."""
import numpy as np

import oracle

H = np.float16


def test_scatter_mean_exact_integers(orc):
    # small integers: every f16 partial sum is exact, so the result is the
    # exact sum divided in F32 and rounded once to f16
    feats = np.array([[1, 2], [3, 4], [5, 6], [7, 8], [9, 10]], H)
    rows = np.array([0, 1, 0, 1, 0], np.int32)
    counts = np.array([4.0, 3.0], np.float32)  # |children| + 1
    out = orc.scatter_mean(feats, rows, counts, 2)
    expect = np.array([[15 / 4, 18 / 4], [10 / 3, 12 / 3]], np.float32).astype(H)
    assert np.array_equal(out, expect)


def test_scatter_mean_f16_rounding_history(orc):
    # 2048 + 1 -> 2049 is a tie between 2048 and 2050: f16 keeps 2048, twice.
    # An F32 accumulator would give 2050; the ascending order 1 + 1 + 2048
    # would give 2050 as well.  Only "f16 partial sums in ascending fine-row
    # order" yields 2048 for row 0.
    feats = np.array([[2048], [1], [1], [1], [1], [2048]], H)
    rows = np.array([0, 0, 0, 1, 1, 1], np.int32)
    counts = np.array([1.0, 1.0], np.float32)
    out = orc.scatter_mean(feats, rows, counts, 2)
    assert out[0, 0] == H(2048) and out[1, 0] == H(2050)


def test_scatter_mean_skips_out_of_range_rows(orc):
    feats = np.array([[1], [2], [4], [8]], H)
    rows = np.array([-1, 0, 2, 0], np.int32)  # -1 and nc=2 are skipped
    out = orc.scatter_mean(feats, rows, np.array([2.0, 1.0], np.float32), 2)
    assert out[:, 0].tolist() == [5.0, 0.0]


def test_scatter_mean_division_is_f32(orc):
    # 1/3 in F32 then to f16, not 1 * f16(1/3)
    out = orc.scatter_mean(np.array([[1]], H), np.array([0], np.int32),
                           np.array([3.0], np.float32), 1)
    assert out[0, 0] == (np.float32(1) / np.float32(3)).astype(H)


def test_scatter_mean_threads_bit_identical(orc):
    rng = np.random.default_rng(0)
    feats = rng.uniform(-4, 4, (5000, 16)).astype(H)
    rows = rng.integers(-1, 700, 5000).astype(np.int32)
    counts = np.bincount(rows[rows >= 0], minlength=700).astype(np.float32) + 1
    a = orc.scatter_mean(feats, rows, counts, 700)
    b = orc.scatter_mean(feats, rows, counts, 700, nthreads=5)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def _blocks(out):
    b = out.reshape(-1, 34)
    return b[:, :2].copy().view(np.float16).reshape(-1), b[:, 2:].view(np.int8)


def test_q8_0_hand_block(orc):
    w = np.zeros(32, np.float32)
    w[:4] = [0.5, -1.0, 0.25, 0.0]
    d, q = _blocks(orc.q8_0_quantize(w))
    # amax = 1: d = fp16(1/127) = 2^-7 * (1 + 8/1024)
    assert d[0] == H(0.0078125 * (1 + 8 / 1024))
    # 0.5 / d = 63.503... -> 64; -1 / d = -127.007 -> -127; 0.25 / d = 31.75 -> 32
    assert q[0, :4].tolist() == [64, -127, 32, 0]


def test_q8_0_ties_to_even(orc):
    # d = 2^-7 exactly (amax = 127 * 2^-7); w / d = 2.5 and 3.5 and -2.5
    s = 2.0 ** -7
    w = np.zeros(32, np.float32)
    w[:4] = [127 * s, 2.5 * s, 3.5 * s, -2.5 * s]
    d, q = _blocks(orc.q8_0_quantize(w))
    assert d[0] == H(s)
    assert q[0, :4].tolist() == [127, 2, 4, -2]  # rint, not round-half-away


def test_q8_0_zero_block(orc):
    d, q = _blocks(orc.q8_0_quantize(np.zeros(64, np.float32)))
    assert np.all(d == 0) and np.all(q == 0)
    deq = orc.q8_0_dequant(orc.q8_0_quantize(np.zeros(64, np.float32)))
    assert np.all(deq == 0)


def test_q8_0_round_trip_bound(orc):
    w = np.random.default_rng(1).normal(0, 0.02, 32 * 4096).astype(np.float32)
    blocks = orc.q8_0_quantize(w)
    d, q = _blocks(blocks)
    deq = orc.q8_0_dequant(blocks)
    dd = np.repeat(d.astype(np.float32), 32)
    amax = np.repeat(np.abs(w.reshape(-1, 32)).max(1), 32)
    assert np.all(np.abs(w - deq) <= dd / 2 + amax * 2.0 ** -10)
    assert np.array_equal(deq, dd * q.reshape(-1).astype(np.float32))
    assert np.abs(q).max() <= 127


def test_q8_0_dequant_f16_rounding(orc):
    w = np.random.default_rng(2).normal(0, 0.02, 32 * 64).astype(np.float32)
    blocks = orc.q8_0_quantize(w)
    f32 = orc.q8_0_dequant(blocks, oracle.F32)
    f16 = orc.q8_0_dequant(blocks, oracle.F16)
    assert np.array_equal(f16, f32.astype(H))


def test_scatter_case_inputs_follow_recipe(orc):
    """The regenerated inputs have the recipe's structure: pinned rows,
    skipped rows -1 / nc, counts = hits, features are f16 in [-4, 4)."""
    f, rows, counts = orc.scatter_case(128, 26281, 5239, 5)
    assert np.array_equal(rows[:5239], np.arange(5239))
    valid = (rows >= 0) & (rows < 5239)
    assert set(np.unique(rows[~valid])) <= {-1, 5239} and (~valid).sum() > 0
    assert np.array_equal(np.bincount(rows[valid], minlength=5239).astype(np.float32), counts)
    v = f.view(np.float16).astype(np.float32)
    assert v.min() >= -4.0 and v.max() <= 4.0 and abs(float(v.mean())) < 0.05
