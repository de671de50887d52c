"""Properties the mathematics of the codec fixes, checked on the C oracle.

Each check is chosen so that a plausible slip (a transposed axis, a dropped
term, half-even instead of half-away rounding, a float instead of double sum)
fails it, independently of how the oracle is written."""

from fractions import Fraction

import numpy as np
import pytest

import datagen
import oracle


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build(reference=False)


def _heads():
    yield datagen.c1_heads(1, 31)[0]
    yield datagen.student_t_heads(1, 32)[0]
    yield datagen.zero_rows_cols_head(33)
    g = datagen.rng(34)
    yield (g.standard_normal((8, 6)) * 0.05).astype(np.float32)


def test_live_columns_reach_127_and_codes_avoid_minus_128():
    for x in _heads():
        codes, s, sc, _, _ = oracle.quantize_kv(x)
        assert codes.min() >= -127
        for v in range(x.shape[1]):
            if sc[v] > 0:
                assert np.abs(codes[:, v].astype(int)).max() == 127
            else:
                assert not codes[:, v].any()


def test_zero_row_and_zero_column():
    x = datagen.zero_rows_cols_head(35)
    codes, s, sc, _, _ = oracle.quantize_kv(x)
    floor_s = np.sqrt(np.float32(1e-8))
    assert s[3] == floor_s and s[40] == floor_s
    assert sc[5] == 0 and sc[100] == 0
    assert not codes[3].any() and not codes[:, 5].any()
    zero_codes, zero_s, zero_sc, _, _ = oracle.quantize_kv(np.zeros((4, 4), np.float32))
    assert (zero_s == floor_s).all() and (zero_sc == 0).all() and not zero_codes.any()


def test_smoothing_is_sqrt_of_exact_mean_when_the_sum_is_exact():
    x = datagen.c1_heads(1, 36)[0]
    _, s, _, _, _ = oracle.quantize_kv(x)
    for k in range(0, 128, 7):
        exact = sum(Fraction(float(abs(v))) for v in x[k])  # exact rational sum
        mean = np.float32(float(exact / 128))
        assert s[k] == np.sqrt(max(mean, np.float32(1e-8)))


def test_power_of_two_scaling_and_sign_flip():
    for x in _heads():
        codes, s, sc, _, _ = oracle.quantize_kv(x)
        c4, s4, sc4, _, _ = oracle.quantize_kv(x * np.float32(4.0))
        # mean scales by 4 exactly, so s by 2 exactly; m = r / s scales by 2.
        live = s > np.sqrt(np.float32(1e-8)) * 2
        assert (s4[live] == 2 * s[live]).all()
        if live.all():
            assert (c4 == codes).all() and (sc4 == 2 * sc).all()
        cn, sn, scn, _, _ = oracle.quantize_kv(-x)
        assert (cn == -codes).all() and (sn == s).all() and (scn == sc).all()


def test_key_permutation_permutes_rows_only():
    x = datagen.c1_heads(1, 37)[0]
    perm = datagen.rng(38).permutation(128)
    codes, s, sc, _, _ = oracle.quantize_kv(x)
    cp, sp, scp, _, _ = oracle.quantize_kv(x[perm])
    assert (cp == codes[perm]).all() and (sp == s[perm]).all() and (scp == sc).all()


def test_round_half_away_from_zero_on_the_tie_head(golden):
    x = golden["ties/input"]
    codes, s, sc, _, _ = oracle.quantize_kv(x)
    m = x / s[:, None]
    val = (m / np.where(sc == 0, 1, sc)[None, :]) * np.float32(127)
    ties = (val - np.floor(val)) == 0.5
    assert ties.sum() >= 16
    away = np.trunc(val + np.copysign(np.float32(0.5), val))
    assert (codes[ties] == away[ties]).all()
    assert (codes[ties] != np.rint(val[ties])).any()  # half-even would differ


def test_dequantize_error_is_within_half_a_code_step():
    for x in _heads():
        codes, s, sc, _, _ = oracle.quantize_kv(x)
        dense = oracle.dequantize_kv(codes, s, sc).astype(np.float64)
        step = (s.astype(np.float64)[:, None] * sc.astype(np.float64)[None, :]) / 127
        err = np.abs(dense - x.astype(np.float64))
        assert (err <= 0.5 * step * (1 + 2e-4) + 1e-30).all()


def test_readout_scaling_is_exact_and_within_the_fp32_bound():
    g = datagen.rng(39)
    x = datagen.c1_heads(1, 40)[0]
    codes, s, sc, _, _ = oracle.quantize_kv(x)
    read = g.standard_normal(128).astype(np.float32)
    out = oracle.read_boundary(codes, s, sc, read)
    out2 = oracle.read_boundary(codes, s, sc, read * np.float32(2))
    assert (out2 == 2 * out).all()
    terms = codes.astype(np.float64) * s[:, None] * read[:, None]  # [k, v]
    exact = terms.sum(0) / 127 * sc
    bound = np.abs(terms).sum(0) / 127 * sc
    assert (np.abs(out - exact) <= 130 * 2.0 ** -24 * bound + 1e-30).all()


def test_dense_readout_agrees_with_the_dequantized_state():
    g = datagen.rng(41)
    x = datagen.c1_heads(1, 42)[0]
    codes, s, sc, _, _ = oracle.quantize_kv(x)
    read = g.standard_normal(128).astype(np.float32)
    dense = oracle.dequantize_kv(codes, s, sc).astype(np.float64)
    out = oracle.read_boundary(codes, s, sc, read).astype(np.float64)
    expect = dense.T @ read.astype(np.float64)
    scale = np.abs(dense.T) @ np.abs(read.astype(np.float64))
    assert (np.abs(out - expect) <= 1e-5 * scale + 1e-30).all()
