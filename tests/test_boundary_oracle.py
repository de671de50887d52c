"""CPU pins of the window-boundary refit oracle (oracle/gdn_boundary_oracle.c).

The oracle restates the reference kernels statement by statement; these tests
check it against what the refit must achieve, computed independently in
numpy float64:
* the refit boundary (plus the fitted compensators) reproduces the window's
  dense state -- boundary x gate product + sum_j key_j corr_j^T suffix_j, the
  capsule's DenseState for scalar gates -- within half a quantization step;
* the record scaling and the fp16 record GEMM equal numpy fp16 / fp32 arithmetic;
* the rank-4 power iteration finds a planted dominant singular pair and lowers
  the residual norm (the reference probe's acceptance criterion,
  window_boundary_runtime_probe.cpp:327-329);
* the Newton square root is within 2 ulp of sqrt;
* on a window whose operator is exactly rank one (one record, one column) the
  refit has a closed form that exposes the start vectors and the Newton root
  of zero (check_rank_one_fit).
"""

from __future__ import annotations

import numpy as np
import pytest

import datagen
import oracle
import windowgen as WG
from oracle import window as W

VK = oracle.LAYOUT_VALUE_KEY


def window_dense(buf, s, with_compensators=False):
    """Exact dense state of state s in [key][value] orientation (float64)."""
    codes = buf["residual"][s].astype(np.float64)          # [v][k]
    sm = buf["smoothing"][s].astype(np.float64)            # by key
    sc = buf["scales"][s].astype(np.float64)               # by value
    gates = buf["record_decay"][s].astype(np.float64)
    suffix = np.ones(16)
    for j in range(14, -1, -1):
        suffix[j] = suffix[j + 1] * gates[j + 1]
    total = suffix[0] * gates[0]
    dense = (codes.T / 127.0) * sm[:, None] * sc[None, :] * total
    if with_compensators:
        ck = W.f16_to_f32(buf["compensator_keys"][s]).astype(np.float64)
        cv = W.f16_to_f32(buf["compensator_values"][s]).astype(np.float64)
        dense += ck @ cv.T * total
    rk = W.f16_to_f32(buf["record_keys"][s]).astype(np.float64)
    rc = W.f16_to_f32(buf["record_corrections"][s]).astype(np.float64)
    dense += (rk * suffix[:, None]).T @ rc
    return dense


def refit_dense(out, s, with_compensators=False):
    codes = out["next_residual"][s].astype(np.float64)
    sm = out["next_smoothing"][s].astype(np.float64)
    sc = out["next_scales"][s].astype(np.float64)
    dense = (codes.T / 127.0) * sm[:, None] * sc[None, :]
    if with_compensators:
        nk = W.f16_to_f32(out["next_compensator_keys"][s]).astype(np.float64)
        nv = W.f16_to_f32(out["next_compensator_values"][s]).astype(np.float64)
        dense += nk @ nv.T
    return dense


def step_bound(out, s):
    sm = out["next_smoothing"][s].astype(np.float64)
    sc = out["next_scales"][s].astype(np.float64)
    return (0.5 + 2.0 ** -5) * sm[:, None] * sc[None, :] / 127.0


def full_window(states, seed):
    buf = WG.window_buffers(states, seed, VK, positions=16, compensated=False)
    return buf


def test_boundary_sqrt_is_within_two_ulp():
    g = np.random.default_rng(3)
    x = np.concatenate([10.0 ** g.uniform(-8, 6, 2000), [1e-8, 1.0, 4.0, 2.0 ** 20]]).astype(np.float32)
    got = np.array([W._bind_boundary(W._l()).gdn_oracle_boundary_sqrt(float(v)) for v in x],
                   np.float32)
    want = np.sqrt(x.astype(np.float64))
    assert (np.abs(got - want) <= 2 * np.spacing(want.astype(np.float32))).all()


@pytest.mark.parametrize("merged", [False, True])
def test_quant_only_refit_reproduces_the_window(merged):
    states = 6
    buf = full_window(states, 41)
    out = W.boundary_outputs(states)
    before = WG.copy_buffers(buf)
    merge = None
    if merged:
        scaled = W.boundary_scale_records(buf["record_decay"], buf["record_keys"])
        merge = W.f16_matmul_at_b(buf["record_corrections"], scaled)
    W.window_boundary_quant_only(buf, out, merge)
    for name in ("residual", "smoothing", "scales", "record_decay", "record_keys",
                 "record_corrections"):
        assert np.array_equal(buf[name], before[name]), name
    assert (buf["positions"][:, 0] == 0).all() and (buf["positions"][:, 1:] == 0xA5A5A5A5).all()
    assert np.array_equal(out["next_smoothing"], buf["smoothing"])
    assert not out["next_compensator_keys"].any() and not out["next_compensator_values"].any()
    for s in range(states):
        exact = window_dense(buf, s)
        got = refit_dense(out, s)
        rk = W.f16_to_f32(buf["record_keys"][s]).astype(np.float64)
        rc = W.f16_to_f32(buf["record_corrections"][s]).astype(np.float64)
        record_scale = np.abs(rk).T @ np.abs(rc)
        # fp32 evaluation, plus (merged) fp16 rounding of the scaled record keys.
        slack = (2.0 ** -10 if merged else 2.0 ** -18) * record_scale + 2.0 ** -18 * np.abs(exact)
        assert (np.abs(got - exact) <= step_bound(out, s) * 1.0001 + slack).all(), s
        live = out["next_scales"][s] > 0
        assert (np.abs(out["next_residual"][s][live]).max(axis=1) == 127).all()


def test_record_scaling_and_merge_gemm_match_numpy():
    states = 3
    buf = full_window(states, 43)
    scaled = W.boundary_scale_records(buf["record_decay"], buf["record_keys"])
    keys = buf["record_keys"].view(np.float16)
    for s in range(states):
        for j in range(16):
            suffix = np.float32(1.0)
            for later in range(j + 1, 16):
                suffix = np.float32(suffix * buf["record_decay"][s, later])
            want = (keys[s, j] * np.float16(suffix)).view(np.uint16)
            assert np.array_equal(scaled[s, j], want)
    merge = W.f16_matmul_at_b(buf["record_corrections"], scaled)
    a = buf["record_corrections"].view(np.float16).astype(np.float32)
    b = scaled.view(np.float16).astype(np.float32)
    want = np.zeros((states, 128, 128), np.float32)
    for k in range(16):
        want = (want + a[:, k, :, None] * b[:, k, None, :]).astype(np.float32)
    assert np.array_equal(merge, want)


def planted_window(states, seed):
    """Full windows whose boundary carries a dominant rank-one term."""
    g = datagen.rng(seed)
    buf = WG.window_buffers(states, seed, VK, positions=16, compensated=True)
    for s in range(states):
        u = g.standard_normal(128)
        v = g.standard_normal(128)
        dense = 0.02 * g.standard_normal((128, 128)) + 4.0 * np.outer(u, v) / 128
        codes, sm, sc = oracle.encode_heads(dense[None].astype(np.float32), VK)
        buf["residual"][s], buf["smoothing"][s], buf["scales"][s] = codes[0], sm[0], sc[0]
    return buf


@pytest.mark.parametrize("iterations", [1, 8, 32])
def test_power_refit_fits_and_reencodes_the_window(iterations):
    states = 4
    buf = planted_window(states, 45)
    buf["positions"][3, 0] = 9  # not full: untouched
    out = W.boundary_outputs(states)
    workspace = np.zeros((states, 128, 128), np.float32)
    before = WG.copy_buffers(buf)
    W.window_boundary_power(buf, out, workspace, iterations)
    assert buf["positions"][3, 0] == 9 and not out["next_residual"][3].any()
    assert np.array_equal(buf["record_keys"][3], before["record_keys"][3])
    for s in range(3):
        assert buf["positions"][s, 0] == 0
        assert not buf["record_decay"][s].any() and not buf["record_keys"][s].any()
        assert not buf["record_corrections"][s].any()
        exact = window_dense(before, s, with_compensators=True)
        nk = W.f16_to_f32(out["next_compensator_keys"][s]).astype(np.float64)
        nv = W.f16_to_f32(out["next_compensator_values"][s]).astype(np.float64)
        fitted = nk @ nv.T
        # The workspace is the fitted residual.
        assert np.allclose(workspace[s], exact - fitted, rtol=0, atol=1e-5 * np.abs(exact).max())
        got = refit_dense(out, s, with_compensators=True)
        assert (np.abs(got - exact) <= step_bound(out, s) * 1.0001
                + 2.0 ** -16 * np.abs(exact).max()).all(), s
        # Each fitted right vector is a unit vector (stored in fp16).
        assert np.allclose(np.linalg.norm(nv, axis=0), 1.0, atol=2e-3)
        # The fit lowers the residual norm (the probe's criterion).
        assert np.linalg.norm(exact - fitted) < np.linalg.norm(exact)
        if iterations >= 8:
            # The planted dominant pair is found.
            u, sigma, vt = np.linalg.svd(exact)
            assert sigma[0] > 2 * sigma[1]
            assert abs(nv[:, 0] @ vt[0]) > 0.999
            assert abs(np.linalg.norm(nk[:, 0]) - sigma[0]) < 1e-2 * sigma[0]


def tie_window():
    """Two full windows whose quant-only refit lands on fp16 ties.  Codes 0,
    smoothing 1, every gate 1 (S = 1, suffixes 1) and a single non-zero record
    (the last), so w[k][v] = key[k] * corr[v] exactly (an fp16 x fp16 product)
    and m = w.

    * State 0: key[0] = 127 and key[k] = k - 0.5, corr[v] = +-1, so
      scale' = 127, the multiplier 127 / scale' is 1 and
      t = m * (127 / scale') is exactly k - 0.5: every cell is a tie.
    * State 1: key[0] = 126, corr[v] = +-(1 + v 2^-10), so the multiplier
      127 / scale' rounds, and key[k] is the fp16 value nearest to
      (k - 0.5) 126 / 127: t lands near the ties, often inside half an fp16
      ulp of one without equalling it."""
    buf = WG.window_buffers(2, 97, VK, positions=16)
    buf["residual"][:] = 0
    buf["smoothing"][:] = 1.0
    buf["scales"][:] = 1.0
    buf["record_decay"][:] = 1.0
    keys = np.zeros((2, 16, 128), np.float32)
    corr = np.zeros((2, 16, 128), np.float32)
    k = np.arange(128, dtype=np.float32)
    sign = np.where(np.arange(128) % 2 == 0, 1.0, -1.0).astype(np.float32)
    keys[0, 15] = k - 0.5
    keys[0, 15, 0] = 127.0
    corr[0, 15] = sign
    keys[1, 15] = ((k - 0.5) * 126.0 / 127.0).astype(np.float16).astype(np.float32)
    keys[1, 15, 0] = 126.0
    corr[1, 15] = sign * (1.0 + np.arange(128, dtype=np.float32) * 2.0 ** -10)
    buf["record_keys"] = keys.astype(np.float16).view(np.uint16)
    buf["record_corrections"] = corr.astype(np.float16).view(np.uint16)
    assert np.array_equal(W.f16_to_f32(buf["record_keys"]), keys)  # every value is fp16
    assert np.array_equal(W.f16_to_f32(buf["record_corrections"]), corr)
    return buf, keys[:, 15], corr[:, 15]


def test_quant_only_refit_rounds_fp16_ties_to_even():
    """window_boundary.cpp:465-475: t = m * (127 / scale'), clamped, cast to
    fp16 (round to nearest even) and then to int8 with CAST_RINT (ties to
    even).  At exact ties that is rint, not lround (half away from zero); near
    ties the fp16 cast comes first, so a t just off a tie still rounds as the
    tie.  The expectation is numpy's IEEE fp32 / fp16 arithmetic and rint."""
    buf, keys, corr = tie_window()
    out = W.boundary_outputs(2)
    W.window_boundary_quant_only(buf, out)
    codes = out["next_residual"].astype(np.int64)           # [state][v][k]
    w = (corr[:, :, None] * keys[:, None, :]).astype(np.float32)   # exact products
    scale = np.abs(w).max(axis=2)
    assert np.array_equal(out["next_scales"], scale.astype(np.float32))
    multiplier = (np.float32(127.0) / scale).astype(np.float32)
    t = np.clip((w * multiplier[:, :, None]).astype(np.float32), -127, 127)
    expected = np.rint(t.astype(np.float16).astype(np.float32)).astype(np.int64)
    assert np.array_equal(codes, expected)
    # State 0: every key but 0 is an exact tie k - 0.5; rint and lround differ
    # on the 64 ties with an even integer part (0.5, 2.5, ..., 126.5) per column.
    lround = (np.sign(t) * np.floor(np.abs(t) + 0.5)).astype(np.int64)
    assert (codes[0] != lround[0]).sum() == 128 * 64
    # State 1: cells where the fp16 cast decides (rint without it differs), and
    # where lround differs.
    without_cast = np.rint(t).astype(np.int64)
    assert (codes[1] != without_cast[1]).sum() > 500
    assert (codes[1] != lround[1]).sum() > 1000


@pytest.mark.parametrize("iterations", [1, 4, 32])
def test_power_refit_oracle_equals_a_numpy_transcription(iterations):
    """The C oracle's power refit against a second transcription of the
    reference kernel (tests/powerfit_numpy.py, numpy float32 in the reference's
    statement order), every output bit: codes, smoothing, scales, fp16
    compensators and the fitted residual.  With one iteration the result
    depends on the start vector ((r+1)(c+3) mod 17 - 8, window_boundary.cpp:270)
    and on the 20-step Newton square root (:17-23): a start vector off by one in
    the column or a correctly rounded sqrt changes the bits, so each is pinned."""
    import powerfit_numpy as P

    states = 3
    buf = planted_window(states, 101 + iterations)
    out = W.boundary_outputs(states)
    workspace = np.zeros((states, 128, 128), np.float32)
    ref = WG.copy_buffers(buf)
    W.window_boundary_power(ref, out, workspace, iterations)
    for s in range(states):
        got = P.power_refit(buf, s, iterations)
        for name in ("next_residual", "next_smoothing", "next_scales", "next_compensator_keys",
                     "next_compensator_values"):
            assert got[name].tobytes() == out[name][s].tobytes(), (s, name)
        assert got["workspace"].tobytes() == workspace[s].tobytes(), s
    if iterations == 1:
        shifted = P.power_refit(buf, 0, 1, start=lambda r: (
            (((r + 1) * (np.arange(128) + 4)) % 17) - 8).astype(np.float32))
        assert shifted["next_compensator_values"].tobytes() != \
            out["next_compensator_values"][0].tobytes()
        rounded = P.power_refit(buf, 0, 1, sqrt=lambda v: np.float32(np.sqrt(v)))
        assert rounded["next_smoothing"].tobytes() != out["next_smoothing"][0].tobytes()


def test_newton_square_root_transcription():
    """The transcription's 20-step Newton root: exact on perfect squares and,
    started at max(v, 1), still far from converged for large v (2^60 gives
    about 2^40, not 2^30) -- the reference's own behaviour, which the oracle
    shares (boundary_sqrt)."""
    import powerfit_numpy as P

    for n in (1, 2, 3, 7, 100, 4095):
        assert P.square_root(np.float32(n * n)) == np.float32(n)
    big = P.square_root(np.float32(2.0 ** 60))
    assert 2.0 ** 39 < big < 2.0 ** 41
    values = np.float32(10.0) ** np.linspace(-30, 30, 61).astype(np.float32)
    want = np.array([P.square_root(v) for v in values], np.float32)
    sqrt_c = W._bind_boundary(W._l()).gdn_oracle_boundary_sqrt
    assert np.array_equal(np.array([sqrt_c(float(v)) for v in values], np.float32), want)


# The reference's start vectors, ((rank + 1) * (column + 3)) % 17 - 8
# (window_boundary.cpp:268-271), one row per rank.
START = (((np.arange(4)[:, None] + 1) * (np.arange(128)[None, :] + 3)) % 17 - 8).astype(np.float64)
# s_0 at these columns: -5, -4, -3, 0, 4, 8, 0, 8, 3; where it is 0 the pair is
# fitted at rank 1 (s_1 = 8 there).
RANK_ONE_COLUMNS = (0, 1, 2, 5, 9, 13, 22, 64, 127)


def rank_one_window(columns, seed):
    """Full windows whose only content is the last record: key k (integers
    +-1..6) times correction a e_j with a = 1/4, one column j per state; codes,
    compensators and the other records zero, every gate 1 (the last record's
    suffix is 1 whatever the gates).  The residual operator is exactly
    k a e_j^T, and every product the refit forms from it is exact or rounds
    the same way on both sides of a deflation."""
    states = len(columns)
    buf = WG.window_buffers(states, seed, VK, positions=16, compensated=False)
    buf["residual"][:] = 0
    buf["smoothing"][:] = 1.0
    buf["scales"][:] = 1.0
    buf["record_decay"][:] = 1.0
    g = np.random.default_rng(seed)
    k = (g.integers(1, 7, (states, 128)) * g.choice([-1, 1], (states, 128))).astype(np.float32)
    keys = np.zeros((states, 16, 128), np.float32)
    corr = np.zeros((states, 16, 128), np.float32)
    keys[:, 15] = k
    corr[np.arange(states), 15, list(columns)] = 0.25
    buf["record_keys"] = keys.astype(np.float16).view(np.uint16)
    buf["record_corrections"] = corr.astype(np.float16).view(np.uint16)
    return buf, k


def check_rank_one_fit(nk_bits, nv_bits, workspace, codes, scales, j, k):
    """The refit of rank_one_window's state, in closed form.  Rank r starts
    from s_r / |s_r|.  If s_r[j] != 0 (the first such rank, r*), one power step
    maps it to sign(s_r[j]) e_j exactly after fp16 storage, and the stored pair
    is (sign a k, sign e_j); the deflated operator is then exactly zero.  Every
    other rank sees a zero operator: the first Normalize fails, the loop breaks,
    and the final left vector is zero, whose 20-step Newton root is 2^-20 (from
    1, halved 20 times), above the 1e-20 cut-off, so the rank stores zero keys
    and fp16(s_r / |s_r|) as values.  A correctly rounded square root (0) would
    store nothing; a misread start vector changes the stored values."""
    nk = W.f16_to_f32(nk_bits).astype(np.float64)
    nv = W.f16_to_f32(nv_bits).astype(np.float64)
    fit = next(r for r in range(4) if START[r, j] != 0)
    sign = np.sign(START[fit, j])
    unit = np.zeros(128)
    unit[j] = sign
    assert np.array_equal(nk[:, fit], sign * 0.25 * k), (j, fit)
    assert np.array_equal(nv[:, fit], unit), (j, fit)
    for r in range(4):
        if r == fit:
            continue
        exact = START[r] / np.linalg.norm(START[r])
        assert not nk[:, r].any(), (j, r)
        assert np.array_equal(nv[:, r], exact.astype(np.float16).astype(np.float64)), (j, r)
    assert not np.asarray(workspace).any() and not np.asarray(codes).any()
    assert not np.asarray(scales).any()


def test_start_vector_margins_for_the_closed_form():
    """check_rank_one_fit compares fp16(s_r / |s_r|) exactly: the float32
    normalization is within a few units of 2^-24 of the exact quotient, so
    every value must lie farther than 2^-18 (relative) from an fp16 rounding
    midpoint, and does."""
    for r in range(4):
        exact = START[r] / np.linalg.norm(START[r])
        nz = exact[exact != 0]
        e = np.floor(np.log2(np.abs(nz)))
        frac = np.abs(nz) / 2.0 ** (e - 10)          # units of the fp16 ulp
        assert (np.abs(frac - np.floor(frac) - 0.5) > 2.0 ** -8).all(), r


@pytest.mark.parametrize("iterations", [1, 4, 32])
def test_power_refit_of_a_rank_one_window_in_closed_form(iterations):
    """The oracle's power refit on rank_one_window against check_rank_one_fit;
    the numpy transcription with a start vector shifted by one column or a
    correctly rounded square root fails the same check."""
    import powerfit_numpy as P

    columns = RANK_ONE_COLUMNS
    buf, k = rank_one_window(columns, 211 + iterations)
    out = W.boundary_outputs(len(columns))
    workspace = np.full((len(columns), 128, 128), 7.0, np.float32)
    ref = WG.copy_buffers(buf)
    W.window_boundary_power(ref, out, workspace, iterations)
    for s, j in enumerate(columns):
        check_rank_one_fit(out["next_compensator_keys"][s], out["next_compensator_values"][s],
                           workspace[s], out["next_residual"][s], out["next_scales"][s], j, k[s])
        assert (out["next_smoothing"][s] == out["next_smoothing"][s][0]).all()
        assert abs(out["next_smoothing"][s][0] - 1e-4) < 2e-11
        assert ref["positions"][s, 0] == 0 and not ref["record_keys"][s].any()
    if iterations == 1:
        s, j = 0, columns[0]
        shifted = P.power_refit(buf, s, 1, start=lambda r: (
            (((r + 1) * (np.arange(128) + 4)) % 17) - 8).astype(np.float32))
        rounded = P.power_refit(buf, s, 1, sqrt=lambda v: np.float32(np.sqrt(v)))
        for bad in (shifted, rounded):
            with pytest.raises(AssertionError):
                check_rank_one_fit(bad["next_compensator_keys"], bad["next_compensator_values"],
                                   bad["workspace"], bad["next_residual"], bad["next_scales"],
                                   j, k[s])
