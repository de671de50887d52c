"""CPU pins of the device rank-4 chain oracle (oracle/gdn_encoded_oracle.c):
finish_encoded_projection, commit_encoded_rank and encoded_requantize
(encoded_projection.cpp:82-163, 778-865; encoded_requantize.cpp:72-166).

* encoded_requantize equals, bit for bit, the re-encode stage of the pinned
  power-refit restatement (gdn_boundary_oracle.c) fed the same window and the
  same fitted ranks: the two kernels evaluate the same residual cell, smoothing,
  scales and codes over transposed layouts.
* finish_encoded_projection and commit_encoded_rank are checked against a
  numpy float64 evaluation of the operator rows they compute, written from the
  reference's formulas with explicit left / right / transpose choices; planted
  mistakes in that evaluation (swapped sides, wrong axis scale, suffix dropped,
  a basis read in the other layout) are shown to exceed the tolerance, so the
  check can tell them apart.
* commit's closed forms: new_right[rank] is the input's fp16 bits, new_left[rank]
  is fp16(corrected), nothing else is written.
* the whole chain (prepare -> int8 GEMM -> finish, both directions, -> commit,
  then requantize), driven as the reference's probe drives it, finds a planted
  dominant pair and re-encodes the window within a quantization step.
"""

from __future__ import annotations

import numpy as np
import pytest

import datagen
import oracle
import windowgen as WG
from oracle import window as W

VK = oracle.LAYOUT_VALUE_KEY
DIM = 128


def encoded_window(states, seed, planted=False, bases=0):
    """Operands of the encoded chain for full windows: the boundary as
    [row = smoothing axis][column = scale axis] codes, old compensators as the
    old bases, records as the record bases; `bases` ranks of random fp16 fitted
    bases ([rank][dim])."""
    g = datagen.rng(seed)
    buf = WG.window_buffers(states, seed, VK, positions=16, compensated=True)
    if planted:
        for s in range(states):
            u, v = g.standard_normal(128), g.standard_normal(128)
            dense = 0.02 * g.standard_normal((128, 128)) + 4.0 * np.outer(u, v) / 128
            codes, sm, sc = oracle.encode_heads(dense[None].astype(np.float32), VK)
            buf["residual"][s], buf["smoothing"][s], buf["scales"][s] = codes[0], sm[0], sc[0]
    new_left = np.zeros((states, 4, DIM), np.uint16)
    new_right = np.zeros((states, 4, DIM), np.uint16)
    if bases:
        new_left[:, :bases] = W.f32_to_f16(g.standard_normal((states, bases, DIM)) * 0.05)
        new_right[:, :bases] = W.f32_to_f16(g.standard_normal((states, bases, DIM)) * 0.05)
    enc = {"smoothing": buf["smoothing"], "scales": buf["scales"],
           "old_left": buf["compensator_keys"], "old_right": buf["compensator_values"],
           "record_decay": buf["record_decay"], "record_left": buf["record_keys"],
           "record_right": buf["record_corrections"], "new_left": new_left,
           "new_right": new_right}
    enc = {k: np.ascontiguousarray(v) for k, v in enc.items()}
    residual = np.ascontiguousarray(buf["residual"].transpose(0, 2, 1))
    return buf, enc, residual


def vector_inputs(states, seed):
    """fp16 [S][128][16]: column 0 the vector, the other columns noise the
    kernels must ignore."""
    g = datagen.rng(seed)
    x = g.standard_normal((states, DIM, 16))
    return W.f32_to_f16(x)


def f64(bits):
    return W.f16_to_f32(bits).astype(np.float64)


def operator_rows(enc, residual_unused, projected, dynamic_scale, inputs, fitted, transpose,
                  mistake=None):
    """float64 evaluation of Value (:125-163) for every row, from the
    reference's formulas: coefficients on the input side's bases, outputs on
    the other side's."""
    left_side = transpose == 1
    if mistake == "swap_sides":
        left_side = not left_side
    old_in = f64(enc["old_left"] if left_side else enc["old_right"])       # [S][dim][rank]
    old_out = f64(enc["old_right"] if left_side else enc["old_left"])
    new_in = f64(enc["new_left"] if left_side else enc["new_right"])       # [S][rank][dim]
    new_out = f64(enc["new_right"] if left_side else enc["new_left"])
    rec_in = f64(enc["record_left"] if left_side else enc["record_right"])  # [S][16][dim]
    rec_out = f64(enc["record_right"] if left_side else enc["record_left"])
    axis = enc["scales"] if transpose == 1 else enc["smoothing"]
    if mistake == "axis":
        axis = enc["smoothing"] if transpose == 1 else enc["scales"]
    if mistake == "basis_layout":  # a [rank][dim] basis read as [dim][rank]
        new_in = new_in.reshape(-1, DIM, 4).transpose(0, 2, 1)
        new_out = new_out.reshape(-1, DIM, 4).transpose(0, 2, 1)
    x = f64(inputs[:, :, 0])
    decay = enc["record_decay"].astype(np.float64)
    states = x.shape[0]
    rows = np.zeros((states, DIM))
    for s in range(states):
        suffix = np.ones(16)
        for j in range(14, -1, -1):
            suffix[j] = suffix[j + 1] * decay[s, j + 1]
        total = suffix[0] * decay[s, 0]
        coef = old_in[s].T @ x[s]
        coef_new = new_in[s] @ x[s]
        rcoef = rec_in[s] @ x[s]
        if mistake != "no_suffix":
            rcoef = rcoef * suffix
        value = (projected[s, :, 0].astype(np.float64) * float(dynamic_scale[s, 0]) / 127.0
                 * axis[s].astype(np.float64) * total)
        value += old_out[s] @ coef * total
        value -= new_out[s][:fitted].T @ coef_new[:fitted]
        value += rec_out[s].T @ rcoef
        rows[s] = value
    return rows


def project(enc, residual, inputs, transpose):
    axis_in = enc["smoothing"] if transpose == 1 else enc["scales"]
    q, dyn = W.prepare_int8_vector(inputs, axis_in)
    return W.int8_matmul(residual, q, transpose), dyn


def close(got, want, rel):
    scale = np.abs(want).max(axis=1, keepdims=True)
    return np.abs(got - want) <= rel * scale


@pytest.mark.parametrize("iterations", [1, 8])
def test_requantize_equals_the_power_refit_reencode(iterations):
    states = 3
    buf, enc, residual = encoded_window(states, 61, planted=True)
    before = WG.copy_buffers(buf)
    out = W.boundary_outputs(states)
    workspace = np.zeros((states, DIM, DIM), np.float32)
    W.window_boundary_power(buf, out, workspace, iterations)
    enc["new_left"] = np.ascontiguousarray(out["next_compensator_keys"].transpose(0, 2, 1))
    enc["new_right"] = np.ascontiguousarray(out["next_compensator_values"].transpose(0, 2, 1))
    for key, name in (("record_decay", "record_decay"), ("record_left", "record_keys"),
                      ("record_right", "record_corrections")):
        enc[key] = before[name]
    got = W.encoded_requantize(enc, residual)
    assert got["workspace"].tobytes() == workspace.tobytes()
    assert got["next_smoothing"].tobytes() == out["next_smoothing"].tobytes()
    assert got["next_scales"].tobytes() == out["next_scales"].tobytes()
    assert np.array_equal(got["next_residual"], out["next_residual"].transpose(0, 2, 1))
    assert np.array_equal(got["next_left"], out["next_compensator_keys"])
    assert np.array_equal(got["next_right"], out["next_compensator_values"])
    # Negative control: the same fit with one committed basis element moved
    # changes the workspace.
    enc["new_left"][0, 0, 5] ^= 0x0400
    moved = W.encoded_requantize(enc, residual)
    assert moved["workspace"][0].tobytes() != workspace[0].tobytes()


@pytest.mark.parametrize("transpose", [0, 1])
@pytest.mark.parametrize("fitted", [0, 2, 4])
def test_finish_normalizes_the_operator_rows(transpose, fitted):
    states = 4
    _, enc, residual = encoded_window(states, 71 + fitted, bases=4)
    inputs = vector_inputs(states, 72)
    projected, dyn = project(enc, residual, inputs, transpose)
    out = W.finish_encoded_projection(enc, projected, dyn, inputs, fitted, transpose)
    assert not out[:, :, 1:].any()
    got = W.f16_to_f32(out[:, :, 0]).astype(np.float64)
    rows = operator_rows(enc, residual, projected, dyn, inputs, fitted, transpose)
    want = rows / np.linalg.norm(rows, axis=1, keepdims=True)
    # fp16 output (2^-11 relative) of fp32 sums over 128 terms.
    assert close(got, want, 2.0 ** -9).all()
    for mistake in ("swap_sides", "axis", "no_suffix", "basis_layout"):
        if mistake == "basis_layout" and fitted == 0:
            continue
        wrong = operator_rows(enc, residual, projected, dyn, inputs, fitted, transpose, mistake)
        wrong /= np.linalg.norm(wrong, axis=1, keepdims=True)
        assert not close(got, wrong, 2.0 ** -9).all(), mistake


def test_finish_of_a_zero_vector_is_zero():
    states = 2
    _, enc, residual = encoded_window(states, 81)
    inputs = np.zeros((states, DIM, 16), np.uint16)
    projected, dyn = project(enc, residual, inputs, 0)
    out = W.finish_encoded_projection(enc, projected, dyn, inputs, 0, 0)
    assert not out.any()


@pytest.mark.parametrize("rank", [0, 1, 3])
def test_commit_closed_forms(rank):
    states = 3
    _, enc, residual = encoded_window(states, 91 + rank, bases=4)
    inputs = vector_inputs(states, 92)
    projected, dyn = project(enc, residual, inputs, 0)
    corrected = datagen.rng(93).standard_normal((states, DIM, 16)).astype(np.float32)
    before = {k: v.copy() for k, v in enc.items()}
    garbage = corrected.copy()
    W.commit_encoded_rank(enc, projected, dyn, inputs, corrected, rank)
    assert np.array_equal(enc["new_right"][:, rank], inputs[:, :, 0])
    assert np.array_equal(enc["new_left"][:, rank], W.f32_to_f16(corrected[:, :, 0]))
    others = [r for r in range(4) if r != rank]
    assert np.array_equal(enc["new_left"][:, others], before["new_left"][:, others])
    assert np.array_equal(enc["new_right"][:, others], before["new_right"][:, others])
    assert np.array_equal(corrected[:, :, 1:], garbage[:, :, 1:])
    rows = operator_rows(before, residual, projected, dyn, inputs, rank, 0)
    assert close(corrected[:, :, 0].astype(np.float64), rows, 2.0 ** -16).all()
    wrong = operator_rows(before, residual, projected, dyn, inputs, rank, 0, "swap_sides")
    assert not close(corrected[:, :, 0].astype(np.float64), wrong, 2.0 ** -16).all()


def run_chain(enc, residual, seeds, iterations):
    """The reference probe's rank chain (encoded_projection_probe.cpp:620-654)."""
    states = residual.shape[0]
    corrected = np.zeros((states, DIM, 16), np.float32)
    for rank in range(4):
        vector = seeds[rank].copy()
        for _ in range(iterations):
            projected, dyn = project(enc, residual, vector, 0)
            output = W.finish_encoded_projection(enc, projected, dyn, vector, rank, 0)
            projected, dyn = project(enc, residual, output, 1)
            vector = W.finish_encoded_projection(enc, projected, dyn, output, rank, 1)
        projected, dyn = project(enc, residual, vector, 0)
        W.commit_encoded_rank(enc, projected, dyn, vector, corrected, rank)
    return W.encoded_requantize(enc, residual)


def test_chain_finds_a_planted_pair_and_reencodes_the_window():
    states = 2
    buf, enc, residual = encoded_window(states, 101, planted=True)
    g = datagen.rng(102)
    seeds = [W.f32_to_f16(np.concatenate(
        [g.standard_normal((states, DIM, 1)), np.zeros((states, DIM, 15))], axis=2))
        for _ in range(4)]
    out = run_chain(enc, residual, seeds, 8)
    for s in range(states):
        dense = WG_window_dense(buf, s)
        left = f64(enc["new_left"][s]).T    # [dim][rank]
        right = f64(enc["new_right"][s]).T
        u, sigma, vt = np.linalg.svd(dense)
        assert sigma[0] > 2 * sigma[1]
        assert abs(right[:, 0] @ vt[0]) / np.linalg.norm(right[:, 0]) > 0.99
        fitted = left @ right.T
        assert np.linalg.norm(dense - fitted) < np.linalg.norm(dense)
        # The workspace is the window minus the committed fit, and the codes
        # re-encode it within half a step.
        assert np.allclose(out["workspace"][s], dense - fitted, rtol=0,
                           atol=1e-5 * np.abs(dense).max())
        codes = out["next_residual"][s].astype(np.float64)
        sm = out["next_smoothing"][s].astype(np.float64)
        sc = out["next_scales"][s].astype(np.float64)
        step = sm[:, None] * sc[None, :] / 127.0
        assert (np.abs(codes / 127.0 * sm[:, None] * sc[None, :] - (dense - fitted))
                <= (0.5 + 2.0 ** -5) * step * 1.0001 + 2.0 ** -16 * np.abs(dense).max()).all()


def WG_window_dense(buf, s):
    """Exact window operator [key][value] (float64) with old compensators."""
    codes = buf["residual"][s].astype(np.float64)          # [v][k]
    sm = buf["smoothing"][s].astype(np.float64)
    sc = buf["scales"][s].astype(np.float64)
    gates = buf["record_decay"][s].astype(np.float64)
    suffix = np.ones(16)
    for j in range(14, -1, -1):
        suffix[j] = suffix[j + 1] * gates[j + 1]
    total = suffix[0] * gates[0]
    dense = (codes.T / 127.0) * sm[:, None] * sc[None, :] * total
    ck = f64(buf["compensator_keys"][s])
    cv = f64(buf["compensator_values"][s])
    dense += ck @ cv.T * total
    rk = f64(buf["record_keys"][s])
    rc = f64(buf["record_corrections"][s])
    dense += (rk * suffix[:, None]).T @ rc
    return dense
