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
* the Newton square root is within 2 ulp of sqrt.
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
