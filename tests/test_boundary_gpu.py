"""GPU parity of the window-boundary refit (include/gdn_state_codec_window.h)
against the oracle (oracle/gdn_boundary_oracle.c), through the C-ABI: every
output bit-exact -- next boundary, smoothing, scales, compensators, workspace,
records and positions -- and untouched buffers untouched."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import windowgen as WG
from gdn_state_codec import native
from oracle import window as W
from test_window_gpu import dev, from_device, stream, to_device, window_ptrs

pytestmark = pytest.mark.gpu

VK = oracle.LAYOUT_VALUE_KEY
OUT_NAMES = ("next_residual", "next_smoothing", "next_scales", "next_compensator_keys",
             "next_compensator_values")


def sentinel_outputs(states):
    out = W.boundary_outputs(states)
    out["next_residual"][:] = 0x5A
    out["next_smoothing"][:] = -3.0
    out["next_scales"][:] = -5.0
    out["next_compensator_keys"][:] = 0x1234
    out["next_compensator_values"][:] = 0x4321
    return out


def out_ptrs(d):
    return [d[k].data_ptr() for k in OUT_NAMES]


def assert_same(got: dict, want: dict, names):
    for name in names:
        assert got[name].tobytes() == want[name].tobytes(), name


def test_quant_only_refit_is_bit_exact(device):
    states = 384
    print(f"quant-only refit states={states}", flush=True)
    buf = WG.window_buffers(states, 61, VK, positions=(list(range(17)) * 23)[:states])
    out = sentinel_outputs(states)
    d, do = to_device(buf, device), to_device(out, device)
    workspace = torch.zeros(16, dtype=torch.float32, device=device)
    assert native().window_boundary_launch_v1(
        stream(), *window_ptrs(d), *out_ptrs(do), workspace.data_ptr(), states, 0) == 0
    torch.cuda.synchronize()
    ref, ref_out = WG.copy_buffers(buf), WG.copy_buffers(out)
    W.window_boundary_quant_only(ref, ref_out)
    assert_same(from_device(do, out), ref_out, OUT_NAMES)
    assert_same(from_device(d, buf), ref, buf.keys())


def test_boundary_runtime_and_cube_finish_are_bit_exact(device):
    states = 32
    print(f"boundary runtime + cube finish states={states}", flush=True)
    buf = WG.window_buffers(states, 63, VK, positions=16)
    out = sentinel_outputs(states)
    d, do = to_device(buf, device), to_device(out, device)
    scaled = torch.zeros((states, 16, 128), dtype=torch.int16, device=device)
    merge = torch.zeros((states, 128, 128), dtype=torch.float32, device=device)
    lib = native()
    handle = lib.boundary_runtime_create_v1(states)
    assert handle
    try:
        assert lib.boundary_runtime_step_v1(
            handle, stream(), d["record_decay"].data_ptr(), d["record_keys"].data_ptr(),
            d["record_corrections"].data_ptr(), scaled.data_ptr(), merge.data_ptr(), states) == 0
    finally:
        lib.boundary_runtime_destroy_v1(handle)
    assert lib.window_boundary_cube_finish_launch_v1(
        stream(), *window_ptrs(d), *out_ptrs(do), merge.data_ptr(), states) == 0
    torch.cuda.synchronize()
    scaled_ref = W.boundary_scale_records(buf["record_decay"], buf["record_keys"])
    merge_ref = W.f16_matmul_at_b(buf["record_corrections"], scaled_ref)
    assert np.array_equal(scaled.cpu().numpy().view(np.uint16), scaled_ref)
    assert merge.cpu().numpy().tobytes() == merge_ref.tobytes()
    ref, ref_out = WG.copy_buffers(buf), WG.copy_buffers(out)
    W.window_boundary_quant_only(ref, ref_out, merge_ref)
    assert_same(from_device(do, out), ref_out, OUT_NAMES)
    assert_same(from_device(d, buf), ref, buf.keys())


def test_scale_records_and_record_gemm_entry_points(device):
    states = 128
    print("scale_records + bf16_cube_matmul", flush=True)
    buf = WG.window_buffers(states, 65, VK, positions=16)
    d = to_device(buf, device)
    scaled = torch.zeros((states, 16, 128), dtype=torch.int16, device=device)
    assert native().boundary_scale_records_launch_v1(
        stream(), d["record_decay"].data_ptr(), d["record_keys"].data_ptr(), scaled.data_ptr(),
        states) == 0
    c = torch.zeros((states, 128, 128), dtype=torch.float32, device=device)
    ws = torch.zeros(16, dtype=torch.int32, device=device)
    assert native().bf16_cube_matmul_launch_v1(
        stream(), d["record_corrections"].data_ptr(), scaled.data_ptr(), c.data_ptr(), states,
        ws.data_ptr(), ws.data_ptr(), states // 2) == 0
    torch.cuda.synchronize()
    scaled_ref = W.boundary_scale_records(buf["record_decay"], buf["record_keys"])
    assert np.array_equal(scaled.cpu().numpy().view(np.uint16), scaled_ref)
    assert c.cpu().numpy().tobytes() == W.f16_matmul_at_b(buf["record_corrections"],
                                                          scaled_ref).tobytes()


@pytest.mark.parametrize("iterations", [1, 5, 32])
def test_power_refit_is_bit_exact(device, iterations):
    states = 10
    print(f"power refit iterations={iterations}", flush=True)
    from test_boundary_oracle import planted_window

    buf = planted_window(states, 67)
    buf["positions"][[2, 7], 0] = [5, 15]  # not full: untouched
    out = sentinel_outputs(states)
    workspace = np.full((states, 128, 128), 7.0, np.float32)
    d, do = to_device(buf, device), to_device(out, device)
    dw = dev(workspace, device)
    assert native().window_boundary_launch_v1(
        stream(), *window_ptrs(d), *out_ptrs(do), dw.data_ptr(), states, iterations) == 0
    torch.cuda.synchronize()
    ref, ref_out, ref_ws = WG.copy_buffers(buf), WG.copy_buffers(out), workspace.copy()
    W.window_boundary_power(ref, ref_out, ref_ws, iterations)
    assert_same(from_device(do, out), ref_out, OUT_NAMES)
    assert_same(from_device(d, buf), ref, buf.keys())
    assert dw.cpu().numpy().tobytes() == ref_ws.tobytes()


@pytest.mark.parametrize("iterations", [1, 32])
def test_power_refit_of_a_rank_one_window_in_closed_form(device, iterations):
    """Windows whose operator is exactly rank one: the kernel's compensators,
    workspace and codes follow the closed form (the fitted pair at the first
    rank whose start vector touches the column, the other ranks' start vectors
    stored as values), and every output equals the oracle's."""
    from test_boundary_oracle import RANK_ONE_COLUMNS, check_rank_one_fit, rank_one_window

    columns = RANK_ONE_COLUMNS
    states = len(columns)
    print(f"power refit, rank-one windows, iterations={iterations}", flush=True)
    buf, k = rank_one_window(columns, 311 + iterations)
    out = sentinel_outputs(states)
    workspace = np.full((states, 128, 128), 7.0, np.float32)
    d, do = to_device(buf, device), to_device(out, device)
    dw = dev(workspace, device)
    assert native().window_boundary_launch_v1(
        stream(), *window_ptrs(d), *out_ptrs(do), dw.data_ptr(), states, iterations) == 0
    torch.cuda.synchronize()
    got, ws = from_device(do, out), dw.cpu().numpy()
    for s, j in enumerate(columns):
        check_rank_one_fit(got["next_compensator_keys"][s], got["next_compensator_values"][s],
                           ws[s], got["next_residual"][s], got["next_scales"][s], j, k[s])
    ref, ref_out, ref_ws = WG.copy_buffers(buf), WG.copy_buffers(out), workspace.copy()
    W.window_boundary_power(ref, ref_out, ref_ws, iterations)
    assert_same(got, ref_out, OUT_NAMES)
    assert_same(from_device(d, buf), ref, buf.keys())
    assert ws.tobytes() == ref_ws.tobytes()


def test_power_refit_with_tiny_rows_is_bit_exact(device):
    """States whose fitted residual has tiny rows (smoothing scaled by
    2^-110, records and compensators zero: non-zero cells below 2^-100 and
    a floored fresh smoothing), large rows (smoothing scaled by 2^10) and
    rows alternating between tiny and ordinary in one state: the re-encode's
    divisions, maxima and codes must be as bit-exact as for ordinary states.
    (A fresh smoothing above 2^20 needs a mean |cell| above 2^40, which the
    fp16 compensator factors cannot carry: such a state overflows them to
    inf first.)"""
    states = 48
    print(f"power refit, tiny and mixed rows, states={states}", flush=True)
    buf = WG.window_buffers(states, 91, VK, positions=16)
    quiet = np.r_[0:16, 32:48]
    for name in ("record_corrections", "compensator_keys", "compensator_values"):
        buf[name][quiet] = 0
    buf["smoothing"][0:16] *= np.float32(2.0 ** -110)
    buf["smoothing"][16:32] *= np.float32(2.0 ** 10)
    buf["smoothing"][32:48, ::2] *= np.float32(2.0 ** -110)
    out = sentinel_outputs(states)
    workspace = np.full((states, 128, 128), 7.0, np.float32)
    d, do = to_device(buf, device), to_device(out, device)
    dw = dev(workspace, device)
    assert native().window_boundary_launch_v1(
        stream(), *window_ptrs(d), *out_ptrs(do), dw.data_ptr(), states, 4) == 0
    torch.cuda.synchronize()
    ref, ref_out, ref_ws = WG.copy_buffers(buf), WG.copy_buffers(out), workspace.copy()
    W.window_boundary_power(ref, ref_out, ref_ws, 4)
    assert_same(from_device(do, out), ref_out, OUT_NAMES)
    assert_same(from_device(d, buf), ref, buf.keys())
    assert dw.cpu().numpy().tobytes() == ref_ws.tobytes()
    tiny = np.abs(ref_ws[0:16])
    assert ((tiny > 0) & (tiny < 2.0 ** -100)).any()  # the data reaches that range


def _full_batch(seed):
    """B = 256 sequences x 32 value heads, the bench's refit batch: every
    seventeenth state is not full (positions 0..15 in turn) and must come back
    untouched."""
    states = 8192
    positions = [16] * states
    for n, s in enumerate(range(0, states, 17)):
        positions[s] = n % 16
    return states, WG.window_buffers(states, seed, VK, positions=positions)


def _subset(buffers: dict, idx):
    return {k: np.ascontiguousarray(v[idx]) for k, v in buffers.items()}


def test_quant_only_refit_full_batch_is_bit_exact(device):
    """All 8192 states of one launch against the oracle, every output bit."""
    states, buf = _full_batch(73)
    print(f"quant-only refit states={states}", flush=True)
    out = sentinel_outputs(states)
    d, do = to_device(buf, device), to_device(out, device)
    workspace = torch.zeros(16, dtype=torch.float32, device=device)
    assert native().window_boundary_launch_v1(
        stream(), *window_ptrs(d), *out_ptrs(do), workspace.data_ptr(), states, 0) == 0
    torch.cuda.synchronize()
    ref, ref_out = WG.copy_buffers(buf), WG.copy_buffers(out)
    W.window_boundary_quant_only(ref, ref_out)
    assert_same(from_device(do, out), ref_out, OUT_NAMES)
    assert_same(from_device(d, buf), ref, buf.keys())


def test_power_refit_full_batch(device):
    """One 4-iteration launch over 8192 states: every fourth state against the
    oracle (outputs, records, positions and its workspace rows), and every
    state that is not full left untouched, its outputs and workspace too."""
    states, buf = _full_batch(79)
    print(f"power refit states={states}", flush=True)
    out = sentinel_outputs(states)
    d, do = to_device(buf, device), to_device(out, device)
    dw = torch.full((states, 128, 128), 7.0, dtype=torch.float32, device=device)
    assert native().window_boundary_launch_v1(
        stream(), *window_ptrs(d), *out_ptrs(do), dw.data_ptr(), states, 4) == 0
    torch.cuda.synchronize()
    got_out, got_buf = from_device(do, out), from_device(d, buf)
    got_ws = dw.cpu().numpy()
    idx = np.arange(0, states, 4)
    ref, ref_out = _subset(buf, idx), _subset(out, idx)
    ref_ws = np.full((idx.size, 128, 128), 7.0, np.float32)
    W.window_boundary_power(ref, ref_out, ref_ws, 4)
    assert_same(_subset(got_out, idx), ref_out, OUT_NAMES)
    assert_same(_subset(got_buf, idx), ref, buf.keys())
    assert got_ws[idx].tobytes() == ref_ws.tobytes()
    waiting = np.flatnonzero(buf["positions"][:, 0] < 16)
    assert waiting.size == len(range(0, states, 17))
    assert_same(_subset(got_out, waiting), _subset(out, waiting), OUT_NAMES)
    assert_same(_subset(got_buf, waiting), _subset(buf, waiting), buf.keys())
    assert (got_ws[waiting] == 7.0).all()


def test_quant_only_refit_outside_the_fast_division_domain(device):
    """States whose smoothing lies outside [2^-20, 2^20], or whose boundary
    values reach the subnormal range, take the IEEE division; they must be as
    bit-exact as the others.  Sixteen states share each wavefront pattern."""
    states = 64
    print(f"quant-only refit, extreme smoothing, states={states}", flush=True)
    buf = WG.window_buffers(states, 83, VK, positions=16)
    buf["smoothing"][0:16] *= np.float32(2.0 ** -30)    # s below the fast domain
    buf["smoothing"][16:32] *= np.float32(2.0 ** 30)    # s above it
    buf["smoothing"][32:48] *= np.float32(2.0 ** -60)   # w/s products near underflow
    buf["residual"][48] = 0                              # w = records only
    buf["smoothing"][49, ::2] = np.float32(2.0 ** -40)   # mixed lanes in one state
    buf["smoothing"][49, 1::2] = np.float32(2.0 ** 40)
    out = sentinel_outputs(states)
    d, do = to_device(buf, device), to_device(out, device)
    workspace = torch.zeros(16, dtype=torch.float32, device=device)
    assert native().window_boundary_launch_v1(
        stream(), *window_ptrs(d), *out_ptrs(do), workspace.data_ptr(), states, 0) == 0
    torch.cuda.synchronize()
    ref, ref_out = WG.copy_buffers(buf), WG.copy_buffers(out)
    W.window_boundary_quant_only(ref, ref_out)
    assert_same(from_device(do, out), ref_out, OUT_NAMES)
    assert_same(from_device(d, buf), ref, buf.keys())


def test_quant_only_refit_at_fp16_ties(device):
    """The window whose requantization lands on fp16 ties (and within half an
    fp16 ulp of them): the GPU's fp16 cast and round-to-even agree with the
    oracle on every code."""
    from test_boundary_oracle import tie_window

    buf, _, _ = tie_window()
    print("quant-only refit at fp16 ties, states=2", flush=True)
    out = sentinel_outputs(2)
    d, do = to_device(buf, device), to_device(out, device)
    workspace = torch.zeros(16, dtype=torch.float32, device=device)
    assert native().window_boundary_launch_v1(
        stream(), *window_ptrs(d), *out_ptrs(do), workspace.data_ptr(), 2, 0) == 0
    torch.cuda.synchronize()
    ref, ref_out = WG.copy_buffers(buf), WG.copy_buffers(out)
    W.window_boundary_quant_only(ref, ref_out)
    assert_same(from_device(do, out), ref_out, OUT_NAMES)
    assert_same(from_device(d, buf), ref, buf.keys())
