"""GPU parity of the windowed decode step (include/gdn_state_codec_window.h)
against the CPU oracle (oracle/gdn_window_oracle.c), through the C-ABI.

Bars:
* fused steps: outputs and stored corrections lie within 2^-14 of the double
  result's error scale (sum of |terms|, out_bound / corr_bound from the
  oracle) plus half an ulp of their 16-bit format; record keys, gates,
  positions and every untouched byte are bit-exact; full windows are skipped.
* decode-pair chain (prepare / int8 projection / finish) and the fused decode
  runtime step: bit-exact with the oracle's statement of the reference kernels.
* dense fp32 step: bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
import windowgen as WG
from gdn_state_codec import native
from oracle import window as W

pytestmark = pytest.mark.gpu

KV, VK = oracle.LAYOUT_KEY_VALUE, oracle.LAYOUT_VALUE_KEY
E_SCALE = 2.0 ** -14
_VIEW = {np.dtype(np.uint16): np.int16, np.dtype(np.uint32): np.int32}
_BACK = {torch.int16: np.uint16, torch.int32: None}


def ulp(x, mantissa_bits):
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -300)))
    return 2.0 ** np.maximum(e - mantissa_bits, -24)


def dev(a, device):
    a = np.ascontiguousarray(a)
    view = _VIEW.get(a.dtype)
    return torch.from_numpy(a.view(view) if view else a.copy()).to(device)


def host(t: torch.Tensor, dtype) -> np.ndarray:
    return t.cpu().numpy().view(dtype)


def stream():
    return torch.cuda.current_stream().cuda_stream


def to_device(buf: dict, device) -> dict:
    return {k: dev(v, device) for k, v in buf.items()}


def from_device(d: dict, like: dict) -> dict:
    return {k: host(d[k], like[k].dtype).reshape(like[k].shape) for k in like}


def window_ptrs(d):
    return [d[k].data_ptr() for k in ("residual", "smoothing", "scales", "compensator_keys",
                                      "compensator_values", "record_decay", "record_keys",
                                      "record_corrections", "positions")]


SENTINEL16 = 0x7E5A  # a bf16 / fp16 pattern no step writes for these inputs


def run_bf16_step(d, di, states, quant_only, device):
    out = torch.full((states, 128), SENTINEL16, dtype=torch.int16, device=device)
    fn = (native().windowed_gdn_step_bf16_quant_only_launch_v1 if quant_only
          else native().windowed_gdn_step_bf16_launch_v1)
    status = fn(stream(), *window_ptrs(d), di["log_decay"].data_ptr(), di["beta"].data_ptr(),
                di["keys"].data_ptr(), di["queries"].data_ptr(), di["values"].data_ptr(),
                out.data_ptr(), states)
    assert status == 0
    torch.cuda.synchronize()
    return host(out, np.uint16)


def check_step(before, after_gpu, after_ref, out_gpu, out_ref, out64, out_bound, corr64,
               corr_bound, out_bits):
    """Compare one step's GPU results with the oracle's (see module docstring)."""
    pos = before["positions"][:, 0]
    live = pos < 16
    for name in ("residual", "smoothing", "scales", "compensator_keys", "compensator_values"):
        assert np.array_equal(after_gpu[name], before[name]), name
    assert np.array_equal(after_gpu["positions"], after_ref["positions"])
    assert np.array_equal(after_gpu["record_decay"], after_ref["record_decay"])
    assert np.array_equal(after_gpu["record_keys"], after_ref["record_keys"])
    # Corrections: every row but the new one is untouched; the new one within bound.
    rc_gpu = after_gpu["record_corrections"].copy()
    rc_ref = after_ref["record_corrections"].copy()
    for s in np.flatnonzero(live):
        p = pos[s]
        c = W.f16_to_f32(rc_gpu[s, p]).astype(np.float64)
        tol = E_SCALE * corr_bound[s] + 0.5 * ulp(np.abs(corr64[s]) + E_SCALE * corr_bound[s], 10)
        bad = np.abs(c - corr64[s]) > tol
        assert not bad.any(), (s, p, np.flatnonzero(bad)[:4], c[bad][:4], corr64[s][bad][:4])
        rc_gpu[s, p] = rc_ref[s, p]
    assert np.array_equal(rc_gpu, rc_ref)
    # Outputs.
    if out_bits == 16:
        got = oracle.bf16_to_f32(out_gpu).astype(np.float64)
        assert (out_gpu[~live] == SENTINEL16).all()
        tol = E_SCALE * out_bound + 0.5 * ulp(np.abs(out64) + E_SCALE * out_bound, 7)
    else:
        got = out_gpu.astype(np.float64)
        assert np.isnan(out_gpu[~live]).all()
        tol = E_SCALE * out_bound
    bad = (np.abs(got - out64) > tol) & live[:, None]
    assert not bad.any(), (np.argwhere(bad)[:4], got[bad][:4], out64[bad][:4])


@pytest.mark.parametrize("quant_only", [False, True])
def test_bf16_step_matches_oracle(device, quant_only):
    states = 96
    print(f"bf16 windowed step quant_only={quant_only} states={states}", flush=True)
    positions = (list(range(18)) * 6)[:states]
    buf = WG.window_buffers(states, 21, VK, positions=positions)
    inp = WG.bf16_inputs(states, 22)
    ref = WG.copy_buffers(buf)
    out_ref, out64, out_bound, corr64, corr_bound = W.windowed_step_bf16(
        ref, **inp, quant_only=quant_only)
    d = to_device(buf, device)
    di = to_device(inp, device)
    out = run_bf16_step(d, di, states, quant_only, device)
    check_step(buf, from_device(d, buf), ref, out, out_ref, out64, out_bound, corr64,
               corr_bound, 16)


def test_f16_step_matches_oracle(device):
    states = 64
    print(f"fp16 windowed step states={states}", flush=True)
    positions = (list(range(18)) * 4)[:states]
    buf = WG.window_buffers(states, 23, KV, positions=positions)
    inp = WG.f16_inputs(states, 24)
    ref = WG.copy_buffers(buf)
    out_ref, out64, out_bound, corr64, corr_bound = W.windowed_step_f16(ref, **inp)
    d = to_device(buf, device)
    di = to_device(inp, device)
    out = torch.full((states, 128), float("nan"), dtype=torch.float32, device=device)
    status = native().windowed_gdn_step_launch_v1(
        stream(), *window_ptrs(d), di["decay"].data_ptr(), di["write_keys"].data_ptr(),
        di["reads"].data_ptr(), di["queries"].data_ptr(), di["values"].data_ptr(),
        out.data_ptr(), states)
    assert status == 0
    torch.cuda.synchronize()
    check_step(buf, from_device(d, buf), ref, out.cpu().numpy(), out_ref, out64, out_bound,
               corr64, corr_bound, 32)


@pytest.mark.parametrize("quant_only", [True, False])
def test_bf16_window_of_sixteen_steps(device, quant_only):
    """A whole window from position 0: each GPU step is checked against the
    oracle applied to the GPU's own buffers before that step; a 17th step on the
    full window changes nothing."""
    states = 32
    print(f"bf16 16-step window quant_only={quant_only}", flush=True)
    buf = WG.window_buffers(states, 25, VK, positions=0, compensated=not quant_only)
    d = to_device(buf, device)
    for step in range(17):
        inp = WG.bf16_inputs(states, 100 + step)
        di = to_device(inp, device)
        before = from_device(d, buf)
        ref = WG.copy_buffers(before)
        out_ref, out64, out_bound, corr64, corr_bound = W.windowed_step_bf16(
            ref, **inp, quant_only=quant_only)
        out = run_bf16_step(d, di, states, quant_only, device)
        check_step(before, from_device(d, buf), ref, out, out_ref, out64, out_bound, corr64,
                   corr_bound, 16)
        expected = min(step + 1, 16)
        assert (from_device(d, buf)["positions"][:, 0] == expected).all()


def test_c3_scale_quant_only_step_on_a_sample(device):
    """B = 256 sequences x 32 value heads (8192 states) in one launch; the
    oracle checks every 32nd state."""
    states = 8192
    print(f"bf16 quant-only step states={states}", flush=True)
    buf = WG.window_buffers(states, 27, VK, compensated=False)
    inp = WG.bf16_inputs(states, 28)
    d = to_device(buf, device)
    di = to_device(inp, device)
    out = run_bf16_step(d, di, states, True, device)
    after = from_device(d, buf)
    heads = np.arange(0, states // 2, 16)                 # every 16th key/query head
    pairs = np.stack([2 * heads, 2 * heads + 1], axis=1).reshape(-1)  # its two value heads
    sub = {k: np.ascontiguousarray(v[pairs]) for k, v in buf.items()}
    sub_in = {k: np.ascontiguousarray(v[heads] if k in ("keys", "queries") else v[pairs])
              for k, v in inp.items()}
    ref = WG.copy_buffers(sub)
    out_ref, out64, out_bound, corr64, corr_bound = W.windowed_step_bf16(ref, **sub_in,
                                                                         quant_only=True)
    check_step(sub, {k: v[pairs] for k, v in after.items()}, ref, out[pairs], out_ref, out64,
               out_bound, corr64, corr_bound, 16)


# ------------------------------------------------------------ decode-pair chain

def test_bf16_decode_pair_chain_is_bit_exact(device):
    states = 64
    print("bf16 decode-pair chain", flush=True)
    buf = WG.window_buffers(states, 31, VK, positions=(list(range(18)) * 4)[:states])
    inp = WG.bf16_inputs(states, 32)
    d = to_device(buf, device)
    di = to_device(inp, device)
    quantized = torch.full((states, 128, 16), 99, dtype=torch.int8, device=device)
    dyn = torch.full((states, 8), -1.0, dtype=torch.float32, device=device)
    assert native().prepare_decode_pair_bf16_launch_v1(
        stream(), di["keys"].data_ptr(), di["queries"].data_ptr(), di["log_decay"].data_ptr(),
        d["smoothing"].data_ptr(), quantized.data_ptr(), dyn.data_ptr(), states) == 0
    q_ref, dyn_ref = W.prepare_decode_pair_bf16(inp["keys"], inp["queries"], inp["log_decay"],
                                                buf["smoothing"])
    torch.cuda.synchronize()
    assert np.array_equal(quantized.cpu().numpy(), q_ref)
    got_dyn = dyn.cpu().numpy()
    assert got_dyn[:, :4].tobytes() == dyn_ref[:, :4].tobytes()
    assert (got_dyn[:, 4:] == -1.0).all()
    # The int8 projection admits at most 128 states per launch, as the reference.
    projected = torch.zeros((states, 128, 16), dtype=torch.int32, device=device)
    scratch = torch.zeros(16, dtype=torch.int32, device=device)
    assert native().int8_cube_matmul_launch_v1(
        stream(), d["residual"].data_ptr(), quantized.data_ptr(), projected.data_ptr(), states,
        0, scratch.data_ptr(), scratch.data_ptr(), (states + 1) // 2) == 0
    p_ref = W.int8_matmul(buf["residual"], q_ref)
    torch.cuda.synchronize()
    assert np.array_equal(projected.cpu().numpy(), p_ref)
    out = torch.full((states, 128), SENTINEL16, dtype=torch.int16, device=device)
    assert native().finish_decode_pair_bf16_launch_v1(
        stream(), projected.data_ptr(), dyn.data_ptr(), d["scales"].data_ptr(),
        d["compensator_keys"].data_ptr(), d["compensator_values"].data_ptr(),
        d["record_decay"].data_ptr(), d["record_keys"].data_ptr(),
        d["record_corrections"].data_ptr(), d["positions"].data_ptr(),
        di["log_decay"].data_ptr(), di["beta"].data_ptr(), di["keys"].data_ptr(),
        di["queries"].data_ptr(), di["values"].data_ptr(), out.data_ptr(), states) == 0
    ref = WG.copy_buffers(buf)
    out_ref = W.finish_decode_pair_bf16(ref, p_ref, dyn_ref, **inp)
    torch.cuda.synchronize()
    live = buf["positions"][:, 0] < 16
    got = host(out, np.uint16)
    assert np.array_equal(got[live], out_ref[live])
    assert (got[~live] == SENTINEL16).all()
    after = from_device(d, buf)
    for name in buf:
        assert np.array_equal(after[name], ref[name]), name


def test_f16_decode_pair_chain_is_bit_exact(device):
    states = 48
    print("fp16 decode-pair chain", flush=True)
    buf = WG.window_buffers(states, 33, VK, positions=(list(range(18)) * 3)[:states])
    inp = WG.f16_inputs(states, 34)
    d = to_device(buf, device)
    di = to_device(inp, device)
    quantized = torch.zeros((states, 128, 16), dtype=torch.int8, device=device)
    dyn = torch.zeros((states, 8), dtype=torch.float32, device=device)
    assert native().prepare_decode_pair_launch_v1(
        stream(), di["reads"].data_ptr(), di["queries"].data_ptr(), di["decay"].data_ptr(),
        d["smoothing"].data_ptr(), quantized.data_ptr(), dyn.data_ptr(), states) == 0
    q_ref, dyn_ref = W.prepare_decode_pair(inp["reads"], inp["queries"], inp["decay"],
                                           buf["smoothing"])
    torch.cuda.synchronize()
    assert np.array_equal(quantized.cpu().numpy(), q_ref)
    assert dyn.cpu().numpy()[:, :4].tobytes() == dyn_ref[:, :4].tobytes()
    p_ref = W.int8_matmul(buf["residual"], q_ref)
    projected = dev(p_ref, device)
    out = torch.full((states, 128), float("nan"), dtype=torch.float32, device=device)
    assert native().finish_decode_pair_launch_v1(
        stream(), projected.data_ptr(), dyn.data_ptr(), d["scales"].data_ptr(),
        d["compensator_keys"].data_ptr(), d["compensator_values"].data_ptr(),
        d["record_decay"].data_ptr(), d["record_keys"].data_ptr(),
        d["record_corrections"].data_ptr(), d["positions"].data_ptr(),
        di["decay"].data_ptr(), di["write_keys"].data_ptr(), di["reads"].data_ptr(),
        di["queries"].data_ptr(), di["values"].data_ptr(), out.data_ptr(), states) == 0
    ref = WG.copy_buffers(buf)
    out_ref = W.finish_decode_pair(ref, p_ref, dyn_ref, **inp)
    torch.cuda.synchronize()
    live = buf["positions"][:, 0] < 16
    got = out.cpu().numpy()
    assert got[live].tobytes() == out_ref[live].tobytes()
    assert np.isnan(got[~live]).all()
    after = from_device(d, buf)
    for name in buf:
        assert np.array_equal(after[name], ref[name]), name


@pytest.mark.parametrize("transpose_a", [0, 1])
def test_int8_matmul_and_int8_vector_are_exact(device, transpose_a):
    states = 128
    print(f"int8 projection transpose_a={transpose_a}", flush=True)
    g = np.random.default_rng(40 + transpose_a)
    a = g.integers(-127, 128, (states, 128, 128), dtype=np.int8)
    b = g.integers(-127, 128, (states, 128, 16), dtype=np.int8)
    c = torch.zeros((states, 128, 16), dtype=torch.int32, device=device)
    scratch = torch.zeros(16, dtype=torch.int32, device=device)
    da, db = dev(a, device), dev(b, device)
    assert native().int8_cube_matmul_launch_v1(
        stream(), da.data_ptr(), db.data_ptr(), c.data_ptr(), states, transpose_a,
        scratch.data_ptr(), scratch.data_ptr(), states // 2) == 0
    torch.cuda.synchronize()
    assert np.array_equal(c.cpu().numpy(), W.int8_matmul(a, b, transpose_a))
    # prepare_int8_vector: column 0 of an fp16 [S][128][16] input.
    x = (g.standard_normal((states, 128, 16)) * 0.3).astype(np.float16).view(np.uint16)
    axis = (0.5 + g.random((states, 128))).astype(np.float32)
    q = torch.full((states, 128, 16), 7, dtype=torch.int8, device=device)
    dyn = torch.zeros((states, 8), dtype=torch.float32, device=device)
    dx, daxis = dev(x, device), dev(axis, device)  # held: a freed temporary's block is reused
    assert native().prepare_int8_vector_launch_v1(
        stream(), dx.data_ptr(), daxis.data_ptr(), q.data_ptr(), dyn.data_ptr(), states) == 0
    q_ref, dyn_ref = W.prepare_int8_vector(x, axis)
    torch.cuda.synchronize()
    assert np.array_equal(q.cpu().numpy(), q_ref)
    assert dyn.cpu().numpy()[:, 0].tobytes() == dyn_ref[:, 0].tobytes()


def test_int8_split_edges_round_by_the_float_half_add(device):
    """The hi/lo split and the int8 vector on inputs at the reference's rounding
    edges (.5 ties, 0.5 - 2^-25): codes derived by hand, and the oracle's."""
    x, s, hi, lo, lo_scale = WG.split_tie_state()
    states = 3
    print("int8 split rounding edges", flush=True)
    reads = np.tile(x.astype(np.float16).view(np.uint16), (states, 1))
    axis = np.tile(s, (states, 1))
    quantized = torch.full((states, 128, 16), 7, dtype=torch.int8, device=device)
    dyn = torch.zeros((states, 8), dtype=torch.float32, device=device)
    dr, ddecay = dev(reads, device), dev(np.ones(states, np.float32), device)
    daxis = dev(axis, device)
    assert native().prepare_decode_pair_launch_v1(
        stream(), dr.data_ptr(), dr.data_ptr(), ddecay.data_ptr(), daxis.data_ptr(),
        quantized.data_ptr(), dyn.data_ptr(), states) == 0
    q_ref, dyn_ref = W.prepare_decode_pair(reads, reads, np.ones(states, np.float32), axis)
    torch.cuda.synchronize()
    q, d = quantized.cpu().numpy(), dyn.cpu().numpy()
    assert np.array_equal(q, q_ref)
    assert d[:, :4].tobytes() == dyn_ref[:, :4].tobytes()
    for c in range(2):
        assert (q[:, :, 2 * c] == hi).all() and (q[:, :, 2 * c + 1] == lo).all()
        assert (d[:, c] == np.float32(0.125)).all() and (d[:, 2 + c] == lo_scale).all()
    operand = np.zeros((states, 128, 16), np.float16)
    operand[:, :, 0] = x.astype(np.float16)
    vq = torch.full((states, 128, 16), 7, dtype=torch.int8, device=device)
    vdyn = torch.zeros((states, 8), dtype=torch.float32, device=device)
    doperand = dev(operand.view(np.uint16), device)
    assert native().prepare_int8_vector_launch_v1(
        stream(), doperand.data_ptr(), daxis.data_ptr(), vq.data_ptr(), vdyn.data_ptr(),
        states) == 0
    vq_ref, vdyn_ref = W.prepare_int8_vector(operand.view(np.uint16), axis)
    torch.cuda.synchronize()
    got = vq.cpu().numpy()
    assert np.array_equal(got, vq_ref) and (got[:, :, 0] == hi).all()
    assert vdyn.cpu().numpy()[:, 0].tobytes() == vdyn_ref[:, 0].tobytes()
    assert (vdyn.cpu().numpy()[:, 0] == np.float32(0.125)).all()


@pytest.mark.parametrize("states", [64, 1024])
def test_fused_decode_runtime_step_equals_the_chain(device, states):
    """decode_runtime_step_v1 fuses prepare, projection and finish; its results
    equal the three-stage chain bit for bit, also above the reference's
    128-state Cube limit."""
    print(f"decode runtime step states={states}", flush=True)
    positions = (list(range(18)) * (states // 18 + 1))[:states]
    buf = WG.window_buffers(states, 35, VK, positions=positions)
    inp = WG.bf16_inputs(states, 36)
    d = to_device(buf, device)
    di = to_device(inp, device)
    lib = native()
    handle = lib.decode_runtime_create_v1(states)
    assert handle
    try:
        out = torch.full((states, 128), SENTINEL16, dtype=torch.int16, device=device)
        status = lib.decode_runtime_step_v1(
            handle, stream(), *window_ptrs(d), di["log_decay"].data_ptr(), di["beta"].data_ptr(),
            di["keys"].data_ptr(), di["queries"].data_ptr(), di["values"].data_ptr(),
            out.data_ptr(), states)
        assert status == 0
        torch.cuda.synchronize()
    finally:
        lib.decode_runtime_destroy_v1(handle)
    q_ref, dyn_ref = W.prepare_decode_pair_bf16(inp["keys"], inp["queries"], inp["log_decay"],
                                                buf["smoothing"])
    p_ref = W.int8_matmul(buf["residual"], q_ref)
    ref = WG.copy_buffers(buf)
    out_ref = W.finish_decode_pair_bf16(ref, p_ref, dyn_ref, **inp)
    live = buf["positions"][:, 0] < 16
    got = host(out, np.uint16)
    assert np.array_equal(got[live], out_ref[live])
    assert (got[~live] == SENTINEL16).all()
    after = from_device(d, buf)
    for name in buf:
        assert np.array_equal(after[name], ref[name]), name


def test_dense_fp32_step_is_bit_exact(device):
    states = 24
    print("dense fp32 step", flush=True)
    g = np.random.default_rng(50)
    state = (g.standard_normal((states, 128, 128)) * 0.05).astype(np.float32)
    inp = WG.f16_inputs(states, 51)
    ref_state = state.copy()
    out_ref = W.gdn_step_f32(ref_state, inp["decay"], inp["write_keys"], inp["reads"],
                             inp["queries"], inp["values"])
    ds = dev(state, device)
    di = to_device(inp, device)
    out = torch.zeros((states, 128), dtype=torch.float32, device=device)
    assert native().fp32_gdn_step_launch_v1(
        stream(), ds.data_ptr(), di["decay"].data_ptr(), di["write_keys"].data_ptr(),
        di["reads"].data_ptr(), di["queries"].data_ptr(), di["values"].data_ptr(),
        out.data_ptr(), states) == 0
    torch.cuda.synchronize()
    assert out.cpu().numpy().tobytes() == out_ref.tobytes()
    assert ds.cpu().numpy().tobytes() == ref_state.tobytes()
