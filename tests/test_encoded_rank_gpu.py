"""GPU parity of the device rank-4 chain over an encoded boundary
(finish_encoded_projection, commit_encoded_rank, encoded_requantize;
include/gdn_state_codec_window.h) against the oracle
(oracle/gdn_encoded_oracle.c), through the C-ABI: every output bit-exact,
buffers the reference leaves alone untouched, and the whole chain as the
reference's probe drives it (encoded_projection_probe.cpp:571-677) equal to
the oracle's chain at every stage."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import datagen
from gdn_state_codec import native
from oracle import window as W
from test_oracle_encoded import encoded_window, project, vector_inputs
from test_window_gpu import dev, host, stream

pytestmark = pytest.mark.gpu

OPERANDS = W.ENCODED_OPERANDS


def upload(enc, device):
    return {k: dev(v, device) for k, v in enc.items()}


def operand_ptrs(d):
    return [d[k].data_ptr() for k in OPERANDS]


@pytest.mark.parametrize("transpose", [0, 1])
@pytest.mark.parametrize("fitted", [0, 1, 4])
def test_finish_encoded_projection_is_bit_exact(device, transpose, fitted):
    states = 256
    print(f"finish_encoded_projection states={states} fitted={fitted} transpose={transpose}",
          flush=True)
    _, enc, residual = encoded_window(states, 111 + fitted, bases=4)
    inputs = vector_inputs(states, 112)
    projected, dyn = project(enc, residual, inputs, transpose)
    want = W.finish_encoded_projection(enc, projected, dyn, inputs, fitted, transpose)
    d = upload(enc, device)
    dp, dd, di = dev(projected, device), dev(dyn, device), dev(inputs, device)
    out = torch.full((states, 128, 16), 0x1357, dtype=torch.int16, device=device)
    assert native().finish_encoded_projection_launch_v1(
        stream(), dp.data_ptr(), dd.data_ptr(), di.data_ptr(), *operand_ptrs(d),
        d["new_left"].data_ptr(), d["new_right"].data_ptr(), out.data_ptr(), states, fitted,
        transpose) == 0
    torch.cuda.synchronize()
    assert np.array_equal(host(out, np.uint16).reshape(want.shape), want)
    for k, v in enc.items():
        assert np.array_equal(host(d[k], v.dtype).reshape(v.shape), v), k


def test_finish_of_zero_vectors_is_zero(device):
    states = 8
    print(f"finish_encoded_projection zero vectors states={states}", flush=True)
    _, enc, residual = encoded_window(states, 121)
    inputs = np.zeros((states, 128, 16), np.uint16)
    projected, dyn = project(enc, residual, inputs, 0)
    d = upload(enc, device)
    dp, dd, di = dev(projected, device), dev(dyn, device), dev(inputs, device)
    out = torch.full((states, 128, 16), 0x1357, dtype=torch.int16, device=device)
    assert native().finish_encoded_projection_launch_v1(
        stream(), dp.data_ptr(), dd.data_ptr(), di.data_ptr(), *operand_ptrs(d),
        d["new_left"].data_ptr(), d["new_right"].data_ptr(), out.data_ptr(), states, 0, 0) == 0
    torch.cuda.synchronize()
    assert not host(out, np.uint16).any()


@pytest.mark.parametrize("rank", [0, 2, 3])
def test_commit_encoded_rank_is_bit_exact(device, rank):
    states = 256
    print(f"commit_encoded_rank states={states} rank={rank}", flush=True)
    _, enc, residual = encoded_window(states, 131 + rank, bases=4)
    inputs = vector_inputs(states, 132)
    projected, dyn = project(enc, residual, inputs, 0)
    corrected = datagen.rng(133).standard_normal((states, 128, 16)).astype(np.float32)
    d = upload(enc, device)
    dp, dd, di = dev(projected, device), dev(dyn, device), dev(inputs, device)
    dc = dev(corrected, device)
    ref = {k: v.copy() for k, v in enc.items()}
    ref_corrected = corrected.copy()
    W.commit_encoded_rank(ref, projected, dyn, inputs, ref_corrected, rank)
    assert native().commit_encoded_rank_launch_v1(
        stream(), dp.data_ptr(), dd.data_ptr(), di.data_ptr(), *operand_ptrs(d),
        d["new_left"].data_ptr(), d["new_right"].data_ptr(), dc.data_ptr(), states, rank) == 0
    torch.cuda.synchronize()
    assert host(dc, np.float32).reshape(corrected.shape).tobytes() == ref_corrected.tobytes()
    for k, v in ref.items():
        assert np.array_equal(host(d[k], v.dtype).reshape(v.shape), v), k


REQUANT_OUT = ("next_residual", "next_smoothing", "next_scales", "next_left", "next_right",
               "workspace")


def run_requantize(d, residual_d, states, device):
    out = {"next_residual": torch.full((states, 128, 128), 0x5A, dtype=torch.int8, device=device),
           "next_smoothing": torch.full((states, 128), -3.0, device=device),
           "next_scales": torch.full((states, 128), -5.0, device=device),
           "next_left": torch.full((states, 128, 4), 0x1234, dtype=torch.int16, device=device),
           "next_right": torch.full((states, 128, 4), 0x4321, dtype=torch.int16, device=device),
           "workspace": torch.full((states, 128, 128), 7.0, device=device)}
    assert native().encoded_requantize_launch_v1(
        stream(), residual_d.data_ptr(), *operand_ptrs(d), d["new_left"].data_ptr(),
        d["new_right"].data_ptr(), *(out[k].data_ptr() for k in REQUANT_OUT), states) == 0
    torch.cuda.synchronize()
    return out


def assert_requantize(out, want):
    for k in REQUANT_OUT:
        got = host(out[k], want[k].dtype).reshape(want[k].shape)
        assert got.tobytes() == want[k].tobytes(), k


@pytest.mark.parametrize("states", [1, 96])
def test_encoded_requantize_is_bit_exact(device, states):
    print(f"encoded_requantize states={states}", flush=True)
    _, enc, residual = encoded_window(states, 141, planted=True, bases=4)
    want = W.encoded_requantize(enc, residual)
    d = upload(enc, device)
    out = run_requantize(d, dev(residual, device), states, device)
    assert_requantize(out, want)
    for k, v in enc.items():
        assert np.array_equal(host(d[k], v.dtype).reshape(v.shape), v), k


def test_rank_chain_matches_the_oracle_chain(device):
    """prepare_int8_vector -> int8_cube_matmul -> finish (forward, then
    transposed) x iterations, then prepare -> GEMM -> commit, per rank; then
    encoded_requantize.  Every intermediate and final buffer equals the
    oracle's."""
    states, iterations = 64, 3
    print(f"encoded rank chain states={states} iterations={iterations}", flush=True)
    _, enc, residual = encoded_window(states, 151, planted=True)
    g = datagen.rng(152)
    seeds = [W.f32_to_f16(np.concatenate(
        [g.standard_normal((states, 128, 1)), np.zeros((states, 128, 15))], axis=2))
        for _ in range(4)]
    lib = native()
    d = upload(enc, device)
    residual_d = dev(residual, device)
    quantized = torch.zeros((states, 128, 16), dtype=torch.int8, device=device)
    dyn = torch.zeros((states, 8), dtype=torch.float32, device=device)
    projected = torch.zeros((states, 128, 16), dtype=torch.int32, device=device)
    scratch = torch.zeros(16, dtype=torch.int32, device=device)
    corrected = torch.zeros((states, 128, 16), dtype=torch.float32, device=device)
    corrected_ref = np.zeros((states, 128, 16), np.float32)
    ref = {k: v.copy() for k, v in enc.items()}

    def gpu_project(vector, transpose):
        axis = d["smoothing"] if transpose else d["scales"]
        assert lib.prepare_int8_vector_launch_v1(stream(), vector.data_ptr(), axis.data_ptr(),
                                                 quantized.data_ptr(), dyn.data_ptr(),
                                                 states) == 0
        assert lib.int8_cube_matmul_launch_v1(
            stream(), residual_d.data_ptr(), quantized.data_ptr(), projected.data_ptr(), states,
            transpose, scratch.data_ptr(), scratch.data_ptr(), (states + 1) // 2) == 0

    def gpu_finish(vector, output, rank, transpose):
        gpu_project(vector, transpose)
        assert lib.finish_encoded_projection_launch_v1(
            stream(), projected.data_ptr(), dyn.data_ptr(), vector.data_ptr(), *operand_ptrs(d),
            d["new_left"].data_ptr(), d["new_right"].data_ptr(), output.data_ptr(), states,
            rank, transpose) == 0

    vector = torch.zeros((states, 128, 16), dtype=torch.int16, device=device)
    output = torch.zeros_like(vector)
    for rank in range(4):
        vector.copy_(dev(seeds[rank], device))
        ref_vector = seeds[rank].copy()
        for _ in range(iterations):
            gpu_finish(vector, output, rank, 0)
            gpu_finish(output, vector, rank, 1)
            p, q = project(ref, residual, ref_vector, 0)
            ref_output = W.finish_encoded_projection(ref, p, q, ref_vector, rank, 0)
            p, q = project(ref, residual, ref_output, 1)
            ref_vector = W.finish_encoded_projection(ref, p, q, ref_output, rank, 1)
        torch.cuda.synchronize()
        assert np.array_equal(host(vector, np.uint16).reshape(ref_vector.shape), ref_vector), rank
        gpu_project(vector, 0)
        assert lib.commit_encoded_rank_launch_v1(
            stream(), projected.data_ptr(), dyn.data_ptr(), vector.data_ptr(), *operand_ptrs(d),
            d["new_left"].data_ptr(), d["new_right"].data_ptr(), corrected.data_ptr(), states,
            rank) == 0
        p, q = project(ref, residual, ref_vector, 0)
        W.commit_encoded_rank(ref, p, q, ref_vector, corrected_ref, rank)
    torch.cuda.synchronize()
    for k in ("new_left", "new_right"):
        assert np.array_equal(host(d[k], np.uint16).reshape(ref[k].shape), ref[k]), k
    assert host(corrected, np.float32).reshape(corrected_ref.shape).tobytes() == \
        corrected_ref.tobytes()
    out = run_requantize(d, residual_d, states, device)
    assert_requantize(out, W.encoded_requantize(ref, residual))


@pytest.mark.parametrize("transpose", [0, 1])
def test_batched_int8_matmul_matches_the_cube_entry_point(device, transpose):
    """int8_matmul_launch_v4 over 300 states in one launch equals the exact
    integer product and int8_cube_matmul_launch_v1 called on chunks of at most
    128 states (the reference's admission), int32 for int32."""
    states = 300
    print(f"int8_matmul_launch_v4 states={states} transpose={transpose}", flush=True)
    g = datagen.rng(160 + transpose)
    a = g.integers(-127, 128, (states, 128, 128), dtype=np.int8)
    b = g.integers(-127, 128, (states, 128, 16), dtype=np.int8)
    lhs = a.astype(np.int64)
    if transpose:
        lhs = lhs.transpose(0, 2, 1)
    want = np.matmul(lhs, b.astype(np.int64)).astype(np.int32)
    lib = native()
    da, db = dev(a, device), dev(b, device)
    batched = torch.full((states, 128, 16), 0x1234, dtype=torch.int32, device=device)
    assert lib.int8_matmul_launch_v4(stream(), da.data_ptr(), db.data_ptr(),
                                     batched.data_ptr(), states, transpose) == 0
    chunked = torch.full((states, 128, 16), 0x4321, dtype=torch.int32, device=device)
    scratch = torch.zeros(16, dtype=torch.int32, device=device)
    for lo in range(0, states, 128):
        n = min(128, states - lo)
        assert lib.int8_cube_matmul_launch_v1(
            stream(), da[lo].data_ptr(), db[lo].data_ptr(), chunked[lo].data_ptr(), n,
            transpose, scratch.data_ptr(), scratch.data_ptr(), (n + 1) // 2) == 0
    torch.cuda.synchronize()
    assert np.array_equal(host(batched, np.int32).reshape(want.shape), want)
    assert torch.equal(batched, chunked)
