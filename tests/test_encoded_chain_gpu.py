"""The device rank-4 chain in one launch (encoded_rank_chain_launch_v4) against
the same chain run stage by stage through the reference's entry points
(prepare_int8_vector -> int8 product -> finish_encoded_projection, forward then
transposed, per iteration; then prepare -> product -> commit_encoded_rank, per
rank; as host/gdn_state_codec_encoded_projection_probe.cpp:611-636 drives them).
new_left, new_right and every rank's committed vector must agree bit for bit.
The stage-by-stage chain is itself pinned to the oracle's chain stage by stage
(tests/test_encoded_rank_gpu.py::test_rank_chain_matches_the_oracle_chain)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import datagen
from gdn_state_codec import native
from oracle import window as W
from test_oracle_encoded import encoded_window
from test_window_gpu import dev, host, stream

OPERANDS = W.ENCODED_OPERANDS


def seeds_for(states, seed):
    """fp16 seed vectors [S][4][128] (one per rank)."""
    return W.f32_to_f16(datagen.rng(seed).standard_normal((states, 4, 128)))


def stage_by_stage(d, residual_d, seeds, states, iterations, device):
    """The chain through the v1 entry points; returns new_left, new_right
    ([S][4][128] fp16 bits) and each rank's corrected column 0 ([S][4][128])."""
    lib = native()
    quantized = torch.zeros((states, 128, 16), dtype=torch.int8, device=device)
    dyn = torch.zeros((states, 8), dtype=torch.float32, device=device)
    projected = torch.zeros((states, 128, 16), dtype=torch.int32, device=device)
    scratch = torch.zeros(16, dtype=torch.int32, device=device)
    corrected = torch.zeros((states, 128, 16), dtype=torch.float32, device=device)
    vector = torch.zeros((states, 128, 16), dtype=torch.int16, device=device)
    output = torch.zeros_like(vector)
    committed = np.zeros((states, 4, 128), np.float32)

    def product(vec, transpose):
        axis = d["smoothing"] if transpose else d["scales"]
        assert lib.prepare_int8_vector_launch_v1(stream(), vec.data_ptr(), axis.data_ptr(),
                                                 quantized.data_ptr(), dyn.data_ptr(),
                                                 states) == 0
        if states <= 128:
            assert lib.int8_cube_matmul_launch_v1(
                stream(), residual_d.data_ptr(), quantized.data_ptr(), projected.data_ptr(),
                states, transpose, scratch.data_ptr(), scratch.data_ptr(),
                (states + 1) // 2) == 0
        else:
            assert lib.int8_matmul_launch_v4(stream(), residual_d.data_ptr(),
                                             quantized.data_ptr(), projected.data_ptr(),
                                             states, transpose) == 0

    ops = [d[k].data_ptr() for k in OPERANDS]
    for rank in range(4):
        column = np.zeros((states, 128, 16), np.uint16)
        column[:, :, 0] = seeds[:, rank]
        vector.copy_(dev(column, device))
        for _ in range(iterations):
            for src, dst, transpose in ((vector, output, 0), (output, vector, 1)):
                product(src, transpose)
                assert lib.finish_encoded_projection_launch_v1(
                    stream(), projected.data_ptr(), dyn.data_ptr(), src.data_ptr(), *ops,
                    d["new_left"].data_ptr(), d["new_right"].data_ptr(), dst.data_ptr(),
                    states, rank, transpose) == 0
        product(vector, 0)
        assert lib.commit_encoded_rank_launch_v1(
            stream(), projected.data_ptr(), dyn.data_ptr(), vector.data_ptr(), *ops,
            d["new_left"].data_ptr(), d["new_right"].data_ptr(), corrected.data_ptr(),
            states, rank) == 0
        committed[:, rank] = host(corrected, np.float32).reshape(states, 128, 16)[:, :, 0]
    torch.cuda.synchronize()
    return (host(d["new_left"], np.uint16).reshape(states, 4, 128),
            host(d["new_right"], np.uint16).reshape(states, 4, 128), committed)


def fused(d, residual_d, seeds, states, iterations, device):
    new_left = torch.full((states, 4, 128), 0x1357, dtype=torch.int16, device=device)
    new_right = torch.full((states, 4, 128), 0x2468, dtype=torch.int16, device=device)
    corrected = torch.full((states, 4, 128), -7.0, dtype=torch.float32, device=device)
    seeds_d = dev(seeds, device)
    assert native().encoded_rank_chain_launch_v4(
        stream(), residual_d.data_ptr(), *[d[k].data_ptr() for k in OPERANDS],
        seeds_d.data_ptr(), new_left.data_ptr(), new_right.data_ptr(), corrected.data_ptr(),
        states, iterations) == 0
    torch.cuda.synchronize()
    return (host(new_left, np.uint16), host(new_right, np.uint16),
            host(corrected, np.float32))


@pytest.mark.gpu
@pytest.mark.parametrize("states,iterations,planted", [(64, 3, True), (300, 8, False),
                                                       (5, 1, True)])
def test_fused_chain_equals_the_stage_by_stage_chain(device, states, iterations, planted):
    print(f"encoded rank chain fused states={states} iterations={iterations}", flush=True)
    _, enc, residual = encoded_window(states, 171 + states, planted=planted)
    seeds = seeds_for(states, 172 + states)
    d = {k: dev(v, device) for k, v in enc.items()}  # new_left / new_right start at zero
    residual_d = dev(residual, device)
    got = fused(d, residual_d, seeds, states, iterations, device)
    want = stage_by_stage(d, residual_d, seeds, states, iterations, device)
    for name, g, w in zip(("new_left", "new_right", "corrected"), got, want):
        assert g.tobytes() == w.tobytes(), name
    # Operands the chain only reads are untouched.
    for k in OPERANDS:
        assert np.array_equal(host(d[k], enc[k].dtype).reshape(enc[k].shape), enc[k]), k


def test_fused_chain_admission():
    """Status 1 before any device work: null pointers, no states or more than
    16384, iterations outside 1..64, a misaligned pointer."""
    from gdn_state_codec import _native

    lib = _native.NativeLibrary()
    p = ctypes.c_void_p(16)
    args = [p] * 12
    for states, iterations in ((0, 1), (16385, 1), (1, 0), (1, 65)):
        assert lib.encoded_rank_chain_launch_v4(None, *args, states, iterations) == 1
    for i in range(12):
        bad = list(args)
        bad[i] = None
        assert lib.encoded_rank_chain_launch_v4(None, *bad, 1, 1) == 1
    bad = list(args)
    bad[3] = ctypes.c_void_p(24)
    assert lib.encoded_rank_chain_launch_v4(None, *bad, 1, 1) == 1
