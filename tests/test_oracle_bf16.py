"""Pin of the oracle's fp32 -> bf16 narrowing (``oracle.f32_to_bf16`` in numpy
and ``gdn_oracle_f32_to_bf16`` in C), the formula of the reference's
FloatToBFloat16 (kernel/gdn_state_codec_windowed_gdn_step.cpp:26-32:
``(bits + 0x7FFF + lsb) >> 16``).  It feeds the bf16 pool decode and the bf16
window-step outputs, which the GPU reproduces bit for bit, so pinning it pins
them.

The independent check is torch's CPU ``Tensor.to(torch.bfloat16)``
(round-to-nearest-even) on 2^24 random bit patterns plus every exponent with
tie and near-tie significands, subnormals, the overflow boundary, zeros and
infinities.  NaN is where the formula and torch part: torch returns the
canonical quiet NaN 0x7FC0 (sign kept), while the formula keeps the top 16 bits
of a NaN whose payload reaches them, turns a NaN whose payload sits in the low
16 bits into an infinity (0x7F800001 -> 0x7F80) and wraps 0xFFFFFFFF to +0.
That mapping is asserted as such below, not compared with torch."""

from __future__ import annotations

import numpy as np
import torch

import oracle


def torch_bf16_bits(values: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(values, np.float32)).to(torch.bfloat16)
    return t.view(torch.int16).numpy().view(np.uint16)


def check(bits: np.ndarray) -> None:
    bits = np.ascontiguousarray(bits, np.uint32)
    keep = ((bits & 0x7F800000) != 0x7F800000) | ((bits & 0x007FFFFF) == 0)
    values = bits[keep].view(np.float32)
    want = torch_bf16_bits(values)
    assert np.array_equal(oracle.f32_to_bf16(values), want)
    assert np.array_equal(oracle.c_f32_to_bf16(values), want)


def test_random_bit_patterns():
    rng = np.random.default_rng(20261202)
    check(rng.integers(0, 2 ** 32, size=1 << 24, dtype=np.uint64).astype(np.uint32))


def test_ties_near_ties_and_every_exponent():
    exponents = np.arange(256, dtype=np.uint32) << 23
    uppers = np.array([0x0000, 0x0001, 0x0002, 0x007F, 0x0080, 0x00FF, 0x3FFE, 0x3FFF,
                       0x4000, 0x7FFE, 0x7FFF], np.uint32) << 16
    lows = np.array([0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    grid = (exponents[:, None, None] | uppers[None, :, None] | lows[None, None, :]).ravel()
    grid = grid & 0x7FFFFFFF
    check(np.concatenate([grid, grid | 0x80000000]))


def test_subnormals_overflow_zeros_and_infinities():
    special = np.array([
        0x00000000, 0x80000000,              # +-0
        0x00000001, 0x00008000, 0x00018000,  # subnormal ties (to even: 0, 0x0002)
        0x007FFFFF, 0x00800000,              # largest subnormal, smallest normal
        0x7F7F0000, 0x7F7F7FFF, 0x7F7F8000,  # max bf16, below / at the overflow tie
        0x7F7FFFFF, 0xFF7FFFFF,              # max float rounds to +-inf
        0x7F800000, 0xFF800000,              # +-inf
    ], np.uint32)
    check(special)
    got = oracle.f32_to_bf16(special.view(np.float32))
    assert got[[2, 3, 4]].tolist() == [0x0000, 0x0000, 0x0002]
    assert got[9] == 0x7F80 and got[10] == 0x7F80 and got[11] == 0xFF80


def test_nan_mapping_of_the_reference_formula():
    nans = np.array([0x7FC00000, 0xFFC00000, 0x7FA00001, 0x7F800001, 0x7F807FFF,
                     0x7F808001, 0xFFFFFFFF], np.uint32).view(np.float32)
    got = oracle.f32_to_bf16(nans)
    assert np.array_equal(got, oracle.c_f32_to_bf16(nans))
    # The formula's own bits: quiet NaNs keep their top half, a low payload
    # becomes an infinity or rounds up into the NaN range, and all-ones wraps.
    assert got.tolist() == [0x7FC0, 0xFFC0, 0x7FA0, 0x7F80, 0x7F80, 0x7F81, 0x0000]
    # torch canonicalizes instead; both stay NaN where the top half is a NaN.
    assert np.isnan(oracle.bf16_to_f32(got[:3])).all()


def test_plausible_mistakes_fail_the_check():
    """Truncation and round-half-up disagree with torch on the tie grid, so the
    checks above would catch either in the oracle."""
    exponents = np.arange(1, 255, dtype=np.uint32) << 23
    bits = (exponents[:, None] | np.array([0x8000, 0x18000, 0x7FFF, 0x8001], np.uint32)).ravel()
    want = torch_bf16_bits(bits.view(np.float32))
    assert not np.array_equal((bits >> 16).astype(np.uint16), want)
    assert not np.array_equal(((bits + 0x8000) >> 16).astype(np.uint16), want)
