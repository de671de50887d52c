"""GPU check of the chunked projection's two-part bf16 split (split2_pair in
csrc/bf16_operands.h) against its definition restated in numpy:
hi = RN_bf16(clamp(w, +-0x1.fep127)) and lo = RN_bf16(w - hi), bit for bit,
over ordinary values, the bottom of the range its error bound covers (2^-110)
and the top of fp32's range, where a split without the clamp gives inf and
-inf.  Every finite w must give finite parts with |w - hi - lo| <= 2^-16 |w|."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import datagen
import oracle
from gdn_state_codec import _native

LARGEST_BF16 = np.float32(np.uint32(0x7F7F0000).view(np.float32))


def _probe():
    lib = ctypes.CDLL(str(_native.library_dir() / "libgdn_state_codec_hbm_probe.so"))
    lib.gdn_split_probe.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_uint32]
    lib.gdn_split_probe.restype = ctypes.c_int32
    return lib


def _inputs():
    g = datagen.rng(811)
    ordinary = (g.standard_normal(4096) * 10.0 ** g.uniform(-25, 30, 4096)).astype(np.float32)
    # Keep every part and remainder a normal fp32 / bf16 number.
    ordinary[np.abs(ordinary) < 2.0 ** -100] = np.float32(1.5)
    bottom = (np.ldexp(1.0 + g.random(512), -110 + g.integers(0, 8, 512))
              * np.where(g.random(512) < 0.5, -1, 1)).astype(np.float32)
    top_bits = np.concatenate([
        np.array([0x7F7F0000, 0x7F7F0001, 0x7F7F7FFF, 0x7F7F8000, 0x7F7F8001, 0x7F7FFFFF,
                  0x7F7EFFFF, 0x7F000000], np.uint32),
        g.integers(0x7F7F0000, 0x7F800000, 504, dtype=np.uint32)])
    top = top_bits.view(np.float32)
    top = np.concatenate([top, -top])
    return np.concatenate([ordinary, bottom, top, np.float32([0.0, -0.0])]).astype(np.float32)


def _split_numpy(w):
    clamped = np.clip(w, -LARGEST_BF16, LARGEST_BF16).astype(np.float32)
    hi = oracle.f32_to_bf16(clamped)
    rest = (w - oracle.bf16_to_f32(hi)).astype(np.float32)
    return hi, oracle.f32_to_bf16(rest)


@pytest.mark.gpu
def test_split_matches_its_definition_and_stays_finite(device):
    print("bf16 split probe", flush=True)
    w = _inputs()
    assert w.size % 2 == 0
    pairs = w.size // 2
    dw = torch.from_numpy(w).to(device)
    hi = torch.zeros(pairs, dtype=torch.int32, device=device)
    lo = torch.zeros(pairs, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    assert _probe().gdn_split_probe(stream, dw.data_ptr(), hi.data_ptr(), lo.data_ptr(),
                                    pairs) == 0
    torch.cuda.synchronize()
    got_hi = hi.cpu().numpy().view(np.uint16)  # low element first: [w0, w1, ...]
    got_lo = lo.cpu().numpy().view(np.uint16)
    want_hi, want_lo = _split_numpy(w)
    assert np.array_equal(got_hi, want_hi)
    assert np.array_equal(got_lo, want_lo)
    h = oracle.bf16_to_f32(got_hi).astype(np.float64)
    l = oracle.bf16_to_f32(got_lo).astype(np.float64)
    assert np.isfinite(h).all() and np.isfinite(l).all()
    covered = (np.abs(w) >= 2.0 ** -110) | (w == 0)
    error = np.abs(w.astype(np.float64) - h - l)
    assert (error[covered] <= 2.0 ** -16 * np.abs(w[covered].astype(np.float64))).all()


def test_unclamped_split_would_overflow_at_the_top_of_the_range():
    """Negative control on the CPU: the same restatement without the clamp
    turns the largest finite floats into an infinite part."""
    w = np.array([np.finfo(np.float32).max, -np.finfo(np.float32).max], np.float32)
    hi = oracle.f32_to_bf16(w)
    assert np.isinf(oracle.bf16_to_f32(hi)).all()
    clamped_hi, clamped_lo = _split_numpy(w)
    assert np.isfinite(oracle.bf16_to_f32(clamped_hi)).all()
    assert np.isfinite(oracle.bf16_to_f32(clamped_lo)).all()
