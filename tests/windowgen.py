"""Synthetic windowed-decode buffers in the device formats of the windowed step
entry points (numpy; the GPU tests copy them to the device).

Magnitudes follow the reference's own device probe
(native/ascendc/gdn_state_codec/host/gdn_state_codec_windowed_gdn_runtime_probe.cpp:
186-236): decays near 0.93-0.99, record keys ~0.03, corrections ~0.08, small
fp16 compensators, while boundaries come from encoding config-1 style heads and
keys/queries are L2-normalised like the model's.
"""

from __future__ import annotations

import numpy as np

import datagen
import oracle
from oracle import window as W

DIM = 128


def _f16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def _bf16(x: np.ndarray) -> np.ndarray:
    return oracle.f32_to_bf16(np.asarray(x, np.float32))


def window_buffers(states: int, seed: int, layout: int, positions=None,
                   compensated: bool = True) -> dict:
    """Boundary (codes in `layout`, smoothing, scales), rank-4 fp16
    compensators, 16 fp16 records and [S][8] positions.  `positions` is an int
    or a per-state sequence (values >= 16 mark a full window)."""
    g = datagen.rng(seed)
    dense = datagen.c1_heads(states, seed + 1)
    codes, s, sc = oracle.encode_heads(dense, layout, threads=8)
    buf = {"residual": codes, "smoothing": s, "scales": sc}
    if compensated:
        buf["compensator_keys"] = _f16(g.standard_normal((states, DIM, 4)) * 0.01)
        buf["compensator_values"] = _f16(g.standard_normal((states, DIM, 4)) * 0.01)
    else:
        buf["compensator_keys"] = np.zeros((states, DIM, 4), np.uint16)
        buf["compensator_values"] = np.zeros((states, DIM, 4), np.uint16)
    buf["record_decay"] = (0.93 + 0.06 * g.random((states, 16))).astype(np.float32)
    buf["record_keys"] = _f16(g.standard_normal((states, 16, DIM)) * 0.03)
    buf["record_corrections"] = _f16(g.standard_normal((states, 16, DIM)) * 0.08)
    if positions is None:
        positions = g.integers(0, 16, states)
    pos = np.broadcast_to(np.asarray(positions, np.uint32), (states,))
    buf["positions"] = np.zeros((states, 8), np.uint32)
    buf["positions"][:, 0] = pos
    buf["positions"][:, 1:] = 0xA5A5A5A5  # untouched padding words
    return {k: np.ascontiguousarray(v) for k, v in buf.items()}


def copy_buffers(buf: dict) -> dict:
    return {k: (None if v is None else v.copy()) for k, v in buf.items()}


def bf16_inputs(states: int, seed: int) -> dict:
    """Model-facing inputs of the bf16 steps: log decay fp32 [S], beta bf16 [S],
    keys / queries bf16 [S/2][128] (L2-normalised), values bf16 [S][128]."""
    g = datagen.rng(seed)
    heads = states // 2
    k = g.standard_normal((heads, DIM))
    q = g.standard_normal((heads, DIM))
    k /= np.linalg.norm(k, axis=1, keepdims=True)
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    return {
        "log_decay": np.log(0.9 + 0.09 * g.random(states)).astype(np.float32),
        "beta": _bf16(0.2 + 0.6 * g.random(states)),
        "keys": _bf16(k),
        "queries": _bf16(q),
        "values": _bf16(g.standard_normal((states, DIM)) * 0.5),
    }


def f16_inputs(states: int, seed: int) -> dict:
    """Inputs of the fp16 v1 step: linear decay fp32 [S], write_keys / reads /
    queries / values fp16 [S][128]."""
    g = datagen.rng(seed)
    decay = (0.9 + 0.09 * g.random(states)).astype(np.float32)
    k = g.standard_normal((states, DIM))
    k /= np.linalg.norm(k, axis=1, keepdims=True)
    q = g.standard_normal((states, DIM))
    q /= np.linalg.norm(q, axis=1, keepdims=True)
    beta = 0.2 + 0.6 * g.random((states, 1))
    return {
        "decay": decay,
        "write_keys": _f16(beta * k),
        "reads": _f16(decay[:, None] * k),
        "queries": _f16(q),
        "values": _f16(g.standard_normal((states, DIM)) * 0.5),
    }


def kv_boundary(buf: dict, state: int, layout: int):
    """The [key][value] codes of one state of a window buffer."""
    c = buf["residual"][state]
    return np.ascontiguousarray(c.T if layout == oracle.LAYOUT_VALUE_KEY else c)


def capsule_at(buf: dict, state: int, layout: int, rank: int = 4) -> W.CapsuleWindow:
    """A capsule window holding exactly the device buffer's state `state`:
    its boundary, widened fp16 compensators and records, and position."""
    cap = W.CapsuleWindow.__new__(W.CapsuleWindow)
    cap.keys = cap.values = DIM
    cap.rank, cap.window = rank, 16
    cap.codes = kv_boundary(buf, state, layout).astype(np.int8)
    cap.smoothing = buf["smoothing"][state].copy()
    cap.scales = buf["scales"][state].copy()
    if rank:
        cap.ck = np.ascontiguousarray(W.f16_to_f32(buf["compensator_keys"][state]))
        cap.cv = np.ascontiguousarray(W.f16_to_f32(buf["compensator_values"][state]))
    else:
        cap.ck = np.zeros((DIM, 1), np.float32)
        cap.cv = np.zeros((DIM, 1), np.float32)
    cap.record_decay = np.repeat(buf["record_decay"][state][:, None], DIM, axis=1).astype(np.float32)
    cap.record_keys = np.ascontiguousarray(W.f16_to_f32(buf["record_keys"][state]))
    cap.record_corrections = np.ascontiguousarray(W.f16_to_f32(buf["record_corrections"][state]))
    import ctypes
    cap.position = ctypes.c_uint32(int(buf["positions"][state, 0]))
    return cap


def split_tie_state():
    """One state whose hi-level divisions land on the reference's rounding
    edges (encoded_projection.cpp:289-296, :326-334: add +-0.5 in float, clamp
    to +-127, truncate).  The largest |x * s| is 15.875 = 127 / 8, so the hi
    scale is exactly 1/8 and x * s / scale is exact:
      row 1:  0.3125            ->  2.5          -> 3   (ties-to-even: 2)
      row 2: -0.3125            -> -2.5          -> -3  (ties-to-even: -2)
      row 3:  2^-4 * (1-2^-24)  ->  0.5 - 2^-25  -> 1   (exact rounding: 0;
              the float add 0.5 - 2^-25 + 0.5 ties to even at 1.0)
      row 4:  1.0               ->  8.0          -> 8
      row 0: 15.875             ->  127          -> 127 (127.5 clamps)
    and every other row is 0 (0 + 0.5 truncates to 0)."""
    x = np.zeros(128, np.float32)
    x[:5] = [15.875, 0.3125, -0.3125, 2.0 ** -4, 1.0]
    s = np.ones(128, np.float32)
    s[3] = np.float32(1.0) - np.float32(2.0 ** -24)
    hi = np.zeros(128, np.int8)
    hi[:5] = [127, 3, -3, 1, 8]
    # The residuals x*s - hi/8 are 0 except rows 1-3; their largest magnitude
    # is 2^-4 + 2^-28 (row 3), which sets the lo scale; rows 1 and 3 map to
    # -127 and row 2 to 127 (126.9999995 +- 0.5, clamped).
    lo = np.zeros(128, np.int8)
    lo[1:4] = [-127, 127, -127]
    lo_scale = np.float32(np.float32(2.0 ** -4 + 2.0 ** -28) / np.float32(127.0))
    return x, s, hi, lo, lo_scale
