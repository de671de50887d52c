"""Deterministic synthetic head tiles shared by the tests and fixture generator.

Distributions follow the benchmark configurations: N(0, 0.05^2) entries with
0.1% outliers at +-2.0 (config 1 style), Student-t(3) * 0.05 (pool config), and
special tiles that exercise the codec's edge cases.
"""

from __future__ import annotations

import numpy as np

DIM = 128


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def c1_heads(heads: int, seed: int) -> np.ndarray:
    """N(0, 0.05^2) fp32 tiles with 0.1% of entries replaced by +-2.0."""
    g = rng(seed)
    x = (g.standard_normal((heads, DIM, DIM), dtype=np.float32) * np.float32(0.05))
    mask = g.random((heads, DIM, DIM)) < 0.001
    signs = np.where(g.random(int(mask.sum())) < 0.5, -2.0, 2.0).astype(np.float32)
    x[mask] = signs
    return np.ascontiguousarray(x, dtype=np.float32)


def student_t_heads(heads: int, seed: int, zero_fraction: float = 0.0) -> np.ndarray:
    g = rng(seed)
    x = (g.standard_t(3.0, size=(heads, DIM, DIM)) * 0.05).astype(np.float32)
    if zero_fraction > 0:
        zero = g.random(heads) < zero_fraction
        x[zero] = 0.0
    return np.ascontiguousarray(x)


def wide_range_head(seed: int) -> np.ndarray:
    """Rows mixing magnitudes 2^-45..2^12 so that double sums of |r| round and
    their value depends on summation order."""
    g = rng(seed)
    x = (g.standard_normal((DIM, DIM)) * 0.05).astype(np.float32)
    exps = g.integers(-45, 12, size=(DIM, DIM))
    pick = g.random((DIM, DIM)) < 0.5
    x[pick] = (np.sign(x[pick]) * np.ldexp(1.0 + g.random(int(pick.sum())), exps[pick])).astype(np.float32)
    return np.ascontiguousarray(x)


def tiny_head(seed: int) -> np.ndarray:
    """Subnormal and near-underflow entries mixed with ordinary ones."""
    g = rng(seed)
    x = (g.standard_normal((DIM, DIM)) * 1e-3).astype(np.float32)
    sub = g.random((DIM, DIM)) < 0.3
    x[sub] = (g.standard_normal(int(sub.sum())) * 1e-40).astype(np.float32)
    # A whole column and a whole row of subnormals.
    x[:, 7] = (g.standard_normal(DIM) * 1e-42).astype(np.float32)
    x[9, :] = (g.standard_normal(DIM) * 1e-41).astype(np.float32)
    return np.ascontiguousarray(x)


def tiny_value_head(seed: int, value_axis: int) -> np.ndarray:
    """Ordinary entries except two values (lines along `value_axis`: 0 for the
    [value][key] layout, 1 for [key][value]) whose every entry has magnitude in
    [2^-100, 2^-98): their scales max |r / s| fall below 2^-90 while every
    non-zero |r| stays at or above 2^-100, so the encoder's fast division by s
    applies and its fast division by the scale does not."""
    g = rng(seed)
    x = (g.standard_normal((DIM, DIM)) * 0.05).astype(np.float32)
    for value in (11, 90):
        line = np.ldexp(1.0 + g.random(DIM), g.integers(-100, -99, size=DIM, endpoint=True))
        line = (line * np.where(g.random(DIM) < 0.5, -1.0, 1.0)).astype(np.float32)
        if value_axis == 0:
            x[value, :] = line
        else:
            x[:, value] = line
    return np.ascontiguousarray(x)


def huge_head(seed: int) -> np.ndarray:
    g = rng(seed)
    return np.ascontiguousarray((g.standard_normal((DIM, DIM)) * 1e30).astype(np.float32))


def zero_rows_cols_head(seed: int) -> np.ndarray:
    g = rng(seed)
    x = (g.standard_normal((DIM, DIM)) * 0.05).astype(np.float32)
    x[3, :] = 0.0
    x[:, 5] = 0.0
    x[40:44, :] = 0.0
    x[:, 100] = -0.0
    x[77, 77] = 0.0
    return np.ascontiguousarray(x)


def constant_head(value: float) -> np.ndarray:
    x = np.full((DIM, DIM), value, np.float32)
    x[::2, 1::2] = -value
    return x
