"""A second transcription of the reference's rank-4 window-boundary refit
(native/ascendc/gdn_state_codec/kernel/gdn_state_codec_window_boundary.cpp:
17-37 SquareRoot / Normalize, :100-111 BuildSuffix, :113-221 ApplyRight /
ApplyTranspose, :223-251 ResidualCell, :253-366 ProcessState), written from
the reference's source in numpy float32, independently of the C oracle
(oracle/gdn_boundary_oracle.c) it is compared with.

Every statement is an IEEE single-precision operation in the reference's
order: numpy float32 arithmetic rounds each product, quotient and sum to
nearest even, and each sequential sum of the reference stays sequential here
(a loop over the summed index, vectorized only across the independent one).
Test infrastructure only.
"""

from __future__ import annotations

import numpy as np

F = np.float32
DIM, RANK, WINDOW = 128, 4, 16


def square_root(value: np.float32) -> np.float32:
    """:17-23: 20 Newton steps from max(value, 1)."""
    estimate = value if value > F(1.0) else F(1.0)
    for _ in range(20):
        estimate = F(0.5) * (estimate + value / estimate)
    return F(estimate)


def sequential_sum(terms: np.ndarray) -> np.ndarray:
    """Sum over the last axis in index order, one fp32 rounding per add."""
    acc = np.zeros(terms.shape[:-1], F)
    for i in range(terms.shape[-1]):
        acc = acc + terms[..., i]
    return acc


def normalize(vector: np.ndarray):
    """:25-37; returns (vector, ok)."""
    squared = sequential_sum((vector * vector)[None])[0]
    if squared <= F(1.0e-20):
        return vector, False
    inverse = F(1.0) / square_root(squared)
    return (vector * inverse).astype(F), True


def start_vector(rank: int) -> np.ndarray:
    """:268-271: ((rank + 1) * (column + 3)) % 17 - 8."""
    column = np.arange(DIM)
    return (((rank + 1) * (column + 3)) % 17 - 8).astype(F)


class State:
    """One state's window in the reference's orientation: code[row][column]
    (rows are keys, columns values), fp16 operands widened to fp32."""

    def __init__(self, buf: dict, s: int):
        h = lambda bits: np.asarray(bits, np.uint16).view(np.float16).astype(F)  # noqa: E731
        self.code = buf["residual"][s].T.astype(F)                 # [row][column]
        self.smoothing = buf["smoothing"][s].astype(F)              # by row
        self.scales = buf["scales"][s].astype(F)                    # by column
        self.ck = h(buf["compensator_keys"][s])                     # [row][rank]
        self.cv = h(buf["compensator_values"][s])                   # [column][rank]
        self.rk = h(buf["record_keys"][s])                          # [record][row]
        self.rc = h(buf["record_corrections"][s])                   # [record][column]
        suffix, record_suffix = F(1.0), np.empty(WINDOW, F)         # BuildSuffix, :100-111
        for record in range(WINDOW - 1, -1, -1):
            record_suffix[record] = suffix
            suffix = F(suffix * F(buf["record_decay"][s][record]))
        self.record_suffix, self.bs = record_suffix, suffix
        # code / 127 * s[row] * scale[column], left to right, per cell.
        self.boundary = (self.code / F(127.0)) * self.smoothing[:, None] * self.scales[None, :]

    def apply_right(self, vector, nk, nv, fitted):
        """:113-166: output[row] = R vector, summed over columns in order."""
        old = sequential_sum(self.cv.T * vector[None, :])                 # [rank]
        records = sequential_sum(self.rc * vector[None, :])               # [record]
        fitted_projection = sequential_sum(nv.T[:fitted] * vector[None, :])
        cells = (self.boundary * vector[None, :]) * self.bs               # [row][column]
        value = sequential_sum(cells)
        for rank in range(RANK):
            value = value + (self.ck[:, rank] * old[rank]) * self.bs
        for record in range(WINDOW):
            value = value + (self.rk[record] * records[record]) * self.record_suffix[record]
        for rank in range(fitted):
            value = value - nk[:, rank] * fitted_projection[rank]
        return value.astype(F)

    def apply_transpose(self, vector, nk, nv, fitted):
        """:168-221: output[column] = R^T vector, summed over rows in order."""
        old = sequential_sum(self.ck.T * vector[None, :])
        records = sequential_sum(self.rk * vector[None, :])
        fitted_projection = sequential_sum(nk.T[:fitted] * vector[None, :])
        cells = (self.boundary * vector[:, None]) * self.bs               # [row][column]
        value = sequential_sum(cells.T)
        for rank in range(RANK):
            value = value + (self.cv[:, rank] * old[rank]) * self.bs
        for record in range(WINDOW):
            value = value + (self.rc[record] * records[record]) * self.record_suffix[record]
        for rank in range(fitted):
            value = value - nv[:, rank] * fitted_projection[rank]
        return value.astype(F)

    def residual(self, nk, nv):
        """:223-251 for every cell: [row][column]."""
        value = self.boundary * self.bs
        for rank in range(RANK):
            value = value + (self.ck[:, rank][:, None] * self.cv[:, rank][None, :]) * self.bs
            value = value - nk[:, rank][:, None] * nv[:, rank][None, :]
        for record in range(WINDOW):
            value = value + (self.rk[record][:, None] * self.rc[record][None, :]) * \
                self.record_suffix[record]
        return value.astype(F)


def power_refit(buf: dict, s: int, iterations: int, start=start_vector, sqrt=square_root):
    """ProcessState (:253-366) of one full window; returns the next codes
    ([column][row], the slot's [value][key] layout), smoothing, scales, fp16
    compensator bits and the fitted residual [row][column]."""
    st = State(buf, s)
    nk = np.zeros((DIM, RANK), F)
    nv = np.zeros((DIM, RANK), F)
    for rank in range(RANK):
        right, _ = normalize(start(rank))
        left = None
        for _ in range(iterations):
            left, ok = normalize(st.apply_right(right, nk, nv, rank))
            if not ok:
                break
            right, ok = normalize(st.apply_transpose(left, nk, nv, rank))
            if not ok:
                break
        left = st.apply_right(right, nk, nv, rank)
        singular = sqrt(sequential_sum((left * left)[None])[0])
        if singular > F(1.0e-20):
            inverse = F(1.0) / singular
            nk[:, rank] = ((left * inverse) * singular).astype(np.float16).astype(F)
            nv[:, rank] = right.astype(np.float16).astype(F)
    cells = st.residual(nk, nv)
    mean = sequential_sum(np.abs(cells)) / F(128.0)
    smoothing = np.array([sqrt(m if m > F(1.0e-8) else F(1.0e-8)) for m in mean], F)
    smoothed = (cells / smoothing[:, None]).astype(F)
    scales = np.zeros(DIM, F)
    for row in range(DIM):  # value > maximum ? value : maximum, rows in order
        scales = np.where(np.abs(smoothed[row]) > scales, np.abs(smoothed[row]), scales)
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(scales[None, :] == 0, F(0.0), (smoothed / scales[None, :]) * F(127.0))
    q = (q + np.where(q >= 0, F(0.5), F(-0.5))).astype(F)
    q = np.where(q > F(127.0), F(127.0), q)
    q = np.where(q < F(-127.0), F(-127.0), q)
    codes = np.trunc(q).astype(np.int8).T                          # [column][row]
    f16 = lambda x: x.astype(np.float16).view(np.uint16)  # noqa: E731
    return {"next_residual": np.ascontiguousarray(codes), "next_smoothing": smoothing,
            "next_scales": scales.astype(F), "next_compensator_keys": f16(nk),
            "next_compensator_values": f16(nv), "workspace": cells}
