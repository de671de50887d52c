"""Windowed decode-step oracle -- TEST INFRASTRUCTURE ONLY.

numpy wrappers over the window functions of ``libgdn_oracle.so``
(``gdn_window_oracle.c``) and over ``gdnref_apply_tokens`` of the reference
harness.  Device-format buffers travel as a dict of numpy arrays named like the
C-ABI arguments; functions that update them in place say so.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _ptr, lib, ref

DIM = 128
TILE = DIM * DIM
RANK = 4
WINDOW = 16
POSITION_STRIDE = 8
QUERY_SCALE = np.float32(0.08838834764831845)

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_I = ctypes.c_int

_bound = False


def _l() -> ctypes.CDLL:
    global _bound
    l = lib()
    if not _bound:
        l.gdn_oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        l.gdn_oracle_f16_to_f32.restype = ctypes.c_float
        l.gdn_oracle_f32_to_f16.argtypes = [ctypes.c_float]
        l.gdn_oracle_f32_to_f16.restype = ctypes.c_uint16
        l.gdn_oracle_read_window.argtypes = [_P] * 5 + [_U32] * 3 + [_P] * 3 + [_U32, _P, _P]
        l.gdn_oracle_read_window.restype = None
        l.gdn_oracle_dense_state.argtypes = [_P] * 5 + [_U32] * 3 + [_P] * 3 + [_U32, _P]
        l.gdn_oracle_dense_state.restype = None
        l.gdn_oracle_apply_token.argtypes = [_P] * 5 + [_U32] * 4 + [_P] * 4 + [_P] * 6
        l.gdn_oracle_apply_token.restype = _I
        l.gdn_oracle_windowed_step_bf16.argtypes = [_P] * 15 + [_U32] + [_P] * 4
        l.gdn_oracle_windowed_step_bf16.restype = None
        l.gdn_oracle_windowed_step_f16.argtypes = [_P] * 15 + [_U32] + [_P] * 4
        l.gdn_oracle_windowed_step_f16.restype = None
        l.gdn_oracle_gdn_step_f32.argtypes = [_P] * 7 + [_U32]
        l.gdn_oracle_gdn_step_f32.restype = None
        for name in ("gdn_oracle_prepare_decode_pair_bf16", "gdn_oracle_prepare_decode_pair"):
            getattr(l, name).argtypes = [_P] * 6 + [_U32]
            getattr(l, name).restype = None
        l.gdn_oracle_prepare_int8_vector.argtypes = [_P] * 4 + [_U32]
        l.gdn_oracle_prepare_int8_vector.restype = None
        l.gdn_oracle_int8_matmul.argtypes = [_P] * 3 + [_U32, _U32]
        l.gdn_oracle_int8_matmul.restype = None
        for name in ("gdn_oracle_finish_decode_pair_bf16", "gdn_oracle_finish_decode_pair"):
            getattr(l, name).argtypes = [_P] * 15 + [_U32]
            getattr(l, name).restype = None
        _bound = True
    return l


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype)


# ------------------------------------------------------------- conversions

def f16_to_f32(values: np.ndarray) -> np.ndarray:
    """Exact widening of fp16 bit patterns (uint16) to fp32."""
    return np.asarray(values, np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16(values: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even narrowing through the oracle's C routine."""
    flat = np.ascontiguousarray(values, np.float32).reshape(-1)
    f = _l().gdn_oracle_f32_to_f16
    return np.array([f(float(x)) for x in flat], np.uint16).reshape(np.shape(values))


# ------------------------------------------------------------ capsule layer

def read_window(codes, smoothing, scales, read, record_decay=None, record_keys=None,
                record_corrections=None, ck=None, cv=None):
    """ReadWindowState over a [key][value] boundary and per-key-decay records."""
    keys, values = codes.shape
    rank = 0 if ck is None else ck.shape[1]
    records = 0 if record_keys is None else record_keys.shape[0]
    out = np.empty(values, np.float32)
    _l().gdn_oracle_read_window(
        _ptr(_c(codes, np.int8)), _ptr(_c(smoothing, np.float32)), _ptr(_c(scales, np.float32)),
        _ptr(_c(ck, np.float32)), _ptr(_c(cv, np.float32)), keys, values, rank,
        _ptr(_c(record_decay, np.float32)), _ptr(_c(record_keys, np.float32)),
        _ptr(_c(record_corrections, np.float32)), records, _ptr(_c(read, np.float32)),
        _ptr(out))
    return out


class CapsuleWindow:
    """ApplyToken-driven window over one head (the capsule semantics)."""

    def __init__(self, dense: np.ndarray, rank: int = 0, window: int = WINDOW):
        from . import quantize_kv

        keys, values = dense.shape
        self.keys, self.values, self.rank, self.window = keys, values, rank, window
        out = quantize_kv(np.ascontiguousarray(dense, np.float32), rank)
        self.codes, self.smoothing, self.scales = (np.ascontiguousarray(a) for a in out[:3])
        self.ck = np.ascontiguousarray(out[3], np.float32) if rank else np.zeros((keys, 1), np.float32)
        self.cv = np.ascontiguousarray(out[4], np.float32) if rank else np.zeros((values, 1), np.float32)
        self.record_decay = np.zeros((window, keys), np.float32)
        self.record_keys = np.zeros((window, keys), np.float32)
        self.record_corrections = np.zeros((window, values), np.float32)
        self.position = ctypes.c_uint32(0)

    def apply(self, decay, key, value, read, query):
        out = np.empty(self.values, np.float32)
        crossed = _l().gdn_oracle_apply_token(
            _ptr(self.codes), _ptr(self.smoothing), _ptr(self.scales), _ptr(self.ck),
            _ptr(self.cv), self.keys, self.values, self.rank, self.window,
            _ptr(self.record_decay), _ptr(self.record_keys), _ptr(self.record_corrections),
            ctypes.byref(self.position), *(_ptr(_c(a, np.float32)) for a in (decay, key, value, read, query)),
            _ptr(out))
        return out, bool(crossed)

    def dense_state(self):
        out = np.empty((self.keys, self.values), np.float32)
        _l().gdn_oracle_dense_state(
            _ptr(self.codes), _ptr(self.smoothing), _ptr(self.scales), _ptr(self.ck),
            _ptr(self.cv), self.keys, self.values, self.rank, _ptr(self.record_decay),
            _ptr(self.record_keys), _ptr(self.record_corrections), self.position.value,
            _ptr(out))
        return out


def ref_apply_tokens(dense, rank, decay, key, value, read, query):
    """The reference capsule over a token sequence (oracle/_ref)."""
    keys, values = dense.shape
    tokens = decay.shape[0]
    outputs = np.empty((tokens, values), np.float32)
    crossed = np.empty(tokens, np.uint8)
    final = np.empty((keys, values), np.float32)
    r = ref()
    r.gdnref_apply_tokens.argtypes = [_P, _U32, _U32, _U32, _U32] + [_P] * 8
    r.gdnref_apply_tokens.restype = _I
    status = r.gdnref_apply_tokens(
        _ptr(_c(dense, np.float32)), keys, values, rank, tokens,
        *(_ptr(_c(a, np.float32)) for a in (decay, key, value, read, query)),
        _ptr(outputs), _ptr(crossed), _ptr(final))
    assert status == 0
    return outputs, crossed.astype(bool), final


# ------------------------------------------------------ device-format layer

WINDOW_BUFFERS = ("residual", "smoothing", "scales", "compensator_keys",
                  "compensator_values", "record_decay", "record_keys",
                  "record_corrections", "positions")


def _window_args(buf):
    return [_ptr(buf["residual"]), _ptr(buf["smoothing"]), _ptr(buf["scales"]),
            _ptr(buf.get("compensator_keys")), _ptr(buf.get("compensator_values")),
            _ptr(buf["record_decay"]), _ptr(buf["record_keys"]),
            _ptr(buf["record_corrections"]), _ptr(buf["positions"])]


def windowed_step_bf16(buf: dict, log_decay, beta, keys, queries, values, quant_only=False):
    """One bf16 windowed step; updates the record/position arrays of ``buf`` in
    place.  Returns (outputs bf16 bits, out64, out_bound, corr64, corr_bound)."""
    states = buf["residual"].shape[0]
    if quant_only:
        buf = dict(buf, compensator_keys=None, compensator_values=None)
    outputs = np.zeros((states, DIM), np.uint16)
    out64, out_bound, corr64, corr_bound = (np.zeros((states, DIM)) for _ in range(4))
    _l().gdn_oracle_windowed_step_bf16(
        *_window_args(buf), _ptr(_c(log_decay, np.float32)), _ptr(_c(beta, np.uint16)),
        _ptr(_c(keys, np.uint16)), _ptr(_c(queries, np.uint16)), _ptr(_c(values, np.uint16)),
        _ptr(outputs), states, _ptr(out64), _ptr(out_bound), _ptr(corr64), _ptr(corr_bound))
    return outputs, out64, out_bound, corr64, corr_bound


def windowed_step_f16(buf: dict, decay, write_keys, reads, queries, values):
    """One fp16 (v1) windowed step; updates ``buf`` in place.  Returns
    (outputs fp32, out64, out_bound, corr64, corr_bound)."""
    states = buf["residual"].shape[0]
    outputs = np.zeros((states, DIM), np.float32)
    out64, out_bound, corr64, corr_bound = (np.zeros((states, DIM)) for _ in range(4))
    _l().gdn_oracle_windowed_step_f16(
        *_window_args(buf), _ptr(_c(decay, np.float32)), _ptr(_c(write_keys, np.uint16)),
        _ptr(_c(reads, np.uint16)), _ptr(_c(queries, np.uint16)), _ptr(_c(values, np.uint16)),
        _ptr(outputs), states, _ptr(out64), _ptr(out_bound), _ptr(corr64), _ptr(corr_bound))
    return outputs, out64, out_bound, corr64, corr_bound


def gdn_step_f32(state, decay, keys, reads, queries, values):
    """Dense fp32 GDN step; updates ``state`` [S,128,128] in place."""
    states = state.shape[0]
    outputs = np.zeros((states, DIM), np.float32)
    _l().gdn_oracle_gdn_step_f32(
        _ptr(state), _ptr(_c(decay, np.float32)), _ptr(_c(keys, np.uint16)),
        _ptr(_c(reads, np.uint16)), _ptr(_c(queries, np.uint16)), _ptr(_c(values, np.uint16)),
        _ptr(outputs), states)
    return outputs


def prepare_decode_pair_bf16(keys, queries, log_decay, smoothing):
    states = smoothing.shape[0]
    quantized = np.zeros((states, DIM, 16), np.int8)
    dynamic_scale = np.zeros((states, POSITION_STRIDE), np.float32)
    _l().gdn_oracle_prepare_decode_pair_bf16(
        _ptr(_c(keys, np.uint16)), _ptr(_c(queries, np.uint16)), _ptr(_c(log_decay, np.float32)),
        _ptr(_c(smoothing, np.float32)), _ptr(quantized), _ptr(dynamic_scale), states)
    return quantized, dynamic_scale


def prepare_decode_pair(reads, queries, decay, smoothing):
    states = smoothing.shape[0]
    quantized = np.zeros((states, DIM, 16), np.int8)
    dynamic_scale = np.zeros((states, POSITION_STRIDE), np.float32)
    _l().gdn_oracle_prepare_decode_pair(
        _ptr(_c(reads, np.uint16)), _ptr(_c(queries, np.uint16)), _ptr(_c(decay, np.float32)),
        _ptr(_c(smoothing, np.float32)), _ptr(quantized), _ptr(dynamic_scale), states)
    return quantized, dynamic_scale


def prepare_int8_vector(inputs, axis_scale):
    states = axis_scale.shape[0]
    quantized = np.zeros((states, DIM, 16), np.int8)
    dynamic_scale = np.zeros((states, POSITION_STRIDE), np.float32)
    _l().gdn_oracle_prepare_int8_vector(
        _ptr(_c(inputs, np.uint16)), _ptr(_c(axis_scale, np.float32)), _ptr(quantized),
        _ptr(dynamic_scale), states)
    return quantized, dynamic_scale


def int8_matmul(a, b, transpose_a=0):
    states = a.shape[0]
    c = np.zeros((states, DIM, 16), np.int32)
    _l().gdn_oracle_int8_matmul(_ptr(_c(a, np.int8)), _ptr(_c(b, np.int8)), _ptr(c), states,
                                transpose_a)
    return c


def finish_decode_pair_bf16(buf: dict, projected, dynamic_scale, log_decay, beta, keys,
                            queries, values):
    states = buf["residual"].shape[0]
    outputs = np.zeros((states, DIM), np.uint16)
    _l().gdn_oracle_finish_decode_pair_bf16(
        _ptr(_c(projected, np.int32)), _ptr(_c(dynamic_scale, np.float32)), _ptr(buf["scales"]),
        _ptr(buf["compensator_keys"]), _ptr(buf["compensator_values"]), _ptr(buf["record_decay"]),
        _ptr(buf["record_keys"]), _ptr(buf["record_corrections"]), _ptr(buf["positions"]),
        _ptr(_c(log_decay, np.float32)), _ptr(_c(beta, np.uint16)), _ptr(_c(keys, np.uint16)),
        _ptr(_c(queries, np.uint16)), _ptr(_c(values, np.uint16)), _ptr(outputs), states)
    return outputs


def finish_decode_pair(buf: dict, projected, dynamic_scale, decay, write_keys, reads,
                       queries, values):
    states = buf["residual"].shape[0]
    outputs = np.zeros((states, DIM), np.float32)
    _l().gdn_oracle_finish_decode_pair(
        _ptr(_c(projected, np.int32)), _ptr(_c(dynamic_scale, np.float32)), _ptr(buf["scales"]),
        _ptr(buf["compensator_keys"]), _ptr(buf["compensator_values"]), _ptr(buf["record_decay"]),
        _ptr(buf["record_keys"]), _ptr(buf["record_corrections"]), _ptr(buf["positions"]),
        _ptr(_c(decay, np.float32)), _ptr(_c(write_keys, np.uint16)), _ptr(_c(reads, np.uint16)),
        _ptr(_c(queries, np.uint16)), _ptr(_c(values, np.uint16)), _ptr(outputs), states)
    return outputs


def ref_read_window(codes, smoothing, scales, read, record_decay, record_keys,
                    record_corrections, ck=None, cv=None):
    """The reference's ReadWindowState with buffered records (oracle/_ref)."""
    keys, values = codes.shape
    rank = 0 if ck is None else ck.shape[1]
    records = record_keys.shape[0]
    out = np.empty(values, np.float32)
    r = ref()
    r.gdnref_read_window.argtypes = [_P] * 5 + [_U32] * 3 + [_P] * 3 + [_U32, _P, _P]
    r.gdnref_read_window.restype = _I
    status = r.gdnref_read_window(
        _ptr(_c(codes, np.int8)), _ptr(_c(smoothing, np.float32)), _ptr(_c(scales, np.float32)),
        _ptr(_c(ck, np.float32)), _ptr(_c(cv, np.float32)), keys, values, rank,
        _ptr(_c(record_decay, np.float32)), _ptr(_c(record_keys, np.float32)),
        _ptr(_c(record_corrections, np.float32)), records, _ptr(_c(read, np.float32)),
        _ptr(out))
    assert status == 0
    return out


# ------------------------------------------------------- window-boundary refit

def _bind_boundary(l):
    if getattr(l, "_boundary_bound", False):
        return l
    l.gdn_oracle_boundary_sqrt.argtypes = [ctypes.c_float]
    l.gdn_oracle_boundary_sqrt.restype = ctypes.c_float
    l.gdn_oracle_window_boundary_quant_only.argtypes = [_P] * 13 + [_U32]
    l.gdn_oracle_window_boundary_quant_only.restype = None
    l.gdn_oracle_boundary_scale_records.argtypes = [_P] * 3 + [_U32]
    l.gdn_oracle_boundary_scale_records.restype = None
    l.gdn_oracle_f16_matmul_at_b.argtypes = [_P] * 3 + [_U32]
    l.gdn_oracle_f16_matmul_at_b.restype = None
    l.gdn_oracle_window_boundary_power.argtypes = [_P] * 15 + [_U32, _U32]
    l.gdn_oracle_window_boundary_power.restype = None
    l._boundary_bound = True
    return l


def boundary_outputs(states: int) -> dict:
    """Zeroed next-boundary buffers of a refit."""
    return {"next_residual": np.zeros((states, DIM, DIM), np.int8),
            "next_smoothing": np.zeros((states, DIM), np.float32),
            "next_scales": np.zeros((states, DIM), np.float32),
            "next_compensator_keys": np.zeros((states, DIM, RANK), np.uint16),
            "next_compensator_values": np.zeros((states, DIM, RANK), np.uint16)}


def window_boundary_quant_only(buf: dict, out: dict, record_merge=None) -> None:
    """The quant-only refit; updates ``out`` and ``buf['positions']`` in place."""
    states = buf["residual"].shape[0]
    _bind_boundary(_l()).gdn_oracle_window_boundary_quant_only(
        _ptr(buf["residual"]), _ptr(buf["smoothing"]), _ptr(buf["scales"]),
        _ptr(buf["record_decay"]), _ptr(buf["record_keys"]), _ptr(buf["record_corrections"]),
        _ptr(buf["positions"]), _ptr(out["next_residual"]), _ptr(out["next_smoothing"]),
        _ptr(out["next_scales"]), _ptr(out["next_compensator_keys"]),
        _ptr(out["next_compensator_values"]), _ptr(_c(record_merge, np.float32)), states)


def boundary_scale_records(record_decay, record_keys):
    states = record_decay.shape[0]
    scaled = np.zeros((states, WINDOW, DIM), np.uint16)
    _bind_boundary(_l()).gdn_oracle_boundary_scale_records(
        _ptr(_c(record_decay, np.float32)), _ptr(_c(record_keys, np.uint16)), _ptr(scaled), states)
    return scaled


def f16_matmul_at_b(a, b):
    states = a.shape[0]
    c = np.zeros((states, DIM, DIM), np.float32)
    _bind_boundary(_l()).gdn_oracle_f16_matmul_at_b(
        _ptr(_c(a, np.uint16)), _ptr(_c(b, np.uint16)), _ptr(c), states)
    return c


def window_boundary_power(buf: dict, out: dict, workspace, power_iterations: int) -> None:
    """The rank-4 power-iteration refit; updates ``out``, ``workspace`` and the
    record/position arrays of ``buf`` in place."""
    states = buf["residual"].shape[0]
    _bind_boundary(_l()).gdn_oracle_window_boundary_power(
        _ptr(buf["residual"]), _ptr(buf["smoothing"]), _ptr(buf["scales"]),
        _ptr(buf["compensator_keys"]), _ptr(buf["compensator_values"]),
        _ptr(buf["record_decay"]), _ptr(buf["record_keys"]), _ptr(buf["record_corrections"]),
        _ptr(buf["positions"]), _ptr(out["next_residual"]), _ptr(out["next_smoothing"]),
        _ptr(out["next_scales"]), _ptr(out["next_compensator_keys"]),
        _ptr(out["next_compensator_values"]), _ptr(workspace), states, power_iterations)


# ------------------------------------------- device rank-4 chain (encoded boundary)

def _bind_encoded(l):
    if getattr(l, "_encoded_bound", False):
        return l
    for name in ("gdn_oracle_finish_encoded_projection",):
        getattr(l, name).argtypes = [_P] * 13 + [_U32] * 3
        getattr(l, name).restype = None
    l.gdn_oracle_commit_encoded_rank.argtypes = [_P] * 13 + [_U32] * 2
    l.gdn_oracle_commit_encoded_rank.restype = None
    l.gdn_oracle_encoded_requantize.argtypes = [_P] * 16 + [_U32]
    l.gdn_oracle_encoded_requantize.restype = None
    l._encoded_bound = True
    return l


ENCODED_OPERANDS = ("smoothing", "scales", "old_left", "old_right", "record_decay",
                    "record_left", "record_right")


def finish_encoded_projection(enc: dict, projected, dynamic_scale, inputs, fitted_ranks: int,
                              transpose: int):
    """finish_encoded_projection_launch_v1 -> fp16 bits [S][128][16].  ``enc``
    holds the operands named in ENCODED_OPERANDS plus new_left / new_right."""
    states = enc["smoothing"].shape[0]
    output = np.zeros((states, DIM, 16), np.uint16)
    _bind_encoded(_l()).gdn_oracle_finish_encoded_projection(
        _ptr(_c(projected, np.int32)), _ptr(_c(dynamic_scale, np.float32)),
        _ptr(_c(inputs, np.uint16)), *(_ptr(enc[k]) for k in ENCODED_OPERANDS),
        _ptr(enc["new_left"]), _ptr(enc["new_right"]), _ptr(output), states, fitted_ranks,
        transpose)
    return output


def commit_encoded_rank(enc: dict, projected, dynamic_scale, inputs, corrected, rank: int):
    """commit_encoded_rank_launch_v1; updates enc['new_left'], enc['new_right']
    (rank ``rank``) and column 0 of ``corrected`` in place."""
    states = enc["smoothing"].shape[0]
    _bind_encoded(_l()).gdn_oracle_commit_encoded_rank(
        _ptr(_c(projected, np.int32)), _ptr(_c(dynamic_scale, np.float32)),
        _ptr(_c(inputs, np.uint16)), *(_ptr(enc[k]) for k in ENCODED_OPERANDS),
        _ptr(enc["new_left"]), _ptr(enc["new_right"]), _ptr(corrected), states, rank)


def encoded_requantize(enc: dict, residual):
    """encoded_requantize_launch_v1 -> dict of next_residual, next_smoothing,
    next_scales, next_left, next_right, workspace."""
    states = enc["smoothing"].shape[0]
    out = {"next_residual": np.zeros((states, DIM, DIM), np.int8),
           "next_smoothing": np.zeros((states, DIM), np.float32),
           "next_scales": np.zeros((states, DIM), np.float32),
           "next_left": np.zeros((states, DIM, RANK), np.uint16),
           "next_right": np.zeros((states, DIM, RANK), np.uint16),
           "workspace": np.zeros((states, DIM, DIM), np.float32)}
    _bind_encoded(_l()).gdn_oracle_encoded_requantize(
        _ptr(_c(residual, np.int8)), *(_ptr(enc[k]) for k in ENCODED_OPERANDS),
        _ptr(enc["new_left"]), _ptr(enc["new_right"]), _ptr(out["next_residual"]),
        _ptr(out["next_smoothing"]), _ptr(out["next_scales"]), _ptr(out["next_left"]),
        _ptr(out["next_right"]), _ptr(out["workspace"]), states)
    return out
