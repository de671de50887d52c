"""Capsule wire-format oracle -- TEST INFRASTRUCTURE ONLY.

numpy wrappers over the LQCAPS01 functions of ``libgdn_oracle.so``
(``gdn_capsule_oracle.c``) and over the capsule entries of the reference
harness (``gdnref_sha256_hex``, ``gdnref_capsule_after_tokens``,
``gdnref_capsule_restore``).  Slot buffers travel as the dict of numpy arrays
the window oracle uses (``oracle.window``).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _ptr, lib, ref
from .window import DIM, RANK, WINDOW

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_I = ctypes.c_int
_F = ctypes.c_float
_C = ctypes.c_char_p

# Restore outcomes (gdn_oracle.h GDN_ORACLE_CAPSULE_*).
OK = 0
TRUNCATED = 1
MAGIC = 2
DIGEST_ENCODING = 3
DIGEST_MISMATCH = 4
PARAMETERS = 5
IDENTITY = 6
RANK_GEOMETRY = 7
POSITION = 8
PHASE = 9
RESIDUAL_DOMAIN = 10
BOUNDARY_PAYLOAD = 11
RECORD_NONFINITE = 12
TRAILING = 13
STATE_NONFINITE = 14
DEVICE_FORMAT = 15
ARGUMENT = 17

# The reference's exception text for each outcome (state_capsule.cpp:24-48,
# 79-104, 476-578): how a reference rejection is named in the tests.
REFERENCE_MESSAGES = {
    TRUNCATED: ("too short", "truncated"),
    MAGIC: ("magic differs",),
    DIGEST_ENCODING: ("checksum encoding is invalid",),
    DIGEST_MISMATCH: ("checksum differs",),
    PARAMETERS: ("quantization parameters differ",),
    IDENTITY: ("identity or geometry differs",),
    RANK_GEOMETRY: ("rank exceeds restored geometry",),
    POSITION: ("window position is invalid",),
    PHASE: ("window phase differs",),
    RESIDUAL_DOMAIN: ("contains -128",),
    BOUNDARY_PAYLOAD: ("boundary payload is invalid",),
    RECORD_NONFINITE: ("update record is non-finite",),
    TRAILING: ("trailing unverified payload",),
    STATE_NONFINITE: ("restored state is non-finite",),
}

SCHEMA, BITS = 1, 8
FLOOR = np.float32(1.0e-8)
HEADER = 120
DIGEST = 64


@dataclass(frozen=True)
class Identity:
    geometry: str = "a" * 64
    generation: int = 7
    epoch: int = 11

    @property
    def geometry_bytes(self) -> bytes:
        return self.geometry.encode("ascii")


_bound = False


def _l() -> ctypes.CDLL:
    global _bound
    l = lib()
    if not _bound:
        l.gdn_oracle_sha256_hex.argtypes = [_P, _U64, _P]
        l.gdn_oracle_sha256_hex.restype = None
        l.gdn_oracle_capsule_bytes.argtypes = [_U32] * 4
        l.gdn_oracle_capsule_bytes.restype = _U64
        l.gdn_oracle_capsule_serialize.argtypes = (
            [_C, _U64, _U64] + [_U32] * 6 + [_F] + [_P] * 5 + [_U32] + [_P] * 4)
        l.gdn_oracle_capsule_serialize.restype = _U64
        l.gdn_oracle_capsule_restore.argtypes = (
            [_P, _U64, _C, _U64, _U64] + [_U32] * 6 + [_F, _U32] + [_P] * 10)
        l.gdn_oracle_capsule_restore.restype = _I
        l.gdn_oracle_slot_capsule_bytes.argtypes = [_U32]
        l.gdn_oracle_slot_capsule_bytes.restype = _U64
        l.gdn_oracle_slot_capsule_serialize.argtypes = [_U32] + [_P] * 8 + [_U32, _C, _U64, _U64, _P]
        l.gdn_oracle_slot_capsule_serialize.restype = _U64
        l.gdn_oracle_slot_capsule_restore.argtypes = [_P, _U64, _C, _U64, _U64, _U32, _U32] + [_P] * 9
        l.gdn_oracle_slot_capsule_restore.restype = _I
        _bound = True
    return l


def _buf(data: bytes) -> np.ndarray:
    return np.frombuffer(bytes(data), np.uint8).copy() if data else np.zeros(1, np.uint8)


# ------------------------------------------------------------------- SHA-256


def sha256_hex(data: bytes) -> str:
    out = ctypes.create_string_buffer(64)
    arr = _buf(data)
    _l().gdn_oracle_sha256_hex(_ptr(arr), len(data), out)
    return out.raw.decode("ascii")


def ref_sha256_hex(data: bytes) -> str:
    r = ref()
    r.gdnref_sha256_hex.argtypes = [_P, _U64, _P]
    r.gdnref_sha256_hex.restype = _I
    out = ctypes.create_string_buffer(64)
    arr = _buf(data)
    r.gdnref_sha256_hex(_ptr(arr), len(data), out)
    return out.raw.decode("ascii")


def refresh_digest(encoded: bytes) -> bytes:
    """The reference test's RefreshChecksum (capsule_test.cpp:147-155)."""
    content = bytes(encoded[:-DIGEST])
    return content + sha256_hex(content).encode("ascii")


# ------------------------------------------------- generic capsule (any K, V)


@dataclass
class Fields:
    """A capsule's payload in the reference's own representation."""

    residual: np.ndarray       # int8 [K][V]
    smoothing: np.ndarray      # fp32 [K]
    scales: np.ndarray         # fp32 [V]
    comp_keys: np.ndarray      # fp32 [K][4]
    comp_values: np.ndarray    # fp32 [V][4]
    decay: np.ndarray          # fp32 [updates][K]
    key: np.ndarray            # fp32 [updates][K]
    correction: np.ndarray     # fp32 [updates][V]

    @property
    def updates(self) -> int:
        return self.decay.shape[0]


def capsule_bytes(keys: int, values: int, updates: int, rank: int = RANK) -> int:
    return int(_l().gdn_oracle_capsule_bytes(keys, values, rank, updates))


def serialize(fields: Fields, identity: Identity, *, schema=SCHEMA, window=WINDOW,
              rank=RANK, bits=BITS, floor=FLOOR) -> bytes:
    keys, values = fields.residual.shape
    c = lambda a, dt: np.ascontiguousarray(a, dt)  # noqa: E731
    arrays = [c(fields.residual, np.int8), c(fields.smoothing, np.float32),
              c(fields.scales, np.float32), c(fields.comp_keys, np.float32),
              c(fields.comp_values, np.float32)]
    records = [c(fields.decay, np.float32), c(fields.key, np.float32),
               c(fields.correction, np.float32)]
    records = [r if r.size else np.zeros(1, np.float32) for r in records]
    out = np.zeros(capsule_bytes(keys, values, fields.updates, rank), np.uint8)
    n = _l().gdn_oracle_capsule_serialize(
        identity.geometry_bytes, identity.generation, identity.epoch, keys, values, schema,
        window, rank, bits, floor, *(_ptr(a) for a in arrays), fields.updates,
        *(_ptr(r) for r in records), _ptr(out))
    assert n == out.size
    return out.tobytes()


def restore(encoded: bytes, identity: Identity, keys: int, values: int,
            expected_position: int, *, schema=SCHEMA, window=WINDOW, rank=RANK, bits=BITS,
            floor=FLOOR):
    """(status, Fields or None)."""
    arr = _buf(encoded)
    f = Fields(np.zeros((keys, values), np.int8), np.zeros(keys, np.float32),
               np.zeros(values, np.float32), np.zeros((keys, rank), np.float32),
               np.zeros((values, rank), np.float32), np.zeros((window, keys), np.float32),
               np.zeros((window, keys), np.float32), np.zeros((window, values), np.float32))
    work = np.zeros(keys * values, np.float32)
    count = ctypes.c_uint32(0)
    status = _l().gdn_oracle_capsule_restore(
        _ptr(arr), len(encoded), identity.geometry_bytes, identity.generation, identity.epoch,
        keys, values, schema, window, rank, bits, floor, expected_position, _ptr(f.residual),
        _ptr(f.smoothing), _ptr(f.scales), _ptr(f.comp_keys), _ptr(f.comp_values),
        _ptr(f.decay), _ptr(f.key), _ptr(f.correction), _ptr(work), ctypes.byref(count))
    if status != OK:
        return status, None
    n = count.value
    f.decay, f.key, f.correction = f.decay[:n].copy(), f.key[:n].copy(), f.correction[:n].copy()
    return status, f


# ----------------------------------------------------- reference (oracle/_ref)


def _bind_ref(r):
    r.gdnref_capsule_after_tokens.argtypes = (
        [_P, _U32, _U32, _U32] + [_P] * 5 + [_C, _U64, _U64, _P, _U64, _P, _P, _U64])
    r.gdnref_capsule_after_tokens.restype = _I
    r.gdnref_capsule_restore.argtypes = (
        [_P, _U64, _C, _U64, _U64] + [_U32] * 6 + [_F, _U32, _P, _U64, _P, _P, _P, _U64])
    r.gdnref_capsule_restore.restype = _I
    return r


def ref_capsule_after_tokens(dense, identity: Identity, decay, key, value, read, query) -> bytes:
    """The reference's own capsule: FromDenseBoundary (rank 4) of `dense`
    [K][V], ApplyToken per token, Serialize."""
    r = _bind_ref(ref())
    dense = np.ascontiguousarray(dense, np.float32)
    keys, values = dense.shape
    tokens = decay.shape[0]
    ins = [np.ascontiguousarray(a, np.float32) for a in (decay, key, value, read, query)]
    ins = [a if a.size else np.zeros(1, np.float32) for a in ins]
    capacity = capsule_bytes(keys, values, WINDOW)
    out = np.zeros(capacity, np.uint8)
    size = ctypes.c_uint64(0)
    message = ctypes.create_string_buffer(256)
    status = r.gdnref_capsule_after_tokens(
        _ptr(dense), keys, values, tokens, *(_ptr(a) for a in ins), identity.geometry_bytes,
        identity.generation, identity.epoch, _ptr(out), capacity, ctypes.byref(size),
        message, 256)
    if status != 0:
        raise RuntimeError(message.value.decode())
    return out[:size.value].tobytes()


def ref_restore(encoded: bytes, identity: Identity, keys: int, values: int,
                expected_position: int, *, schema=SCHEMA, window=WINDOW, rank=RANK,
                bits=BITS, floor=FLOOR):
    """(None, reserialized bytes, DenseState) on success, (message, None, None)
    when the reference's Restore rejects the capsule."""
    r = _bind_ref(ref())
    arr = _buf(encoded)
    capacity = len(encoded) + 1
    out = np.zeros(capacity, np.uint8)
    size = ctypes.c_uint64(0)
    dense = np.zeros((keys, values), np.float32)
    message = ctypes.create_string_buffer(256)
    status = r.gdnref_capsule_restore(
        _ptr(arr), len(encoded), identity.geometry_bytes, identity.generation, identity.epoch,
        keys, values, schema, window, rank, bits, floor, expected_position, _ptr(out),
        capacity, ctypes.byref(size), _ptr(dense), message, 256)
    if status != 0:
        return message.value.decode(), None, None
    return None, out[:size.value].tobytes(), dense


def outcome_of_message(message: str) -> int:
    """The oracle outcome a reference exception message names."""
    for status, needles in REFERENCE_MESSAGES.items():
        if any(n in message for n in needles):
            return status
    raise AssertionError(f"unmapped reference message: {message!r}")


# ------------------------------------------------------- device window slots


def slot_capsule_bytes(position: int) -> int:
    return int(_l().gdn_oracle_slot_capsule_bytes(position))


_SLOT_NAMES = ("residual", "smoothing", "scales", "compensator_keys", "compensator_values",
               "record_decay", "record_keys", "record_corrections")


def slot_serialize(buf: dict, state: int, layout: int, identity: Identity) -> bytes:
    """Capsule of state `state` of a window-slot buffer dict (b"" when its
    position is 16 or more)."""
    position = int(buf["positions"][state, 0])
    parts = [np.ascontiguousarray(buf[name][state]) for name in _SLOT_NAMES]
    out = np.zeros(max(slot_capsule_bytes(position), 1), np.uint8)
    n = _l().gdn_oracle_slot_capsule_serialize(
        layout, *(_ptr(p) for p in parts), position, identity.geometry_bytes,
        identity.generation, identity.epoch, _ptr(out))
    return out[:n].tobytes()


def slot_restore(encoded: bytes, buf: dict, state: int, layout: int, identity: Identity,
                 expected_position: int) -> int:
    """Restore a capsule into state `state` of `buf` (in place, only on
    success); returns the outcome."""
    arr = _buf(encoded)
    parts = [np.ascontiguousarray(buf[name][state]) for name in _SLOT_NAMES]
    word = np.array([buf["positions"][state, 0]], np.uint32)
    status = _l().gdn_oracle_slot_capsule_restore(
        _ptr(arr), len(encoded), identity.geometry_bytes, identity.generation, identity.epoch,
        expected_position, layout, *(_ptr(p) for p in parts), _ptr(word))
    if status == OK:
        for name, part in zip(_SLOT_NAMES, parts):
            buf[name][state] = part
        buf["positions"][state, 0] = word[0]
    return status
