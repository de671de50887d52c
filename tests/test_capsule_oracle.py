"""CPU pins of the capsule wire-format oracle (oracle/gdn_capsule_oracle.c)
and of the capsule ApplyToken oracle against the reference test's own
trajectory anchors.

* SHA-256: FIPS 180-4 example digests, hashlib on every length 0..300 and on
  multi-block messages, and the reference's Sha256Hex (oracle/_ref).
* Serialize / Restore: byte equality and identical accept/reject decisions
  against the reference's own Serialize / Restore (oracle/_ref) on capsules
  the reference built, on the reference test's corruptions
  (native/tests/gdn_state_codec_state_capsule_test.cpp:292-371) and on further
  truncations, trailing bytes and invalid payloads.
* Slot capsules: the reference's Restore admits them and re-serializes the
  same bytes, and its DenseState equals the oracle's capsule dense state of the
  same slot buffers bit for bit (and float64 within fp32 rounding).
"""

from __future__ import annotations

import ctypes
import hashlib

import numpy as np
import pytest

import oracle
import windowgen as WG
from oracle import capsule as C
from oracle import window as W

pytestmark = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")

VK, KV = oracle.LAYOUT_VALUE_KEY, oracle.LAYOUT_KEY_VALUE
KEYS, VALUES = 8, 6  # the reference test's geometry (capsule_test.cpp:26-27)
IDENTITY = C.Identity("a" * 64, 7, 11)  # capsule_test.cpp:33-38

# ------------------------------------------------------------------ SHA-256


def test_sha256_matches_fips_vectors_hashlib_and_the_reference():
    fips = {
        b"abc": "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad",
        b"": "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855",
        b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq":
            "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1",
    }
    for message, digest in fips.items():
        assert C.sha256_hex(message) == digest
    g = np.random.default_rng(5)
    for n in list(range(301)) + [4095, 4096, 4097, 21624, 44664]:
        data = g.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert C.sha256_hex(data) == hashlib.sha256(data).hexdigest(), n
    for n in (0, 63, 64, 65, 1000, 21624):
        data = g.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert C.ref_sha256_hex(data) == hashlib.sha256(data).hexdigest(), n


# ------------------------------------- the reference test's inputs, via libm


_libm = ctypes.CDLL("libm.so.6")
for _name in ("sinf", "cosf"):
    getattr(_libm, _name).argtypes = [ctypes.c_float]
    getattr(_libm, _name).restype = ctypes.c_float
f32 = np.float32


def initial_state() -> np.ndarray:
    """InitialState() (capsule_test.cpp:40-48), evaluated in fp32 with the
    same libm sinf the reference test calls."""
    state = np.zeros(KEYS * VALUES, np.float32)
    for i in range(state.size):
        base = f32(_libm.sinf(f32(f32(i + 1) * f32(0.37)))) * f32(0.4)
        state[i] = base + (f32(3.5) if i % 17 == 0 else f32(0.0))
    return state.reshape(KEYS, VALUES)


def token(step: int, bias: float = 0.0):
    """Token(step, bias) (capsule_test.cpp:50-73) -> decay, key, value, read, query."""
    b = f32(bias)
    d, k, r, q = (np.zeros(KEYS, np.float32) for _ in range(4))
    v = np.zeros(VALUES, np.float32)
    for row in range(KEYS):
        d[row] = f32(0.985) - f32(0.001) * f32((step + row) % 5)
        k[row] = f32(0.025) * f32(_libm.sinf(f32(f32((step + 1) * (row + 1)) * f32(0.13)))) + b
        r[row] = f32(0.02) * f32(_libm.cosf(f32(f32((step + 2) * (row + 1)) * f32(0.11))))
        q[row] = f32(0.03) * f32(_libm.sinf(f32(f32((step + 3) * (row + 1)) * f32(0.07))))
    for c in range(VALUES):
        v[c] = f32(0.2) * f32(_libm.cosf(f32(f32((step + 1) * (c + 2)) * f32(0.09)))) + b
    return d, k, v, r, q


def tokens(count: int):
    toks = [token(s) for s in range(count)]
    widths = (KEYS, KEYS, VALUES, KEYS, KEYS)
    return [np.stack([t[i] for t in toks]) if toks else np.zeros((0, widths[i]), np.float32)
            for i in range(5)]


def test_capsule_trajectory_matches_the_reference_test_anchors():
    """CheckTrajectory (capsule_test.cpp:167-209) on the oracle's capsule:
    256 tokens, 16 window crossings, the first/last output anchors and the
    canonical output digest the reference test fixes."""
    cap = W.CapsuleWindow(initial_state(), rank=4)
    fp32 = initial_state().astype(np.float64)
    outputs, expected, crossings = [], [], 0
    for step in range(256):
        d, k, v, r, q = token(step)
        out, crossed = cap.apply(d, k, v, r, q)
        crossings += crossed
        outputs.append(out)
        correction = v - fp32.T @ r
        fp32 = d[:, None] * fp32 + np.outer(k, correction)
        expected.append(fp32.T @ q)
    outputs = np.concatenate(outputs)
    assert crossings == 16 and cap.position.value == 0
    assert abs(outputs[0] - 0.0243581) < 1e-6 and abs(outputs[-1] + 0.00297543) < 1e-6
    # CanonicalFloatDigest (capsule_test.cpp:130-141): llround(value * 1e4f).
    fixed = np.array([np.round(np.float64(f32(x) * f32(1.0e4))) for x in outputs])
    halfway = np.abs(np.float64(outputs * f32(1.0e4)) % 1.0) == 0.5
    assert not halfway.any()  # np.round is half-even; llround is half-away
    digest = hashlib.sha256(fixed.astype("<i8").tobytes()).hexdigest()
    assert digest == "6ab3da8358cd8c5ca5394bf10ad78015bc3f556804da1075ba91d49a5db30561"
    rel = lambda a, b: np.sqrt(((a - b) ** 2).sum() / (b ** 2).sum())  # noqa: E731
    assert rel(cap.dense_state().astype(np.float64), fp32) < 0.025
    assert rel(outputs.astype(np.float64), np.concatenate(expected)) < 0.025


# --------------------------------------------- reference-built capsules


@pytest.fixture(scope="module")
def hibernated() -> bytes:
    """CheckHibernateResume's capsule (capsule_test.cpp:292-296): 7 tokens."""
    return C.ref_capsule_after_tokens(initial_state(), IDENTITY, *tokens(7))


def test_reference_capsule_round_trips_through_the_oracle(hibernated):
    assert len(hibernated) == C.capsule_bytes(KEYS, VALUES, 7)
    assert hibernated[:8] == b"LQCAPS01"
    status, fields = C.restore(hibernated, IDENTITY, KEYS, VALUES, 7)
    assert status == C.OK and fields.updates == 7
    assert C.serialize(fields, IDENTITY) == hibernated
    message, again, _ = C.ref_restore(hibernated, IDENTITY, KEYS, VALUES, 7)
    assert message is None and again == hibernated
    # A capsule at position 0 and one just before the window closes.
    for count in (0, 15):
        enc = C.ref_capsule_after_tokens(initial_state(), IDENTITY, *tokens(count))
        status, fields = C.restore(enc, IDENTITY, KEYS, VALUES, count)
        assert status == C.OK and C.serialize(fields, IDENTITY) == enc


def _patched(encoded: bytes, offset: int, raw: bytes, refresh: bool = True) -> bytes:
    out = bytearray(encoded)
    out[offset:offset + len(raw)] = raw
    return C.refresh_digest(bytes(out)) if refresh else bytes(out)


def _f(value: float) -> bytes:
    return np.array([value], "<f4").tobytes()


def corruptions(encoded: bytes, keys: int, values: int, position: int):
    """(name, bytes, identity, expected position, expected outcome)."""
    residual = C.HEADER
    smoothing = residual + keys * values
    scales = smoothing + 4 * keys
    comps = scales + 4 * values
    records = comps + 4 * 4 * (keys + values)
    flipped = bytearray(encoded)
    flipped[len(flipped) // 2] ^= 0x01
    cases = [
        # The reference test's own cases (capsule_test.cpp:304-371).
        ("corrupt", bytes(flipped), IDENTITY, position, C.DIGEST_MISMATCH),
        ("foreign schema", _patched(encoded, 8, b"\x02"), IDENTITY, position, C.PARAMETERS),
        ("residual -128", _patched(encoded, residual, b"\x80"), IDENTITY, position,
         C.RESIDUAL_DOMAIN),
        ("overflow", _patched(_patched(_patched(encoded, residual, b"\x7f", False), smoothing,
                                       _f(np.finfo(np.float32).max), False),
                              scales, _f(np.finfo(np.float32).max)),
         IDENTITY, position, C.STATE_NONFINITE),
        ("generation", encoded, C.Identity("a" * 64, 8, 11), position, C.IDENTITY),
        ("geometry", encoded, C.Identity("b" * 64, 7, 11), position, C.IDENTITY),
        ("phase", encoded, IDENTITY, position - 1 if position else position + 1, C.PHASE),
        # Further checks of Restore, in its order.
        ("too short", encoded[:71], IDENTITY, position, C.TRUNCATED),
        ("magic", _patched(encoded, 0, b"X"), IDENTITY, position, C.MAGIC),
        ("digest case", encoded[:-64] + encoded[-64:].upper(), IDENTITY, position,
         C.DIGEST_ENCODING if encoded[-64:].upper() != encoded[-64:] else C.OK),
        ("epoch", _patched(encoded, 36, b"\x0c"), IDENTITY, position, C.IDENTITY),
        ("rank field", _patched(encoded, 16, b"\x05"), IDENTITY, position, C.PARAMETERS),
        ("floor field", _patched(encoded, 24, _f(2.0e-8)), IDENTITY, position, C.PARAMETERS),
        ("window position 16", _patched(encoded, 52, b"\x10"), IDENTITY, 16, C.POSITION),
        ("truncated record", C.refresh_digest(encoded[:-68] + encoded[-64:]), IDENTITY,
         position, C.TRUNCATED if position else C.TRUNCATED),
        ("trailing", C.refresh_digest(encoded[:-64] + b"\0\0\0\0" + encoded[-64:]),
         IDENTITY, position, C.TRAILING),
        ("header only", C.refresh_digest(encoded[:119] + encoded[-64:]), IDENTITY, position,
         C.TRUNCATED),
        ("smoothing zero", _patched(encoded, smoothing + 4, _f(0.0)), IDENTITY, position,
         C.BOUNDARY_PAYLOAD),
        ("scale negative", _patched(encoded, scales, _f(-1.0)), IDENTITY, position,
         C.BOUNDARY_PAYLOAD),
        ("compensator nan", _patched(encoded, comps + 8, _f(np.nan)), IDENTITY, position,
         C.BOUNDARY_PAYLOAD),
        # Finite, though s * 127 would overflow: only an exact evaluation of
        # DenseState admits it.
        ("large smoothing", _patched(_patched(encoded, residual, b"\x32" * values, False),
                                     smoothing, _f(3.0e36)), IDENTITY, position, C.OK),
    ]
    if position:
        cases.append(("record inf", _patched(encoded, records + 4 * keys, _f(np.inf)),
                      IDENTITY, position, C.RECORD_NONFINITE))
        # A later record's non-finite value loses to an earlier truncation
        # only when that truncation comes first: cut inside the last record.
        nan_first = _patched(encoded, records, _f(np.nan), False)
        cases.append(("record nan then truncated",
                      C.refresh_digest(nan_first[:-68] + nan_first[-64:]), IDENTITY, position,
                      C.RECORD_NONFINITE))
    return cases


def test_restore_rejects_what_the_reference_rejects(hibernated):
    for name, enc, identity, pos, want in corruptions(hibernated, KEYS, VALUES, 7):
        status, _ = C.restore(enc, identity, KEYS, VALUES, pos)
        assert status == want, name
        message, again, _ = C.ref_restore(enc, identity, KEYS, VALUES, pos)
        if want == C.OK:
            assert message is None and again == enc, name
        else:
            assert message is not None, name
            assert C.outcome_of_message(message) == want, (name, message)


def test_invalid_expected_identity_or_parameters_are_argument_errors(hibernated):
    cases = [(C.Identity("A" * 64, 7, 11), {}), (C.Identity("a" * 63 + "g", 7, 11), {}),
             (C.Identity("a" * 64, 0, 11), {}), (C.Identity("a" * 64, 7, 0), {}),
             (IDENTITY, {"window": 8}), (IDENTITY, {"rank": 2}), (IDENTITY, {"bits": 4}),
             (IDENTITY, {"schema": 2}), (IDENTITY, {"floor": np.float32(0.0)})]
    for identity, params in cases:
        status, _ = C.restore(hibernated, identity, KEYS, VALUES, 7, **params)
        assert status == C.ARGUMENT, (identity, params)
        message, _, _ = C.ref_restore(hibernated, identity, KEYS, VALUES, 7, **params)
        assert message is not None, (identity, params)


# ---------------------------------------------------------- slot capsules


def window_dense64(buf, s, layout):
    """The window's dense state [K][V] in float64 and the sum of |terms|."""
    codes = WG.kv_boundary(buf, s, layout).astype(np.float64)
    sm = buf["smoothing"][s].astype(np.float64)
    sc = buf["scales"][s].astype(np.float64)
    ck = W.f16_to_f32(buf["compensator_keys"][s]).astype(np.float64)
    cv = W.f16_to_f32(buf["compensator_values"][s]).astype(np.float64)
    p = int(buf["positions"][s, 0])
    g = buf["record_decay"][s].astype(np.float64)
    rk = W.f16_to_f32(buf["record_keys"][s]).astype(np.float64)
    rc = W.f16_to_f32(buf["record_corrections"][s]).astype(np.float64)
    base = codes / 127.0 * sm[:, None] * sc[None, :] + ck @ cv.T
    size = np.abs(codes) / 127.0 * sm[:, None] * sc[None, :] + np.abs(ck) @ np.abs(cv).T
    dense, mag = base, size
    for j in range(p):
        dense = g[j] * dense + np.outer(rk[j], rc[j])
        mag = g[j] * mag + np.abs(np.outer(rk[j], rc[j]))
    return dense, mag


@pytest.mark.parametrize("layout", [VK, KV])
def test_slot_capsules_are_reference_capsules_of_the_window(layout):
    states = 18
    positions = list(range(16)) + [16, 3]
    buf = WG.window_buffers(states, 71, layout, positions=positions)
    identity = C.Identity("0123456789abcdef" * 4, 3, 9)
    for s in range(states):
        p = positions[s]
        enc = C.slot_serialize(buf, s, layout, identity)
        if p >= 16:
            assert enc == b"" and C.slot_capsule_bytes(p) == 0
            continue
        assert len(enc) == C.slot_capsule_bytes(p) == 21688 + 1536 * p
        message, again, dense = C.ref_restore(enc, identity, 128, 128, p)
        assert message is None and again == enc, (s, message)
        assert dense.tobytes() == WG.capsule_at(buf, s, layout).dense_state().tobytes(), s
        want, mag = window_dense64(buf, s, layout)
        assert (np.abs(dense - want) <= 2.0 ** -18 * mag + 1e-30).all(), s
        # And back into a slot: bit-exact, records beyond p untouched.
        fresh = WG.window_buffers(states, 72, layout, positions=9)
        before = WG.copy_buffers(fresh)
        assert C.slot_restore(enc, fresh, s, layout, identity, p) == C.OK
        for name in ("residual", "smoothing", "scales", "compensator_keys",
                     "compensator_values"):
            assert np.array_equal(fresh[name][s], buf[name][s]), (s, name)
        for name in ("record_decay", "record_keys", "record_corrections"):
            assert np.array_equal(fresh[name][s][:p], buf[name][s][:p]), (s, name)
            assert np.array_equal(fresh[name][s][p:], before[name][s][p:]), (s, name)
        assert fresh["positions"][s, 0] == p
        assert (fresh["positions"][s, 1:] == before["positions"][s, 1:]).all()
        others = [i for i in range(states) if i != s]
        for name in fresh:
            assert np.array_equal(fresh[name][others], before[name][others]), (s, name)


def test_slot_restore_refuses_capsules_outside_the_device_format():
    buf = WG.window_buffers(2, 73, VK, positions=5)
    enc = C.slot_serialize(buf, 0, VK, IDENTITY)
    records = C.HEADER + 128 * 128 + 4 * 256 + 16 * 256
    cases = {
        "decay differs across keys": _patched(enc, records + 4 * 7, _f(0.5)),
        "record key not fp16": _patched(enc, records + 4 * 128 + 4,
                                        _f(np.float32(1.0) + np.float32(2.0 ** -20))),
        "compensator not fp16": _patched(enc, C.HEADER + 128 * 128 + 1024,
                                         _f(np.float32(0.1))),
    }
    for name, bad in cases.items():
        message, again, _ = C.ref_restore(bad, IDENTITY, 128, 128, 5)
        assert message is None and again == bad, name  # a valid capsule ...
        target = WG.copy_buffers(buf)
        status = C.slot_restore(bad, target, 1, VK, IDENTITY, 5)
        assert status == C.DEVICE_FORMAT, name      # ... the slot cannot hold
        for key in buf:
            assert np.array_equal(target[key], buf[key]), (name, key)
    # The reference's own 128x128 capsule carries fp32 rank-4 compensators.
    dense = np.random.default_rng(3).standard_normal((128, 128)).astype(np.float32) * 0.05
    ref_enc = C.ref_capsule_after_tokens(dense, IDENTITY, *(np.zeros((0, 128), np.float32)
                                                            for _ in range(5)))
    assert C.slot_restore(ref_enc, WG.copy_buffers(buf), 0, VK, IDENTITY, 0) == C.DEVICE_FORMAT


def test_slot_restore_reports_the_reference_outcome_for_corruptions():
    buf = WG.window_buffers(1, 74, VK, positions=6)
    enc = C.slot_serialize(buf, 0, VK, IDENTITY)
    for name, bad, identity, pos, want in corruptions(enc, 128, 128, 6):
        target = WG.copy_buffers(buf)
        status = C.slot_restore(bad, target, 0, VK, identity, pos)
        assert status == want, name
        message, _, _ = C.ref_restore(bad, identity, 128, 128, pos)
        assert (message is None) == (want == C.OK), name
        if message is not None:
            assert C.outcome_of_message(message) == want, (name, message)
