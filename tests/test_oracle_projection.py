"""Pins of the projection oracle (oracle.project_decode / project_chunked):
the GQA map (value head h reads query head h // (H / Hq), Qwen's consecutive
pairs, kernel/gdn_state_codec_windowed_gdn_step.cpp:340), the [value][key]
tile indexing and the batch / token strides, at B = 3, H = 32, Hq = 16 in both
layouts.  Three independent checks:

* a float64 brute force written directly from the reference's boundary
  readout (native/src/gdn_state_codec_state_capsule.cpp:281-290) with explicit
  indexing: q[b, h // 2] and an explicit transpose of a [value][key] tile;
* the reference's own golden readouts (tests/golden, written by the reference's
  ReadWindowState) tiled into a batch so that both heads of a GQA pair carry
  the same golden head, in both layouts, bit for bit;
* where oracle/_ref is built, the reference's ReadWindowState per head on
  reads and [key][value] tiles assembled here, bit for bit.

Negative controls show each check rejects a plausible slip: an h % Hq map, an
untransposed [value][key] tile, a dropped smoothing factor.  A mutated copy of
the oracle's C source (wrong GQA map, transposed operand) fails them too."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle

KV, VK = oracle.LAYOUT_KEY_VALUE, oracle.LAYOUT_VALUE_KEY
B, H, HQ, T = 3, 32, 16, 3
QSCALE = np.float32(0.08838834764831845)
ORACLE_SOURCE = Path(oracle.__file__).resolve().parent / "gdn_oracle.c"


def _encoded(shape, seed):
    rng = np.random.default_rng(seed)
    codes = rng.integers(-127, 128, size=shape + (128, 128), dtype=np.int64).astype(np.int8)
    smoothing = (0.5 + rng.random(shape + (128,))).astype(np.float32) * np.float32(0.03)
    scales = (0.5 + rng.random(shape + (128,))).astype(np.float32) * np.float32(2.0)
    return codes, smoothing, scales


def _queries(shape, seed):
    rng = np.random.default_rng(seed)
    return oracle.f32_to_bf16(rng.standard_normal(shape).astype(np.float32))


def _x(q_bits, qscale):
    """The fp32 read vector the readout sees: query_scale * bf16 -> fp32."""
    return (np.float32(qscale) * oracle.bf16_to_f32(q_bits)).astype(np.float64)


def brute_readout(codes, smoothing, scales, x, layout, transpose=True, drop_smoothing=False):
    """out[v] = sum_k code[k][v] * s[k] * x[k] / 127 * scale[v] in float64 for
    one tile; a [value][key] tile is transposed explicitly."""
    tile = codes.astype(np.float64)
    key_value = tile.T if (layout == VK and transpose) else tile
    s = np.ones(128) if drop_smoothing else smoothing.astype(np.float64)
    terms = key_value * (s * x)[:, None]
    scale = scales.astype(np.float64) / 127.0
    return terms.sum(axis=0) * scale, np.abs(terms).sum(axis=0) * scale


def brute_decode(codes, smoothing, scales, q_bits, layout, qscale, gqa=None, **kw):
    heads, qheads = codes.shape[1], q_bits.shape[1]
    gqa = gqa or (lambda h: h // (heads // qheads))
    out = np.empty(codes.shape[:2] + (128,))
    mag = np.empty_like(out)
    for b in range(codes.shape[0]):
        for h in range(heads):
            out[b, h], mag[b, h] = brute_readout(codes[b, h], smoothing[b, h], scales[b, h],
                                                 _x(q_bits[b, gqa(h)], qscale), layout, **kw)
    return out, mag


def brute_chunked(codes, smoothing, scales, q_bits, layout, qscale, gqa=None, **kw):
    seqs, heads = codes.shape[:2]
    tokens, qheads = q_bits.shape[1:3]
    gqa = gqa or (lambda h: h // (heads // qheads))
    out = np.empty((seqs, tokens, heads, 128))
    mag = np.empty_like(out)
    for n in range(seqs):
        for t in range(tokens):
            for h in range(heads):
                out[n, t, h], mag[n, t, h] = brute_readout(
                    codes[n, h], smoothing[n, h], scales[n, h], _x(q_bits[n, t, gqa(h)], qscale),
                    layout, **kw)
    return out, mag


def within(got32, exact, magnitude):
    """An fp32 sequential sum of 128 terms lies within 2^-15 * sum|terms|."""
    return np.abs(got32.astype(np.float64) - exact) <= 2.0 ** -15 * magnitude + 1e-30


@pytest.mark.parametrize("layout", [KV, VK])
def test_decode_oracle_matches_brute_force(layout):
    codes, s, sc = _encoded((B, H), 1 + layout)
    q = _queries((B, HQ, 128), 3 + layout)
    out32, out64, bound = oracle.project_decode(codes, s, sc, q, QSCALE, layout)
    exact, magnitude = brute_decode(codes, s, sc, q, layout, QSCALE)
    assert np.allclose(out64, exact, rtol=1e-12, atol=1e-12 * magnitude.max())
    assert np.allclose(bound, magnitude, rtol=1e-12)
    assert within(out32, exact, magnitude).all()
    # Negative controls: each plausible slip moves some output far outside the bound.
    for slip in (dict(gqa=lambda h: h % HQ), dict(drop_smoothing=True)) + (
            (dict(transpose=False),) if layout == VK else ()):
        wrong, _ = brute_decode(codes, s, sc, q, layout, QSCALE, **slip)
        assert not within(out32, wrong, magnitude).all(), slip


@pytest.mark.parametrize("layout", [KV, VK])
def test_chunked_oracle_matches_brute_force(layout):
    codes, s, sc = _encoded((B, H), 5 + layout)
    q = _queries((B, T, HQ, 128), 7 + layout)
    out32, out64, bound = oracle.project_chunked(codes, s, sc, q, QSCALE, layout)
    exact, magnitude = brute_chunked(codes, s, sc, q, layout, QSCALE)
    assert np.allclose(out64, exact, rtol=1e-12, atol=1e-12 * magnitude.max())
    assert np.allclose(bound, magnitude, rtol=1e-12)
    assert within(out32, exact, magnitude).all()
    for slip in (dict(gqa=lambda h: h % HQ), dict(drop_smoothing=True)) + (
            (dict(transpose=False),) if layout == VK else ()):
        wrong, _ = brute_chunked(codes, s, sc, q, layout, QSCALE, **slip)
        assert not within(out32, wrong, magnitude).all(), slip


def _golden_batch(golden, layout):
    """B x H tiles of golden heads: value heads 2j, 2j+1 of sequence b both
    carry golden head (b * 16 + j) mod 9 and query head j its query, so each
    expected output is that head's reference readout."""
    names = [str(n) for n in golden["names"]]
    pick = [[names[(b * HQ + h // 2) % len(names)] for h in range(H)] for b in range(B)]
    codes = np.stack([[golden[f"{n}/codes"] for n in row] for row in pick])
    if layout == VK:
        codes = np.ascontiguousarray(codes.swapaxes(-1, -2))
    s = np.stack([[golden[f"{n}/smoothing"] for n in row] for row in pick])
    sc = np.stack([[golden[f"{n}/scales"] for n in row] for row in pick])
    q = np.stack([[golden[f"{names[(b * HQ + j) % len(names)]}/query_bf16"] for j in range(HQ)]
                  for b in range(B)])
    want = np.stack([[golden[f"{n}/readout"] for n in row] for row in pick])
    return codes, s, sc, q, want


@pytest.mark.parametrize("layout", [KV, VK])
def test_decode_oracle_reproduces_golden_readouts_in_a_batch(golden, layout):
    codes, s, sc, q, want = _golden_batch(golden, layout)
    out32, _, _ = oracle.project_decode(codes, s, sc, q, 1.0, layout)
    assert out32.tobytes() == want.astype(np.float32).tobytes()
    # An h % Hq map: one query per value head (group 1), value head h given
    # query head h % 16, which differs from h // 2 from head 2 on.
    wrong = oracle.project_decode(codes, s, sc, np.ascontiguousarray(q[:, np.arange(H) % HQ]),
                                  1.0, layout)[0]
    assert wrong.tobytes() != want.astype(np.float32).tobytes()


@pytest.mark.parametrize("layout", [KV, VK])
def test_chunked_oracle_reproduces_golden_readouts_in_a_batch(golden, layout):
    codes, s, sc, q, want = _golden_batch(golden, layout)
    tokens = np.stack([q, q[::-1]], axis=1)  # token 1 of sequence b uses sequence 2-b's queries
    out32, _, _ = oracle.project_chunked(codes, s, sc, tokens, 1.0, layout)
    assert out32[:, 0].tobytes() == want.astype(np.float32).tobytes()
    flipped, _, _ = oracle.project_decode(codes, s, sc, np.ascontiguousarray(q[::-1]), 1.0, layout)
    assert out32[:, 1].tobytes() == flipped.tobytes()


def _ref_outputs(codes, s, sc, reads, layout):
    """The reference's ReadWindowState per head: [key][value] tiles assembled
    here (an explicit transpose of [value][key] tiles) and fp32 reads."""
    kv = codes if layout == KV else np.ascontiguousarray(codes.swapaxes(-1, -2))
    heads = kv.shape[0] * kv.shape[1]
    return oracle.ref_read_boundary_heads(kv.reshape(heads, 128, 128), s.reshape(heads, 128),
                                          sc.reshape(heads, 128),
                                          reads.reshape(heads, -1, 128).astype(np.float32))


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (needs the reference)")
@pytest.mark.parametrize("layout", [KV, VK])
def test_decode_oracle_is_bit_exact_with_the_reference_readout(layout):
    codes, s, sc = _encoded((B, H), 11 + layout)
    q = _queries((B, HQ, 128), 13 + layout)
    out32, _, _ = oracle.project_decode(codes, s, sc, q, QSCALE, layout)
    reads = np.stack([[_x(q[b, h // 2], QSCALE) for h in range(H)] for b in range(B)])
    ref = _ref_outputs(codes, s, sc, reads, layout).reshape(B, H, 128)
    assert out32.tobytes() == ref.tobytes()


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (needs the reference)")
@pytest.mark.parametrize("layout", [KV, VK])
def test_chunked_oracle_is_bit_exact_with_the_reference_readout(layout):
    codes, s, sc = _encoded((B, H), 17 + layout)
    q = _queries((B, T, HQ, 128), 19 + layout)
    out32, _, _ = oracle.project_chunked(codes, s, sc, q, QSCALE, layout)
    reads = np.stack([[[_x(q[n, t, h // 2], QSCALE) for t in range(T)] for h in range(H)]
                      for n in range(B)])  # [N][H][T][128]
    ref = _ref_outputs(codes, s, sc, reads, layout).reshape(B, H, T, 128)
    assert out32.tobytes() == np.ascontiguousarray(ref.transpose(0, 2, 1, 3)).tobytes()


MUTATIONS = {
    "gqa_modulo": ("h * query_heads / value_heads", "h % query_heads"),
    "transposed_operand": (": codes[v * TILE_DIM + k]", ": codes[k * TILE_DIM + v]"),
}


@pytest.mark.parametrize("mutation", sorted(MUTATIONS))
def test_a_mutated_oracle_fails_the_pins(tmp_path, mutation):
    """Plant the mistake in a copy of the oracle's C source, build it, and show
    the brute-force pin rejects its outputs."""
    old, new = MUTATIONS[mutation]
    source = ORACLE_SOURCE.read_text()
    assert source.count(old) >= 1, f"mutation anchor {old!r} not found in gdn_oracle.c"
    mutated = tmp_path / "gdn_oracle_mutant.c"
    mutated.write_text(source.replace(old, new))
    library = tmp_path / "libmutant.so"
    subprocess.run(["gcc", "-std=c11", "-O2", "-ffp-contract=off", "-fPIC", "-shared",
                    "-pthread", f"-I{ORACLE_SOURCE.parent}", str(mutated), "-o", str(library),
                    "-lm"], check=True)
    lib = ctypes.CDLL(str(library))
    fn = lib.gdn_oracle_project_decode
    fn.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_uint32] * 3 + [ctypes.c_float,
                                                                    ctypes.c_uint32] + [
        ctypes.c_void_p] * 3
    fn.restype = None
    layout = VK
    codes, s, sc = _encoded((B, H), 23)
    q = _queries((B, HQ, 128), 29)
    out = np.empty((B, H, 128), np.float32)
    fn(codes.ctypes.data, s.ctypes.data, sc.ctypes.data, q.ctypes.data, B, H, HQ, QSCALE,
       layout, out.ctypes.data, None, None)
    exact, magnitude = brute_decode(codes, s, sc, q, layout, QSCALE)
    assert not within(out, exact, magnitude).all()
