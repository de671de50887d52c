"""CPU pins of the windowed decode-step oracle (oracle/gdn_window_oracle.c).

* The capsule layer (ReadWindowState, ApplyToken, DenseState) must equal the
  reference capsule compiled from its sources (oracle/_ref) bit for bit.
* Each device-format step must equal the capsule applied to the same state
  under the entry point's documented input mapping (the reference kernel lines
  cited per test), bit for bit before the final fp16/bf16 rounding.
* The double-precision results and error scales the GPU tests use must agree
  with the fp32 results within that scale, and the dense fp32 step must agree
  with the windowed step on the reconstructed state, as the reference's own
  device probe checks (windowed_gdn_runtime_probe.cpp:94-147, 346-349).
"""

from __future__ import annotations

import numpy as np
import pytest

import datagen
import oracle
import windowgen as WG
from oracle import window as W

KV, VK = oracle.LAYOUT_KEY_VALUE, oracle.LAYOUT_VALUE_KEY
needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")


def ulp(x, mantissa_bits: int, min_exponent: int = -24):
    """Spacing of a binary format with `mantissa_bits` stored bits around x."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -300)))
    return 2.0 ** np.maximum(e - mantissa_bits, min_exponent)


def _tokens(count: int, seed: int):
    g = datagen.rng(seed)
    decay = (0.9 + 0.1 * g.random((count, 128))).astype(np.float32)
    key = (g.standard_normal((count, 128)) * 0.1).astype(np.float32)
    read = (decay * key).astype(np.float32)
    query = (g.standard_normal((count, 128)) * 0.1).astype(np.float32)
    value = (g.standard_normal((count, 128)) * 0.5).astype(np.float32)
    return decay, key, value, read, query


def test_fp16_conversions_round_to_nearest_even():
    g = datagen.rng(1)
    x = np.concatenate([
        g.standard_normal(4000).astype(np.float32) * np.float32(10.0) ** g.integers(-9, 5, 4000),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
                  3 * 2.0 ** -26, 2.0 ** -14 - 2.0 ** -25, np.inf, -np.inf], np.float32)])
    with np.errstate(over="ignore"):
        expected = x.astype(np.float16)
    ours = W.f32_to_f16(x)
    assert ours.tobytes() == expected.view(np.uint16).tobytes()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    finite = (bits & 0x7C00) != 0x7C00
    widened = np.array([W._l().gdn_oracle_f16_to_f32(int(b)) for b in bits[finite]], np.float32)
    assert widened.tobytes() == bits[finite].view(np.float16).astype(np.float32).tobytes()


@needs_ref
@pytest.mark.parametrize("rank", [0, 4])
@pytest.mark.parametrize("records", [0, 1, 7, 16])
def test_read_window_matches_reference(rank, records):
    dense = datagen.c1_heads(1, 20 + records)[0]
    codes, s, sc, ck, cv = oracle.quantize_kv(dense, rank)
    decay, key, value, read, _ = _tokens(max(records, 1), 30 + rank)
    ck = ck if rank else None
    cv = cv if rank else None
    ours = W.read_window(codes, s, sc, read[0], decay[:records], key[:records],
                         value[:records], ck, cv)
    theirs = W.ref_read_window(codes, s, sc, read[0], decay[:records], key[:records],
                               value[:records], ck, cv)
    assert ours.tobytes() == theirs.tobytes()


@needs_ref
def test_apply_token_matches_reference_capsule_across_two_windows():
    dense = datagen.c1_heads(1, 11)[0]
    decay, key, value, read, query = _tokens(40, 3)
    ref_out, ref_crossed, ref_final = W.ref_apply_tokens(dense, 4, decay, key, value, read, query)
    cap = W.CapsuleWindow(dense, 4)
    outs, crossed = [], []
    for t in range(40):
        o, c = cap.apply(decay[t], key[t], value[t], read[t], query[t])
        outs.append(o)
        crossed.append(c)
    assert np.stack(outs).tobytes() == ref_out.tobytes()
    assert crossed == ref_crossed.tolist()
    assert np.flatnonzero(ref_crossed).tolist() == [15, 31]
    assert cap.dense_state().tobytes() == ref_final.tobytes()


@pytest.mark.parametrize("quant_only", [False, True])
def test_bf16_step_equals_capsule_under_device_mapping(quant_only):
    """windowed_gdn_step.cpp:344-455 maps a bf16 step onto ApplyToken with
    decay = g = exp(log_decay) (per key), key = beta*k, read = g*k,
    query = 0.08838834764831845*q, value = v; value head h reads k/q head h/2."""
    states = 12
    buf = WG.window_buffers(states, 5, VK, positions=[0, 1, 2, 3, 5, 8, 13, 15, 16, 17, 0, 9],
                            compensated=not quant_only)
    inp = WG.bf16_inputs(states, 6)
    before = WG.copy_buffers(buf)
    outputs, *_ = W.windowed_step_bf16(buf, **inp, quant_only=quant_only)
    for s in range(states):
        p = int(before["positions"][s, 0])
        if p >= 16:
            for name in W.WINDOW_BUFFERS:
                assert np.array_equal(buf[name][s], before[name][s]), (s, name)
            assert not outputs[s].any()
            continue
        cap = WG.capsule_at(before, s, VK, rank=0 if quant_only else 4)
        g = np.float32(np.exp(np.float64(inp["log_decay"][s])))
        k = oracle.bf16_to_f32(inp["keys"][s // 2])
        q = (np.float32(0.08838834764831845) * oracle.bf16_to_f32(inp["queries"][s // 2])).astype(np.float32)
        b = oracle.bf16_to_f32(inp["beta"][s:s + 1])[0]
        key = (b * k).astype(np.float32)
        read = (g * k).astype(np.float32)
        out, _ = cap.apply(np.full(128, g, np.float32), key,
                           oracle.bf16_to_f32(inp["values"][s]), read, q)
        corr = cap.record_corrections[p]
        assert outputs[s].tobytes() == oracle.f32_to_bf16(out).tobytes(), s
        assert buf["record_corrections"][s, p].tobytes() == W.f32_to_f16(corr).tobytes(), s
        assert buf["record_keys"][s, p].tobytes() == W.f32_to_f16(key).tobytes(), s
        assert buf["record_decay"][s, p] == g
        assert buf["positions"][s, 0] == p + 1
        assert (buf["positions"][s, 1:] == 0xA5A5A5A5).all()


def test_f16_step_equals_capsule_under_device_mapping():
    """windowed_gdn_step.cpp:80-176: decay is linear, read / write key / query
    are taken as given, outputs stay fp32, the record key is the write key."""
    states = 8
    buf = WG.window_buffers(states, 7, KV, positions=[0, 1, 4, 7, 11, 15, 16, 3])
    inp = WG.f16_inputs(states, 8)
    before = WG.copy_buffers(buf)
    outputs, *_ = W.windowed_step_f16(buf, **inp)
    for s in range(states):
        p = int(before["positions"][s, 0])
        if p >= 16:
            assert not outputs[s].any()
            continue
        cap = WG.capsule_at(before, s, KV)
        d = inp["decay"][s]
        out, _ = cap.apply(np.full(128, d, np.float32), W.f16_to_f32(inp["write_keys"][s]),
                           W.f16_to_f32(inp["values"][s]), W.f16_to_f32(inp["reads"][s]),
                           W.f16_to_f32(inp["queries"][s]))
        assert outputs[s].tobytes() == out.tobytes(), s
        assert buf["record_keys"][s, p].tobytes() == inp["write_keys"][s].tobytes()
        assert buf["record_corrections"][s, p].tobytes() == W.f32_to_f16(cap.record_corrections[p]).tobytes()
        assert buf["record_decay"][s, p] == d and buf["positions"][s, 0] == p + 1


def test_double_results_bound_the_fp32_results():
    states = 16
    buf = WG.window_buffers(states, 9, VK)
    inp = WG.bf16_inputs(states, 10)
    b2 = WG.copy_buffers(buf)
    outputs, out64, out_bound, corr64, corr_bound = W.windowed_step_bf16(b2, **inp)
    live = buf["positions"][:, 0] < 16
    # bf16 output within half a bf16 ulp of the double result (+ fp32 error).
    got = oracle.bf16_to_f32(outputs).astype(np.float64)
    assert (np.abs(got - out64)[live] <= 0.5 * ulp(out64, 7)[live]
            + 2.0 ** -16 * out_bound[live]).all()
    # fp16 corrections likewise.
    pos = buf["positions"][:, 0]
    for s in np.flatnonzero(live):
        c = W.f16_to_f32(b2["record_corrections"][s, pos[s]]).astype(np.float64)
        assert (np.abs(c - corr64[s]) <= 0.5 * ulp(corr64[s], 10)
                + 2.0 ** -16 * corr_bound[s]).all()


def test_dense_fp32_step_agrees_with_windowed_step_on_reconstructed_state():
    """The reference probe's check: reconstruct the dense state from boundary,
    compensators and records, run the dense fp32 step, compare outputs."""
    states = 6
    buf = WG.window_buffers(states, 11, KV, positions=[0, 3, 6, 9, 12, 15])
    inp = WG.f16_inputs(states, 12)
    dense = np.stack([
        W.CapsuleWindow.dense_state(WG.capsule_at(buf, s, KV)) for s in range(states)])
    out_dense = W.gdn_step_f32(dense, inp["decay"], inp["write_keys"], inp["reads"],
                               inp["queries"], inp["values"])
    b2 = WG.copy_buffers(buf)
    out, out64, out_bound, _, _ = W.windowed_step_f16(b2, **inp)
    err = np.abs(out_dense.astype(np.float64) - out64)
    assert (err <= 2.0 ** -12 * out_bound).all(), (err / out_bound).max()
    assert (np.abs(out - out64) <= 2.0 ** -16 * out_bound).all()


def test_decode_pair_chain_matches_windowed_step_within_vector_quantization():
    """prepare_decode_pair_bf16 -> int8 matmul -> finish_decode_pair_bf16 is the
    bf16 step with the read and output vectors x*s held as hi/lo int8 pairs;
    its error is at most half a low step per element, times sum |code|."""
    states = 16
    buf = WG.window_buffers(states, 13, VK)
    inp = WG.bf16_inputs(states, 14)
    quantized, dyn = W.prepare_decode_pair_bf16(inp["keys"], inp["queries"], inp["log_decay"],
                                                buf["smoothing"])
    assert not quantized[:, :, 4:].any()
    projected = W.int8_matmul(buf["residual"], quantized)
    exact = np.einsum("svk,skc->svc", buf["residual"].astype(np.int64), quantized.astype(np.int64))
    assert np.array_equal(projected, exact)
    chain = WG.copy_buffers(buf)
    out_chain = W.finish_decode_pair_bf16(chain, projected, dyn, **inp)
    direct = WG.copy_buffers(buf)
    _, out64, out_bound, _, _ = W.windowed_step_bf16(direct, **inp)
    for name in ("record_keys", "record_decay", "positions"):
        assert np.array_equal(chain[name], direct[name]), name
    abs_codes = np.abs(buf["residual"].astype(np.float64)).sum(axis=2)  # [S][V]
    suffix = np.ones(states)
    for s in range(states):
        for j in range(int(buf["positions"][s, 0])):
            suffix[s] *= buf["record_decay"][s, j]
    scale = buf["scales"] / 127.0 * suffix[:, None]
    beta = oracle.bf16_to_f32(inp["beta"]).astype(np.float64)
    qk = np.abs(oracle.bf16_to_f32(inp["keys"]).astype(np.float64) * 0.0884 *
                oracle.bf16_to_f32(inp["queries"])).sum(axis=1).repeat(2)
    e_read = 0.5 * dyn[:, 2:3] * abs_codes * scale
    e_out = 0.5 * dyn[:, 3:4] * abs_codes * scale
    bound = e_out + (beta * qk)[:, None] * e_read + 2.0 ** -14 * out_bound
    got = oracle.bf16_to_f32(out_chain).astype(np.float64)
    live = buf["positions"][:, 0] < 16
    tol = bound + 0.5 * ulp(out64 + bound, 7)
    assert (np.abs(got - out64)[live] <= tol[live]).all()


def test_int8_split_rounds_by_the_float_half_add():
    """The oracle's hi/lo split (prepare_decode_pair) against codes derived by
    hand from the reference's rounding on inputs at its edges: .5 ties round
    away from zero, and 0.5 - 2^-25 rounds up because the float add itself
    rounds.  Round-half-even (np.rint) and exact round-half-away (lround) both
    give different codes on these rows, so either slip fails this test."""
    x, s, hi, lo, lo_scale = WG.split_tie_state()
    f16 = x.astype(np.float16)
    assert np.array_equal(f16.astype(np.float32), x)  # every input is exact in fp16
    reads = f16.view(np.uint16)[None]
    q, dyn = W.prepare_decode_pair(reads, reads, np.ones(1, np.float32), s[None])
    for c in range(2):  # both vectors of the pair: the read and the output side
        assert np.array_equal(q[0, :, 2 * c], hi)
        assert np.array_equal(q[0, :, 2 * c + 1], lo)
        assert dyn[0, c] == np.float32(0.125)
        assert dyn[0, 2 + c] == lo_scale
    assert not q[0, :, 4:].any()
    exact = (x.astype(np.float64) * s) / 0.125
    assert not np.array_equal(np.rint(exact).astype(np.int8), hi)        # ties-to-even
    assert not np.array_equal((np.sign(exact) * np.floor(np.abs(exact) + 0.5)).clip(-127, 127)
                              .astype(np.int8), hi)                      # exact half-away


def test_int8_vector_rounds_by_the_float_half_add():
    """prepare_int8_vector (encoded_projection.cpp:179-234) on the same edge
    inputs, column 0 of an fp16 [128][16] operand: one level, the hi codes."""
    x, s, hi, _, _ = WG.split_tie_state()
    operand = np.zeros((1, 128, 16), np.float16)
    operand[0, :, 0] = x.astype(np.float16)
    q, dyn = W.prepare_int8_vector(operand.view(np.uint16), s[None])
    assert np.array_equal(q[0, :, 0], hi)
    assert not q[0, :, 1:].any()
    assert dyn[0, 0] == np.float32(0.125)
