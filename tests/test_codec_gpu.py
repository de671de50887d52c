"""GPU parity of the codec entry points: bit-exact against the reference's
golden outputs and against the C oracle, through the C-ABI."""

import ctypes
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import datagen
import oracle
from gdn_state_codec import codec, native

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"
KV, VK = codec.LAYOUT_KEY_VALUE, codec.LAYOUT_VALUE_KEY


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def to_gpu(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def to_np(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def stream():
    return torch.cuda.current_stream().cuda_stream


def _stack_golden(golden):
    names = list(golden["names"])
    x = np.stack([golden[f"{n}/input"] for n in names])
    codes = np.stack([golden[f"{n}/codes"] for n in names])
    s = np.stack([golden[f"{n}/smoothing"] for n in names])
    sc = np.stack([golden[f"{n}/scales"] for n in names])
    return names, x, codes, s, sc


@pytest.mark.parametrize("layout", [KV, VK])
def test_encode_v4_matches_reference_golden(device, golden, layout):
    names, x, codes, s, sc = _stack_golden(golden)
    if layout == VK:
        x = x.transpose(0, 2, 1)
    c_gpu, s_gpu, sc_gpu = codec.encode(to_gpu(x, device), layout)
    got = to_np(c_gpu)
    if layout == VK:
        got = got.transpose(0, 2, 1)
    for i, name in enumerate(names):
        print(f"encode golden layout={layout} head={name}", flush=True)
        assert got[i].tobytes() == codes[i].tobytes(), name
        assert to_np(s_gpu)[i].tobytes() == s[i].tobytes(), name
        assert to_np(sc_gpu)[i].tobytes() == sc[i].tobytes(), name


@pytest.mark.parametrize("layout", [KV, VK])
def test_decode_v4_matches_reference_golden(device, golden, layout):
    names, _, codes, s, sc = _stack_golden(golden)
    summary = json.loads((GOLDEN / "codec_heads.json").read_text())
    if layout == VK:
        codes = codes.transpose(0, 2, 1)
    dense = to_np(codec.decode(to_gpu(codes, device), to_gpu(s, device), to_gpu(sc, device),
                               layout))
    if layout == VK:
        dense = dense.transpose(0, 2, 1)
    for i, name in enumerate(names):
        assert sha(dense[i]) == summary[name]["dequant_sha256"], name


def test_reference_v1_entry_points_match_golden(device, golden):
    lib = native()
    summary = json.loads((GOLDEN / "codec_heads.json").read_text())
    for name in golden["names"]:
        print(f"v1 head={name}", flush=True)
        x = to_gpu(golden[f"{name}/input"], device)
        s = torch.empty(128, dtype=torch.float32, device=device)
        assert lib.smoothing_launch_v1(stream(), x.data_ptr(), s.data_ptr()) == 0
        assert to_np(s).tobytes() == golden[f"{name}/smoothing"].tobytes(), name
        codes = torch.empty((128, 128), dtype=torch.int8, device=device)
        sc = torch.empty(128, dtype=torch.float32, device=device)
        assert lib.quantize_launch_v1(stream(), x.data_ptr(), s.data_ptr(), codes.data_ptr(),
                                      sc.data_ptr()) == 0
        assert to_np(codes).tobytes() == golden[f"{name}/codes"].tobytes(), name
        assert to_np(sc).tobytes() == golden[f"{name}/scales"].tobytes(), name
        zeros = torch.zeros((128, 4), dtype=torch.float32, device=device)
        dense = torch.empty((128, 128), dtype=torch.float32, device=device)
        assert lib.dequantize_launch_v1(stream(), codes.data_ptr(), s.data_ptr(), sc.data_ptr(),
                                        zeros.data_ptr(), zeros.data_ptr(),
                                        dense.data_ptr()) == 0
        # rank-4 zero compensators add 0*0 four times, as the reference's
        # quant_only boundary does; equal to the rank-0 dequant up to -0 -> +0.
        got = to_np(dense)
        expect = oracle.dequantize_kv(golden[f"{name}/codes"], golden[f"{name}/smoothing"],
                                      golden[f"{name}/scales"], np.zeros((128, 4), np.float32),
                                      np.zeros((128, 4), np.float32))
        assert got.tobytes() == expect.tobytes(), name


def test_dequantize_v1_with_rank4_compensators(device, golden):
    lib = native()
    summary = json.loads((GOLDEN / "codec_heads.json").read_text())
    for name in ("c1_style", "student_t"):
        args = [to_gpu(golden[f"{name}/rank4_{k}"], device)
                for k in ("codes", "smoothing", "scales", "comp_keys", "comp_values")]
        dense = torch.empty((128, 128), dtype=torch.float32, device=device)
        assert lib.dequantize_launch_v1(stream(), *[a.data_ptr() for a in args],
                                        dense.data_ptr()) == 0
        assert sha(to_np(dense)) == summary[name]["rank4_dequant_sha256"], name


def test_provider_v2_split_and_v3_fused_match_reference(device, golden):
    lib = native()
    names, x, codes, s, sc = _stack_golden(golden)
    provider = to_gpu(x.transpose(0, 2, 1), device)
    heads = provider.shape[0]
    s2 = torch.empty((heads, 128), dtype=torch.float32, device=device)
    c2 = torch.empty(provider.shape, dtype=torch.int8, device=device)
    sc2 = torch.empty((heads, 128), dtype=torch.float32, device=device)
    assert lib.provider_smoothing_launch_v2(stream(), provider.data_ptr(), s2.data_ptr(),
                                            heads) == 0
    assert lib.provider_quantize_launch_v2(stream(), provider.data_ptr(), s2.data_ptr(),
                                           c2.data_ptr(), sc2.data_ptr(), heads) == 0
    s3 = torch.empty_like(s2)
    c3 = torch.empty_like(c2)
    sc3 = torch.empty_like(sc2)
    assert lib.provider_initialize_launch_v3(stream(), provider.data_ptr(), s3.data_ptr(),
                                             c3.data_ptr(), sc3.data_ptr(), heads) == 0
    expect_codes = np.ascontiguousarray(codes.transpose(0, 2, 1))
    for got_c, got_s, got_sc in ((c2, s2, sc2), (c3, s3, sc3)):
        assert to_np(got_c).tobytes() == expect_codes.tobytes()
        assert to_np(got_s).tobytes() == s.tobytes()
        assert to_np(got_sc).tobytes() == sc.tobytes()


def test_config1_round_trip_matches_reference_digests(device):
    d = json.loads((GOLDEN / "c1_digests.json").read_text())
    x = datagen.c1_heads(32, d["seed"])
    assert sha(x) == d["input_sha256"]
    codes, s, sc = codec.encode(to_gpu(x, device), KV)
    assert sha(to_np(codes)) == d["codes_sha256"]
    assert sha(to_np(s)) == d["smoothing_sha256"]
    assert sha(to_np(sc)) == d["scales_sha256"]
    dense = codec.decode(codes, s, sc, KV)
    assert sha(to_np(dense)) == d["dequant_sha256"]


@pytest.mark.parametrize("layout", [KV, VK])
@pytest.mark.parametrize("kind", ["c1", "student_t", "wide", "tiny_and_huge", "tiny_value",
                                  "requantize"])
def test_encode_decode_match_oracle_on_random_heads(device, layout, kind):
    print(f"random parity layout={layout} kind={kind}", flush=True)
    if kind == "c1":
        x = datagen.c1_heads(384, 5)
    elif kind == "student_t":
        x = datagen.student_t_heads(384, 6, zero_fraction=0.02)
    elif kind == "wide":
        x = np.stack([datagen.wide_range_head(100 + i) for i in range(48)])
    elif kind == "tiny_and_huge":
        x = np.stack([datagen.tiny_head(200 + i) for i in range(24)]
                     + [datagen.huge_head(300 + i) for i in range(24)])
    elif kind == "tiny_value":
        axis = 1 if layout == KV else 0
        x = np.stack([datagen.tiny_value_head(350 + i, axis) for i in range(16)])
    else:
        # A window boundary re-encodes dequantized states: every code 0 became
        # an exact zero.  Half of those zeros are made -0.
        x = datagen.student_t_heads(256, 7)
        x = oracle.decode_heads(*oracle.encode_heads(x, layout, threads=8), layout, threads=8)
        zeros = np.flatnonzero(x == 0)
        assert zeros.size > 0
        x.reshape(-1)[zeros[::2]] = -0.0
    codes, s, sc = oracle.encode_heads(x, layout, threads=8)
    c_gpu, s_gpu, sc_gpu = codec.encode(to_gpu(x, device), layout)
    assert to_np(c_gpu).tobytes() == codes.tobytes()
    assert to_np(s_gpu).tobytes() == s.tobytes()
    assert to_np(sc_gpu).tobytes() == sc.tobytes()
    dense = oracle.decode_heads(codes, s, sc, layout, threads=8)
    assert to_np(codec.decode(c_gpu, s_gpu, sc_gpu, layout)).tobytes() == dense.tobytes()


def test_decode_v4_with_compensators_matches_oracle(device):
    g = datagen.rng(77)
    x = datagen.c1_heads(16, 8)
    codes, s, sc = oracle.encode_heads(x, KV)
    ck = (g.standard_normal((16, 128, 4)) * 0.01).astype(np.float32)
    cv = (g.standard_normal((16, 128, 4)) * 0.01).astype(np.float32)
    got = to_np(codec.decode(to_gpu(codes, device), to_gpu(s, device), to_gpu(sc, device), KV,
                             to_gpu(ck, device), to_gpu(cv, device)))
    for h in range(16):
        expect = oracle.dequantize_kv(codes[h], s[h], sc[h], ck[h], cv[h])
        assert got[h].tobytes() == expect.tobytes(), h


def test_encode_is_deterministic_and_leaves_input_untouched(device):
    x = to_gpu(datagen.c1_heads(64, 9), device)
    before = x.clone()
    a = codec.encode(x, KV)
    b = codec.encode(x, KV)
    torch.cuda.synchronize()
    assert torch.equal(x, before)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


def test_full_config2_shape_properties(device):
    """BASELINE config 2 at full size ([30,256,32,128,128] fp32): codes within
    +-127, every live column reaches 127, round-trip error within half a code
    step s*scale/127 (plus 2e-4 of it for the six fp32 roundings of the
    encode/decode chain, at most 6 * 127 * 2^-24 of a step), and 64 sampled
    heads bit-exact against the oracle."""
    print("full config-2 properties", flush=True)
    shape = (30, 256, 32, 128, 128)
    gen = torch.Generator(device=device)
    gen.manual_seed(1234)
    state = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    state.mul_(0.05)
    codes, s, sc = codec.encode(state, KV)
    dense = codec.decode(codes, s, sc, KV)
    torch.cuda.synchronize()
    flat_codes = codes.view(-1, 128, 128)
    flat_sc = sc.view(-1, 128)
    flat_s = s.view(-1, 128)
    for layer in range(shape[0]):  # one layer at a time bounds the temporaries
        rows = slice(layer * 8192, (layer + 1) * 8192)
        c = flat_codes[rows]
        assert int(c.min()) >= -127 and int(c.max()) <= 127
        live_max = c.abs().amax(dim=1)  # [tiles, value]
        assert bool(((live_max == 127) | (flat_sc[rows] == 0)).all())
        step = flat_s[rows].view(-1, 128, 1) * flat_sc[rows].view(-1, 1, 128) / 127
        err = (dense.view(-1, 128, 128)[rows] - state.view(-1, 128, 128)[rows]).abs_()
        assert bool((err <= 0.5 * step * (1 + 2e-4) + 1e-30).all()), layer
        del step, err, live_max
    idx = torch.randint(0, flat_codes.shape[0], (64,), generator=gen, device=device)
    sample = state.view(-1, 128, 128)[idx].cpu().numpy()
    ocodes, os, osc = oracle.encode_heads(sample, KV, threads=8)
    assert flat_codes[idx].cpu().numpy().tobytes() == ocodes.tobytes()
    assert flat_s[idx].cpu().numpy().tobytes() == os.tobytes()
    assert flat_sc[idx].cpu().numpy().tobytes() == osc.tobytes()
    odense = oracle.decode_heads(ocodes, os, osc, KV, threads=8)
    assert dense.view(-1, 128, 128)[idx].cpu().numpy().tobytes() == odense.tobytes()
    del state, dense, codes


def test_admission_statuses_on_device_pointers(device):
    lib = native()
    x = torch.zeros((65, 128, 128), dtype=torch.float32, device=device)
    out = torch.empty((65, 128), dtype=torch.float32, device=device)
    assert lib.provider_smoothing_launch_v2(stream(), x.data_ptr(), out.data_ptr(), 65) == 1
    assert lib.provider_smoothing_launch_v2(stream(), x.data_ptr(), out.data_ptr(), 0) == 1
    assert lib.provider_smoothing_launch_v2(stream(), x.data_ptr(), out.data_ptr(), 64) == 0
    with pytest.raises(RuntimeError):
        codec.encode(x.to(torch.float64))
    with pytest.raises(RuntimeError):
        codec.encode(x[:, :, :64])
