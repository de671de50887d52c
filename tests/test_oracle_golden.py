"""The C oracle against the reference's own outputs (golden fixtures written by
tests/golden/make_golden.py from oracle/_ref) and known answers."""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import datagen
import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build(reference=False)


def test_special_heads_bit_exact(golden):
    summary = json.loads((GOLDEN / "codec_heads.json").read_text())
    for name in golden["names"]:
        x = golden[f"{name}/input"]
        codes, s, sc, _, _ = oracle.quantize_kv(x)
        assert codes.tobytes() == golden[f"{name}/codes"].tobytes(), name
        assert s.tobytes() == golden[f"{name}/smoothing"].tobytes(), name
        assert sc.tobytes() == golden[f"{name}/scales"].tobytes(), name
        assert sha(oracle.dequantize_kv(codes, s, sc)) == summary[name]["dequant_sha256"], name
        read = oracle.bf16_to_f32(golden[f"{name}/query_bf16"])
        out = oracle.read_boundary(codes, s, sc, read)
        assert out.tobytes() == golden[f"{name}/readout"].tobytes(), name


def test_fixture_covers_edge_cases():
    summary = json.loads((GOLDEN / "codec_heads.json").read_text())
    assert summary["ties"]["ties"] >= 16
    assert summary["wide_range"]["order_dependent_rows"] >= 16
    assert summary["wide_range"]["order_dependent_cols"] >= 16


def test_rank4_heads_bit_exact(golden):
    summary = json.loads((GOLDEN / "codec_heads.json").read_text())
    for name in ("c1_style", "student_t"):
        codes, s, sc, ck, cv = oracle.quantize_kv(golden[f"{name}/input"], rank=4)
        assert codes.tobytes() == golden[f"{name}/rank4_codes"].tobytes()
        assert s.tobytes() == golden[f"{name}/rank4_smoothing"].tobytes()
        assert sc.tobytes() == golden[f"{name}/rank4_scales"].tobytes()
        assert ck.tobytes() == golden[f"{name}/rank4_comp_keys"].tobytes()
        assert cv.tobytes() == golden[f"{name}/rank4_comp_values"].tobytes()
        dense = oracle.dequantize_kv(codes, s, sc, ck, cv)
        assert sha(dense) == summary[name]["rank4_dequant_sha256"]


def test_config1_round_trip_digests():
    d = json.loads((GOLDEN / "c1_digests.json").read_text())
    x = datagen.c1_heads(32, d["seed"])
    assert sha(x) == d["input_sha256"], "synthetic generator changed"
    codes, s, sc = oracle.encode_heads(x, oracle.LAYOUT_KEY_VALUE, threads=4)
    assert sha(codes) == d["codes_sha256"]
    assert sha(s) == d["smoothing_sha256"]
    assert sha(sc) == d["scales_sha256"]
    dense = oracle.decode_heads(codes, s, sc, oracle.LAYOUT_KEY_VALUE)
    assert sha(dense) == d["dequant_sha256"]


def test_config1_provider_layout_is_the_transpose():
    d = json.loads((GOLDEN / "c1_digests.json").read_text())
    x = datagen.c1_heads(32, d["seed"])
    provider = np.ascontiguousarray(x.transpose(0, 2, 1))
    codes, s, sc = oracle.encode_heads(provider, oracle.LAYOUT_VALUE_KEY, threads=4)
    assert sha(np.ascontiguousarray(codes.transpose(0, 2, 1))) == d["codes_sha256"]
    assert sha(s) == d["smoothing_sha256"]
    assert sha(sc) == d["scales_sha256"]
    dense = oracle.decode_heads(codes, s, sc, oracle.LAYOUT_VALUE_KEY)
    assert sha(np.ascontiguousarray(dense.transpose(0, 2, 1))) == d["dequant_sha256"]


def test_adapter_known_answer():
    d = json.loads((GOLDEN / "adapter.json").read_text())
    # native/tests/gdn_state_codec_qwen38_gdn_adapter_test.cpp:20-31
    assert d["codec"] == [1, 4, 2, 5, 3, 6]
    provider = np.array(d["provider"], np.float32)
    codec = oracle.provider_to_codec(provider, d["keys"], d["values"])
    assert codec.tolist() == d["codec"]
    assert oracle.codec_to_provider(codec, d["keys"], d["values"]).tolist() == d["provider"]
