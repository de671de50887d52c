"""GPU parity of the capsule path's boundary encode with the rank-r compensator
fit (quantize_boundary_launch_v1; FromDenseBoundary -> QuantizeBoundary,
native/src/gdn_state_codec_state_capsule.cpp:129-226, 318-335): bit-exact
against the outputs the reference's own C++ wrote for the golden heads and
against the C oracle (pinned to that C++ at every rank 0..4 by
test_oracle_reference.py), through the C-ABI."""

from pathlib import Path

import numpy as np
import pytest
import torch

import datagen
import oracle
from gdn_state_codec import codec

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def to_gpu(a, device):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(device)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def assert_matches_oracle(heads, got, rank):
    codes, s, sc, ck, cv = (host(t) for t in got[:5])
    for h, x in enumerate(heads):
        e_codes, e_s, e_sc, e_ck, e_cv = oracle.quantize_kv(x, rank)
        assert codes[h].tobytes() == e_codes.tobytes(), (rank, h, "codes")
        assert s[h].tobytes() == e_s.tobytes(), (rank, h, "smoothing")
        assert sc[h].tobytes() == e_sc.tobytes(), (rank, h, "scales")
        assert ck[h].tobytes() == np.ascontiguousarray(e_ck).tobytes(), (rank, h, "keys")
        assert cv[h].tobytes() == np.ascontiguousarray(e_cv).tobytes(), (rank, h, "values")


def test_rank4_boundary_matches_reference_fixtures(device):
    """The two golden heads the reference's QuantizeBoundary encoded at rank 4
    (tests/golden/codec_heads.npz, written through oracle/_ref): codes,
    smoothing, scales and both compensators bit for bit."""
    golden = np.load(GOLDEN / "codec_heads.npz")
    names = ("c1_style", "student_t")
    dense = np.stack([golden[f"{name}/input"] for name in names])
    print(f"rank-4 boundary encode, golden heads {names}", flush=True)
    got = codec.quantize_boundary(to_gpu(dense, device), rank=4)
    for i, name in enumerate(names):
        for k, key in enumerate(("codes", "smoothing", "scales", "comp_keys", "comp_values")):
            expect = np.ascontiguousarray(golden[f"{name}/rank4_{key}"])
            assert host(got[k])[i].tobytes() == expect.tobytes(), (name, key)
    assert (host(got[6]) == 0).all()


@pytest.mark.parametrize("rank", [0, 1, 2, 3, 4])
def test_boundary_encode_matches_oracle_at_every_rank(device, rank):
    """Ordinary heads (C1-style and Student-t with zeros), and heads where the
    fit's own branches fire: all zeros (every left normalization fails, so the
    loop ends at once and the singular value is 0), exactly rank 1 (the later
    ranks fit what rounding leaves), constant, rows and columns of zeros,
    tiny and huge magnitudes, and a wide exponent range."""
    heads = np.concatenate([
        datagen.c1_heads(4, 31),
        datagen.student_t_heads(4, 32, zero_fraction=0.05),
        np.stack([
            np.zeros((128, 128), np.float32),
            np.outer(datagen.rng(33).standard_normal(128),
                     datagen.rng(34).standard_normal(128)).astype(np.float32),
            datagen.constant_head(0.25),
            datagen.zero_rows_cols_head(35),
            datagen.tiny_head(36),
            datagen.huge_head(37),
            datagen.wide_range_head(38),
        ]),
    ]).astype(np.float32)
    print(f"boundary encode vs oracle, rank={rank}, heads={len(heads)}", flush=True)
    got = codec.quantize_boundary(to_gpu(heads, device), rank=rank)
    assert (host(got[6]) == 0).all()
    assert_matches_oracle(heads, got, rank)


def test_boundary_encode_rejects_what_the_reference_rejects(device):
    """FromDenseBoundary refuses a head with a non-finite value (status 1) and
    QuantizeBoundary one whose singular value overflows (status 2: a head of
    1e38 everywhere overflows the first product to inf, and the fit then turns
    NaN); the other heads of the batch are encoded as usual, and the checked
    wrapper raises for the first refused head."""
    heads = datagen.c1_heads(5, 41).astype(np.float32)
    heads[1, 3, 7] = np.nan
    heads[3, 100, 0] = np.inf
    heads[4] = np.float32(1e38)
    print("boundary encode rejections, heads=5", flush=True)
    got = codec.quantize_boundary(to_gpu(heads, device), rank=4, check=False)
    assert host(got[6]).tolist() == [0, 1, 0, 1, 2]
    for h in (0, 2):
        e_codes, e_s, e_sc, e_ck, e_cv = oracle.quantize_kv(heads[h], 4)
        assert host(got[0])[h].tobytes() == e_codes.tobytes()
        assert host(got[3])[h].tobytes() == np.ascontiguousarray(e_ck).tobytes()
    with pytest.raises(ValueError, match="head 1 holds a non-finite value"):
        codec.quantize_boundary(to_gpu(heads, device), rank=4)


def test_fitted_residual_is_what_the_quant_stage_encodes(device):
    """The residual output is the dense head minus the fit, and the codes are
    the plain encode of that residual (the batched quant stage)."""
    heads = datagen.student_t_heads(6, 43, zero_fraction=0.02).astype(np.float32)
    print("boundary encode residual, heads=6", flush=True)
    dense = to_gpu(heads, device)
    codes, s, sc, ck, cv, residual, status = codec.quantize_boundary(dense, rank=4)
    plain = codec.encode(residual, codec.LAYOUT_KEY_VALUE)
    assert host(plain[0]).tobytes() == host(codes).tobytes()
    assert host(plain[1]).tobytes() == host(s).tobytes()
    fit = np.einsum("hkr,hvr->hkv", host(ck).astype(np.float64), host(cv).astype(np.float64))
    assert np.abs(host(residual) - (heads - fit)).max() < 1e-5 * np.abs(heads).max()


def test_boundary_encode_over_several_rounds_of_workgroups(device):
    """1,536 heads (three times what the GPU holds at once): every status 0,
    and every 97th head bit-exact against the oracle, so workgroups of every
    round and on every XCD are covered."""
    heads = np.concatenate([datagen.c1_heads(768, 51),
                            datagen.student_t_heads(768, 52, zero_fraction=0.02)]).astype(np.float32)
    print(f"boundary encode, heads={len(heads)}", flush=True)
    got = codec.quantize_boundary(to_gpu(heads, device), rank=4)
    assert (host(got[6]) == 0).all()
    sample = list(range(0, len(heads), 97))
    codes, s, sc, ck, cv = (host(t) for t in got[:5])
    for h in sample:
        e_codes, e_s, e_sc, e_ck, e_cv = oracle.quantize_kv(heads[h], 4)
        assert codes[h].tobytes() == e_codes.tobytes(), h
        assert s[h].tobytes() == e_s.tobytes(), h
        assert ck[h].tobytes() == np.ascontiguousarray(e_ck).tobytes(), h
        assert cv[h].tobytes() == np.ascontiguousarray(e_cv).tobytes(), h
