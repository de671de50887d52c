"""The C oracle against the reference's compiled CPU code (oracle/_ref) on
random, adversarial and odd-geometry inputs: every output bit-exact."""

import numpy as np
import pytest

import datagen
import oracle

pytestmark = pytest.mark.skipif(
    not oracle.ref_available(), reason="oracle/_ref not built (needs /root/reference)"
)


def _cases():
    g = datagen.rng(2024)
    shapes = [(128, 128), (8, 6), (3, 2), (17, 33), (1, 5), (64, 1)]
    for i in range(36):
        keys, values = shapes[i % len(shapes)]
        x = (g.standard_normal((keys, values)) * 0.05).astype(np.float32)
        if i % 3 == 0:
            x[g.random((keys, values)) < 0.01] = 2.0
        if i % 4 == 1:
            x *= (np.float32(2.0) ** g.integers(-60, 60, size=(keys, values))).astype(np.float32)
        if i % 5 == 2:
            x[g.random((keys, values)) < 0.2] = 0.0
        if i % 7 == 3:
            x[:, 0] = 0.0
        yield i, x
    yield 100, datagen.wide_range_head(5)
    yield 101, datagen.tiny_head(6)
    yield 102, datagen.huge_head(7)


@pytest.mark.parametrize("rank", [0, 1, 2, 3, 4])
def test_quantize_dequantize_readout_match_reference(rank):
    g = datagen.rng(11)
    for i, x in _cases():
        r = rank if min(x.shape) >= rank else 0
        ours = oracle.quantize_kv(x, r)
        ref = oracle.ref_quantize_kv(x, r)
        for a, b in zip(ours, ref):
            assert a.tobytes() == b.tobytes(), (i, r)
        ck = ours[3] if r else None
        cv = ours[4] if r else None
        assert (oracle.dequantize_kv(*ours[:3], ck, cv).tobytes()
                == oracle.ref_dequantize_kv(*ref[:3], ck, cv).tobytes()), i
        read = g.standard_normal(x.shape[0]).astype(np.float32)
        assert (oracle.read_boundary(*ours[:3], read, ck, cv).tobytes()
                == oracle.ref_read_boundary(*ref[:3], read, ck, cv).tobytes()), i


def test_batched_heads_match_reference():
    x = np.concatenate([datagen.c1_heads(24, 3), datagen.student_t_heads(8, 4, 0.25)])
    ours = oracle.encode_heads(x, oracle.LAYOUT_KEY_VALUE, threads=4)
    ref = oracle.ref_quantize_heads(x)
    for a, b in zip(ours, ref):
        assert a.tobytes() == b.tobytes()
    assert (oracle.decode_heads(*ours, oracle.LAYOUT_KEY_VALUE).tobytes()
            == oracle.ref_dequantize_heads(*ref).tobytes())


def test_provider_transposes_match_reference():
    g = datagen.rng(12)
    for keys, values in [(3, 2), (128, 128), (5, 9)]:
        provider = g.standard_normal(keys * values).astype(np.float32)
        assert (oracle.provider_to_codec(provider, keys, values).tobytes()
                == oracle.ref_provider_to_codec(provider, keys, values).tobytes())
