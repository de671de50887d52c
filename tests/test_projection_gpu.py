"""GPU parity of the encoded projection (decode GEMV and chunked MFMA) against
the oracle readout and the reference's golden readouts.

Tolerance (fp32): |out - exact| <= 2^-15 * sum_k |code * s * x| * scale / 127
for the decode GEMV, where exact is the fp64 evaluation of the same closed form
from the same inputs; the fp32 oracle itself stays within 2^-17 of that
magnitude.  The chunked MFMA path splits each weight s * x into two bf16 parts
(remainder below 2^-16 of it) and accumulates 256 exact products in fp32, so
its bound is 2^-14 of the same magnitude; test_chunked_error_is_far_inside_its_bound
shows the largest error of a config-4 shaped batch stays below the split's own
worst case, 2^-16 (it measured about 2^-17.6)."""

import numpy as np
import pytest
import torch

import datagen
import oracle
from gdn_state_codec import codec

pytestmark = pytest.mark.gpu
KV, VK = codec.LAYOUT_KEY_VALUE, codec.LAYOUT_VALUE_KEY
TOL = 2.0 ** -15
CHUNKED_TOL = 2.0 ** -14


def to_gpu(a, device):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def to_np(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _encoded(tiles_shape, seed, layout):
    x = datagen.c1_heads(int(np.prod(tiles_shape)), seed)
    if layout == VK:
        x = np.ascontiguousarray(x.transpose(0, 2, 1))
    codes, s, sc = oracle.encode_heads(x, layout, threads=8)
    shape = tuple(tiles_shape)
    return codes.reshape(shape + (128, 128)), s.reshape(shape + (128,)), sc.reshape(shape + (128,))


def _queries(shape, seed):
    g = datagen.rng(seed)
    q = g.standard_normal(shape).astype(np.float32)
    q /= np.linalg.norm(q, axis=-1, keepdims=True)  # L2-normalised per head
    return oracle.f32_to_bf16(q)


def _within(got, exact, bound, tol=TOL):
    err = np.abs(got.astype(np.float64) - exact)
    return err <= tol * bound + 1e-30


@pytest.mark.parametrize("layout", [VK, KV])
@pytest.mark.parametrize("batch,heads,qheads,qscale", [
    (4, 32, 16, 1.0), (3, 32, 16, 128 ** -0.5), (5, 8, 8, 1.0), (2, 6, 2, 0.5)])
def test_decode_projection_matches_oracle(device, layout, batch, heads, qheads, qscale):
    print(f"decode projection layout={layout} B={batch} H={heads} Hq={qheads}", flush=True)
    codes, s, sc = _encoded((batch, heads), 10 + batch, layout)
    q = _queries((batch, qheads, 128), 20 + batch)
    out32, out64, bound = oracle.project_decode(codes, s, sc, q, qscale, layout)
    got = to_np(codec.project_decode(to_gpu(codes, device), to_gpu(s, device),
                                     to_gpu(sc, device), to_gpu(q, device).view(torch.bfloat16),
                                     qscale, layout))
    assert _within(got, out64, bound).all()
    assert _within(out32, out64, bound).all()


def test_decode_projection_matches_reference_readouts(device, golden):
    for name in golden["names"]:
        codes = golden[f"{name}/codes"][None, None]
        s = golden[f"{name}/smoothing"][None, None]
        sc = golden[f"{name}/scales"][None, None]
        q = golden[f"{name}/query_bf16"][None, None]
        _, out64, bound = oracle.project_decode(codes, s, sc, q, 1.0, KV)
        ref = golden[f"{name}/readout"]
        got = to_np(codec.project_decode(to_gpu(codes, device), to_gpu(s, device),
                                         to_gpu(sc, device), to_gpu(q, device).view(torch.bfloat16),
                                         1.0, KV))[0, 0]
        assert _within(got, out64[0, 0], bound[0, 0]).all(), name
        assert _within(ref, out64[0, 0], bound[0, 0]).all(), name


def test_decode_projection_full_config3(device):
    """B=256, 16 query heads GQA-mapped to 32 value heads."""
    codes, s, sc = _encoded((256, 32), 30, VK)
    q = _queries((256, 16, 128), 31)
    _, out64, bound = oracle.project_decode(codes, s, sc, q, 1.0, VK)
    got = to_np(codec.project_decode(to_gpu(codes, device), to_gpu(s, device), to_gpu(sc, device),
                                     to_gpu(q, device).view(torch.bfloat16), 1.0, VK))
    assert _within(got, out64, bound).all()


@pytest.mark.parametrize("layout", [VK, KV])
@pytest.mark.parametrize("seqs,tokens,heads,qheads", [
    (2, 64, 32, 32), (3, 37, 8, 4), (2, 1, 4, 4), (1, 96, 4, 2), (2, 20, 8, 2)])
def test_chunked_projection_matches_oracle(device, layout, seqs, tokens, heads, qheads):
    print(f"chunked projection layout={layout} N={seqs} T={tokens} H={heads} Hq={qheads}",
          flush=True)
    codes, s, sc = _encoded((seqs, heads), 40 + tokens, layout)
    q = _queries((seqs, tokens, qheads, 128), 50 + tokens)
    out32, out64, bound = oracle.project_chunked(codes, s, sc, q, 1.0, layout, threads=8)
    got = to_np(codec.project_chunked(to_gpu(codes, device), to_gpu(s, device),
                                      to_gpu(sc, device), to_gpu(q, device).view(torch.bfloat16),
                                      1.0, layout))
    assert _within(got, out64, bound, CHUNKED_TOL).all()
    assert _within(out32, out64, bound).all()


def test_chunked_projection_full_config4(device):
    """64 sequences x T=64 x 32 heads."""
    codes, s, sc = _encoded((64, 32), 60, VK)
    q = _queries((64, 64, 32, 128), 61)
    _, out64, bound = oracle.project_chunked(codes, s, sc, q, 1.0, VK, threads=8)
    got = to_np(codec.project_chunked(to_gpu(codes, device), to_gpu(s, device),
                                      to_gpu(sc, device), to_gpu(q, device).view(torch.bfloat16),
                                      1.0, VK))
    assert _within(got, out64, bound, CHUNKED_TOL).all()


@pytest.mark.parametrize("layout", [VK, KV])
def test_chunked_rounds_of_32_and_16_tokens_agree(device, layout):
    """Token counts that are multiples of 32 take 32-token rounds, others
    16-token rounds with a clamped tail: the first 64 outputs of a 65-token
    call (16-token rounds) equal a 64-token call (32-token rounds) bit for
    bit, since each output row depends only on its own query row."""
    codes, s, sc = _encoded((3, 8), 90, layout)
    q = _queries((3, 65, 4, 128), 91)
    g = [to_gpu(a, device) for a in (codes, s, sc)]
    q65 = to_gpu(q, device).view(torch.bfloat16)
    q64 = to_gpu(np.ascontiguousarray(q[:, :64]), device).view(torch.bfloat16)
    out65 = codec.project_chunked(*g, q65, 0.75, layout)
    out64 = codec.project_chunked(*g, q64, 0.75, layout)
    assert torch.equal(out65[:, :64], out64)


def test_chunked_error_is_far_inside_its_bound(device):
    """The two-part split's worst case is 2^-16 of sum |terms| per output; on
    config-4 shaped data the largest error over 2M outputs stays below it, 4x
    inside the 2^-14 bound the other tests use."""
    codes, s, sc = _encoded((8, 32), 62, VK)
    q = _queries((8, 64, 32, 128), 63)
    _, out64, bound = oracle.project_chunked(codes, s, sc, q, 1.0, VK, threads=8)
    got = to_np(codec.project_chunked(to_gpu(codes, device), to_gpu(s, device),
                                      to_gpu(sc, device), to_gpu(q, device).view(torch.bfloat16),
                                      1.0, VK))
    ratio = np.abs(got.astype(np.float64) - out64) / np.maximum(bound, 1e-300)
    print(f"chunked max error / sum|terms| = {ratio.max():.3e}", flush=True)
    assert ratio.max() <= 2.0 ** -16


def test_chunked_equals_decode_token_by_token(device):
    codes, s, sc = _encoded((2, 8), 70, VK)
    q = _queries((2, 5, 4, 128), 71)
    g = [to_gpu(a, device) for a in (codes, s, sc)]
    chunked = to_np(codec.project_chunked(*g, to_gpu(q, device).view(torch.bfloat16), 1.0, VK))
    _, out64, bound = oracle.project_chunked(codes, s, sc, q, 1.0, VK)
    for t in range(5):
        dec = to_np(codec.project_decode(*g, to_gpu(q[:, t], device).view(torch.bfloat16),
                                         1.0, VK))
        assert _within(dec, out64[:, t], bound[:, t]).all()
        assert _within(chunked[:, t], out64[:, t], bound[:, t], CHUNKED_TOL).all()


def test_projection_without_checks_is_identical(device):
    """`validate=False` only skips the host-side tensor checks."""
    codes, s, sc = _encoded((2, 8), 80, VK)
    g = [to_gpu(a, device) for a in (codes, s, sc)]
    qd = to_gpu(_queries((2, 4, 128), 81), device).view(torch.bfloat16)
    qc = to_gpu(_queries((2, 7, 4, 128), 82), device).view(torch.bfloat16)
    assert torch.equal(codec.project_decode(*g, qd, 0.5, VK),
                       codec.project_decode(*g, qd, 0.5, VK, validate=False))
    assert torch.equal(codec.project_chunked(*g, qc, 0.5, VK),
                       codec.project_chunked(*g, qc, 0.5, VK, validate=False))
