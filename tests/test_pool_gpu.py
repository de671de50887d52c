"""GPU parity of the slot-indexed pool codec (gather -> encode, decode ->
scatter) against the oracle, fp32 and bf16 pools, with -1 padding."""

import numpy as np
import pytest
import torch

import datagen
import oracle
from gdn_state_codec import codec

pytestmark = pytest.mark.gpu
KV, VK = codec.LAYOUT_KEY_VALUE, codec.LAYOUT_VALUE_KEY


def to_np(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def _pool(layers, slots, heads, seed, bf16):
    x = datagen.student_t_heads(layers * slots * heads, seed, zero_fraction=0.02)
    x = x.reshape(layers, slots, heads, 128, 128)
    if bf16:
        return oracle.f32_to_bf16(x).reshape(x.shape)
    return x


def _as_torch(pool, device):
    t = torch.from_numpy(np.ascontiguousarray(pool)).to(device)
    return t.view(torch.bfloat16) if pool.dtype == np.uint16 else t


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("layout", [KV, VK])
def test_pool_encode_decode_match_oracle(device, bf16, layout):
    print(f"pool codec bf16={bf16} layout={layout}", flush=True)
    layers, slots, heads = 3, 24, 4
    pool = _pool(layers, slots, heads, 90 + bf16, bf16)
    g = datagen.rng(91)
    ids = g.permutation(slots)[:10].astype(np.int32)
    ids[[2, 7]] = -1  # padding
    oc, os, osc = oracle.pool_encode(pool, ids, layout, threads=8)
    slot_ids = torch.from_numpy(ids).to(device)
    tpool = _as_torch(pool, device)
    c, s, sc = codec.pool_encode(tpool, slot_ids, layout)
    assert to_np(c).tobytes() == oc.tobytes()
    assert to_np(s).tobytes() == os.tobytes()
    assert to_np(sc).tobytes() == osc.tobytes()

    # Scatter back into a poisoned pool: live slots receive the decode, every
    # other slot (padding, unused) keeps its poison.
    poison = np.full_like(pool, 0x7FC0 if bf16 else 0)
    if not bf16:
        poison[...] = np.float32(123.25)
    expect = oracle.pool_decode(oc, os, osc, ids, poison.copy(), layout, threads=8)
    tdst = _as_torch(poison, device)
    codec.pool_decode(c, s, sc, slot_ids, tdst, layout)
    got = to_np(tdst.view(torch.uint16) if bf16 else tdst)
    assert got.tobytes() == expect.tobytes()
    untouched = [slot for slot in range(slots) if slot not in set(ids.tolist())]
    assert (got[:, untouched] == poison[:, untouched]).all()


@pytest.mark.parametrize("layout", [KV, VK])
@pytest.mark.parametrize("kind", ["c1", "student_t", "wide", "tiny_and_huge", "tiny_value",
                                  "zeros", "requantize"])
def test_bf16_pool_encode_edge_cases_match_oracle(device, layout, kind):
    """bf16 tiles in [value][key] keep q0 = RN(r * RN(1/s)) on the fast
    domains: the codes come from it directly (the certified lift of
    codec_math.h), with the exact path, which recovers r from q0, for values
    inside its margin; tiles outside the fast domains read their rows again
    (subnormal and 1e30-scale entries: the division by s; values whose scale
    is below 2^-90: the division by the scale).  Every kind of tile the fp32
    parity test uses, rounded to bf16, bit-exact in both layouts."""
    print(f"bf16 pool edge cases layout={layout} kind={kind}", flush=True)
    if kind == "c1":
        x = datagen.c1_heads(64, 15)
    elif kind == "student_t":
        x = datagen.student_t_heads(64, 16, zero_fraction=0.05)
    elif kind == "wide":
        x = np.stack([datagen.wide_range_head(400 + i) for i in range(24)])
    elif kind == "tiny_and_huge":
        x = np.stack([datagen.tiny_head(500 + i) for i in range(12)]
                     + [datagen.huge_head(600 + i) for i in range(12)])
    elif kind == "tiny_value":
        axis = 1 if layout == KV else 0
        x = np.stack([datagen.tiny_value_head(650 + i, axis) for i in range(12)])
    elif kind == "zeros":
        x = np.stack([datagen.zero_rows_cols_head(700 + i) for i in range(16)])
    else:
        # Re-encoded dequantized states: exact zeros, half of them -0.
        x = datagen.student_t_heads(48, 17)
        x = oracle.decode_heads(*oracle.encode_heads(x, layout, threads=8), layout, threads=8)
        zeros = np.flatnonzero(x == 0)
        x.reshape(-1)[zeros[::2]] = -0.0
    pool = oracle.f32_to_bf16(x).reshape((1, x.shape[0], 1, 128, 128))
    ids = np.arange(x.shape[0], dtype=np.int32)[::-1].copy()
    oc, os, osc = oracle.pool_encode(pool, ids, layout, threads=8)
    c, s, sc = codec.pool_encode(_as_torch(pool, device), torch.from_numpy(ids).to(device), layout)
    assert to_np(c).tobytes() == oc.tobytes()
    assert to_np(s).tobytes() == os.tobytes()
    assert to_np(sc).tobytes() == osc.tobytes()


def test_out_of_range_slot_ids_are_skipped(device):
    pool = _pool(1, 4, 2, 92, False)
    ids = np.array([0, 4, 1000, -5, 3], np.int32)  # 4 and 1000 are >= slots
    c, s, sc = codec.pool_encode(_as_torch(pool, device), torch.from_numpy(ids).to(device), KV)
    got = to_np(c)
    assert not got[:, 1:4].any()  # untouched zero-initialised outputs
    oc, _, _ = oracle.pool_encode(pool, np.array([0, -1, -1, -1, 3], np.int32), KV)
    assert got.tobytes() == oc.tobytes()


@pytest.mark.parametrize("dtype_name", ["f32", "bf16"])
def test_full_config5_pool(device, dtype_name):
    """BASELINE config 5 at full size, in the provider's [value][key] layout
    (the reference's slot map, runtime.py:603-625): a [30][2048][32] fp32
    (128.8 GB) or bf16 (64.4 GB) pool of Student-t(3) * 0.05 entries with 2%
    all-zero heads, 512 unique random slot ids of which 26 are -1.  After
    pool_encode and a pool_decode back into the same pool: codes within +-127
    and every live column reaching 127; zero heads with zero codes,
    s = sqrtf(1e-8) and scale 0; padding entries of the encoded batch
    untouched; slots outside the batch unchanged; and 96 sampled tiles
    bit-exact against the oracle in both directions."""
    print(f"full config-5 {dtype_name} pool", flush=True)
    bf16 = dtype_name == "bf16"
    dtype = torch.bfloat16 if bf16 else torch.float32
    bits = torch.int16 if bf16 else torch.int32
    layers, slots, heads, batch = 30, 2048, 32, 512
    gen = torch.Generator(device=device)
    gen.manual_seed(55 + 2 * (not bf16))
    pool = torch.empty((layers, slots, heads, 128, 128), dtype=dtype, device=device)
    for layer in range(layers):
        for part in range(0, slots, 256):
            shape = (256, heads, 128, 128)
            z = torch.randn(shape, generator=gen, device=device)
            chi = torch.zeros(shape, device=device)
            for _ in range(3):
                w = torch.randn(shape, generator=gen, device=device)
                chi.addcmul_(w, w)
            pool[layer, part:part + 256] = (z * torch.rsqrt(chi / 3) * 0.05).to(dtype)
            del z, chi, w
    zero = torch.rand((layers, slots, heads), generator=gen, device=device) < 0.02
    pool[zero] = 0
    ids = torch.randperm(slots, generator=gen, device=device)[:batch].to(torch.int32)
    ids[torch.randperm(batch, generator=gen, device=device)[:26]] = -1
    live = ids >= 0
    outside = torch.ones(slots, dtype=torch.bool, device=device)
    outside[ids[live].long()] = False
    outside_slots = torch.nonzero(outside).flatten()[:64]
    before = pool[:, outside_slots].view(bits).to(torch.int64).sum(dim=(2, 3, 4))

    codes = torch.full((layers, batch, heads, 128, 128), 0x55, dtype=torch.int8, device=device)
    s = torch.full((layers, batch, heads, 128), -1.0, dtype=torch.float32, device=device)
    sc = torch.full((layers, batch, heads, 128), -1.0, dtype=torch.float32, device=device)
    codec.pool_encode(pool, ids, VK, codes, s, sc)
    torch.cuda.synchronize()

    # Sampled tiles, taken before the decode overwrites the pool.
    g = datagen.rng(56 + 2 * (not bf16))
    live_entries = torch.nonzero(live).flatten().cpu().numpy()
    picks = [(int(g.integers(layers)), int(g.choice(live_entries)), int(g.integers(heads)))
             for _ in range(96)]
    slot_of = ids.cpu().numpy()

    def tile(l, b, h):
        t = pool[l, slot_of[b], h]
        return t.view(torch.int16).cpu().numpy().view(np.uint16) if bf16 else t.cpu().numpy()

    src = np.stack([tile(l, b, h) for l, b, h in picks])
    src32 = oracle.bf16_to_f32(src) if bf16 else src
    ocodes, os_, osc = oracle.encode_heads(src32.reshape(-1, 128, 128), VK, threads=8)
    for n, (l, b, h) in enumerate(picks):
        assert codes[l, b, h].cpu().numpy().tobytes() == ocodes[n].tobytes(), (l, b, h)
        assert s[l, b, h].cpu().numpy().tobytes() == os_[n].tobytes(), (l, b, h)
        assert sc[l, b, h].cpu().numpy().tobytes() == osc[n].tobytes(), (l, b, h)

    pad = torch.nonzero(~live).flatten()
    assert bool((codes[:, pad] == 0x55).all()) and bool((s[:, pad] == -1).all())
    assert bool((sc[:, pad] == -1).all())
    live_idx = torch.nonzero(live).flatten()
    floor = float(np.sqrt(np.float32(1e-8), dtype=np.float32))
    for layer in range(layers):
        c = codes[layer, live_idx]
        assert int(c.min()) >= -127 and int(c.max()) <= 127
        col_max = c.abs().amax(dim=3)  # [entries, heads, value]: VK tiles are [value][key]
        assert bool(((col_max == 127) | (sc[layer, live_idx] == 0)).all()), layer
        z = zero[layer, ids[live_idx].long()]
        assert bool((c[z] == 0).all()) and bool((sc[layer, live_idx][z] == 0).all())
        assert bool((s[layer, live_idx][z] == floor).all())
        del c, col_max, z

    codec.pool_decode(codes, s, sc, ids, pool, VK)
    torch.cuda.synchronize()
    odense = oracle.decode_heads(ocodes, os_, osc, VK, threads=8)
    if bf16:
        odense = oracle.f32_to_bf16(odense.reshape(-1)).reshape(odense.shape)
    for n, (l, b, h) in enumerate(picks):
        assert tile(l, b, h).tobytes() == odense[n].tobytes(), (l, b, h)
    after = pool[:, outside_slots].view(bits).to(torch.int64).sum(dim=(2, 3, 4))
    assert torch.equal(before, after)
    del pool, codes, s, sc
    torch.cuda.empty_cache()
