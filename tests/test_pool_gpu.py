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


def test_out_of_range_slot_ids_are_skipped(device):
    pool = _pool(1, 4, 2, 92, False)
    ids = np.array([0, 4, 1000, -5, 3], np.int32)  # 4 and 1000 are >= slots
    c, s, sc = codec.pool_encode(_as_torch(pool, device), torch.from_numpy(ids).to(device), KV)
    got = to_np(c)
    assert not got[:, 1:4].any()  # untouched zero-initialised outputs
    oc, _, _ = oracle.pool_encode(pool, np.array([0, -1, -1, -1, 3], np.int32), KV)
    assert got.tobytes() == oc.tobytes()
