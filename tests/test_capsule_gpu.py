"""GPU parity of the capsule wire format (include/gdn_state_codec_capsule.h)
against the oracle (oracle/gdn_capsule_oracle.c), through the C-ABI:
serialized capsules byte-identical, restore outcomes identical (the check
that fails, in the reference's order), restored slots bit-exact and refused
states untouched."""

from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

import oracle
import windowgen as WG
from gdn_state_codec import native
from oracle import capsule as C
from test_capsule_oracle import corruptions
from test_window_gpu import dev, from_device, stream, to_device, window_ptrs

pytestmark = pytest.mark.gpu

VK, KV = oracle.LAYOUT_VALUE_KEY, oracle.LAYOUT_KEY_VALUE
IDENTITY = C.Identity("0123456789abcdef" * 4, 5, 9)
FILL = 0xA5


def pack_blobs(blobs, pad=8):
    """One buffer holding the blobs at 8-aligned offsets (FILL between)."""
    offsets, total = [], 0
    for b in blobs:
        offsets.append(total)
        total += (len(b) + pad - 1) // pad * pad + pad
    buf = np.full(max(total, 8), FILL, np.uint8)
    for o, b in zip(offsets, blobs):
        buf[o:o + len(b)] = np.frombuffer(b, np.uint8)
    return buf, np.array(offsets, np.uint64), np.array([len(b) for b in blobs], np.uint32)


def serialize_on_gpu(d, states, layout, offsets, capacity, device, identity=IDENTITY):
    out = torch.full((capacity,), FILL, dtype=torch.uint8, device=device)
    lengths = torch.full((states,), -1, dtype=torch.int32, device=device)
    doff = dev(offsets, device)
    assert native().capsule_serialize_launch_v1(
        stream(), *window_ptrs(d), layout, identity.geometry_bytes, identity.generation,
        identity.epoch, out.data_ptr(), doff.data_ptr(), capacity, lengths.data_ptr(),
        states) == 0
    torch.cuda.synchronize()
    return out.cpu().numpy(), lengths.cpu().numpy().view(np.uint32)


def restore_on_gpu(buf, offsets, lengths, expected, d, states, layout, device,
                   identity=IDENTITY, capacity=None):
    dbuf, doff, dlen = dev(buf, device), dev(offsets, device), dev(lengths, device)
    dexp = dev(np.asarray(expected, np.uint32), device)
    status = torch.full((states,), -1, dtype=torch.int32, device=device)
    assert native().capsule_restore_launch_v1(
        stream(), dbuf.data_ptr(), doff.data_ptr(), dlen.data_ptr(),
        buf.size if capacity is None else capacity, identity.geometry_bytes,
        identity.generation, identity.epoch, dexp.data_ptr(), layout, *window_ptrs(d),
        status.data_ptr(), states) == 0
    torch.cuda.synchronize()
    return status.cpu().numpy()


@pytest.mark.parametrize("layout", [VK, KV])
def test_serialize_is_byte_identical_to_the_oracle(device, layout):
    states = 40
    positions = list(range(17)) + list(np.random.default_rng(1).integers(0, 17, states - 17))
    print(f"capsule serialize layout={layout} states={states}", flush=True)
    buf = WG.window_buffers(states, 81, layout, positions=positions)
    want = [C.slot_serialize(buf, s, layout, IDENTITY) for s in range(states)]
    sizes = [C.slot_capsule_bytes(min(p, 15)) for p in positions]
    offsets = np.cumsum([0] + [(n + 15) // 8 * 8 for n in sizes[:-1]]).astype(np.uint64)
    capacity = int(offsets[-1]) + sizes[-1] + 8
    d = to_device(buf, device)
    got, lengths = serialize_on_gpu(d, states, layout, offsets, capacity, device)
    covered = np.zeros(capacity, bool)
    for s in range(states):
        assert lengths[s] == len(want[s]), s
        o = int(offsets[s])
        blob = got[o:o + lengths[s]].tobytes()
        assert blob == want[s], s
        if blob:
            assert blob[-64:].decode() == hashlib.sha256(blob[:-64]).hexdigest()
        covered[o:o + lengths[s]] = True
    assert (got[~covered] == FILL).all()  # nothing written outside the capsules
    after = from_device(d, buf)
    for name in buf:
        assert np.array_equal(after[name], buf[name]), name


def test_serialize_skips_capsules_that_do_not_fit(device):
    states = 4
    print("capsule serialize extent", flush=True)
    buf = WG.window_buffers(states, 82, VK, positions=[3, 3, 3, 3])
    n = C.slot_capsule_bytes(3)
    offsets = np.array([0, n + 4, 2 * n + 8, 3 * n + 64], np.uint64)  # misaligned, fits, past end
    capacity = 3 * n + 64 + n - 1
    got, lengths = serialize_on_gpu(to_device(buf, device), states, VK, offsets, capacity, device)
    assert list(lengths) == [n, 0, n, 0]
    assert got[:n].tobytes() == C.slot_serialize(buf, 0, VK, IDENTITY)
    assert (got[n:2 * n + 8] == FILL).all() and (got[3 * n + 64:] == FILL).all()


@pytest.mark.parametrize("layout", [VK, KV])
def test_restore_round_trips_bit_exactly(device, layout):
    states = 34
    positions = list(range(16)) * 2 + [16, 7]
    print(f"capsule restore layout={layout}", flush=True)
    src = WG.window_buffers(states, 83, layout, positions=positions)
    blobs = [C.slot_serialize(src, s, layout, IDENTITY) for s in range(states)]
    packed, offsets, lengths = pack_blobs(blobs)
    target = WG.window_buffers(states, 84, layout, positions=11)
    d = to_device(target, device)
    expected = [min(p, 15) for p in positions]
    status = restore_on_gpu(packed, offsets, lengths, expected, d, states, layout, device)
    want = WG.copy_buffers(target)
    want_status = [C.slot_restore(blobs[s], want, s, layout, IDENTITY, expected[s])
                   for s in range(states)]
    assert list(status) == want_status
    assert want_status[:32] == [C.OK] * 32 and want_status[32] == C.TRUNCATED
    got = from_device(d, target)
    for name in target:
        assert np.array_equal(got[name], want[name]), name


def test_restore_outcomes_match_the_oracle(device):
    """The reference test's corruptions and the further Restore checks, each in
    its own state of one launch, plus the device-only extent outcome."""
    print("capsule restore outcomes", flush=True)
    base = WG.window_buffers(1, 85, VK, positions=6)
    # corruptions() expects the reference test's identity; a launch has one
    # expected identity, so its two foreign-identity cases are replaced by a
    # capsule signed under another identity.
    ident = C.Identity("a" * 64, 7, 11)
    enc = C.slot_serialize(base, 0, VK, ident)
    cases = [(name, bad, pos, want) for name, bad, i, pos, want in
             corruptions(enc, 128, 128, 6) if i == ident]
    # Truncation sweep: every tail length of the digest's final block.
    for cut in range(1, 70):
        cases.append((f"cut {cut}", C.refresh_digest(enc[:-64 - cut] + enc[-64:]), 6, None))
    cases.append(("foreign identity", C.slot_serialize(base, 0, VK, IDENTITY), 6, C.IDENTITY))
    not_half = bytearray(enc)  # compensator key 0 = 0.1f, not an fp16 number
    key0 = C.HEADER + 128 * 128 + 1024
    not_half[key0:key0 + 4] = np.array([0.1], "<f4").tobytes()
    cases.append(("device format", C.refresh_digest(bytes(not_half)), 6, C.DEVICE_FORMAT))
    states = len(cases) + 2
    blobs = [bad for _, bad, _, _ in cases] + [enc, enc]
    packed, offsets, lengths = pack_blobs(blobs)
    offsets[-2] += 4                      # misaligned
    lengths[-1] = packed.size             # runs past the buffer
    expected = [pos for _, _, pos, _ in cases] + [6, 6]
    target = WG.window_buffers(states, 86, VK, positions=2)
    d = to_device(target, device)
    status = restore_on_gpu(packed, offsets, lengths, expected, d, states, VK, device,
                            identity=ident)
    want = WG.copy_buffers(target)
    for s, (name, bad, pos, outcome) in enumerate(cases):
        oracle_status = C.slot_restore(bad, want, s, VK, ident, pos)
        if outcome is not None:
            assert oracle_status == outcome, name
        assert status[s] == oracle_status, (name, status[s], oracle_status)
    assert list(status[-2:]) == [C_EXTENT, C_EXTENT]
    got = from_device(d, target)
    for name in target:
        assert np.array_equal(got[name], want[name]), name


C_EXTENT = 16


def test_python_mirror_hibernates_and_resumes(device):
    from gdn_state_codec import capsule as mirror
    from gdn_state_codec.window import WindowSlot

    states = 64
    print("capsule python mirror", flush=True)
    src = WG.window_buffers(states, 87, VK)
    d = to_device(src, device)
    slot = WindowSlot(d["residual"], d["smoothing"], d["scales"], d["compensator_keys"],
                      d["compensator_values"], d["record_decay"], d["record_keys"],
                      d["record_corrections"], d["positions"])
    identity = mirror.CapsuleIdentity(IDENTITY.geometry, IDENTITY.generation, IDENTITY.epoch)
    blobs = mirror.serialize_to_host(slot, identity)
    assert blobs == [C.slot_serialize(src, s, VK, IDENTITY) for s in range(states)]
    fresh = WindowSlot.allocate(states, device)
    status = mirror.restore_from_host(fresh, blobs, identity, src["positions"][:, 0])
    assert (status.cpu().numpy() == 0).all()
    back = from_device({k: getattr(fresh, k) for k in src}, src)
    for name in ("residual", "smoothing", "scales", "compensator_keys", "compensator_values"):
        assert np.array_equal(back[name], src[name]), name
    for s in range(states):
        p = int(src["positions"][s, 0])
        for name in ("record_decay", "record_keys", "record_corrections"):
            assert np.array_equal(back[name][s][:p], src[name][s][:p]), (s, name)
    assert np.array_equal(back["positions"][:, 0], src["positions"][:, 0])
    with pytest.raises(ValueError, match="digest"):
        mirror.serialize(slot, mirror.CapsuleIdentity("A" * 64, 1, 1))


def test_large_batch_round_trip(device):
    """Size-independent property at 4096 states: restore(serialize(slot))
    reproduces every state, and every capsule's digest is hashlib's."""
    from gdn_state_codec import capsule as mirror
    from gdn_state_codec.window import WindowSlot

    states = 4096
    print(f"capsule round trip states={states}", flush=True)
    g = torch.Generator(device=device).manual_seed(3)
    slot = WindowSlot.allocate(states, device)
    slot.residual.copy_(torch.randint(-127, 128, slot.residual.shape, device=device,
                                      generator=g, dtype=torch.int8))
    for t in (slot.smoothing, slot.scales, slot.record_decay):
        t.uniform_(0.5, 1.5, generator=g)
    for t in (slot.compensator_keys, slot.compensator_values, slot.record_keys,
              slot.record_corrections):
        t.copy_((torch.randn(t.shape, device=device, generator=g) * 0.05).to(torch.float16))
    slot.positions[:, 0] = torch.randint(0, 16, (states,), device=device, generator=g,
                                         dtype=torch.int32)
    identity = mirror.CapsuleIdentity(IDENTITY.geometry, 1, 2)
    capsules, offsets, lengths = mirror.serialize(slot, identity)
    fresh = WindowSlot.allocate(states, device)
    status = mirror.restore(fresh, capsules, offsets, lengths, identity, slot.positions[:, 0])
    assert (status == 0).all().item()
    for name in ("residual", "smoothing", "scales", "compensator_keys", "compensator_values",
                 "positions"):
        assert torch.equal(getattr(fresh, name), getattr(slot, name)), name
    p = slot.positions[:, 0].long()
    live = torch.arange(16, device=device)[None, :] < p[:, None]
    for name in ("record_decay", "record_keys", "record_corrections"):
        a, b = getattr(fresh, name), getattr(slot, name)
        mask = live if a.dim() == 2 else live[:, :, None].expand_as(a)
        assert torch.equal(a[mask], b[mask]), name
    host = capsules.cpu().numpy()
    for s in range(0, states, 97):
        o, n = int(offsets[s]), int(lengths[s])
        blob = host[o:o + n].tobytes()
        assert blob[-64:].decode() == hashlib.sha256(blob[:-64]).hexdigest(), s
