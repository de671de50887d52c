"""torch-facing capsule wire format (include/gdn_state_codec_capsule.h).

Hibernate a batch of window slots as LQCAPS01 capsules -- the bytes
``GdnStateCodecCapsule::Serialize`` writes
(``native/src/gdn_state_codec_state_capsule.cpp:446-474``) -- and restore them
with the checks of ``GdnStateCodecCapsule::Restore`` (``:476-578``), on the
device.  An invalid expected identity raises ``ValueError`` (the reference's
``std::invalid_argument`` from ``ValidateIdentity``, ``:40-48``); a capsule the
restore refuses is reported per state through the returned status tensor,
whose codes name the reference check that failed (``OUTCOMES``).
"""

from __future__ import annotations

import re
from dataclasses import dataclass

import torch

from ._native import native
from .window import WindowSlot

LAYOUT_KEY_VALUE = 0
LAYOUT_VALUE_KEY = 1

OK = 0
OUTCOMES = {
    0: "ok",
    1: "capsule is truncated",
    2: "capsule magic differs",
    3: "capsule checksum encoding is invalid",
    4: "capsule checksum differs",
    5: "capsule quantization parameters differ",
    6: "capsule identity or geometry differs",
    7: "compensator rank exceeds restored geometry",
    8: "capsule window position is invalid",
    9: "capsule window phase differs",
    10: "INT8 residual contains -128",
    11: "boundary payload is invalid",
    12: "update record is non-finite",
    13: "capsule contains trailing unverified payload",
    14: "restored state is non-finite",
    15: "capsule is valid but not representable in the fp16 slot format",
    16: "capsule extent lies outside the buffer or is misaligned",
}

_HEX = re.compile(r"[0-9a-f]{64}")


@dataclass(frozen=True)
class CapsuleIdentity:
    """GdnStateCodecIdentity for 128 x 128 heads
    (``gdn_state_codec_state_capsule.h:22-30``)."""

    model_geometry_sha256: str
    generation: int
    epoch: int

    def validate(self) -> None:
        if not (isinstance(self.model_geometry_sha256, str)
                and _HEX.fullmatch(self.model_geometry_sha256)):
            raise ValueError("GDN State Codec model geometry digest is invalid")
        if not 0 < self.generation < 2 ** 64:
            raise ValueError("GDN State Codec generation must be positive")
        if not 0 < self.epoch < 2 ** 64:
            raise ValueError("GDN State Codec epoch must be positive")

    @property
    def geometry_bytes(self) -> bytes:
        return self.model_geometry_sha256.encode("ascii")


def capsule_bytes(window_position: int) -> int:
    """Bytes of the capsule of a state at `window_position` (0 if >= 16)."""
    return int(native().capsule_bytes_v1(window_position))


MAX_CAPSULE_BYTES = 21688 + 1536 * 15  # position 15


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def serialize(slot: WindowSlot, identity: CapsuleIdentity,
              layout: int = LAYOUT_VALUE_KEY, validate: bool = True):
    """Capsules of every state of `slot` -> (capsules uint8 [S * stride],
    offsets int64 [S], lengths int32 [S]) on the slot's device.  Capsule i is
    capsules[offsets[i] : offsets[i] + lengths[i]]; lengths[i] == 0 for a
    state at position >= 16 (a full window has no capsule)."""
    identity.validate()
    if validate:
        slot.validate()
    s, dev = slot.states, slot.device
    capsules = torch.empty(s * MAX_CAPSULE_BYTES, dtype=torch.uint8, device=dev)
    offsets = torch.arange(s, dtype=torch.int64, device=dev) * MAX_CAPSULE_BYTES
    lengths = torch.empty(s, dtype=torch.int32, device=dev)
    status = native().capsule_serialize_launch_v1(
        _stream(), *slot.pointers(), layout, identity.geometry_bytes, identity.generation,
        identity.epoch, capsules.data_ptr(), offsets.data_ptr(), capsules.numel(),
        lengths.data_ptr(), s)
    if status != 0:
        raise RuntimeError(f"capsule_serialize_launch_v1 failed with status {status}")
    return capsules, offsets, lengths


def serialize_to_host(slot: WindowSlot, identity: CapsuleIdentity,
                      layout: int = LAYOUT_VALUE_KEY) -> list[bytes]:
    """Hibernate: one ``bytes`` capsule per state (b"" at a full window)."""
    capsules, offsets, lengths = serialize(slot, identity, layout)
    host = capsules.cpu().numpy()
    return [host[o:o + n].tobytes() for o, n in zip(offsets.cpu().tolist(), lengths.cpu().tolist())]


def restore(slot: WindowSlot, capsules: torch.Tensor, offsets: torch.Tensor,
            lengths: torch.Tensor, identity: CapsuleIdentity, expected_positions,
            layout: int = LAYOUT_VALUE_KEY, validate: bool = True) -> torch.Tensor:
    """Restore capsule i into state i of `slot`; returns the int32 outcome per
    state (``OUTCOMES``).  A state is written only when its outcome is 0."""
    identity.validate()
    if validate:
        slot.validate()
    s, dev = slot.states, slot.device
    if not isinstance(expected_positions, torch.Tensor):
        expected_positions = torch.tensor([int(p) for p in expected_positions], dtype=torch.int32)
    expected_positions = expected_positions.to(device=dev, dtype=torch.int32).contiguous()
    for name, t, dtype, n in (("capsules", capsules, torch.uint8, None),
                              ("offsets", offsets, torch.int64, s),
                              ("lengths", lengths, torch.int32, s),
                              ("expected_positions", expected_positions, torch.int32, s)):
        if t.dtype != dtype or t.device != dev or not t.is_contiguous() or t.dim() != 1 or (
                n is not None and t.numel() != n):
            raise RuntimeError(f"{name} must be a contiguous 1-d {dtype} tensor on {dev}"
                               + (f" with {n} elements" if n is not None else ""))
    status = torch.empty(s, dtype=torch.int32, device=dev)
    rc = native().capsule_restore_launch_v1(
        _stream(), capsules.data_ptr(), offsets.data_ptr(), lengths.data_ptr(), capsules.numel(),
        identity.geometry_bytes, identity.generation, identity.epoch,
        expected_positions.data_ptr(), layout, *slot.pointers(), status.data_ptr(), s)
    if rc != 0:
        raise RuntimeError(f"capsule_restore_launch_v1 failed with status {rc}")
    return status


def restore_from_host(slot: WindowSlot, blobs: list[bytes], identity: CapsuleIdentity,
                      expected_positions, layout: int = LAYOUT_VALUE_KEY) -> torch.Tensor:
    """Resume: restore one host ``bytes`` capsule per state of `slot`."""
    if len(blobs) != slot.states:
        raise RuntimeError(f"expected {slot.states} capsules, got {len(blobs)}")
    sizes = [len(b) for b in blobs]
    starts, total = [], 0
    for n in sizes:
        starts.append(total)
        total += (n + 7) // 8 * 8
    host = bytearray(max(total, 8))
    for start, blob in zip(starts, blobs):
        host[start:start + len(blob)] = blob
    dev = slot.device
    capsules = torch.frombuffer(host, dtype=torch.uint8).to(dev)
    offsets = torch.tensor(starts, dtype=torch.int64).to(dev)
    lengths = torch.tensor(sizes, dtype=torch.int32).to(dev)
    return restore(slot, capsules, offsets, lengths, identity, expected_positions, layout)
