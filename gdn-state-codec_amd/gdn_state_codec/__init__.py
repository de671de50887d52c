"""MI355X (gfx950) GDN state codec: int8 codec of Qwen3.5 gated-delta-net
recurrent-state head tiles, the encoded projection, the windowed decode step,
its window-boundary refit and the LQCAPS01 capsule wire format, behind the
reference's ``statecentric_gdn_state_codec_*`` C-ABI."""

from ._native import NativeLibrary, library_dir, library_path, native
from .codec import (
    LAYOUT_KEY_VALUE,
    LAYOUT_VALUE_KEY,
    decode,
    encode,
    pool_decode,
    pool_encode,
    project_chunked,
    project_decode,
)
from .capsule import CapsuleIdentity
from .runtime import GdnStateCodecExperiment, GdnStateCodecRuntime
from .window import DecodeRuntime, WindowSlot

__all__ = [
    "CapsuleIdentity",
    "LAYOUT_KEY_VALUE",
    "LAYOUT_VALUE_KEY",
    "DecodeRuntime",
    "GdnStateCodecExperiment",
    "GdnStateCodecRuntime",
    "WindowSlot",
    "NativeLibrary",
    "decode",
    "encode",
    "library_dir",
    "library_path",
    "native",
    "pool_decode",
    "pool_encode",
    "project_chunked",
    "project_decode",
]
