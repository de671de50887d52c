"""Slot runtime for the GDN state codec on MI355X.

Mirrors the codec-facing part of the reference's ``GdnStateCodecRuntime``
(``src/gdn_state_codec/runtime.py``): the library loader keyed on the
reference's library file names (``:48-237``), quant-only slot encoding of a
provider state ``[H,V,K]`` (``_encode_quant_only_provider``, ``:460-547``), the
slot map keyed on the cache index (``_slot``, ``:603-625``), invalidation
(``:563-565``), the fallback bookkeeping (``:567-601``) and ``reconstruct``
(``:549-561``).  Names, argument meaning and error behaviour follow the
reference: contract violations and non-zero launch statuses raise
``RuntimeError``.  The windowed decode step and the window-boundary refit are
not part of this build; ``project`` evaluates the boundary readout the step
is built on.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from pathlib import Path

import torch

from . import codec
from ._native import SIGNATURES, library_dir as default_library_dir

KEY_DIMENSION = 128
VALUE_DIMENSION = 128
COMPENSATOR_RANK = 4
WINDOW_SIZE = 16
POSITION_STRIDE = 8
# Provider-launch admission of the reference (gdn_state_codec_quantize.cpp:207-211).
PROVIDER_STATE_LIMIT = 64


@dataclass(slots=True)
class _EncodedSlot:
    residual: torch.Tensor
    smoothing: torch.Tensor
    scales: torch.Tensor
    compensator_keys: torch.Tensor
    compensator_values: torch.Tensor
    record_decay: torch.Tensor
    record_keys: torch.Tensor
    record_corrections: torch.Tensor
    positions: torch.Tensor
    output: torch.Tensor
    steps: int = 0


class _GdnStateCodecLibraries:
    """Loads the codec entry points by the reference's library file names."""

    _NAMES = {
        "provider_smoothing": ("libstatecentric_gdn_state_codec_smoothing_kernel.so",
                               "statecentric_gdn_state_codec_provider_smoothing_launch_v2"),
        "provider_quantize": ("libstatecentric_gdn_state_codec_quantize_kernel.so",
                              "statecentric_gdn_state_codec_provider_quantize_launch_v2"),
        "provider_initialize": ("libstatecentric_gdn_state_codec_provider_runtime.so",
                                "statecentric_gdn_state_codec_provider_initialize_launch_v3"),
        "encode": ("libstatecentric_gdn_state_codec_quantize_kernel.so",
                   "statecentric_gdn_state_codec_encode_launch_v4"),
        "decode": ("libstatecentric_gdn_state_codec_dequantize_kernel.so",
                   "statecentric_gdn_state_codec_decode_launch_v4"),
        "project_decode": ("libstatecentric_gdn_state_codec_encoded_projection_kernel.so",
                           "statecentric_gdn_state_codec_encoded_projection_decode_launch_v4"),
    }

    def __init__(self, library_dir: Path) -> None:
        self._handles: dict[str, ctypes.CDLL] = {}
        for attribute, (file_name, symbol) in self._NAMES.items():
            path = library_dir / file_name
            if not path.is_file():
                raise RuntimeError(f"GDN State Codec native library is missing: {path}")
            handle = self._handles.setdefault(file_name, ctypes.CDLL(str(path)))
            fn = getattr(handle, symbol)
            fn.argtypes = SIGNATURES[symbol]
            fn.restype = ctypes.c_int32
            setattr(self, attribute, fn)


class GdnStateCodecRuntime:
    """Per-layer compressed-slot runtime (quant_only initializer)."""

    def __init__(self, library_dir: Path | None = None, prefix: str = "") -> None:
        self.prefix = prefix
        self._libraries = _GdnStateCodecLibraries(Path(library_dir or default_library_dir()))
        self._slots: dict[int, _EncodedSlot] = {}
        self.native_fallbacks = 0
        self.native_fallback_reasons: dict[str, int] = {}

    @staticmethod
    def _stream() -> int:
        return torch.cuda.current_stream().cuda_stream

    @staticmethod
    def _allocate_slot(residual, smoothing, scales, compensator_keys,
                       compensator_values) -> _EncodedSlot:
        heads = residual.shape[0]
        device = residual.device
        return _EncodedSlot(
            residual=residual,
            smoothing=smoothing,
            scales=scales,
            compensator_keys=compensator_keys,
            compensator_values=compensator_values,
            record_decay=torch.ones((heads, WINDOW_SIZE), dtype=torch.float32, device=device),
            record_keys=torch.zeros((heads, WINDOW_SIZE, KEY_DIMENSION),
                                    dtype=torch.float16, device=device),
            record_corrections=torch.zeros((heads, WINDOW_SIZE, VALUE_DIMENSION),
                                           dtype=torch.float16, device=device),
            positions=torch.zeros((heads, POSITION_STRIDE), dtype=torch.int32, device=device),
            output=torch.empty((1, 1, heads, VALUE_DIMENSION), dtype=torch.float32,
                               device=device),
        )

    def _encode_quant_only_provider(self, provider_dense: torch.Tensor) -> _EncodedSlot:
        if provider_dense.ndim != 3 or tuple(provider_dense.shape[-2:]) != (
            VALUE_DIMENSION,
            KEY_DIMENSION,
        ):
            raise RuntimeError("GDN State Codec requires provider states shaped [H,128,128]")
        if provider_dense.dtype != torch.float32:
            raise RuntimeError("GDN State Codec provider state must be FP32")
        if not provider_dense.is_contiguous():
            raise RuntimeError("GDN State Codec provider state must be contiguous")
        if not provider_dense.is_cuda:
            raise RuntimeError("GDN State Codec provider state must be a device tensor")
        heads = provider_dense.shape[0]
        device = provider_dense.device
        residual = torch.empty_like(provider_dense, dtype=torch.int8)
        smoothing = torch.empty((heads, KEY_DIMENSION), dtype=torch.float32, device=device)
        scales = torch.empty((heads, VALUE_DIMENSION), dtype=torch.float32, device=device)
        compensator_keys = torch.zeros((heads, KEY_DIMENSION, COMPENSATOR_RANK),
                                       dtype=torch.float16, device=device)
        compensator_values = torch.zeros((heads, VALUE_DIMENSION, COMPENSATOR_RANK),
                                         dtype=torch.float16, device=device)
        stream = self._stream()
        if heads <= PROVIDER_STATE_LIMIT:
            status = self._libraries.provider_initialize(
                stream, provider_dense.data_ptr(), smoothing.data_ptr(),
                residual.data_ptr(), scales.data_ptr(), heads)
            what = "provider initializer"
        else:
            status = self._libraries.encode(
                stream, provider_dense.data_ptr(), residual.data_ptr(),
                smoothing.data_ptr(), scales.data_ptr(), heads, codec.LAYOUT_VALUE_KEY)
            what = "batched provider encode"
        if status != 0:
            raise RuntimeError(f"GDN State Codec {what} launch failed: {status}")
        return self._allocate_slot(residual, smoothing, scales, compensator_keys,
                                   compensator_values)

    def reconstruct(self, slot: _EncodedSlot) -> torch.Tensor:
        """Dense [H,K,V] fp32 state of a quant-only slot, dequantized on the GPU.

        Rounds as the portable C++ DequantizeBoundary (((s*code)/127)*scale),
        which the reference's torch expression only approximates."""
        dense = torch.empty(slot.residual.shape, dtype=torch.float32,
                            device=slot.residual.device)
        status = self._libraries.decode(
            self._stream(), slot.residual.data_ptr(), slot.smoothing.data_ptr(),
            slot.scales.data_ptr(), None, None, dense.data_ptr(), slot.residual.shape[0],
            codec.LAYOUT_VALUE_KEY)
        if status != 0:
            raise RuntimeError(f"GDN State Codec decode launch failed: {status}")
        return dense.transpose(-2, -1)

    def project(self, slot: _EncodedSlot, query: torch.Tensor,
                query_scale: float = KEY_DIMENSION ** -0.5) -> torch.Tensor:
        """Boundary readout of a slot for one decode query [1,1,H/2,128] bf16.

        Returns [1,1,H,128] fp32: sum_k code(v,k) s[k] (query_scale q[h/2,k]) / 127 * scale[v]."""
        heads = slot.residual.shape[0]
        if tuple(query.shape) != (1, 1, heads // 2, KEY_DIMENSION):
            raise RuntimeError("GDN State Codec Qwen3.5 gate requires [1,1,H/2,128] query")
        if query.dtype != torch.bfloat16 or not query.is_contiguous():
            raise RuntimeError("GDN State Codec Qwen3.5 gate requires contiguous BF16 query")
        status = self._libraries.project_decode(
            self._stream(), slot.residual.data_ptr(), slot.smoothing.data_ptr(),
            slot.scales.data_ptr(), query.data_ptr(), slot.output.data_ptr(), 1, heads,
            heads // 2, float(query_scale), codec.LAYOUT_VALUE_KEY)
        if status != 0:
            raise RuntimeError(f"GDN State Codec projection launch failed: {status}")
        return slot.output

    def invalidate(self, cache_indices: tuple[int, ...]) -> None:
        for cache_index in cache_indices:
            self._slots.pop(cache_index, None)

    @staticmethod
    def decode_fallback_reason(*, num_prefills: int, num_decodes: int, speculative: bool,
                               cache_index_count: int | None = None) -> str | None:
        """Return why an invocation must use the dense recurrent op (runtime.py:567-585)."""
        if speculative:
            return "speculative decode"
        if num_prefills > 0 and num_decodes > 0:
            return "mixed prefill/decode batch"
        if num_decodes > 0 and (
            num_decodes != 1 or (cache_index_count is not None and cache_index_count != 1)
        ):
            return "multi-request decode batch"
        return None

    def fall_back_to_native(self, reason: str) -> None:
        """Discard compressed slots before the provider updates dense state."""
        self._slots.clear()
        self.native_fallbacks += 1
        self.native_fallback_reasons[reason] = self.native_fallback_reasons.get(reason, 0) + 1

    def _slot(self, provider_state: torch.Tensor, cache_index: int) -> _EncodedSlot:
        slot = self._slots.get(cache_index)
        if slot is not None:
            return slot
        if cache_index < 0 or cache_index >= provider_state.shape[0]:
            raise RuntimeError("GDN State Codec cache index is out of range")
        slot = self._encode_quant_only_provider(provider_state[cache_index])
        self._slots[cache_index] = slot
        return slot
