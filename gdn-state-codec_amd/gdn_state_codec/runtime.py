"""Slot runtime for the GDN state codec on MI355X.

Mirrors the device-facing part of the reference's ``GdnStateCodecRuntime``
(``src/gdn_state_codec/runtime.py``):

* the library loader keyed on the reference's library file names and symbols
  (``_GdnStateCodecLibraries``, ``:48-274``), including the decode and boundary
  runtime handles;
* quant-only slot encoding of a provider state ``[H,V,K]``
  (``_encode_quant_only_provider``, ``:460-547``) and the slot buffers
  (``_allocate_slot``, ``:392-458``);
* the per-token windowed decode ``step`` on the vector or cube backend
  (``:750-843``) and the window-boundary refit every 16 tokens
  (``_refit_boundary``, ``:627-741``);
* the slot map keyed on the cache index, invalidation, fallback bookkeeping
  and ``reconstruct`` (``:549-625``).

Names, argument meaning and error behaviour follow the reference: contract
violations and non-zero launch statuses raise ``RuntimeError``.  The vLLM
configuration parsing, shadow observers and the exact-SVD initializer are not
part of this build; :class:`GdnStateCodecExperiment` carries only the fields
the runtime reads.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from pathlib import Path

import torch

from . import codec
from ._native import OTHER_SIGNATURES, SIGNATURES, library_dir as default_library_dir

KEY_DIMENSION = 128
VALUE_DIMENSION = 128
COMPENSATOR_RANK = 4
WINDOW_SIZE = 16
POSITION_STRIDE = 8
# Provider-launch admission of the reference (gdn_state_codec_quantize.cpp:207-211).
PROVIDER_STATE_LIMIT = 64


@dataclass
class GdnStateCodecExperiment:
    """The experiment fields the runtime reads (src/gdn_state_codec/config.py:20-100)."""

    library_dir: Path = field(default_factory=default_library_dir)
    initializer: str = "quant_only"
    boundary_power_iterations: int = 0
    decode_backend: str = "vector"
    mode: str = "serve"

    def __post_init__(self) -> None:
        self.library_dir = Path(self.library_dir)
        if self.initializer != "quant_only":
            raise RuntimeError("GDN State Codec on MI355X supports the quant_only initializer")
        if (not isinstance(self.boundary_power_iterations, int)
                or not 0 <= self.boundary_power_iterations <= 32):
            raise RuntimeError("gdn_state_codec.boundary_power_iterations must be in [0,32]")
        if self.decode_backend not in ("vector", "cube"):
            raise RuntimeError("gdn_state_codec.decode_backend must be 'vector' or 'cube'")


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
    scratch_residual: torch.Tensor
    scratch_smoothing: torch.Tensor
    scratch_scales: torch.Tensor
    scratch_compensator_keys: torch.Tensor
    scratch_compensator_values: torch.Tensor
    residual_workspace: torch.Tensor
    scaled_record_keys: torch.Tensor
    output: torch.Tensor
    kernel_state_pointers: tuple[int, ...] = ()
    steps: int = 0


class _GdnStateCodecLibraries:
    """Loads the entry points by the reference's library file names."""

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
        "window_step": ("libstatecentric_gdn_state_codec_windowed_gdn_step_kernel.so",
                        "statecentric_gdn_state_codec_windowed_gdn_step_launch_v1"),
        "window_step_bf16": ("libstatecentric_gdn_state_codec_windowed_gdn_step_kernel.so",
                             "statecentric_gdn_state_codec_windowed_gdn_step_bf16_launch_v1"),
        "window_step_bf16_quant_only": (
            "libstatecentric_gdn_state_codec_windowed_gdn_step_kernel.so",
            "statecentric_gdn_state_codec_windowed_gdn_step_bf16_quant_only_launch_v1"),
        "window_boundary": ("libstatecentric_gdn_state_codec_window_boundary_kernel.so",
                            "statecentric_gdn_state_codec_window_boundary_launch_v1"),
        "window_boundary_cube_finish": (
            "libstatecentric_gdn_state_codec_window_boundary_kernel.so",
            "statecentric_gdn_state_codec_window_boundary_cube_finish_launch_v1"),
        "boundary_runtime_step": ("libstatecentric_gdn_state_codec_boundary_runtime.so",
                                  "statecentric_gdn_state_codec_boundary_runtime_step_v1"),
        "decode_runtime_step": ("libstatecentric_gdn_state_codec_decode_runtime.so",
                                "statecentric_gdn_state_codec_decode_runtime_step_v1"),
    }
    _HANDLES = {
        "_decode_runtime_create": ("libstatecentric_gdn_state_codec_decode_runtime.so",
                                   "statecentric_gdn_state_codec_decode_runtime_create_v1"),
        "_decode_runtime_destroy": ("libstatecentric_gdn_state_codec_decode_runtime.so",
                                    "statecentric_gdn_state_codec_decode_runtime_destroy_v1"),
        "_boundary_runtime_create": ("libstatecentric_gdn_state_codec_boundary_runtime.so",
                                     "statecentric_gdn_state_codec_boundary_runtime_create_v1"),
        "_boundary_runtime_destroy": ("libstatecentric_gdn_state_codec_boundary_runtime.so",
                                      "statecentric_gdn_state_codec_boundary_runtime_destroy_v1"),
    }

    def __init__(self, library_dir: Path) -> None:
        self._handles: dict[str, ctypes.CDLL] = {}
        for attribute, (file_name, symbol) in self._NAMES.items():
            fn = getattr(self._open(library_dir, file_name), symbol)
            fn.argtypes = SIGNATURES[symbol]
            fn.restype = ctypes.c_int32
            setattr(self, attribute, fn)
        for attribute, (file_name, symbol) in self._HANDLES.items():
            fn = getattr(self._open(library_dir, file_name), symbol)
            fn.argtypes, fn.restype = OTHER_SIGNATURES[symbol]
            setattr(self, attribute, fn)
        self._decode_handle: int | None = None
        self._boundary_handle: int | None = None

    def _open(self, library_dir: Path, file_name: str) -> ctypes.CDLL:
        path = library_dir / file_name
        if not path.is_file():
            raise RuntimeError(f"GDN State Codec native library is missing: {path}")
        return self._handles.setdefault(file_name, ctypes.CDLL(str(path)))

    def decode_handle(self, states: int) -> int:
        if self._decode_handle is None:
            handle = self._decode_runtime_create(states)
            if not handle:
                raise RuntimeError("GDN State Codec Cube decode runtime creation failed")
            self._decode_handle = int(handle)
        return self._decode_handle

    def boundary_handle(self, states: int) -> int:
        if self._boundary_handle is None:
            handle = self._boundary_runtime_create(states)
            if not handle:
                raise RuntimeError("GDN State Codec Cube boundary runtime creation failed")
            self._boundary_handle = int(handle)
        return self._boundary_handle

    def close(self) -> None:
        if self._decode_handle is not None:
            self._decode_runtime_destroy(self._decode_handle)
            self._decode_handle = None
        if self._boundary_handle is not None:
            self._boundary_runtime_destroy(self._boundary_handle)
            self._boundary_handle = None


class GdnStateCodecRuntime:
    """Per-layer compressed-slot runtime: quant-only initializer, windowed
    decode step, window-boundary refit."""

    def __init__(self, experiment: GdnStateCodecExperiment | None = None,
                 prefix: str = "", library_dir: Path | None = None) -> None:
        if experiment is None:
            experiment = GdnStateCodecExperiment(
                library_dir=Path(library_dir or default_library_dir()))
        self.experiment = experiment
        self.prefix = prefix
        self._libraries = _GdnStateCodecLibraries(experiment.library_dir)
        self._slots: dict[int, _EncodedSlot] = {}
        self._input_contract_validated = False
        self.boundary_refits = 0
        self.native_fallbacks = 0
        self.native_fallback_reasons: dict[str, int] = {}

    def close(self) -> None:
        """Release the decode / boundary runtime handles (also done on deletion)."""
        libraries = getattr(self, "_libraries", None)
        if libraries is not None:
            libraries.close()

    def __del__(self) -> None:
        self.close()

    @staticmethod
    def _stream() -> int:
        return torch.cuda.current_stream().cuda_stream

    @staticmethod
    def _allocate_slot(residual, smoothing, scales, compensator_keys,
                       compensator_values) -> _EncodedSlot:
        heads = residual.shape[0]
        device = residual.device
        record_keys = torch.zeros((heads, WINDOW_SIZE, KEY_DIMENSION),
                                  dtype=torch.float16, device=device)
        slot = _EncodedSlot(
            # [value,key]: one contiguous 128-byte int8 row per output value.
            residual=residual,
            smoothing=smoothing,
            scales=scales,
            compensator_keys=compensator_keys,
            compensator_values=compensator_values,
            record_decay=torch.ones((heads, WINDOW_SIZE), dtype=torch.float32, device=device),
            record_keys=record_keys,
            record_corrections=torch.zeros((heads, WINDOW_SIZE, VALUE_DIMENSION),
                                           dtype=torch.float16, device=device),
            # Read by the kernels as uint32 window positions.
            positions=torch.zeros((heads, POSITION_STRIDE), dtype=torch.int32, device=device),
            scratch_residual=torch.empty_like(residual),
            scratch_smoothing=torch.empty_like(smoothing),
            scratch_scales=torch.empty_like(scales),
            scratch_compensator_keys=torch.empty_like(compensator_keys),
            scratch_compensator_values=torch.empty_like(compensator_values),
            residual_workspace=torch.empty(residual.shape, dtype=torch.float32, device=device),
            scaled_record_keys=torch.empty_like(record_keys),
            output=torch.empty((1, 1, heads, VALUE_DIMENSION), dtype=torch.bfloat16,
                               device=device),
        )
        slot.kernel_state_pointers = GdnStateCodecRuntime._pointers(slot)
        return slot

    @staticmethod
    def _pointers(slot: _EncodedSlot) -> tuple[int, ...]:
        return (slot.residual.data_ptr(), slot.smoothing.data_ptr(), slot.scales.data_ptr(),
                slot.compensator_keys.data_ptr(), slot.compensator_values.data_ptr(),
                slot.record_decay.data_ptr(), slot.record_keys.data_ptr(),
                slot.record_corrections.data_ptr(), slot.positions.data_ptr())

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
        """Dense [H,K,V] fp32 boundary of a quant-only slot, dequantized on the GPU.

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
        out = torch.empty((1, 1, heads, VALUE_DIMENSION), dtype=torch.float32,
                          device=slot.residual.device)
        status = self._libraries.project_decode(
            self._stream(), slot.residual.data_ptr(), slot.smoothing.data_ptr(),
            slot.scales.data_ptr(), query.data_ptr(), out.data_ptr(), 1, heads,
            heads // 2, float(query_scale), codec.LAYOUT_VALUE_KEY)
        if status != 0:
            raise RuntimeError(f"GDN State Codec projection launch failed: {status}")
        return out

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

    def _use_cube_boundary(self) -> bool:
        return self.experiment.boundary_power_iterations == 0

    def _slot(self, provider_state: torch.Tensor, cache_index: int) -> _EncodedSlot:
        slot = self._slots.get(cache_index)
        if slot is not None:
            return slot
        if cache_index < 0 or cache_index >= provider_state.shape[0]:
            raise RuntimeError("GDN State Codec cache index is out of range")
        slot = self._encode_quant_only_provider(provider_state[cache_index])
        if self._use_cube_boundary():
            self._libraries.boundary_handle(slot.residual.shape[0])
        self._slots[cache_index] = slot
        return slot

    def _refit_boundary(self, slot: _EncodedSlot) -> None:
        """Fold a full window into a new boundary (runtime.py:627-741): the cube
        record merge plus quant-only refit, or the power-iteration refit."""
        stream = self._stream()
        heads = slot.residual.shape[0]
        use_cube = self._use_cube_boundary()
        if use_cube:
            handle = self._libraries.boundary_handle(heads)
            status = self._libraries.boundary_runtime_step(
                handle, stream, slot.record_decay.data_ptr(), slot.record_keys.data_ptr(),
                slot.record_corrections.data_ptr(), slot.scaled_record_keys.data_ptr(),
                slot.residual_workspace.data_ptr(), heads)
            if status != 0:
                raise RuntimeError(f"GDN State Codec Cube boundary merge failed: {status}")
        pointers = (stream, *self._pointers(slot), slot.scratch_residual.data_ptr(),
                    slot.scratch_smoothing.data_ptr(), slot.scratch_scales.data_ptr(),
                    slot.scratch_compensator_keys.data_ptr(),
                    slot.scratch_compensator_values.data_ptr(),
                    slot.residual_workspace.data_ptr())
        if use_cube:
            status = self._libraries.window_boundary_cube_finish(*pointers, heads)
        else:
            status = self._libraries.window_boundary(
                *pointers, heads, self.experiment.boundary_power_iterations)
        if status != 0:
            raise RuntimeError(f"GDN State Codec boundary-refit launch failed: {status}")
        slot.residual, slot.scratch_residual = slot.scratch_residual, slot.residual
        slot.smoothing, slot.scratch_smoothing = slot.scratch_smoothing, slot.smoothing
        slot.scales, slot.scratch_scales = slot.scratch_scales, slot.scales
        slot.compensator_keys, slot.scratch_compensator_keys = (
            slot.scratch_compensator_keys, slot.compensator_keys)
        slot.compensator_values, slot.scratch_compensator_values = (
            slot.scratch_compensator_values, slot.compensator_values)
        slot.kernel_state_pointers = self._pointers(slot)
        slot.steps = 0
        self.boundary_refits += 1

    def step(self, provider_state: torch.Tensor, cache_index: int, query: torch.Tensor,
             key: torch.Tensor, value: torch.Tensor, log_decay: torch.Tensor,
             beta: torch.Tensor, query_scale: float) -> torch.Tensor:
        """One decode token of one request (runtime.py:750-843): refit a full
        window first, then the windowed step; returns bf16 [1,1,H,128]."""
        slot = self._slot(provider_state, cache_index)
        if slot.steps == WINDOW_SIZE:
            self._refit_boundary(slot)
        elif slot.steps > WINDOW_SIZE:
            raise RuntimeError("GDN State Codec runtime window position exceeded p=16")
        heads = slot.residual.shape[0]
        if not self._input_contract_validated:
            query_shape = (1, 1, heads // 2, KEY_DIMENSION)
            if tuple(query.shape) != query_shape or tuple(key.shape) != query_shape:
                raise RuntimeError("GDN State Codec Qwen3.5 gate requires [1,1,H/2,128] query/key")
            if tuple(value.shape) != (1, 1, heads, VALUE_DIMENSION):
                raise RuntimeError("GDN State Codec Qwen3.5 gate requires [1,1,H,128] value")
            if tuple(log_decay.shape) != (1, 1, heads) or tuple(beta.shape) != (1, 1, heads):
                raise RuntimeError("GDN State Codec Qwen3.5 gate requires [1,1,H] decay/beta")
            if log_decay.dtype != torch.float32:
                raise RuntimeError("GDN State Codec Qwen3.5 gate requires FP32 log decay")
            if query.dtype != torch.bfloat16 or key.dtype != torch.bfloat16:
                raise RuntimeError("GDN State Codec Qwen3.5 gate requires BF16 query/key")
            if value.dtype != torch.bfloat16 or beta.dtype != torch.bfloat16:
                raise RuntimeError("GDN State Codec Qwen3.5 gate requires BF16 value/beta")
            if abs(query_scale - KEY_DIMENSION ** -0.5) > 1.0e-8:
                raise RuntimeError("GDN State Codec Qwen3.5 query scale is unsupported")
            if not all(t.is_contiguous() for t in (query, key, value, log_decay, beta)):
                raise RuntimeError("GDN State Codec Qwen3.5 inputs must be contiguous")
            self._input_contract_validated = True
        pointers = (self._stream(), *slot.kernel_state_pointers, log_decay.data_ptr(),
                    beta.data_ptr(), key.data_ptr(), query.data_ptr(), value.data_ptr(),
                    slot.output.data_ptr())
        if self.experiment.decode_backend == "vector":
            vector_step = (self._libraries.window_step_bf16_quant_only
                           if self.experiment.boundary_power_iterations == 0
                           else self._libraries.window_step_bf16)
            status = vector_step(*pointers, heads)
        else:
            handle = self._libraries.decode_handle(heads)
            status = self._libraries.decode_runtime_step(handle, *pointers, heads)
        if status != 0:
            raise RuntimeError(f"GDN State Codec decode-step launch failed: {status}")
        slot.steps += 1
        return slot.output
