"""Compressed-slot runtime of the GDN state codec on MI355X.

The reference keeps, per GDN layer, a map from the vLLM cache index to an
encoded slot and advances the slot one decode token at a time
(``src/gdn_state_codec/runtime.py:275-868``).  This module offers the same
service on the gfx950 library, assembled from this package's own parts:

* :class:`_GdnStateCodecLibraries` resolves every entry point through the
  library file names the reference's ``ctypes`` loader opens
  (``runtime.py:48-274``), so a library directory laid out for the reference
  serves this runtime unchanged;
* a :class:`_Slot` is a :class:`~gdn_state_codec.window.WindowSlot` (the live
  boundary and its 16-record window) plus a spare boundary generation: a
  window-boundary refit writes the spare and the two trade places, so the
  refit never reads and writes the same buffers;
* :class:`GdnStateCodecRuntime` owns the slots of one layer: it encodes a
  provider state on the first decode of a cache index, validates every token's
  tensors against a contract fixed by the slot's head count, folds a full
  window into a new boundary before the next token, and runs the vector or
  cube decode backend.

The interface is the reference runtime's: the method names
(``_encode_quant_only_provider``, ``_encode_dense_boundary``, ``reconstruct``,
``project``, ``_slot``, ``invalidate``, ``decode_fallback_reason``,
``fall_back_to_native``, ``step``), the slot buffer names, the fallback reason
keys, the two initializers (``quant_only`` and ``exact_svd``, the latter by
the library's Jacobi SVD kernel instead of ``torch.linalg.svd``), and
``RuntimeError`` for a violated contract or a non-zero launch status.  vLLM
configuration parsing and the shadow observers are not part of this build;
:class:`GdnStateCodecExperiment` carries only the fields read here.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from pathlib import Path
from typing import Callable

import torch

from . import codec
from ._native import OTHER_SIGNATURES, SIGNATURES, library_dir as default_library_dir
from .window import POSITION_STRIDE, RANK, WINDOW, WindowSlot

DIM = 128
QWEN_QUERY_SCALE = DIM ** -0.5
# The reference's provider launchers admit at most 64 states per call
# (gdn_state_codec_quantize.cpp:207-211); larger slots use the batched encode.
PROVIDER_LAUNCH_STATES = 64
# The Cube-backed refit entry points admit at most 128 states
# (window_boundary.cpp:698-703, 724-731).
CUBE_REFIT_STATES = 128


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
        if self.initializer not in ("quant_only", "exact_svd"):
            raise RuntimeError(f"gdn_state_codec.initializer {self.initializer!r} is neither "
                               "'quant_only' nor 'exact_svd'")
        if (not isinstance(self.boundary_power_iterations, int)
                or isinstance(self.boundary_power_iterations, bool)
                or not 0 <= self.boundary_power_iterations <= 32):
            raise RuntimeError("gdn_state_codec.boundary_power_iterations must be in [0,32]")
        # A fitted boundary is refitted by power iteration: the Cube refit
        # that runs with no iterations zeroes the compensators (config.py:77-86).
        if self.boundary_power_iterations == 0 and self.initializer != "quant_only":
            raise RuntimeError("gdn_state_codec: the exact_svd initializer needs "
                               "boundary_power_iterations in [1,32]")
        if self.decode_backend not in ("vector", "cube"):
            raise RuntimeError("gdn_state_codec.decode_backend must be 'vector' or 'cube'")


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
        "exact_svd_boundary": ("libstatecentric_gdn_state_codec_quantize_kernel.so",
                               "statecentric_gdn_state_codec_exact_svd_boundary_launch_v1"),
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


# ------------------------------------------------------------------- slots

_BOUNDARY_FIELDS = ("residual", "smoothing", "scales", "compensator_keys",
                    "compensator_values")


@dataclass
class _Generation:
    """One encoded boundary of H heads: int8 codes [H][value][key], fp32
    smoothing [H][key] and scales [H][value], fp16 rank-4 compensators."""

    residual: torch.Tensor
    smoothing: torch.Tensor
    scales: torch.Tensor
    compensator_keys: torch.Tensor
    compensator_values: torch.Tensor

    def blank(self) -> "_Generation":
        """Uninitialised buffers of the same geometry (a refit's destination)."""
        return _Generation(*(torch.empty_like(getattr(self, name)) for name in _BOUNDARY_FIELDS))


class _Slot:
    """The compressed state of one cache index.

    ``window`` holds the live boundary and its record window in the layout the
    step and refit kernels read; ``spare`` is the boundary generation the next
    refit writes.  ``residual_workspace`` serves the refit (the power
    iteration's fitted residual, or the Cube record merge), ``scaled_record_keys``
    the Cube record scaling, ``output`` the step's bf16 result.  ``steps``
    counts the tokens recorded since the live boundary was formed."""

    def __init__(self, boundary: _Generation) -> None:
        heads = boundary.residual.shape[0]
        device = boundary.residual.device
        self.window = WindowSlot(
            *(getattr(boundary, name) for name in _BOUNDARY_FIELDS),
            record_decay=torch.ones((heads, WINDOW), dtype=torch.float32, device=device),
            record_keys=torch.zeros((heads, WINDOW, DIM), dtype=torch.float16, device=device),
            record_corrections=torch.zeros((heads, WINDOW, DIM), dtype=torch.float16,
                                           device=device),
            positions=torch.zeros((heads, POSITION_STRIDE), dtype=torch.int32, device=device))
        self.spare = boundary.blank()
        self.residual_workspace = torch.empty((heads, DIM, DIM), dtype=torch.float32,
                                              device=device)
        self.scaled_record_keys = torch.empty((heads, WINDOW, DIM), dtype=torch.float16,
                                              device=device)
        self.output = torch.empty((1, 1, heads, DIM), dtype=torch.bfloat16, device=device)
        self.steps = 0

    @property
    def heads(self) -> int:
        return self.window.states

    @property
    def window_full(self) -> bool:
        return self.steps >= WINDOW

    def trade_generations(self) -> None:
        """Make the freshly written spare boundary live; the old one becomes the spare."""
        for name in _BOUNDARY_FIELDS:
            live, fresh = getattr(self.window, name), getattr(self.spare, name)
            setattr(self.window, name, fresh)
            setattr(self.spare, name, live)
        self.steps = 0

    def __getattr__(self, name: str):
        # The slot buffer names of the reference runtime (runtime.py:25-45)
        # read through to the live window.
        window = self.__dict__.get("window")
        if window is not None and name in WindowSlot.__dataclass_fields__:
            return getattr(window, name)
        raise AttributeError(name)


# ---------------------------------------------------------- token contract

@dataclass(frozen=True)
class _Expect:
    shape: tuple
    dtype: torch.dtype


def _token_contract(heads: int) -> dict[str, _Expect]:
    """The tensors of one Qwen3.5 decode token for a slot of `heads` value
    heads: query and key per GQA pair, value per head, gate inputs per head."""
    pair = (1, 1, heads // 2, DIM)
    return {"query": _Expect(pair, torch.bfloat16), "key": _Expect(pair, torch.bfloat16),
            "value": _Expect((1, 1, heads, DIM), torch.bfloat16),
            "log_decay": _Expect((1, 1, heads), torch.float32),
            "beta": _Expect((1, 1, heads), torch.bfloat16)}


def _enforce(tensor: torch.Tensor, what: str, expect: _Expect, device) -> None:
    if (not isinstance(tensor, torch.Tensor) or tuple(tensor.shape) != expect.shape
            or tensor.dtype != expect.dtype or not tensor.is_contiguous()
            or tensor.device != device):
        got = (f"{tensor.dtype} {tuple(tensor.shape)} on {tensor.device}, "
               f"{'' if tensor.is_contiguous() else 'not '}contiguous"
               if isinstance(tensor, torch.Tensor) else type(tensor).__name__)
        raise RuntimeError(f"GDN State Codec: {what} must be a contiguous {expect.dtype} "
                           f"tensor {expect.shape} on {device}; got {got}")


def _launched(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"GDN State Codec {what} returned status {status}")


# ------------------------------------------------------------------ runtime

# Why a decode invocation must use the dense recurrent op, tested in order
# (the reference's reason keys, runtime.py:567-585).
_FALLBACK_RULES: tuple[tuple[str, Callable[..., bool]], ...] = (
    ("speculative decode", lambda p, d, spec, n: spec),
    ("mixed prefill/decode batch", lambda p, d, spec, n: p > 0 and d > 0),
    ("multi-request decode batch",
     lambda p, d, spec, n: d > 0 and (d != 1 or (n is not None and n != 1))),
)


class GdnStateCodecRuntime:
    """The compressed slots of one GDN layer: quant-only initializer, windowed
    decode step on the vector or cube backend, window-boundary refit."""

    def __init__(self, experiment: GdnStateCodecExperiment | None = None,
                 prefix: str = "", library_dir: Path | None = None) -> None:
        if experiment is None:
            experiment = GdnStateCodecExperiment(
                library_dir=Path(library_dir or default_library_dir()))
        self.experiment = experiment
        self.prefix = prefix
        self._libraries = _GdnStateCodecLibraries(experiment.library_dir)
        self._slots: dict[int, _Slot] = {}
        self._contracts: dict[int, dict[str, _Expect]] = {}
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

    @property
    def _compensated(self) -> bool:
        """Whether the slots can carry non-zero compensators: an exact-SVD
        boundary, or any boundary after a power-iteration refit."""
        return (self.experiment.initializer != "quant_only"
                or self.experiment.boundary_power_iterations > 0)

    @property
    def _cube_refit(self) -> bool:
        """The quant-only refit folds the records with the Cube record GEMM, as
        the reference runtime does when no power iterations are configured."""
        return self.experiment.boundary_power_iterations == 0

    # -- slot map ------------------------------------------------------------

    def _slot(self, provider_state: torch.Tensor, cache_index: int) -> _Slot:
        """The slot of `cache_index`, encoded from provider_state[cache_index]
        on first use."""
        slot = self._slots.get(cache_index)
        if slot is None:
            if not 0 <= cache_index < provider_state.shape[0]:
                raise RuntimeError(f"GDN State Codec: cache index {cache_index} is out of range "
                                   f"for a provider state of {provider_state.shape[0]} slots")
            if self.experiment.initializer == "quant_only":
                slot = self._encode_quant_only_provider(provider_state[cache_index])
            else:
                slot = self._encode_exact_svd_provider(provider_state[cache_index])
            if self._cube_refit:
                self._libraries.boundary_handle(slot.heads)
            self._slots[cache_index] = slot
        return slot

    def invalidate(self, cache_indices) -> None:
        """Forget the slots of `cache_indices` (their dense state changed)."""
        for cache_index in cache_indices:
            self._slots.pop(cache_index, None)

    @staticmethod
    def decode_fallback_reason(*, num_prefills: int, num_decodes: int, speculative: bool,
                               cache_index_count: int | None = None) -> str | None:
        """The reason key when this invocation must use the dense op, else None."""
        for reason, applies in _FALLBACK_RULES:
            if applies(num_prefills, num_decodes, speculative, cache_index_count):
                return reason
        return None

    def fall_back_to_native(self, reason: str) -> None:
        """Drop every slot before the dense op updates the provider state, and count why."""
        self._slots.clear()
        self.native_fallbacks += 1
        self.native_fallback_reasons[reason] = self.native_fallback_reasons.get(reason, 0) + 1

    # -- boundary ------------------------------------------------------------

    @staticmethod
    def _provider_boundary(provider_dense: torch.Tensor) -> _Generation:
        """Checks one provider state [H][value][key] fp32 (device, contiguous)
        and allocates the boundary generation it encodes into."""
        if provider_dense.ndim != 3:
            raise RuntimeError("GDN State Codec: the provider state must be [H,128,128] "
                               f"(value x key per head), got {tuple(provider_dense.shape)}")
        _enforce(provider_dense, "the provider state",
                 _Expect((provider_dense.shape[0], DIM, DIM), torch.float32),
                 provider_dense.device)
        if not provider_dense.is_cuda:
            raise RuntimeError("GDN State Codec: the provider state must live on the GPU")
        heads, device = provider_dense.shape[0], provider_dense.device
        return _Generation(
            residual=torch.empty((heads, DIM, DIM), dtype=torch.int8, device=device),
            smoothing=torch.empty((heads, DIM), dtype=torch.float32, device=device),
            scales=torch.empty((heads, DIM), dtype=torch.float32, device=device),
            compensator_keys=torch.zeros((heads, DIM, RANK), dtype=torch.float16, device=device),
            compensator_values=torch.zeros((heads, DIM, RANK), dtype=torch.float16,
                                           device=device))

    def _encode_quant_only_provider(self, provider_dense: torch.Tensor) -> _Slot:
        """A new slot from one provider state [H][value][key] fp32 (device,
        contiguous): codes, smoothing and scales of the quant-only initializer,
        zero compensators, an empty window."""
        boundary = self._provider_boundary(provider_dense)
        heads = provider_dense.shape[0]
        source = provider_dense.data_ptr()
        codes, smoothing, scales = (boundary.residual.data_ptr(), boundary.smoothing.data_ptr(),
                                    boundary.scales.data_ptr())
        if heads <= PROVIDER_LAUNCH_STATES:  # the reference's own v3 entry point
            _launched(self._libraries.provider_initialize(self._stream(), source, smoothing,
                                                          codes, scales, heads),
                      "provider initialize")
        else:
            _launched(self._libraries.encode(self._stream(), source, codes, smoothing, scales,
                                             heads, codec.LAYOUT_VALUE_KEY), "batched encode")
        return _Slot(boundary)

    def _encode_exact_svd_provider(self, provider_dense: torch.Tensor) -> _Slot:
        """A new slot from one provider state [H][value][key] fp32 with the
        exact-SVD initializer (runtime.py:335-389): fp16 rank-4 compensators
        U*S and V of each dense head's truncated SVD, and the quant-only codes
        of the residual, by one launch of the library's Jacobi SVD.  Raises
        for a head with a non-finite value or one whose iteration did not
        converge."""
        boundary = self._provider_boundary(provider_dense)
        heads = provider_dense.shape[0]
        slot = _Slot(boundary)
        status = torch.empty((heads,), dtype=torch.int32, device=provider_dense.device)
        _launched(self._libraries.exact_svd_boundary(
            self._stream(), provider_dense.data_ptr(), slot.residual_workspace.data_ptr(),
            boundary.residual.data_ptr(), boundary.smoothing.data_ptr(),
            boundary.scales.data_ptr(), boundary.compensator_keys.data_ptr(),
            boundary.compensator_values.data_ptr(), status.data_ptr(), heads),
            "exact SVD initializer")
        flat = status.cpu()
        rejected = torch.nonzero(flat).reshape(-1)
        if rejected.numel():
            head = int(rejected[0])
            raise RuntimeError(f"GDN State Codec exact SVD initializer: head {head} "
                               f"{codec.SVD_STATUS.get(int(flat[head]), 'failed')}")
        return slot

    def _encode_dense_boundary(self, dense: torch.Tensor,
                               initializer: str = "exact_svd") -> _Slot:
        """A new slot from dense [H][key][value] heads (the reference's entry,
        runtime.py:335-389): the provider layout is their transpose."""
        if dense.ndim != 3 or tuple(dense.shape[-2:]) != (DIM, DIM):
            raise RuntimeError("GDN State Codec: dense boundaries must be [H,128,128] "
                               f"(key x value per head), got {tuple(dense.shape)}")
        provider = dense.to(torch.float32).transpose(-2, -1).contiguous()
        if initializer == "exact_svd":
            return self._encode_exact_svd_provider(provider)
        if initializer == "quant_only":
            return self._encode_quant_only_provider(provider)
        raise RuntimeError(f"GDN State Codec: no initializer named {initializer!r}")

    def reconstruct(self, slot: _Slot) -> torch.Tensor:
        """The dense [H][key][value] fp32 boundary of a slot, dequantized on the
        GPU in the portable reference's rounding order ((s * code) / 127) * scale,
        plus the rank-4 compensator product keys * values^T when the slots can
        carry one (the reference's reconstruct, runtime.py:550-561)."""
        dense = torch.empty((slot.heads, DIM, DIM), dtype=torch.float32,
                            device=slot.window.device)
        keys = values = None
        if self._compensated:  # fp16 -> fp32 widening is exact
            keys = slot.compensator_keys.to(torch.float32)
            values = slot.compensator_values.to(torch.float32)
        _launched(self._libraries.decode(
            self._stream(), slot.residual.data_ptr(), slot.smoothing.data_ptr(),
            slot.scales.data_ptr(), None if keys is None else keys.data_ptr(),
            None if values is None else values.data_ptr(), dense.data_ptr(), slot.heads,
            codec.LAYOUT_VALUE_KEY), "decode")
        return dense.transpose(-2, -1)

    def project(self, slot: _Slot, query: torch.Tensor,
                query_scale: float = QWEN_QUERY_SCALE) -> torch.Tensor:
        """The readout of a slot's quantized boundary residual for one decode
        query, [1,1,H/2,128] bf16 (value head h reads query head h/2); returns
        [1,1,H,128] fp32.  This is the encoded projection's contract: the
        compensator term is not part of it."""
        _enforce(query, "the query", _Expect((1, 1, slot.heads // 2, DIM), torch.bfloat16),
                 slot.window.device)
        out = torch.empty((1, 1, slot.heads, DIM), dtype=torch.float32,
                          device=slot.window.device)
        _launched(self._libraries.project_decode(
            self._stream(), slot.residual.data_ptr(), slot.smoothing.data_ptr(),
            slot.scales.data_ptr(), query.data_ptr(), out.data_ptr(), 1, slot.heads,
            slot.heads // 2, float(query_scale), codec.LAYOUT_VALUE_KEY), "projection")
        return out

    def _refit_boundary(self, slot: _Slot) -> None:
        """Fold the slot's full window into a new boundary in its spare
        generation, then make that generation live.  With no power iterations
        the records are merged by the Cube record GEMM and requantized with the
        existing smoothing; otherwise the rank-4 power iteration refits."""
        stream, heads = self._stream(), slot.heads
        destination = (slot.spare.residual.data_ptr(), slot.spare.smoothing.data_ptr(),
                       slot.spare.scales.data_ptr(), slot.spare.compensator_keys.data_ptr(),
                       slot.spare.compensator_values.data_ptr())
        if self._cube_refit:
            if heads > CUBE_REFIT_STATES:
                raise RuntimeError(f"GDN State Codec: the Cube refit serves at most "
                                   f"{CUBE_REFIT_STATES} heads, this slot has {heads}")
            merge = slot.residual_workspace
            _launched(self._libraries.boundary_runtime_step(
                self._libraries.boundary_handle(heads), stream, slot.record_decay.data_ptr(),
                slot.record_keys.data_ptr(), slot.record_corrections.data_ptr(),
                slot.scaled_record_keys.data_ptr(), merge.data_ptr(), heads),
                "Cube record merge")
            _launched(self._libraries.window_boundary_cube_finish(
                stream, *slot.window.pointers(), *destination, merge.data_ptr(), heads),
                "Cube refit")
        else:
            _launched(self._libraries.window_boundary(
                stream, *slot.window.pointers(), *destination,
                slot.residual_workspace.data_ptr(), heads,
                self.experiment.boundary_power_iterations), "power refit")
        slot.trade_generations()
        self.boundary_refits += 1

    # -- decode --------------------------------------------------------------

    def step(self, provider_state: torch.Tensor, cache_index: int, query: torch.Tensor,
             key: torch.Tensor, value: torch.Tensor, log_decay: torch.Tensor,
             beta: torch.Tensor, query_scale: float) -> torch.Tensor:
        """One decode token of one request: the slot of `cache_index` (encoded
        on first use) refits its boundary if its window is full, then takes the
        windowed step.  Returns the bf16 output [1,1,H,128] (the slot's buffer)."""
        slot = self._slot(provider_state, cache_index)
        if slot.steps > WINDOW:
            raise RuntimeError("GDN State Codec: slot window holds more than 16 records")
        if slot.window_full:
            self._refit_boundary(slot)
        contract = self._contracts.get(slot.heads)
        if contract is None:
            contract = self._contracts.setdefault(slot.heads, _token_contract(slot.heads))
        device = slot.window.device
        for what, tensor in (("query", query), ("key", key), ("value", value),
                             ("log_decay", log_decay), ("beta", beta)):
            _enforce(tensor, what, contract[what], device)
        if abs(query_scale - QWEN_QUERY_SCALE) > 1.0e-8:
            raise RuntimeError(f"GDN State Codec: the decode kernels apply Qwen3.5's query "
                               f"scale 128^-1/2, not {query_scale}")
        operands = (*slot.window.pointers(), log_decay.data_ptr(), beta.data_ptr(),
                    key.data_ptr(), query.data_ptr(), value.data_ptr(), slot.output.data_ptr(),
                    slot.heads)
        if self.experiment.decode_backend == "cube":
            status = self._libraries.decode_runtime_step(
                self._libraries.decode_handle(slot.heads), self._stream(), *operands)
        elif self.experiment.boundary_power_iterations == 0:
            status = self._libraries.window_step_bf16_quant_only(self._stream(), *operands)
        else:
            status = self._libraries.window_step_bf16(self._stream(), *operands)
        _launched(status, f"{self.experiment.decode_backend} decode step")
        slot.steps += 1
        return slot.output
