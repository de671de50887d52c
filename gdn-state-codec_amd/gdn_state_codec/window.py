"""torch-facing windowed decode step (include/gdn_state_codec_window.h).

A :class:`WindowSlot` holds the device buffers of one encoded slot exactly as
the reference runtime keeps them (``src/gdn_state_codec/runtime.py:25-45,
392-458``): the int8 boundary with its smoothing and scales, rank-4 fp16
compensators, the 16-record fp16 window and the [states][8] positions.  The
step functions validate shapes, dtypes and devices, then launch the gfx950
kernels on torch's current stream; a nonzero status raises ``RuntimeError``
as in ``runtime.py:514-540, 840-841``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from ._native import native

DIM = 128
RANK = 4
WINDOW = 16
POSITION_STRIDE = 8


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _check(t: torch.Tensor, name: str, shape: tuple, dtypes, device) -> None:
    if not isinstance(t, torch.Tensor):
        raise RuntimeError(f"{name} must be a tensor")
    if tuple(t.shape) != tuple(shape):
        raise RuntimeError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if t.dtype not in dtypes:
        raise RuntimeError(f"{name} has dtype {t.dtype}, expected one of {dtypes}")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")
    if t.device != device:
        raise RuntimeError(f"{name} must be on {device}")


_HALF = (torch.float16, torch.int16)
_BF16 = (torch.bfloat16, torch.int16)
_POS = (torch.int32,)


@dataclass
class WindowSlot:
    """Device buffers of `states` encoded heads plus their record window."""

    residual: torch.Tensor            # int8 [S,128,128]
    smoothing: torch.Tensor           # fp32 [S,128]
    scales: torch.Tensor              # fp32 [S,128]
    compensator_keys: torch.Tensor    # fp16 [S,128,4]
    compensator_values: torch.Tensor  # fp16 [S,128,4]
    record_decay: torch.Tensor        # fp32 [S,16]
    record_keys: torch.Tensor         # fp16 [S,16,128]
    record_corrections: torch.Tensor  # fp16 [S,16,128]
    positions: torch.Tensor           # int32 [S,8] (word 0: window position)

    @classmethod
    def allocate(cls, states: int, device) -> "WindowSlot":
        """Zeroed buffers: an empty window over an all-zero boundary."""
        z = lambda shape, dtype: torch.zeros(shape, dtype=dtype, device=device)  # noqa: E731
        return cls(z((states, DIM, DIM), torch.int8), z((states, DIM), torch.float32),
                   z((states, DIM), torch.float32), z((states, DIM, RANK), torch.float16),
                   z((states, DIM, RANK), torch.float16), z((states, WINDOW), torch.float32),
                   z((states, WINDOW, DIM), torch.float16),
                   z((states, WINDOW, DIM), torch.float16),
                   z((states, POSITION_STRIDE), torch.int32))

    @property
    def states(self) -> int:
        return self.residual.shape[0]

    @property
    def device(self):
        return self.residual.device

    def validate(self) -> None:
        s, dev = self.states, self.device
        _check(self.residual, "residual", (s, DIM, DIM), (torch.int8,), dev)
        _check(self.smoothing, "smoothing", (s, DIM), (torch.float32,), dev)
        _check(self.scales, "scales", (s, DIM), (torch.float32,), dev)
        _check(self.compensator_keys, "compensator_keys", (s, DIM, RANK), _HALF, dev)
        _check(self.compensator_values, "compensator_values", (s, DIM, RANK), _HALF, dev)
        _check(self.record_decay, "record_decay", (s, WINDOW), (torch.float32,), dev)
        _check(self.record_keys, "record_keys", (s, WINDOW, DIM), _HALF, dev)
        _check(self.record_corrections, "record_corrections", (s, WINDOW, DIM), _HALF, dev)
        _check(self.positions, "positions", (s, POSITION_STRIDE), _POS, dev)

    def pointers(self) -> tuple:
        return (self.residual.data_ptr(), self.smoothing.data_ptr(), self.scales.data_ptr(),
                self.compensator_keys.data_ptr(), self.compensator_values.data_ptr(),
                self.record_decay.data_ptr(), self.record_keys.data_ptr(),
                self.record_corrections.data_ptr(), self.positions.data_ptr())


def _bf16_inputs(slot: WindowSlot, log_decay, beta, keys, queries, values):
    s, dev = slot.states, slot.device
    if s % 2 != 0:
        raise RuntimeError("bf16 windowed steps need an even number of states (GQA pairs)")
    _check(log_decay, "log_decay", (s,), (torch.float32,), dev)
    _check(beta, "beta", (s,), _BF16, dev)
    _check(keys, "keys", (s // 2, DIM), _BF16, dev)
    _check(queries, "queries", (s // 2, DIM), _BF16, dev)
    _check(values, "values", (s, DIM), _BF16, dev)


def step_bf16(slot: WindowSlot, log_decay, beta, keys, queries, values, out=None,
              quant_only: bool = False, validate: bool = True) -> torch.Tensor:
    """One Qwen3.5 decode token for every state of `slot` (bf16 model tensors:
    keys / queries [S/2,128], values [S,128], beta [S]; fp32 log decay [S]);
    returns the bf16 outputs [S,128].  `quant_only` drops the compensator term
    (windowed_gdn_step_bf16_quant_only_launch_v1)."""
    s = slot.states
    if out is None:
        out = torch.empty((s, DIM), dtype=torch.bfloat16, device=slot.device)
    if validate:
        slot.validate()
        _bf16_inputs(slot, log_decay, beta, keys, queries, values)
        _check(out, "out", (s, DIM), _BF16, slot.device)
    lib = native()
    fn = (lib.windowed_gdn_step_bf16_quant_only_launch_v1 if quant_only
          else lib.windowed_gdn_step_bf16_launch_v1)
    status = fn(_stream(), *slot.pointers(), log_decay.data_ptr(), beta.data_ptr(),
                keys.data_ptr(), queries.data_ptr(), values.data_ptr(), out.data_ptr(), s)
    if status != 0:
        raise RuntimeError(f"GDN State Codec decode-step launch failed: {status}")
    return out


def step_f16(slot: WindowSlot, decay, write_keys, reads, queries, values, out=None,
             validate: bool = True) -> torch.Tensor:
    """The fp16 step on a [key][value] boundary (windowed_gdn_step_launch_v1):
    fp16 vectors [S,128], linear decay fp32 [S]; returns fp32 outputs [S,128]."""
    s, dev = slot.states, slot.device
    if out is None:
        out = torch.empty((s, DIM), dtype=torch.float32, device=dev)
    if validate:
        slot.validate()
        _check(decay, "decay", (s,), (torch.float32,), dev)
        for name, t in (("write_keys", write_keys), ("reads", reads), ("queries", queries),
                        ("values", values)):
            _check(t, name, (s, DIM), _HALF, dev)
        _check(out, "out", (s, DIM), (torch.float32,), dev)
    status = native().windowed_gdn_step_launch_v1(
        _stream(), *slot.pointers(), decay.data_ptr(), write_keys.data_ptr(), reads.data_ptr(),
        queries.data_ptr(), values.data_ptr(), out.data_ptr(), s)
    if status != 0:
        raise RuntimeError(f"GDN State Codec decode-step launch failed: {status}")
    return out


def dense_step_f32(state, decay, keys, reads, queries, values, out=None) -> torch.Tensor:
    """The reference's dense fp32 GDN step on [S,128,128] fp32 (in place)."""
    s, dev = state.shape[0], state.device
    _check(state, "state", (s, DIM, DIM), (torch.float32,), dev)
    _check(decay, "decay", (s,), (torch.float32,), dev)
    for name, t in (("keys", keys), ("reads", reads), ("queries", queries), ("values", values)):
        _check(t, name, (s, DIM), _HALF, dev)
    if out is None:
        out = torch.empty((s, DIM), dtype=torch.float32, device=dev)
    status = native().fp32_gdn_step_launch_v1(
        _stream(), state.data_ptr(), decay.data_ptr(), keys.data_ptr(), reads.data_ptr(),
        queries.data_ptr(), values.data_ptr(), out.data_ptr(), s)
    if status != 0:
        raise RuntimeError(f"GDN State Codec fp32 step launch failed: {status}")
    return out


class DecodeRuntime:
    """The decode runtime handle (decode_runtime_{create,step,destroy}_v1):
    the fused prepare / int8 projection / finish chain, bit-identical to the
    reference's three-stage cube decode."""

    def __init__(self, states: int) -> None:
        self._lib = native()
        self.states = states
        self.handle = self._lib.decode_runtime_create_v1(states)
        if not self.handle:
            raise RuntimeError("GDN State Codec Cube decode backend is unavailable")

    def step(self, slot: WindowSlot, log_decay, beta, keys, queries, values, out=None,
             validate: bool = True) -> torch.Tensor:
        s = slot.states
        if out is None:
            out = torch.empty((s, DIM), dtype=torch.bfloat16, device=slot.device)
        if validate:
            slot.validate()
            _bf16_inputs(slot, log_decay, beta, keys, queries, values)
        status = self._lib.decode_runtime_step_v1(
            self.handle, _stream(), *slot.pointers(), log_decay.data_ptr(), beta.data_ptr(),
            keys.data_ptr(), queries.data_ptr(), values.data_ptr(), out.data_ptr(), s)
        if status != 0:
            raise RuntimeError(f"GDN State Codec decode-step launch failed: {status}")
        return out

    def close(self) -> None:
        if self.handle:
            self._lib.decode_runtime_destroy_v1(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        self.close()
