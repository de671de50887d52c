"""ctypes bindings of the gfx950 C-ABI library (``include/*.h``).

The library is loaded from ``$GDN_STATE_CODEC_LIBRARY_DIR`` when set (the
reference's variable, ``manifests/vllm-hust-extension-v0.3.json:58-63``) and
otherwise from the in-tree ``lib/`` directory built by ``build.py``.  A missing
library raises: there is no CPU or torch fallback on the product path.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent.parent
DEFAULT_LIBRARY_DIR = PACKAGE_DIR / "lib"
LIBRARY_NAME = "libstatecentric_gdn_state_codec.so"

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_F = ctypes.c_float
_I32 = ctypes.c_int32
_C = ctypes.c_char_p

# name -> argtypes (all return int32 status)
SIGNATURES: dict[str, list] = {
    # codec, reference entry points
    "statecentric_gdn_state_codec_smoothing_launch_v1": [_P, _P, _P],
    "statecentric_gdn_state_codec_provider_smoothing_launch_v2": [_P, _P, _P, _U32],
    "statecentric_gdn_state_codec_quantize_launch_v1": [_P, _P, _P, _P, _P],
    "statecentric_gdn_state_codec_provider_quantize_launch_v2": [_P, _P, _P, _P, _P, _U32],
    "statecentric_gdn_state_codec_provider_initialize_launch_v3": [_P, _P, _P, _P, _P, _U32],
    "statecentric_gdn_state_codec_dequantize_launch_v1": [_P, _P, _P, _P, _P, _P, _P],
    # codec, batched
    "statecentric_gdn_state_codec_encode_launch_v4": [_P, _P, _P, _P, _P, _U64, _U32],
    "statecentric_gdn_state_codec_decode_launch_v4": [_P, _P, _P, _P, _P, _P, _P, _U64, _U32],
    "statecentric_gdn_state_codec_quantize_boundary_launch_v1": [_P] * 9 + [_U64, _U32],
    "statecentric_gdn_state_codec_exact_svd_boundary_launch_v1": [_P] * 9 + [_U64],
    "statecentric_gdn_state_codec_exact_svd_boundary_sweeps_launch_v1": [_P] * 9 + [_U64, _U32],
    "statecentric_gdn_state_codec_pool_encode_launch_v4": [
        _P, _P, _U32, _P, _U32, _U32, _U32, _U32, _U32, _P, _P, _P],
    "statecentric_gdn_state_codec_pool_decode_launch_v4": [
        _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _P, _U32],
    # encoded projection
    "statecentric_gdn_state_codec_encoded_projection_decode_launch_v4": [
        _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _F, _U32],
    "statecentric_gdn_state_codec_encoded_projection_chunked_launch_v4": [
        _P, _P, _P, _P, _P, _P, _U32, _U32, _U32, _U32, _F, _U32],
    # windowed decode step (include/gdn_state_codec_window.h)
    "statecentric_gdn_state_codec_windowed_gdn_step_launch_v1": [_P] * 16 + [_U32],
    "statecentric_gdn_state_codec_windowed_gdn_step_bf16_launch_v1": [_P] * 16 + [_U32],
    "statecentric_gdn_state_codec_windowed_gdn_step_bf16_quant_only_launch_v1": [_P] * 16 + [_U32],
    "statecentric_gdn_state_codec_fp32_gdn_step_launch_v1": [_P] * 8 + [_U32],
    "statecentric_gdn_state_codec_prepare_int8_vector_launch_v1": [_P] * 5 + [_U32],
    "statecentric_gdn_state_codec_prepare_decode_pair_launch_v1": [_P] * 7 + [_U32],
    "statecentric_gdn_state_codec_prepare_decode_pair_bf16_launch_v1": [_P] * 7 + [_U32],
    "statecentric_gdn_state_codec_finish_decode_pair_launch_v1": [_P] * 16 + [_U32],
    "statecentric_gdn_state_codec_finish_decode_pair_bf16_launch_v1": [_P] * 16 + [_U32],
    "statecentric_gdn_state_codec_int8_cube_matmul_launch_v1": [
        _P, _P, _P, _P, _U32, _U32, _P, _P, _U32],
    "statecentric_gdn_state_codec_int8_matmul_launch_v4": [_P, _P, _P, _P, _U32, _U32],
    "statecentric_gdn_state_codec_decode_runtime_step_v1": [_P] * 17 + [_U32],
    # device rank-4 chain over an encoded boundary
    "statecentric_gdn_state_codec_finish_encoded_projection_launch_v1":
        [_P] * 14 + [_U32, _U32, _U32],
    "statecentric_gdn_state_codec_commit_encoded_rank_launch_v1": [_P] * 14 + [_U32, _U32],
    "statecentric_gdn_state_codec_encoded_requantize_launch_v1": [_P] * 17 + [_U32],
    "statecentric_gdn_state_codec_encoded_rank_chain_launch_v4": [_P] * 13 + [_U32, _U32],
    # window-boundary refit
    "statecentric_gdn_state_codec_window_boundary_launch_v1": [_P] * 16 + [_U32, _U32],
    "statecentric_gdn_state_codec_window_boundary_noalloc_launch_v1": [_P] * 15 + [_U32, _U32],
    "statecentric_gdn_state_codec_boundary_scale_records_launch_v1": [_P] * 4 + [_U32],
    "statecentric_gdn_state_codec_window_boundary_cube_finish_launch_v1": [_P] * 16 + [_U32],
    "statecentric_gdn_state_codec_bf16_cube_matmul_launch_v1": [_P] * 4 + [_U32, _P, _P, _U32],
    "statecentric_gdn_state_codec_boundary_runtime_step_v1": [_P] * 7 + [_U32],
    # include/gdn_state_codec_capsule.h
    "statecentric_gdn_state_codec_capsule_serialize_launch_v1":
        [_P] * 10 + [_U32, _C, _U64, _U64, _P, _P, _U64, _P, _U32],
    "statecentric_gdn_state_codec_capsule_restore_launch_v1":
        [_P] * 4 + [_U64, _C, _U64, _U64, _P, _U32] + [_P] * 10 + [_U32],
}

# Entry points that do not return a status: name -> (argtypes, restype).
OTHER_SIGNATURES: dict[str, tuple] = {
    "statecentric_gdn_state_codec_decode_runtime_create_v1": ([_U32], _P),
    "statecentric_gdn_state_codec_decode_runtime_destroy_v1": ([_P], None),
    "statecentric_gdn_state_codec_boundary_runtime_create_v1": ([_U32], _P),
    "statecentric_gdn_state_codec_boundary_runtime_destroy_v1": ([_P], None),
    "statecentric_gdn_state_codec_capsule_bytes_v1": ([_U32], _U64),
}


def library_dir() -> Path:
    override = os.environ.get("GDN_STATE_CODEC_LIBRARY_DIR")
    return Path(override) if override else DEFAULT_LIBRARY_DIR


def library_path() -> Path:
    return library_dir() / LIBRARY_NAME


class NativeLibrary:
    """The loaded library with typed entry points as attributes."""

    def __init__(self, path: Path | None = None) -> None:
        path = path or library_path()
        if not path.is_file():
            raise RuntimeError(
                f"GDN State Codec native library is missing: {path} "
                "(run gdn-state-codec_amd/build.py)"
            )
        self.path = path
        self._lib = ctypes.CDLL(str(path))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(self._lib, name)
            fn.argtypes = argtypes
            fn.restype = _I32
            setattr(self, name.removeprefix("statecentric_gdn_state_codec_"), fn)
        for name, (argtypes, restype) in OTHER_SIGNATURES.items():
            fn = getattr(self._lib, name)
            fn.argtypes = argtypes
            fn.restype = restype
            setattr(self, name.removeprefix("statecentric_gdn_state_codec_"), fn)

    def symbol(self, name: str):
        return getattr(self._lib, name)


_library: NativeLibrary | None = None


def native() -> NativeLibrary:
    global _library
    if _library is None:
        _library = NativeLibrary()
    return _library
