"""CPU oracle for the GDN state codec hot path -- TEST INFRASTRUCTURE ONLY.

Thin numpy/ctypes wrappers over ``oracle/build/libgdn_oracle.so`` (the C
restatement in ``gdn_oracle.c``) and, when it has been built from the reference
sources, ``oracle/_ref/libgdn_ref.so`` (the reference's own portable C++ path
behind ``ref_harness.cpp``).  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg import this package, and only as the checker.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
ORACLE_LIB = ORACLE_DIR / "build" / "libgdn_oracle.so"
REF_LIB = ORACLE_DIR / "_ref" / "libgdn_ref.so"
REFERENCE_ROOT = Path("/root/reference")

LAYOUT_KEY_VALUE = 0
LAYOUT_VALUE_KEY = 1
DTYPE_F32 = 0
DTYPE_BF16 = 1
DIM = 128
TILE = DIM * DIM
SMOOTHING_FLOOR = np.float32(1.0e-8)

_P = ctypes.c_void_p
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_I = ctypes.c_int
_F = ctypes.c_float


def build(reference: bool | None = None) -> None:
    """Compile the oracle (and oracle/_ref when the reference tree is present)."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    if reference is None:
        reference = REFERENCE_ROOT.is_dir()
    if reference:
        subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "ref"], check=True)


def _ptr(array: np.ndarray | None) -> int | None:
    if array is None:
        return None
    assert array.flags["C_CONTIGUOUS"]
    return array.ctypes.data


_lib: ctypes.CDLL | None = None
_ref: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not ORACLE_LIB.is_file():
            build(reference=False)
        l = ctypes.CDLL(str(ORACLE_LIB))
        l.gdn_oracle_quantize_kv.argtypes = [_P, _U32, _U32, _U32, _F, _P, _P, _P, _P, _P, _P]
        l.gdn_oracle_quantize_kv.restype = None
        l.gdn_oracle_dequantize_kv.argtypes = [_P, _P, _P, _P, _P, _U32, _U32, _U32, _P]
        l.gdn_oracle_dequantize_kv.restype = None
        l.gdn_oracle_read_boundary.argtypes = [_P, _P, _P, _P, _P, _U32, _U32, _U32, _P, _P]
        l.gdn_oracle_read_boundary.restype = None
        l.gdn_oracle_provider_to_codec.argtypes = [_P, _U32, _U32, _P]
        l.gdn_oracle_codec_to_provider.argtypes = [_P, _U32, _U32, _P]
        l.gdn_oracle_encode_heads.argtypes = [_P, _U64, _U32, _P, _P, _P, _I]
        l.gdn_oracle_encode_heads.restype = None
        l.gdn_oracle_decode_heads.argtypes = [_P, _P, _P, _U64, _U32, _P, _I]
        l.gdn_oracle_decode_heads.restype = None
        l.gdn_oracle_project_decode.argtypes = [_P, _P, _P, _P, _U32, _U32, _U32, _F, _U32, _P, _P, _P]
        l.gdn_oracle_project_decode.restype = None
        l.gdn_oracle_project_chunked.argtypes = [_P, _P, _P, _P, _U32, _U32, _U32, _U32, _F, _U32, _P, _P, _P, _I]
        l.gdn_oracle_project_chunked.restype = None
        l.gdn_oracle_pool_encode.argtypes = [_P, _U32, _P, _U32, _U32, _U32, _U32, _U32, _P, _P, _P, _I]
        l.gdn_oracle_pool_encode.restype = None
        l.gdn_oracle_pool_decode.argtypes = [_P, _P, _P, _P, _U32, _U32, _U32, _U32, _U32, _P, _U32, _I]
        l.gdn_oracle_pool_decode.restype = None
        l.gdn_oracle_f32_to_bf16.argtypes = [_F]
        l.gdn_oracle_f32_to_bf16.restype = ctypes.c_uint16
        l.gdn_oracle_f32_to_bf16_array.argtypes = [_P, _U64, _P]
        l.gdn_oracle_f32_to_bf16_array.restype = None
        _lib = l
    return _lib


def ref_available() -> bool:
    return REF_LIB.is_file()


def ref() -> ctypes.CDLL:
    """The reference's own CPU code (oracle/_ref), or raise if not built."""
    global _ref
    if _ref is None:
        if not REF_LIB.is_file():
            raise FileNotFoundError(f"{REF_LIB} is not built (needs /root/reference)")
        r = ctypes.CDLL(str(REF_LIB))
        r.gdnref_quantize_boundary.argtypes = [_P, _U32, _U32, _U32, _P, _P, _P, _P, _P]
        r.gdnref_quantize_boundary.restype = _I
        r.gdnref_dequantize_boundary.argtypes = [_P, _P, _P, _P, _P, _U32, _U32, _U32, _P]
        r.gdnref_dequantize_boundary.restype = _I
        r.gdnref_read_boundary.argtypes = [_P, _P, _P, _P, _P, _U32, _U32, _U32, _P, _P]
        r.gdnref_read_boundary.restype = _I
        r.gdnref_provider_to_codec.argtypes = [_P, _U32, _U32, _P]
        r.gdnref_provider_to_codec.restype = _I
        r.gdnref_codec_to_provider.argtypes = [_P, _U32, _U32, _P]
        r.gdnref_codec_to_provider.restype = _I
        r.gdnref_quantize_heads.argtypes = [_P, _U64, _U32, _U32, _P, _P, _P]
        r.gdnref_quantize_heads.restype = _I
        r.gdnref_dequantize_heads.argtypes = [_P, _P, _P, _U64, _U32, _U32, _P]
        r.gdnref_dequantize_heads.restype = _I
        r.gdnref_read_boundary_heads.argtypes = [_P, _P, _P, _U64, _U32, _U32, _U32, _P, _P]
        r.gdnref_read_boundary_heads.restype = _I
        _ref = r
    return _ref


# ----------------------------------------------------------------- single head


def quantize_kv(dense: np.ndarray, rank: int = 0):
    """QuantizeBoundary of one [K][V] head -> (codes, smoothing, scales, ck, cv)."""
    dense = np.ascontiguousarray(dense, dtype=np.float32)
    keys, values = dense.shape
    codes = np.empty((keys, values), np.int8)
    smoothing = np.empty(keys, np.float32)
    scales = np.empty(values, np.float32)
    ck = np.zeros((keys, max(rank, 1)), np.float32)
    cv = np.zeros((values, max(rank, 1)), np.float32)
    work = np.empty(keys * values, np.float32)
    lib().gdn_oracle_quantize_kv(_ptr(dense), keys, values, rank, SMOOTHING_FLOOR,
                                 _ptr(codes), _ptr(smoothing), _ptr(scales),
                                 _ptr(ck), _ptr(cv), _ptr(work))
    return codes, smoothing, scales, ck[:, :rank], cv[:, :rank]


def dequantize_kv(codes, smoothing, scales, ck=None, cv=None):
    keys, values = codes.shape
    rank = 0 if ck is None else ck.shape[1]
    dense = np.empty((keys, values), np.float32)
    ck = None if ck is None else np.ascontiguousarray(ck, np.float32)
    cv = None if cv is None else np.ascontiguousarray(cv, np.float32)
    lib().gdn_oracle_dequantize_kv(_ptr(np.ascontiguousarray(codes)), _ptr(smoothing),
                                   _ptr(scales), _ptr(ck), _ptr(cv), keys, values,
                                   rank, _ptr(dense))
    return dense


def read_boundary(codes, smoothing, scales, read, ck=None, cv=None):
    keys, values = codes.shape
    rank = 0 if ck is None else ck.shape[1]
    out = np.empty(values, np.float32)
    ck = None if ck is None else np.ascontiguousarray(ck, np.float32)
    cv = None if cv is None else np.ascontiguousarray(cv, np.float32)
    read = np.ascontiguousarray(read, np.float32)
    lib().gdn_oracle_read_boundary(_ptr(np.ascontiguousarray(codes)), _ptr(smoothing),
                                   _ptr(scales), _ptr(ck), _ptr(cv), keys, values,
                                   rank, _ptr(read), _ptr(out))
    return out


def provider_to_codec(provider: np.ndarray, keys: int, values: int) -> np.ndarray:
    provider = np.ascontiguousarray(provider, np.float32)
    out = np.empty(keys * values, np.float32)
    lib().gdn_oracle_provider_to_codec(_ptr(provider), keys, values, _ptr(out))
    return out


def codec_to_provider(codec: np.ndarray, keys: int, values: int) -> np.ndarray:
    codec = np.ascontiguousarray(codec, np.float32)
    out = np.empty(keys * values, np.float32)
    lib().gdn_oracle_codec_to_provider(_ptr(codec), keys, values, _ptr(out))
    return out


# ------------------------------------------------------------- batched heads


def encode_heads(state: np.ndarray, layout: int = LAYOUT_KEY_VALUE, threads: int = 1):
    """Quant-only encode of [..., 128, 128] fp32 tiles."""
    state = np.ascontiguousarray(state, np.float32)
    heads = state.size // TILE
    lead = state.shape[:-2]
    codes = np.empty(state.shape, np.int8)
    smoothing = np.empty(lead + (DIM,), np.float32)
    scales = np.empty(lead + (DIM,), np.float32)
    lib().gdn_oracle_encode_heads(_ptr(state), heads, layout, _ptr(codes),
                                  _ptr(smoothing), _ptr(scales), threads)
    return codes, smoothing, scales


def decode_heads(codes, smoothing, scales, layout: int = LAYOUT_KEY_VALUE, threads: int = 1):
    codes = np.ascontiguousarray(codes, np.int8)
    heads = codes.size // TILE
    state = np.empty(codes.shape, np.float32)
    lib().gdn_oracle_decode_heads(_ptr(codes), _ptr(np.ascontiguousarray(smoothing, np.float32)),
                                  _ptr(np.ascontiguousarray(scales, np.float32)), heads,
                                  layout, _ptr(state), threads)
    return state


def project_decode(codes, smoothing, scales, queries_bf16, query_scale=1.0,
                   layout: int = LAYOUT_VALUE_KEY):
    """codes [B,H,128,128]; queries_bf16 uint16 [B,Hq,128] -> (out f32, out f64, bound)."""
    batch, value_heads = codes.shape[:2]
    query_heads = queries_bf16.shape[1]
    out = np.empty((batch, value_heads, DIM), np.float32)
    out64 = np.empty((batch, value_heads, DIM), np.float64)
    bound = np.empty((batch, value_heads, DIM), np.float64)
    lib().gdn_oracle_project_decode(
        _ptr(np.ascontiguousarray(codes, np.int8)),
        _ptr(np.ascontiguousarray(smoothing, np.float32)),
        _ptr(np.ascontiguousarray(scales, np.float32)),
        _ptr(np.ascontiguousarray(queries_bf16, np.uint16)), batch, value_heads,
        query_heads, query_scale, layout, _ptr(out), _ptr(out64), _ptr(bound))
    return out, out64, bound


def project_chunked(codes, smoothing, scales, queries_bf16, query_scale=1.0,
                    layout: int = LAYOUT_VALUE_KEY, threads: int = 1):
    """codes [N,H,128,128]; queries_bf16 [N,T,Hq,128] -> out [N,T,H,128] (+f64, bound)."""
    seqs, value_heads = codes.shape[:2]
    tokens, query_heads = queries_bf16.shape[1:3]
    shape = (seqs, tokens, value_heads, DIM)
    out = np.empty(shape, np.float32)
    out64 = np.empty(shape, np.float64)
    bound = np.empty(shape, np.float64)
    lib().gdn_oracle_project_chunked(
        _ptr(np.ascontiguousarray(codes, np.int8)),
        _ptr(np.ascontiguousarray(smoothing, np.float32)),
        _ptr(np.ascontiguousarray(scales, np.float32)),
        _ptr(np.ascontiguousarray(queries_bf16, np.uint16)), seqs, tokens,
        value_heads, query_heads, query_scale, layout, _ptr(out), _ptr(out64),
        _ptr(bound), threads)
    return out, out64, bound


def pool_encode(pool, slot_ids, layout: int = LAYOUT_KEY_VALUE, codes=None,
                smoothing=None, scales=None, threads: int = 1):
    """pool [L,S,H,128,128] f32 or bf16(uint16) -> compact [L,B,H,...] encodes."""
    layers, slots, heads = pool.shape[:3]
    batch = len(slot_ids)
    dtype = DTYPE_F32 if pool.dtype == np.float32 else DTYPE_BF16
    if codes is None:
        codes = np.zeros((layers, batch, heads, DIM, DIM), np.int8)
        smoothing = np.zeros((layers, batch, heads, DIM), np.float32)
        scales = np.zeros((layers, batch, heads, DIM), np.float32)
    slot_ids = np.ascontiguousarray(slot_ids, np.int32)
    lib().gdn_oracle_pool_encode(_ptr(np.ascontiguousarray(pool)), dtype, _ptr(slot_ids),
                                 batch, layers, slots, heads, layout, _ptr(codes),
                                 _ptr(smoothing), _ptr(scales), threads)
    return codes, smoothing, scales


def pool_decode(codes, smoothing, scales, slot_ids, pool, layout: int = LAYOUT_KEY_VALUE,
                threads: int = 1):
    """Scatter-decode compact encodes into pool (modified in place)."""
    layers, slots, heads = pool.shape[:3]
    batch = len(slot_ids)
    dtype = DTYPE_F32 if pool.dtype == np.float32 else DTYPE_BF16
    assert pool.flags["C_CONTIGUOUS"]
    slot_ids = np.ascontiguousarray(slot_ids, np.int32)
    lib().gdn_oracle_pool_decode(_ptr(np.ascontiguousarray(codes, np.int8)),
                                 _ptr(np.ascontiguousarray(smoothing, np.float32)),
                                 _ptr(np.ascontiguousarray(scales, np.float32)),
                                 _ptr(slot_ids), batch, layers, slots, heads, layout,
                                 _ptr(pool), dtype, threads)
    return pool


# ----------------------------------------------------------------- bf16 / data


def f32_to_bf16(values: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even narrowing, the reference's FloatToBFloat16."""
    bits = np.ascontiguousarray(values, np.float32).view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    return ((bits + 0x7FFF + lsb) >> 16).astype(np.uint16)


def c_f32_to_bf16(values: np.ndarray) -> np.ndarray:
    """The C restatement's narrowing (gdn_oracle_f32_to_bf16), elementwise."""
    values = np.ascontiguousarray(values, np.float32)
    out = np.empty(values.shape, np.uint16)
    lib().gdn_oracle_f32_to_bf16_array(_ptr(values), values.size, _ptr(out))
    return out


def bf16_to_f32(values: np.ndarray) -> np.ndarray:
    return (np.asarray(values, np.uint16).astype(np.uint32) << 16).view(np.float32)


# -------------------------------------------------------- reference (oracle/_ref)


def ref_quantize_kv(dense: np.ndarray, rank: int = 0):
    dense = np.ascontiguousarray(dense, dtype=np.float32)
    keys, values = dense.shape
    codes = np.empty((keys, values), np.int8)
    smoothing = np.empty(keys, np.float32)
    scales = np.empty(values, np.float32)
    ck = np.zeros((keys, max(rank, 1)), np.float32)
    cv = np.zeros((values, max(rank, 1)), np.float32)
    status = ref().gdnref_quantize_boundary(_ptr(dense), keys, values, rank, _ptr(codes),
                                            _ptr(smoothing), _ptr(scales), _ptr(ck), _ptr(cv))
    if status != 0:
        raise ValueError("reference QuantizeBoundary rejected the input")
    return codes, smoothing, scales, ck[:, :rank], cv[:, :rank]


def ref_dequantize_kv(codes, smoothing, scales, ck=None, cv=None):
    keys, values = codes.shape
    rank = 0 if ck is None else ck.shape[1]
    dense = np.empty((keys, values), np.float32)
    ck = None if ck is None else np.ascontiguousarray(ck, np.float32)
    cv = None if cv is None else np.ascontiguousarray(cv, np.float32)
    status = ref().gdnref_dequantize_boundary(_ptr(np.ascontiguousarray(codes)),
                                              _ptr(smoothing), _ptr(scales), _ptr(ck),
                                              _ptr(cv), keys, values, rank, _ptr(dense))
    assert status == 0
    return dense


def ref_read_boundary(codes, smoothing, scales, read, ck=None, cv=None):
    keys, values = codes.shape
    rank = 0 if ck is None else ck.shape[1]
    out = np.empty(values, np.float32)
    ck = None if ck is None else np.ascontiguousarray(ck, np.float32)
    cv = None if cv is None else np.ascontiguousarray(cv, np.float32)
    read = np.ascontiguousarray(read, np.float32)
    status = ref().gdnref_read_boundary(_ptr(np.ascontiguousarray(codes)), _ptr(smoothing),
                                        _ptr(scales), _ptr(ck), _ptr(cv), keys, values,
                                        rank, _ptr(read), _ptr(out))
    assert status == 0
    return out


def ref_provider_to_codec(provider: np.ndarray, keys: int, values: int) -> np.ndarray:
    provider = np.ascontiguousarray(provider, np.float32)
    out = np.empty(keys * values, np.float32)
    assert ref().gdnref_provider_to_codec(_ptr(provider), keys, values, _ptr(out)) == 0
    return out


def ref_quantize_heads(state: np.ndarray):
    """The reference's quant-only encode over [...,128,128] [K][V] tiles."""
    state = np.ascontiguousarray(state, np.float32)
    heads = state.size // TILE
    lead = state.shape[:-2]
    codes = np.empty(state.shape, np.int8)
    smoothing = np.empty(lead + (DIM,), np.float32)
    scales = np.empty(lead + (DIM,), np.float32)
    status = ref().gdnref_quantize_heads(_ptr(state), heads, DIM, DIM, _ptr(codes),
                                         _ptr(smoothing), _ptr(scales))
    assert status == 0
    return codes, smoothing, scales


def ref_dequantize_heads(codes, smoothing, scales):
    codes = np.ascontiguousarray(codes, np.int8)
    heads = codes.size // TILE
    state = np.empty(codes.shape, np.float32)
    status = ref().gdnref_dequantize_heads(_ptr(codes), _ptr(np.ascontiguousarray(smoothing)),
                                           _ptr(np.ascontiguousarray(scales)), heads, DIM,
                                           DIM, _ptr(state))
    assert status == 0
    return state


def ref_read_boundary_heads(codes, smoothing, scales, reads):
    """The reference's ReadWindowState boundary readout: codes [N,128,128]
    [K][V], smoothing/scales [N,128], reads fp32 [N,T,128] -> [N,T,128]."""
    codes = np.ascontiguousarray(codes, np.int8)
    heads = codes.size // TILE
    reads = np.ascontiguousarray(reads, np.float32).reshape(heads, -1, DIM)
    tokens = reads.shape[1]
    out = np.empty((heads, tokens, DIM), np.float32)
    status = ref().gdnref_read_boundary_heads(
        _ptr(codes), _ptr(np.ascontiguousarray(smoothing, np.float32)),
        _ptr(np.ascontiguousarray(scales, np.float32)), heads, tokens, DIM, DIM,
        _ptr(reads), _ptr(out))
    assert status == 0
    return out
