"""Torch-facing wrappers of the gfx950 codec and encoded-projection entry points.

Each function validates shapes, dtypes, devices and contiguity on the host
(raising ``RuntimeError`` like the reference runtime,
``src/gdn_state_codec/runtime.py:460-547``), launches the HIP kernel on the
current torch stream through the C-ABI and raises ``RuntimeError`` on a
non-zero status.  Tensors are only allocated here when the caller passes no
output; the kernels themselves never allocate.
"""

from __future__ import annotations

import torch

from ._native import native

DIM = 128
LAYOUT_KEY_VALUE = 0  # codec/capsule [key][value]
LAYOUT_VALUE_KEY = 1  # Qwen provider [value][key]
DTYPE_F32 = 0
DTYPE_BF16 = 1


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _require(condition: bool, message: str) -> None:
    if not condition:
        raise RuntimeError(message)


def _check(status: int, what: str) -> None:
    if status != 0:
        raise RuntimeError(f"GDN State Codec {what} launch failed: {status}")


def _tiles(t: torch.Tensor, dtype: torch.dtype, name: str) -> int:
    _require(t.is_cuda, f"GDN State Codec {name} must be a device tensor")
    _require(t.dtype == dtype, f"GDN State Codec {name} must be {dtype}")
    _require(t.is_contiguous(), f"GDN State Codec {name} must be contiguous")
    _require(t.dim() >= 2 and tuple(t.shape[-2:]) == (DIM, DIM),
             f"GDN State Codec {name} must be [...,128,128] tiles")
    return t.numel() // (DIM * DIM)


def _vectors(t: torch.Tensor, tiles: int, name: str) -> None:
    _require(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous(),
             f"GDN State Codec {name} must be a contiguous fp32 device tensor")
    _require(t.numel() == tiles * DIM, f"GDN State Codec {name} must hold [tiles,128]")


def encode(state: torch.Tensor, layout: int = LAYOUT_KEY_VALUE, codes=None,
           smoothing=None, scales=None):
    """Quant-only int8 encode of fp32 [...,128,128] tiles -> (codes, smoothing, scales)."""
    tiles = _tiles(state, torch.float32, "state")
    lead = tuple(state.shape[:-2])
    if codes is None:
        codes = torch.empty(state.shape, dtype=torch.int8, device=state.device)
        smoothing = torch.empty(lead + (DIM,), dtype=torch.float32, device=state.device)
        scales = torch.empty(lead + (DIM,), dtype=torch.float32, device=state.device)
    _require(_tiles(codes, torch.int8, "codes") == tiles, "codes geometry differs")
    _vectors(smoothing, tiles, "smoothing")
    _vectors(scales, tiles, "scales")
    _check(native().encode_launch_v4(_stream(), state.data_ptr(), codes.data_ptr(),
                                     smoothing.data_ptr(), scales.data_ptr(), tiles,
                                     layout), "encode")
    return codes, smoothing, scales


FIT_STATUS = {1: "holds a non-finite value", 2: "has a non-finite compensator fit"}
SVD_STATUS = {1: "holds a non-finite value",
              2: "did not converge within the Jacobi sweep limit"}


def quantize_boundary(dense: torch.Tensor, rank: int = 4, check: bool = True):
    """The capsule factory's boundary encode (``FromDenseBoundary`` ->
    ``QuantizeBoundary``, ``native/src/gdn_state_codec_state_capsule.cpp:129-226,
    318-335``) of fp32 [...,128,128] [key][value] heads: the rank-``rank``
    compensator fit, then the quant stage on the fitted residual.

    Returns ``(codes, smoothing, scales, compensator_keys, compensator_values,
    residual, status)``; the compensators are fp32 [...,128,rank].  With
    ``check`` (the default) the call synchronizes and raises ``ValueError`` for
    the first head the reference would reject (non-finite input or fit);
    otherwise ``status`` (int32 per head: 0 ok, 1 non-finite input, 2
    non-finite fit) is left for the caller to read."""
    _require(0 <= rank <= 4, "GDN State Codec compensator rank must be 0..4")
    heads = _tiles(dense, torch.float32, "dense boundary")
    lead = tuple(dense.shape[:-2])
    device = dense.device
    codes = torch.empty(dense.shape, dtype=torch.int8, device=device)
    smoothing = torch.empty(lead + (DIM,), dtype=torch.float32, device=device)
    scales = torch.empty(lead + (DIM,), dtype=torch.float32, device=device)
    keys = torch.empty(lead + (DIM, rank), dtype=torch.float32, device=device)
    values = torch.empty(lead + (DIM, rank), dtype=torch.float32, device=device)
    residual = torch.empty(dense.shape, dtype=torch.float32, device=device)
    status = torch.empty(lead, dtype=torch.int32, device=device)
    _check(native().quantize_boundary_launch_v1(
        _stream(), dense.data_ptr(), residual.data_ptr(), codes.data_ptr(),
        smoothing.data_ptr(), scales.data_ptr(), keys.data_ptr() if rank else 0,
        values.data_ptr() if rank else 0, status.data_ptr(), heads, rank),
        "quantize boundary")
    if check:
        flat = status.reshape(-1).cpu()
        bad = torch.nonzero(flat).reshape(-1)
        if bad.numel():
            head = int(bad[0])
            raise ValueError(f"GDN State Codec boundary head {head} "
                             f"{FIT_STATUS.get(int(flat[head]), 'failed')}")
    return codes, smoothing, scales, keys, values, residual, status


def exact_svd_boundary(provider: torch.Tensor, check: bool = True, residual=None,
                       max_sweeps: int | None = None):
    """The reference runtime's ``exact_svd`` initializer
    (``GdnStateCodecRuntime._encode_dense_boundary``,
    ``src/gdn_state_codec/runtime.py:335-389``) for fp32 [...,128,128]
    provider heads ([value][key], the dense state transposed): the rank-4
    truncated SVD of each dense head by one-sided Jacobi on the GPU, then the
    quant-only encode of the fitted residual in the provider layout.

    Returns ``(codes, smoothing, scales, compensator_keys, compensator_values,
    residual, status)``: codes int8 [...,value,key], fp16 compensators
    [...,128,4] (keys = U*S, values = V), the fp32 residual [...,value,key]
    (``residual`` may name the buffer to write) and int32 ``status`` per head
    (0 ok, 1 non-finite input, 2 not converged within the sweep limit:
    ``max_sweeps``, 1..30, default 30).  With ``check`` the call synchronizes
    and raises ``ValueError`` for the first head with a nonzero status."""
    heads = _tiles(provider, torch.float32, "provider state")
    lead = tuple(provider.shape[:-2])
    device = provider.device
    codes = torch.empty(provider.shape, dtype=torch.int8, device=device)
    smoothing = torch.empty(lead + (DIM,), dtype=torch.float32, device=device)
    scales = torch.empty(lead + (DIM,), dtype=torch.float32, device=device)
    keys = torch.empty(lead + (DIM, 4), dtype=torch.float16, device=device)
    values = torch.empty(lead + (DIM, 4), dtype=torch.float16, device=device)
    if residual is None:
        residual = torch.empty(provider.shape, dtype=torch.float32, device=device)
    _require(residual.dtype == torch.float32 and residual.is_contiguous()
             and residual.numel() == provider.numel() and residual.device == device,
             "GDN State Codec SVD residual must be a contiguous fp32 buffer of the "
             "provider's size on its device")
    status = torch.empty(lead, dtype=torch.int32, device=device)
    pointers = (_stream(), provider.data_ptr(), residual.data_ptr(), codes.data_ptr(),
                smoothing.data_ptr(), scales.data_ptr(), keys.data_ptr(), values.data_ptr(),
                status.data_ptr(), heads)
    if max_sweeps is None:
        _check(native().exact_svd_boundary_launch_v1(*pointers), "exact SVD boundary")
    else:
        _check(native().exact_svd_boundary_sweeps_launch_v1(*pointers, max_sweeps),
               "exact SVD boundary")
    if check:
        flat = status.reshape(-1).cpu()
        bad = torch.nonzero(flat).reshape(-1)
        if bad.numel():
            raise ValueError(f"GDN State Codec boundary head {int(bad[0])} "
                             f"{SVD_STATUS.get(int(flat[int(bad[0])]), 'failed')}")
    return codes, smoothing, scales, keys, values, residual, status


def decode(codes: torch.Tensor, smoothing: torch.Tensor, scales: torch.Tensor,
           layout: int = LAYOUT_KEY_VALUE, compensator_keys=None,
           compensator_values=None, out=None) -> torch.Tensor:
    """Dequantize int8 tiles to fp32 (rank-4 fp32 compensators optional)."""
    tiles = _tiles(codes, torch.int8, "codes")
    _vectors(smoothing, tiles, "smoothing")
    _vectors(scales, tiles, "scales")
    ck = cv = 0
    if compensator_keys is not None or compensator_values is not None:
        _require(compensator_keys is not None and compensator_values is not None,
                 "GDN State Codec compensators come in pairs")
        for t, name in ((compensator_keys, "compensator keys"),
                        (compensator_values, "compensator values")):
            _require(t.is_cuda and t.dtype == torch.float32 and t.is_contiguous()
                     and t.numel() == tiles * DIM * 4,
                     f"GDN State Codec {name} must be contiguous fp32 [tiles,128,4]")
        ck, cv = compensator_keys.data_ptr(), compensator_values.data_ptr()
    if out is None:
        out = torch.empty(codes.shape, dtype=torch.float32, device=codes.device)
    _require(_tiles(out, torch.float32, "dense output") == tiles, "output geometry differs")
    _check(native().decode_launch_v4(_stream(), codes.data_ptr(), smoothing.data_ptr(),
                                     scales.data_ptr(), ck or None, cv or None,
                                     out.data_ptr(), tiles, layout), "decode")
    return out


def _pool_dtype(pool: torch.Tensor) -> int:
    if pool.dtype == torch.float32:
        return DTYPE_F32
    if pool.dtype == torch.bfloat16:
        return DTYPE_BF16
    raise RuntimeError("GDN State Codec pool must be fp32 or bf16")


def _pool_geometry(pool: torch.Tensor, slot_ids: torch.Tensor):
    _require(pool.is_cuda and pool.is_contiguous() and pool.dim() == 5
             and tuple(pool.shape[-2:]) == (DIM, DIM),
             "GDN State Codec pool must be a contiguous [layers,slots,heads,128,128] tensor")
    _require(slot_ids.is_cuda and slot_ids.dtype == torch.int32 and slot_ids.dim() == 1
             and slot_ids.is_contiguous(), "GDN State Codec slot ids must be device int32 [batch]")
    layers, slots, heads = pool.shape[:3]
    return layers, slots, heads, slot_ids.numel()


def pool_encode(pool: torch.Tensor, slot_ids: torch.Tensor, layout: int = LAYOUT_KEY_VALUE,
                codes=None, smoothing=None, scales=None):
    """Gather pool[l, slot_ids[b], h] and encode into compact [layers,batch,heads] outputs.

    Entries with slot id -1 (padding) are skipped and their outputs left as they were."""
    layers, slots, heads, batch = _pool_geometry(pool, slot_ids)
    if codes is None:
        dev = pool.device
        codes = torch.zeros((layers, batch, heads, DIM, DIM), dtype=torch.int8, device=dev)
        smoothing = torch.zeros((layers, batch, heads, DIM), dtype=torch.float32, device=dev)
        scales = torch.zeros((layers, batch, heads, DIM), dtype=torch.float32, device=dev)
    tiles = layers * batch * heads
    _require(_tiles(codes, torch.int8, "codes") == tiles, "codes geometry differs")
    _vectors(smoothing, tiles, "smoothing")
    _vectors(scales, tiles, "scales")
    _check(native().pool_encode_launch_v4(
        _stream(), pool.data_ptr(), _pool_dtype(pool), slot_ids.data_ptr(), batch, layers,
        slots, heads, layout, codes.data_ptr(), smoothing.data_ptr(), scales.data_ptr()),
        "pool encode")
    return codes, smoothing, scales


def pool_decode(codes: torch.Tensor, smoothing: torch.Tensor, scales: torch.Tensor,
                slot_ids: torch.Tensor, pool: torch.Tensor,
                layout: int = LAYOUT_KEY_VALUE) -> torch.Tensor:
    """Decode compact [layers,batch,heads] encodes and scatter into pool slots."""
    layers, slots, heads, batch = _pool_geometry(pool, slot_ids)
    tiles = layers * batch * heads
    _require(_tiles(codes, torch.int8, "codes") == tiles, "codes geometry differs")
    _vectors(smoothing, tiles, "smoothing")
    _vectors(scales, tiles, "scales")
    _check(native().pool_decode_launch_v4(
        _stream(), codes.data_ptr(), smoothing.data_ptr(), scales.data_ptr(),
        slot_ids.data_ptr(), batch, layers, slots, heads, layout, pool.data_ptr(),
        _pool_dtype(pool)), "pool decode")
    return pool


def _projection_inputs(codes, smoothing, scales, queries, heads_dim: int):
    _require(codes.is_cuda and codes.dtype == torch.int8 and codes.is_contiguous()
             and codes.dim() == 4 and tuple(codes.shape[-2:]) == (DIM, DIM),
             "GDN State Codec residual must be contiguous int8 [N,H,128,128]")
    tiles = codes.shape[0] * codes.shape[1]
    _vectors(smoothing, tiles, "smoothing")
    _vectors(scales, tiles, "scales")
    _require(queries.is_cuda and queries.dtype == torch.bfloat16 and queries.is_contiguous()
             and queries.shape[-1] == DIM, "GDN State Codec queries must be contiguous bf16")
    value_heads = codes.shape[1]
    query_heads = queries.shape[heads_dim]
    _require(query_heads > 0 and value_heads % query_heads == 0,
             "GDN State Codec value heads must be a multiple of query heads")
    return value_heads, query_heads


def project_decode(codes: torch.Tensor, smoothing: torch.Tensor, scales: torch.Tensor,
                   queries: torch.Tensor, query_scale: float = 1.0,
                   layout: int = LAYOUT_VALUE_KEY, out=None,
                   validate: bool = True) -> torch.Tensor:
    """o[b,h,v] = sum_k code(v,k) s[k] (query_scale q[b, h*Hq/H, k]) / 127 * scale[v].

    codes [B,H,128,128] int8; queries [B,Hq,128] bf16; returns fp32 [B,H,128].
    `validate=False` skips the tensor checks for callers that already made them
    on the same buffers (a decode loop); the library still checks its arguments."""
    batch = codes.shape[0]
    if validate:
        value_heads, query_heads = _projection_inputs(codes, smoothing, scales, queries, 1)
        _require(queries.dim() == 3 and queries.shape[0] == batch,
                 "GDN State Codec decode queries must be [B,Hq,128]")
    else:
        value_heads, query_heads = codes.shape[1], queries.shape[1]
    if out is None:
        out = torch.empty((batch, value_heads, DIM), dtype=torch.float32, device=codes.device)
    if validate:
        _require(out.is_contiguous() and out.dtype == torch.float32
                 and out.numel() == batch * value_heads * DIM, "output geometry differs")
    _check(native().encoded_projection_decode_launch_v4(
        _stream(), codes.data_ptr(), smoothing.data_ptr(), scales.data_ptr(),
        queries.data_ptr(), out.data_ptr(), batch, value_heads, query_heads,
        float(query_scale), layout), "decode projection")
    return out


def project_chunked(codes: torch.Tensor, smoothing: torch.Tensor, scales: torch.Tensor,
                    queries: torch.Tensor, query_scale: float = 1.0,
                    layout: int = LAYOUT_VALUE_KEY, out=None,
                    validate: bool = True) -> torch.Tensor:
    """Chunked projection of T query tokens per sequence against each sequence's state.

    codes [N,H,128,128] int8; queries [N,T,Hq,128] bf16; returns fp32 [N,T,H,128].
    `validate=False` skips the tensor checks, as for project_decode."""
    seqs = codes.shape[0]
    if validate:
        value_heads, query_heads = _projection_inputs(codes, smoothing, scales, queries, 2)
        _require(queries.dim() == 4 and queries.shape[0] == seqs,
                 "GDN State Codec chunked queries must be [N,T,Hq,128]")
    else:
        value_heads, query_heads = codes.shape[1], queries.shape[2]
    tokens = queries.shape[1]
    if out is None:
        out = torch.empty((seqs, tokens, value_heads, DIM), dtype=torch.float32,
                          device=codes.device)
    if validate:
        _require(out.is_contiguous() and out.dtype == torch.float32
                 and out.numel() == seqs * tokens * value_heads * DIM, "output geometry differs")
    _check(native().encoded_projection_chunked_launch_v4(
        _stream(), codes.data_ptr(), smoothing.data_ptr(), scales.data_ptr(),
        queries.data_ptr(), out.data_ptr(), seqs, tokens, value_heads, query_heads,
        float(query_scale), layout), "chunked projection")
    return out
