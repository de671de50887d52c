"""The C-ABI library: it loads without a GPU, exports every entry point the
headers under include/ declare, is reachable under the reference's library
file names, and rejects bad arguments with the reference's status 1 before any
HIP call (so these run on the CPU)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
INCLUDE = ROOT / "include"


def _declared_symbols():
    names = set()
    for header in INCLUDE.glob("*.h"):
        text = header.read_text()
        names.update(re.findall(r"\b(statecentric_gdn_state_codec_\w+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib():
    from gdn_state_codec import _native

    path = _native.library_path()
    if not path.is_file():
        import subprocess
        import sys

        subprocess.run([sys.executable, str(ROOT / "gdn-state-codec_amd" / "build.py")],
                       check=True)
    return _native.NativeLibrary()


def test_headers_declare_the_hot_path():
    symbols = _declared_symbols()
    for required in (
        "statecentric_gdn_state_codec_smoothing_launch_v1",
        "statecentric_gdn_state_codec_quantize_launch_v1",
        "statecentric_gdn_state_codec_dequantize_launch_v1",
        "statecentric_gdn_state_codec_provider_smoothing_launch_v2",
        "statecentric_gdn_state_codec_provider_quantize_launch_v2",
        "statecentric_gdn_state_codec_provider_initialize_launch_v3",
        "statecentric_gdn_state_codec_encode_launch_v4",
        "statecentric_gdn_state_codec_decode_launch_v4",
        "statecentric_gdn_state_codec_encoded_projection_decode_launch_v4",
        "statecentric_gdn_state_codec_encoded_projection_chunked_launch_v4",
    ):
        assert required in symbols


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_symbols():
        assert hasattr(lib._lib, name), name


def test_reference_library_names_resolve(lib):
    from gdn_state_codec import _native
    from gdn_state_codec.runtime import _GdnStateCodecLibraries

    libraries = _GdnStateCodecLibraries(_native.library_dir())
    assert libraries.provider_initialize is not None
    for file_name, symbol in _GdnStateCodecLibraries._NAMES.values():
        handle = ctypes.CDLL(str(_native.library_dir() / file_name))
        assert hasattr(handle, symbol)


def test_null_and_out_of_range_arguments_return_status_1(lib):
    p = ctypes.c_void_p(16)  # never dereferenced: admission fails first
    assert lib.smoothing_launch_v1(None, None, p) == 1
    assert lib.quantize_launch_v1(None, p, p, p, None) == 1
    assert lib.dequantize_launch_v1(None, p, p, p, None, p, p) == 1
    for states in (0, 65):
        assert lib.provider_smoothing_launch_v2(None, p, p, states) == 1
        assert lib.provider_quantize_launch_v2(None, p, p, p, p, states) == 1
        assert lib.provider_initialize_launch_v3(None, p, p, p, p, states) == 1
    assert lib.encode_launch_v4(None, p, p, p, p, 0, 0) == 1
    assert lib.encode_launch_v4(None, p, p, p, p, 4, 2) == 1
    assert lib.encode_launch_v4(None, p, None, p, p, 4, 0) == 1
    assert lib.decode_launch_v4(None, p, p, p, p, None, p, 4, 0) == 1  # unpaired compensators
    assert lib.pool_encode_launch_v4(None, p, 2, p, 1, 1, 1, 1, 0, p, p, p) == 1  # dtype
    assert lib.pool_decode_launch_v4(None, p, p, p, None, 1, 1, 1, 1, 0, p, 0) == 1
    assert lib.encoded_projection_decode_launch_v4(None, p, p, p, p, p, 1, 32, 3, 1.0, 1) == 1
    assert lib.encoded_projection_decode_launch_v4(None, p, p, p, p, p, 0, 32, 16, 1.0, 1) == 1
    assert lib.encoded_projection_chunked_launch_v4(None, p, p, p, p, p, 1, 0, 32, 16, 1.0, 1) == 1
    assert lib.encoded_projection_chunked_launch_v4(None, p, p, p, p, p, 1, 4, 32, 16, 1.0, 7) == 1
    # One sequence's output rows must span fewer than 2^32 bytes (32-bit lane offsets).
    assert lib.encoded_projection_chunked_launch_v4(None, p, p, p, p, p, 1, 1 << 18, 32, 16,
                                                    1.0, 1) == 1


def test_windowed_entry_points_admit_like_the_reference(lib):
    """windowed_gdn_step.cpp:675-678, 729-734, 757-762; encoded_projection.cpp:
    867-963; int8_cube_matmul.cpp:57-63: status 1 for a null pointer, a count
    outside 1..16384 and (bf16) an odd count, before any device work."""
    p = ctypes.c_void_p(16)
    sixteen = [p] * 15
    for states in (0, 16385):
        assert lib.windowed_gdn_step_launch_v1(None, *sixteen, states) == 1
        assert lib.windowed_gdn_step_bf16_launch_v1(None, *sixteen, states) == 1
        assert lib.windowed_gdn_step_bf16_quant_only_launch_v1(None, *sixteen, states) == 1
        assert lib.fp32_gdn_step_launch_v1(None, *([p] * 7), states) == 1
        assert lib.prepare_int8_vector_launch_v1(None, p, p, p, p, states) == 1
        assert lib.prepare_decode_pair_launch_v1(None, *([p] * 6), states) == 1
        assert lib.prepare_decode_pair_bf16_launch_v1(None, *([p] * 6), states) == 1
        assert lib.finish_decode_pair_launch_v1(None, *sixteen, states) == 1
        assert lib.finish_decode_pair_bf16_launch_v1(None, *sixteen, states) == 1
    assert lib.windowed_gdn_step_bf16_launch_v1(None, *sixteen, 7) == 1
    assert lib.windowed_gdn_step_bf16_quant_only_launch_v1(None, *sixteen, 7) == 1
    assert lib.prepare_decode_pair_bf16_launch_v1(None, *([p] * 6), 7) == 1
    assert lib.finish_decode_pair_bf16_launch_v1(None, *sixteen, 7) == 1
    for i in range(15):  # every pointer is required, compensators included
        args = list(sixteen)
        args[i] = None
        assert lib.windowed_gdn_step_bf16_quant_only_launch_v1(None, *args, 2) == 1
        assert lib.windowed_gdn_step_launch_v1(None, *args, 2) == 1
    # int8 projection: states 1..128, blocks == (states + 1) / 2, workspace and
    # tiling present, transpose_a <= 1.
    assert lib.int8_cube_matmul_launch_v1(None, p, p, p, 129, 0, p, p, 65) == 1
    assert lib.int8_cube_matmul_launch_v1(None, p, p, p, 8, 0, p, p, 3) == 1
    assert lib.int8_cube_matmul_launch_v1(None, p, p, p, 8, 2, p, p, 4) == 1
    assert lib.int8_cube_matmul_launch_v1(None, p, p, p, 8, 0, None, p, 4) == 1
    # The batched product: 1..16384 states, transpose_a <= 1, 16-byte aligned.
    for states, transpose in ((0, 0), (16385, 0), (8, 2)):
        assert lib.int8_matmul_launch_v4(None, p, p, p, states, transpose) == 1
    assert lib.int8_matmul_launch_v4(None, None, p, p, 8, 0) == 1
    assert lib.int8_matmul_launch_v4(None, p, p, ctypes.c_void_p(20), 8, 0) == 1
    # The exact-SVD sweep limit: 1..30.
    for sweeps in (0, 31):
        assert lib.exact_svd_boundary_sweeps_launch_v1(None, *[p] * 8, 1, sweeps) == 1


def test_decode_runtime_lifecycle(lib):
    """decode_runtime.cpp:72-148: one live handle per process, bound to its
    state count, reference-counted; foreign handles are rejected."""
    p = ctypes.c_void_p(16)
    assert not lib.decode_runtime_create_v1(0)
    assert not lib.decode_runtime_create_v1(16385)
    a = lib.decode_runtime_create_v1(64)
    assert a
    assert lib.decode_runtime_create_v1(64) == a
    assert not lib.decode_runtime_create_v1(32)
    assert lib.decode_runtime_step_v1(a, None, *([p] * 15), 32) == 1  # other count
    assert lib.decode_runtime_step_v1(p, None, *([p] * 15), 64) == 1  # foreign handle
    assert lib.decode_runtime_step_v1(a, None, *([p] * 15), 63) == 1
    args = [p] * 15
    args[11] = None  # keys: the prepare stage's argument
    assert lib.decode_runtime_step_v1(a, None, *args, 64) == 2
    args = [p] * 15
    args[14] = None  # outputs: the finish stage's argument
    assert lib.decode_runtime_step_v1(a, None, *args, 64) == 4
    lib.decode_runtime_destroy_v1(p)  # ignored
    lib.decode_runtime_destroy_v1(a)
    assert lib.decode_runtime_create_v1(64) == a  # still live: one reference left
    lib.decode_runtime_destroy_v1(a)
    lib.decode_runtime_destroy_v1(a)
    b = lib.decode_runtime_create_v1(32)  # released: a new count is accepted
    assert b
    lib.decode_runtime_destroy_v1(b)


def test_boundary_entry_points_admit_like_the_reference(lib):
    """window_boundary.cpp:661-669, 705-712, 724-731; bf16_cube_matmul.cpp:56-60."""
    p = ctypes.c_void_p(16)
    assert lib.window_boundary_launch_v1(None, *([p] * 15), 8, 33) == 1
    for states in (0, 16385):
        assert lib.window_boundary_launch_v1(None, *([p] * 15), states, 0) == 1
    for i in range(15):
        args = [p] * 15
        args[i] = None
        assert lib.window_boundary_launch_v1(None, *args, 8, 0) == 1
        assert lib.window_boundary_cube_finish_launch_v1(None, *args, 8) == 1
    for states in (0, 129):
        assert lib.window_boundary_cube_finish_launch_v1(None, *([p] * 15), states) == 1
        assert lib.boundary_scale_records_launch_v1(None, p, p, p, states) == 1
    assert lib.bf16_cube_matmul_launch_v1(None, p, p, p, 8, p, p, 3) == 1
    assert lib.bf16_cube_matmul_launch_v1(None, p, p, p, 8, None, p, 4) == 1
    assert lib.bf16_cube_matmul_launch_v1(None, p, p, p, 130, p, p, 65) == 1


def test_encoded_rank_chain_admits_like_the_reference(lib):
    """encoded_projection.cpp:972-976, 1000-1004; encoded_requantize.cpp:200-204:
    every pointer required, 1 <= states <= 16384, fitted_ranks <= 4,
    transpose <= 1, rank < 4; all rejected before any HIP call."""
    p = ctypes.c_void_p(16)
    thirteen = [p] * 13
    for states, fitted, transpose in ((0, 0, 0), (16385, 0, 0), (8, 5, 0), (8, 0, 2)):
        assert lib.finish_encoded_projection_launch_v1(
            None, *thirteen, states, fitted, transpose) == 1
    for states, rank in ((0, 0), (16385, 0), (8, 4)):
        assert lib.commit_encoded_rank_launch_v1(None, *thirteen, states, rank) == 1
    for states in (0, 16385):
        assert lib.encoded_requantize_launch_v1(None, *([p] * 16), states) == 1
    for i in range(13):
        args = list(thirteen)
        args[i] = None
        assert lib.finish_encoded_projection_launch_v1(None, *args, 8, 4, 1) == 1
        assert lib.commit_encoded_rank_launch_v1(None, *args, 8, 3) == 1
    for i in range(16):
        args = [p] * 16
        args[i] = None
        assert lib.encoded_requantize_launch_v1(None, *args, 8) == 1


def test_quantize_boundary_admission(lib):
    """The rank-r boundary encode: every pointer required except the
    compensators at rank 0, 1 <= heads <= 2^31-1 and rank <= 4; all rejected
    before any HIP call."""
    p = ctypes.c_void_p(16)
    eight = [p] * 8
    for heads, rank in ((0, 4), (1 << 31, 4), (2, 5)):
        assert lib.quantize_boundary_launch_v1(None, *eight, heads, rank) == 1
    for i in range(8):
        args = list(eight)
        args[i] = None
        assert lib.quantize_boundary_launch_v1(None, *args, 2, 4) == 1
        if i not in (5, 6):  # the compensators may be null at rank 0
            assert lib.quantize_boundary_launch_v1(None, *args, 2, 0) == 1


def test_exact_svd_boundary_admission(lib):
    """The exact-SVD initializer: every pointer required and
    1 <= heads <= 2^31-1; all rejected before any HIP call."""
    p = ctypes.c_void_p(16)
    eight = [p] * 8
    for heads in (0, 1 << 31):
        assert lib.exact_svd_boundary_launch_v1(None, *eight, heads) == 1
    for i in range(8):
        args = list(eight)
        args[i] = None
        assert lib.exact_svd_boundary_launch_v1(None, *args, 2) == 1


def test_noalloc_refit_admission(lib):
    """The allocation-free refit: every pointer required, at most 512 states
    when the power refit needs the scratch workspace, 16384 without it, and
    at most 32 iterations; all rejected before any HIP call."""
    p = ctypes.c_void_p(16)
    fourteen = [p] * 14
    assert lib.window_boundary_noalloc_launch_v1(None, *fourteen, 8, 33) == 1
    for states, iterations in ((0, 0), (0, 4), (16385, 0), (513, 1), (513, 32), (4096, 4)):
        assert lib.window_boundary_noalloc_launch_v1(None, *fourteen, states, iterations) == 1
    for i in range(14):
        args = list(fourteen)
        args[i] = None
        assert lib.window_boundary_noalloc_launch_v1(None, *args, 8, 0) == 1
        assert lib.window_boundary_noalloc_launch_v1(None, *args, 8, 4) == 1


def test_boundary_runtime_lifecycle(lib):
    """boundary_runtime.cpp:60-128."""
    p = ctypes.c_void_p(16)
    assert not lib.boundary_runtime_create_v1(0)
    assert not lib.boundary_runtime_create_v1(129)
    a = lib.boundary_runtime_create_v1(32)
    assert a and lib.boundary_runtime_create_v1(32) == a
    assert not lib.boundary_runtime_create_v1(16)
    assert lib.boundary_runtime_step_v1(a, None, p, p, p, p, p, 16) == 1
    assert lib.boundary_runtime_step_v1(p, None, p, p, p, p, p, 32) == 1
    assert lib.boundary_runtime_step_v1(a, None, p, None, p, p, p, 32) == 1
    lib.boundary_runtime_destroy_v1(a)
    lib.boundary_runtime_destroy_v1(a)
    b = lib.boundary_runtime_create_v1(16)
    assert b
    lib.boundary_runtime_destroy_v1(b)


def test_capsule_entry_points_admit_and_size_capsules(lib):
    """The capsule entry points reject before any HIP call: null pointers,
    states outside 1..16384, layouts other than 0/1 and an identity that
    ValidateIdentity refuses (state_capsule.cpp:40-48)."""
    for p in range(16):
        assert lib.capsule_bytes_v1(p) == 21688 + 1536 * p
    assert lib.capsule_bytes_v1(16) == 0 and lib.capsule_bytes_v1(2 ** 32 - 1) == 0
    p = ctypes.c_void_p(16)
    good = b"0123456789abcdef" * 4

    def ser(args=None, layout=1, geometry=good, generation=1, epoch=1, states=4):
        args = [p] * 12 if args is None else args
        return lib.capsule_serialize_launch_v1(None, *args[:9], layout, geometry, generation,
                                               epoch, args[9], args[10], 1 << 20, args[11],
                                               states)

    def res(args=None, layout=1, geometry=good, generation=1, epoch=1, states=4):
        args = [p] * 14 if args is None else args
        return lib.capsule_restore_launch_v1(None, *args[:3], 1 << 20, geometry, generation,
                                             epoch, args[3], layout, *args[4:], states)

    for fn, n in ((ser, 12), (res, 14)):
        for i in range(n):
            args = [p] * n
            args[i] = None
            assert fn(args) == 1, (fn.__name__, i)
        for states in (0, 16385):
            assert fn(states=states) == 1
        assert fn(layout=2) == 1
        for geometry in (b"A" * 64, b"0123456789abcdeg" + b"0" * 48, None):
            assert fn(geometry=geometry) == 1
        assert fn(generation=0) == 1 and fn(epoch=0) == 1


# Argument templates of every entry point with valid counts: "P" marks a device
# pointer the kernels access (it must be 16-byte aligned), other entries are
# passed as written (the stream, host pointers, unused Cube workspace/tiling).
_GEOMETRY = b"0123456789abcdef" * 4
_ALIGNMENT_CASES = {
    "smoothing_launch_v1": [None, "P", "P"],
    "quantize_launch_v1": [None] + ["P"] * 4,
    "dequantize_launch_v1": [None] + ["P"] * 6,
    "provider_smoothing_launch_v2": [None, "P", "P", 4],
    "provider_quantize_launch_v2": [None] + ["P"] * 4 + [4],
    "provider_initialize_launch_v3": [None] + ["P"] * 4 + [4],
    "encode_launch_v4": [None] + ["P"] * 4 + [4, 0],
    "decode_launch_v4": [None] + ["P"] * 6 + [4, 0],
    "pool_encode_launch_v4": [None, "P", 0, "P", 2, 1, 4, 2, 0, "P", "P", "P"],
    "pool_decode_launch_v4": [None, "P", "P", "P", "P", 2, 1, 4, 2, 0, "P", 0],
    "encoded_projection_decode_launch_v4": [None] + ["P"] * 5 + [1, 32, 16, 1.0, 1],
    "encoded_projection_chunked_launch_v4": [None] + ["P"] * 5 + [1, 4, 32, 16, 1.0, 1],
    "windowed_gdn_step_launch_v1": [None] + ["P"] * 15 + [2],
    "windowed_gdn_step_bf16_launch_v1": [None] + ["P"] * 15 + [2],
    "windowed_gdn_step_bf16_quant_only_launch_v1": [None] + ["P"] * 15 + [2],
    "fp32_gdn_step_launch_v1": [None] + ["P"] * 7 + [2],
    "prepare_int8_vector_launch_v1": [None] + ["P"] * 4 + [2],
    "prepare_decode_pair_launch_v1": [None] + ["P"] * 6 + [2],
    "prepare_decode_pair_bf16_launch_v1": [None] + ["P"] * 6 + [2],
    "int8_cube_matmul_launch_v1": [None, "P", "P", "P", 2, 0, 16, 16, 1],
    "finish_decode_pair_launch_v1": [None] + ["P"] * 15 + [2],
    "finish_decode_pair_bf16_launch_v1": [None] + ["P"] * 15 + [2],
    "window_boundary_launch_v1": [None] + ["P"] * 15 + [2, 0],
    "finish_encoded_projection_launch_v1": [None] + ["P"] * 13 + [2, 4, 1],
    "commit_encoded_rank_launch_v1": [None] + ["P"] * 13 + [2, 3],
    "encoded_requantize_launch_v1": [None] + ["P"] * 16 + [2],
    "window_boundary_noalloc_launch_v1": [None] + ["P"] * 14 + [2, 4],
    "boundary_scale_records_launch_v1": [None] + ["P"] * 3 + [2],
    "window_boundary_cube_finish_launch_v1": [None] + ["P"] * 15 + [2],
    "bf16_cube_matmul_launch_v1": [None, "P", "P", "P", 2, 16, 16, 1],
    "quantize_boundary_launch_v1": [None] + ["P"] * 8 + [2, 4],
    "exact_svd_boundary_launch_v1": [None] + ["P"] * 8 + [2],
    "capsule_serialize_launch_v1": [None] + ["P"] * 9 + [1, _GEOMETRY, 1, 1, "P", "P", 1 << 20,
                                                          "P", 2],
    "capsule_restore_launch_v1": [None, "P", "P", "P", 1 << 20, _GEOMETRY, 1, 1, "P", 1]
                                 + ["P"] * 10 + [2],
}


@pytest.mark.parametrize("name", sorted(_ALIGNMENT_CASES))
def test_misaligned_pointers_return_status_1(lib, name):
    """Each device pointer in turn 4 bytes off a 16-byte boundary, every other
    argument valid: status 1, before any HIP call (this runs without a GPU)."""
    template = _ALIGNMENT_CASES[name]
    fn = getattr(lib, name)
    slots = [i for i, a in enumerate(template) if a == "P"]
    assert slots and len(template) == len(fn.argtypes), name
    for slot in slots:
        args = [ctypes.c_void_p(20 if i == slot else 16) if a == "P" else a
                for i, a in enumerate(template)]
        assert fn(*args) == 1, (name, slot)


def test_runtime_steps_reject_misaligned_pointers(lib):
    """The decode and boundary runtime steps: a misaligned pointer is a bad
    argument (status 1), whatever stage it belongs to."""
    decode = lib.decode_runtime_create_v1(2)
    boundary = lib.boundary_runtime_create_v1(2)
    assert decode and boundary
    try:
        for slot in range(15):
            args = [ctypes.c_void_p(20 if i == slot else 16) for i in range(15)]
            assert lib.decode_runtime_step_v1(decode, None, *args, 2) == 1, slot
        for slot in range(5):
            args = [ctypes.c_void_p(20 if i == slot else 16) for i in range(5)]
            assert lib.boundary_runtime_step_v1(boundary, None, *args, 2) == 1, slot
    finally:
        lib.decode_runtime_destroy_v1(decode)
        lib.boundary_runtime_destroy_v1(boundary)
