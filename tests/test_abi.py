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
