"""The LDS residency probe behind `bench.py --lds-residency`
(gdn-state-codec_amd/csrc/bench/lds_probe.hip): its argument limits, checked
on the host before any launch, and one small launch on the GPU in which every
workgroup waits at least the requested ticks and reads back its LDS."""

from __future__ import annotations

import ctypes

import pytest

from gdn_state_codec import _native


def _lib():
    lib = ctypes.CDLL(str(_native.library_dir() / "libgdn_state_codec_hbm_probe.so"))
    lib.gdn_lds_residency_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32,
                                            ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64]
    lib.gdn_lds_residency_probe.restype = ctypes.c_int32
    return lib


@pytest.mark.parametrize("blocks, threads, lds, ticks, null_sink", [
    (256, 128, 4096, 100, True),          # no sink
    (0, 128, 4096, 100, False),           # no workgroups
    ((1 << 20) + 1, 128, 4096, 100, False),
    (256, 32, 4096, 100, False),          # threads other than 64 / 128
    (256, 256, 4096, 100, False),
    (256, 128, 511, 100, False),          # LDS below one word per thread
    (256, 128, 160 * 1024 + 1, 100, False),
    (256, 128, 4096, 0, False),           # no wait
    (256, 128, 4096, 10_000_001, False),  # wait above 0.1 s
])
def test_probe_rejects_arguments_outside_its_limits(blocks, threads, lds, ticks, null_sink):
    sink = ctypes.create_string_buffer(16)  # never dereferenced: the checks come first
    pointer = None if null_sink else ctypes.addressof(sink)
    assert _lib().gdn_lds_residency_probe(None, pointer, blocks, threads, lds, ticks) == 1


@pytest.mark.gpu
@pytest.mark.parametrize("threads, lds", [(64, 5120), (128, 32000)])
def test_probe_waits_and_reads_its_lds(device, threads, lds):
    import torch

    print(f"lds residency probe threads={threads} lds={lds}", flush=True)
    blocks, ticks = 2 * 256, 2000  # 20 us on the 100 MHz counter
    sink = torch.zeros(blocks, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    assert _lib().gdn_lds_residency_probe(stream, sink.data_ptr(), blocks, threads, lds,
                                          ticks) == 0
    torch.cuda.synchronize()
    got = sink.cpu()
    # Thread 0 of each workgroup stores lds[1] (= 1, written by thread 1) plus
    # the ticks it waited, at least `ticks`.
    assert (got >= ticks + 1).all()
    assert (got < ticks + 1 + 10_000_000).all()
