"""GPU check of the wavefront exchanges (csrc/lane_exchange.h) that the window
step, the projections and the decode-pair chain reduce with: DPP partners
lane ^ 1, 2, 4, 8, the gfx950 permlane swaps for lane ^ 16, 32, the butterfly
sum and the DPP maximum, each against the same arithmetic in numpy.  Sums
must match bit for bit: each lane adds the same two float32 operands."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from gdn_state_codec import _native

pytestmark = pytest.mark.gpu
LANES = 64
MASKS = (32, 16, 8, 4, 2, 1)


def _probe():
    lib = ctypes.CDLL(str(_native.library_dir() / "libgdn_state_codec_hbm_probe.so"))
    lib.gdn_lane_probe.argtypes = [ctypes.c_void_p] * 3
    lib.gdn_lane_probe.restype = ctypes.c_int32
    lib.gdn_lane_probe_outputs.restype = ctypes.c_uint32
    return lib


def _fold(lo, hi, mask):
    lanes = np.arange(LANES)
    partner = lanes ^ mask
    up = (lanes & mask) != 0
    return np.where(up, hi + hi[partner], lo + lo[partner])


def _butterfly_sum(x):
    for mask in MASKS:
        x = x + x[np.arange(LANES) ^ mask]
    return x


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_lane_exchanges_match_numpy(device, seed):
    print(f"lane exchange probe seed={seed}", flush=True)
    lib = _probe()
    g = np.random.default_rng(seed)
    x = (g.standard_normal(LANES) * np.exp2(g.integers(-20, 20, LANES))).astype(np.float32)
    y = (g.standard_normal(LANES) * np.exp2(g.integers(-20, 20, LANES))).astype(np.float32)
    if seed == 2:  # exact zeros and a negative maximum magnitude pattern
        x[::7] = 0.0
        x = -np.abs(x)
    data = torch.from_numpy(np.concatenate([x, y])).to(device)
    out = torch.empty(lib.gdn_lane_probe_outputs(), dtype=torch.float32, device=device)
    assert lib.gdn_lane_probe(torch.cuda.current_stream().cuda_stream, data.data_ptr(),
                              out.data_ptr()) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().reshape(-1, LANES)
    for block, mask in enumerate(MASKS):
        assert got[block].tobytes() == _fold(x, y, mask).tobytes(), ("fold", mask)
        partner = x + x[np.arange(LANES) ^ mask]
        assert got[6 + block].tobytes() == partner.tobytes(), ("add_partner", mask)
    assert got[12].tobytes() == _butterfly_sum(x).tobytes()
    assert (got[13] == np.max(x)).all()
    xi, yi = x.view(np.int32), y.view(np.int32)
    for block, mask in zip((14, 15, 16), (4, 2, 1)):
        lanes = np.arange(LANES)
        want = np.where((lanes & mask) != 0, yi + yi[lanes ^ mask], xi + xi[lanes ^ mask])
        assert got[block].view(np.int32).tobytes() == want.astype(np.int32).tobytes(), mask
