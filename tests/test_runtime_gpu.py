"""The slot runtime (reference-runtime mirror) on the GPU: slot encode of a
provider state, reconstruct, boundary projection, slot map and errors."""

import numpy as np
import pytest
import torch

import datagen
import oracle
from gdn_state_codec import GdnStateCodecRuntime, codec

pytestmark = pytest.mark.gpu


def to_np(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("heads", [32, 80])
def test_slot_encode_reconstruct_and_project(device, heads):
    print(f"runtime slot heads={heads}", flush=True)
    runtime = GdnStateCodecRuntime()
    provider = datagen.c1_heads(3 * heads, 5).reshape(3, heads, 128, 128)  # [slots,H,V,K]
    state = torch.from_numpy(provider).to(device)
    slot = runtime._slot(state, 1)
    codes, s, sc = oracle.encode_heads(provider[1], oracle.LAYOUT_VALUE_KEY, threads=8)
    assert to_np(slot.residual).tobytes() == codes.tobytes()
    assert to_np(slot.smoothing).tobytes() == s.tobytes()
    assert to_np(slot.scales).tobytes() == sc.tobytes()
    assert runtime._slot(state, 1) is slot
    dense = to_np(runtime.reconstruct(slot))  # [H,K,V]
    expect = oracle.decode_heads(codes, s, sc, oracle.LAYOUT_VALUE_KEY).transpose(0, 2, 1)
    assert dense.tobytes() == np.ascontiguousarray(expect).tobytes()
    g = datagen.rng(6)
    q = oracle.f32_to_bf16(g.standard_normal((1, 1, heads // 2, 128)).astype(np.float32))
    out = to_np(runtime.project(slot, torch.from_numpy(q).to(device).view(torch.bfloat16)))
    _, out64, bound = oracle.project_decode(codes[None], s[None], sc[None], q[0], 128 ** -0.5,
                                            oracle.LAYOUT_VALUE_KEY)
    assert (np.abs(out[0] - out64) <= 2.0 ** -15 * bound + 1e-30).all()
    runtime.invalidate((1,))
    assert runtime._slot(state, 1) is not slot


def test_runtime_contract_errors(device):
    runtime = GdnStateCodecRuntime()
    state = torch.zeros((2, 4, 128, 128), dtype=torch.float32, device=device)
    with pytest.raises(RuntimeError, match="out of range"):
        runtime._slot(state, 2)
    with pytest.raises(RuntimeError, match="FP32"):
        runtime._encode_quant_only_provider(state[0].to(torch.float16))
    with pytest.raises(RuntimeError, match="contiguous"):
        runtime._encode_quant_only_provider(state[0].transpose(-2, -1))
    slot = runtime._slot(state, 0)
    with pytest.raises(RuntimeError, match="H/2"):
        runtime.project(slot, torch.zeros((1, 1, 4, 128), dtype=torch.bfloat16, device=device))
    runtime.fall_back_to_native("multi-request decode batch")
    assert runtime.native_fallbacks == 1 and not runtime._slots
