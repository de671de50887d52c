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
    runtime.close()


def test_runtime_contract_errors(device):
    runtime = GdnStateCodecRuntime()
    state = torch.zeros((2, 4, 128, 128), dtype=torch.float32, device=device)
    with pytest.raises(RuntimeError, match="out of range"):
        runtime._slot(state, 2)
    with pytest.raises(RuntimeError, match="float32"):
        runtime._encode_quant_only_provider(state[0].to(torch.float16))
    with pytest.raises(RuntimeError, match="not contiguous"):
        runtime._encode_quant_only_provider(state[0].transpose(-2, -1))
    with pytest.raises(RuntimeError, match=r"\[H,128,128\]"):
        runtime._encode_quant_only_provider(state)
    slot = runtime._slot(state, 0)
    with pytest.raises(RuntimeError, match=r"\(1, 1, 2, 128\)"):
        runtime.project(slot, torch.zeros((1, 1, 4, 128), dtype=torch.bfloat16, device=device))
    runtime.fall_back_to_native("multi-request decode batch")
    assert runtime.native_fallbacks == 1 and not runtime._slots
    assert runtime.native_fallback_reasons == {"multi-request decode batch": 1}
    runtime.close()


def test_runtime_checks_every_token(device):
    """The token contract is enforced on every call, not only the first: a
    later token with a wrong shape, dtype, layout, device or query scale raises
    before any launch and leaves the slot's window position unchanged."""
    runtime = GdnStateCodecRuntime()
    heads = 4
    state = torch.zeros((1, heads, 128, 128), dtype=torch.float32, device=device)
    bf = lambda *shape: torch.zeros(shape, dtype=torch.bfloat16, device=device)  # noqa: E731
    good = dict(query=bf(1, 1, 2, 128), key=bf(1, 1, 2, 128), value=bf(1, 1, heads, 128),
                log_decay=torch.zeros((1, 1, heads), dtype=torch.float32, device=device),
                beta=bf(1, 1, heads))
    run = lambda **kw: runtime.step(state, 0, query_scale=kw.pop("scale", 128 ** -0.5),  # noqa
                                    **{**good, **kw})
    run()
    torch.cuda.synchronize()
    slot = runtime._slot(state, 0)
    assert slot.steps == 1
    bad = {"query": bf(1, 1, 4, 128),
           "key": bf(1, 1, 2, 256)[..., ::2],
           "value": torch.zeros((1, 1, heads, 128), dtype=torch.float32, device=device),
           "log_decay": torch.zeros((1, 1, heads), dtype=torch.float32),
           "beta": bf(1, 1, heads + 2)}
    for name, tensor in bad.items():
        with pytest.raises(RuntimeError, match=name):
            run(**{name: tensor})
    with pytest.raises(RuntimeError, match="query scale"):
        run(scale=1.0)
    assert slot.steps == 1
    run()
    torch.cuda.synchronize()
    assert slot.steps == 2 and int(slot.positions[0, 0]) == 2
    runtime.close()


def slot_buffers(slot) -> dict:
    """Host copy of a slot in the oracle's buffer naming."""
    torch.cuda.synchronize()
    h = lambda t, dt: t.cpu().numpy().view(dt).copy()  # noqa: E731
    return {"residual": h(slot.residual, np.int8), "smoothing": h(slot.smoothing, np.float32),
            "scales": h(slot.scales, np.float32),
            "compensator_keys": h(slot.compensator_keys, np.uint16),
            "compensator_values": h(slot.compensator_values, np.uint16),
            "record_decay": h(slot.record_decay, np.float32),
            "record_keys": h(slot.record_keys, np.uint16),
            "record_corrections": h(slot.record_corrections, np.uint16),
            "positions": h(slot.positions, np.uint32)}


@pytest.mark.parametrize("backend,power,initializer", [
    ("vector", 0, "quant_only"), ("cube", 0, "quant_only"), ("vector", 3, "quant_only"),
    ("vector", 3, "exact_svd"), ("cube", 2, "exact_svd")])
def test_runtime_steps_through_two_window_refits(device, backend, power, initializer):
    """40 decode tokens through GdnStateCodecRuntime.step (two refits): every
    step and refit is checked against the oracle applied to the slot's own
    buffers just before it.  With the exact-SVD initializer the first window
    runs on a boundary with fitted compensators."""
    from gdn_state_codec import GdnStateCodecExperiment
    from oracle import window as W
    import windowgen as WG
    from test_window_gpu import check_step

    print(f"runtime steps backend={backend} power={power} initializer={initializer}",
          flush=True)
    heads = 32
    runtime = GdnStateCodecRuntime(GdnStateCodecExperiment(
        decode_backend=backend, boundary_power_iterations=power, initializer=initializer))
    provider = datagen.c1_heads(2 * heads, 9).reshape(2, heads, 128, 128)
    state = torch.from_numpy(provider).to(device)
    slot = runtime._slot(state, 1)
    if initializer == "exact_svd":
        assert slot.compensator_keys.abs().max().item() > 0
    try:
        for t in range(40):
            inp = WG.bf16_inputs(heads, 300 + t)
            before = slot_buffers(slot)
            steps = slot.steps
            if steps == 16:
                out = W.boundary_outputs(heads)
                if power == 0:
                    scaled = W.boundary_scale_records(before["record_decay"], before["record_keys"])
                    merge = W.f16_matmul_at_b(before["record_corrections"], scaled)
                    W.window_boundary_quant_only(before, out, merge)
                else:
                    W.window_boundary_power(before, out, np.zeros((heads, 128, 128), np.float32),
                                            power)
                before.update(residual=out["next_residual"], smoothing=out["next_smoothing"],
                              scales=out["next_scales"],
                              compensator_keys=out["next_compensator_keys"],
                              compensator_values=out["next_compensator_values"])
            as_torch = lambda a, shape: torch.from_numpy(a.reshape(shape)).to(device)  # noqa
            got = runtime.step(
                state, 1,
                as_torch(inp["queries"].view(np.int16), (1, 1, heads // 2, 128)).view(torch.bfloat16),
                as_torch(inp["keys"].view(np.int16), (1, 1, heads // 2, 128)).view(torch.bfloat16),
                as_torch(inp["values"].view(np.int16), (1, 1, heads, 128)).view(torch.bfloat16),
                as_torch(inp["log_decay"], (1, 1, heads)),
                as_torch(inp["beta"].view(np.int16), (1, 1, heads)).view(torch.bfloat16),
                128 ** -0.5)
            after = slot_buffers(slot)
            if steps == 16:  # the refit's new boundary, bit-exact
                for name in ("residual", "smoothing", "scales", "compensator_keys",
                             "compensator_values"):
                    assert after[name].tobytes() == before[name].tobytes(), (t, name)
            out_gpu = got.view(torch.int16).cpu().numpy().view(np.uint16).reshape(heads, 128)
            ref = WG.copy_buffers(before)
            if backend == "vector":
                out_ref, out64, out_bound, corr64, corr_bound = W.windowed_step_bf16(
                    ref, **inp, quant_only=power == 0)
                check_step(before, after, ref, out_gpu, out_ref, out64, out_bound, corr64,
                           corr_bound, 16)
            else:
                q, dyn = W.prepare_decode_pair_bf16(inp["keys"], inp["queries"],
                                                    inp["log_decay"], before["smoothing"])
                out_ref = W.finish_decode_pair_bf16(
                    ref, W.int8_matmul(before["residual"], q), dyn, **inp)
                assert out_gpu.tobytes() == out_ref.tobytes(), t
                for name in ref:
                    assert after[name].tobytes() == ref[name].tobytes(), (t, name)
        assert runtime.boundary_refits == 2
    finally:
        runtime.close()


def test_exact_svd_slot_and_reconstruct(device):
    """The exact-SVD initializer's slot holds what codec.exact_svd_boundary
    writes for the same provider state (byte for byte), an empty window, and
    reconstructs to the dequantized residual plus the fp16 compensator product;
    the reference's dense entry point (_encode_dense_boundary, [key][value]
    heads) gives the same slot."""
    from gdn_state_codec import GdnStateCodecExperiment

    heads = 16
    print(f"runtime exact SVD slot, heads={heads}", flush=True)
    runtime = GdnStateCodecRuntime(GdnStateCodecExperiment(
        initializer="exact_svd", boundary_power_iterations=2))
    provider = datagen.student_t_heads(2 * heads, 83).reshape(2, heads, 128, 128)
    state = torch.from_numpy(provider).to(device)
    try:
        slot = runtime._slot(state, 0)
        expect = codec.exact_svd_boundary(state[0].contiguous())
        for name, want in zip(("residual", "smoothing", "scales", "compensator_keys",
                               "compensator_values"), expect):
            assert to_np(getattr(slot, name)).tobytes() == to_np(want).tobytes(), name
        assert not to_np(slot.positions).any()
        dense = runtime._encode_dense_boundary(state[0].transpose(-2, -1))
        assert to_np(dense.residual).tobytes() == to_np(slot.residual).tobytes()
        assert (to_np(dense.compensator_keys).tobytes()
                == to_np(slot.compensator_keys).tobytes())
        got = to_np(runtime.reconstruct(slot))
        codes, s, sc = (to_np(slot.residual), to_np(slot.smoothing), to_np(slot.scales))
        base = oracle.decode_heads(codes, s, sc, oracle.LAYOUT_VALUE_KEY).transpose(0, 2, 1)
        keys = to_np(slot.compensator_keys).astype(np.float64)
        values = to_np(slot.compensator_values).astype(np.float64)
        want = base + keys @ values.transpose(0, 2, 1)
        assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max()
        assert np.abs(got - provider[0].transpose(0, 2, 1)).max() < 0.05 * np.abs(provider).max()
    finally:
        runtime.close()
