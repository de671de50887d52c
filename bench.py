"""Benchmark of the MI355X GDN state codec hot path.

Headline workload: one step = quantize + dequantize of a
[30 layers, 256 seqs, 32 heads, 128, 128] fp32 GDN state (16.1 GB, layout
[L,B,H,K,V]).  Also measured each run: the decode encoded projection at B=256
(config 3) and the chunked projection 64 x T=64 x 32 heads (config 4), both
rotating over 5 distinct state copies so the 256 MB Infinity Cache cannot hold
the working set.  Kernel durations come from HIP events recorded on the stream
the kernels are launched on (torch's current stream).  The windowed decode
step, its window-boundary refit, the encoded rank-4 chain, the capsule wire
format (serialize / restore), the rank-4 boundary encode of the capsule
factory, the runtime's exact-SVD initializer, config 1 (the 32-head round
trip) and config 5 (the slot-indexed fp32 and bf16 pools) are reported beside
the headline line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-pool]

Prints one JSON line (rank 0).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "gdn-state-codec_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "codec GB/s + % HBM peak; encoded-proj µs/decode step at B=256"
HBM_PEAK_GBPS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0

C2_SHAPE = (30, 256, 32, 128, 128)
C2_TILES = 30 * 256 * 32
C2_ELEMENTS = C2_TILES * 128 * 128
# quantize: fp32 in + int8 codes + fp32 smoothing & scales out; dequantize mirrors it.
C2_BYTES = C2_ELEMENTS * 4 + C2_ELEMENTS + C2_TILES * 2 * 128 * 4  # 20,384,317,440
C3_BYTES = 256 * 32 * 128 * 128 + 2 * 256 * 32 * 128 * 4 + 256 * 16 * 128 * 2 + 256 * 32 * 128 * 4
C4_BYTES = 64 * 32 * 128 * 128 + 2 * 64 * 32 * 128 * 4 + 64 * 64 * 32 * 128 * 2 + 64 * 64 * 32 * 128 * 4
C4_FLOPS = 2 * 64 * 64 * 32 * 128 * 128
ROTATIONS = 5
# Back-to-back timing of the short kernels: warm-up and minimum timed launches
# (the profile pass, which only needs a few launches per kernel, lowers them).
# The warm phase runs about 1.2 s of the leg's own launches: for about a second
# after a heavy leg (the config-2 codec, the HBM probes) the config-4 projection
# ran at 24.9-25.3 us per launch and then settled at 23.2-23.9 us while still
# launching back to back (measured in 100 ms windows); with a 100 ms warm phase
# the bench reported the unsettled figure.
WARM_MS, WARM_LAUNCHES = 1200.0, 60000
TIMED_MS, TIMED_LAUNCHES = 30.0, 1000
PROBE_TILES = 65536
PROBE_TILE_BYTES = PROBE_TILES * (128 * 128 * 4 + 128 * 128)


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _events_ms(pairs) -> list[float]:
    import torch

    torch.cuda.synchronize()
    return [start.elapsed_time(end) for start, end in pairs]


CODEC_CLOCKS: dict = {}  # what _ClockSampler saw during the config-2 timing


def bench_codec(steps: int, warmup: int):
    import torch

    from gdn_state_codec import codec

    dev = torch.device("cuda:0")
    _log(f"config 2: allocating {C2_SHAPE} fp32 state")
    gen = torch.Generator(device=dev)
    gen.manual_seed(20261201)
    state = torch.randn(C2_SHAPE, generator=gen, device=dev, dtype=torch.float32)
    state.mul_(0.05)
    codes = torch.empty(C2_SHAPE, dtype=torch.int8, device=dev)
    smoothing = torch.empty(C2_SHAPE[:-1], dtype=torch.float32, device=dev)
    scales = torch.empty(C2_SHAPE[:-1], dtype=torch.float32, device=dev)
    dense = torch.empty_like(state)
    layout = codec.LAYOUT_KEY_VALUE

    def step():
        codec.encode(state, layout, codes, smoothing, scales)
        codec.decode(codes, smoothing, scales, layout, out=dense)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    enc, dec = [], []
    with _ClockSampler(_device_sysfs()) as sampler:
        t0 = time.perf_counter()
        for _ in range(steps):
            e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
            e0.record()
            codec.encode(state, layout, codes, smoothing, scales)
            e1.record()
            codec.decode(codes, smoothing, scales, layout, out=dense)
            e2.record()
            enc.append((e0, e1))
            dec.append((e1, e2))
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    CODEC_CLOCKS.update(sampler.summary())
    enc_ms = sum(_events_ms(enc)) / steps
    dec_ms = sum(_events_ms(dec)) / steps
    _log(f"config 2: quantize {enc_ms:.3f} ms, dequantize {dec_ms:.3f} ms")
    return state, codes, smoothing, scales, dense, enc_ms, dec_ms, wall * 1e3 / steps


def _probe_library():
    import ctypes

    from gdn_state_codec import _native

    path = _native.library_dir() / "libgdn_state_codec_hbm_probe.so"
    lib = ctypes.CDLL(str(path))
    for name in ("gdn_hbm_probe_copy", "gdn_hbm_probe_read"):
        getattr(lib, name).argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_uint64, ctypes.c_uint32]
        getattr(lib, name).restype = ctypes.c_int32
    lib.gdn_hbm_probe_write.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_uint64, ctypes.c_uint32]
    lib.gdn_hbm_probe_write.restype = ctypes.c_int32
    for name in ("gdn_hbm_probe_expand", "gdn_hbm_probe_contract", "gdn_hbm_probe_halve"):
        getattr(lib, name).argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_uint64, ctypes.c_uint32]
        getattr(lib, name).restype = ctypes.c_int32
    lib.gdn_hbm_probe_grid.restype = ctypes.c_uint32
    lib.gdn_valu_probe.argtypes = [ctypes.c_void_p] * 2 + [ctypes.c_uint32] * 3
    lib.gdn_valu_probe.restype = ctypes.c_int32
    return lib


def bench_valu_probe(repeats: int = 5):
    """VALU issue ceiling of this GPU in wavefront instructions per second:
    8192 workgroups of 4 wavefronts, each wavefront issuing 16 independent
    operations per round for 2048 rounds (fp32 fma, u32 xor-add, fp64 add), no
    memory traffic.  The figure that VALU-heavy kernels' SQ_INSTS_VALU rates
    are compared with."""
    import torch

    lib = _probe_library()
    dev = torch.device("cuda:0")
    blocks, rounds = 8192, 2048
    sink = torch.empty(blocks * 256, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    instructions = blocks * 4 * 16 * rounds
    out = {}
    for mode, name in ((0, "fma_f32"), (1, "xad_u32"), (2, "add_f64")):
        for _ in range(2):
            assert lib.gdn_valu_probe(stream, sink.data_ptr(), blocks, rounds, mode) == 0
        pairs = []
        for _ in range(repeats):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            assert lib.gdn_valu_probe(stream, sink.data_ptr(), blocks, rounds, mode) == 0
            b.record()
            pairs.append((a, b))
        ms = sorted(_events_ms(pairs))[len(pairs) // 2]
        out[f"{name}_Ginst_per_s"] = instructions / (ms * 1e-3) / 1e9
    del sink
    _log("valu probe: " + ", ".join(f"{k}={v:.0f}" for k, v in out.items()))
    return out


def bench_hbm_probe(repeats: int = 5):
    """Sustained HBM bandwidth of plain streaming kernels (4 GiB buffers), with
    plain accesses and with the nontemporal hint the codec kernels use, each in
    the dispatcher's interleaved order and in the XCD-contiguous order the codec
    kernels use (XCD x streams the x-th eighth of the buffer): copy, read,
    write, and the codec-shaped mixed streams expand (1:4 read:write, a 16 KiB
    byte tile in and a 64 KiB fp32 tile out per workgroup, the dequantize's mix),
    contract (4:1, the quantize's mix) and halve (2:1, a 32 KiB bf16 tile in and
    a 16 KiB byte tile out, the bf16 pool encode's mix)."""
    import torch

    lib = _probe_library()
    dev = torch.device("cuda:0")
    nbytes = 4 << 30
    src = torch.ones(nbytes // 4, dtype=torch.int32, device=dev)
    dst = torch.empty_like(src)
    sink = torch.empty(lib.gdn_hbm_probe_grid() * 256, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    out = {}
    # mode bit 0: nontemporal; bit 1: the XCD-contiguous order of the codec kernels.
    for mode, suffix in ((0, ""), (1, "_nt"), (2, "_xcd"), (3, "_nt_xcd")):
        launches = {
            "copy": (lambda: lib.gdn_hbm_probe_copy(stream, src.data_ptr(), dst.data_ptr(), nbytes,
                                                    mode), 2 * nbytes),
            "read": (lambda: lib.gdn_hbm_probe_read(stream, src.data_ptr(), sink.data_ptr(), nbytes,
                                                    mode), nbytes),
            "write": (lambda: lib.gdn_hbm_probe_write(stream, dst.data_ptr(), nbytes, mode), nbytes),
            # 65,536 tiles: 1 GiB of bytes <-> 4 GiB of fp32.
            "expand": (lambda: lib.gdn_hbm_probe_expand(stream, src.data_ptr(), dst.data_ptr(),
                                                        PROBE_TILES, mode), PROBE_TILE_BYTES),
            "contract": (lambda: lib.gdn_hbm_probe_contract(stream, src.data_ptr(), dst.data_ptr(),
                                                            PROBE_TILES, mode), PROBE_TILE_BYTES),
            # 65,536 tiles: 2 GiB of bf16 -> 1 GiB of bytes (the bf16 pool encode's mix).
            "halve": (lambda: lib.gdn_hbm_probe_halve(stream, src.data_ptr(), dst.data_ptr(),
                                                      PROBE_TILES, mode),
                      PROBE_TILES * (128 * 128 * 2 + 128 * 128)),
        }
        for name, (fn, moved) in launches.items():
            for _ in range(2):
                assert fn() == 0
            pairs = []
            for _ in range(repeats):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                assert fn() == 0
                b.record()
                pairs.append((a, b))
            ms = sorted(_events_ms(pairs))[len(pairs) // 2]
            out[f"{name}{suffix}_GBps"] = moved / (ms * 1e-3) / 1e9
    del src, dst, sink
    _log("hbm probe: " + ", ".join(f"{k}={v:.0f}" for k, v in out.items()))
    return out


def same_size_probe(kind: str, nbytes: int, steps: int) -> dict:
    """The nontemporal probe `kind` ("read" or "copy") over a stream of the
    size a projection step moves, timed like the projection legs: back-to-back
    launches over ROTATIONS buffer copies (so the MALL does not hold them),
    after the same warm phase.  `nbytes` is the total of bytes read and
    written.  It is the ceiling a kernel of that size can reach on this GPU,
    launch ramp and drain included, which the 4 GiB probes do not show."""
    import torch

    lib = _probe_library()
    dev = torch.device("cuda:0")
    each = nbytes // 2 if kind == "copy" else nbytes
    each -= each % 128
    stream = torch.cuda.current_stream().cuda_stream
    grid = lib.gdn_hbm_probe_grid()
    bufs = []
    for _ in range(ROTATIONS):
        src = torch.ones(each // 4, dtype=torch.int32, device=dev)
        dst = torch.empty_like(src) if kind == "copy" else torch.empty(grid * 256, dtype=torch.int32,
                                                                       device=dev)
        bufs.append((src, dst))
    fn = lib.gdn_hbm_probe_copy if kind == "copy" else lib.gdn_hbm_probe_read
    # Nontemporal, in the interleaved (mode 1) and XCD-contiguous (mode 3) orders;
    # the faster one is the ceiling.
    timed = {}
    for mode, order in ((1, "interleaved"), (3, "xcd")):
        calls = [(stream, src.data_ptr(), dst.data_ptr(), each, mode) for src, dst in bufs]
        timed[order] = _time_back_to_back(fn, calls, steps)
    order = min(timed, key=timed.get)
    us = timed[order]
    moved = 2 * each if kind == "copy" else each
    del bufs
    return {"kind": f"{kind}_nt", "order": order, "bytes": moved, "us": us,
            "GBps": moved / (us * 1e-6) / 1e9,
            "us_by_order": {k: round(v, 3) for k, v in timed.items()}}


def _c1_style_state(shape, gen, dev):
    import torch

    x = torch.randn(shape, generator=gen, device=dev, dtype=torch.float32).mul_(0.05)
    mask = torch.rand(shape, generator=gen, device=dev) < 0.001
    signs = torch.where(torch.rand(shape, generator=gen, device=dev) < 0.5, -2.0, 2.0)
    return torch.where(mask, signs, x)


def _time_back_to_back(fn, calls, steps: int) -> float:
    """Microseconds per launch of `fn` over back-to-back launches cycling
    through the argument tuples `calls` (one per rotated state copy), between
    one event pair: the per-step time of a loop issuing one launch after
    another.  The entry point is called with prepared arguments so that the
    host keeps ahead of the GPU (about 4 us of host time per launch, against
    23-25 us per config-3/4 launch).  A warm phase of the same launches first
    brings the GPU to the kernel's own steady state, which a short timed region
    right after an idle host-side phase or another heavy leg would not see: the
    clocks of 25 us kernels keep rising for some 30 ms of continuous launches,
    and the state a heavy leg leaves behind takes about a second to settle.  It
    runs about WARM_MS of launches, at most WARM_LAUNCHES.  The timed region is
    at least `steps` launches per copy and about TIMED_MS, at most
    TIMED_LAUNCHES."""
    import torch

    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(20):
        assert fn(*calls[i % len(calls)]) == 0
    b.record()
    estimate_ms = max(_events_ms([(a, b)])[0] / 20, 1e-3)
    for i in range(min(WARM_LAUNCHES, int(WARM_MS / estimate_ms) + 1)):
        assert fn(*calls[i % len(calls)]) == 0
    n = max(steps * len(calls), min(TIMED_LAUNCHES, int(TIMED_MS / estimate_ms) + 1))
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(n):
        fn(*calls[i % len(calls)])
    b.record()
    return _events_ms([(a, b)])[0] / n * 1e3


def bench_decode_projection(steps: int, warmup: int):
    import torch

    from gdn_state_codec import codec, native

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    sets = []
    for _ in range(ROTATIONS):
        x = _c1_style_state((256, 32, 128, 128), gen, dev)
        c, s, sc = codec.encode(x, codec.LAYOUT_VALUE_KEY)
        q = torch.randn((256, 16, 128), generator=gen, device=dev)
        q = (q / q.norm(dim=-1, keepdim=True)).to(torch.bfloat16)
        out = torch.empty((256, 32, 128), dtype=torch.float32, device=dev)
        sets.append((c, s, sc, q, out))
        del x
    for i in range(warmup * ROTATIONS):  # validated calls: shapes, dtypes, devices
        c, s, sc, q, out = sets[i % ROTATIONS]
        codec.project_decode(c, s, sc, q, 1.0, codec.LAYOUT_VALUE_KEY, out)
    fn = native().encoded_projection_decode_launch_v4
    stream = torch.cuda.current_stream().cuda_stream
    calls = [(stream, c.data_ptr(), s.data_ptr(), sc.data_ptr(), q.data_ptr(), out.data_ptr(),
              256, 32, 16, 1.0, codec.LAYOUT_VALUE_KEY) for c, s, sc, q, out in sets]
    us = _time_back_to_back(fn, calls, steps)
    _log(f"config 3: decode projection {us:.2f} us/step")
    return us, sets[0]


def bench_chunked_projection(steps: int, warmup: int):
    import torch

    from gdn_state_codec import codec, native

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    sets = []
    for _ in range(ROTATIONS):
        x = _c1_style_state((64, 32, 128, 128), gen, dev)
        c, s, sc = codec.encode(x, codec.LAYOUT_VALUE_KEY)
        q = torch.randn((64, 64, 32, 128), generator=gen, device=dev).to(torch.bfloat16)
        out = torch.empty((64, 64, 32, 128), dtype=torch.float32, device=dev)
        sets.append((c, s, sc, q, out))
        del x
    for i in range(warmup * ROTATIONS):  # validated calls: shapes, dtypes, devices
        c, s, sc, q, out = sets[i % ROTATIONS]
        codec.project_chunked(c, s, sc, q, 1.0, codec.LAYOUT_VALUE_KEY, out)
    fn = native().encoded_projection_chunked_launch_v4
    stream = torch.cuda.current_stream().cuda_stream
    calls = [(stream, c.data_ptr(), s.data_ptr(), sc.data_ptr(), q.data_ptr(), out.data_ptr(),
              64, 64, 32, 32, 1.0, codec.LAYOUT_VALUE_KEY) for c, s, sc, q, out in sets]
    us = _time_back_to_back(fn, calls, steps)
    _log(f"config 4: chunked projection {us:.2f} us/step")
    return us, sets[0]


def cpu_baseline_projection(sample, chunked: bool, gpu_us: float, target_seconds: float = 6.0):
    """The reference's own CPU readout (oracle/_ref: ReadWindowState with an
    empty window, state_capsule.cpp:253-306) over the whole config-3 step
    (8,192 heads) or config-4 step (2,048 heads x 64 tokens), on identical
    input bits: the [value][key] codes transposed to the reference's [key][value]
    layout and the bf16 queries widened to fp32 (query scale 1) before timing.
    One thread over the whole step, then every allowed core with the heads
    split contiguously, repeated to about `target_seconds`.  The CPU outputs of
    the first 256 heads and the GPU's are each checked against the exact value:
    the CPU within 2^-15 * sum|terms|, the GPU within 2^-15 (decode) or 2^-14
    (chunked, whose weights are split into two bf16 parts)."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    import torch

    import oracle

    if not oracle.ref_available():
        return None
    codes_d, smoothing_d, scales_d, queries_d, out_d = sample
    torch.cuda.synchronize()
    codes_vk = codes_d.cpu().numpy()
    seqs, heads = codes_vk.shape[:2]
    codes = np.ascontiguousarray(codes_vk.swapaxes(-1, -2)).reshape(-1, 128, 128)
    smoothing = smoothing_d.cpu().numpy().reshape(-1, 128)
    scales = scales_d.cpu().numpy().reshape(-1, 128)
    q_bits = queries_d.view(torch.int16).cpu().numpy().view(np.uint16)
    gpu_out = out_d.cpu().numpy()
    if chunked:  # q [N,T,Hq,128] -> reads [N*H, T, 128]
        group = heads // q_bits.shape[2]
        q = np.repeat(q_bits, group, axis=2).transpose(0, 2, 1, 3)
        reads = oracle.bf16_to_f32(q).reshape(seqs * heads, -1, 128)
        gpu = gpu_out.transpose(0, 2, 1, 3).reshape(seqs * heads, -1, 128)
    else:  # q [B,Hq,128] -> reads [B*H, 1, 128]
        group = heads // q_bits.shape[1]
        reads = oracle.bf16_to_f32(np.repeat(q_bits, group, axis=1)).reshape(-1, 1, 128)
        gpu = gpu_out.reshape(-1, 1, 128)
    reads = np.ascontiguousarray(reads, np.float32)
    total = codes.shape[0]

    def run(lo, hi):
        return oracle.ref_read_boundary_heads(codes[lo:hi], smoothing[lo:hi], scales[lo:hi],
                                              reads[lo:hi])

    t0 = time.perf_counter()
    cpu_out = run(0, total)
    single = time.perf_counter() - t0
    threads = _cpu_threads()
    bounds = np.linspace(0, total, threads + 1).astype(int)
    reps = max(1, int(target_seconds * threads / max(single, 1e-6) / 2))
    reps = min(reps, 50)

    def part(i):
        for _ in range(reps):
            run(bounds[i], bounds[i + 1])

    t0 = time.perf_counter()
    with ThreadPoolExecutor(threads) as pool:
        list(pool.map(part, range(threads)))
    multi = (time.perf_counter() - t0) / reps
    # Parity on the first 256 heads against the oracle's exact value and bound.
    n = min(256, total)
    if chunked:
        idx_q = q_bits.reshape(seqs, q_bits.shape[1], q_bits.shape[2], 128)
        sub = n // heads or 1
        _, exact, bound = oracle.project_chunked(codes_vk[:sub], smoothing_d.cpu().numpy()[:sub],
                                                 scales_d.cpu().numpy()[:sub], idx_q[:sub], 1.0,
                                                 oracle.LAYOUT_VALUE_KEY, threads=threads)
        exact = exact.transpose(0, 2, 1, 3).reshape(sub * heads, -1, 128)
        bound = bound.transpose(0, 2, 1, 3).reshape(sub * heads, -1, 128)
        n = sub * heads
    else:
        sub = n // heads or 1
        _, exact, bound = oracle.project_decode(codes_vk[:sub], smoothing_d.cpu().numpy()[:sub],
                                                scales_d.cpu().numpy()[:sub], q_bits[:sub], 1.0,
                                                oracle.LAYOUT_VALUE_KEY)
        exact, bound = exact.reshape(-1, 1, 128), bound.reshape(-1, 1, 128)
        n = sub * heads
    gpu_tol = 2.0 ** -14 if chunked else 2.0 ** -15  # the two-part bf16 split of the chunked path
    within = bool((np.abs(gpu[:n] - exact) <= gpu_tol * bound + 1e-30).all()
                  and (np.abs(cpu_out[:n] - exact) <= 2.0 ** -15 * bound + 1e-30).all())
    name = "config 4" if chunked else "config 3"
    _log(f"cpu baseline {name} (reference): {single * 1e6:.0f} us/step on 1 thread, "
         f"{multi * 1e6:.0f} us/step on {threads} threads; GPU within bound={within}")
    step = (f"{total} heads x {reads.shape[1]} tokens" if chunked else f"{total} heads")
    return {"value": multi * 1e6, "unit": "us/step", "cores": threads, "kind": "reference",
            "cpu_model": _cpu_model(),
            "sample": f"the whole step ({step}), the reference's ReadWindowState per read, "
                      f"heads split contiguously over {threads} threads, {reps} passes",
            "gpu_speedup": multi * 1e6 / gpu_us,
            "single_thread": {"value": single * 1e6, "unit": "us/step", "cores": 1,
                              "sample": "one pass over the whole step"},
            "gpu_within_fp32_bound_on_first_heads": within}


WINDOW_STATES = 256 * 32  # B = 256 sequences x 32 value heads


def window_step_bytes(position: int, compensated: bool) -> int:
    """Algorithmic HBM bytes of one windowed bf16 step on one state at window
    position p: the int8 boundary with its smoothing and scales, the model
    vectors (a key/query pair is shared by two value heads), p stored records
    read, the new record, output and position written."""
    boundary = 128 * 128 + 2 * 128 * 4
    vectors = (2 * 128 * 2) // 2 + 128 * 2 + 4 + 2     # k,q / 2, values, log decay, beta
    compensators = 2 * 128 * 4 * 2 if compensated else 0
    records = position * (2 * 128 * 2 + 4)             # keys + corrections + gate
    writes = 128 * 2 + 2 * 128 * 2 + 4                 # output, record key + correction, gate
    return boundary + vectors + compensators + records + writes + 4 + 4  # position in/out


def bench_window_step(warmup: int):
    """The windowed decode step at B=256 (8192 states): 5 slot copies, each
    stepped through a whole window (positions 0..15) between one event pair,
    launches interleaved across copies so consecutive launches touch different
    states.  A warm phase of about WARM_MS of whole windows comes first (the
    projections' warm phase), then the mean over about TIMED_MS of windows."""
    import torch

    from gdn_state_codec import codec
    from gdn_state_codec.window import DecodeRuntime, WindowSlot, step_bf16

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(7)
    states = WINDOW_STATES
    slots, inputs = [], []
    for _ in range(ROTATIONS):
        x = _c1_style_state((states, 128, 128), gen, dev)
        slot = WindowSlot.allocate(states, dev)
        codec.encode(x, codec.LAYOUT_VALUE_KEY, slot.residual, slot.smoothing, slot.scales)
        slot.compensator_keys.copy_(torch.randn(slot.compensator_keys.shape, generator=gen,
                                                device=dev) * 0.01)
        slot.compensator_values.copy_(torch.randn(slot.compensator_values.shape, generator=gen,
                                                  device=dev) * 0.01)
        del x
        k = torch.randn((states // 2, 128), generator=gen, device=dev)
        q = torch.randn((states // 2, 128), generator=gen, device=dev)
        inputs.append(dict(
            log_decay=torch.log(0.9 + 0.09 * torch.rand(states, generator=gen, device=dev)),
            beta=(0.2 + 0.6 * torch.rand(states, generator=gen, device=dev)).to(torch.bfloat16),
            keys=(k / k.norm(dim=-1, keepdim=True)).to(torch.bfloat16),
            queries=(q / q.norm(dim=-1, keepdim=True)).to(torch.bfloat16),
            values=(0.5 * torch.randn((states, 128), generator=gen, device=dev)).to(torch.bfloat16)))
        slots.append(slot)
    outs = [torch.empty((states, 128), dtype=torch.bfloat16, device=dev) for _ in range(ROTATIONS)]
    runtime = DecodeRuntime(states)
    kinds = {
        "quant_only": lambda r: step_bf16(slots[r], **inputs[r], out=outs[r], quant_only=True,
                                          validate=False),
        "compensated": lambda r: step_bf16(slots[r], **inputs[r], out=outs[r], validate=False),
        "decode_runtime": lambda r: runtime.step(slots[r], **inputs[r], out=outs[r],
                                                 validate=False),
    }
    results = {}

    def window(run):
        """One whole window (positions 0..15) of every copy between one event
        pair; the positions are reset before it, outside the events."""
        for slot in slots:
            slot.positions.zero_()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for t in range(16):
            for r in range(ROTATIONS):
                run(r)
        b.record()
        return a, b

    for name, run in kinds.items():
        # Warm phase of whole windows, as the projections' (WARM_MS of launches),
        # then the mean of the timed windows (about TIMED_MS of them).
        for _ in range(max(warmup, 1)):
            window(run)
        estimate_ms = _events_ms([window(run)])[0]
        for _ in range(min(3000, WARM_LAUNCHES, int(WARM_MS / max(estimate_ms, 1e-3)) + 1)):
            window(run)
        windows = max(3, min(50, int(TIMED_MS / max(estimate_ms, 1e-3)) + 1))
        pairs = [window(run) for _ in range(windows)]
        launches = 16 * ROTATIONS
        us = sum(_events_ms(pairs)) / (windows * launches) * 1e3
        assert all(bool((slot.positions[:, 0] == 16).all()) for slot in slots)
        compensated = name != "quant_only"
        nbytes = sum(window_step_bytes(p, compensated) for p in range(16)) * states / 16
        results[name] = {"us_per_step": us, "GBps": nbytes / (us * 1e-6) / 1e9,
                         "hbm_frac": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
                         "bytes_per_step": nbytes, "timed_windows": windows}
        _log(f"windowed step {name}: {us:.2f} us/step, {results[name]['GBps']:.0f} GB/s")
    runtime.close()
    results["workload"] = ("windowed bf16 decode step, B=256 x 32 value heads (GQA from 16), "
                           "int8 [value][key] boundary, positions 0..15 averaged")
    results["rotated_state_copies"] = ROTATIONS
    del slots, inputs, outs
    return results


REFIT_POWER_ITERATIONS = 4


def refit_bytes(power: bool) -> int:
    """Algorithmic HBM bytes of one window-boundary refit of one full window:
    the boundary codes, smoothing and scales, the 16 records (gates, fp16 keys
    and corrections) read; the next codes, smoothing, scales and compensators
    and the position written.  The power refit also reads the compensators and
    writes the fitted residual workspace (fp32 [128][128]) and the cleared
    records."""
    read = 128 * 128 + 2 * 128 * 4 + 16 * 4 + 2 * 16 * 128 * 2
    write = 128 * 128 + 2 * 128 * 4 + 2 * 128 * 4 * 2 + 4
    if power:
        read += 2 * 128 * 4 * 2 + 4
        write += 128 * 128 * 4 + 16 * 4 + 2 * 16 * 128 * 2
    return read + write


def bench_refit(steps: int, warmup: int):
    """Window-boundary refit of B=256 x 32 heads (8192 full windows): the
    quant-only refit (keep smoothing, fold the 16 records in, requantize) and
    the rank-4 power-iteration refit, each over 5 rotated slot copies."""
    import torch

    from gdn_state_codec import codec, native
    from gdn_state_codec.window import WindowSlot

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(13)
    states = WINDOW_STATES
    copies = []
    for _ in range(ROTATIONS):
        x = _c1_style_state((states, 128, 128), gen, dev)
        slot = WindowSlot.allocate(states, dev)
        codec.encode(x, codec.LAYOUT_VALUE_KEY, slot.residual, slot.smoothing, slot.scales)
        del x
        for t in (slot.compensator_keys, slot.compensator_values, slot.record_keys,
                  slot.record_corrections):
            t.copy_((torch.randn(t.shape, device=dev, generator=gen) * 0.02).to(torch.float16))
        slot.record_decay.uniform_(0.93, 0.99, generator=gen)
        nxt = WindowSlot.allocate(states, dev)
        # The power refit clears the window it folds; every launch gets the
        # full window back (outside the timed events).
        saved = (slot.record_decay.clone(), slot.record_keys.clone(),
                 slot.record_corrections.clone())
        copies.append((slot, nxt, saved))
    workspace = torch.empty((states, 128, 128), dtype=torch.float32, device=dev)
    lib, stream = native(), torch.cuda.current_stream().cuda_stream

    def refit(r, power):
        slot, nxt, _ = copies[r]
        return lib.window_boundary_launch_v1(
            stream, *slot.pointers(), nxt.residual.data_ptr(), nxt.smoothing.data_ptr(),
            nxt.scales.data_ptr(), nxt.compensator_keys.data_ptr(),
            nxt.compensator_values.data_ptr(), workspace.data_ptr(), states, power)

    def timed(i, power):
        r = i % ROTATIONS
        slot, _, saved = copies[r]
        slot.positions[:, 0] = 16  # a full window (the power refit clears it)
        if power:
            for dst, src in zip((slot.record_decay, slot.record_keys,
                                 slot.record_corrections), saved):
                dst.copy_(src)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        assert refit(r, power) == 0
        b.record()
        return a, b

    results = {}
    for name, power in (("quant_only", 0), ("power", REFIT_POWER_ITERATIONS)):
        # Warm phase: about WARM_MS of refits (at least `warmup` per copy), as
        # the projections and the window step get; then `steps` timed refits.
        first = [timed(i, power) for i in range(max(warmup, 1) * ROTATIONS)]
        estimate_ms = max(sorted(_events_ms(first))[len(first) // 2], 1e-3)
        for i in range(min(10000, WARM_LAUNCHES, int(WARM_MS / estimate_ms) + 1)):
            timed(i, power)
        pairs = [timed(i, power) for i in range(steps)]
        us = sum(_events_ms(pairs)) / len(pairs) * 1e3
        assert all(bool((c[0].positions[:, 0] == 0).all()) for c in copies)
        nbytes = refit_bytes(power > 0) * states
        results[name] = {"us_per_refit": us, "GBps": nbytes / (us * 1e-6) / 1e9,
                         "hbm_frac": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
                         "bytes_per_refit": nbytes}
        _log(f"window refit {name}: {us:.1f} us, {results[name]['GBps']:.0f} GB/s")
    results["workload"] = ("window-boundary refit of B=256 x 32 heads (8192 full windows, "
                           "[value][key] codes)")
    results["power_iterations"] = REFIT_POWER_ITERATIONS
    results["rotated_state_copies"] = ROTATIONS
    del copies, workspace
    return results


def encoded_rank_bytes() -> dict:
    """Algorithmic HBM bytes per state of the device rank-4 chain's finishing
    kernels: finish / commit read column 0 of the int32 projection and the fp16
    input (128 values each), the output-axis scales, the dynamic scale, both
    old and both fitted fp16 bases ([128][4] and [4][128], 1 KiB each), both
    fp16 record sides (4 KiB each) and the 16 gates; finish writes the fp16
    [128][16] output, commit column 0 of the fp32 corrected vector and one rank
    of each fitted basis.  encoded_requantize reads the int8 boundary, smoothing,
    scales, the four bases, the gates and records, and writes the codes,
    smoothing, scales, the transposed bases and the fp32 workspace."""
    operands = 128 * 4 + 128 * 2 + 128 * 4 + 4 + 4 * 1024 + 2 * 4096 + 16 * 4
    return {"finish": operands + 128 * 16 * 2,
            "commit": operands + 128 * 4 + 2 * 128 * 2,
            "requantize": (128 * 128 + 2 * 128 * 4 + 4 * 1024 + 16 * 4 + 2 * 4096)
                          + (128 * 128 + 2 * 128 * 4 + 2 * 1024 + 128 * 128 * 4)}


def bench_encoded_rank(steps: int):
    """The finishing kernels of the reference's device rank-4 chain over an
    encoded boundary at 8192 states (B=256 x 32 heads): finish_encoded_projection
    (4 fitted ranks), commit_encoded_rank (rank 3) and encoded_requantize, each
    timed back to back over rotated operand copies after a warm phase."""
    import torch

    from gdn_state_codec import native

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(17)
    states = WINDOW_STATES

    def f16(*shape, scale=0.05):
        return (torch.randn(shape, generator=gen, device=dev) * scale).to(torch.float16)

    sets = []
    for _ in range(ROTATIONS):
        op = {"projected": torch.randint(-200000, 200000, (states, 128, 16), generator=gen,
                                         device=dev, dtype=torch.int32),
              "dyn": torch.full((states, 8), 1e-3, device=dev),
              "input": f16(states, 128, 16, scale=0.1),
              "smoothing": torch.rand((states, 128), generator=gen, device=dev) + 0.5,
              "scales": torch.rand((states, 128), generator=gen, device=dev) + 0.5,
              "old_left": f16(states, 128, 4), "old_right": f16(states, 128, 4),
              "decay": torch.rand((states, 16), generator=gen, device=dev) * 0.06 + 0.93,
              "record_left": f16(states, 16, 128), "record_right": f16(states, 16, 128),
              "new_left": f16(states, 4, 128), "new_right": f16(states, 4, 128),
              "residual": torch.randint(-127, 128, (states, 128, 128), generator=gen,
                                        device=dev, dtype=torch.int8),
              "output": torch.empty((states, 128, 16), dtype=torch.float16, device=dev),
              "corrected": torch.empty((states, 128, 16), device=dev)}
        sets.append(op)
    nxt = {"residual": torch.empty((states, 128, 128), dtype=torch.int8, device=dev),
           "smoothing": torch.empty((states, 128), device=dev),
           "scales": torch.empty((states, 128), device=dev),
           "left": torch.empty((states, 128, 4), dtype=torch.float16, device=dev),
           "right": torch.empty((states, 128, 4), dtype=torch.float16, device=dev),
           "workspace": torch.empty((states, 128, 128), device=dev)}
    lib, stream = native(), torch.cuda.current_stream().cuda_stream

    def operands(op):
        return [op[k].data_ptr() for k in ("smoothing", "scales", "old_left", "old_right",
                                           "decay", "record_left", "record_right")]

    finish = [(stream, op["projected"].data_ptr(), op["dyn"].data_ptr(), op["input"].data_ptr(),
               *operands(op), op["new_left"].data_ptr(), op["new_right"].data_ptr(),
               op["output"].data_ptr(), states, 4, 0) for op in sets]
    commit = [(stream, op["projected"].data_ptr(), op["dyn"].data_ptr(), op["input"].data_ptr(),
               *operands(op), op["new_left"].data_ptr(), op["new_right"].data_ptr(),
               op["corrected"].data_ptr(), states, 3) for op in sets]
    requantize = [(stream, op["residual"].data_ptr(), *operands(op), op["new_left"].data_ptr(),
                   op["new_right"].data_ptr(), *(nxt[k].data_ptr() for k in nxt), states)
                  for op in sets]
    per_state = encoded_rank_bytes()
    results = {}
    for name, fn, calls in (
            ("finish", lib.finish_encoded_projection_launch_v1, finish),
            ("commit", lib.commit_encoded_rank_launch_v1, commit),
            ("requantize", lib.encoded_requantize_launch_v1, requantize)):
        us = _time_back_to_back(fn, calls, steps)
        nbytes = per_state[name] * states
        results[name] = {"us_per_launch": us, "GBps": nbytes / (us * 1e-6) / 1e9,
                         "hbm_frac": nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
                         "bytes_per_launch": nbytes}
        _log(f"encoded rank chain {name}: {us:.1f} us, {results[name]['GBps']:.0f} GB/s")
    results["workload"] = ("device rank-4 chain over an encoded boundary, 8192 states: "
                           "finish (4 fitted ranks), commit (rank 3), requantize")
    results["rotated_state_copies"] = ROTATIONS
    del sets, nxt
    return results


GATE_WINDOW = 16
GATE_PROBE_STATES = 32            # encoded_projection_probe.cpp:20 (kStates)
GATE_CHAIN_ITERATIONS = 8         # encoded_projection_probe.cpp:465 (kPowerIterations)
GATE_REPETITIONS = 11             # encoded_projection_probe.cpp:940-987


def bench_compression_gate():
    """The reference's own speed gate, "compressed cycle faster than fp32"
    (encoded_projection_probe.cpp:905-999, windowed_gdn_runtime_probe.cpp:
    352-388), at B = 256 x 32 heads over rotated copies and at the probe's own
    32 states."""
    results = {"b256": _compression_gate(WINDOW_STATES, ROTATIONS),
               "probe_shape": _compression_gate(GATE_PROBE_STATES, 1)}
    results["workload"] = (
        "one window cycle per slot: 16 windowed decode steps then the boundary "
        "update, against 16 dense fp32 GDN steps (fp32_gdn_step_launch_v1) on the same "
        "model vectors; median of 11 repetitions alternating compressed and fp32 as the "
        "reference's probe does, each timed between HIP events on the launch stream")
    return results


def _compression_gate(states: int, copies: int) -> dict:
    """Cycles at `states` states per slot over `copies` rotated slot copies
    (launches interleaved across copies, step t of every copy before step t+1,
    so consecutive launches touch different states and the 256 MB MALL cannot
    hold a slot between its steps).  Compressed cycles:

    * quant_only: 16 bf16 quant-only steps, then the quant-only refit
      (window_boundary_launch_v1, power 0);
    * power: 16 compensated bf16 steps, then the rank-4 power refit at
      REFIT_POWER_ITERATIONS iterations;
    * encoded_chain: the probe's cycle, 16 fp16 windowed steps
      (windowed_gdn_step_launch_v1), the device rank chain (per rank: the seed
      copied in, GATE_CHAIN_ITERATIONS x (prepare_int8_vector -> int8 product ->
      finish_encoded_projection) forward and transposed, then prepare -> product ->
      commit_encoded_rank), then encoded_requantize.  The product is
      int8_cube_matmul_launch_v1 at the probe's 32 states and the batched
      int8_matmul_launch_v4 at B = 256;
    * encoded_chain_fused: the same cycle with the rank chain as one launch of
      encoded_rank_chain_launch_v4 per slot (bit-identical bases).

    Positions, fitted bases and nothing else are reset outside the timed
    region, as the probe's restore_cycle / reset_bases do."""
    import torch

    from gdn_state_codec import codec, native
    from gdn_state_codec.window import WindowSlot

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(19 + states)
    lib, stream = native(), torch.cuda.current_stream().cuda_stream

    def unit(shape, scale):
        v = torch.randn(shape, generator=gen, device=dev)
        return v / v.norm(dim=-1, keepdim=True) * scale

    slots, nxt, bf16_in, f16_in, dense, bases = [], [], [], [], [], []
    for _ in range(copies):
        x = _c1_style_state((states, 128, 128), gen, dev)
        slot = WindowSlot.allocate(states, dev)
        codec.encode(x, codec.LAYOUT_VALUE_KEY, slot.residual, slot.smoothing, slot.scales)
        for t in (slot.compensator_keys, slot.compensator_values):
            t.copy_(torch.randn(t.shape, generator=gen, device=dev) * 0.01)
        slots.append(slot)
        nxt.append(WindowSlot.allocate(states, dev))
        dense.append(x)
        log_decay = torch.log(0.9 + 0.09 * torch.rand(states, generator=gen, device=dev))
        bf16_in.append([log_decay,
                        (0.2 + 0.6 * torch.rand(states, generator=gen, device=dev)
                         ).to(torch.bfloat16),
                        unit((states // 2, 128), 1.0).to(torch.bfloat16),
                        unit((states // 2, 128), 1.0).to(torch.bfloat16),
                        (0.5 * torch.randn((states, 128), generator=gen, device=dev)
                         ).to(torch.bfloat16)])
        f16_in.append([torch.exp(log_decay),
                       unit((states, 128), 0.25).to(torch.float16),
                       unit((states, 128), 1.0).to(torch.float16),
                       unit((states, 128), 1.0).to(torch.float16),
                       (0.5 * torch.randn((states, 128), generator=gen, device=dev)
                        ).to(torch.float16)])
        bases.append((torch.zeros((states, 4, 128), dtype=torch.float16, device=dev),
                      torch.zeros((states, 4, 128), dtype=torch.float16, device=dev)))
    out_bf16 = torch.empty((states, 128), dtype=torch.bfloat16, device=dev)
    out_f32 = torch.empty((states, 128), dtype=torch.float32, device=dev)
    workspace = torch.empty((states, 128, 128), dtype=torch.float32, device=dev)
    seeds = torch.zeros((4, states, 128, 16), dtype=torch.float16, device=dev)
    seeds[..., 0] = torch.randn((4, states, 128), generator=gen, device=dev).to(torch.float16)
    vector = torch.empty((states, 128, 16), dtype=torch.float16, device=dev)
    output = torch.empty_like(vector)
    quantized = torch.empty((states, 128, 16), dtype=torch.int8, device=dev)
    dyn = torch.empty((states, 8), dtype=torch.float32, device=dev)
    projected = torch.empty((states, 128, 16), dtype=torch.int32, device=dev)
    corrected = torch.empty((states, 128, 16), dtype=torch.float32, device=dev)
    req = [torch.empty((states, 128, 128), dtype=torch.int8, device=dev),
           torch.empty((states, 128), device=dev), torch.empty((states, 128), device=dev),
           torch.empty((states, 128, 4), dtype=torch.float16, device=dev),
           torch.empty((states, 128, 4), dtype=torch.float16, device=dev), workspace]
    scratch = torch.zeros(16, dtype=torch.int32, device=dev)
    bf16_ptr = [[t.data_ptr() for t in args] for args in bf16_in]
    f16_ptr = [[t.data_ptr() for t in args] for args in f16_in]

    def ok(status):
        if status != 0:
            raise RuntimeError(f"compression gate launch failed: {status}")

    def operands(r):
        s = slots[r]
        return [s.smoothing.data_ptr(), s.scales.data_ptr(), s.compensator_keys.data_ptr(),
                s.compensator_values.data_ptr(), s.record_decay.data_ptr(),
                s.record_keys.data_ptr(), s.record_corrections.data_ptr()]

    def product(r, vec, transpose):
        s = slots[r]
        axis = s.smoothing if transpose else s.scales
        ok(lib.prepare_int8_vector_launch_v1(stream, vec.data_ptr(), axis.data_ptr(),
                                             quantized.data_ptr(), dyn.data_ptr(), states))
        if states <= 128:
            ok(lib.int8_cube_matmul_launch_v1(
                stream, s.residual.data_ptr(), quantized.data_ptr(), projected.data_ptr(),
                states, transpose, scratch.data_ptr(), scratch.data_ptr(), (states + 1) // 2))
        else:
            ok(lib.int8_matmul_launch_v4(stream, s.residual.data_ptr(), quantized.data_ptr(),
                                         projected.data_ptr(), states, transpose))

    def rank_chain(r):
        left, right = bases[r]
        for rank in range(4):
            vector.copy_(seeds[rank])
            for _ in range(GATE_CHAIN_ITERATIONS):
                for src, dst, transpose in ((vector, output, 0), (output, vector, 1)):
                    product(r, src, transpose)
                    ok(lib.finish_encoded_projection_launch_v1(
                        stream, projected.data_ptr(), dyn.data_ptr(), src.data_ptr(),
                        *operands(r), left.data_ptr(), right.data_ptr(), dst.data_ptr(),
                        states, rank, transpose))
            product(r, vector, 0)
            ok(lib.commit_encoded_rank_launch_v1(
                stream, projected.data_ptr(), dyn.data_ptr(), vector.data_ptr(), *operands(r),
                left.data_ptr(), right.data_ptr(), corrected.data_ptr(), states, rank))
        ok(lib.encoded_requantize_launch_v1(
            stream, slots[r].residual.data_ptr(), *operands(r), left.data_ptr(),
            right.data_ptr(), *(t.data_ptr() for t in req), states))

    compact_seeds = seeds[..., 0].permute(1, 0, 2).contiguous()  # [S][4][128]
    fused_corrected = torch.empty((states, 4, 128), dtype=torch.float32, device=dev)

    def fused_chain(r):
        left, right = bases[r]
        s = slots[r]
        ok(lib.encoded_rank_chain_launch_v4(
            stream, s.residual.data_ptr(), *operands(r), compact_seeds.data_ptr(),
            left.data_ptr(), right.data_ptr(), fused_corrected.data_ptr(), states,
            GATE_CHAIN_ITERATIONS))
        ok(lib.encoded_requantize_launch_v1(
            stream, s.residual.data_ptr(), *operands(r), left.data_ptr(),
            right.data_ptr(), *(t.data_ptr() for t in req), states))

    def refit(r, power):
        n = nxt[r]
        ok(lib.window_boundary_launch_v1(
            stream, *slots[r].pointers(), n.residual.data_ptr(), n.smoothing.data_ptr(),
            n.scales.data_ptr(), n.compensator_keys.data_ptr(), n.compensator_values.data_ptr(),
            workspace.data_ptr(), states, power))

    def windowed(kind):
        fn = {"quant_only": lib.windowed_gdn_step_bf16_quant_only_launch_v1,
              "power": lib.windowed_gdn_step_bf16_launch_v1}.get(kind)
        for _ in range(GATE_WINDOW):
            for r in range(copies):
                if fn is None:
                    ok(lib.windowed_gdn_step_launch_v1(stream, *slots[r].pointers(), *f16_ptr[r],
                                                       out_f32.data_ptr(), states))
                else:
                    ok(fn(stream, *slots[r].pointers(), *bf16_ptr[r], out_bf16.data_ptr(),
                          states))
        for r in range(copies):
            if kind == "quant_only":
                refit(r, 0)
            elif kind == "power":
                refit(r, REFIT_POWER_ITERATIONS)
            elif kind == "encoded_chain_fused":
                fused_chain(r)
            else:
                rank_chain(r)

    def fp32_cycle(_kind):
        for _ in range(GATE_WINDOW):
            for r in range(copies):
                ok(lib.fp32_gdn_step_launch_v1(stream, dense[r].data_ptr(), *f16_ptr[r],
                                               out_f32.data_ptr(), states))

    def restore(kind):
        for r in range(copies):
            slots[r].positions.zero_()
            if kind.startswith("encoded_chain"):
                for b in bases[r]:
                    b.zero_()

    def timed(cycle, kind):
        restore(kind)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        a.record()
        cycle(kind)
        b.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        return a.elapsed_time(b) * 1e3 / copies, wall * 1e6 / copies

    kinds = ("quant_only", "power", "encoded_chain", "encoded_chain_fused")
    # Warm phase: whole cycles of every kind until about WARM_MS has run.
    t0 = time.perf_counter()
    while True:
        for kind in kinds:
            timed(windowed, kind)
        timed(fp32_cycle, "fp32")
        if (time.perf_counter() - t0) * 1e3 >= WARM_MS:
            break
    samples = {kind: [] for kind in (*kinds, "fp32")}
    for rep in range(GATE_REPETITIONS):
        order = [*kinds, "fp32"] if rep % 2 == 0 else ["fp32", *kinds]
        for kind in order:
            samples[kind].append(timed(fp32_cycle if kind == "fp32" else windowed, kind))

    def median(values):
        return sorted(values)[len(values) // 2]

    fp32_us = median([s[0] for s in samples["fp32"]])
    result = {"states": states, "rotated_state_copies": copies,
              "fp32_us_per_cycle": fp32_us,
              "fp32_wall_us_per_cycle": median([s[1] for s in samples["fp32"]])}
    for kind in kinds:
        us = median([s[0] for s in samples[kind]])
        result[kind] = {"us_per_cycle": us,
                        "wall_us_per_cycle": median([s[1] for s in samples[kind]]),
                        "speedup_vs_fp32": fp32_us / us,
                        "compressed_faster_than_fp32": bool(us < fp32_us)}
        _log(f"compression gate {states} states, {kind}: {us:.1f} us per cycle against "
             f"{fp32_us:.1f} us fp32 ({fp32_us / us:.2f}x)")
    result["power_refit_iterations"] = REFIT_POWER_ITERATIONS
    result["chain_power_iterations"] = GATE_CHAIN_ITERATIONS
    result["chain_product"] = ("int8_cube_matmul_launch_v1" if states <= 128
                               else "int8_matmul_launch_v4")

    # The windowed runtime probe's single step (windowed_gdn_runtime_probe.cpp:
    # 282-305, 352-370): one fp16 windowed step at position 7 against one fp32
    # step, median of 11 alternating.
    step = {"windowed": [], "fp32": []}
    for rep in range(GATE_REPETITIONS):
        for kind in (("windowed", "fp32") if rep % 2 == 0 else ("fp32", "windowed")):
            for slot in slots:
                slot.positions[:, 0] = 7
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for r in range(copies):
                if kind == "windowed":
                    ok(lib.windowed_gdn_step_launch_v1(stream, *slots[r].pointers(),
                                                       *f16_ptr[r], out_f32.data_ptr(), states))
                else:
                    ok(lib.fp32_gdn_step_launch_v1(stream, dense[r].data_ptr(), *f16_ptr[r],
                                                   out_f32.data_ptr(), states))
            b.record()
            step[kind].append(_events_ms([(a, b)])[0] * 1e3 / copies)
    result["single_step_position_7"] = {
        "windowed_median_us": median(step["windowed"]), "fp32_median_us": median(step["fp32"])}
    del slots, nxt, dense, workspace, req
    torch.cuda.empty_cache()
    return result


def bench_config1(steps: int, cpu: bool):
    """Config 1, the reference's CPU-runnable case: quantize + dequantize of 32
    C1-style [key][value] heads (2 MiB in).  The GPU round trip is timed back to
    back; the CPU baseline is the reference's own C++ (oracle/_ref; the C
    restatement where _ref is absent) on the same 32 heads, 3 warm-ups then the
    median of 11 repetitions, on one thread and with the heads split over the
    host's cores, and the GPU's codes are checked against it bit for bit."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    import torch

    import oracle
    from gdn_state_codec import native

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(31)
    heads = 32
    state = _c1_style_state((heads, 128, 128), gen, dev)
    codes = torch.empty(state.shape, dtype=torch.int8, device=dev)
    smoothing = torch.empty((heads, 128), device=dev)
    scales = torch.empty((heads, 128), device=dev)
    dense = torch.empty_like(state)
    lib, stream = native(), torch.cuda.current_stream().cuda_stream

    def round_trip_gpu():
        status = lib.encode_launch_v4(stream, state.data_ptr(), codes.data_ptr(),
                                      smoothing.data_ptr(), scales.data_ptr(), heads, 0)
        return status or lib.decode_launch_v4(stream, codes.data_ptr(), smoothing.data_ptr(),
                                              scales.data_ptr(), None, None, dense.data_ptr(),
                                              heads, 0)

    us = _time_back_to_back(lambda: round_trip_gpu(), [()], steps)
    nbytes = 2 * heads * (128 * 128 * 5 + 2 * 128 * 4)
    error = (dense.double() - state.double())
    mse = float(error.square().mean())
    results = {"workload": "config 1: quantize + dequantize of 32 C1-style [key][value] heads",
               "us_per_round_trip": us, "GBps": nbytes / (us * 1e-6) / 1e9,
               "bytes_per_round_trip": nbytes, "mse": mse,
               "relative_rms": (mse / float(state.double().square().mean())) ** 0.5}
    _log(f"config 1: {heads} heads round trip in {us:.1f} us, mse {mse:.3e}")
    if not cpu:
        return results
    kind = "reference" if oracle.ref_available() else "port"
    x = state.cpu().numpy()

    def round_trip_cpu(part):
        if kind == "reference":
            c, s, sc = oracle.ref_quantize_heads(part)
            oracle.ref_dequantize_heads(c, s, sc)
        else:
            c, s, sc = oracle.encode_heads(part, oracle.LAYOUT_KEY_VALUE, threads=1)
            oracle.decode_heads(c, s, sc, oracle.LAYOUT_KEY_VALUE, threads=1)
        return c

    def median_seconds(fn):
        for _ in range(3):
            fn()
        times = []
        for _ in range(11):
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
        return float(np.median(times))

    single = median_seconds(lambda: round_trip_cpu(x))
    threads = _cpu_threads()
    bounds = np.linspace(0, heads, threads + 1).astype(int)
    pool = ThreadPoolExecutor(threads)
    multi = median_seconds(lambda: list(pool.map(
        round_trip_cpu, [x[lo:hi] for lo, hi in zip(bounds, bounds[1:]) if hi > lo])))
    pool.shutdown()
    torch.cuda.synchronize()
    exact = codes.cpu().numpy().tobytes() == round_trip_cpu(x).tobytes()
    results["cpu_baseline"] = {
        "value": multi * 1e6, "unit": "us per round trip", "cores": threads, "kind": kind,
        "cpu_model": _cpu_model(), "sample": "the same 32 heads, median of 11 after 3 warm-ups",
        "single_thread": {"value": single * 1e6, "unit": "us per round trip", "cores": 1},
        "gpu_codes_bit_exact": bool(exact)}
    _log(f"cpu config 1 ({kind}): {single * 1e6:.0f} us on 1 thread, {multi * 1e6:.0f} us on "
         f"{threads} threads; GPU codes bit-exact={exact}")
    return results


def bench_boundary_fit(steps: int, cpu: bool):
    """The capsule path's boundary encode with the rank-4 compensator fit
    (quantize_boundary_launch_v1: FromDenseBoundary -> QuantizeBoundary,
    state_capsule.cpp:129-226) on C1-style heads: 32 heads (config 1's size,
    one round of workgroups) and 8,192 heads (a B=256 x 32-head layer), timed
    back to back.  Its time is the fit's sequential chains (norms, the singular
    value's 16,384-term sum), not HBM.  The CPU baseline runs the reference's
    own QuantizeBoundary (oracle/_ref; the C restatement where _ref is absent)
    over a bounded sample of the same heads, on one thread and on the host's
    cores, and checks the GPU's codes and compensators on it bit for bit."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    import torch

    import oracle
    from gdn_state_codec import native

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(29)
    heads = WINDOW_STATES
    dense = _c1_style_state((heads, 128, 128), gen, dev)
    out = {"residual": torch.empty_like(dense),
           "codes": torch.empty((heads, 128, 128), dtype=torch.int8, device=dev),
           "smoothing": torch.empty((heads, 128), device=dev),
           "scales": torch.empty((heads, 128), device=dev),
           "keys": torch.empty((heads, 128, 4), device=dev),
           "values": torch.empty((heads, 128, 4), device=dev),
           "status": torch.empty((heads,), dtype=torch.int32, device=dev)}
    lib, stream = native(), torch.cuda.current_stream().cuda_stream
    fn = lib.quantize_boundary_launch_v1

    def call(n):
        return (stream, dense.data_ptr(), *(out[k].data_ptr() for k in out), n, 4)

    results = {"workload": "rank-4 boundary encode (fit + quant stage) of C1-style "
                           "[key][value] heads", "rank": 4}
    for n in (32, heads):
        us = _time_back_to_back(fn, [call(n)], max(steps // 4, 2))
        results[f"heads_{n}"] = {"ms_per_batch": us / 1e3, "heads_per_s": n / (us * 1e-6)}
        _log(f"boundary fit: {n} heads in {us / 1e3:.3f} ms ({n / (us * 1e-6):.0f} heads/s)")
    torch.cuda.synchronize()
    assert int(out["status"].abs().sum()) == 0
    if not cpu:
        return results
    kind = "reference" if oracle.ref_available() else "port"
    fit = oracle.ref_quantize_kv if kind == "reference" else oracle.quantize_kv
    x = dense.cpu().numpy()

    def run(indices):
        return [fit(x[i], rank=4) if kind == "reference" else fit(x[i], 4) for i in indices]

    t0 = time.perf_counter()
    run(range(8))
    probe = (time.perf_counter() - t0) / 8
    n = int(min(heads, max(8, 6.0 / max(probe, 1e-6))))
    t0 = time.perf_counter()
    single = run(range(n))
    single_s = time.perf_counter() - t0
    names = ("codes", "smoothing", "scales", "keys", "values")
    gpu = {k: out[k][:n].cpu().numpy() for k in names}
    exact = all(gpu[k][i].tobytes() == np.ascontiguousarray(single[i][j]).tobytes()
                for i in range(n) for j, k in enumerate(names))
    threads = _cpu_threads()
    m = int(min(heads, n * threads))
    bounds = np.linspace(0, m, threads + 1).astype(int)
    t0 = time.perf_counter()
    with ThreadPoolExecutor(threads) as pool:
        list(pool.map(run, [range(lo, hi) for lo, hi in zip(bounds, bounds[1:])]))
    multi_s = time.perf_counter() - t0
    results["cpu_baseline"] = {
        "value": m / multi_s, "unit": "heads/s", "cores": threads, "kind": kind,
        "cpu_model": _cpu_model(), "seconds": multi_s,
        "sample": f"the first {m} of the 8192 heads, split contiguously over {threads} threads",
        "single_thread": {"value": n / single_s, "unit": "heads/s", "cores": 1,
                          "sample": f"the first {n} heads", "seconds": single_s},
        "gpu_bit_exact_on_sample": bool(exact)}
    _log(f"cpu boundary fit ({kind}): {n / single_s:.1f} heads/s on 1 thread, "
         f"{m / multi_s:.1f} heads/s on {threads} threads; GPU bit-exact={exact}")
    return results


def bench_exact_svd(steps: int, cpu: bool):
    """The runtime's exact-SVD boundary initializer
    (exact_svd_boundary_launch_v1; runtime.py:335-389) on C1-style provider
    heads: 32 heads (one layer slot) and 8,192, timed back to back.  The Jacobi
    sweeps are a chain of 127 rounds per sweep behind one barrier each, so the
    time is the chain, not HBM.  The CPU baseline is the reference's own call,
    torch.linalg.svd in fp32 on the host, over the 32-head slot plus the
    residual and the quant stage (the oracle's encode), on the host's cores;
    the GPU's rank-4 product is checked against the float64 SVD on it."""
    import numpy as np
    import torch

    import oracle
    from gdn_state_codec import native
    from oracle import svd as S

    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(31)
    heads = WINDOW_STATES
    provider = _c1_style_state((heads, 128, 128), gen, dev)
    out = {"residual": torch.empty_like(provider),
           "codes": torch.empty((heads, 128, 128), dtype=torch.int8, device=dev),
           "smoothing": torch.empty((heads, 128), device=dev),
           "scales": torch.empty((heads, 128), device=dev),
           "keys": torch.empty((heads, 128, 4), dtype=torch.float16, device=dev),
           "values": torch.empty((heads, 128, 4), dtype=torch.float16, device=dev),
           "status": torch.empty((heads,), dtype=torch.int32, device=dev)}
    lib, stream = native(), torch.cuda.current_stream().cuda_stream
    fn = lib.exact_svd_boundary_launch_v1

    def call(n):
        return (stream, provider.data_ptr(), *(out[k].data_ptr() for k in out), n)

    results = {"workload": "exact-SVD initializer (rank-4 truncated SVD by Jacobi + quant "
                           "stage) of C1-style provider heads"}
    for n in (32, heads):
        us = _time_back_to_back(fn, [call(n)], max(steps // 4, 2))
        results[f"heads_{n}"] = {"ms_per_batch": us / 1e3, "heads_per_s": n / (us * 1e-6)}
        _log(f"exact SVD: {n} heads in {us / 1e3:.3f} ms ({n / (us * 1e-6):.0f} heads/s)")
    torch.cuda.synchronize()
    assert int(out["status"].abs().sum()) == 0
    sample = 32
    x = provider[:sample].cpu().numpy()
    residual = out["residual"][:sample].cpu().numpy()
    top = np.empty(sample)
    error = np.empty(sample)
    for h in range(sample):
        _, _, singular, product = S.svd_fit(x[h].T)
        fit = (x[h].astype(np.float64) - residual[h]).T
        top[h] = singular[0]
        error[h] = np.abs(fit - product).max() / singular[0]
    results["rank4_product_error_vs_float64_svd"] = {
        "max_over_top_singular_value": float(error.max()), "heads_checked": sample}
    if not cpu:
        return results
    threads = _cpu_threads()
    torch.set_num_threads(threads)
    dense = torch.from_numpy(x).transpose(-2, -1).contiguous()

    def reference_path():
        u, s, vt = torch.linalg.svd(dense, full_matrices=False)
        left = u[:, :, :4] * s[:, None, :4]
        right = vt[:, :4, :].transpose(-2, -1)
        fitted = dense - torch.bmm(left, right.transpose(-2, -1))
        oracle.encode_heads(fitted.transpose(-2, -1).contiguous().numpy(),
                            oracle.LAYOUT_VALUE_KEY, threads=threads)

    reference_path()
    repeats = 0
    t0 = time.perf_counter()
    while repeats < 3 or (time.perf_counter() - t0 < 5.0 and repeats < 200):
        reference_path()
        repeats += 1
    seconds = (time.perf_counter() - t0) / repeats
    results["cpu_baseline"] = {
        "value": sample / seconds, "unit": "heads/s", "cores": threads, "kind": "port",
        "cpu_model": _cpu_model(), "seconds_per_batch": seconds,
        "sample": f"the first {sample} heads (one slot): fp32 torch.linalg.svd, the fitted "
                  f"residual and the quant stage, {repeats} repeats"}
    _log(f"cpu exact SVD ({threads} threads): {sample / seconds:.1f} heads/s, "
         f"{seconds * 1e3:.2f} ms per {sample}-head slot; GPU rank-4 product within "
         f"{error.max():.2e} of the float64 SVD")
    return results


CAPSULE_GEOMETRY = "0123456789abcdef" * 4
SHA_BLOCKS_PER_CAPSULE = lambda p: (21624 + 1536 * p + 9 + 63) // 64  # noqa: E731


def capsule_slot(states: int, dev, seed: int = 11):
    """A window slot of `states` random states; the 32 heads of a sequence
    share one window position, sequences cycle through positions 0..15."""
    import torch

    from gdn_state_codec.window import WindowSlot

    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    slot = WindowSlot.allocate(states, dev)
    slot.residual.copy_(torch.randint(-127, 128, slot.residual.shape, device=dev, generator=gen,
                                      dtype=torch.int8))
    for t in (slot.smoothing, slot.scales, slot.record_decay):
        t.uniform_(0.5, 1.5, generator=gen)
    for t in (slot.compensator_keys, slot.compensator_values, slot.record_keys,
              slot.record_corrections):
        t.copy_((torch.randn(t.shape, device=dev, generator=gen) * 0.05).to(torch.float16))
    slot.positions[:, 0] = (torch.arange(states, device=dev, dtype=torch.int32) // 32) % 16
    return slot


def bench_capsule(steps: int, warmup: int):
    """Capsule wire format at B=256 (8192 states): serialize (pack + SHA-256)
    and restore (SHA-256 verify + validate/unpack) of a whole slot batch."""
    import torch

    from gdn_state_codec import capsule as cap
    from gdn_state_codec import native
    from gdn_state_codec.window import WindowSlot

    dev = torch.device("cuda:0")
    states = WINDOW_STATES
    slot = capsule_slot(states, dev)
    fresh = WindowSlot.allocate(states, dev)
    identity = cap.CapsuleIdentity(CAPSULE_GEOMETRY, 1, 1)
    capsules, offsets, lengths = cap.serialize(slot, identity)
    expected = slot.positions[:, 0].contiguous()
    status = cap.restore(fresh, capsules, offsets, lengths, identity, expected)
    torch.cuda.synchronize()
    assert bool((status == 0).all()) and bool((lengths > 0).all())
    lib, stream = native(), torch.cuda.current_stream().cuda_stream
    geometry = identity.geometry_bytes

    def serialize():
        return lib.capsule_serialize_launch_v1(
            stream, *slot.pointers(), 1, geometry, 1, 1, capsules.data_ptr(), offsets.data_ptr(),
            capsules.numel(), lengths.data_ptr(), states)

    def restore():
        return lib.capsule_restore_launch_v1(
            stream, capsules.data_ptr(), offsets.data_ptr(), lengths.data_ptr(), capsules.numel(),
            geometry, 1, 1, expected.data_ptr(), 1, *fresh.pointers(), status.data_ptr(), states)

    results = {}
    capsule_bytes = int(lengths.sum().item())
    positions = expected.cpu().tolist()
    blocks = sum(SHA_BLOCKS_PER_CAPSULE(p) for p in positions)
    for name, run in (("serialize", serialize), ("restore", restore)):
        for _ in range(max(warmup, 1)):
            assert run() == 0
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            run()
        b.record()
        us = _events_ms([(a, b)])[0] / steps * 1e3
        results[name] = {"us_per_batch": us, "capsules_per_s": states / (us * 1e-6),
                         "capsule_GBps": capsule_bytes / (us * 1e-6) / 1e9,
                         "sha256_blocks_per_s": blocks / (us * 1e-6)}
        _log(f"capsule {name}: {us:.1f} us for {states} capsules "
             f"({results[name]['capsule_GBps']:.0f} GB/s of capsule bytes)")
    assert bool((status == 0).all())
    # SHA-256 is one serial chain per capsule, so the serialize time is the
    # chain of the longest capsule (window position 15) whatever the number of
    # capsules: the same serialize on an eighth of the batch (every window
    # position still present) takes nearly as long.  The floor of one chain is
    # its VALU instructions (905 per 64-byte block on the consumer wavefront
    # in this build: 6 v_alignbit, 4 v_bitop3 and about 4 adds per round) at
    # one instruction per 4 cycles at the 2.4 GHz peak engine clock.
    small = states // 8
    small_slot = capsule_slot(small, dev)
    small_caps, small_offsets, small_lengths = cap.serialize(small_slot, identity)

    def serialize_small():
        return lib.capsule_serialize_launch_v1(
            stream, *small_slot.pointers(), 1, geometry, 1, 1, small_caps.data_ptr(),
            small_offsets.data_ptr(), small_caps.numel(), small_lengths.data_ptr(), small)

    for _ in range(max(warmup, 1)):
        assert serialize_small() == 0
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        serialize_small()
    b.record()
    longest = SHA_BLOCKS_PER_CAPSULE(15)
    results["serialize_eighth_batch"] = {"capsules": small,
                                         "us_per_batch": _events_ms([(a, b)])[0] / steps * 1e3}
    results["longest_capsule_sha256_blocks"] = longest
    results["chain_issue_floor_us"] = longest * 905 * 4 / 2.4e3
    results["serialize_frac_of_chain_floor"] = (results["chain_issue_floor_us"]
                                                / results["serialize"]["us_per_batch"])
    _log(f"capsule serialize of {small} capsules: "
         f"{results['serialize_eighth_batch']['us_per_batch']:.1f} us; chain floor "
         f"{results['chain_issue_floor_us']:.1f} us")
    del small_slot, small_caps
    results["workload"] = ("LQCAPS01 serialize / restore of B=256 x 32 heads (8192 window "
                           "states), sequence s at window position s mod 16")
    results["capsule_bytes"] = capsule_bytes
    results["sha256_blocks"] = blocks
    results["capsules"] = states
    del slot, fresh, capsules
    return results


def cpu_baseline_capsule(target_seconds: float = 8.0):
    """Part of the cpu_baseline leg: the C restatement's slot serialize and
    restore over the whole bench_capsule batch (8192 states, every window
    position equally often), on one thread and then on every host core this
    process may use with the states dealt round-robin to the threads.  The one-thread
    capsules are byte-compared with the GPU's serialize of the same slot."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np
    import torch

    from gdn_state_codec import capsule as cap
    from oracle import capsule as C

    dev = torch.device("cuda:0")
    slot = capsule_slot(WINDOW_STATES, dev)
    gpu_blobs = cap.serialize_to_host(slot, cap.CapsuleIdentity(CAPSULE_GEOMETRY, 1, 1))
    names = ("residual", "smoothing", "scales", "compensator_keys", "compensator_values",
             "record_decay", "record_keys", "record_corrections", "positions")
    buf = {}
    for n in names:
        t = getattr(slot, n).cpu()
        buf[n] = t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.float16 else (
            t.numpy().view(np.uint32) if n == "positions" else t.numpy())
    del slot
    identity = C.Identity(CAPSULE_GEOMETRY, 1, 1)
    states = WINDOW_STATES
    positions = buf["positions"][:, 0].copy()

    def serialize_some(work):
        # ctypes releases the GIL for the duration of each foreign call.
        ids, reps = work
        out = []
        for _ in range(reps):
            out = [C.slot_serialize(buf, s, 1, identity) for s in ids]
        return out

    target = {n: v.copy() for n, v in buf.items()}  # threads restore disjoint states

    def restore_some(work):
        ids, reps = work
        bad = 0
        for _ in range(reps):
            for s in ids:
                bad += C.slot_restore(blobs[s], target, s, 1, identity, int(positions[s])) != C.OK
        return bad

    def timed(fn, threads, reps):
        # Thread i takes states i, i + threads, ...: every thread sees every
        # window position (capsule size grows with the position).
        work = [(range(i, states, threads), reps) for i in range(threads)]
        t0 = time.perf_counter()
        with ThreadPoolExecutor(threads) as pool:
            parts = list(pool.map(fn, work))
        return time.perf_counter() - t0, parts

    ser_1, parts = timed(serialize_some, 1, 1)
    blobs = parts[0]
    nbytes = sum(len(b) for b in blobs)
    identical = blobs == gpu_blobs
    res_1, bad = timed(restore_some, 1, 1)
    threads = _cpu_threads()
    reps = max(1, int(target_seconds / 2 * threads / max(ser_1 + res_1, 1e-6)))
    ser_n, _ = timed(serialize_some, threads, reps)
    res_n, bad_n = timed(restore_some, threads, reps)
    ok = identical and sum(bad) == 0 and sum(bad_n) == 0
    _log(f"cpu capsule (port): serialize {states} capsules in {ser_1:.2f} s, restore in "
         f"{res_1:.2f} s on 1 thread; x{reps} in {ser_n:.2f} / {res_n:.2f} s on {threads} "
         f"threads; GPU capsules byte-identical={identical}")

    def rates(seconds, count):
        return {"capsules_per_s": count / seconds, "capsule_GBps": nbytes * count / states
                / seconds / 1e9}

    return {"serialize": {**rates(ser_n, states * reps), "cores": threads,
                          "single_thread": {**rates(ser_1, states), "cores": 1}},
            "restore": {**rates(res_n, states * reps), "cores": threads,
                        "single_thread": {**rates(res_1, states), "cores": 1}},
            "kind": "port", "cpu_model": _cpu_model(),
            "sample": f"the whole {states}-capsule bench batch ({nbytes} capsule bytes), "
                      f"{reps} passes with the states dealt round-robin to {threads} threads; "
                      f"one pass on 1 thread",
            "gpu_capsules_byte_identical": bool(ok)}


POOL_LAYERS, POOL_SLOTS, POOL_HEADS, POOL_BATCH, POOL_PADDING = 30, 2048, 32, 512, 26


def pool_bytes_per_direction(dtype_bytes: int) -> int:
    """Algorithmic bytes of one config-5 direction: per valid (layer, slot,
    head) tile the pool tile (fp32 65,536 B or bf16 32,768 B), the int8 codes
    (16,384 B) and the fp32 smoothing and scales (1,024 B)."""
    per_head = 128 * 128 * dtype_bytes + 128 * 128 + 2 * 128 * 4
    return (POOL_BATCH - POOL_PADDING) * POOL_LAYERS * POOL_HEADS * per_head


def _warm_for(fn, warmup: int) -> None:
    """At least `warmup` calls of `fn`, continued until about WARM_MS has
    run (at most WARM_LAUNCHES calls): the same warm phase the back-to-back
    legs get, for legs whose launches are timed one by one."""
    import torch

    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    fn()
    b.record()
    estimate_ms = max(_events_ms([(a, b)])[0], 1e-3)
    for _ in range(max(warmup - 1, min(WARM_LAUNCHES, int(WARM_MS / estimate_ms)))):
        fn()


def bench_pool(steps: int, warmup: int, dtype_name: str, cpu: bool = True):
    """Config 5: a [30 layers][2048 slots][32 heads][128][128] state pool in
    the provider's [value][key] layout (fp32 128.8 GB or bf16 64.4 GB),
    Student-t(3) x 0.05 entries with 2% all-zero heads, a batch of 512 random
    unique slot ids of which 26 are padding (-1).  Gather-encode (pool ->
    compact codes) and decode-scatter (codes -> pool) are timed separately,
    each launch between its own HIP events.  Every encode, warm-up included,
    runs before the first decode, so each one reads the pool as generated;
    the decodes then write the same values back on every launch.  Each
    direction first warms for about WARM_MS of its own launches.  A sample of
    the gathered tiles (the first live tiles in batch order) is checked bit
    for bit in both directions and timed on the host as the CPU baseline."""
    import torch

    from gdn_state_codec import codec

    dev = torch.device("cuda:0")
    dtype = torch.float32 if dtype_name == "f32" else torch.bfloat16
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    layers, slots, heads, batch = POOL_LAYERS, POOL_SLOTS, POOL_HEADS, POOL_BATCH
    _log(f"config 5: generating a {dtype_name} pool {layers}x{slots}x{heads}x128x128")
    pool = torch.empty((layers, slots, heads, 128, 128), dtype=dtype, device=dev)
    for layer in range(layers):
        if layer % 10 == 0:
            _log(f"config 5: pool layers {layer}..{min(layer + 10, layers) - 1}")
        # Student-t(3) = Z / sqrt(chi2_3 / 3), chi2_3 a sum of three squared normals.
        for part in range(0, slots, 256):
            shape = (min(256, slots - part), heads, 128, 128)
            z = torch.randn(shape, generator=gen, device=dev)
            chi = torch.zeros(shape, device=dev)
            for _ in range(3):
                chi.addcmul_(w := torch.randn(shape, generator=gen, device=dev), w)
            pool[layer, part:part + shape[0]] = (z * torch.rsqrt(chi / 3) * 0.05).to(dtype)
            del z, chi, w
    zero = torch.rand((layers, slots, heads), generator=gen, device=dev) < 0.02
    pool[zero] = 0
    del zero
    perm = torch.randperm(slots, generator=gen, device=dev)[:batch].to(torch.int32)
    pad = torch.randperm(batch, generator=gen, device=dev)[:POOL_PADDING]
    perm[pad] = -1
    layout = codec.LAYOUT_VALUE_KEY
    codes = torch.empty((layers, batch, heads, 128, 128), dtype=torch.int8, device=dev)
    s = torch.empty((layers, batch, heads, 128), dtype=torch.float32, device=dev)
    sc = torch.empty_like(s)

    _warm_for(lambda: codec.pool_encode(pool, perm, layout, codes, s, sc), warmup)
    enc = []
    for _ in range(steps):
        e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(2))
        e0.record()
        codec.pool_encode(pool, perm, layout, codes, s, sc)
        e1.record()
        enc.append((e0, e1))
    enc_ms = sum(_events_ms(enc)) / steps
    sample = _pool_sample(pool, perm, codes, s, sc) if cpu else None
    _warm_for(lambda: codec.pool_decode(codes, s, sc, perm, pool, layout), warmup)
    dec = []
    for _ in range(steps):
        e0, e1 = (torch.cuda.Event(enable_timing=True) for _ in range(2))
        e0.record()
        codec.pool_decode(codes, s, sc, perm, pool, layout)
        e1.record()
        dec.append((e0, e1))
    dec_ms = sum(_events_ms(dec)) / steps
    nbytes = pool_bytes_per_direction(4 if dtype_name == "f32" else 2)
    result = {"encode_ms": enc_ms, "decode_ms": dec_ms,
              "encode_GBps": nbytes / (enc_ms * 1e-3) / 1e9,
              "decode_GBps": nbytes / (dec_ms * 1e-3) / 1e9,
              "encode_hbm_frac": nbytes / (enc_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
              "decode_hbm_frac": nbytes / (dec_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS,
              "bytes_per_direction": nbytes, "pool_dtype": dtype_name, "layout": "[value][key]",
              "valid_slots": batch - POOL_PADDING, "steps": steps,
              "timing": "all gather-encodes first (each reads the generated pool), then all "
                        "decode-scatters"}
    _log(f"config 5 ({dtype_name} pool): gather-encode {enc_ms:.3f} ms "
         f"({result['encode_GBps']:.0f} GB/s), decode-scatter {dec_ms:.3f} ms "
         f"({result['decode_GBps']:.0f} GB/s)")
    if sample is not None:
        sample["decoded"] = _pool_sample_tiles(pool, perm, sample["count"])
        result["cpu_baseline"], result["gpu_bit_exact_on_sample"] = cpu_baseline_pool(
            sample, dtype_name)
    del pool, codes, s, sc
    torch.cuda.empty_cache()
    return result


def _pool_sample_tiles(pool, slot_ids, count: int):
    """The first `count` live tiles of the gathered batch, in batch order
    (layer, batch entry, head), copied to the host: fp32 or bf16 bits."""
    import torch

    live = torch.nonzero(slot_ids >= 0).flatten()
    slots = slot_ids[live].long()
    per_layer = live.numel() * pool.shape[2]
    parts = []
    for layer in range((count + per_layer - 1) // per_layer):
        parts.append(pool[layer].index_select(0, slots).reshape(-1, 128, 128))
    tiles = torch.cat(parts)[:count]
    if tiles.dtype == torch.bfloat16:
        return tiles.view(torch.int16).cpu().numpy().view("uint16")
    return tiles.cpu().numpy()


def _pool_sample(pool, slot_ids, codes, smoothing, scales, count: int = 49152):
    """Gathered source tiles and the GPU's encode of them, for the CPU
    baseline and the parity check: `count` tiles (about 3.2 GB of fp32)."""
    import torch

    torch.cuda.synchronize()
    live = torch.nonzero(slot_ids >= 0).flatten()
    per_layer = live.numel() * pool.shape[2]
    layers = (count + per_layer - 1) // per_layer

    def gathered(t):
        return torch.cat([t[layer].index_select(0, live).reshape(-1, *t.shape[3:])
                          for layer in range(layers)])[:count].cpu().numpy()

    return {"count": count, "source": _pool_sample_tiles(pool, slot_ids, count),
            "codes": gathered(codes), "smoothing": gathered(smoothing),
            "scales": gathered(scales)}


def cpu_baseline_pool(sample, dtype_name: str, target_seconds: float = 4.0):
    """The reference's CPU path for a gathered pool batch: each provider
    [value][key] tile transposed to the codec's [key][value]
    (adapter.cpp:21-57), QuantizeBoundary's quant stage and DequantizeBoundary
    (state_capsule.cpp:190-251, through oracle/_ref; the C restatement where
    _ref is absent), and the result transposed back.  bf16 tiles are widened
    before and narrowed (round to nearest even) after, since the reference's
    pools are fp32 (runtime.py:468-469).  Timed on one thread over a bounded
    prefix of the sample, then on every allowed core over the whole sample;
    the GPU's codes, smoothing, scales and decoded tiles are compared with the
    multi-thread results bit for bit."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    import oracle

    kind = "reference" if oracle.ref_available() else "port"
    bf16 = dtype_name == "bf16"

    def round_trip(x):
        x = oracle.bf16_to_f32(x) if bf16 else x
        if kind == "reference":
            c, s, sc = oracle.ref_quantize_heads(np.ascontiguousarray(x.transpose(0, 2, 1)))
            d = oracle.ref_dequantize_heads(c, s, sc)
            c = np.ascontiguousarray(c.transpose(0, 2, 1))
            d = np.ascontiguousarray(d.transpose(0, 2, 1))
        else:
            c, s, sc = oracle.encode_heads(x, oracle.LAYOUT_VALUE_KEY, threads=1)
            d = oracle.decode_heads(c, s, sc, oracle.LAYOUT_VALUE_KEY, threads=1)
        if bf16:
            d = oracle.f32_to_bf16(d.reshape(-1)).reshape(d.shape)
        return c, s, sc, d

    def run(x, threads):
        bounds = np.linspace(0, len(x), threads + 1).astype(int)
        t0 = time.perf_counter()
        if threads == 1:
            out = round_trip(x)
        else:
            with ThreadPoolExecutor(threads) as workers:
                parts = list(workers.map(round_trip, [x[lo:hi] for lo, hi in
                                                      zip(bounds, bounds[1:]) if hi > lo]))
            out = tuple(np.concatenate([part[i] for part in parts]) for i in range(4))
        return time.perf_counter() - t0, out

    source = sample["source"]
    per_tile = 2 * (128 * 128 * (4 if not bf16 else 2) + 128 * 128 + 2 * 128 * 4)
    probe, _ = run(source[:64], 1)
    n = int(min(max(64, target_seconds / max(probe, 1e-6) * 64), len(source)))
    seconds, _ = run(source[:n], 1)
    single = n * per_tile / seconds / 1e9
    threads = _cpu_threads()
    m_seconds, (c, s, sc, d) = run(source, threads)
    multi = len(source) * per_tile / m_seconds / 1e9
    exact = (c.tobytes() == sample["codes"].tobytes()
             and s.tobytes() == sample["smoothing"].tobytes()
             and sc.tobytes() == sample["scales"].tobytes()
             and d.tobytes() == sample["decoded"].tobytes())
    _log(f"cpu config 5 ({dtype_name}, {kind}): {single:.3f} GB/s on 1 thread ({n} tiles), "
         f"{multi:.3f} GB/s on {threads} threads ({len(source)} tiles); "
         f"GPU bit-exact on the sample={exact}")
    widen = "; bf16 widened before and narrowed after in numpy" if bf16 else ""
    return ({"value": multi, "unit": "GB/s", "cores": threads, "kind": kind,
             "cpu_model": _cpu_model(),
             "sample": f"the first {len(source)} live gathered tiles in batch order (layer, "
                       f"entry, head): [value][key] -> [key][value] transpose, quantize, "
                       f"dequantize, transpose back, split contiguously over {threads} "
                       f"threads{widen}",
             "seconds": m_seconds,
             "single_thread": {"value": single, "unit": "GB/s", "cores": 1,
                               "sample": f"the first {n} of those tiles", "seconds": seconds}},
            bool(exact))


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for every cpu_baseline."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def _cpu_threads() -> int:
    """The host cores this process may use, at most 16 (one GPU's share of the box)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline(state, codes, smoothing, scales, target_seconds: float = 8.0):
    """The reference's own C++ CPU path (oracle/_ref) when it is present, else
    the C restatement, over a bounded sample of heads of the same config-2
    state: on one thread, then on every host core this process may use with
    the heads split contiguously.  The reported value is the multi-thread one;
    the GPU codes of the single-thread sample are checked bit-exactly."""
    from concurrent.futures import ThreadPoolExecutor

    import numpy as np

    import oracle

    kind = "reference" if oracle.ref_available() else "port"
    flat = state.view(-1, 128, 128)

    def round_trip(x):
        # ctypes releases the GIL for the duration of each foreign call.
        if kind == "reference":
            c, s, sc = oracle.ref_quantize_heads(x)
            oracle.ref_dequantize_heads(c, s, sc)
        else:
            c, s, sc = oracle.encode_heads(x, oracle.LAYOUT_KEY_VALUE, threads=1)
            oracle.decode_heads(c, s, sc, oracle.LAYOUT_KEY_VALUE, threads=1)
        return c, s, sc

    def run(n, threads=1):
        x = flat[:n].cpu().numpy()
        bounds = np.linspace(0, n, threads + 1).astype(int)
        t0 = time.perf_counter()
        if threads == 1:
            c, s, sc = round_trip(x)
        else:
            with ThreadPoolExecutor(threads) as pool:
                parts = list(pool.map(round_trip, [x[lo:hi] for lo, hi in zip(bounds, bounds[1:])]))
            c, s, sc = (np.concatenate([part[i] for part in parts]) for i in range(3))
        return time.perf_counter() - t0, c, s, sc

    per_head = 2 * (128 * 128 * 5 + 2 * 128 * 4)  # quantize + dequantize bytes
    run(64)  # the first call pays the library's and the pages' first-touch costs
    probe, _, _, _ = run(64)
    n = int(min(max(64, target_seconds / max(probe, 1e-6) * 64), 131072))
    seconds, c, s, sc = run(n)
    parity = (codes.view(-1, 128, 128)[:n].cpu().numpy().tobytes() == c.tobytes()
              and smoothing.view(-1, 128)[:n].cpu().numpy().tobytes() == s.tobytes()
              and scales.view(-1, 128)[:n].cpu().numpy().tobytes() == sc.tobytes())
    single = n * per_head / seconds / 1e9
    _log(f"cpu baseline ({kind}): {n} heads in {seconds:.1f} s on 1 thread -> {single:.3f} GB/s, "
         f"parity={parity}")
    threads = _cpu_threads()
    m = int(min(n * threads, flat.shape[0]))
    m_seconds, mc, _, _ = run(m, threads)
    multi = m * per_head / m_seconds / 1e9
    same = mc[:n].tobytes() == c.tobytes()
    _log(f"cpu baseline ({kind}): {m} heads in {m_seconds:.1f} s on {threads} threads -> "
         f"{multi:.3f} GB/s")
    return {"value": multi, "unit": "GB/s", "cores": threads, "kind": kind,
            "cpu_model": _cpu_model(),
            "sample": f"{m} heads (the first {m} of the config-2 state), quantize+dequantize, "
                      f"heads split contiguously over {threads} threads",
            "seconds": m_seconds,
            "single_thread": {"value": single, "unit": "GB/s", "cores": 1,
                              "sample": f"the first {n} of those heads", "seconds": seconds},
            "gpu_codes_bit_exact_on_sample": bool(parity and same)}


_SYSFS_FIELDS = ("current_memory_partition", "current_compute_partition", "pp_dpm_mclk",
                 "pp_dpm_fclk", "pp_dpm_sclk", "pp_dpm_socclk",
                 "power_dpm_force_performance_level", "mem_info_vram_total")


def _box_info(with_smi: bool = True) -> dict:
    """What the box reports about the GPU this process uses: its PCI address
    and CU count (torch), the amdgpu sysfs partition modes and DPM clock tables
    (the '*' marks the current level), and rocm-smi's partition and clock
    report.  Taken before and after the config-2 timing, to correlate the
    run-to-run spread of the dequantize with the box's state."""
    import subprocess

    import torch

    info = {}
    try:
        props = torch.cuda.get_device_properties(0)
        info["device"] = {"name": props.name, "arch": props.gcnArchName,
                          "cus": props.multi_processor_count,
                          "pci": f"{props.pci_domain_id:04x}:{props.pci_bus_id:02x}:"
                                 f"{props.pci_device_id:02x}"}
        bus = f"{props.pci_domain_id:04x}:{props.pci_bus_id:02x}:{props.pci_device_id:02x}"
    except (AttributeError, RuntimeError):
        bus = None
    for card in sorted(Path("/sys/class/drm").glob("card*/device")):
        try:
            address = card.resolve().name  # e.g. 0000:75:00.0
        except OSError:
            continue
        if bus is not None and not address.startswith(bus):
            continue
        fields = {}
        for name in _SYSFS_FIELDS:
            try:
                fields[name] = (card / name).read_text().strip()
            except OSError:
                pass
        # Board power limits (hwmon, microwatts): a lower cap on some boxes
        # would show as a lower shader clock under the write-heavy dequantize.
        for path in sorted(card.glob("hwmon/hwmon*/power*_cap*")):
            try:
                fields[path.name] = path.read_text().strip()
            except OSError:
                pass
        if fields:
            info.setdefault("sysfs", {})[address] = fields
    if with_smi:
        try:
            proc = subprocess.run(["rocm-smi", "--showmemorypartition", "--showcomputepartition",
                                   "--showclocks", "--json"], capture_output=True, text=True,
                                  timeout=30)
            info["rocm_smi"] = json.loads(proc.stdout) if proc.returncode == 0 else \
                {"returncode": proc.returncode, "stderr": proc.stderr[-300:]}
        except (OSError, ValueError, subprocess.TimeoutExpired) as error:
            info["rocm_smi"] = {"error": str(error)[-300:]}
        try:
            proc = subprocess.run(["amd-smi", "metric", "--json"], capture_output=True,
                                  text=True, timeout=60)
            data = json.loads(proc.stdout) if proc.returncode == 0 else None
            if isinstance(data, dict):
                data = data.get("gpu_data", [data])
            keep = ("clock", "power", "temperature", "throttle", "violation", "perf")
            info["amd_smi_metric"] = [
                {key: value for key, value in entry.items()
                 if key == "gpu" or any(word in key.lower() for word in keep)}
                for entry in data if isinstance(entry, dict)] if isinstance(data, list) else \
                {"returncode": proc.returncode, "stderr": proc.stderr[-300:]}
        except (OSError, ValueError, subprocess.TimeoutExpired) as error:
            info["amd_smi_metric"] = {"error": str(error)[-300:]}
    return info


class _ClockSampler:
    """Samples the GPU's current shader clock (the '*' level of amdgpu's
    pp_dpm_sclk) and its hwmon frequency, power and temperature readings from
    a host thread every ~2 ms while a timed region runs; `summary()` gives
    min / median / max per reading.  Reads sysfs only: it does not touch the
    GPU's queues."""

    def __init__(self, device_dir):
        import threading

        self.dir = device_dir
        self.samples: dict[str, list[float]] = {}
        self._stop = threading.Event()
        self._thread = threading.Thread(target=self._run, daemon=True)
        self.hwmon = sorted(p for p in (device_dir / "hwmon").glob("hwmon*/*_input")
                            if p.name.startswith(("freq", "power", "temp"))) \
            if device_dir is not None else []
        self.hwmon += sorted(p for p in (device_dir / "hwmon").glob("hwmon*/power*_average")) \
            if device_dir is not None else []

    def _read(self):
        try:
            for line in (self.dir / "pp_dpm_sclk").read_text().splitlines():
                if line.endswith("*"):
                    mhz = float(line.split(":")[1].strip().rstrip("*").strip().rstrip("Mhz"))
                    self.samples.setdefault("sclk_MHz", []).append(mhz)
        except (OSError, ValueError, IndexError):
            pass
        for path in self.hwmon:
            try:
                self.samples.setdefault(path.name, []).append(float(path.read_text()))
            except (OSError, ValueError):
                pass

    def _run(self):
        while not self._stop.is_set():
            self._read()
            self._stop.wait(0.002)

    def __enter__(self):
        if self.dir is not None:
            self._thread.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        if self.dir is not None:
            self._thread.join()

    def summary(self) -> dict:
        out = {}
        for name, values in self.samples.items():
            values = sorted(values)
            out[name] = {"min": values[0], "median": values[len(values) // 2],
                         "max": values[-1], "samples": len(values)}
        return out


def _device_sysfs():
    """The amdgpu sysfs directory of the GPU this process uses, or None."""
    import torch

    try:
        props = torch.cuda.get_device_properties(0)
        bus = f"{props.pci_domain_id:04x}:{props.pci_bus_id:02x}:{props.pci_device_id:02x}"
    except (AttributeError, RuntimeError):
        return None
    for card in sorted(Path("/sys/class/drm").glob("card*/device")):
        try:
            if card.resolve().name.startswith(bus):
                return card
        except OSError:
            continue
    return None


def _traffic(kernel: str):
    """HBM bytes per launch of `kernel` at config 2, from the rocprofv3
    FETCH_SIZE / WRITE_SIZE summary committed under profiles/."""
    path = ROOT / "profiles" / f"{kernel}_c2_traffic.json"
    if not path.is_file():
        return None
    try:
        return json.loads(path.read_text()).get("bytes_per_launch")
    except (ValueError, OSError):
        return None


def codec_roofline(enc_ms: float, dec_ms: float) -> dict:
    """The roofline object of the config-2 codec: the slower (dominant) of the
    two kernels at the top level, both under "kernels"."""
    kernels = {}
    for name, label, ms in (("decode_kernel", "dequantize", dec_ms),
                            ("encode_kernel", "quantize", enc_ms)):
        achieved = C2_BYTES / (ms * 1e-3) / 1e9
        kernels[name] = {"kernel": f"{name} ({label})", "bound": "hbm", "achieved": achieved,
                         "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBPS,
                         "traffic": _traffic(name), "algorithmic_bytes_per_launch": C2_BYTES,
                         "ms": ms}
    dominant = "decode_kernel" if dec_ms >= enc_ms else "encode_kernel"
    return {**kernels[dominant], "dominant": True, "kernels": kernels}


def _pool_probe_fractions(pool: dict, probe) -> None:
    """Each config-5 direction against the same run's tile-stream probe of its
    read:write mix (the fastest of its four forms): the fp32 encode against the
    4:1 contract probe, the fp32 decode against the 1:4 expand probe, the bf16
    encode against the 2:1 halve probe."""
    if not probe:
        return
    def ceiling(name):
        return max(probe[f"{name}{suffix}_GBps"] for suffix in ("", "_nt", "_xcd", "_nt_xcd"))
    for dtype, key, name in (("f32", "encode", "contract"), ("f32", "decode", "expand"),
                             ("bf16", "encode", "halve")):
        leg = pool[dtype]
        leg[f"{key}_probe"] = {"kind": name, "GBps": ceiling(name),
                               "frac": leg[f"{key}_GBps"] / ceiling(name)}


def _expand_probe_fraction(probe, dec_gbps: float) -> dict:
    """The dequantize against the 1:4 read:write probe of the same run (the
    fastest of its plain and nontemporal forms in either order): the ceiling of
    its traffic mix."""
    if not probe:
        return {}
    ceiling = max(probe[f"expand{suffix}_GBps"] for suffix in ("", "_nt", "_xcd", "_nt_xcd"))
    return {"expand_probe_GBps": ceiling, "frac_of_expand_probe": dec_gbps / ceiling}


def profile_pass(codec_only: bool = False) -> int:
    """Two launches of each kernel at the benchmark shapes, and of the 4 GiB
    copy probe (the known-size reference for FETCH_SIZE / WRITE_SIZE);
    `codec_only` stops after the config-2 codec and the probes."""
    import torch

    global WARM_LAUNCHES, TIMED_LAUNCHES
    WARM_LAUNCHES, TIMED_LAUNCHES = 0, 1
    bench_codec(2, 0)
    torch.cuda.empty_cache()
    bench_hbm_probe(repeats=2)
    if codec_only:
        torch.cuda.synchronize()
        print(json.dumps({"profile_pass": "codec"}), flush=True)
        return 0
    bench_valu_probe(repeats=1)
    bench_decode_projection(1, 0)
    bench_chunked_projection(1, 0)
    bench_window_step(0)
    bench_refit(1, 0)
    bench_encoded_rank(1)
    bench_capsule(1, 0)
    torch.cuda.empty_cache()
    bench_boundary_fit(1, False)
    bench_exact_svd(1, False)
    torch.cuda.empty_cache()
    bench_pool(1, 0, "f32", False)
    bench_pool(1, 0, "bf16", False)
    torch.cuda.synchronize()
    print(json.dumps({"profile_pass": "done"}), flush=True)
    return 0


def lds_residency_pass(wait_ticks: int = 20000, repeats: int = 3) -> int:
    """How many workgroups share a CU as a function of their LDS size
    (csrc/bench/lds_probe.hip).  For k = 2..8, k x (CUs) workgroups of 128
    threads each wait 200 us; their LDS size is swept across 163,840 / k in
    steps of 64 bytes.  The kernel takes one wait while k fit on a CU and about
    two once they do not.  Reports, per k, the largest size that still ran in
    one wait, the smallest that took two, and the granule (the spacing of the
    steps) the thresholds imply.  Then, for one-wavefront (64-thread)
    workgroups at a few LDS sizes, the largest k that runs in one wait.  One
    JSON line."""
    import ctypes

    import torch

    lib = _probe_library()
    lib.gdn_lds_residency_probe.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32,
                                            ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64]
    lib.gdn_lds_residency_probe.restype = ctypes.c_int32
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    stream = torch.cuda.current_stream()
    wait_us = wait_ticks / 100.0  # the real-time counter runs at 100 MHz
    result = {"metric": "workgroups resident per CU against LDS bytes", "cus": cus,
              "wait_us": wait_us, "k": {}}

    def rounds_at(k, lds, threads=128):
        sink = torch.empty(k * cus, dtype=torch.int32, device="cuda:0")
        times = []
        for _ in range(repeats):
            start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(stream)
            status = lib.gdn_lds_residency_probe(stream.cuda_stream, sink.data_ptr(), k * cus,
                                                 threads, lds, wait_ticks)
            stop.record(stream)
            if status != 0:
                raise RuntimeError(f"lds residency probe status {status} at {lds} bytes")
            torch.cuda.synchronize()
            times.append(start.elapsed_time(stop) * 1e3)
        return sorted(times)[repeats // 2] / wait_us

    for k in range(2, 9):
        centre = 163840 // k
        sizes = list(range(centre - 3072 - centre % 64, centre + 512, 64))
        ratios = {lds: rounds_at(k, lds) for lds in sizes}
        one = [lds for lds, r in ratios.items() if r < 1.5]
        two = [lds for lds, r in ratios.items() if r >= 1.5]
        entry = {"largest_in_one_wait": max(one) if one else None,
                 "smallest_in_two_waits": min(two) if two else None,
                 "rounds": {str(lds): round(r, 3) for lds, r in ratios.items()}}
        if one and two:
            # The allocation is ceil(lds / G) * G, and k of them fit in 163,840
            # bytes: the largest fitting size is floor(163840 / k / G) * G.
            entry["granules_consistent_with"] = [
                g for g in (256, 512, 768, 1024, 1280, 1536, 2048)
                if max(one) <= (163840 // k // g) * g < min(two)]
        result["k"][str(k)] = entry
        _log(f"lds residency k={k}: one wait up to {entry['largest_in_one_wait']}, "
             f"two from {entry['smallest_in_two_waits']}")
    result["one_wavefront"] = {}
    for lds in (512, 5120, 5184, 6400, 6656, 7168):
        ratios = {k: rounds_at(k, lds, threads=64) for k in range(8, 35)}
        resident = max((k for k, r in ratios.items() if r < 1.5), default=None)
        result["one_wavefront"][str(lds)] = {
            "resident": resident, "rounds": {str(k): round(r, 3) for k, r in ratios.items()}}
        _log(f"lds residency, 64-thread workgroups of {lds} B: {resident} per CU")
    print(json.dumps(result), flush=True)
    return 0


def placement_pass(buffers: int = 4, rounds: int = 2) -> int:
    """The config-2 dequantize into `buffers` separately allocated 16 GB output
    buffers, from two 4 GB code buffers, with each output buffer's own plain
    write and read probes (nontemporal, XCD-contiguous) and the 1:4 expand
    probe on the same (codes, output) pair.  Placement in physical memory is
    the driver's; the rates it gives a buffer are what this pass shows.  One
    JSON line; every decode output is checked equal to the first."""
    import torch

    from gdn_state_codec import codec

    lib = _probe_library()
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(20261201)
    state = torch.randn(C2_SHAPE, generator=gen, device=dev, dtype=torch.float32).mul_(0.05)
    codes = [torch.empty(C2_SHAPE, dtype=torch.int8, device=dev) for _ in range(2)]
    smoothing = torch.empty(C2_SHAPE[:-1], dtype=torch.float32, device=dev)
    scales = torch.empty(C2_SHAPE[:-1], dtype=torch.float32, device=dev)
    layout = codec.LAYOUT_KEY_VALUE
    codec.encode(state, layout, codes[0], smoothing, scales)
    codes[1].copy_(codes[0])
    outs = [state] + [torch.empty_like(state) for _ in range(buffers - 1)]
    sink = torch.empty(lib.gdn_hbm_probe_grid() * 256, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    tiles = state.numel() // (128 * 128)
    nbytes = state.numel() * 4

    def timed(fn, reps=5):
        fn()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record()
        for _ in range(reps):
            fn()
        ev[1].record()
        torch.cuda.synchronize()
        return ev[0].elapsed_time(ev[1]) / reps

    reference = None
    rows = []
    for rnd in range(rounds):
        for i, out in enumerate(outs):
            row = {"round": rnd, "output": i,
                   "write_GBps": nbytes / timed(lambda: lib.gdn_hbm_probe_write(
                       stream, out.data_ptr(), nbytes, 3)) / 1e6,
                   "read_GBps": nbytes / timed(lambda: lib.gdn_hbm_probe_read(
                       stream, out.data_ptr(), sink.data_ptr(), nbytes, 3)) / 1e6}
            for c, code in enumerate(codes):
                row[f"codes{c}_decode_ms"] = timed(
                    lambda: codec.decode(code, smoothing, scales, layout, out=out))
                if reference is None:
                    reference = out.clone()
                elif not torch.equal(out, reference):
                    raise RuntimeError("dequantize outputs differ between buffers")
                row[f"codes{c}_expand_ms"] = timed(lambda: lib.gdn_hbm_probe_expand(
                    stream, code.data_ptr(), out.data_ptr(), tiles, 3))
            _log(json.dumps(row))
            rows.append(row)
    print(json.dumps({"placement_pass": "config 2 dequantize", "buffers": buffers,
                      "rounds": rounds, "rows": rows}), flush=True)
    return 0


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--no-pool", action="store_true",
                        help="skip config 5 (the fp32 and bf16 slot pools)")
    parser.add_argument("--only-codec", action="store_true", help="config 2 only")
    parser.add_argument("--profile", action="store_true",
                        help="a few launches of every kernel, for rocprofv3 counter passes")
    parser.add_argument("--profile-codec", action="store_true",
                        help="the --profile launches of the config-2 codec and the probes only")
    parser.add_argument("--placement", action="store_true",
                        help="the config-2 dequantize and HBM probes on several output buffers")
    parser.add_argument("--lds-residency", action="store_true",
                        help="workgroups resident per CU against their LDS size")
    args = parser.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (every head "
              "tile is independent, so ranks would take contiguous tile ranges with no "
              "exchange).", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    torch.cuda.init()
    if args.profile or args.profile_codec:
        return profile_pass(codec_only=args.profile_codec)
    if args.placement:
        return placement_pass()
    if args.lds_residency:
        return lds_residency_pass()
    box = {"before": _box_info()}
    state, codes, smoothing, scales, dense, enc_ms, dec_ms, wall_ms = bench_codec(
        args.steps, args.warmup)
    box["after_codec"] = _box_info(with_smi=False)
    box["during_codec"] = dict(CODEC_CLOCKS)
    _log(f"config 2 clocks and sensors: {json.dumps(CODEC_CLOCKS)}")
    step_ms = enc_ms + dec_ms
    value = 2 * C2_BYTES / (step_ms * 1e-3) / 1e9
    enc_gbps = C2_BYTES / (enc_ms * 1e-3) / 1e9
    dec_gbps = C2_BYTES / (dec_ms * 1e-3) / 1e9
    cpu = None if args.no_cpu else cpu_baseline(state, codes, smoothing, scales)
    del state, dense, codes, smoothing, scales
    torch.cuda.empty_cache()
    extra = {}
    if not args.only_codec:
        extra["hbm_probe"] = bench_hbm_probe()
        extra["valu_probe"] = bench_valu_probe()
        dec_us, dec_sample = bench_decode_projection(args.steps, args.warmup)
        extra["decode_projection"] = {
            "workload": "config 3: B=256, 32 value heads (GQA from 16), int8 [256,32,128,128]",
            "us_per_step": dec_us, "GBps": C3_BYTES / (dec_us * 1e-6) / 1e9,
            "hbm_frac": C3_BYTES / (dec_us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
            "bytes_per_step": C3_BYTES, "rotated_state_copies": ROTATIONS}
        probe = same_size_probe("read", C3_BYTES, args.steps)
        probe["kernel_frac_of_probe"] = probe["us"] / dec_us
        extra["decode_projection"]["same_size_probe"] = probe
        if not args.no_cpu:
            extra["decode_projection"]["cpu_baseline"] = cpu_baseline_projection(
                dec_sample, False, dec_us)
        del dec_sample
        torch.cuda.empty_cache()
        chunk_us, chunk_sample = bench_chunked_projection(args.steps, args.warmup)
        extra["chunked_projection"] = {
            "workload": "config 4: 64 seqs x T=64 x 32 heads, bf16 MFMA",
            "us_per_step": chunk_us, "GBps": C4_BYTES / (chunk_us * 1e-6) / 1e9,
            "hbm_frac": C4_BYTES / (chunk_us * 1e-6) / 1e9 / HBM_PEAK_GBPS,
            "TFLOPs": C4_FLOPS / (chunk_us * 1e-6) / 1e12,
            "mfma_frac_of_useful_flops": C4_FLOPS / (chunk_us * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "bytes_per_step": C4_BYTES, "rotated_state_copies": ROTATIONS}
        probe = same_size_probe("copy", C4_BYTES, args.steps)
        probe["kernel_frac_of_probe"] = probe["us"] / chunk_us
        extra["chunked_projection"]["same_size_probe"] = probe
        if not args.no_cpu:
            extra["chunked_projection"]["cpu_baseline"] = cpu_baseline_projection(
                chunk_sample, True, chunk_us)
        del chunk_sample
        torch.cuda.empty_cache()
        extra["windowed_step"] = bench_window_step(args.warmup)
        torch.cuda.empty_cache()
        extra["window_refit"] = bench_refit(max(args.steps // 2, 5), 1)
        torch.cuda.empty_cache()
        extra["encoded_rank_chain"] = bench_encoded_rank(args.steps)
        torch.cuda.empty_cache()
        extra["capsule"] = bench_capsule(max(args.steps // 4, 3), args.warmup)
        if not args.no_cpu:
            extra["capsule"]["cpu_baseline"] = cpu_baseline_capsule()
        torch.cuda.empty_cache()
        extra["boundary_fit"] = bench_boundary_fit(args.steps, not args.no_cpu)
        extra["exact_svd"] = bench_exact_svd(args.steps, not args.no_cpu)
        extra["config1"] = bench_config1(args.steps, not args.no_cpu)
        torch.cuda.empty_cache()
        extra["compression_gate"] = bench_compression_gate()
    if not args.no_pool and not args.only_codec:
        torch.cuda.empty_cache()
        extra["pool_codec"] = {
            "workload": "config 5: slot-indexed pool [30][2048][32][128][128], batch 512 random "
                        "unique slot ids with 26 padding (-1), Student-t(3) x 0.05, 2% zero heads",
            "f32": bench_pool(max(args.steps // 4, 3), 1, "f32", not args.no_cpu),
            "bf16": bench_pool(max(args.steps // 4, 3), 1, "bf16", not args.no_cpu)}
        _pool_probe_fractions(extra["pool_codec"], extra.get("hbm_probe"))
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": step_ms,
        "wall_ms_per_step": wall_ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (torch.randn * 0.05, seeded, generated on the GPU)",
        "config": {"workload": "config 2: batched quantize + dequantize of a [30,256,32,128,128] "
                               "fp32 GDN state, layout [L,B,H,K,V]",
                   "tiles": C2_TILES, "bytes_per_direction": C2_BYTES},
        "quantize": {"ms": enc_ms, "GBps": enc_gbps, "hbm_frac": enc_gbps / HBM_PEAK_GBPS},
        "dequantize": {"ms": dec_ms, "GBps": dec_gbps, "hbm_frac": dec_gbps / HBM_PEAK_GBPS,
                       **_expand_probe_fraction(extra.get("hbm_probe"), dec_gbps)},
        "roofline": codec_roofline(enc_ms, dec_ms),
        "cpu_baseline": cpu,
        **extra,
        "box": box,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
