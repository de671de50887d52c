"""How the exact-SVD slot's quant stage differs from the reference runtime's.

The reference runtime's ``exact_svd`` initializer quantizes its fp32 residual
with torch ops (``src/gdn_state_codec/runtime.py:371-377``): the smoothing is
``sqrt(clamp(mean(|r|, value axis), 1e-8))`` with the mean in fp32 in torch's
reduction order, and the codes are ``torch.round`` (half to even) of
``r / s / scale * 127``.  ``exact_svd_kernel`` runs the codec's quant stage
instead, the reference's C++ arithmetic (``state_capsule.cpp:190-226``): the
key sum in double, ``lround`` (half away from zero).  Everything else is the
same IEEE fp32 operation in the same order (``r / s``, the column maximum,
``/ scale * 127``).

This test restates runtime.py:371-377 in torch (CPU, float32), runs both
stages on the same fp32 residuals (``D - fl32(U S) fl32(V)^T`` of C1-style and
Student-t(3) heads, from a float64 SVD) and on the dense heads themselves (the
quant-only initializer's residual), and names the cause of every code that
differs:

* ``mean``: the fp32 mean and the double sum round to smoothing values one ulp
  apart, so the row's ``r / s`` (or a column maximum built from such a row)
  differs;
* ``tie``: the smoothing and scale agree, ``r / s / scale * 127`` lands exactly
  on ``n + 0.5`` and the two rounding rules pick neighbouring codes.

No other cause may appear, and the counts are pinned.  They depend on torch's
CPU reduction order for the mean (the reference runs the same ops on its own
device, whose order can differ), so they describe this torch build.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import datagen
import oracle
from oracle import svd

HEADS = 32


def torch_quant_stage(residual: np.ndarray):
    """runtime.py:371-377 on [H][key][value] fp32 residuals: codes in
    [key][value] order (before the runtime's transpose to [value][key]),
    smoothing [H][key], scales [H][value]."""
    r = torch.from_numpy(np.ascontiguousarray(residual, np.float32))
    smoothing = torch.sqrt(torch.clamp(r.abs().mean(dim=2), min=1.0e-8))
    smoothed = r / smoothing.unsqueeze(2)
    scales = smoothed.abs().amax(dim=1)
    safe = torch.where(scales == 0, torch.ones_like(scales), scales)
    quantized = torch.round(smoothed / safe.unsqueeze(1) * 127.0).clamp_(-127, 127)
    return (quantized.to(torch.int8).numpy(), smoothing.numpy(), scales.numpy())


def svd_residuals(dense: np.ndarray) -> np.ndarray:
    """D - fl32(U S) fl32(V)^T per head, rounded once to fp32: the residual the
    exact-SVD initializer quantizes."""
    out = np.empty_like(dense)
    for n, head in enumerate(dense):
        left, right, _, _ = svd.svd_fit(head)
        product = left.astype(np.float32).astype(np.float64) @ \
            right.astype(np.float32).astype(np.float64).T
        out[n] = (head.astype(np.float64) - product).astype(np.float32)
    return out


def classify(residual: np.ndarray, stage=torch_quant_stage):
    """Both stages on the same residuals -> counts of differing codes by cause
    (and of rows whose smoothing differs, with the largest distance in ulps);
    raises on a code that neither cause explains."""
    codes, smoothing, scales = oracle.encode_heads(residual, oracle.LAYOUT_KEY_VALUE)
    tcodes, tsmoothing, tscales = stage(residual)
    ulps = np.abs(smoothing.view(np.int32).astype(np.int64)
                  - tsmoothing.view(np.int32).astype(np.int64))
    counts = {"codes": int(codes.size), "mean": 0, "tie": 0,
              "smoothing_rows": int((ulps != 0).sum()), "smoothing_max_ulps": int(ulps.max())}
    for head, key, value in zip(*np.nonzero(codes != tcodes)):
        same_row = smoothing[head, key] == tsmoothing[head, key]
        same_column = scales[head, value] == tscales[head, value]
        if not (same_row and same_column):
            counts["mean"] += 1
            continue
        m = np.float32(residual[head, key, value]) / smoothing[head, key]
        x = np.float32(np.float32(m / scales[head, value]) * np.float32(127.0))
        assert abs(x) % 1 == 0.5, (head, key, value, x)  # the only other cause
        assert abs(int(codes[head, key, value]) - int(tcodes[head, key, value])) == 1
        counts["tie"] += 1
    return counts


CASES = {
    # name: (residual builder, pinned counts over 32 heads = 524,288 codes)
    "c1_quant_only": (lambda: datagen.c1_heads(HEADS, 701),
                      {"mean": 1, "tie": 0, "smoothing_rows": 1058, "smoothing_max_ulps": 2}),
    "c1_exact_svd": (lambda: svd_residuals(datagen.c1_heads(HEADS, 701)),
                     {"mean": 0, "tie": 0, "smoothing_rows": 1001, "smoothing_max_ulps": 2}),
    "student_t_exact_svd": (lambda: svd_residuals(datagen.student_t_heads(HEADS, 702)),
                            {"mean": 1, "tie": 1, "smoothing_rows": 1076,
                             "smoothing_max_ulps": 2}),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_quant_stage_differences_are_pinned(case):
    build, pinned = CASES[case]
    counts = classify(build())
    print(case, counts)
    assert {k: counts[k] for k in pinned} == pinned, counts


def test_a_planted_tie_is_reported_as_a_tie():
    """A head whose (key 1, value 0) lands exactly on 64.5 after the fp32
    arithmetic: the value is solved for by a few fixed-point steps (it moves
    the row's own smoothing), then the fp32 neighbours around it are scanned.
    lround gives 65 and round-half-even 64, reported under "tie"."""
    head = datagen.c1_heads(1, 703)
    for _ in range(6):
        _, s, sc = oracle.encode_heads(head, oracle.LAYOUT_KEY_VALUE)
        head[0, 1, 0] = np.float32(np.float32(64.5) / np.float32(127.0)) * sc[0, 0] * s[0, 1]
    candidates = [head[0, 1, 0]]
    for _ in range(1024):
        candidates.append(np.nextafter(candidates[-1], np.float32(1.0)))
        candidates.insert(0, np.nextafter(candidates[0], np.float32(0.0)))
    heads = np.repeat(head, len(candidates), axis=0)
    heads[:, 1, 0] = np.array(candidates, np.float32)
    _, s2, sc2 = oracle.encode_heads(heads, oracle.LAYOUT_KEY_VALUE)
    m = heads[:, 1, 0] / s2[:, 1]
    x = (m / sc2[:, 0]).astype(np.float32) * np.float32(127.0)
    hits = np.nonzero(x == np.float32(64.5))[0]
    assert hits.size, "no fp32 neighbour lands on the tie"
    for hit in hits:
        counts = classify(heads[hit:hit + 1])
        if counts["mean"] == 0:
            assert counts["tie"] == 1, counts
            codes, _, _ = oracle.encode_heads(heads[hit:hit + 1], oracle.LAYOUT_KEY_VALUE)
            tcodes, _, _ = torch_quant_stage(heads[hit:hit + 1])
            assert (int(codes[0, 1, 0]), int(tcodes[0, 1, 0])) == (65, 64)
            return
    pytest.fail("every tie candidate also moved the fp32 mean")


def test_an_unexplained_difference_is_rejected():
    """Negative control: a torch stage with truncation in place of round-half-
    even differs from the C++ stage at codes that are neither ties nor
    smoothing differences, and the classifier must refuse them."""

    def truncating_stage(residual):
        codes, smoothing, scales = torch_quant_stage(residual)
        r = torch.from_numpy(np.ascontiguousarray(residual, np.float32))
        s = torch.from_numpy(smoothing)
        safe = torch.from_numpy(np.where(scales == 0, np.float32(1), scales))
        x = r / s.unsqueeze(2) / safe.unsqueeze(1) * 127.0
        return torch.trunc(x).clamp_(-127, 127).to(torch.int8).numpy(), smoothing, scales

    with pytest.raises(AssertionError):
        classify(datagen.c1_heads(2, 704), stage=truncating_stage)
