"""GPU parity of the exact-SVD boundary initializer
(exact_svd_boundary_launch_v1; the reference runtime's exact_svd initializer,
src/gdn_state_codec/runtime.py:335-389, which calls torch.linalg.svd) through
the C-ABI, against the float64 LAPACK SVD of oracle/svd.py.

The reference's result is its library's fp32 SVD, so no bit pattern is fixed;
the tests hold the fp32 rank-4 product to 4e-7 of the largest singular value,
the singular values likewise, the fp16 compensators to their own rounding of
that product, and the codes bit-exact to the oracle's quant stage applied to
the residual the kernel wrote.  The kernel iterates in double, so what remains
is the fp32 rounding of its outputs: keys and values rounded to fp32 and a
four-term fp32 product, a few units of 2^-24 of the largest singular value
(the bench measures 7.3e-8 on C1 heads).  4e-7 leaves that a margin of about
five, so an accumulation that loses ten times the precision fails; torch's
fp32 SVD, the reference's own call, lands at 3e-7..3e-6 on Gaussian heads."""

import numpy as np
import pytest
import torch

import datagen
import oracle
from gdn_state_codec import codec
from oracle import svd as S

pytestmark = pytest.mark.gpu
FIT_TOLERANCE = 4e-7  # of the largest singular value


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def planted_head(seed, spectrum):
    g = np.random.default_rng(seed)
    q1, _ = np.linalg.qr(g.standard_normal((128, 128)))
    q2, _ = np.linalg.qr(g.standard_normal((128, 128)))
    return ((q1 * spectrum) @ q2.T).astype(np.float32)


def dense_heads():
    g = datagen.rng(71)
    spread = np.concatenate([[40.0, 20.0, 10.0, 5.0], np.linspace(1.0, 0.01, 124)])
    return {
        "c1": datagen.c1_heads(4, 72),
        "student_t": datagen.student_t_heads(4, 73),
        "planted": np.stack([planted_head(74, spread), planted_head(75, spread * 1e-3)]),
        "special": np.stack([
            datagen.wide_range_head(76),
            datagen.tiny_head(77),
            datagen.zero_rows_cols_head(78),
            np.outer(g.standard_normal(128), g.standard_normal(128)).astype(np.float32),
            datagen.constant_head(0.25),
            np.zeros((128, 128), np.float32),
        ]),
    }


def run(dense):
    provider = torch.from_numpy(np.ascontiguousarray(dense.transpose(0, 2, 1))).cuda()
    out = codec.exact_svd_boundary(provider)
    return provider, [host(t) for t in out]


def check_heads(dense, got, rank_deficient=()):
    codes, s, sc, keys16, values16, residual, status = got
    assert (status == 0).all()
    provider = dense.transpose(0, 2, 1)
    left, right, singular, product = S.svd_fit_heads(provider)
    keys = keys16.view(np.float16).astype(np.float64)
    values = values16.view(np.float16).astype(np.float64)
    for h in range(len(dense)):
        top = max(singular[h, 0], 1e-30)
        # The fp32 fit the residual was formed with, [key][value].
        fit = (provider[h].astype(np.float64) - residual[h].astype(np.float64)).T
        assert np.abs(fit - product[h]).max() <= FIT_TOLERANCE * top, h
        # fp16 compensators: their product is the fit, to fp16 rounding.
        pair = keys[h] @ values[h].T
        bound = 2.0 ** -10 * (np.abs(keys[h]) @ np.abs(values[h]).T) + 2.0 ** -23 * top
        assert (np.abs(pair - fit) <= bound + FIT_TOLERANCE * top).all(), h
        norms = np.linalg.norm(keys[h], axis=0)
        assert np.abs(norms - singular[h, :4]).max() <= 2.0 ** -10 * top + FIT_TOLERANCE * top, h
        if h not in rank_deficient:
            gram = values[h].T @ values[h]
            assert np.abs(gram - np.eye(4)).max() <= 4e-3, h
    # The quant stage: the oracle's encode of the residual the kernel wrote.
    e_codes, e_s, e_sc = oracle.encode_heads(residual, oracle.LAYOUT_VALUE_KEY, threads=8)
    assert codes.tobytes() == e_codes.tobytes()
    assert s.tobytes() == e_s.tobytes()
    assert sc.tobytes() == e_sc.tobytes()


@pytest.mark.parametrize("family", ["c1", "student_t", "planted"])
def test_exact_svd_matches_float64_svd(device, family):
    dense = dense_heads()[family]
    print(f"exact SVD initializer, {family}, heads={len(dense)}", flush=True)
    provider, got = run(dense)
    check_heads(dense, got)


def test_planted_vectors_are_recovered_up_to_sign(device):
    """Heads with well separated singular values: each compensator pair is the
    planted (sigma u, v) up to one sign per pair, to fp16 rounding."""
    dense = dense_heads()["planted"]
    print("exact SVD initializer, planted vectors", flush=True)
    _, got = run(dense)
    keys = got[3].view(np.float16).astype(np.float64)
    values = got[4].view(np.float16).astype(np.float64)
    left, right, singular, _ = S.svd_fit_heads(dense.transpose(0, 2, 1))
    for h in range(len(dense)):
        for r in range(4):
            sign = np.sign(values[h, :, r] @ right[h, :, r])
            assert np.abs(sign * values[h, :, r] - right[h, :, r]).max() <= 2e-3
            assert (np.abs(sign * keys[h, :, r] - left[h, :, r]).max()
                    <= 2e-3 * singular[h, r] + FIT_TOLERANCE * singular[h, 0])


def test_special_heads(device):
    """Wide exponent range, subnormals, zero rows and columns, rank 1, a
    constant head and an all-zero head (zero compensators, residual = input)."""
    dense = dense_heads()["special"]
    print(f"exact SVD initializer, special heads={len(dense)}", flush=True)
    provider, got = run(dense)
    check_heads(dense, got, rank_deficient=(3, 4, 5))
    keys16, values16, residual = got[3], got[4], got[5]
    assert not keys16[5].any() and not values16[5].any()
    assert residual[5].tobytes() == host(provider)[5].tobytes()


def test_non_finite_heads_are_rejected(device):
    dense = datagen.c1_heads(4, 79)
    dense[1, 5, 9] = np.nan
    dense[2, 0, 127] = -np.inf
    print("exact SVD initializer, rejections", flush=True)
    provider = torch.from_numpy(np.ascontiguousarray(dense.transpose(0, 2, 1))).cuda()
    got = codec.exact_svd_boundary(provider, check=False)
    assert host(got[6]).tolist() == [0, 1, 1, 0]
    with pytest.raises(ValueError, match="head 1 holds a non-finite value"):
        codec.exact_svd_boundary(provider)


def test_many_heads(device):
    """1,024 heads (four rounds of one workgroup per CU): every status 0, and
    every 61st head checked against the float64 SVD."""
    dense = np.concatenate([datagen.c1_heads(512, 81), datagen.student_t_heads(512, 82)])
    print(f"exact SVD initializer, heads={len(dense)}", flush=True)
    _, got = run(dense)
    sample = list(range(0, len(dense), 61))
    check_heads(dense[sample], [g[sample] for g in got])


def test_sweep_limit_flags_unconverged_heads(device):
    """exact_svd_boundary_sweeps_launch_v1: after one sweep no C1 head has
    converged (status 2, and exact_svd_boundary raises), while an all-zero
    head, which never rotates, has (status 0); at the full limit of 30 sweeps
    every output equals the default entry point's bit for bit."""
    print("exact SVD sweep limit", flush=True)
    dense = np.concatenate([datagen.c1_heads(3, 79), np.zeros((1, 128, 128), np.float32)])
    provider = torch.from_numpy(np.ascontiguousarray(dense.transpose(0, 2, 1))).cuda()
    *_, status = codec.exact_svd_boundary(provider, check=False, max_sweeps=1)
    assert host(status).tolist() == [2, 2, 2, 0]
    with pytest.raises(ValueError, match="did not converge"):
        codec.exact_svd_boundary(provider, max_sweeps=1)
    full = [host(t) for t in codec.exact_svd_boundary(provider, max_sweeps=30)]
    default = [host(t) for t in codec.exact_svd_boundary(provider)]
    for a, b in zip(full, default):
        assert a.tobytes() == b.tobytes()
    assert (full[-1] == 0).all()
