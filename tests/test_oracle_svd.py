"""Pins of the exact-SVD oracle (oracle/svd.py) on the CPU: a head built from a
known SVD, the Eckart-Young closed form of the rank-4 error, and torch's own
SVD (the reference's call, runtime.py:347-356) on the same heads.  A transposed
head, a dropped singular value and a rank-3 truncation fail them."""

import numpy as np
import pytest
import torch

import datagen
from oracle import svd as S


def planted_head(seed, spectrum):
    """D = Q1 diag(spectrum) Q2^T with random orthogonal Q1, Q2."""
    g = np.random.default_rng(seed)
    q1, _ = np.linalg.qr(g.standard_normal((128, 128)))
    q2, _ = np.linalg.qr(g.standard_normal((128, 128)))
    return q1, q2, (q1 * spectrum) @ q2.T


def test_fit_recovers_a_planted_decomposition():
    spectrum = np.concatenate([[40.0, 20.0, 10.0, 5.0], np.linspace(1.0, 0.01, 124)])
    q1, q2, d = planted_head(3, spectrum)
    left, right, singular, product = S.svd_fit(d)
    np.testing.assert_allclose(singular, spectrum, rtol=1e-12, atol=1e-12)
    for r in range(4):
        sign = np.sign(right[:, r] @ q2[:, r])  # an SVD fixes the pair's product only
        np.testing.assert_allclose(sign * right[:, r], q2[:, r], atol=1e-10)
        np.testing.assert_allclose(sign * left[:, r], spectrum[r] * q1[:, r], atol=1e-9)
    np.testing.assert_allclose(product, (q1[:, :4] * spectrum[:4]) @ q2[:, :4].T, atol=1e-9)


@pytest.mark.parametrize("maker", ["c1", "student_t", "wide"])
def test_rank4_error_is_the_eckart_young_minimum(maker):
    d = {"c1": lambda: datagen.c1_heads(1, 11)[0],
         "student_t": lambda: datagen.student_t_heads(1, 12)[0],
         "wide": lambda: datagen.wide_range_head(13)}[maker]().astype(np.float64)
    left, right, singular, product = S.svd_fit(d)
    error = np.linalg.norm(d - product) ** 2
    assert abs(error - (singular[4:] ** 2).sum()) <= 1e-9 * (singular ** 2).sum()
    np.testing.assert_allclose(right.T @ right, np.eye(4), atol=1e-12)
    # A rank-3 truncation leaves S[3]^2 more.
    rank3 = (left[:, :3] @ right[:, :3].T)
    assert np.linalg.norm(d - rank3) ** 2 > error + 0.5 * singular[3] ** 2


def test_provider_heads_are_transposed_dense_heads():
    """svd_fit_heads reads provider [value][key] tiles: its product equals the
    dense fit, and fitting the untransposed tile would give the transposed
    product (so a layout mistake shows on any non-symmetric head)."""
    dense = datagen.c1_heads(3, 14).astype(np.float64)
    provider = dense.transpose(0, 2, 1).copy()
    left, right, singular, product = S.svd_fit_heads(provider)
    for h in range(3):
        np.testing.assert_allclose(product[h], S.svd_fit(dense[h])[3], atol=1e-12)
        wrong = S.svd_fit(provider[h])[3]
        assert np.abs(wrong - product[h]).max() > 1e-3 * singular[h, 0]
    assert left.shape == (3, 128, 4) and right.shape == (3, 128, 4)


def test_fit_agrees_with_torch_svd():
    """torch.linalg.svd (the reference's call) in float64 on the CPU gives the
    same rank-4 product and singular values."""
    for h, d in enumerate(datagen.student_t_heads(2, 15).astype(np.float64)):
        u, s, vt = torch.linalg.svd(torch.from_numpy(d), full_matrices=False)
        product = ((u[:, :4] * s[:4]) @ vt[:4]).numpy()
        left, right, singular, ours = S.svd_fit(d)
        np.testing.assert_allclose(singular, s.numpy(), rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(ours, product, atol=1e-10 * singular[0])
