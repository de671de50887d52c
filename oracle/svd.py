"""CPU oracle for the exact-SVD boundary initializer -- TEST INFRASTRUCTURE ONLY.

The reference runtime's ``exact_svd`` initializer
(``src/gdn_state_codec/runtime.py:335-389``) takes ``torch.linalg.svd`` of each
dense [key][value] head D and keeps

    left  = U[:, :4] * S[:4]      (compensator keys, [key][4])
    right = V[:, :4]              (compensator values, [value][4])
    residual = D - left @ right^T

before quantizing the residual.  The SVD is a library routine whose signs and,
for equal singular values, whose basis are the library's own; this restatement
uses LAPACK's float64 SVD (numpy) as the checker, and the product
``left @ right^T`` (the best rank-4 approximation, unique when S[3] > S[4])
together with S as the quantities compared.  Only ``tests/`` and ``bench.py``'s
cpu_baseline leg use it.
"""

from __future__ import annotations

import numpy as np

RANK = 4


def svd_fit(dense: np.ndarray):
    """The rank-4 truncated SVD of one dense [key][value] head in float64.

    Returns ``(left, right, singular, product)``: left [key][4] = U*S,
    right [value][4] = V, the 128 singular values in decreasing order and the
    rank-4 product left @ right^T [key][value]."""
    d = np.asarray(dense, dtype=np.float64)
    u, s, vt = np.linalg.svd(d)
    left = u[:, :RANK] * s[:RANK]
    right = vt[:RANK].T
    return left, right, s, left @ right.T


def svd_fit_heads(provider: np.ndarray):
    """svd_fit for [..., 128, 128] provider heads ([value][key], the dense
    state transposed); returns stacked left, right, singular values and
    products (the products in [key][value] order)."""
    provider = np.asarray(provider)
    flat = provider.reshape(-1, provider.shape[-2], provider.shape[-1])
    fits = [svd_fit(p.T) for p in flat]
    lead = provider.shape[:-2]
    stack = lambda i: np.stack([f[i] for f in fits]).reshape(lead + fits[0][i].shape)  # noqa
    return stack(0), stack(1), stack(2), stack(3)
