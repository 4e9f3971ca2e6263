"""Pins of the FFN-site oracle (hyper-connection, hyper_residual, RMSNorm).

The reference's own case (``tests/test_mhc.py:12-47``: its inputs, and its
expectations restated here with plain numpy in the test's own steps), closed
forms, and invariants chosen so that a dropped term, a transposed ``comb`` or a
wrong count of Sinkhorn normalisations fails.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import mhc_oracle as H


def _sig(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def test_reference_case():
    # tests/test_mhc.py:13-23: hidden 2, hc_mult 2, three Sinkhorn iterations
    eps, hc_eps, iters = 1e-6, 1e-6, 3
    streams = np.array([[[0.5, -1.0], [1.5, 0.25]]], np.float32)  # [T=1, hc=2, d=2]
    fn = np.arange(8 * 4, dtype=np.float32).reshape(8, 4) / 80.0 - 0.2
    base = np.linspace(-0.2, 0.2, 8, dtype=np.float32)
    scale = np.array([0.5, 0.75, 1.25], np.float32)
    post, comb, collapsed = H.hyper_connection(streams, fn, base, scale, sinkhorn_iters=iters,
                                               rms_eps=eps, hc_eps=hc_eps)
    # the test's expectation, in float64
    flat = streams.reshape(1, 4).astype(np.float64)
    flat = flat / np.sqrt(np.mean(flat * flat, axis=-1, keepdims=True) + eps)
    mixed = flat @ fn.astype(np.float64).T
    pre = _sig(mixed[:, 0:2] * 0.5 + base[0:2]) + hc_eps
    want_post = 2 * _sig(mixed[:, 2:4] * 0.75 + base[2:4])
    logits = mixed[:, 4:].reshape(1, 2, 2) * 1.25 + base[4:].reshape(2, 2)
    ex = np.exp(logits - logits.max(axis=-1, keepdims=True))
    want_comb = ex / ex.sum(axis=-1, keepdims=True) + hc_eps
    want_comb /= want_comb.sum(axis=-2, keepdims=True) + hc_eps
    for _ in range(iters - 1):
        want_comb /= want_comb.sum(axis=-1, keepdims=True) + hc_eps
        want_comb /= want_comb.sum(axis=-2, keepdims=True) + hc_eps
    want_collapsed = (pre[..., None] * streams).sum(axis=1)
    np.testing.assert_allclose(post, want_post, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(comb, want_comb, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(collapsed, want_collapsed, rtol=1e-5, atol=1e-6)
    # tests/test_mhc.py:42-47
    sub = np.array([[0.2, -0.3]], np.float32)
    got = H.hyper_residual(streams, sub, post, comb)
    want = want_post[..., None] * sub[:, None, :] + np.swapaxes(want_comb, -1, -2) @ streams
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("hc,iters", [(2, 1), (4, 3), (4, 20)])
def test_zero_weights_closed_form(hc, iters):
    """fn = base = 0: every gate logit is 0, so pre = 1/2 + eps, post = 1 and
    all comb entries stay equal; each normalisation maps c -> c / (hc c + eps).
    A large eps makes every normalisation visible."""
    hc_eps, d, T = 0.05, 8, 3
    rng = np.random.default_rng(hc * 10 + iters)
    streams = rng.standard_normal((T, hc, d)).astype(np.float32)
    M = 2 * hc + hc * hc
    post, comb, collapsed = H.hyper_connection(
        streams, np.zeros((M, hc * d), np.float32), np.zeros(M, np.float32),
        np.array([0.3, 0.7, 1.1], np.float32), sinkhorn_iters=iters, rms_eps=1e-6, hc_eps=hc_eps)
    np.testing.assert_array_equal(post, np.ones((T, hc), np.float32))
    c = 1.0 / hc + hc_eps
    for _ in range(1 + 2 * (iters - 1)):
        c = c / (hc * c + hc_eps)
    np.testing.assert_allclose(comb, np.full((T, hc, hc), c), rtol=2e-6)
    np.testing.assert_allclose(collapsed, (0.5 + hc_eps) * streams.sum(axis=1), rtol=1e-5,
                               atol=1e-6)


def test_sinkhorn_ends_on_a_column_normalisation():
    rng = np.random.default_rng(3)
    hc, d, T, hc_eps = 4, 16, 5, 1e-3
    M = 2 * hc + hc * hc
    streams = rng.standard_normal((T, hc, d)).astype(np.float32)
    fn = rng.standard_normal((M, hc * d)).astype(np.float32)
    base = rng.standard_normal(M).astype(np.float32)
    _, comb, _ = H.hyper_connection(streams, fn, base, np.ones(3, np.float32), sinkhorn_iters=4,
                                    rms_eps=1e-6, hc_eps=hc_eps)
    col = comb.astype(np.float64).sum(axis=1)  # after the last x / (colsum + eps)
    assert np.all(col < 1.0) and np.all(col > 1.0 - 2 * hc_eps)
    assert np.all(comb > 0)


def test_rms_norm_closed_form():
    x = np.array([[3.0] * 8, [0.0] * 8, [-2.0] * 8], np.float32)
    w = np.linspace(0.5, 1.5, 8).astype(np.float32)
    eps = 1e-2
    got = H.rms_norm(x, w, eps)
    for r, a in enumerate((3.0, 0.0, -2.0)):
        np.testing.assert_allclose(got[r], a / np.sqrt(a * a + eps) * w, rtol=1e-6)
    np.testing.assert_allclose(H.rms_norm(x, None, eps)[0], 3.0 / np.sqrt(9.0 + eps), rtol=1e-6)


def test_hyper_residual_identity_and_placement():
    rng = np.random.default_rng(4)
    T, hc, d = 2, 4, 12
    res = rng.standard_normal((T, hc, d)).astype(np.float32)
    y = rng.standard_normal((T, d)).astype(np.float32)
    eye = np.broadcast_to(np.eye(hc, dtype=np.float32), (T, hc, hc))
    np.testing.assert_array_equal(H.hyper_residual(res, y, np.zeros((T, hc), np.float32), eye),
                                  res)
    out = H.hyper_residual(res, y, np.ones((T, hc), np.float32), np.zeros((T, hc, hc), np.float32))
    np.testing.assert_array_equal(out, np.broadcast_to(y[:, None, :], (T, hc, d)))
    # comb is applied transposed: out_j sums comb[i][j] residual_i
    comb = np.zeros((T, hc, hc), np.float32)
    comb[:, 2, 0] = 1.0
    out = H.hyper_residual(res, y, np.zeros((T, hc), np.float32), comb)
    np.testing.assert_array_equal(out[:, 0], res[:, 2])
    np.testing.assert_array_equal(out[:, 2], np.zeros((T, d), np.float32))


def test_bf16_stream_rounding_points():
    """With bf16 streams collapsed is rounded to bf16, and hyper_residual
    rounds post, comb and the mixing sum to bf16 before the f32 add."""
    from oracle.moe_oracle import bf16_round
    rng = np.random.default_rng(5)
    T, hc, d = 2, 4, 16
    M = 2 * hc + hc * hc
    streams = bf16_round(rng.standard_normal((T, hc, d)).astype(np.float32))
    fn = rng.standard_normal((M, hc * d)).astype(np.float32) * 0.1
    base = rng.standard_normal(M).astype(np.float32)
    scale = np.array([1.0, 1.0, 1.0], np.float32)
    kw = dict(sinkhorn_iters=3, rms_eps=1e-6, hc_eps=1e-6)
    post, comb, c32 = H.hyper_connection(streams, fn, base, scale, **kw)
    _, _, c16 = H.hyper_connection(streams, fn, base, scale, bf16_streams=True, **kw)
    np.testing.assert_array_equal(c16, bf16_round(c32))
    y = rng.standard_normal((T, d)).astype(np.float32)
    got = H.hyper_residual(streams, y, post, comb, bf16_streams=True)
    p16, k16 = bf16_round(post), bf16_round(comb)
    want = np.zeros((T, hc, d), np.float32)
    for t in range(T):
        for j in range(hc):
            mix = sum(k16[t, i, j].astype(np.float64) * streams[t, i].astype(np.float64)
                      for i in range(hc))
            want[t, j] = (p16[t, j] * y[t]).astype(np.float32) + bf16_round(
                mix.astype(np.float32))
    np.testing.assert_array_equal(got, want)
