"""CPU oracle for the FFN site around the MoE layer -- TEST INFRASTRUCTURE ONLY.

Restates in numpy the reference's hyper-connection (``mhc.py:23-60``) and
RMSNorm (``layers.py:119-140``), and composes them with the MoE oracle into the
FFN site of a decoder layer (``model.py:132-136``).  Imported only by
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU baseline, as the
checker; the product path never calls it.

MLX-internal choices stated explicitly: dot products and means are exact
(float64) and rounded once to f32; elementwise steps run in f32 in the order
the reference writes them; the hc-axis sums run in ascending order.
"""

from __future__ import annotations

import numpy as np

from .moe_oracle import bf16_round, moe_layer, sigmoid_f32

F32 = np.float32


def rms_norm(x, weight, eps: float) -> np.ndarray:
    """``mx.fast.rms_norm(x, weight, eps)`` on f32 rows (``layers.py:126-131``;
    unweighted ``layers.py:139-140``): ``x * (1 / sqrt(mean(x^2) + eps)) * w``."""
    x = np.asarray(x, dtype=F32)
    ms = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True).astype(F32)
    inv = (F32(1.0) / np.sqrt(ms + F32(eps))).astype(F32)
    y = (x * inv).astype(F32)
    if weight is not None:
        y = (y * np.asarray(weight, dtype=F32)).astype(F32)
    return y


def _softmax_rows(x) -> np.ndarray:
    m = x.max(axis=-1, keepdims=True)
    e = np.exp((x - m).astype(F32)).astype(F32)
    s = np.zeros(e.shape[:-1] + (1,), dtype=F32)
    for q in range(e.shape[-1]):
        s = (s + e[..., q:q + 1]).astype(F32)
    return (e / s).astype(F32)


def _axis_sum(x, axis: int) -> np.ndarray:
    """Sum over a short axis in ascending order (f32)."""
    moved = np.moveaxis(x, axis, -1)
    s = np.zeros(moved.shape[:-1], dtype=F32)
    for q in range(moved.shape[-1]):
        s = (s + moved[..., q]).astype(F32)
    return np.expand_dims(s, axis)


def hyper_connection(streams, fn, base, scale, *, sinkhorn_iters: int, rms_eps: float,
                     hc_eps: float, bf16_streams: bool = False):
    """``HyperConnection.__call__`` (``mhc.py:23-48``) on streams ``[T, hc, d]``
    (f32 values; ``bf16_streams``: the model holds them in bf16, so collapsed is
    rounded to bf16, ``mhc.py:46``): returns ``(post [T, hc], comb [T, hc, hc],
    collapsed [T, d])``."""
    streams = np.asarray(streams, dtype=F32)
    T, hc, d = streams.shape
    flat = rms_norm(streams.reshape(T, hc * d), None, rms_eps)
    mixed = (flat.astype(np.float64) @ np.asarray(fn, np.float64).T).astype(F32)
    base = np.asarray(base, dtype=F32)
    scale = np.asarray(scale, dtype=F32)
    pre_w, post_w, comb_w = mixed[:, :hc], mixed[:, hc:2 * hc], mixed[:, 2 * hc:]
    pre = (sigmoid_f32((pre_w * scale[0] + base[:hc]).astype(F32)) + F32(hc_eps)).astype(F32)
    post = (F32(2.0) * sigmoid_f32((post_w * scale[1] + base[hc:2 * hc]).astype(F32))).astype(F32)
    logits = (comb_w.reshape(T, hc, hc) * scale[2]).astype(F32) + base[2 * hc:].reshape(hc, hc)
    comb = (_softmax_rows(logits.astype(F32)) + F32(hc_eps)).astype(F32)
    comb = (comb / (_axis_sum(comb, -2) + F32(hc_eps))).astype(F32)
    for _ in range(sinkhorn_iters - 1):
        comb = (comb / (_axis_sum(comb, -1) + F32(hc_eps))).astype(F32)
        comb = (comb / (_axis_sum(comb, -2) + F32(hc_eps))).astype(F32)
    collapsed = np.zeros((T, d), dtype=F32)
    for i in range(hc):
        collapsed = (collapsed + pre[:, i:i + 1] * streams[:, i, :]).astype(F32)
    if bf16_streams:
        collapsed = bf16_round(collapsed)
    return post, comb, collapsed


def hyper_residual(residual, y, post, comb, *, bf16_streams: bool = False) -> np.ndarray:
    """``hyper_residual`` (``mhc.py:51-60``):
    ``out[t, j] = post[t, j] y[t] + sum_i comb[t, i, j] residual[t, i]`` with an
    f32 ``y``.  ``bf16_streams``: the residual is bf16 in the model, so ``post``
    and ``comb`` are cast to bf16 and the mixing product is a bf16 matmul
    (rounded once), added to the f32 placement in f32."""
    residual = np.asarray(residual, dtype=F32)
    post = np.asarray(post, F32)
    comb = np.asarray(comb, F32)
    if bf16_streams:
        post, comb = bf16_round(post), bf16_round(comb)
    placed = (post[:, :, None] * np.asarray(y, F32)[:, None, :]).astype(F32)
    mixed = np.einsum("tij,tid->tjd", comb.astype(np.float64),
                      residual.astype(np.float64)).astype(F32)
    if bf16_streams:
        mixed = bf16_round(mixed)
    return (placed + mixed).astype(F32)


def ffn_site(streams, hc_weights, norm_weight, moe_args, *, sinkhorn_iters: int,
             rms_eps: float, hc_eps: float, norm_eps: float, bf16_streams: bool = False):
    """The MoE FFN site of ``GLMDecoderLayer.__call__`` (``model.py:132-136``):
    ``post, comb, collapsed = ffn_hc(h)``; ``y = mlp(norm(collapsed))`` with the
    MoE on the bf16 cast of the normalised row (``native_expert_ssd.py:655-658``);
    ``hyper_residual(h, y, post, comb)``.  ``hc_weights = (fn, base, scale)``;
    ``moe_args`` are ``moe_layer``'s positional and keyword arguments after x."""
    post, comb, collapsed = hyper_connection(streams, *hc_weights, sinkhorn_iters=sinkhorn_iters,
                                             rms_eps=rms_eps, hc_eps=hc_eps,
                                             bf16_streams=bf16_streams)
    normed = bf16_round(rms_norm(collapsed, norm_weight, norm_eps))
    args, kwargs = moe_args
    y = moe_layer(normed, *args, **kwargs)
    out = hyper_residual(streams, y, post, comb, bf16_streams=bf16_streams)
    return out, {"post": post, "comb": comb, "collapsed": collapsed, "normed": normed, "y": y}


PINNING = {
    "rms_norm": "closed form on constant rows (x / sqrt(x^2 + eps) * w) and zero rows",
    "hyper_connection": "the reference's own case tests/test_mhc.py:12-40 restated independently; "
                        "closed form with fn = base = 0 (gates 0.5 + eps and 1, the Sinkhorn "
                        "recursion c -> c / (hc c + eps) counted per normalisation with a large "
                        "eps); column sums S / (S + eps) after the last normalisation",
    "hyper_residual": "tests/test_mhc.py:42-47 case; identity comb / zero post gives the residual, "
                      "zero comb / unit post gives y in every stream",
}
