"""Manifold-constrained hyper-connections around a decoder sublayer.

Mirrors the reference's ``mhc.py`` on torch tensors: ``HyperConnection``
(``mhc.py:12-48``) and ``hyper_residual`` (``mhc.py:51-60``), computed by
libglm53moe (``glm_hc_pre``, ``glm_hc_post``).  Streams are ``[..., hc, d]``
in f32 (the live residual) or bf16 (the residual before the first MoE layer);
bf16 streams are handed to the kernels as their exact f32 values with the
bf16 rounding points of the reference switched on.
"""

from __future__ import annotations

import torch

from . import _native as N
from .contract import ContractError
from .layers import RMSNorm, _f32_param
from .model_config import GLMTextConfig

_STREAM_DTYPES = (torch.float32, torch.bfloat16)


class HyperConnection:
    """``mhc.py:12-48``.  Attributes ``fn`` (``[2 hc + hc^2, hc d]``), ``base``
    (``[2 hc + hc^2]``) and ``scale`` (``[3]``) are attached after construction
    and read as f32."""

    def __init__(self, config: GLMTextConfig):
        self.hc_mult = config.hc_mult
        self.hc_sinkhorn_iters = config.hc_sinkhorn_iters
        self.hc_eps = config.hc_eps
        self.rms_eps = config.rms_norm_eps
        self.fn = None
        self.base = None
        self.scale = None
        self._f32: dict = {}
        self._workspace: torch.Tensor | None = None

    def _params(self):
        return [_f32_param(getattr(self, attr), self._f32, attr, f"hyper_connection.{attr}")
                for attr in ("fn", "base", "scale")]

    def _run(self, streams: torch.Tensor, norm: RMSNorm | None):
        hc = self.hc_mult
        N.require_device(streams, "streams", _STREAM_DTYPES)
        if streams.ndim < 2 or streams.shape[-2] != hc:
            raise ContractError(f"streams must be [..., {hc}, d], got {tuple(streams.shape)}")
        d = streams.shape[-1]
        lead = streams.shape[:-2]
        fn, base, scale = self._params()
        M = 2 * hc + hc * hc
        if tuple(fn.shape) != (M, hc * d) or base.numel() != M or scale.numel() != 3:
            raise ContractError(f"hyper-connection weights fn {tuple(fn.shape)}, base "
                                f"{tuple(base.shape)}, scale {tuple(scale.shape)} do not fit "
                                f"hc {hc}, d {d}")
        rows = streams.reshape(-1, hc, d)
        T = rows.shape[0]
        bf16 = streams.dtype == torch.bfloat16
        xf = rows.to(torch.float32) if bf16 else rows
        dev = streams.device
        post = torch.empty((T, hc), dtype=torch.float32, device=dev)
        comb = torch.empty((T, hc, hc), dtype=torch.float32, device=dev)
        collapsed = normed = None
        if norm is None:
            collapsed = torch.empty((T, d), dtype=torch.float32, device=dev)
        else:
            if norm.dims != d:
                raise ContractError(f"norm over {norm.dims} features, streams of {d}")
            normed = torch.empty((T, d), dtype=torch.bfloat16, device=dev)
        need = int(N.native.load().glm_hc_workspace_bytes(T, hc, d))
        ws = self._workspace
        if ws is None or ws.numel() < need or ws.device != dev:
            ws = self._workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        N.call("glm_hc_pre", N.stream_of(streams), xf.data_ptr(), T, hc, d, fn.data_ptr(),
               base.data_ptr(), scale.data_ptr(), int(self.hc_sinkhorn_iters),
               float(self.rms_eps), float(self.hc_eps),
               None if norm is None else norm.weight_f32().data_ptr(),
               0.0 if norm is None else float(norm.eps),
               N.native.GLM_HC_BF16_STREAMS if bf16 else 0, ws.data_ptr(), ws.numel(),
               post.data_ptr(), comb.data_ptr(), N.ptr(collapsed), N.ptr(normed))
        post = post.reshape(*lead, hc)
        comb = comb.reshape(*lead, hc, hc)
        if norm is None:
            return post, comb, collapsed.to(streams.dtype).reshape(*lead, d)
        return post, comb, normed.reshape(*lead, d)

    def __call__(self, streams: torch.Tensor):
        """``(post [..., hc], comb [..., hc, hc], collapsed [..., d])``; collapsed
        in the streams' dtype (``mhc.py:46``)."""
        return self._run(streams, None)

    def with_norm(self, streams: torch.Tensor, norm: RMSNorm):
        """``post, comb`` and ``bf16(norm(collapsed))`` in one pass: the FFN
        site's ``post_attention_layernorm`` (``model.py:135``) fused, its output
        rounded to bf16 for the MoE layer (``native_expert_ssd.py:655-658``)."""
        return self._run(streams, norm)


def hyper_residual(residual: torch.Tensor, sublayer_output: torch.Tensor, post: torch.Tensor,
                   comb: torch.Tensor) -> torch.Tensor:
    """``mhc.py:51-60``: ``post[j] * y + sum_i comb[i][j] residual[i]`` for an f32
    sublayer output (the MoE layer's); f32 result of the residual's shape."""
    N.require_device(residual, "residual", _STREAM_DTYPES)
    N.require_device(sublayer_output, "sublayer_output", (torch.float32,))
    hc, d = residual.shape[-2], residual.shape[-1]
    rows = residual.reshape(-1, hc, d)
    T = rows.shape[0]
    if sublayer_output.numel() != T * d or post.numel() != T * hc or comb.numel() != T * hc * hc:
        raise ContractError("hyper_residual: residual, sublayer output, post and comb disagree "
                            "in shape")
    N.require_device(post, "post", (torch.float32,))
    N.require_device(comb, "comb", (torch.float32,))
    bf16 = residual.dtype == torch.bfloat16
    rf = rows.to(torch.float32) if bf16 else rows
    out = torch.empty((T, hc, d), dtype=torch.float32, device=residual.device)
    N.call("glm_hc_post", N.stream_of(residual), rf.data_ptr(), T, hc, d,
           sublayer_output.data_ptr(), post.data_ptr(), comb.data_ptr(),
           N.native.GLM_HC_BF16_STREAMS if bf16 else 0, out.data_ptr())
    return out.reshape(residual.shape)


__all__ = ["HyperConnection", "hyper_residual"]
