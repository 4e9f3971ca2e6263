"""The MoE FFN site of a GLM-5.3-Flash decoder layer.

``GLMDecoderLayer`` (``model.py:47-136`` of the reference) runs attention and
then, for a sparse layer, this FFN block on the hyper-connection streams
(``model.py:132-136``)::

    post, comb, collapsed = ffn_hc(hidden_states)
    fed_forward = mlp(post_attention_layernorm(collapsed))
    return hyper_residual(hidden_states, fed_forward, post, comb)

``MoEDecoderFFN`` is that block with the reference's attribute names
(``ffn_hc``, ``post_attention_layernorm``, ``mlp``; ``model.py:55-59``).  The
hyper-connection, the norm and its bf16 cast run as one library call
(``glm_hc_pre``), the MoE layer and the residual update as another
(``glm_moe_forward_hc``; at a few tokens the update rides in the layer's last
kernel): two kernels before the MoE's own, no host synchronisation.  Attention is not part of this package.
"""

from __future__ import annotations

import torch

from .layers import RMSNorm
from .mhc import HyperConnection
from .model_config import GLMTextConfig
from .moe import ExpertSSDFactory, ExpertSSDMoE


class MoEDecoderFFN:
    def __init__(self, config: GLMTextConfig, layer_idx: int, expert_factory: ExpertSSDFactory):
        self.config = config
        self.layer_idx = layer_idx
        self.ffn_hc = HyperConnection(config)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.mlp = ExpertSSDMoE(config, layer_idx, expert_factory)

    def __call__(self, hidden_states: torch.Tensor) -> torch.Tensor:
        """``hidden_states [..., hc, d]`` (f32, or bf16 before the first MoE
        layer) -> f32 of the same shape."""
        post, comb, normed = self.ffn_hc.with_norm(hidden_states, self.post_attention_layernorm)
        hc, d = hidden_states.shape[-2], hidden_states.shape[-1]
        bf16 = hidden_states.dtype == torch.bfloat16
        residual = hidden_states.reshape(-1, hc, d)
        if bf16:
            residual = residual.to(torch.float32)  # exact; the bf16 rounding points apply
        out = self.mlp.with_hyper_residual(normed.reshape(-1, d), residual, post, comb, bf16)
        return out.reshape(hidden_states.shape)
