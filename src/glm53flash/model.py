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
(``glm_hc_pre``), the MoE layer as one (``glm_moe_forward``), the residual
update as one (``glm_hc_post``): five kernels around the MoE's own for a
decode step, no host synchronisation.  Attention is not part of this package.
"""

from __future__ import annotations

import torch

from .layers import RMSNorm
from .mhc import HyperConnection, hyper_residual
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
        fed_forward = self.mlp(normed)
        return hyper_residual(hidden_states, fed_forward, post, comb)
