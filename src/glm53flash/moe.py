"""GLM routed-MoE layer (router + HBM expert bank + shared expert + merge).

Mirrors ``moe.py:19-201`` of the reference: ``TopKRouter`` and
``ExpertSSDMoE`` keep their constructors, attributes and call signatures; the
whole forward runs as one stream-ordered sequence of HIP kernels
(``glm_moe_forward``) with no host synchronisation.
"""

from __future__ import annotations

from collections.abc import Callable

import torch

from . import _native as N
from .contract import ContractError
from .expert_ssd import HBMExpertBank
from .layers import DenseMLP, require_weight
from .model_config import GLMTextConfig


class TopKRouter:
    """``moe.py:19-63``: sigmoid scores + correction bias, group top-2 mask,
    top-k in ascending order (best expert last), unbiased normalised weights."""

    def __init__(self, config: GLMTextConfig):
        self.top_k = config.num_experts_per_tok
        self.num_experts = config.n_routed_experts
        self.hidden_dim = config.hidden_size
        self.routed_scaling_factor = config.routed_scaling_factor
        self.num_group = config.n_group
        self.topk_group = config.topk_group
        self.norm_topk_prob = config.norm_topk_prob
        self.weight: torch.Tensor | None = None
        self.e_score_correction_bias: torch.Tensor | None = None

    def _params(self) -> tuple[torch.Tensor, torch.Tensor]:
        w = require_weight(self.weight, "router.weight")
        b = require_weight(self.e_score_correction_bias, "router.e_score_correction_bias")
        if w.dtype != torch.float32 or b.dtype != torch.float32:
            raise ContractError("router weight and bias must be float32")
        N.require_device(w, "router.weight")
        N.require_device(b, "router.e_score_correction_bias")
        if tuple(w.shape) != (self.num_experts, self.hidden_dim) or b.numel() != self.num_experts:
            raise ContractError(f"router weight {tuple(w.shape)} / bias {tuple(b.shape)} do not "
                                f"match E={self.num_experts}, d={self.hidden_dim}")
        return w, b

    def __call__(self, hidden_states: torch.Tensor):
        w, b = self._params()
        N.require_device(hidden_states, "hidden_states", (torch.bfloat16,))
        rows = hidden_states.reshape(-1, self.hidden_dim)
        T = rows.shape[0]
        dev = rows.device
        logits = torch.empty((T, self.num_experts), dtype=torch.float32, device=dev)
        weights = torch.empty((T, self.top_k), dtype=torch.float32, device=dev)
        indices = torch.empty((T, self.top_k), dtype=torch.int32, device=dev)
        N.call("glm_router_topk", N.stream_of(rows), rows.data_ptr(), T, self.hidden_dim,
               w.data_ptr(), b.data_ptr(), self.num_experts, self.top_k, self.num_group,
               self.topk_group, int(self.norm_topk_prob), float(self.routed_scaling_factor),
               logits.data_ptr(), weights.data_ptr(), indices.data_ptr())
        return logits, weights, indices


ExpertSSDFactory = Callable[[int], HBMExpertBank]


class ExpertSSDMoE:
    """Shared MLP plus routed MXFP4 experts from an HBM-resident bank
    (``moe.py:70-201``).  Output is float32 (bf16 route outputs times f32
    weights promote, ``moe.py:199-201``) with the input's shape."""

    def __init__(self, config: GLMTextConfig, layer_idx: int, expert_factory: ExpertSSDFactory):
        config.validate()
        self.config = config
        self.layer_idx = layer_idx
        self.hidden_size = config.hidden_size
        self.gate = TopKRouter(config)
        self.experts = expert_factory(layer_idx)
        if not isinstance(self.experts, HBMExpertBank):
            raise ContractError(
                f"sparse layer {layer_idx} must be backed by an HBM expert bank, got "
                f"{type(self.experts).__name__}")
        self.shared_experts = DenseMLP(
            config.hidden_size,
            config.moe_intermediate_size * config.n_shared_experts,
            config.swiglu_limit,
        )
        self.last_weights: torch.Tensor | None = None
        self.last_indices: torch.Tensor | None = None
        self._workspace: torch.Tensor | None = None

    def _workspace_for(self, T: int, device) -> torch.Tensor:
        cfg = self.config
        need = N.workspace_bytes(T, cfg.hidden_size, cfg.n_routed_experts,
                                 cfg.num_experts_per_tok, cfg.moe_intermediate_size,
                                 self.shared_experts.intermediate_size)
        ws = self._workspace
        if ws is None or ws.numel() < need or ws.device != device:
            ws = torch.empty(max(need, 256), dtype=torch.uint8, device=device)
            N.call("glm_moe_workspace_init", N.stream_of(ws), ws.data_ptr(), ws.numel())
            self._workspace = ws
        return ws

    def __call__(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return self._forward(hidden_states, None)

    def with_hyper_residual(self, hidden_states: torch.Tensor, residual: torch.Tensor,
                            post: torch.Tensor, comb: torch.Tensor,
                            bf16_streams: bool = False) -> torch.Tensor:
        """The layer followed by the FFN site's ``hyper_residual(residual, y,
        post, comb)`` (``mhc.py:51-60``) in one library call
        (``glm_moe_forward_hc``); ``residual`` f32 ``[T, hc, d]``."""
        return self._forward(hidden_states, (residual, post, comb, bf16_streams))

    def _forward(self, hidden_states: torch.Tensor, hc) -> torch.Tensor:
        cfg = self.config
        d = self.hidden_size
        original_shape = hidden_states.shape
        N.require_device(hidden_states, "hidden_states", (torch.bfloat16,))
        rows = hidden_states.reshape(-1, d)
        T = rows.shape[0]
        dev = rows.device
        rw, rb = self.gate._params()
        bank = self.experts
        bank._require_active()
        shared = self.shared_experts
        fmt = shared.fused_format()
        if fmt is None:
            raise ContractError("shared expert projections must share one storage format")
        sg = require_weight(shared.gate_proj.weight, "shared gate_proj.weight")
        su = require_weight(shared.up_proj.weight, "shared up_proj.weight")
        sd = require_weight(shared.down_proj.weight, "shared down_proj.weight")
        k = cfg.num_experts_per_tok
        out = torch.empty((T, d), dtype=torch.float32, device=dev)
        weights = torch.empty((T, k), dtype=torch.float32, device=dev)
        indices = torch.empty((T, k), dtype=torch.int32, device=dev)
        hc_args, hc_out = (), None
        if hc is not None:
            residual, post, comb, bf16_streams = hc
            N.require_device(residual, "residual", (torch.float32,))
            hcm = residual.shape[-2]
            if residual.numel() != T * hcm * d or post.numel() != T * hcm or \
                    comb.numel() != T * hcm * hcm:
                raise ContractError("residual, post and comb do not match the layer's tokens")
            N.require_device(post, "post", (torch.float32,))
            N.require_device(comb, "comb", (torch.float32,))
            hc_out = torch.empty((T, hcm, d), dtype=torch.float32, device=dev)
            hc_args = (residual.data_ptr(), hcm, post.data_ptr(), comb.data_ptr(),
                       N.native.GLM_HC_BF16_STREAMS if bf16_streams else 0, hc_out.data_ptr())
        if T == 0:  # an empty batch: empty results, nothing to launch
            self.last_weights = weights
            self.last_indices = indices
            return out.reshape(original_shape) if hc is None else hc_out
        ws = self._workspace_for(T, dev)
        gw, gs = bank.projection("gate_proj")
        uw, us = bank.projection("up_proj")
        dw, ds = bank.projection("down_proj")
        N.call("glm_moe_forward" if hc is None else "glm_moe_forward_hc",
               N.stream_of(rows), rows.data_ptr(), T, d, rw.data_ptr(),
               rb.data_ptr(), cfg.n_routed_experts, k, cfg.n_group, cfg.topk_group,
               int(cfg.norm_topk_prob), float(cfg.routed_scaling_factor),
               cfg.moe_intermediate_size, gw.data_ptr(), gs.data_ptr(), uw.data_ptr(),
               us.data_ptr(), dw.data_ptr(), ds.data_ptr(), shared.intermediate_size, fmt,
               sg.data_ptr(), N.ptr(shared.gate_proj.scales), su.data_ptr(),
               N.ptr(shared.up_proj.scales), sd.data_ptr(), N.ptr(shared.down_proj.scales), None,
               float(cfg.swiglu_limit), ws.data_ptr(), ws.numel(), out.data_ptr(),
               weights.data_ptr(), indices.data_ptr(), *hc_args)
        self.last_weights = weights
        self.last_indices = indices
        return out.reshape(original_shape) if hc is None else hc_out

    @property
    def last_route(self) -> tuple[int, ...]:
        """Flattened routed ids of the last call (synchronises with the device),
        the reference's ``last_route`` (``moe.py:179,200``)."""
        if self.last_indices is None:
            return ()
        return tuple(int(v) for v in self.last_indices.reshape(-1).tolist())
