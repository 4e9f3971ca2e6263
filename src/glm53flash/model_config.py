"""GLM text configuration (subset that the routed-MoE layer reads).

Mirrors ``GLMTextConfig`` of the reference (``model_config.py:11-54``): the
MoE fields keep their names and meaning; the attention/mHC fields are kept with
neutral defaults so that configurations written for the reference construct
unchanged, but nothing here reads them.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any

from .contract import ContractError


@dataclass(frozen=True)
class GLMTextConfig:
    hidden_size: int = 4096
    moe_intermediate_size: int = 2048
    n_routed_experts: int = 288
    num_experts_per_tok: int = 8
    n_shared_experts: int = 1
    n_group: int = 1
    topk_group: int = 1
    norm_topk_prob: bool = True
    routed_scaling_factor: float = 2.5
    swiglu_limit: float = 10.0
    hidden_act: str = "silu"
    scoring_func: str = "sigmoid"
    topk_method: str = "noaux_tc"
    # Fields the MoE layer does not read (kept for drop-in construction).
    vocab_size: int = 0
    intermediate_size: int = 0
    num_hidden_layers: int = 0
    first_k_dense_replace: int = 0
    layer_types: tuple[str, ...] = ()
    mlp_layer_types: tuple[str, ...] = ()
    rms_norm_eps: float = 1e-6
    hc_mult: int = 1
    hc_sinkhorn_iters: int = 1
    hc_eps: float = 1e-6
    num_attention_heads: int = 1
    num_key_value_heads: int = 1
    q_lora_rank: int = 0
    kv_lora_rank: int = 0
    qk_nope_head_dim: int = 0
    qk_rope_head_dim: int = 0
    v_head_dim: int = 0
    linear_num_heads: int = 0
    linear_head_dim: int = 0
    linear_conv_kernel: int = 1
    linear_gate_lower_bound: float | None = None
    index_n_heads: int = 0
    index_head_dim: int = 0
    index_topk: int = 1
    index_kpool: int = 1
    index_kpool_always_select_tail: bool = True
    eos_token_ids: tuple[int, ...] = field(default_factory=tuple)
    pad_token_id: int = 0
    max_position_embeddings: int = 0

    @classmethod
    def from_model_dict(cls, config: dict[str, Any]) -> "GLMTextConfig":
        """Reads the MoE fields of a checkpoint ``config.json`` (``text_config``
        object, as ``model_config.py:56-140`` does) and validates them."""
        text = config.get("text_config", config)
        if not isinstance(text, dict):
            raise ContractError("config has no text_config object")

        def integer(key: str) -> int:
            value = text.get(key)
            if isinstance(value, bool) or not isinstance(value, int):
                raise ContractError(f"configuration field must be an integer: {key}")
            return value

        def number(key: str) -> float:
            value = text.get(key)
            if isinstance(value, bool) or not isinstance(value, (int, float)):
                raise ContractError(f"configuration field must be numeric: {key}")
            return float(value)

        result = cls(
            hidden_size=integer("hidden_size"),
            moe_intermediate_size=integer("moe_intermediate_size"),
            n_routed_experts=integer("n_routed_experts"),
            num_experts_per_tok=integer("num_experts_per_tok"),
            n_shared_experts=integer("n_shared_experts"),
            n_group=integer("n_group"),
            topk_group=integer("topk_group"),
            norm_topk_prob=bool(text.get("norm_topk_prob", True)),
            routed_scaling_factor=number("routed_scaling_factor"),
            swiglu_limit=float(text.get("swiglu_limit", 0.0) or 0.0),
            hidden_act=str(text.get("hidden_act", "silu")),
            scoring_func=str(text.get("scoring_func", "sigmoid")),
            topk_method=str(text.get("topk_method", "noaux_tc")),
            # the decoder FFN site's hyper-connection and norm (model_config.py:102-105);
            # optional here, so that MoE-only configs stay valid
            rms_norm_eps=float(text.get("rms_norm_eps", 1e-6)),
            hc_mult=int(text.get("hc_mult", 1)),
            hc_sinkhorn_iters=int(text.get("hc_sinkhorn_iters", 1)),
            hc_eps=float(text.get("hc_eps", 1e-6)),
        )
        result.validate()
        return result

    def validate(self) -> None:
        """The MoE subset of ``GLMTextConfig.validate`` (``model_config.py:142-176``)."""
        if self.hidden_act != "silu":
            raise ContractError(f"only SiLU is supported, got {self.hidden_act!r}")
        if self.scoring_func != "sigmoid" or self.topk_method != "noaux_tc":
            raise ContractError("only sigmoid/noaux_tc routing is supported")
        if not 1 <= self.num_experts_per_tok <= self.n_routed_experts:
            raise ContractError("invalid routed top-k geometry")
        if self.n_group < 1 or self.n_routed_experts % self.n_group:
            raise ContractError("expert count must be divisible by n_group")
        if not 1 <= self.topk_group <= self.n_group:
            raise ContractError("invalid topk_group")
        if self.n_routed_experts // self.n_group < 2:
            raise ContractError("router groups must contain at least two experts")
        if self.hidden_size % 32 or self.moe_intermediate_size % 32:
            raise ContractError("group-32 MX experts need hidden and intermediate sizes % 32 == 0")
        if self.hc_mult < 1 or self.hc_sinkhorn_iters < 1:
            raise ContractError("hyper-connection settings must be positive")
