"""CPU checks of the Python mirror of the reference's MoE interface
(``src/glm53flash``): configuration parsing, the backend gate, deferred
weights and the bank's bookkeeping.  Nothing here launches a kernel."""

from __future__ import annotations

import pytest

from glm53flash.contract import ContractError
from glm53flash.expert_ssd import ExpertSSD, HBMExpertBank, NativeExpertSSD
from glm53flash.layers import DeferredLinear, DenseMLP, require_weight
from glm53flash.model_config import GLMTextConfig
from glm53flash.moe import ExpertSSDMoE, TopKRouter

SMALL = {
    "hidden_size": 1024, "moe_intermediate_size": 512, "n_routed_experts": 16,
    "num_experts_per_tok": 2, "n_shared_experts": 1, "n_group": 1, "topk_group": 1,
    "norm_topk_prob": True, "routed_scaling_factor": 2.5, "swiglu_limit": 10.0,
}


def test_config_from_model_dict_reads_text_config():
    cfg = GLMTextConfig.from_model_dict({"text_config": dict(SMALL)})
    assert (cfg.hidden_size, cfg.n_routed_experts, cfg.num_experts_per_tok) == (1024, 16, 2)
    assert cfg.routed_scaling_factor == 2.5 and cfg.swiglu_limit == 10.0
    assert GLMTextConfig.from_model_dict(dict(SMALL)) == cfg


@pytest.mark.parametrize("key,value", [("hidden_size", "1024"), ("n_group", True),
                                       ("routed_scaling_factor", "2.5")])
def test_config_rejects_mistyped_fields(key, value):
    bad = dict(SMALL, **{key: value})
    with pytest.raises(ContractError):
        GLMTextConfig.from_model_dict(bad)


@pytest.mark.parametrize("change", [{"n_group": 3}, {"topk_group": 2}, {"num_experts_per_tok": 17},
                                    {"hidden_size": 1000}, {"hidden_act": "gelu"},
                                    {"n_group": 16, "topk_group": 1}])
def test_config_validation(change):
    with pytest.raises(ContractError):
        GLMTextConfig(**dict(SMALL, **change)).validate()


def _bank(layer=0, defer=True):
    return HBMExpertBank(layer=layer, num_experts=16, hidden_size=1024, intermediate_size=512,
                         swiglu_limit=10.0, defer_slots=defer)


def test_moe_rejects_a_backend_that_is_not_an_expert_bank():
    # the reference's MoE only accepts its ExpertSSD backends (moe.py:84-88)
    cfg = GLMTextConfig(**SMALL)
    with pytest.raises(ContractError):
        ExpertSSDMoE(cfg, 3, lambda layer: object())
    moe = ExpertSSDMoE(cfg, 3, lambda layer: _bank(layer))
    assert moe.experts.layer == 3 and moe.last_route == ()
    assert NativeExpertSSD is HBMExpertBank and ExpertSSD is HBMExpertBank


def test_unloaded_weights_raise():
    cfg = GLMTextConfig(**SMALL)
    with pytest.raises(ContractError, match="router.weight"):
        TopKRouter(cfg)._params()
    with pytest.raises(ContractError):
        require_weight(None, "w")
    lin = DeferredLinear(64, 32)
    with pytest.raises(ContractError):
        lin.quantize_to_mxfp8()
    mlp = DenseMLP(64, 32, 10.0)
    assert mlp.fused_format() == 0  # three bf16 projections fuse


def test_deferred_linear_quantisation_guards():
    lin = DeferredLinear(64, 32, quantize_resident=False)
    with pytest.raises(ContractError):
        lin.quantize_to_mxfp8()
    with pytest.raises(ContractError):
        DeferredLinear(64, 32).quantize_to_mxfp(6)


def test_bank_shapes_and_lifecycle():
    bank = _bank()
    shapes = bank.shapes()
    assert shapes["gate_proj.weight_packed"] == (16, 512, 512)
    assert shapes["gate_proj.weight_scale"] == (16, 512, 32)
    assert shapes["down_proj.weight_packed"] == (16, 1024, 256)
    assert shapes["down_proj.weight_scale"] == (16, 1024, 16)
    # one expert record: 3 projections x (I*d/2 codes + I*d/32 scales) = 3*I*d*17/32
    assert bank.expert_bytes == 3 * 512 * 1024 * 17 // 32 == 835_584
    real = HBMExpertBank(layer=0, num_experts=288, hidden_size=4096, intermediate_size=2048,
                         swiglu_limit=10.0, defer_slots=True)
    assert real.expert_bytes == 13_369_344  # the reference's record size (expert_source.py:370)
    st = bank.stats()
    assert (st.capacity, st.resident, st.misses, st.evictions) == (16, 0, 0, 0)
    assert bank.resident_experts == () and bank.last_expert_ids == ()
    with pytest.raises(RuntimeError):
        bank._require_active()
    bank.close()
    with pytest.raises(RuntimeError):
        bank.activate()


def test_bank_rejects_bad_geometry():
    with pytest.raises(ContractError):
        HBMExpertBank(layer=0, num_experts=0, hidden_size=1024, intermediate_size=512,
                      swiglu_limit=10.0, defer_slots=True)
    with pytest.raises(ContractError):
        HBMExpertBank(layer=0, num_experts=4, hidden_size=1000, intermediate_size=512,
                      swiglu_limit=10.0, defer_slots=True)
