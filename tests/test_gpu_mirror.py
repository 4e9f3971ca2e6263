"""GPU checks of the Python mirror of the reference's MoE interface
(``src/glm53flash``) against the CPU oracle: router, expert bank, shared MLP,
resident MXFP8/MXFP4 linears and the whole ``ExpertSSDMoE`` layer."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O
from livglm_amd.workloads import BANK_KEYS, SHAPES, make_layer

pytestmark = pytest.mark.gpu

REL_L2 = 2e-3


@pytest.fixture(scope="module")
def gu():
    import gpu_util
    return gpu_util


def _config(shape):
    from glm53flash.model_config import GLMTextConfig
    return GLMTextConfig.from_model_dict({"text_config": {
        "hidden_size": shape.d, "moe_intermediate_size": shape.I,
        "n_routed_experts": shape.E, "num_experts_per_tok": shape.k,
        "n_shared_experts": shape.I_shared // shape.I, "n_group": shape.n_group,
        "topk_group": shape.topk_group, "norm_topk_prob": True,
        "routed_scaling_factor": shape.routed_scaling_factor,
        "swiglu_limit": shape.swiglu_limit}})


def _moe(gu, shape, layer):
    from glm53flash.expert_ssd import HBMExpertBank
    from glm53flash.moe import ExpertSSDMoE
    cfg = _config(shape)
    moe = ExpertSSDMoE(cfg, 1, lambda i: HBMExpertBank(
        layer=i, num_experts=shape.E, hidden_size=shape.d, intermediate_size=shape.I,
        swiglu_limit=shape.swiglu_limit, device="cuda"))
    dl = gu.upload_layer(layer, bank_layout=False)  # load_bank takes checkpoint bytes
    moe.gate.weight = dl["router_weight"]
    moe.gate.e_score_correction_bias = dl["router_bias"]
    moe.shared_experts.gate_proj.weight = dl["shared.gate"]
    moe.shared_experts.up_proj.weight = dl["shared.up"]
    moe.shared_experts.down_proj.weight = dl["shared.down"]
    moe.experts.load_bank({key: dl[key] for key in BANK_KEYS})
    return moe, dl


def _oracle(layer, shape):
    x = O.bf16_bits_to_f32(layer["x"])
    sw = tuple(O.bf16_bits_to_f32(layer[k]) for k in ("shared.gate", "shared.up", "shared.down"))
    return O.moe_layer(x, layer["router_weight"], layer["router_bias"],
                       O.Bank(*(layer[k] for k in BANK_KEYS)), sw, top_k=shape.k,
                       n_group=shape.n_group, topk_group=shape.topk_group, norm_topk_prob=True,
                       routed_scaling_factor=shape.routed_scaling_factor,
                       swiglu_limit=shape.swiglu_limit, return_intermediates=True)


@pytest.mark.parametrize("name", ["decode_t1", "verify_t2", "batch_t64"])
def test_expert_ssd_moe_layer(gu, name):
    import torch
    shape = SHAPES[name]
    layer = make_layer(shape, 7100 + shape.T)
    moe, dl = _moe(gu, shape, layer)
    want, inter = _oracle(layer, shape)
    x = dl["x"].reshape(1, shape.T, shape.d)  # leading batch dim, as a decoder layer passes it
    out = moe(x)
    assert out.dtype == torch.float32 and tuple(out.shape) == (1, shape.T, shape.d)
    assert O.rel_l2(gu.host(out).reshape(shape.T, shape.d), want) < REL_L2
    assert moe.last_route == tuple(int(v) for v in inter["indices"].reshape(-1))
    # a second call reuses the cached workspace
    out2 = moe(x)
    assert np.array_equal(gu.host(out).view(np.uint32), gu.host(out2).view(np.uint32))


def test_router_and_bank_call(gu):
    shape = SHAPES["verify_t2"]
    layer = make_layer(shape, 7200)
    moe, dl = _moe(gu, shape, layer)
    x = O.bf16_bits_to_f32(layer["x"])
    logits_w, w_w, idx_w, _ = O.router(x, layer["router_weight"], layer["router_bias"],
                                       top_k=shape.k, n_group=1, topk_group=1,
                                       norm_topk_prob=True, routed_scaling_factor=2.5)
    logits, w, idx = moe.gate(dl["x"])
    assert np.array_equal(gu.host(idx).astype(np.uint32), idx_w)
    np.testing.assert_allclose(gu.host(w), w_w, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(gu.host(logits), logits_w, rtol=1e-4, atol=1e-5)
    # backend call: [T, k, d] bf16 in route order (expert_ssd.py:185-188)
    y = moe.experts(dl["x"], idx)
    y_want = O.routed_experts(x, idx_w, O.Bank(*(layer[k] for k in BANK_KEYS)),
                              shape.swiglu_limit)
    assert tuple(y.shape) == (shape.T, shape.k, shape.d)
    assert O.rel_l2(O.bf16_bits_to_f32(gu.bf16_bits(y)), y_want) < REL_L2
    assert moe.experts.last_expert_ids == tuple(int(v) for v in idx_w.reshape(-1))
    plan = moe.experts.prepare(idx)
    plan.check(shape.E)


def test_bank_rejects_out_of_range_ids(gu):
    import torch
    from glm53flash.contract import ContractError
    shape = SHAPES["decode_t1"]
    moe, dl = _moe(gu, shape, make_layer(shape, 7300))
    plan = moe.experts.prepare(torch.tensor([[1, shape.E + 3]], dtype=torch.int32, device="cuda"))
    with pytest.raises(ContractError):
        plan.check(shape.E)


@pytest.mark.parametrize("bits,seed,rtol,atol", [(8, 5308, 0.03, 0.015), (4, 5304, 0.20, 0.04)])
def test_resident_mx_reference_case(gu, bits, seed, rtol, atol):
    # the reference's own case (tests/test_resident_mxfp8.py:7-52): same seeds,
    # shapes, distributions, byte counts and tolerances
    from glm53flash.layers import DeferredLinear
    rng = np.random.default_rng(seed)
    w = O.f32_to_bf16_bits(rng.normal(0, 0.05, (64, 32)).astype(np.float32))
    v = O.f32_to_bf16_bits(rng.normal(0, 0.2, (2, 32)).astype(np.float32))
    lin = DeferredLinear(32, 64)
    lin.weight = gu.to_dev(w)
    expected = O.bf16_bits_to_f32(gu.bf16_bits(lin(gu.to_dev(v))))
    src, dst = lin.quantize_to_mxfp(bits)
    assert src == 64 * 32 * 2
    assert dst == (64 * 32 if bits == 8 else 64 * 16) + 64
    assert dst < src and lin.quantization_mode == f"mxfp{bits}"
    actual = O.bf16_bits_to_f32(gu.bf16_bits(lin(gu.to_dev(v))))
    np.testing.assert_allclose(actual, expected, rtol=rtol, atol=atol)


@pytest.mark.parametrize("bits", [8, 4])
def test_deferred_linear_resident_mx(gu, bits):
    # a 2048x2048 resident linear: codes/scales bit-exact, output within the
    # bf16 bar of the oracle, and the quantisation error of the nearest scale
    # rule (it saturates the largest elements of ~1.6 % of MXFP8 groups)
    from glm53flash.layers import DeferredLinear
    rng = np.random.default_rng(5308 if bits == 8 else 5304)
    out_f, in_f, T = 2048, 2048, 3
    w = O.f32_to_bf16_bits(rng.normal(0, 0.02, (out_f, in_f)).astype(np.float32))
    x = O.f32_to_bf16_bits(rng.normal(0, 1, (T, in_f)).astype(np.float32))
    lin = DeferredLinear(in_f, out_f)
    lin.weight = gu.to_dev(w)
    dense = O.bf16_bits_to_f32(gu.bf16_bits(lin(gu.to_dev(x))))
    src, dst = lin.quantize_to_mxfp(bits)
    assert src == out_f * in_f * 2
    assert dst == out_f * in_f * bits // 8 + out_f * in_f // 32
    got = O.bf16_bits_to_f32(gu.bf16_bits(lin(gu.to_dev(x))))
    codes, scales = O.quantize_mx(w, bits, O.MX_RULE_NEAREST)
    assert np.array_equal(gu.host(lin.weight), codes) and np.array_equal(gu.host(lin.scales), scales)
    deq = O.dequant_mxfp8(codes, scales) if bits == 8 else O.dequant_mxfp4(codes, scales)
    want = O.linear_bf16(O.bf16_bits_to_f32(x), deq)
    assert O.rel_l2(got, want) < REL_L2
    assert O.rel_l2(got, dense) < (0.07 if bits == 8 else 0.15)


def test_dense_mlp_and_swiglu_wrappers(gu):
    from glm53flash.expert_ssd import limited_swiglu
    from glm53flash.layers import DenseMLP
    rng = np.random.default_rng(41)
    d, I, T = 1024, 512, 2
    ws = [O.f32_to_bf16_bits(rng.normal(0, 0.02, s).astype(np.float32))
          for s in [(I, d), (I, d), (d, I)]]
    x = O.f32_to_bf16_bits(rng.normal(0, 1, (T, d)).astype(np.float32))
    mlp = DenseMLP(d, I, 10.0)
    mlp.gate_proj.weight, mlp.up_proj.weight, mlp.down_proj.weight = (gu.to_dev(w) for w in ws)
    got = O.bf16_bits_to_f32(gu.bf16_bits(mlp(gu.to_dev(x))))
    want = O.dense_mlp(O.bf16_bits_to_f32(x), *(O.bf16_bits_to_f32(w) for w in ws), 10.0)
    assert O.rel_l2(got, want) < REL_L2
    g = O.f32_to_bf16_bits(rng.uniform(9, 10, 4096).astype(np.float32))
    u = O.f32_to_bf16_bits(rng.normal(0, 3, 4096).astype(np.float32))
    h = gu.bf16_bits(limited_swiglu(gu.to_dev(g), gu.to_dev(u), 10.0))
    want_h = O.f32_to_bf16_bits(O.limited_swiglu_bf16(O.bf16_bits_to_f32(g),
                                                      O.bf16_bits_to_f32(u), 10.0))
    assert np.array_equal(h, want_h)


def test_expert_ssd_moe_empty_batch(gu):
    # an empty token batch returns an empty f32 result of the input's shape
    import torch
    shape = SHAPES["verify_t2"]
    moe, dl = _moe(gu, shape, make_layer(shape, 7400))
    x = torch.empty((1, 0, shape.d), dtype=torch.bfloat16, device="cuda")
    out = moe(x)
    assert out.dtype == torch.float32 and tuple(out.shape) == (1, 0, shape.d)
    assert moe.last_route == ()
