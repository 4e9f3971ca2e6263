"""The decoder FFN site on the GPU against the CPU oracle: the hyper-connection
(``glm_hc_pre``), ``hyper_residual`` (``glm_hc_post``), RMSNorm
(``glm_rms_norm``), their Python mirror, and the whole site around the MoE
layer (``model.py:132-136``).

Tolerances: f32 outputs (post, comb, collapsed, residual update) within 2e-5
relative of the oracle, whose dot products are exact and rounded once (the
kernels sum in f32 in another order); bf16 outputs at most one bf16 ulp apart
and 99 % identical; the site's f32 output rel-L2 < 2e-3 (the MoE layer's bar).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import mhc_oracle as H
from oracle import moe_oracle as O
from livglm_amd.workloads import BANK_KEYS, SHAPES, make_hc, make_layer

pytestmark = pytest.mark.gpu

REL_L2 = 2e-3


@pytest.fixture(scope="module")
def gu():
    import gpu_util
    return gpu_util


def _bf16_close(got_bits, want_f32):
    want = O.f32_to_bf16_bits(want_f32).astype(np.int32)
    got = got_bits.astype(np.int32)
    diff = np.abs(got - want)
    assert diff.max() <= 1, f"bf16 outputs differ by {diff.max()} ulp"
    assert np.mean(diff == 0) >= 0.99


def _hc_pre(gu, h, hc, d, iters, *, norm=True, bf16=False, rms_eps=1e-6, hc_eps=1e-6,
            norm_eps=1e-5):
    import torch
    T = h["streams"].shape[0]
    lib = gu.native.load()
    ws_bytes = int(lib.glm_hc_workspace_bytes(T, hc, d))
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device="cuda")
    post = torch.empty((T, hc), dtype=torch.float32, device="cuda")
    comb = torch.empty((T, hc, hc), dtype=torch.float32, device="cuda")
    collapsed = torch.empty((T, d), dtype=torch.float32, device="cuda")
    normed = torch.empty((T, d), dtype=torch.bfloat16, device="cuda") if norm else None
    flags = gu.native.GLM_HC_BF16_STREAMS if bf16 else 0
    gu.call("glm_hc_pre", gu.stream(), gu.p(gu.to_dev(h["streams"])), T, hc, d,
            gu.p(gu.to_dev(h["fn"])), gu.p(gu.to_dev(h["base"])), gu.p(gu.to_dev(h["scale"])),
            iters, rms_eps, hc_eps, gu.p(gu.to_dev(h["norm_weight"])) if norm else None,
            norm_eps, flags, gu.p(ws), ws.numel(), gu.p(post), gu.p(comb), gu.p(collapsed),
            gu.p(normed))
    return (gu.host(post), gu.host(comb), gu.host(collapsed),
            gu.bf16_bits(normed) if norm else None)


@pytest.mark.parametrize("T,hc,d,iters,bf16", [
    (1, 4, 2048, 20, False), (2, 4, 2048, 20, False), (2, 4, 4096, 20, False),
    (5, 2, 256, 3, False), (3, 4, 1024, 20, True), (2, 8, 512, 5, False), (9, 1, 64, 1, False),
    # hc = 3: the mixing-matrix sums through LDS (hc not a power of two);
    # hc d = 32768: 128 column chunks over 64 workgroups
    (2, 3, 512, 4, False), (3, 8, 4096, 6, False),
])
def test_hc_pre_matches_oracle(gu, T, hc, d, iters, bf16):
    print(f"hc_pre T={T} hc={hc} d={d} iters={iters} bf16={bf16}", flush=True)
    h = make_hc(T, hc, d, 5400 + T * 7 + hc, bf16_streams=bf16)
    post, comb, collapsed, normed = _hc_pre(gu, h, hc, d, iters, bf16=bf16)
    wpost, wcomb, wcol = H.hyper_connection(h["streams"], h["fn"], h["base"], h["scale"],
                                            sinkhorn_iters=iters, rms_eps=1e-6, hc_eps=1e-6,
                                            bf16_streams=bf16)
    np.testing.assert_allclose(post, wpost, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(comb, wcomb, rtol=2e-5, atol=2e-6)
    if bf16:
        _bf16_close(O.f32_to_bf16_bits(collapsed), wcol)
    else:
        np.testing.assert_allclose(collapsed, wcol, rtol=2e-5, atol=2e-5)
    # the fused post-attention norm, from the kernel's own collapsed row
    _bf16_close(normed, H.rms_norm(collapsed, h["norm_weight"], 1e-5))
    # unweighted, and without the norm output
    post2, comb2, col2, none = _hc_pre(gu, h, hc, d, iters, norm=False, bf16=bf16)
    assert none is None
    np.testing.assert_array_equal(post2, post)
    np.testing.assert_array_equal(col2, collapsed)


@pytest.mark.parametrize("bf16", [False, True])
def test_hc_post_matches_oracle(gu, bf16):
    import torch
    T, hc, d = 3, 4, 2048
    print(f"hc_post T={T} hc={hc} d={d} bf16={bf16}", flush=True)
    h = make_hc(T, hc, d, 5500 + bf16, bf16_streams=bf16)
    post, comb, _ = H.hyper_connection(h["streams"], h["fn"], h["base"], h["scale"],
                                       sinkhorn_iters=20, rms_eps=1e-6, hc_eps=1e-6)
    y = np.random.default_rng(5501).standard_normal((T, d)).astype(np.float32)
    out = torch.empty((T, hc, d), dtype=torch.float32, device="cuda")
    flags = gu.native.GLM_HC_BF16_STREAMS if bf16 else 0
    gu.call("glm_hc_post", gu.stream(), gu.p(gu.to_dev(h["streams"])), T, hc, d,
            gu.p(gu.to_dev(y)), gu.p(gu.to_dev(post)), gu.p(gu.to_dev(comb)), flags, gu.p(out))
    want = H.hyper_residual(h["streams"], y, post, comb, bf16_streams=bf16)
    got = gu.host(out)
    if bf16:
        # the bf16 mixing sum may round one bf16 ulp apart; the f32 placement
        # is the same product in both
        mixed = H.hyper_residual(h["streams"], np.zeros_like(y), post, comb, bf16_streams=True)
        assert np.all(np.abs(got - want) <= np.abs(mixed) * 2.0 ** -7 + 1e-6)
        assert np.mean(got == want) >= 0.98
    else:
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)


def test_rms_norm_matches_oracle(gu):
    import torch
    T, d = 5, 2048
    rng = np.random.default_rng(5600)
    x = (rng.standard_normal((T, d)) * 3).astype(np.float32)
    w = rng.normal(1.0, 0.1, d).astype(np.float32)
    for weight in (w, None):
        out = torch.empty((T, d), dtype=torch.float32, device="cuda")
        out16 = torch.empty((T, d), dtype=torch.bfloat16, device="cuda")
        gu.call("glm_rms_norm", gu.stream(), gu.p(gu.to_dev(x)), T, d,
                None if weight is None else gu.p(gu.to_dev(weight)), 1e-6, gu.p(out), gu.p(out16))
        want = H.rms_norm(x, weight, 1e-6)
        np.testing.assert_allclose(gu.host(out), want, rtol=2e-6, atol=1e-7)
        _bf16_close(gu.bf16_bits(out16), want)


def _ffn(gu, shape, layer, h, hc, iters):
    import torch

    from glm53flash.expert_ssd import HBMExpertBank
    from glm53flash.model import MoEDecoderFFN
    from glm53flash.model_config import GLMTextConfig
    cfg = GLMTextConfig.from_model_dict({"text_config": {
        "hidden_size": shape.d, "moe_intermediate_size": shape.I,
        "n_routed_experts": shape.E, "num_experts_per_tok": shape.k,
        "n_shared_experts": shape.I_shared // shape.I, "n_group": shape.n_group,
        "topk_group": shape.topk_group, "norm_topk_prob": True,
        "routed_scaling_factor": shape.routed_scaling_factor,
        "swiglu_limit": shape.swiglu_limit, "hc_mult": hc, "hc_sinkhorn_iters": iters,
        "hc_eps": 1e-6, "rms_norm_eps": 1e-6}})
    site = MoEDecoderFFN(cfg, 3, lambda i: HBMExpertBank(
        layer=i, num_experts=shape.E, hidden_size=shape.d, intermediate_size=shape.I,
        swiglu_limit=shape.swiglu_limit, device="cuda"))
    dl = gu.upload_layer(layer, bank_layout=False)  # load_bank takes checkpoint bytes
    moe = site.mlp
    moe.gate.weight = dl["router_weight"]
    moe.gate.e_score_correction_bias = dl["router_bias"]
    moe.shared_experts.gate_proj.weight = dl["shared.gate"]
    moe.shared_experts.up_proj.weight = dl["shared.up"]
    moe.shared_experts.down_proj.weight = dl["shared.down"]
    moe.experts.load_bank({key: dl[key] for key in BANK_KEYS})
    site.ffn_hc.fn = gu.to_dev(h["fn"])
    site.ffn_hc.base = gu.to_dev(h["base"])
    site.ffn_hc.scale = gu.to_dev(h["scale"])
    site.post_attention_layernorm.weight = gu.to_dev(h["norm_weight"]).to(torch.bfloat16)
    return site


@pytest.mark.parametrize("bf16", [False, True])
def test_moe_ffn_site_matches_oracle(gu, bf16):
    import torch
    shape = SHAPES["verify_t2"]
    hc, iters = 4, 20
    print(f"ffn site verify_t2 hc={hc} bf16={bf16}", flush=True)
    layer = make_layer(shape, 5700 + bf16)
    h = make_hc(shape.T, hc, shape.d, 5701 + bf16, bf16_streams=bf16)
    site = _ffn(gu, shape, layer, h, hc, iters)
    streams = gu.to_dev(h["streams"]).reshape(1, shape.T, hc, shape.d)
    if bf16:
        streams = streams.to(torch.bfloat16)
    out = site(streams)
    assert out.dtype == torch.float32 and tuple(out.shape) == (1, shape.T, hc, shape.d)
    sw = tuple(O.bf16_bits_to_f32(layer[k]) for k in ("shared.gate", "shared.up", "shared.down"))
    moe_args = ((layer["router_weight"], layer["router_bias"],
                 O.Bank(*(layer[k] for k in BANK_KEYS)), sw),
                dict(top_k=shape.k, n_group=shape.n_group, topk_group=shape.topk_group,
                     norm_topk_prob=True, routed_scaling_factor=shape.routed_scaling_factor,
                     swiglu_limit=shape.swiglu_limit))
    want, inter = H.ffn_site(h["streams"], (h["fn"], h["base"], h["scale"]), h["norm_weight"],
                             moe_args, sinkhorn_iters=iters, rms_eps=1e-6, hc_eps=1e-6,
                             norm_eps=1e-6, bf16_streams=bf16)
    got = gu.host(out).reshape(shape.T, hc, shape.d)
    assert O.rel_l2(got, want) < REL_L2
    # the MoE's contribution alone (out minus the residual mixing) also meets the bar
    mix = H.hyper_residual(h["streams"], np.zeros((shape.T, shape.d), np.float32),
                           inter["post"], inter["comb"], bf16_streams=bf16)
    assert O.rel_l2(got - mix, want - mix) < REL_L2
    # the route equals the oracle's on every token whose top-k margin is clear
    # (the kernel's normalised input may differ from the oracle's by a bf16 ulp)
    _, _, idx, masked = O.router(inter["normed"], layer["router_weight"], layer["router_bias"],
                                 top_k=shape.k, n_group=1, topk_group=1, norm_topk_prob=True,
                                 routed_scaling_factor=shape.routed_scaling_factor)
    margin = O.topk_margin(masked, shape.k)
    got_idx = np.array(site.mlp.last_route, dtype=np.int64).reshape(shape.T, shape.k)
    for t in range(shape.T):
        if margin[t] > 1e-4:
            assert np.array_equal(got_idx[t], idx[t].astype(np.int64)), t
    # the Python pieces on their own: HyperConnection, RMSNorm, hyper_residual
    post, comb, collapsed = site.ffn_hc(streams)
    assert collapsed.dtype == streams.dtype
    np.testing.assert_allclose(gu.host(post).reshape(shape.T, hc), inter["post"], rtol=2e-5,
                               atol=2e-6)
    normed = site.post_attention_layernorm(collapsed.reshape(shape.T, shape.d).float())
    np.testing.assert_allclose(
        gu.host(normed), H.rms_norm(gu.host(collapsed.float()).reshape(shape.T, shape.d),
                                    h["norm_weight"], 1e-6), rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("name,T,bf16,hc", [("verify_t2", 2, False, 4), ("verify_t2", 2, True, 4),
                                            ("verify_t2", 20, False, 4), ("decode_t1", 1, False, 4),
                                            ("decode_t1", 3, False, 8)])
def test_moe_forward_hc_equals_forward_then_hc_post(gu, name, T, bf16, hc):
    """glm_moe_forward_hc (the update inside the layer's last kernel at T <= 4,
    a separate launch at T = 20) is bit-identical to glm_moe_forward followed
    by glm_hc_post; decode_t1 runs the fused kernel with k = 2 (256 threads)."""
    import torch
    shape = SHAPES[name]
    print(f"moe_forward_hc {name} T={T} bf16={bf16} hc={hc}", flush=True)
    layer = make_layer(shape, 5800 + T + bf16, T=T)
    dl = gu.upload_layer(layer)
    h = make_hc(T, hc, shape.d, 5801 + T, bf16_streams=bf16)
    post, comb, _ = H.hyper_connection(h["streams"], h["fn"], h["base"], h["scale"],
                                       sinkhorn_iters=20, rms_eps=1e-6, hc_eps=1e-6)
    res, post_d, comb_d = gu.to_dev(h["streams"]), gu.to_dev(post), gu.to_dev(comb)
    flags = gu.native.GLM_HC_BF16_STREAMS if bf16 else 0
    out, _, _ = gu.run_layer(dl, shape, T=T)
    ref = torch.empty((T, hc, shape.d), dtype=torch.float32, device="cuda")
    gu.call("glm_hc_post", gu.stream(), gu.p(res), T, hc, shape.d, gu.p(out), gu.p(post_d),
            gu.p(comb_d), flags, gu.p(ref))
    d, E, k, I, Is = shape.d, shape.E, shape.k, shape.I, shape.I_shared
    lib = gu.native.load()
    ws_bytes = lib.glm_moe_workspace_bytes(T, d, E, k, I, Is)
    ws = gu.workspace(ws_bytes)
    out2 = torch.empty((T, d), dtype=torch.float32, device="cuda")
    hc_out = torch.empty((T, hc, d), dtype=torch.float32, device="cuda")
    args = [gu.stream(), gu.p(dl["x"]), T, d, gu.p(dl["router_weight"]), gu.p(dl["router_bias"]),
            E, k, shape.n_group, shape.topk_group, int(shape.norm_topk_prob),
            shape.routed_scaling_factor, I, *(gu.p(dl[key]) for key in BANK_KEYS), Is,
            gu.native.GLM_FMT_BF16, gu.p(dl["shared.gate"]), None, gu.p(dl["shared.up"]), None,
            gu.p(dl["shared.down"]), None, None, shape.swiglu_limit, gu.p(ws), ws_bytes,
            gu.p(out2), None, None, gu.p(res), hc, gu.p(post_d), gu.p(comb_d), flags,
            gu.p(hc_out)]
    gu.call("glm_moe_forward_hc", *args)
    assert np.array_equal(gu.host(out2).view(np.uint32), gu.host(out).view(np.uint32))
    assert np.array_equal(gu.host(hc_out).view(np.uint32), gu.host(ref).view(np.uint32))
