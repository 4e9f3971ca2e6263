"""GPU parity of the decode stack: per layer the resident MXFP8 linear
(layers.py:56-65, quantised at start-up as layers.py:72-99 and
model.py:228-260 do) -- behind an RMSNorm of the previous layer's f32 output
(layers.py:119-131, the decoder's norm in front of each block, model.py:
132-136), fused into the linear -- and the MoE layer (moe.py:123-201) on its
output, with the per-step Markov routing biases of the layer-stack workload,
fed one token per step as the decode loop does (runtime.py:721-765).

Two geometries: a small one (d 1024, E 16, k 2, I 512) and the 42-layer
decode stack's own (d 2048, E 128, k 8, I 768 with a 2048 x 2048 MXFP8
linear quantised on the GPU).  Each layer is checked against the oracle on
the very input the GPU gave it (so rounding differences do not compound), the
routed experts must be the set the bias trace forces, and one step captured in
a HIP graph must replay bit-identically to the eager step, several times over.
At the full 42 layers x 16 steps the checks are size-independent: the routed
set equals the forced set, the route weights equal the oracle router's on the
GPU's own linear output, the outputs are finite, and every step's graph
replays its eager result bit for bit."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O
from livglm_amd import native
from livglm_amd.workloads import BANK_KEYS, MoEShape, make_layer, markov_bias_trace

pytestmark = pytest.mark.gpu

REL_L2 = 2e-3
NORM_EPS = 1e-6
SHAPES_UNDER_TEST = {
    "small": MoEShape("stack_small", T=1, d=1024, E=16, k=2, I=512, I_shared=512,
                      routing="markov", layers=3, steps=4),
    # the decode stack's geometry (42 x this layer), a few layers and steps
    "c4": MoEShape("stack_c4", T=1, d=2048, E=128, k=8, I=768, I_shared=768, routing="markov",
                   layers=3, steps=3),
}


def _quantize_linear_on_gpu(w_bits):
    """The resident linear's start-up quantisation on the GPU (glm_mx_quantize,
    nearest scale rule); returns device (codes, scales) after checking them
    bit for bit against the oracle's quantiser."""
    import torch

    import gpu_util as gu
    n_out, n_in = w_bits.shape
    codes = torch.empty((n_out, n_in), dtype=torch.uint8, device="cuda")
    scales = torch.empty((n_out, n_in // 32), dtype=torch.uint8, device="cuda")
    gu.call("glm_mx_quantize", gu.stream(), gu.p(gu.to_dev(w_bits)), n_out, n_in,
            native.GLM_FMT_MXFP8, native.GLM_MX_RULE_NEAREST, gu.p(codes), gu.p(scales))
    want_c, want_s = O.quantize_mx(w_bits, 8, O.MX_RULE_NEAREST)
    np.testing.assert_array_equal(gu.host(codes), want_c)
    np.testing.assert_array_equal(gu.host(scales), want_s)
    return codes, scales, (want_c, want_s)


@pytest.fixture(scope="module", params=list(SHAPES_UNDER_TEST))
def stack(request):
    import torch

    import gpu_util as gu
    native.load()
    s = SHAPES_UNDER_TEST[request.param]
    rng = np.random.default_rng(7400)
    layers = [make_layer(s, 7400 + i) for i in range(s.layers)]
    lin, lin_dev = [], []
    for _ in range(s.layers):
        w = O.f32_to_bf16_bits(rng.normal(0, 0.02, (s.d, s.d)).astype(np.float32))
        if request.param == "c4":
            codes, scales, host_q = _quantize_linear_on_gpu(w)
            lin.append(host_q)
            lin_dev.append((codes, scales))
        else:
            lin.append(O.quantize_mx(w, 8, O.MX_RULE_NEAREST))
            lin_dev.append(tuple(gu.to_dev(a) for a in lin[-1]))
    trace = markov_bias_trace(s.E, s.k, s.layers, s.steps, rng)
    xs = O.f32_to_bf16_bits(rng.normal(0, 1, (s.steps, s.T, s.d)).astype(np.float32))
    norms = [O.bf16_bits_to_f32(O.f32_to_bf16_bits(rng.normal(1.0, 0.1, s.d).astype(np.float32)))
             for _ in range(s.layers)]
    dev = {
        "layers": [gu.upload_layer(layer) for layer in layers],
        "lin": lin_dev,
        "norm": [gu.to_dev(n) for n in norms],
        "trace": gu.to_dev(trace),
        "xs": gu.to_dev(xs),
    }
    lib = native.load()
    ws_bytes = lib.glm_moe_workspace_bytes(s.T, s.d, s.E, s.k, s.I, s.I_shared)
    bufs = {
        "ws": gu.workspace(ws_bytes), "ws_bytes": ws_bytes,
        "act": torch.empty((s.T, s.d), dtype=torch.bfloat16, device="cuda"),
        "carry": torch.empty((s.T, s.d), dtype=torch.bfloat16, device="cuda"),
    }
    return {"np": (layers, lin, trace, xs, norms), "dev": dev, "bufs": bufs, "torch": torch,
            "shape": s}


def _step(st, step):
    """One decode step through the stack, stream-ordered with no host
    synchronisation (capturable).  Returns per layer (input, linear output,
    MoE output, weights, indices) as fresh device tensors."""
    torch, s, dev, bufs = st["torch"], st["shape"], st["dev"], st["bufs"]
    stream = torch.cuda.current_stream().cuda_stream
    x = dev["xs"][step]
    records = []
    for layer in range(s.layers):
        dl = dev["layers"][layer]
        codes, scales = dev["lin"][layer]
        a = torch.empty((s.T, s.d), dtype=torch.bfloat16, device="cuda")
        # layers past the first read the previous f32 output through the norm
        if x.dtype == torch.bfloat16:
            native.call("glm_linear", stream, x.data_ptr(), s.T, s.d, codes.data_ptr(),
                        scales.data_ptr(), native.GLM_FMT_MXFP8, s.d, a.data_ptr())
        else:
            native.call("glm_rms_norm_linear", stream, x.data_ptr(), s.T, s.d,
                        dev["norm"][layer].data_ptr(), NORM_EPS, codes.data_ptr(),
                        scales.data_ptr(), native.GLM_FMT_MXFP8, s.d, a.data_ptr())
        out = torch.empty((s.T, s.d), dtype=torch.float32, device="cuda")
        w = torch.empty((s.T, s.k), dtype=torch.float32, device="cuda")
        idx = torch.empty((s.T, s.k), dtype=torch.int32, device="cuda")
        native.call("glm_moe_forward", stream, a.data_ptr(), s.T, s.d,
                    dl["router_weight"].data_ptr(), dev["trace"][step, layer].data_ptr(), s.E,
                    s.k, s.n_group, s.topk_group, 1, s.routed_scaling_factor, s.I,
                    *(dl[key].data_ptr() for key in BANK_KEYS), s.I_shared, native.GLM_FMT_BF16,
                    dl["shared.gate"].data_ptr(), None, dl["shared.up"].data_ptr(), None,
                    dl["shared.down"].data_ptr(), None, None, s.swiglu_limit,
                    bufs["ws"].data_ptr(), bufs["ws_bytes"], out.data_ptr(), w.data_ptr(),
                    idx.data_ptr())
        records.append((x, a, out, w, idx))
        x = out  # the next layer's input, f32
    return records


def test_stack_layers_match_oracle_on_their_inputs(stack):
    import gpu_util as gu
    torch = stack["torch"]
    from oracle import mhc_oracle as H
    layers, lin, trace, _, norms = stack["np"]
    s = stack["shape"]
    for step in range(s.steps):
        recs = _step(stack, step)
        torch.cuda.synchronize()
        for layer, (x, a, out, w, idx) in enumerate(recs):
            if x.dtype == torch.bfloat16:
                xb = gu.bf16_bits(x)
            else:  # the norm of the previous output, rounded to bf16: what the linear multiplies
                xb = O.f32_to_bf16_bits(H.rms_norm(gu.host(x), norms[layer], NORM_EPS))
            codes, scales = lin[layer]
            a_want = O.linear_bf16(O.bf16_bits_to_f32(xb), O.dequant_mxfp8(codes, scales))
            a_got = O.bf16_bits_to_f32(gu.bf16_bits(a))
            assert O.rel_l2(a_got, a_want) < REL_L2
            assert np.mean(a_got == a_want) > 0.97
            ly = dict(layers[layer], x=gu.bf16_bits(a), router_bias=trace[step, layer])
            sw = tuple(O.bf16_bits_to_f32(ly[k]) for k in ("shared.gate", "shared.up",
                                                            "shared.down"))
            want, inter = O.moe_layer(O.bf16_bits_to_f32(ly["x"]), ly["router_weight"],
                                      ly["router_bias"], O.Bank(*(ly[k] for k in BANK_KEYS)), sw,
                                      top_k=s.k, n_group=1, topk_group=1, norm_topk_prob=True,
                                      routed_scaling_factor=s.routed_scaling_factor,
                                      swiglu_limit=s.swiglu_limit, return_intermediates=True)
            got_idx = gu.host(idx).astype(np.uint32)
            assert np.array_equal(got_idx, inter["indices"]), (step, layer)
            forced = np.nonzero(trace[step, layer] > 0)[0]
            assert sorted(got_idx.reshape(-1).tolist()) == sorted(forced.tolist())
            np.testing.assert_allclose(gu.host(w), inter["weights"], rtol=2e-6, atol=1e-7)
            assert O.rel_l2(gu.host(out), want) < REL_L2, (step, layer)


def test_stack_step_graph_replays_bit_identical(stack):
    torch = stack["torch"]
    eager = _step(stack, 1)
    torch.cuda.synchronize()
    want = [r[2].cpu().numpy().view(np.uint32).copy() for r in eager]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        captured = _step(stack, 1)
    for _ in range(3):
        _step(stack, 2)  # other eager work between replays
        torch.cuda.synchronize()
        for rec in captured:
            rec[2].zero_()
        g.replay()
        torch.cuda.synchronize()
        for layer, rec in enumerate(captured):
            assert np.array_equal(rec[2].cpu().numpy().view(np.uint32), want[layer]), layer


def test_stack42_full_size_properties():
    """The decode stack at its full size: 42 layers x 16 steps at d 2048, E 128,
    k 8, I 768 with the 2048 x 2048 MXFP8 linears quantised on the GPU (each
    behind the RMSNorm of the previous layer's output), routed by the Markov
    bias trace.  Size-independent checks: per layer and step the routed set is
    the forced set, in the order the oracle's router gives on the GPU's own
    linear output, with the oracle router's weights; every output is finite;
    each step captured in a HIP graph replays its eager result bit for bit
    (eager work of other steps in between)."""
    import torch

    s = MoEShape("stack42", T=1, d=2048, E=128, k=8, I=768, I_shared=768, routing="markov",
                 layers=42, steps=16)
    native.load()
    dev = torch.device("cuda")
    gen = torch.Generator(device=dev)
    gen.manual_seed(7420)
    T, d, E, k, I, Is = s.T, s.d, s.E, s.k, s.I, s.I_shared
    stream = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    banks = []
    for _ in range(s.layers):
        b = {
            "gate_proj.weight_packed": torch.randint(0, 256, (E, I, d // 2), dtype=torch.uint8,
                                                     device=dev, generator=gen),
            "gate_proj.weight_scale": torch.randint(119, 128, (E, I, d // 32), dtype=torch.uint8,
                                                    device=dev, generator=gen),
            "up_proj.weight_packed": torch.randint(0, 256, (E, I, d // 2), dtype=torch.uint8,
                                                   device=dev, generator=gen),
            "up_proj.weight_scale": torch.randint(119, 128, (E, I, d // 32), dtype=torch.uint8,
                                                  device=dev, generator=gen),
            "down_proj.weight_packed": torch.randint(0, 256, (E, d, I // 2), dtype=torch.uint8,
                                                     device=dev, generator=gen),
            "down_proj.weight_scale": torch.randint(119, 128, (E, d, I // 32), dtype=torch.uint8,
                                                    device=dev, generator=gen),
            "router_weight": torch.randn((E, d), device=dev, generator=gen) * 0.02,
            "shared.gate": (torch.randn((Is, d), device=dev, generator=gen) * 0.02).bfloat16(),
            "shared.up": (torch.randn((Is, d), device=dev, generator=gen) * 0.02).bfloat16(),
            "shared.down": (torch.randn((d, Is), device=dev, generator=gen) * 0.02).bfloat16(),
            "lin.codes": torch.empty((d, d), dtype=torch.uint8, device=dev),
            "lin.scales": torch.empty((d, d // 32), dtype=torch.uint8, device=dev),
            "norm": (1.0 + 0.1 * torch.randn(d, device=dev, generator=gen)).bfloat16().float(),
        }
        w = (torch.randn((d, d), device=dev, generator=gen) * 0.02).bfloat16()
        native.call("glm_mx_quantize", stream(), w.data_ptr(), d, d, native.GLM_FMT_MXFP8,
                    native.GLM_MX_RULE_NEAREST, b["lin.codes"].data_ptr(),
                    b["lin.scales"].data_ptr())
        banks.append(b)
    trace_np = markov_bias_trace(E, k, s.layers, s.steps, np.random.default_rng(7420))
    routers = [b["router_weight"].cpu().numpy() for b in banks]
    trace = torch.from_numpy(trace_np).to(dev)
    xs = (torch.randn((s.steps, T, d), device=dev, generator=gen)).bfloat16()
    lib = native.load()
    ws_bytes = lib.glm_moe_workspace_bytes(T, d, E, k, I, Is)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    native.call("glm_moe_workspace_init", stream(), ws.data_ptr(), ws_bytes)
    acts = torch.empty((s.layers, T, d), dtype=torch.bfloat16, device=dev)
    outs = torch.empty((s.layers, T, d), dtype=torch.float32, device=dev)
    wts = torch.empty((s.layers, T, k), dtype=torch.float32, device=dev)
    idx = torch.empty((s.layers, T, k), dtype=torch.int32, device=dev)

    def step(st):
        for layer in range(s.layers):
            b = banks[layer]
            if layer == 0:
                native.call("glm_linear", stream(), xs[st].data_ptr(), T, d,
                            b["lin.codes"].data_ptr(), b["lin.scales"].data_ptr(),
                            native.GLM_FMT_MXFP8, d, acts[layer].data_ptr())
            else:
                native.call("glm_rms_norm_linear", stream(), outs[layer - 1].data_ptr(), T, d,
                            b["norm"].data_ptr(), 1e-6, b["lin.codes"].data_ptr(),
                            b["lin.scales"].data_ptr(), native.GLM_FMT_MXFP8, d,
                            acts[layer].data_ptr())
            native.call("glm_moe_forward", stream(), acts[layer].data_ptr(), T, d,
                        b["router_weight"].data_ptr(), trace[st, layer].data_ptr(), E, k, 1, 1, 1,
                        s.routed_scaling_factor, I, *(b[key].data_ptr() for key in BANK_KEYS), Is,
                        native.GLM_FMT_BF16, b["shared.gate"].data_ptr(), None,
                        b["shared.up"].data_ptr(), None, b["shared.down"].data_ptr(), None, None,
                        s.swiglu_limit, ws.data_ptr(), ws_bytes, outs[layer].data_ptr(),
                        wts[layer].data_ptr(), idx[layer].data_ptr())

    eager = []
    for st in range(s.steps):
        step(st)
        torch.cuda.synchronize()
        got_idx = idx.cpu().numpy().astype(np.uint32)
        got_w = wts.cpu().numpy()
        o = outs.cpu().numpy()
        a = O.bf16_bits_to_f32(acts.view(torch.int16).cpu().numpy().view(np.uint16))
        assert np.isfinite(o).all(), f"step {st}: non-finite MoE output"
        for layer in range(s.layers):
            forced = np.nonzero(trace_np[st, layer] > 0)[0]
            assert sorted(got_idx[layer].reshape(-1).tolist()) == sorted(forced.tolist()), \
                (st, layer)
            _, w_want, i_want, choice = O.router(a[layer], routers[layer],
                                                 trace_np[st, layer], top_k=k, n_group=1,
                                                 topk_group=1, norm_topk_prob=True,
                                                 routed_scaling_factor=s.routed_scaling_factor)
            # order within the chosen set: exact unless the oracle's two choice
            # scores are within 1e-5 (the f32 summation order of the logits)
            g_i, w_i = got_idx[layer][0], i_want[0]
            for j in np.nonzero(g_i != w_i)[0]:
                assert abs(float(choice[0, g_i[j]]) - float(choice[0, w_i[j]])) < 1e-5, \
                    (st, layer, j)
            order_g, order_w = np.argsort(g_i), np.argsort(w_i)
            np.testing.assert_allclose(got_w[layer][0][order_g], w_want[0][order_w], rtol=2e-6,
                                       atol=1e-7, err_msg=str((st, layer)))
        eager.append(o.view(np.uint32).copy())
    # graph replays of a few steps, other eager steps in between
    for st in (0, 7, 15):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            step(st)
        for rep in range(2):
            step((st + 3) % s.steps)
            torch.cuda.synchronize()
            outs.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert np.array_equal(outs.cpu().numpy().view(np.uint32), eager[st]), (st, rep)
        del g
    del banks
    torch.cuda.empty_cache()
