"""GPU parity of a short decode stack: per layer the resident MXFP8 linear
(layers.py:56-65) and the MoE layer (moe.py:123-201) on its output, with the
per-step Markov routing biases of the layer-stack workload.

Each layer is checked against the oracle on the very input the GPU gave it
(so rounding differences do not compound), the routed experts must be the
set the bias trace forces, and one step captured in a HIP graph must replay
bit-identically to the eager step, several times over."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O
from livglm_amd import native
from livglm_amd.workloads import BANK_KEYS, MoEShape, make_layer, markov_bias_trace

pytestmark = pytest.mark.gpu

REL_L2 = 2e-3
SHAPE = MoEShape("stack_small", T=1, d=1024, E=16, k=2, I=512, I_shared=512, routing="markov",
                 layers=3, steps=4)


@pytest.fixture(scope="module")
def stack():
    import torch

    import gpu_util as gu
    native.load()
    s = SHAPE
    rng = np.random.default_rng(7400)
    layers = [make_layer(s, 7400 + i) for i in range(s.layers)]
    lin = []
    for _ in range(s.layers):
        w = O.f32_to_bf16_bits(rng.normal(0, 0.02, (s.d, s.d)).astype(np.float32))
        lin.append(O.quantize_mx(w, 8, O.MX_RULE_NEAREST))
    trace = markov_bias_trace(s.E, s.k, s.layers, s.steps, rng)
    xs = O.f32_to_bf16_bits(rng.normal(0, 1, (s.steps, s.T, s.d)).astype(np.float32))
    dev = {
        "layers": [gu.upload_layer(layer) for layer in layers],
        "lin": [(gu.to_dev(c), gu.to_dev(sc)) for c, sc in lin],
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
    return {"np": (layers, lin, trace, xs), "dev": dev, "bufs": bufs, "torch": torch}


def _step(st, step):
    """One decode step through the stack, stream-ordered with no host
    synchronisation (capturable).  Returns per layer (input, linear output,
    MoE output, weights, indices) as fresh device tensors."""
    torch, s, dev, bufs = st["torch"], SHAPE, st["dev"], st["bufs"]
    stream = torch.cuda.current_stream().cuda_stream
    x = dev["xs"][step]
    records = []
    for layer in range(s.layers):
        dl = dev["layers"][layer]
        codes, scales = dev["lin"][layer]
        a = torch.empty((s.T, s.d), dtype=torch.bfloat16, device="cuda")
        # layers past the first read the previous f32 output, rounded as read
        fn = "glm_linear" if x.dtype == torch.bfloat16 else "glm_linear_f32"
        native.call(fn, stream, x.data_ptr(), s.T, s.d, codes.data_ptr(),
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
    layers, lin, trace, _ = stack["np"]
    s = SHAPE
    for step in range(s.steps):
        recs = _step(stack, step)
        torch.cuda.synchronize()
        for layer, (x, a, out, w, idx) in enumerate(recs):
            xb = gu.bf16_bits(x.to(torch.bfloat16))  # what the linear reads
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
