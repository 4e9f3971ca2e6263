"""GPU checks of glm_moe_forward_scalex: the few-token layer reading its
routed experts' E8M0 scales as ScaleX Mode-B rows and decoding them inside
the kernels (the reference decodes 512-scale tiles in threadgroup memory
inside its QMV, src/glm53flash/native_expert_ssd.py:653-694) must match the
oracle's layer on the decoded scales -- indices exact on clear-margin rows,
weights to f32 rounding, outputs within rel-L2 2e-3 -- and must give, bit for
bit, what glm_moe_forward gives on the decoded scales (the coding is
lossless: docs/scalex-mode-b.md:8-20).  Banks mix the codec's three forms
(one bit with exceptions, two bits, raw), and planted exceptions sit on
512-scale tile edges, on the first and last scale and at the borders of the
gate, down and up segments."""

from __future__ import annotations

import numpy as np
import pytest

from glm53flash import scale_codec as C
from livglm_amd import native
from oracle import moe_oracle as O
from livglm_amd.workloads import BANK_KEYS, MoEShape, concentrated_scales, make_layer

pytestmark = pytest.mark.gpu

REL_L2 = 2e-3  # bf16 layer-output tolerance against the oracle
MARGIN = 1e-5  # choice-score gap below which top-k order may flip


def _torch():
    import torch
    return torch


@pytest.fixture(scope="module")
def gu():
    import gpu_util
    native.load()
    return gpu_util


def _scales(shape, rng, kinds):
    E, d, I = shape.E, shape.d, shape.I
    gs = np.empty((E, I, d // 32), np.uint8)
    ds = np.empty((E, d, I // 32), np.uint8)
    us = np.empty((E, I, d // 32), np.uint8)
    for e in range(E):
        kind = kinds[e % len(kinds)]
        gs[e] = concentrated_scales(rng, (I, d // 32), kind)
        ds[e] = concentrated_scales(rng, (d, I // 32), kind)
        us[e] = concentrated_scales(rng, (I, d // 32), kind)
        if kind == "one_bit":
            # exceptions on tile edges, the stream's ends and the segments' borders
            flat = np.concatenate([gs[e].ravel(), ds[e].ravel(), us[e].ravel()])
            n, seg = flat.size, I * (d // 32)
            for p in (0, 511, 512, 1023, 1024, seg - 1, seg, 2 * seg - 1, 2 * seg, n - 513, n - 1):
                flat[p] = 100 + (p % 17)
            gs[e] = flat[:seg].reshape(I, d // 32)
            ds[e] = flat[seg:2 * seg].reshape(d, I // 32)
            us[e] = flat[2 * seg:].reshape(I, d // 32)
    return gs, ds, us


def _forward(gu, dl, shape, T, scalex=None):
    torch = _torch()
    d, E, k, I, Is = shape.d, shape.E, shape.k, shape.I, shape.I_shared
    lib = native.load()
    ws_bytes = lib.glm_moe_workspace_bytes(T, d, E, k, I, Is)
    ws = gu.workspace(ws_bytes)
    out = torch.empty((T, d), dtype=torch.float32, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    args = [gu.stream(), gu.p(dl["x"]), T, d, gu.p(dl["router_weight"]), gu.p(dl["router_bias"]),
            E, k, shape.n_group, shape.topk_group, int(shape.norm_topk_prob),
            shape.routed_scaling_factor, I]
    if scalex is None:
        args += [gu.p(dl[key]) for key in BANK_KEYS]
    else:
        rows, stride = scalex
        args += [gu.p(dl["gate_proj.weight_packed"]), gu.p(dl["up_proj.weight_packed"]),
                 gu.p(dl["down_proj.weight_packed"]), gu.p(rows), stride]
    if Is:
        args += [Is, native.GLM_FMT_BF16, gu.p(dl["shared.gate"]), None, gu.p(dl["shared.up"]),
                 None, gu.p(dl["shared.down"]), None, None]
    else:
        args += [0, native.GLM_FMT_BF16, None, None, None, None, None, None, None]
    args += [shape.swiglu_limit, gu.p(ws), ws_bytes, gu.p(out), gu.p(w), gu.p(idx)]
    gu.call("glm_moe_forward_scalex" if scalex is not None else "glm_moe_forward", *args)
    return gu.host(out), gu.host(w), gu.host(idx)


def _oracle(layer, shape):
    x = O.bf16_bits_to_f32(layer["x"])
    sw = None
    if shape.I_shared:
        sw = tuple(O.bf16_bits_to_f32(layer[key])
                   for key in ("shared.gate", "shared.up", "shared.down"))
    return O.moe_layer(x, layer["router_weight"], layer["router_bias"],
                       O.Bank(*(layer[key] for key in BANK_KEYS)), sw, top_k=shape.k,
                       n_group=shape.n_group, topk_group=shape.topk_group,
                       norm_topk_prob=shape.norm_topk_prob,
                       routed_scaling_factor=shape.routed_scaling_factor,
                       swiglu_limit=shape.swiglu_limit, return_intermediates=True)


CASES = [
    # (T, d, E, k, I, I_shared, kinds)
    (2, 2048, 128, 8, 768, 768, ("one_bit",)),
    (1, 2048, 64, 8, 768, 0, ("one_bit", "two_bit", "raw")),
    (4, 1024, 16, 2, 512, 256, ("two_bit", "one_bit")),
    (3, 3072, 24, 4, 256, 128, ("raw", "one_bit")),
    # the real expert geometry: several tiles per block in both kernels
    (2, 4096, 32, 8, 2048, 2048, ("one_bit", "one_bit", "two_bit")),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"T{c[0]}-d{c[1]}-E{c[2]}-I{c[4]}")
def test_scalex_forward_matches_oracle_and_decoded_scales(gu, case):
    T, d, E, k, I, Is, kinds = case
    shape = MoEShape("scalex", T, d, E, k, I, Is)
    layer = make_layer(shape, 2100 + d + E)
    rng = np.random.default_rng(77 + E)
    gs, ds, us = _scales(shape, rng, kinds)
    layer["gate_proj.weight_scale"], layer["down_proj.weight_scale"] = gs, ds
    layer["up_proj.weight_scale"] = us
    rows, stride, coded = C.mode_b_bank(gs, ds, us)
    # the rows decode back to the scales (host codec), and the coded bank is
    # smaller than the raw one unless every expert is raw
    for e in range(E):
        raw = C.decode_mode_a(C.mode_b_record(rows[e], 3 * I * (d // 32)))
        assert raw == gs[e].tobytes() + ds[e].tobytes() + us[e].tobytes()
    dl = gu.upload_layer({key: layer[key] for key in layer})
    rows_dev = gu.to_dev(rows)
    want = _forward(gu, dl, shape, T)
    got = _forward(gu, dl, shape, T, scalex=(rows_dev, stride))
    for g, w_ in zip(got, want):
        assert np.array_equal(g.view(np.uint32) if g.dtype == np.float32 else g,
                              w_.view(np.uint32) if w_.dtype == np.float32 else w_)
    # the in-kernel decode against the oracle's layer on the decoded scales
    ref, inter = _oracle(layer, shape)
    out, w, idx = got
    idx = idx.astype(np.uint32)
    sure = O.topk_margin(inter["choice"], k) > MARGIN
    assert not np.any(np.any(idx != inter["indices"], axis=1) & sure)
    same = np.all(idx == inter["indices"], axis=1)
    assert same.sum() >= T - 1
    np.testing.assert_allclose(w[same], inter["weights"][same], rtol=2e-6, atol=1e-7)
    assert O.rel_l2(out[same], ref[same]) < REL_L2


def test_scalex_forward_rejects_what_it_cannot_take(gu):
    # more tokens than the few-token kernels take, and a misaligned stride
    torch = _torch()
    shape = MoEShape("scalex", 8, 2048, 16, 2, 512, 0)
    layer = make_layer(shape, 5)
    dl = gu.upload_layer({key: layer[key] for key in layer})
    rows = torch.zeros((16, 1024), dtype=torch.uint8, device="cuda")
    lib = native.load()
    ws = gu.workspace(lib.glm_moe_workspace_bytes(8, 2048, 16, 2, 512, 0))
    out = torch.empty((8, 2048), dtype=torch.float32, device="cuda")
    base = [gu.stream(), gu.p(dl["x"]), 8, 2048, gu.p(dl["router_weight"]),
            gu.p(dl["router_bias"]), 16, 2, 1, 1, 1, 2.5, 512, gu.p(dl["gate_proj.weight_packed"]),
            gu.p(dl["up_proj.weight_packed"]), gu.p(dl["down_proj.weight_packed"]), gu.p(rows)]
    tail = [0, native.GLM_FMT_BF16, None, None, None, None, None, None, None, 10.0, gu.p(ws),
            ws.numel(), gu.p(out), None, None]
    rc = lib.glm_moe_forward_scalex(*base, 1024, *tail)
    assert rc == native.GLM_ERR_UNSUPPORTED_SHAPE and b"few-token" in lib.glm_last_error()
    rc = lib.glm_moe_forward_scalex(*base, 1000, *tail)
    assert rc == native.GLM_ERR_INVALID_ARGUMENT
