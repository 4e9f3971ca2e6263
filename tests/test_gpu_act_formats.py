"""GPU checks of the grouped GEMMs' activation formats through the C ABI.

* the split kernels write, bit for bit, the codes, scales and byte layout of
  the numpy model in ``tests/act_formats.py`` (FP8X2, FP6X2, FP4, FP8FP6);
* each format's grouped gate/up and down GEMMs equal the oracle's products of
  the model's dequantised split with the MXFP4 weights (the kernels' only
  freedom is the f32 summation order), so the format's error is all there is;
* the routed layer composed from the format's split, gate/up, split of h,
  down and combine is compared with the exact oracle layer; its relative L2
  error is printed (the accuracy column of the format comparison).
"""

from __future__ import annotations

import numpy as np
import pytest

import act_formats as A
from oracle import moe_oracle as O
from livglm_amd import native
from livglm_amd.workloads import BANK_KEYS, MoEShape, make_layer

pytestmark = pytest.mark.gpu

REL_L2 = 2e-3
FORMATS = [A.FP8X2, A.FP6X2, A.FP4, A.FP8FP6]
# the routed layer's relative L2 error against the exact oracle, per format (only
# FP8X2 meets the 2e-3 bar of the layer's bf16 output; FP6X2 lands near 2.3e-3 and FP4
# near 0.30; FP8FP6's lo term limits it as FP6X2's does)
LAYER_BOUND = {A.FP8X2: 2e-3, A.FP6X2: 5e-3, A.FP4: 0.5, A.FP8FP6: 5e-3}


def _torch():
    import torch
    return torch


@pytest.fixture(scope="module")
def gu():
    import gpu_util
    native.load()
    return gpu_util


def _split_gpu(gu, x_dev, rows, K, fmt):
    torch = _torch()
    buf = torch.zeros(native.load().glm_act_split_bytes_fmt(rows, K, fmt), dtype=torch.uint8,
                      device="cuda")
    gu.call("glm_act_split", gu.stream(), gu.p(x_dev), rows, K, fmt, gu.p(buf))
    return buf


@pytest.mark.parametrize("fmt", FORMATS, ids=[A.NAMES[f] for f in FORMATS])
def test_act_split_bit_exact(gu, fmt):
    # groups of N(0, s) with s over 12 binades, zero and negative-zero groups,
    # single-element groups, a group spanning 30 binades, values near the
    # bf16 maximum and subnormal bf16 values
    rng = np.random.default_rng(31 + fmt)
    rows, K = 96, 512
    x = rng.normal(0, 1, (rows, K // 32, 32)) * np.ldexp(1.0, rng.integers(-6, 6, (rows, K // 32, 1)))
    x[0, :3] = 0.0
    x[0, 3] = -0.0
    x[1, 0, 1:] = 0.0
    x[2, 0] = np.ldexp(rng.uniform(1, 2, 32), rng.integers(-20, 10, 32))
    x[3, 0] = rng.uniform(-1, 1, 32) * 3.0e38
    x[3, 1] = rng.uniform(-1, 1, 32) * 1e-39
    xb = O.f32_to_bf16_bits(x.reshape(rows, K).astype(np.float32))
    got = gu.host(_split_gpu(gu, gu.to_dev(xb), rows, K, fmt))
    want = A.pack(A.split(xb, K, fmt), rows, K, fmt)
    assert got.shape == want.shape
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (bad[:8], got[bad[:8]], want[bad[:8]])


def _route(layer, shape):
    x = O.bf16_bits_to_f32(layer["x"])
    _, w, idx, _ = O.router(x, layer["router_weight"], layer["router_bias"], top_k=shape.k,
                            n_group=1, topk_group=1, norm_topk_prob=True,
                            routed_scaling_factor=shape.routed_scaling_factor)
    return w, idx


def _tiles(gu, counts, offsets, active, E, P):
    torch = _torch()
    work = np.tile(np.array([-1, 0, 0, 0], np.int32), (E, 1))
    for u, e in enumerate(active):
        work[u] = (e, offsets[e], counts[e], 0)
    max_tiles = (P + 127) // 128 + E
    tiles = torch.empty((max_tiles, 4), dtype=torch.int32, device="cuda")
    ntiles = torch.empty(1, dtype=torch.int32, device="cuda")
    gu.call("glm_moe_tiles", gu.stream(), gu.p(gu.to_dev(work)), E, gu.p(tiles), gu.p(ntiles))
    return tiles, ntiles, max_tiles


def _grouped(gu, layer, shape, idx, fmt):
    """x split -> gate/up -> split of h -> down, all in format fmt; returns
    (h, y) in sorted order as device tensors, and the dispatch."""
    torch = _torch()
    T, k, E, d, I = layer["x"].shape[0], shape.k, shape.E, shape.d, shape.I
    P = T * k
    counts, offsets, perm, inv, active = O.dispatch(idx, E)
    dl = gu.upload_layer({key: layer[key] for key in ("x",) + BANK_KEYS})
    tiles, ntiles, max_tiles = _tiles(gu, counts, offsets, active, E, P)
    d_tok = gu.to_dev((perm // k).astype(np.int32))
    h = torch.empty((P, I), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((P, d), dtype=torch.bfloat16, device="cuda")
    x_split = _split_gpu(gu, dl["x"], T, d, fmt)
    gu.call("glm_expert_gate_up_grouped_fmt", gu.stream(), fmt, gu.p(x_split), T, d, I,
            *(gu.p(dl[key]) for key in BANK_KEYS[:4]), gu.p(d_tok), gu.p(tiles), gu.p(ntiles),
            max_tiles, shape.swiglu_limit, gu.p(h))
    h_split = _split_gpu(gu, h, P, I, fmt)
    gu.call("glm_expert_down_grouped_fmt", gu.stream(), fmt, gu.p(h_split), P, I, d,
            gu.p(dl[BANK_KEYS[4]]), gu.p(dl[BANK_KEYS[5]]), gu.p(tiles), gu.p(ntiles), max_tiles,
            gu.p(y))
    return h, y, (counts, offsets, perm, inv, active)


@pytest.mark.parametrize("d", [512, 2048])
def test_gate_up_every_token_block_count(gu, d):
    # expert sizes chosen so that the row tiles (at most 160 rows; an
    # expert's 16-row blocks dealt over its tiles) hold 1 to 10 blocks, full
    # and ragged, so the eight-wave gate/up's two token waves run every block
    # count 0..5; d = 512 is four K chunks (the shortest K loop), d = 2048
    # sixteen
    counts = [3, 17, 33, 47, 64, 81, 100, 127, 144, 160, 161, 250, 320]
    E, I = len(counts), 256
    T = sum(counts)
    shape = MoEShape("blocks", T, d, E, 1, I, 0)
    layer = make_layer(shape, 4242 + d)
    rng = np.random.default_rng(d)
    idx = rng.permutation(np.repeat(np.arange(E, dtype=np.int64), counts)).reshape(T, 1)
    h, _, (_, _, _, inv, _) = _grouped(gu, layer, shape, idx, A.FP8X2)
    bank = O.Bank(*(layer[key] for key in BANK_KEYS))
    xq = A.dequant(A.split(layer["x"], d, A.FP8X2), d, A.FP8X2).astype(np.float32)
    _, inter = O.routed_experts(xq, idx, bank, shape.swiglu_limit, return_intermediates=True)
    h_got = O.bf16_bits_to_f32(gu.bf16_bits(h))[inv].reshape(T, 1, I)
    assert O.rel_l2(h_got, inter["h"]) < REL_L2
    assert np.mean(h_got == inter["h"]) > 0.97


@pytest.mark.parametrize("fmt", FORMATS, ids=[A.NAMES[f] for f in FORMATS])
def test_grouped_gemms_equal_products_of_the_split(gu, fmt):
    # 400 tokens, d = 1024, 32 experts, top-4, I = 256: partial tiles and
    # experts spanning several tiles
    shape = MoEShape("grouped", 400, 1024, 32, 4, 256, 0)
    layer = make_layer(shape, 1717)
    T, k, d, I = shape.T, shape.k, shape.d, shape.I
    _, idx = _route(layer, shape)
    h, y, (counts, offsets, perm, inv, active) = _grouped(gu, layer, shape, idx, fmt)
    bank = O.Bank(*(layer[key] for key in BANK_KEYS))
    # gate/up against the oracle on the dequantised split of x
    xq = A.dequant(A.split(layer["x"], d, fmt), d, fmt).astype(np.float32)
    _, inter = O.routed_experts(xq, idx, bank, shape.swiglu_limit, return_intermediates=True)
    h_bits = gu.bf16_bits(h)
    h_got = O.bf16_bits_to_f32(h_bits)[inv].reshape(T, k, I)
    assert O.rel_l2(h_got, inter["h"]) < REL_L2
    assert np.mean(h_got == inter["h"]) > 0.97
    # down against the oracle on the dequantised split of the kernel's own h
    hq = A.dequant(A.split(h_bits, I, fmt), I, fmt).astype(np.float32)
    y_want = np.zeros((T * k, d), dtype=np.float32)
    for e in active:
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        y_want[lo:hi] = O.linear_bf16(hq[lo:hi], bank.projection("down_proj", e))
    y_got = O.bf16_bits_to_f32(gu.bf16_bits(y))
    assert O.rel_l2(y_got, y_want) < REL_L2
    assert np.mean(y_got == y_want) > 0.97


@pytest.mark.parametrize("fmt", FORMATS, ids=[A.NAMES[f] for f in FORMATS])
def test_routed_layer_error_per_format(gu, fmt):
    # the prefill geometry (d = 2048, 128 experts, top-8, I = 768) on 256
    # tokens: the routed layer (without the shared expert) composed in
    # format fmt against the exact oracle
    torch = _torch()
    shape = MoEShape("prefill", 256, 2048, 128, 8, 768, 0)
    layer = make_layer(shape, 4096)
    T, k, d = shape.T, shape.k, shape.d
    w, idx = _route(layer, shape)
    _, y, (counts, offsets, perm, inv, active) = _grouped(gu, layer, shape, idx, fmt)
    out = torch.empty((T, d), dtype=torch.float32, device="cuda")
    gu.call("glm_moe_combine", gu.stream(), gu.p(y), gu.p(gu.to_dev(inv.astype(np.int32))),
            gu.p(gu.to_dev(w.astype(np.float32))), None, T, k, d, gu.p(out))
    bank = O.Bank(*(layer[key] for key in BANK_KEYS))
    x = O.bf16_bits_to_f32(layer["x"])
    want = O.combine(O.routed_experts(x, idx, bank, shape.swiglu_limit), w, None)
    err = O.rel_l2(gu.host(out), want)
    print(f"\nrouted layer rel-L2 [{A.NAMES[fmt]}] = {err:.3e}")
    assert err < LAYER_BOUND[fmt]
