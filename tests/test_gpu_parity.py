"""GPU parity of the HIP kernels (through the C ABI) against the CPU oracle.

Integer and byte work (dequantised values, quantised codes, routing indices,
permutation) must be bit-exact; bf16 layer outputs must be within rel-L2 2e-3
of the oracle.  Router indices are compared exactly on every row whose top-k
margin (f64, over the top k+1 choice scores) exceeds MARGIN; rows under it may
legitimately flip under a different f32 summation order and are counted.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import moe_oracle as O
from livglm_amd import native
from livglm_amd.workloads import SHAPES, BANK_KEYS, MoEShape, make_layer

pytestmark = pytest.mark.gpu

REL_L2 = 2e-3  # bf16 layer-output tolerance: rel-L2 against the exact oracle
MARGIN = 1e-5  # choice-score gap below which top-k order may flip


def _torch():
    import torch
    return torch


@pytest.fixture(scope="module")
def gu():
    import gpu_util
    native.load()
    return gpu_util


def _bank(layer):
    return O.Bank(*(layer[k] for k in BANK_KEYS))


def _oracle_layer(layer, shape, shared=True):
    x = O.bf16_bits_to_f32(layer["x"])
    sw = None
    if shared:
        sw = tuple(O.bf16_bits_to_f32(layer[k]) for k in ("shared.gate", "shared.up", "shared.down"))
    return O.moe_layer(x, layer["router_weight"], layer["router_bias"], _bank(layer), sw,
                       top_k=shape.k, n_group=shape.n_group, topk_group=shape.topk_group,
                       norm_topk_prob=shape.norm_topk_prob,
                       routed_scaling_factor=shape.routed_scaling_factor,
                       swiglu_limit=shape.swiglu_limit, return_intermediates=True)


def _check_indices(got, want, choice, k):
    margin = O.topk_margin(choice, k)
    sure = margin > MARGIN
    mism = np.any(got != want, axis=1)
    assert not np.any(mism & sure), f"index mismatch on unambiguous rows {np.nonzero(mism & sure)[0][:10]}"
    return int(np.sum(~sure))


# --------------------------------------------------------------------------- codecs


# Scale bytes whose decoded values stay inside bf16's range: the kernels
# dequantise to bf16 in registers, which is exact for E2M1 when e >= 1 and for
# E4M3FN when e >= 3.  Smaller scales (group scales of 2^-127..2^-125) flush
# their subnormal tail and are outside the supported domain; real checkpoints
# and the synthetic banks use e in [119, 127].
MXFP4_SCALES = np.array([1, 2, 3, 64, 100, 119, 120, 123, 125, 126, 127, 130, 200, 253, 254, 255],
                        np.uint8)
MXFP8_SCALES = np.array([3, 4, 64, 100, 119, 121, 124, 127, 128, 140, 200, 253, 254, 255], np.uint8)


def _dequant_case(gu, codes, scl, K, fmt):
    torch = _torch()
    R = len(scl)
    scales = np.repeat(scl[:, None], K // 32, axis=1)
    with np.errstate(over="ignore", invalid="ignore"):
        want = O.dequant_mxfp4(codes, scales) if fmt == native.GLM_FMT_MXFP4 \
            else O.dequant_mxfp8(codes, scales)
    out = torch.empty((R, K), dtype=torch.float32, device="cuda")
    gu.call("glm_mx_dequantize", gu.stream(), gu.p(gu.to_dev(codes)), gu.p(gu.to_dev(scales)), R,
            K, fmt, gu.p(out))
    got = gu.host(out)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_mxfp4_dequant_bit_exact(gu):
    # every packed byte (all 16x16 code pairs) under every scale class
    codes = np.tile(np.arange(256, dtype=np.uint8), (len(MXFP4_SCALES), 1))
    _dequant_case(gu, codes, MXFP4_SCALES, 512, native.GLM_FMT_MXFP4)


def test_mxfp8_dequant_bit_exact(gu):
    codes = np.tile(np.arange(256, dtype=np.uint8), (len(MXFP8_SCALES), 1))
    _dequant_case(gu, codes, MXFP8_SCALES, 256, native.GLM_FMT_MXFP8)


def test_mxfp4_dequant_random_bank_bit_exact(gu):
    rng = np.random.default_rng(5)
    codes = rng.integers(0, 256, (64, 1024), dtype=np.uint8)
    scl = rng.integers(119, 128, 64).astype(np.uint8)
    _dequant_case(gu, codes, scl, 2048, native.GLM_FMT_MXFP4)


def _quant_inputs():
    rng = np.random.default_rng(77)
    a = rng.normal(0, 0.02, (64, 256)).astype(np.float32)
    a[0, :32] = 0.0  # all-zero group
    a[1, :32] = rng.normal(0, 1e-30, 32)  # tiny
    a[2, :32] = rng.normal(0, 1e4, 32)  # large
    a[3] = np.linspace(-3, 3, 256)  # ties and boundaries
    a[4, :32] = -0.0
    return O.f32_to_bf16_bits(a)


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("rule", [O.MX_RULE_NEAREST, O.MX_RULE_OCP])
def test_mx_quantize_bit_exact(gu, bits, rule):
    torch = _torch()
    w = _quant_inputs()
    rows, cols = w.shape
    want_codes, want_scales = O.quantize_mx(w, bits, rule)
    codes = torch.empty(want_codes.shape, dtype=torch.uint8, device="cuda")
    scales = torch.empty(want_scales.shape, dtype=torch.uint8, device="cuda")
    fmt = native.GLM_FMT_MXFP8 if bits == 8 else native.GLM_FMT_MXFP4
    gu.call("glm_mx_quantize", gu.stream(), gu.p(gu.to_dev(w)), rows, cols, fmt, rule, gu.p(codes),
            gu.p(scales))
    np.testing.assert_array_equal(gu.host(scales), want_scales)
    np.testing.assert_array_equal(gu.host(codes), want_codes)


# --------------------------------------------------------------------------- router / dispatch


def _router_case(shape, seed, T=None, n_group=1, topk_group=1):
    layer = make_layer(shape, seed, T=T)
    return layer, MoEShape(shape.name, layer["x"].shape[0], shape.d, shape.E, shape.k, shape.I,
                           shape.I_shared, shape.routing, n_group, topk_group)


@pytest.mark.parametrize("name,T,groups", [
    ("decode_t1", None, (1, 1)),
    ("verify_t2", None, (1, 1)),
    ("batch_t64", None, (1, 1)),
    ("verify_t2", 300, (8, 4)),
    ("prefill_t4096", 1024, (1, 1)),
])
def test_router_parity(gu, name, T, groups):
    torch = _torch()
    shape, seed = SHAPES[name], 5300 + list(SHAPES).index(name)
    layer, sh = _router_case(shape, seed, T, *groups)
    T = sh.T
    x = O.bf16_bits_to_f32(layer["x"])
    logits, w, idx, choice = O.router(x, layer["router_weight"], layer["router_bias"], top_k=sh.k,
                                      n_group=sh.n_group, topk_group=sh.topk_group,
                                      norm_topk_prob=True, routed_scaling_factor=2.5)
    dl = gu.upload_layer({k: layer[k] for k in ("x", "router_weight", "router_bias")})
    g_logits = torch.empty((T, sh.E), dtype=torch.float32, device="cuda")
    g_w = torch.empty((T, sh.k), dtype=torch.float32, device="cuda")
    g_idx = torch.empty((T, sh.k), dtype=torch.int32, device="cuda")
    gu.call("glm_router_topk", gu.stream(), gu.p(dl["x"]), T, sh.d, gu.p(dl["router_weight"]),
            gu.p(dl["router_bias"]), sh.E, sh.k, sh.n_group, sh.topk_group, 1, 2.5, gu.p(g_logits),
            gu.p(g_w), gu.p(g_idx))
    np.testing.assert_allclose(gu.host(g_logits), logits, rtol=1e-4, atol=1e-5)
    got_idx = gu.host(g_idx).astype(np.uint32)
    ambiguous = _check_indices(got_idx, idx, choice, sh.k)
    assert ambiguous <= max(1, T // 100)
    same = np.all(got_idx == idx, axis=1)
    np.testing.assert_allclose(gu.host(g_w)[same], w[same], rtol=2e-6, atol=1e-7)


def test_router_reference_known_answer(gu):
    # reference tests/test_moe.py:10-23 through the kernel
    torch = _torch()
    x = np.zeros((1, 32), np.uint16)
    W = np.zeros((4, 32), np.float32)
    bias = np.array([10.0, 9.0, 1.0, 0.0], np.float32)
    lg = torch.empty((1, 4), dtype=torch.float32, device="cuda")
    w = torch.empty((1, 2), dtype=torch.float32, device="cuda")
    idx = torch.empty((1, 2), dtype=torch.int32, device="cuda")
    gu.call("glm_router_topk", gu.stream(), gu.p(gu.to_dev(x)), 1, 32, gu.p(gu.to_dev(W)),
            gu.p(gu.to_dev(bias)), 4, 2, 2, 1, 1, 2.5, gu.p(lg), gu.p(w), gu.p(idx))
    assert gu.host(idx).tolist() == [[1, 0]]
    np.testing.assert_allclose(gu.host(w), [[1.25, 1.25]], atol=1e-6)


@pytest.mark.parametrize("T,groups", [(2, (1, 1)), (40, (4, 2))])
def test_router_nan_choice_ranks_as_minus_inf(gu, T, groups):
    # a NaN router row (NaN logit, NaN choice) with a large bias: never chosen,
    # by the router kernel and by the few-token / decode layer kernels, as in
    # the oracle
    torch = _torch()
    shape = MoEShape("nan", T, 1024, 16, 4, 256, 0, n_group=groups[0], topk_group=groups[1])
    layer = make_layer(shape, 4242)
    layer["router_weight"][7, 5] = np.nan
    layer["router_bias"][:] = 0.0
    layer["router_bias"][7] = 5.0
    x = O.bf16_bits_to_f32(layer["x"])
    _, w, idx, choice = O.router(x, layer["router_weight"], layer["router_bias"], top_k=4,
                                 n_group=groups[0], topk_group=groups[1], norm_topk_prob=True,
                                 routed_scaling_factor=shape.routed_scaling_factor)
    assert not (idx == 7).any()
    dl = gu.upload_layer(layer)
    g_logits = torch.empty((T, 16), dtype=torch.float32, device="cuda")
    g_w = torch.empty((T, 4), dtype=torch.float32, device="cuda")
    g_idx = torch.empty((T, 4), dtype=torch.int32, device="cuda")
    gu.call("glm_router_topk", gu.stream(), gu.p(dl["x"]), T, 1024, gu.p(dl["router_weight"]),
            gu.p(dl["router_bias"]), 16, 4, groups[0], groups[1], 1,
            shape.routed_scaling_factor, gu.p(g_logits), gu.p(g_w), gu.p(g_idx))
    got = gu.host(g_idx).astype(np.uint32)
    assert not (got == 7).any()
    _check_indices(got, idx, choice, 4)
    _, _, l_idx = gu.run_layer(dl, shape, shared=False)
    got_l = gu.host(l_idx).astype(np.uint32)
    assert not (got_l == 7).any()
    _check_indices(got_l, idx, choice, 4)


def _row_tiles(e, off, c):
    """glm_moe_tiles' rule: ceil(c / 160) tiles, the 16-row blocks dealt out
    evenly (tile i starts at block floor(i B / nt))."""
    nt, blocks = -(-c // 160), -(-c // 16)
    starts = [16 * (i * blocks // nt) for i in range(nt)] + [c]
    return [(e, off + starts[i], min(starts[i + 1], c) - starts[i]) for i in range(nt)]


def _work_list(counts, offsets, active, E):
    work = np.tile(np.array([-1, 0, 0, 0], np.int32), (E, 1))
    for u, e in enumerate(active):
        work[u] = (e, offsets[e], counts[e], 0)
    return work


def _dispatch(gu, idx, E):
    torch = _torch()
    T, k = idx.shape
    P = T * k
    i32 = dict(dtype=torch.int32, device="cuda")
    bufs = {n: torch.full((s,), -7, **i32) for n, s in
            [("counts", E), ("offsets", E + 1), ("perm", P), ("inv", P), ("pair_token", P),
             ("active", E), ("num_active", 1), ("work", 4 * E), ("status", 1)]}
    gu.call("glm_moe_dispatch", gu.stream(), gu.p(gu.to_dev(idx.astype(np.uint32))), T, k, E,
            *(gu.p(bufs[n]) for n in ("counts", "offsets", "perm", "inv", "pair_token", "active",
                                      "num_active", "work", "status")))
    return {n: gu.host(t) for n, t in bufs.items()}


# (16384, 8, 288): the chunk histograms (128 x 288) exceed one workgroup's
# 64 KB, so count and scan run as separate kernels; every other case above
# 4096 pairs counts inside the scan's workgroup
@pytest.mark.parametrize("T,k,E,kind", [
    (1, 2, 16, "distinct"), (2, 8, 128, "distinct"), (64, 8, 128, "skew"),
    (4096, 8, 128, "distinct"), (3000, 8, 288, "skew"), (5, 4, 8, "dups"), (1, 1, 1, "distinct"),
    (16384, 8, 288, "dups"),
])
def test_dispatch_bit_exact(gu, T, k, E, kind):
    rng = np.random.default_rng(T * 31 + k + E)
    if kind == "distinct":
        idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
    elif kind == "skew":
        p = 1.0 / np.arange(1, E + 1) ** 1.1
        idx = np.stack([rng.choice(E, k, replace=False, p=p / p.sum()) for _ in range(T)])
    else:
        idx = rng.integers(0, E, (T, k))
    got = _dispatch(gu, idx, E)
    counts, offsets, perm, inv, active = O.dispatch(idx, E)
    np.testing.assert_array_equal(got["counts"], counts)
    np.testing.assert_array_equal(got["offsets"], offsets)
    np.testing.assert_array_equal(got["perm"], perm)
    np.testing.assert_array_equal(got["inv"], inv)
    np.testing.assert_array_equal(got["pair_token"], perm // k)
    assert got["num_active"][0] == len(active)
    np.testing.assert_array_equal(got["active"][: len(active)], active)
    assert np.all(got["active"][len(active):] == -1)
    np.testing.assert_array_equal(got["work"].reshape(E, 4), _work_list(counts, offsets, active, E))
    assert got["status"][0] == 0


@pytest.mark.parametrize("T,k,E", [(2, 2, 4), (900, 8, 32), (9000, 8, 448)])
def test_dispatch_flags_out_of_range(gu, T, k, E):
    # pairs with an index >= E are dropped on the one-workgroup path, the
    # chunk-parallel one with the counts in the scan's workgroup (900 x 8
    # pairs) and with a separate count kernel (9000 x 8 x 448): status 1, inv -1, the valid pairs
    # sorted as if the others were absent, -1 past them in perm and pair_token
    rng = np.random.default_rng(E + T)
    idx = rng.integers(0, E, (T, k)).astype(np.int64)
    bad = rng.random((T, k)) < 0.05
    bad.flat[1] = True
    idx[bad] = E + rng.integers(0, 3, int(bad.sum()))
    got = _dispatch(gu, idx, E)
    assert got["status"][0] == 1
    flat = idx.reshape(-1)
    valid = np.flatnonzero(flat < E)
    order = valid[np.argsort(flat[valid], kind="stable")]
    n = len(order)
    assert got["offsets"][-1] == n
    np.testing.assert_array_equal(got["counts"], np.bincount(flat[valid], minlength=E))
    np.testing.assert_array_equal(got["perm"][:n], order)
    np.testing.assert_array_equal(got["pair_token"][:n], order // k)
    assert np.all(got["perm"][n:] == -1) and np.all(got["pair_token"][n:] == -1)
    inv = np.full(T * k, -1)
    inv[order] = np.arange(n)
    np.testing.assert_array_equal(got["inv"], inv)


# --------------------------------------------------------------------------- experts


def _expert_parity(gu, shape, seed, T=None):
    torch = _torch()
    layer = make_layer(shape, seed, T=T)
    T = layer["x"].shape[0]
    k, E, d, I = shape.k, shape.E, shape.d, shape.I
    x = O.bf16_bits_to_f32(layer["x"])
    _, _, idx, _ = O.router(x, layer["router_weight"], layer["router_bias"], top_k=k, n_group=1,
                            topk_group=1, norm_topk_prob=True, routed_scaling_factor=2.5)
    y_want, inter = O.routed_experts(x, idx, _bank(layer), shape.swiglu_limit,
                                     return_intermediates=True)
    counts, offsets, perm, inv, active = O.dispatch(idx, E)
    dl = gu.upload_layer({key: layer[key] for key in ("x",) + BANK_KEYS})
    P = T * k
    i32 = dict(dtype=torch.int32, device="cuda")
    d_tok = gu.to_dev((perm // k).astype(np.int32))
    d_work = gu.to_dev(_work_list(counts, offsets, active, E))
    h = torch.empty((P, I), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((P, d), dtype=torch.bfloat16, device="cuda")
    gu.call("glm_expert_gate_up", gu.stream(), gu.p(dl["x"]), T, d, I, E, k,
            *(gu.p(dl[key]) for key in BANK_KEYS[:4]), gu.p(d_tok), gu.p(d_work),
            shape.swiglu_limit, gu.p(h))
    gu.call("glm_expert_down", gu.stream(), gu.p(h), T, k, I, d, E, gu.p(dl[BANK_KEYS[4]]),
            gu.p(dl[BANK_KEYS[5]]), gu.p(d_work), gu.p(y))
    h_got = O.bf16_bits_to_f32(gu.bf16_bits(h))[inv].reshape(T, k, I)
    y_got = O.bf16_bits_to_f32(gu.bf16_bits(y))[inv].reshape(T, k, d)
    return h_got, inter["h"], y_got, y_want


@pytest.mark.parametrize("name,T", [("decode_t1", None), ("verify_t2", None), ("batch_t64", None),
                                    ("verify_t2", 40)])
def test_routed_experts_parity(gu, name, T):
    shape = SHAPES[name]
    h_got, h_want, y_got, y_want = _expert_parity(gu, shape, 900 + len(name), T)
    assert O.rel_l2(h_got, h_want) < REL_L2
    assert O.rel_l2(y_got, y_want) < REL_L2
    # bf16 results differ from the oracle only by summation order: nearly all bit-exact
    assert np.mean(h_got == h_want) > 0.97
    assert np.mean(y_got == y_want) > 0.97


@pytest.mark.parametrize("name,T,E", [("decode_t1", None, None), ("verify_t2", None, None),
                                      ("verify_t2", 4, 256), ("verify_t2", 3, 300)])
def test_route_gate_up_parity(gu, name, T, E):
    # few-token fused selection + gate/up: routing bit-exact with the router,
    # h in pair order within the bf16 tolerance of the oracle
    torch = _torch()
    base = SHAPES[name]
    shape = MoEShape(base.name, base.T if T is None else T, base.d, E or base.E, base.k, base.I,
                     base.I_shared)
    layer = make_layer(shape, 61 + shape.T + shape.E)
    T, k, E, d, I = shape.T, shape.k, shape.E, shape.d, shape.I
    x = O.bf16_bits_to_f32(layer["x"])
    logits, w_want, idx_want, _ = O.router(x, layer["router_weight"], layer["router_bias"],
                                           top_k=k, n_group=1, topk_group=1,
                                           norm_topk_prob=True, routed_scaling_factor=2.5)
    _, inter = O.routed_experts(x, idx_want, _bank(layer), shape.swiglu_limit,
                                return_intermediates=True)
    dl = gu.upload_layer({key: layer[key] for key in ("x", "router_bias") + BANK_KEYS})
    d_logits = gu.to_dev(np.asarray(logits, np.float32))
    h = torch.empty((T * k, I), dtype=torch.bfloat16, device="cuda")
    w = torch.empty((T, k), dtype=torch.float32, device="cuda")
    idx = torch.empty((T, k), dtype=torch.int32, device="cuda")
    gu.call("glm_route_gate_up", gu.stream(), gu.p(d_logits), gu.p(dl["router_bias"]), T, E, k,
            1, 1, 1, 2.5, gu.p(dl["x"]), d, I, *(gu.p(dl[key]) for key in BANK_KEYS[:4]),
            shape.swiglu_limit, gu.p(w), gu.p(idx), gu.p(h))
    assert np.array_equal(gu.host(idx).astype(np.uint32), idx_want)
    np.testing.assert_allclose(gu.host(w), w_want, rtol=2e-6, atol=1e-7)
    h_got = O.bf16_bits_to_f32(gu.bf16_bits(h)).reshape(T, k, I)
    assert O.rel_l2(h_got, inter["h"]) < REL_L2
    assert np.mean(h_got == inter["h"]) > 0.97


def test_grouped_expert_gemms_parity(gu):
    # prefill grouped GEMMs through the C ABI: dispatch -> tiles -> gate/up -> down
    torch = _torch()
    shape = MoEShape("grouped", 400, 1024, 32, 4, 256, 0)
    layer = make_layer(shape, 1717)
    T, k, E, d, I = shape.T, shape.k, shape.E, shape.d, shape.I
    x = O.bf16_bits_to_f32(layer["x"])
    _, _, idx, _ = O.router(x, layer["router_weight"], layer["router_bias"], top_k=k, n_group=1,
                            topk_group=1, norm_topk_prob=True, routed_scaling_factor=2.5)
    y_want, inter = O.routed_experts(x, idx, _bank(layer), shape.swiglu_limit,
                                     return_intermediates=True)
    counts, offsets, perm, inv, active = O.dispatch(idx, E)
    dl = gu.upload_layer({key: layer[key] for key in ("x",) + BANK_KEYS})
    P = T * k
    max_tiles = (P + 127) // 128 + E
    work = gu.to_dev(_work_list(counts, offsets, active, E))
    tiles = torch.empty((max_tiles, 4), dtype=torch.int32, device="cuda")
    ntiles = torch.empty(1, dtype=torch.int32, device="cuda")
    gu.call("glm_moe_tiles", gu.stream(), gu.p(work), E, gu.p(tiles), gu.p(ntiles))
    want_tiles = [t for e in active for t in _row_tiles(e, int(offsets[e]), int(counts[e]))]
    assert int(gu.host(ntiles)[0]) == len(want_tiles)
    got_tiles = [tuple(int(v) for v in t[:3]) for t in gu.host(tiles)[:len(want_tiles)]]
    assert got_tiles == want_tiles
    # the tiles partition every expert's rows, at most 160 rows each, all but
    # an expert's last a whole number of 16-row blocks, the fewest possible
    for e in active:
        mine = [t for t in got_tiles if t[0] == e]
        assert len(mine) == -(-int(counts[e]) // 160)
        assert mine[0][1] == int(offsets[e])
        assert all(a[1] + a[2] == b[1] for a, b in zip(mine, mine[1:]))
        assert mine[-1][1] + mine[-1][2] == int(offsets[e]) + int(counts[e])
        assert all(0 < t[2] <= 160 for t in mine) and all(t[2] % 16 == 0 for t in mine[:-1])
    d_tok = gu.to_dev((perm // k).astype(np.int32))
    h = torch.empty((P, I), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((P, d), dtype=torch.bfloat16, device="cuda")
    lib = native.load()
    x_split = gu.workspace(lib.glm_act_split_bytes(T, d))
    h_split = gu.workspace(lib.glm_act_split_bytes(P, I))
    gu.call("glm_act_split_fp8", gu.stream(), gu.p(dl["x"]), T, d, gu.p(x_split))
    gu.call("glm_expert_gate_up_grouped", gu.stream(), gu.p(x_split), T, d, I,
            *(gu.p(dl[key]) for key in BANK_KEYS[:4]), gu.p(d_tok), gu.p(tiles), gu.p(ntiles),
            max_tiles, shape.swiglu_limit, gu.p(h))
    gu.call("glm_act_split_fp8", gu.stream(), gu.p(h), P, I, gu.p(h_split))
    gu.call("glm_expert_down_grouped", gu.stream(), gu.p(h_split), P, I, d,
            gu.p(dl[BANK_KEYS[4]]), gu.p(dl[BANK_KEYS[5]]), gu.p(tiles), gu.p(ntiles), max_tiles,
            gu.p(y))
    h_got = O.bf16_bits_to_f32(gu.bf16_bits(h))[inv].reshape(T, k, I)
    y_got = O.bf16_bits_to_f32(gu.bf16_bits(y))[inv].reshape(T, k, d)
    assert O.rel_l2(h_got, inter["h"]) < REL_L2 and np.mean(h_got == inter["h"]) > 0.97
    assert O.rel_l2(y_got, y_want) < REL_L2 and np.mean(y_got == y_want) > 0.97


def test_moe_forward_grouped_equals_public_composition(gu):
    # glm_moe_forward's grouped path (multi-workgroup dispatch, h split fused
    # into the gate/up epilogue) must equal, bit for bit, the public entry
    # points composed by hand on the forward's own route: dispatch, tiles, x
    # split, gate/up to bf16 h, split of h, down, combine.  Its route (bf16
    # MFMA on the f32 router weights split three ways) is checked against the
    # oracle's.
    torch = _torch()
    shape = MoEShape("grouped", 400, 1024, 32, 4, 256, 0)
    layer = make_layer(shape, 1718)
    T, k, E, d, I = shape.T, shape.k, shape.E, shape.d, shape.I
    P = T * k
    dl = gu.upload_layer(layer)
    lib = native.load()
    ws_bytes = lib.glm_moe_workspace_bytes(T, d, E, k, I, 0)
    ws = gu.workspace(ws_bytes)
    f32 = dict(dtype=torch.float32, device="cuda")
    i32 = dict(dtype=torch.int32, device="cuda")
    out = torch.empty((T, d), **f32)
    wts, idx = torch.empty((T, k), **f32), torch.empty((T, k), **i32)
    gu.call("glm_moe_forward", gu.stream(), gu.p(dl["x"]), T, d, gu.p(dl["router_weight"]),
            gu.p(dl["router_bias"]), E, k, 1, 1, 1, shape.routed_scaling_factor, I,
            *(gu.p(dl[key]) for key in BANK_KEYS), 0, native.GLM_FMT_BF16, None, None, None,
            None, None, None, None, shape.swiglu_limit, gu.p(ws), ws_bytes, gu.p(out), gu.p(wts),
            gu.p(idx))
    # the forward's route against the oracle's: same experts wherever the
    # top-k margin is clear, weights to f32 rounding
    _, w_want, i_want, choice = O.router(O.bf16_bits_to_f32(layer["x"]), layer["router_weight"],
                                         layer["router_bias"], top_k=k, n_group=1, topk_group=1,
                                         norm_topk_prob=True,
                                         routed_scaling_factor=shape.routed_scaling_factor)
    got_i = gu.host(idx).astype(np.uint32)
    assert _check_indices(got_i, i_want, choice, k) <= max(1, T // 100)
    same = np.all(got_i == i_want, axis=1)
    np.testing.assert_allclose(gu.host(wts)[same], w_want[same], rtol=2e-6, atol=1e-7)
    b = {n: torch.empty((s,), **i32) for n, s in
         [("counts", E), ("offsets", E + 1), ("perm", P), ("inv", P), ("tok", P), ("active", E),
          ("num_active", 1), ("work", 4 * E), ("status", 1)]}
    gu.call("glm_moe_dispatch", gu.stream(), gu.p(idx), T, k, E, *(gu.p(b[n]) for n in
            ("counts", "offsets", "perm", "inv", "tok", "active", "num_active", "work", "status")))
    max_tiles = (P + 127) // 128 + E
    tiles, ntiles = torch.empty((max_tiles, 4), **i32), torch.empty(1, **i32)
    gu.call("glm_moe_tiles", gu.stream(), gu.p(b["work"]), E, gu.p(tiles), gu.p(ntiles))
    x_split = gu.workspace(lib.glm_act_split_bytes(T, d))
    h_split = gu.workspace(lib.glm_act_split_bytes(P, I))
    h = torch.empty((P, I), dtype=torch.bfloat16, device="cuda")
    y = torch.empty((P, d), dtype=torch.bfloat16, device="cuda")
    gu.call("glm_act_split_fp8", gu.stream(), gu.p(dl["x"]), T, d, gu.p(x_split))
    gu.call("glm_expert_gate_up_grouped", gu.stream(), gu.p(x_split), T, d, I,
            *(gu.p(dl[key]) for key in BANK_KEYS[:4]), gu.p(b["tok"]), gu.p(tiles), gu.p(ntiles),
            max_tiles, shape.swiglu_limit, gu.p(h))
    gu.call("glm_act_split_fp8", gu.stream(), gu.p(h), P, I, gu.p(h_split))
    gu.call("glm_expert_down_grouped", gu.stream(), gu.p(h_split), P, I, d,
            gu.p(dl[BANK_KEYS[4]]), gu.p(dl[BANK_KEYS[5]]), gu.p(tiles), gu.p(ntiles), max_tiles,
            gu.p(y))
    want = torch.empty((T, d), **f32)
    gu.call("glm_moe_combine", gu.stream(), gu.p(y), gu.p(b["inv"]), gu.p(wts), None, T, k, d,
            gu.p(want))
    assert np.array_equal(gu.host(out).view(np.uint32), gu.host(want).view(np.uint32))


def _split_model(xb, K):
    """numpy model of the FP8 activation split: per 32-element group the
    smallest E8M0 scale keeping the group within 448, hi = RNE E4M3FN of the
    scaled group, lo = RNE E4M3FN of the exact residual under its own scale."""
    x = O.bf16_bits_to_f32(xb).reshape(-1, K // 32, 32)

    def scale_byte(amax):
        m, e = np.frexp(amax.astype(np.float64))
        k = np.where(m <= 0.875, e - 9, e - 8)
        return np.where(amax > 0, np.clip(k + 127, 0, 254), 127).astype(np.int64)

    bh = scale_byte(np.abs(x).max(axis=2))
    hi = O.e4m3fn_encode(np.ldexp(x, (127 - bh)[..., None]))
    back = (O.e4m3fn_table()[hi].astype(np.float64) * np.ldexp(1.0, bh - 127)[..., None])
    r = (x.astype(np.float64) - back).astype(np.float32)
    bl = scale_byte(np.abs(r).max(axis=2))
    lo = O.e4m3fn_encode(np.ldexp(r, (127 - bl)[..., None]))
    return hi.reshape(-1, K), lo.reshape(-1, K), bh.astype(np.uint8), bl.astype(np.uint8)


def _split_parts(buf, rows, K):
    def up(v):
        return (v + 255) // 256 * 256
    raw = buf.cpu().numpy()
    c, sc = up(rows * K), up(rows * K // 32)
    return (raw[:rows * K].reshape(rows, K), raw[c:c + rows * K].reshape(rows, K),
            raw[2 * c:2 * c + rows * K // 32].reshape(rows, K // 32),
            raw[2 * c + sc:2 * c + sc + rows * K // 32].reshape(rows, K // 32))


def test_act_split_fp8_exact(gu):
    # the FP8 split of bf16 activations: codes and scales bit-exact against
    # the numpy model, and hi + lo reproduce every element exactly for
    # normal-range data (groups of N(0, s) with s over 12 binades, zero groups,
    # single-element groups)
    rng = np.random.default_rng(29)
    rows, K = 96, 512
    x = rng.normal(0, 1, (rows, K // 32, 32)) * np.ldexp(1.0, rng.integers(-6, 6, (rows, K // 32, 1)))
    x[0, :3] = 0.0
    x[1, 0, 1:] = 0.0
    xb = O.f32_to_bf16_bits(x.reshape(rows, K).astype(np.float32))
    lib = native.load()
    buf = gu.workspace(lib.glm_act_split_bytes(rows, K))
    gu.call("glm_act_split_fp8", gu.stream(), gu.p(gu.to_dev(xb)), rows, K, gu.p(buf))
    hi, lo, shi, slo = _split_parts(buf, rows, K)
    w_hi, w_lo, w_shi, w_slo = _split_model(xb, K)
    assert np.array_equal(shi, w_shi.reshape(rows, -1)) and np.array_equal(slo, w_slo.reshape(rows, -1))
    assert np.array_equal(hi, w_hi) and np.array_equal(lo, w_lo)
    tab = O.e4m3fn_table().astype(np.float64)
    recon = (tab[hi].reshape(rows, -1, 32) * np.ldexp(1.0, shi.astype(np.int64) - 127)[..., None]
             + tab[lo].reshape(rows, -1, 32) * np.ldexp(1.0, slo.astype(np.int64) - 127)[..., None])
    assert np.array_equal(recon.reshape(rows, K), O.bf16_bits_to_f32(xb).astype(np.float64))


def test_act_split_fp8_extreme_scales(gu):
    # the split at the ends of the E8M0 range: groups of bf16 denormals and
    # near-denormals (scale byte 0), groups near the bf16 maximum (byte ~245),
    # and groups with one large element over small ones (the lo term's scale
    # far below hi's); codes and scales bit-exact against the numpy model
    rng = np.random.default_rng(31)
    rows, K = 64, 256
    g = K // 32
    x = rng.normal(0, 1, (rows, g, 32))
    binade = np.empty((rows, g, 1), dtype=np.int64)
    binade[:16] = rng.integers(-140, -118, (16, g, 1))   # tiny: scale byte 0 .. a few
    binade[16:32] = rng.integers(110, 125, (16, g, 1))   # huge: scale byte ~234 .. 245
    binade[32:] = rng.integers(-20, 20, (rows - 32, g, 1))
    x = x * np.ldexp(1.0, binade)
    x[32:48, :, 0] *= np.ldexp(1.0, 40)                  # one element 2^40 above the rest
    x[48:, :, 5] = np.ldexp(1.0, rng.integers(-30, 30, (rows - 48, g)))
    xb = O.f32_to_bf16_bits(x.reshape(rows, K).astype(np.float32))
    lib = native.load()
    buf = gu.workspace(lib.glm_act_split_bytes(rows, K))
    gu.call("glm_act_split_fp8", gu.stream(), gu.p(gu.to_dev(xb)), rows, K, gu.p(buf))
    hi, lo, shi, slo = _split_parts(buf, rows, K)
    w_hi, w_lo, w_shi, w_slo = _split_model(xb, K)
    assert (w_shi == 0).any() and w_shi.max() >= 240  # both ends of the range are reached
    assert np.array_equal(shi, w_shi.reshape(rows, -1)) and np.array_equal(slo, w_slo.reshape(rows, -1))
    assert np.array_equal(hi, w_hi) and np.array_equal(lo, w_lo)


def test_routed_experts_generic_shapes(gu):
    # tiny geometry of the reference's tests (tests/helpers.py: d=32, I=32) and
    # one more that is not a multiple of the 128-wide MFMA chunk
    for d, I, E, k, T in [(32, 32, 4, 2, 3), (96, 64, 5, 3, 7)]:
        shape = MoEShape("tiny", T=T, d=d, E=E, k=k, I=I, I_shared=32)
        h_got, h_want, y_got, y_want = _expert_parity(gu, shape, 11 + d, T)
        assert O.rel_l2(y_got, y_want) < REL_L2
        assert np.mean(y_got == y_want) > 0.95


def _swiglu_gpu(gu, g_bits, u_bits, limit):
    torch = _torch()
    out = torch.empty(g_bits.size, dtype=torch.bfloat16, device="cuda")
    gu.call("glm_limited_swiglu", gu.stream(), gu.p(gu.to_dev(g_bits)), gu.p(gu.to_dev(u_bits)),
            g_bits.size, limit, gu.p(out))
    return gu.bf16_bits(out)


def test_limited_swiglu_rounding_bit_exact(gu):
    # gates in [9, 10] have bf16(sigmoid) == 1 exactly, so each output is the
    # round-to-nearest-even bf16 of the exact f32 product g*u: ties, subnormal
    # and normal results, both signs
    rng = np.random.default_rng(17)
    n = 1 << 16
    g = O.f32_to_bf16_bits(rng.uniform(9.0, 10.0, n).astype(np.float32))
    u = np.concatenate([rng.normal(0, 1, n // 4), rng.normal(0, 1, n // 4) * 1e-38,
                        rng.normal(0, 1, n // 4) * 1e-36, rng.uniform(-10, 10, n // 4)])
    u = O.f32_to_bf16_bits(u.astype(np.float32))
    want = O.f32_to_bf16_bits(O.limited_swiglu_bf16(O.bf16_bits_to_f32(g),
                                                    O.bf16_bits_to_f32(u), 10.0))
    got = _swiglu_gpu(gu, g, u, 10.0)
    np.testing.assert_array_equal(got, want)


def test_limited_swiglu_general(gu):
    # any gate: the f32 sigmoid may differ from the oracle's exp by an ulp, which
    # moves bf16(sigmoid) only when it lies on a rounding boundary
    rng = np.random.default_rng(18)
    n = 1 << 16
    g = O.f32_to_bf16_bits((rng.normal(0, 4, n)).astype(np.float32))
    u = O.f32_to_bf16_bits((rng.normal(0, 4, n)).astype(np.float32))
    for limit in (7.0, 0.0):
        want = O.f32_to_bf16_bits(O.limited_swiglu_bf16(O.bf16_bits_to_f32(g),
                                                        O.bf16_bits_to_f32(u), limit))
        got = _swiglu_gpu(gu, g, u, limit)
        assert np.mean(got == want) > 0.999
        assert np.max(np.abs(got.astype(np.int32) - want.astype(np.int32))) <= 1


def test_limited_swiglu_nan_and_infinities(gu):
    # NaN in the gate or the up value passes the clamps (mx.minimum / mx.clip),
    # +-inf is clamped to the limit, a gate of -inf without a limit gives NaN
    vals = np.float32([np.nan, np.inf, -np.inf, 0.0, -0.0, 1.0, -3.0, 12.0, -12.0])
    g, u = (a.ravel() for a in np.meshgrid(vals, vals, indexing="ij"))
    gb, ub = O.f32_to_bf16_bits(g), O.f32_to_bf16_bits(u)
    for limit in (10.0, 0.0):
        want = O.f32_to_bf16_bits(O.limited_swiglu_bf16(O.bf16_bits_to_f32(gb),
                                                        O.bf16_bits_to_f32(ub), limit))
        got = _swiglu_gpu(gu, gb, ub, limit)
        gf, wf = O.bf16_bits_to_f32(got), O.bf16_bits_to_f32(want)
        assert np.array_equal(np.isnan(gf), np.isnan(wf))
        np.testing.assert_array_equal(got[~np.isnan(wf)], want[~np.isnan(wf)])


@pytest.mark.parametrize("T,d,E,k,I,Is", [(2, 2048, 128, 8, 768, 768), (40, 1024, 64, 8, 512, 512),
                                          (200, 2048, 64, 8, 768, 0)])
def test_moe_layer_nan_gate_scale(gu, T, d, E, k, I, Is):
    # one routed expert's gate row with a NaN scale byte (E8M0 255): its gate
    # value is NaN beside a finite up value, the NaN passes the SwiGLU clamp and
    # every output of the tokens routed to that expert is NaN -- on the
    # few-token, decode and grouped paths, as in the oracle
    shape = MoEShape("nan_scale", T, d, E, k, I, Is)
    layer = make_layer(shape, 6100 + T)
    _, _, i0, _ = O.router(O.bf16_bits_to_f32(layer["x"]), layer["router_weight"],
                           layer["router_bias"], top_k=k, n_group=1, topk_group=1,
                           norm_topk_prob=True, routed_scaling_factor=shape.routed_scaling_factor)
    # token 0's expert shared by the fewest tokens, so that some rows stay finite
    e = int(min(i0[0], key=lambda c: (i0 == c).any(axis=1).sum()))
    layer["gate_proj.weight_scale"][e, 5, 1] = 255
    want, inter = _oracle_layer(layer, shape, shared=Is > 0)
    hit = (inter["indices"] == e).any(axis=1)
    assert hit.any() and not hit.all()
    assert np.array_equal(np.isnan(want).all(axis=1), hit) and not np.isnan(want[~hit]).any()
    out, w, idx = gu.run_layer(gu.upload_layer(layer), shape, shared=Is > 0)
    got_idx = gu.host(idx).astype(np.uint32)
    _check_indices(got_idx, inter["indices"], inter["choice"], k)
    same = np.all(got_idx == inter["indices"], axis=1)
    assert same[0] and same.sum() >= T - 1
    got = gu.host(out)
    assert np.array_equal(np.isnan(got[same]), np.isnan(want[same]))
    ok = same & ~hit
    assert O.rel_l2(got[ok], want[ok]) < REL_L2


def test_combine_bit_exact(gu):
    torch = _torch()
    rng = np.random.default_rng(3)
    T, k, d = 5, 4, 256
    y = O.f32_to_bf16_bits(rng.normal(0, 1, (T * k, d)).astype(np.float32))
    w = rng.uniform(0, 1, (T, k)).astype(np.float32)
    shared = O.f32_to_bf16_bits(rng.normal(0, 1, (T, d)).astype(np.float32))
    inv = rng.permutation(T * k).astype(np.int32)
    want = O.combine(O.bf16_bits_to_f32(y)[inv].reshape(T, k, d), w, O.bf16_bits_to_f32(shared))
    out = torch.empty((T, d), dtype=torch.float32, device="cuda")
    gu.call("glm_moe_combine", gu.stream(), gu.p(gu.to_dev(y)), gu.p(gu.to_dev(inv)),
            gu.p(gu.to_dev(w)), gu.p(gu.to_dev(shared)), T, k, d, gu.p(out))
    np.testing.assert_array_equal(gu.host(out).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt,T", [(native.GLM_FMT_BF16, 3), (native.GLM_FMT_MXFP8, 3),
                                   (native.GLM_FMT_BF16, 300)])
def test_dense_mlp_parity(gu, fmt, T):
    # T=300 runs the tiled MFMA GEMMs (dense mode of the grouped kernels)
    torch = _torch()
    rng = np.random.default_rng(21)
    d, I = 2048, 768
    ws = [O.f32_to_bf16_bits(rng.normal(0, 0.02, s).astype(np.float32)) for s in [(I, d), (I, d), (d, I)]]
    x = O.f32_to_bf16_bits(rng.normal(0, 1, (T, d)).astype(np.float32))
    if fmt == native.GLM_FMT_BF16:
        mats = [O.bf16_bits_to_f32(w) for w in ws]
        dev = [(gu.to_dev(w), None) for w in ws]
    else:
        q = [O.quantize_mx(w, 8, O.MX_RULE_NEAREST) for w in ws]
        mats = [O.dequant_mxfp8(c, s) for c, s in q]
        dev = [(gu.to_dev(c), gu.to_dev(s)) for c, s in q]
    want = O.dense_mlp(O.bf16_bits_to_f32(x), *mats, 10.0)
    h = torch.empty((T, I), dtype=torch.bfloat16, device="cuda")
    out = torch.empty((T, d), dtype=torch.bfloat16, device="cuda")
    gu.call("glm_dense_mlp", gu.stream(), gu.p(gu.to_dev(x)), T, d, I, fmt,
            gu.p(dev[0][0]), gu.p(dev[0][1]), gu.p(dev[1][0]), gu.p(dev[1][1]), gu.p(dev[2][0]),
            gu.p(dev[2][1]), 10.0, gu.p(h), gu.p(out))
    got = O.bf16_bits_to_f32(gu.bf16_bits(out))
    assert O.rel_l2(got, want) < REL_L2
    assert np.mean(got == want) > 0.97


@pytest.mark.parametrize("fmt", [native.GLM_FMT_MXFP8, native.GLM_FMT_MXFP4, native.GLM_FMT_BF16])
@pytest.mark.parametrize("T", [1, 3, 4, 5, 20])
def test_linear_parity_and_f32_input(gu, fmt, T):
    # T <= 4 runs the vector-ALU rows kernel, T > 4 the MFMA tiles; the f32
    # entry point must equal glm_linear of the bf16 cast bit for bit
    torch = _torch()
    rng = np.random.default_rng(5310 + T)
    out_f, in_f = 1024, 2048
    w = O.f32_to_bf16_bits(rng.normal(0, 0.02, (out_f, in_f)).astype(np.float32))
    if fmt == native.GLM_FMT_BF16:
        mat, codes, scales = O.bf16_bits_to_f32(w), gu.to_dev(w), None
    else:
        c, sc = O.quantize_mx(w, 8 if fmt == native.GLM_FMT_MXFP8 else 4, O.MX_RULE_NEAREST)
        mat = O.dequant_mxfp8(c, sc) if fmt == native.GLM_FMT_MXFP8 else O.dequant_mxfp4(c, sc)
        codes, scales = gu.to_dev(c), gu.to_dev(sc)
    x32 = (rng.normal(0, 1, (T, in_f)) * (1 + 2.0 ** -12)).astype(np.float32)  # not bf16 values
    xb = O.f32_to_bf16_bits(x32)
    want = O.linear_bf16(O.bf16_bits_to_f32(xb), mat)
    y = torch.empty((T, out_f), dtype=torch.bfloat16, device="cuda")
    gu.call("glm_linear", gu.stream(), gu.p(gu.to_dev(xb)), T, in_f, gu.p(codes), gu.p(scales),
            fmt, out_f, gu.p(y))
    got = O.bf16_bits_to_f32(gu.bf16_bits(y))
    assert O.rel_l2(got, want) < REL_L2
    assert np.mean(got == want) > 0.97
    y32 = torch.empty_like(y)
    x32_dev = torch.from_numpy(x32).cuda()
    if T <= 4:
        gu.call("glm_linear_f32", gu.stream(), gu.p(x32_dev), T, in_f, gu.p(codes), gu.p(scales),
                fmt, out_f, gu.p(y32))
        assert np.array_equal(gu.bf16_bits(y32), gu.bf16_bits(y))
    else:
        rc = native.load().glm_linear_f32(gu.stream(), gu.p(x32_dev), T, in_f, gu.p(codes),
                                          gu.p(scales), fmt, out_f, gu.p(y32))
        assert rc == native.GLM_ERR_UNSUPPORTED_SHAPE


@pytest.mark.parametrize("in_f", [1024, 2048, 4096])
@pytest.mark.parametrize("T", [1, 4])
@pytest.mark.parametrize("weighted", [True, False])
def test_rms_norm_linear_parity(gu, in_f, T, weighted):
    # the fused RMSNorm + MXFP8 linear against the oracle's norm (mhc_oracle.rms_norm,
    # layers.py:119-140) rounded to bf16 and its linear; K = 1024 and 2048 take the
    # norm from the pass's own loads, 4096 from a pre-pass over the row; and against
    # glm_rms_norm + glm_linear (the same arithmetic up to the sum-of-squares order)
    from oracle import mhc_oracle as H
    torch = _torch()
    rng = np.random.default_rng(5510 + in_f + T + weighted)
    out_f, eps = 512, 1e-6
    w = O.f32_to_bf16_bits(rng.normal(0, 0.02, (out_f, in_f)).astype(np.float32))
    c, sc = O.quantize_mx(w, 8, O.MX_RULE_NEAREST)
    mat = O.dequant_mxfp8(c, sc)
    codes, scales = gu.to_dev(c), gu.to_dev(sc)
    x32 = (rng.normal(0, 1, (T, in_f)) * rng.uniform(0.1, 300.0, (T, 1))).astype(np.float32)
    nw = rng.normal(1.0, 0.1, in_f).astype(np.float32) if weighted else None
    xn = O.f32_to_bf16_bits(H.rms_norm(x32, nw, eps))
    want = O.linear_bf16(O.bf16_bits_to_f32(xn), mat)
    y = torch.empty((T, out_f), dtype=torch.bfloat16, device="cuda")
    x_dev = torch.from_numpy(x32).cuda()
    nw_dev = torch.from_numpy(nw).cuda() if weighted else None
    gu.call("glm_rms_norm_linear", gu.stream(), gu.p(x_dev), T, in_f, gu.p(nw_dev), eps,
            gu.p(codes), gu.p(scales), native.GLM_FMT_MXFP8, out_f, gu.p(y))
    got = O.bf16_bits_to_f32(gu.bf16_bits(y))
    assert O.rel_l2(got, want) < REL_L2
    assert np.mean(got == want) > 0.97
    xb = torch.empty((T, in_f), dtype=torch.bfloat16, device="cuda")
    gu.call("glm_rms_norm", gu.stream(), gu.p(x_dev), T, in_f, gu.p(nw_dev), eps, None, gu.p(xb))
    y2 = torch.empty_like(y)
    gu.call("glm_linear", gu.stream(), gu.p(xb), T, in_f, gu.p(codes), gu.p(scales),
            native.GLM_FMT_MXFP8, out_f, gu.p(y2))
    assert np.mean(gu.bf16_bits(y) == gu.bf16_bits(y2)) > 0.99


@pytest.mark.parametrize("in_f", [1024, 2304, 4096])
@pytest.mark.parametrize("T", [1, 4])
def test_linear_mxfp8_column_steps(gu, in_f, T):
    # the MXFP8 few-token linear walks K in passes of eight 256-column steps:
    # K = 1024 fills half a pass, 2304 one pass and one step, 4096 two passes
    torch = _torch()
    rng = np.random.default_rng(5410 + in_f + T)
    out_f = 512
    w = O.f32_to_bf16_bits(rng.normal(0, 0.02, (out_f, in_f)).astype(np.float32))
    c, sc = O.quantize_mx(w, 8, O.MX_RULE_NEAREST)
    mat = O.dequant_mxfp8(c, sc)
    codes, scales = gu.to_dev(c), gu.to_dev(sc)
    x32 = (rng.normal(0, 1, (T, in_f)) * (1 + 2.0 ** -12)).astype(np.float32)
    xb = O.f32_to_bf16_bits(x32)
    want = O.linear_bf16(O.bf16_bits_to_f32(xb), mat)
    y = torch.empty((T, out_f), dtype=torch.bfloat16, device="cuda")
    gu.call("glm_linear", gu.stream(), gu.p(gu.to_dev(xb)), T, in_f, gu.p(codes), gu.p(scales),
            native.GLM_FMT_MXFP8, out_f, gu.p(y))
    got = O.bf16_bits_to_f32(gu.bf16_bits(y))
    assert O.rel_l2(got, want) < REL_L2
    assert np.mean(got == want) > 0.97
    y32 = torch.empty_like(y)
    gu.call("glm_linear_f32", gu.stream(), gu.p(torch.from_numpy(x32).cuda()), T, in_f,
            gu.p(codes), gu.p(scales), native.GLM_FMT_MXFP8, out_f, gu.p(y32))
    assert np.array_equal(gu.bf16_bits(y32), gu.bf16_bits(y))


# --------------------------------------------------------------------------- whole layer


@pytest.mark.parametrize("name", ["decode_t1", "verify_t2", "batch_t64"])
def test_moe_layer_parity(gu, name):
    shape = SHAPES[name]
    layer = make_layer(shape, 5300 + list(SHAPES).index(name))
    want, inter = _oracle_layer(layer, shape)
    out, w, idx = gu.run_layer(gu.upload_layer(layer), shape)
    got_idx = gu.host(idx).astype(np.uint32)
    _check_indices(got_idx, inter["indices"], inter["choice"], shape.k)
    assert np.array_equal(got_idx, inter["indices"]), "standard seeds have no near-ties"
    np.testing.assert_allclose(gu.host(w), inter["weights"], rtol=2e-6, atol=1e-7)
    assert O.rel_l2(gu.host(out), want) < REL_L2


# Shapes around the few-token (T <= 4, k <= 8) and decode (T <= 64) kernel
# paths: expert counts per lane 1..8, k not a multiple of 4, idle waves, group
# masks, the smallest and largest chunk counts, with and without the shared expert.
SMALL_LAYERS = [
    # T, d, E, k, I, Is, (n_group, topk_group)
    (1, 1024, 64, 6, 256, 256, (1, 1)),
    (3, 1024, 256, 8, 512, 128, (8, 4)),
    (4, 3072, 32, 4, 768, 0, (4, 2)),
    (2, 4096, 16, 3, 1024, 512, (1, 1)),
    # two 16-row tiles per routed block (32 pairs x 48 tiles)
    (4, 2048, 64, 8, 768, 768, (1, 1)),
    (4, 2048, 448, 8, 128, 256, (1, 1)),
    (5, 1024, 64, 6, 256, 256, (1, 1)),
    (9, 2048, 96, 5, 384, 0, (3, 2)),
    # grouped MFMA GEMMs (T > 64): partial tiles, experts spanning two tiles
    (96, 1024, 16, 4, 256, 256, (1, 1)),
    (600, 1024, 16, 4, 256, 256, (1, 1)),
    (200, 2048, 64, 8, 768, 0, (4, 2)),
    # many pairs: the multi-workgroup dispatch (6 chunks of 1024 pairs, the last partial)
    (700, 1024, 32, 8, 256, 0, (1, 1)),
    # the decode path beyond 16 tokens (MFMA router, per-token selection, token groups)
    (40, 1024, 64, 8, 512, 512, (1, 1)),
    # 33-64 tokens at d % 2048 == 0: the shared gate/up tiles in the router's
    # launch (a partial last token tile and token group)
    (50, 2048, 64, 8, 768, 768, (1, 1)),
    # 16-32 tokens: the shared expert's tiles in the routed expert kernels (two
    # chunks per shared down K range; one chunk at I_shared 128, two token groups)
    (16, 2048, 64, 8, 768, 768, (1, 1)),
    (24, 1024, 32, 4, 256, 128, (2, 1)),
    (32, 4096, 24, 8, 2048, 1024, (1, 1)),
    # k = 64, every expert of E = 64 chosen by every token (the top-k upper bound)
    (3, 256, 64, 64, 64, 64, (1, 1)),
    # the real expert geometry with few experts (d = 4096, I = 2048, I_shared 1024)
    (3, 4096, 24, 8, 2048, 1024, (1, 1)),
    # shapes the decode kernels do not cover (d / 512 = 3) but the grouped GEMMs
    # do: up to 64 tokens they run the tiled GEMV kernels over the work list with
    # many pairs per expert (several 16-token batches, the act_index loop), from
    # 65 tokens the grouped GEMMs -- both sides of the threshold
    (40, 1536, 8, 8, 256, 256, (1, 1)),
    (64, 1536, 16, 8, 256, 256, (1, 1)),
    (65, 1536, 16, 8, 256, 256, (1, 1)),
    # the real GLM expert geometry (d 4096, I 2048: 16 chunks of 128 in the down
    # projection): E 288 on the few-token path; 64 tokens over 24 experts on the
    # decode path (~21 pairs per expert, two 16-row h batches)
    (2, 4096, 288, 8, 2048, 2048, (1, 1)),
    (64, 4096, 24, 8, 2048, 2048, (1, 1)),
]


@pytest.mark.parametrize("T,d,E,k,I,Is,groups", SMALL_LAYERS)
def test_moe_layer_small_shapes(gu, T, d, E, k, I, Is, groups):
    shape = MoEShape("small", T, d, E, k, I, Is, n_group=groups[0], topk_group=groups[1])
    layer = make_layer(shape, 900 + T * 7 + k)
    if T * d * I > (1 << 28):
        # large: the route from the numpy oracle, the layer from its C restatement
        from oracle import cpu as cpu_oracle
        x = O.bf16_bits_to_f32(layer["x"])
        _, w_r, i_r, choice = O.router(x, layer["router_weight"], layer["router_bias"], top_k=k,
                                       n_group=groups[0], topk_group=groups[1],
                                       norm_topk_prob=True,
                                       routed_scaling_factor=shape.routed_scaling_factor)
        want, _, c_idx = cpu_oracle.moe_layer(layer, shape, shared=Is > 0)
        assert np.array_equal(c_idx, i_r)
        inter = {"indices": i_r, "weights": w_r, "choice": choice}
    else:
        want, inter = _oracle_layer(layer, shape, shared=Is > 0)
    out, w, idx = gu.run_layer(gu.upload_layer(layer), shape, shared=Is > 0)
    got_idx = gu.host(idx).astype(np.uint32)
    _check_indices(got_idx, inter["indices"], inter["choice"], k)
    same = np.all(got_idx == inter["indices"], axis=1)
    assert same.sum() >= T - 1
    np.testing.assert_allclose(gu.host(w)[same], inter["weights"][same], rtol=2e-6, atol=1e-7)
    assert O.rel_l2(gu.host(out)[same], want[same]) < REL_L2


def test_moe_layer_grouped_skewed_routing(gu):
    # Zipf-biased routing: a few experts take several 128-row tiles, many take
    # one partial tile or none
    shape = MoEShape("skew", 512, 1024, 32, 4, 256, 256, routing="zipf")
    layer = make_layer(shape, 4711)
    want, inter = _oracle_layer(layer, shape)
    counts = np.bincount(inter["indices"].reshape(-1).astype(np.int64), minlength=shape.E)
    assert counts.max() > 256
    out, w, idx = gu.run_layer(gu.upload_layer(layer), shape)
    got_idx = gu.host(idx).astype(np.uint32)
    _check_indices(got_idx, inter["indices"], inter["choice"], shape.k)
    same = np.all(got_idx == inter["indices"], axis=1)
    assert same.mean() > 0.99
    assert O.rel_l2(gu.host(out)[same], want[same]) < REL_L2


@pytest.mark.parametrize("T", [2, 8])
def test_moe_layer_mxfp8_shared_expert(gu, T):
    # an MXFP8 shared expert runs as its own dense MLP before the routed kernels
    shape = MoEShape("mx8shared", T, 2048, 128, 8, 768, 768)
    layer = make_layer(shape, 4242 + T)
    mats = []
    for key in ("shared.gate", "shared.up", "shared.down"):
        codes, scales = O.quantize_mx(layer[key], 8, O.MX_RULE_NEAREST)
        layer[key] = codes
        layer[key + ".scales"] = scales
        mats.append(O.dequant_mxfp8(codes, scales))
    x = O.bf16_bits_to_f32(layer["x"])
    want, inter = O.moe_layer(x, layer["router_weight"], layer["router_bias"], _bank(layer),
                              tuple(mats), top_k=shape.k, n_group=1, topk_group=1,
                              norm_topk_prob=True, routed_scaling_factor=2.5, swiglu_limit=10.0,
                              return_intermediates=True)
    out, _, idx = gu.run_layer(gu.upload_layer(layer), shape, shared_fmt=native.GLM_FMT_MXFP8)
    assert np.array_equal(gu.host(idx).astype(np.uint32), inter["indices"])
    assert O.rel_l2(gu.host(out), want) < REL_L2


def test_moe_layer_golden_vectors(gu):
    # the committed fixture (tests/golden/moe_small.npz): d=256 runs the general
    # kernels, with group-limited routing
    import os
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                             "moe_small.npz"))
    shape = MoEShape("golden", 3, 256, 8, 2, 128, 128, n_group=2, topk_group=1)
    layer = {key: z[key] for key in z.files if not key.startswith("expected.")}
    out, w, idx = gu.run_layer(gu.upload_layer(layer), shape)
    assert np.array_equal(gu.host(idx).astype(np.uint32), z["expected.indices"])
    np.testing.assert_allclose(gu.host(w), z["expected.weights"], rtol=2e-6, atol=1e-7)
    assert O.rel_l2(gu.host(out), z["expected.out"]) < REL_L2


def test_moe_layer_prefill_sampled(gu):
    shape = SHAPES["prefill_t4096"]
    layer = make_layer(shape, 5303)
    out, w, idx = gu.run_layer(gu.upload_layer(layer), shape)
    x = O.bf16_bits_to_f32(layer["x"])
    _, w_want, idx_want, choice = O.router(x, layer["router_weight"], layer["router_bias"],
                                           top_k=shape.k, n_group=1, topk_group=1,
                                           norm_topk_prob=True, routed_scaling_factor=2.5)
    got_idx = gu.host(idx).astype(np.uint32)
    amb = _check_indices(got_idx, idx_want, choice, shape.k)
    assert amb <= 41
    # every token routed once per slot: counts sum to T*k (size-independent check)
    assert np.bincount(got_idx.reshape(-1), minlength=shape.E).sum() == shape.T * shape.k
    # 512 sampled tokens (4096 pairs) through the C restatement of the oracle:
    # every expert appears in the sample, so every expert's grouped tiles are
    # checked
    from oracle import cpu as cpu_oracle
    rng = np.random.default_rng(0)
    sample = np.sort(rng.choice(shape.T, 512, replace=False))
    assert len(np.unique(idx_want[sample])) == shape.E
    sub = dict(layer)
    sub["x"] = layer["x"][sample]
    want, _, c_idx = cpu_oracle.moe_layer(sub, shape)
    assert np.array_equal(c_idx, idx_want[sample])
    same = np.all(got_idx[sample] == idx_want[sample], axis=1)
    assert same.sum() >= len(sample) - 8
    got = gu.host(out)[sample]
    assert O.rel_l2(got[same], want[same]) < REL_L2
    # per token as well: no token far off while the total passes
    per_tok = np.sqrt(np.sum((got - want) ** 2, axis=1) / np.sum(want ** 2, axis=1))
    assert per_tok[same].max() < 4 * REL_L2


def test_moe_layer_deterministic(gu):
    shape = SHAPES["batch_t64"]
    dl = gu.upload_layer(make_layer(shape, 42))
    a, _, _ = gu.run_layer(dl, shape)
    b, _, _ = gu.run_layer(dl, shape)
    assert np.array_equal(gu.host(a).view(np.uint32), gu.host(b).view(np.uint32))


def test_moe_layer_repeated_calls_share_workspace(gu):
    # the device-side hand-off counters must return to zero after every call
    shape = SHAPES["verify_t2"]
    layer = make_layer(shape, 77)
    dl = gu.upload_layer(layer)
    lib = native.load()
    ws = gu.workspace(lib.glm_moe_workspace_bytes(shape.T, shape.d, shape.E, shape.k, shape.I,
                                                  shape.I_shared))
    rng = np.random.default_rng(1)
    for it in range(4):
        x = O.f32_to_bf16_bits(rng.standard_normal((shape.T, shape.d)).astype(np.float32))
        dl["x"] = gu.to_dev(x)
        out, _, idx = gu.run_layer(dl, shape, ws=ws)
        sub = dict(layer)
        sub["x"] = x
        want, inter = _oracle_layer(sub, shape)
        assert np.array_equal(gu.host(idx).astype(np.uint32), inter["indices"]), it
        assert O.rel_l2(gu.host(out), want) < REL_L2, it


def test_moe_layer_with_caller_computed_shared(gu):
    # shared expert computed separately (glm_dense_mlp, as a second stream
    # would) and handed in: same result as the fused layer
    torch = _torch()
    shape = SHAPES["verify_t2"]
    layer = make_layer(shape, 99)
    dl = gu.upload_layer(layer)
    T, d, Is = shape.T, shape.d, shape.I_shared
    h = torch.empty((T, Is), dtype=torch.bfloat16, device="cuda")
    shared = torch.empty((T, d), dtype=torch.bfloat16, device="cuda")
    gu.call("glm_dense_mlp", gu.stream(), gu.p(dl["x"]), T, d, Is, native.GLM_FMT_BF16,
            gu.p(dl["shared.gate"]), None, gu.p(dl["shared.up"]), None, gu.p(dl["shared.down"]),
            None, shape.swiglu_limit, gu.p(h), gu.p(shared))
    want, _ = _oracle_layer(layer, shape)
    b, _, _ = gu.run_layer(dl, shape, shared=False, shared_in=shared)
    assert O.rel_l2(gu.host(b), want) < REL_L2
