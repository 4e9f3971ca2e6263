"""Pins the CPU oracle (oracle/moe_oracle.py) before it is trusted as the checker.

Every check here is independent of the oracle's own formula: reference
known-answer tests, closed forms derived from the format's bit layout, brute
force over all codes, or per-element exact sums.  A plausible mistake (a
swapped nibble, a dropped scale, a wrong tie rule, a transposed operand, an
off-by-one in a prefix sum) fails at least one of them.
"""

from __future__ import annotations

import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import moe_oracle as O


# --------------------------------------------------------------------------- codecs


def _e2m1_from_bits(code: int) -> float:
    """E2M1 from its bit fields (OCP MX v1.0, sec. 5.3.3): s|ee|m, bias 1."""
    sign = -1.0 if code & 0x8 else 1.0
    e = (code >> 1) & 0x3
    m = code & 0x1
    if e == 0:
        return sign * m * 0.5
    return sign * (2.0 ** (e - 1)) * (1.0 + m / 2.0)


def test_e2m1_table_matches_bit_fields():
    table = O.e2m1_table()
    for code in range(16):
        assert table[code] == _e2m1_from_bits(code), code


def test_e4m3fn_reference_known_answers():
    # tests/test_fp8.py:8-12 of the reference
    raw = np.array([0x00, 0x01, 0x38, 0x3C, 0x7E, 0xB8], dtype=np.uint8)
    expected = np.array([0.0, 2**-9, 1.0, 1.5, 448.0, -1.0], np.float32)
    np.testing.assert_array_equal(O.e4m3fn_table()[raw], expected)
    # tests/test_fp8.py:32-36: 0x7F is the non-finite code
    assert math.isnan(O.e4m3fn_table()[0x7F]) and math.isnan(O.e4m3fn_table()[0xFF])
    finite = O.e4m3fn_table()[np.arange(256) % 128 != 0x7F]
    assert np.all(np.isfinite(finite))


def test_e8m0_closed_form_all_bytes():
    s = O.e8m0_to_f32(np.arange(256))
    for e in range(255):
        assert float(s[e]) == math.ldexp(1.0, e - 127), e
    assert math.isnan(s[255])


def test_mxfp4_nibble_order_known_answer():
    # byte 0x21: element 0 <- low nibble (code 1 = 0.5), element 1 <- high nibble (code 2 = 1.0)
    packed = np.zeros((1, 16), dtype=np.uint8)
    packed[0, 0] = 0x21
    packed[0, 1] = 0xF9  # element 2 <- 9 (-0.5), element 3 <- 15 (-6)
    scales = np.array([[127]], dtype=np.uint8)
    out = O.dequant_mxfp4(packed, scales)
    np.testing.assert_array_equal(out[0, :4], [0.5, 1.0, -0.5, -6.0])
    assert np.all(out[0, 4:] == 0)


def test_mxfp4_group_scale_broadcast_is_per_32_elements():
    packed = np.full((2, 32), 0x22, dtype=np.uint8)  # every element = 1.0 before scaling
    scales = np.array([[127, 130], [120, 0]], dtype=np.uint8)
    out = O.dequant_mxfp4(packed, scales)
    assert np.all(out[0, :32] == 1.0) and np.all(out[0, 32:] == 8.0)
    assert np.all(out[1, :32] == 2.0**-7) and np.all(out[1, 32:] == 2.0**-127)


def test_mxfp8_group_scale_and_codes():
    codes = np.tile(np.array([0x38, 0xB8, 0x7E, 0x01], dtype=np.uint8), (1, 16))  # 64 elems
    scales = np.array([[127, 125]], dtype=np.uint8)
    out = O.dequant_mxfp8(codes, scales)
    np.testing.assert_array_equal(out[0, :4], [1.0, -1.0, 448.0, 2**-9])
    np.testing.assert_array_equal(out[0, 32:36], [0.25, -0.25, 112.0, 2**-11])


def test_bf16_round_is_nearest_even():
    cases = {
        0x3F800000: 0x3F80,  # 1.0
        0x3F808000: 0x3F80,  # halfway, even stays
        0x3F818000: 0x3F82,  # halfway, odd rounds up
        0x3F808001: 0x3F81,  # just above halfway
        0x7F7FFFFF: 0x7F80,  # overflow to inf
        0x7FC00001: 0x7FC0,  # NaN stays NaN
    }
    for f32_bits, bf16_bits in cases.items():
        x = np.array([f32_bits], dtype=np.uint32).view(np.float32)
        assert int(O.f32_to_bf16_bits(x)[0]) == bf16_bits, hex(f32_bits)


# --------------------------------------------------------------------------- quantiser


def _brute_nearest_even(value: float, table: np.ndarray, max_code: int) -> int:
    """Nearest finite code (by exact rational distance), ties to even mantissa LSB."""
    v = Fraction(value)
    best = None
    for code in range(max_code + 1):
        t = table[code]
        if not np.isfinite(t):
            continue
        dist = abs(v - Fraction(float(t)))
        key = (dist, code & 1)
        if best is None or key < best[0]:
            best = (key, code)
    return best[1]


def test_e4m3fn_encode_matches_brute_force():
    rng = np.random.default_rng(1)
    table = O.e4m3fn_table()
    pos = table[:0x7F]
    mids = ((pos[1:].astype(np.float64) + pos[:-1]) / 2).astype(np.float32)  # ties
    samples = np.concatenate([
        rng.uniform(0, 460, 400).astype(np.float32),
        np.exp2(rng.uniform(-12, 9, 400)).astype(np.float32),
        mids, pos, np.array([0.0, 500.0, 1e-12], np.float32),
    ])
    got = O.e4m3fn_encode(samples)
    for v, c in zip(samples, got):
        want = _brute_nearest_even(min(float(v), 448.0), table, 0x7E)
        assert int(c) == want, (float(v), int(c), want)
    neg = O.e4m3fn_encode(-samples[:50])
    assert np.all((neg[samples[:50] > 0] & 0x80) == 0x80)


def test_e2m1_encode_matches_brute_force():
    table = O.e2m1_table()
    mags = np.array(O.E2M1_MAGNITUDES, np.float32)
    samples = np.concatenate([np.linspace(0, 7, 141).astype(np.float32),
                              ((mags[1:] + mags[:-1]) / 2).astype(np.float32)])
    got = O.e2m1_encode(samples)
    for v, c in zip(samples, got):
        want = _brute_nearest_even(min(float(v), 6.0), table, 7)
        assert int(c) == want, (float(v), int(c), want)


def test_scale_exponent_nearest_rule_matches_log2():
    rng = np.random.default_rng(2)
    amax = np.exp2(rng.uniform(-20, 10, 2000)).astype(np.float32)
    for a in amax:
        s = float(np.float32(a / np.float32(448.0)))
        want = math.floor(math.log2(s) + 0.5)  # log2(s) is never an exact .5 for f32 s
        assert O.mx_scale_exponent(float(a), 448.0, 8, O.MX_RULE_NEAREST) == want
    # the sqrt(2) mantissa boundary on both sides
    below = np.array([O._SQRT2_F32_BITS], np.uint32).view(np.float32)[0]
    above = np.array([O._SQRT2_F32_BITS + 1], np.uint32).view(np.float32)[0]
    assert O.mx_scale_exponent(float(below * 448.0 * 2**-10), 448.0, 8, O.MX_RULE_NEAREST) == -10
    assert O.mx_scale_exponent(float(above * np.float32(448.0) * 2**-10), 448.0, 8,
                               O.MX_RULE_NEAREST) == -9
    assert O.mx_scale_exponent(0.0, 448.0, 8, O.MX_RULE_NEAREST) == -127


def test_scale_exponent_ocp_rule():
    # OCP MX v1.0 sec. 6.3: X = floor(log2(amax)) - emax_elem
    for a, want in [(1.0, -8), (448.0, 0), (511.0, 0), (512.0, 1), (0.75, -9), (2**-30, -38)]:
        assert O.mx_scale_exponent(a, 448.0, 8, O.MX_RULE_OCP) == want
    assert O.mx_scale_exponent(6.0, 6.0, 2, O.MX_RULE_OCP) == 0


def _bf16_matrix(rng, shape, std):
    return O.f32_to_bf16_bits(rng.normal(0, std, shape).astype(np.float32))


@pytest.mark.parametrize("rule", [O.MX_RULE_NEAREST, O.MX_RULE_OCP])
def test_quantize_mx_reference_storage_and_tolerances(rule):
    # reference tests/test_resident_mxfp8.py:7-52 (shapes, seeds, byte counts, tolerances)
    for bits, seed, rtol, atol, dst in [(8, 5308, 0.03, 0.015, 64 * 32 + 64),
                                         (4, 5304, 0.20, 0.04, 64 * 16 + 64)]:
        rng = np.random.default_rng(seed)
        w = _bf16_matrix(rng, (64, 32), 0.05)
        x = O.bf16_round(rng.normal(0, 0.2, (2, 32)).astype(np.float32))
        codes, scales = O.quantize_mx(w, bits, rule)
        assert codes.nbytes + scales.nbytes == dst
        assert 64 * 32 * 2 > dst
        deq = O.dequant_mxfp8(codes, scales) if bits == 8 else O.dequant_mxfp4(codes, scales)
        expected = O.linear_bf16(x, O.bf16_bits_to_f32(w))
        actual = O.linear_bf16(x, deq)
        np.testing.assert_allclose(actual, expected, rtol=rtol, atol=atol)


def test_mxfp4_roundtrip_cosine_pins_nibble_order():
    # The reference's preflight measures cosine 0.993 between MXFP4 and BF16
    # projections (reports/preflight.json:22-155).  Our quantise->dequantise
    # round trip reaches that scale only when the nibble order is consistent.
    rng = np.random.default_rng(3)
    w = _bf16_matrix(rng, (256, 512), 0.02)
    codes, scales = O.quantize_mx(w, 4, O.MX_RULE_NEAREST)
    ref = O.bf16_bits_to_f32(w)
    deq = O.dequant_mxfp4(codes, scales)
    cos = float(np.sum(deq * ref) / (np.linalg.norm(deq) * np.linalg.norm(ref)))
    assert cos > 0.95
    swapped = ((codes >> 4) | (codes << 4)).astype(np.uint8)
    deq_bad = O.dequant_mxfp4(swapped, scales)
    cos_bad = float(np.sum(deq_bad * ref) / (np.linalg.norm(deq_bad) * np.linalg.norm(ref)))
    assert cos_bad < 0.5


def test_quantize_mx8_exact_on_representable_input():
    # values already on the E4M3 grid times a power of two survive bit-exactly
    rng = np.random.default_rng(4)
    codes = rng.integers(0, 0x7E, (8, 64)).astype(np.uint8)
    codes[:, ::32] = 0x7E  # every group holds 448 so the nearest rule picks e = 0 + shift
    vals = O.e4m3fn_table()[codes] * np.float32(2.0**-12)
    w = O.f32_to_bf16_bits(vals)
    assert np.array_equal(O.bf16_bits_to_f32(w), vals)
    q, s = O.quantize_mx(w, 8, O.MX_RULE_NEAREST)
    assert np.all(s == 127 - 12)
    np.testing.assert_array_equal(q, codes)


# --------------------------------------------------------------------------- elementwise


def test_sigmoid_against_f64():
    x = np.linspace(-30, 30, 4001).astype(np.float32)
    got = O.sigmoid_f32(x).astype(np.float64)
    want = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 4 * ulp + 1e-45)  # exp, add and divide in f32


def test_limited_swiglu_known_values():
    g = np.array([20.0, -3.0, 0.0, 1.0], np.float32)
    u = np.array([-20.0, 2.0, 5.0, 0.5], np.float32)
    h = O.limited_swiglu_bf16(g, u, 10.0)
    # 20 -> 10, silu(10) rounds to 10 in bf16, times clip(-20) = -10 -> -100
    assert h[0] == -100.0
    assert h[2] == 0.0
    s1 = O.bf16_round(np.float32(1.0 / (1.0 + math.exp(-1.0))))
    assert h[3] == O.bf16_round(O.bf16_round(s1) * np.float32(0.5))
    # no clamp when limit <= 0: gate stays 20
    h2 = O.limited_swiglu_bf16(np.array([20.0], np.float32), np.array([1.0], np.float32), 0.0)
    assert h2[0] == 20.0


def test_limited_swiglu_nan_and_infinities():
    # expert_ssd.py:103-107 clamps with mx.minimum / mx.clip, whose float forms
    # return a NaN operand (MLX's Minimum / Maximum), and nn.silu is x * sigmoid(x):
    # NaN in either input gives NaN, +inf is clamped to the limit, a gate of
    # -inf gives -inf * 0 = NaN
    L = 10.0
    g = np.array([np.nan, 1.0, np.inf, -np.inf, 1.0, 2.0], np.float32)
    u = np.array([1.0, np.nan, 1.0, 1.0, np.inf, -np.inf], np.float32)
    h = O.limited_swiglu_bf16(g, u, L)
    assert np.isnan(h[:2]).all() and np.isnan(h[3])
    assert h[2] == O.limited_swiglu_bf16(np.float32([L]), np.float32([1.0]), L)[0] == 10.0
    s1 = O.bf16_round(O.sigmoid_f32(np.float32(1.0)))
    assert h[4] == O.bf16_round(O.bf16_round(np.float32(1.0) * s1) * np.float32(L))
    s2 = O.bf16_round(O.sigmoid_f32(np.float32(2.0)))
    assert h[5] == O.bf16_round(O.bf16_round(np.float32(2.0) * s2) * np.float32(-L))
    # no limit: nothing is clamped
    h0 = O.limited_swiglu_bf16(np.float32([np.inf, np.nan]), np.float32([1.0, 1.0]), 0.0)
    assert h0[0] == np.inf and np.isnan(h0[1])


# --------------------------------------------------------------------------- router


def test_router_reference_known_answer():
    # reference tests/test_moe.py:10-23
    _, w, idx, _ = O.router(np.zeros((1, 32), np.float32), np.zeros((4, 32), np.float32),
                            np.array([10.0, 9.0, 1.0, 0.0], np.float32), top_k=2, n_group=2,
                            topk_group=1, norm_topk_prob=True, routed_scaling_factor=2.5)
    assert set(idx.reshape(-1).tolist()) == {0, 1}
    np.testing.assert_allclose(w, [[1.25, 1.25]], atol=1e-6)
    assert idx.tolist() == [[1, 0]]  # ascending: best expert last


def _brute_router(x, W, bias, k, n_group, topk_group, norm, scale):
    T = x.shape[0]
    E = W.shape[0]
    out_idx, out_w = [], []
    for t in range(T):
        logits = [float(np.float32(math.fsum(float(a) * float(b) for a, b in zip(x[t], W[e]))))
                  for e in range(E)]
        scores = [float(O.sigmoid_f32(np.float32(l))) for l in logits]
        choice = [float(np.float32(s + float(b))) for s, b in zip(scores, bias)]
        per = E // n_group
        gs = []
        for g in range(n_group):
            top = sorted(choice[g * per:(g + 1) * per])[-2:]
            gs.append((float(np.float32(top[0] + top[1])), g))
        keep = {g for _, g in sorted(gs)[-topk_group:]}
        masked = [(choice[e] if e // per in keep else -math.inf, e) for e in range(E)]
        chosen = [e for _, e in sorted(masked)[-k:]]
        w = [scores[e] for e in chosen]
        if norm:
            tot = np.float32(0)
            for v in w:
                tot = np.float32(tot + np.float32(v))
            w = [float(np.float32(np.float32(v) / np.float32(tot + np.float32(1e-20)))) for v in w]
        out_idx.append(chosen)
        out_w.append([float(np.float32(np.float32(v) * np.float32(scale))) for v in w])
    return np.array(out_idx), np.array(out_w, np.float32)


@pytest.mark.parametrize("n_group,topk_group", [(1, 1), (2, 1), (4, 2)])
def test_router_matches_brute_force(n_group, topk_group):
    rng = np.random.default_rng(10 + n_group)
    T, d, E, k = 6, 48, 16, 3
    x = O.bf16_round(rng.normal(0, 1, (T, d)).astype(np.float32))
    W = rng.normal(0, 0.1, (E, d)).astype(np.float32)
    bias = rng.normal(0, 0.05, E).astype(np.float32)
    _, w, idx, _ = O.router(x, W, bias, top_k=k, n_group=n_group, topk_group=topk_group,
                            norm_topk_prob=True, routed_scaling_factor=2.5)
    bidx, bw = _brute_router(x, W, bias, k, n_group, topk_group, True, 2.5)
    np.testing.assert_array_equal(idx, bidx)
    np.testing.assert_allclose(w, bw, rtol=1e-6)


def test_router_ties_rank_larger_index_last():
    # equal choice scores: stable ascending sort keeps index order, so the
    # larger index ends in the "best" (last) column
    _, _, idx, _ = O.router(np.zeros((1, 8), np.float32), np.zeros((4, 8), np.float32),
                            np.zeros(4, np.float32), top_k=2, n_group=1, topk_group=1,
                            norm_topk_prob=False, routed_scaling_factor=1.0)
    assert idx.tolist() == [[2, 3]]


def test_router_nan_choice_ranks_as_minus_inf():
    # A NaN logit (NaN choice) is never chosen ahead of a finite choice, in the
    # group scores or in the top-k; forced in only when fewer finite experts
    # than k remain, by index like any other -inf.  The kernels do the same.
    rng = np.random.default_rng(17)
    T, d, E, k = 3, 32, 8, 3
    x = O.bf16_round(rng.normal(0, 1, (T, d)).astype(np.float32))
    W = rng.normal(0, 0.1, (E, d)).astype(np.float32)
    W[5, 3] = np.nan  # expert 5's logit is NaN for every token
    bias = np.zeros(E, np.float32)
    bias[5] = 10.0  # would be the best by far if NaN ranked high
    _, w, idx, choice = O.router(x, W, bias, top_k=k, n_group=1, topk_group=1,
                                 norm_topk_prob=True, routed_scaling_factor=1.0)
    assert not (idx == 5).any()
    assert np.all(choice[:, 5] == -np.inf)
    finite = np.delete(np.arange(E), 5)
    c = O.router(x, np.delete(W, 5, axis=0), np.delete(bias, 5), top_k=k, n_group=1,
                 topk_group=1, norm_topk_prob=True, routed_scaling_factor=1.0)
    np.testing.assert_array_equal(idx, finite[c[2].astype(np.int64)])
    # groups: the NaN expert's group scores only its finite members
    _, _, gidx, _ = O.router(x, W, bias, top_k=2, n_group=4, topk_group=1,
                             norm_topk_prob=True, routed_scaling_factor=1.0)
    assert not (gidx == 5).any()
    # all but two experts masked out of k = 3: the NaN one is forced in by index
    W2 = np.full((4, d), np.nan, np.float32)
    W2[1] = W[1]
    W2[3] = W[3]
    _, _, idx2, _ = O.router(x, W2, np.zeros(4, np.float32), top_k=3, n_group=1, topk_group=1,
                             norm_topk_prob=False, routed_scaling_factor=1.0)
    assert idx2[:, 0].tolist() == [2] * T  # the largest-index -inf expert ranks highest


# --------------------------------------------------------------------------- dispatch


def test_dispatch_matches_brute_force_and_invariants():
    rng = np.random.default_rng(5)
    T, k, E = 37, 4, 11
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.uint32)
    counts, offsets, perm, inv, active = O.dispatch(idx, E)
    pairs = sorted(range(T * k), key=lambda p: (int(idx.reshape(-1)[p]), p))
    assert perm.tolist() == pairs
    assert counts.sum() == T * k and offsets[-1] == T * k and offsets[0] == 0
    assert np.array_equal(inv[perm], np.arange(T * k))
    for e in range(E):
        seg = perm[offsets[e]:offsets[e + 1]]
        assert np.all(np.diff(seg) > 0)
        assert np.all(idx.reshape(-1)[seg] == e)
    assert active.tolist() == [e for e in range(E) if counts[e]]


def test_dispatch_rejects_out_of_range():
    with pytest.raises(ValueError):
        O.dispatch(np.array([[0, 5]], np.uint32), 4)


# --------------------------------------------------------------------------- experts


def _tiny_bank(rng, E, d, I):
    def scales(shape):
        return rng.integers(119, 128, shape).astype(np.uint8)
    return O.Bank(
        rng.integers(0, 256, (E, I, d // 2)).astype(np.uint8), scales((E, I, d // 32)),
        rng.integers(0, 256, (E, I, d // 2)).astype(np.uint8), scales((E, I, d // 32)),
        rng.integers(0, 256, (E, d, I // 2)).astype(np.uint8), scales((E, d, I // 32)))


def test_routed_experts_route_order_and_exact_sums():
    rng = np.random.default_rng(8)
    E, d, I = 3, 64, 32
    bank = _tiny_bank(rng, E, d, I)
    x = O.bf16_round(rng.normal(0, 1, (2, d)).astype(np.float32))
    idx = np.array([[2, 0], [1, 2]], np.uint32)
    y, inter = O.routed_experts(x, idx, bank, 10.0, return_intermediates=True)
    assert y.shape == (2, 2, d)
    for t in range(2):
        for j in range(2):
            e = int(idx[t, j])
            Wg = O.dequant_mxfp4(bank.gate_w[e], bank.gate_s[e])
            Wu = O.dequant_mxfp4(bank.up_w[e], bank.up_s[e])
            Wd = O.dequant_mxfp4(bank.down_w[e], bank.down_s[e])
            g = np.array([math.fsum(float(a) * float(b) for a, b in zip(x[t], Wg[i]))
                          for i in range(I)], np.float32)
            u = np.array([math.fsum(float(a) * float(b) for a, b in zip(x[t], Wu[i]))
                          for i in range(I)], np.float32)
            np.testing.assert_array_equal(inter["gate"][t, j], O.bf16_round(g))
            np.testing.assert_array_equal(inter["up"][t, j], O.bf16_round(u))
            h = O.limited_swiglu_bf16(O.bf16_round(g), O.bf16_round(u), 10.0)
            yy = np.array([math.fsum(float(a) * float(b) for a, b in zip(h, Wd[r]))
                           for r in range(d)], np.float32)
            np.testing.assert_array_equal(y[t, j], O.bf16_round(yy))


def test_dense_mlp_is_transpose_correct():
    rng = np.random.default_rng(9)
    d, I = 32, 64
    Wg = O.bf16_round(rng.normal(0, 0.1, (I, d)).astype(np.float32))
    Wu = O.bf16_round(rng.normal(0, 0.1, (I, d)).astype(np.float32))
    Wd = O.bf16_round(rng.normal(0, 0.1, (d, I)).astype(np.float32))
    x = O.bf16_round(rng.normal(0, 1, (3, d)).astype(np.float32))
    out = O.dense_mlp(x, Wg, Wu, Wd, 10.0)
    assert out.shape == (3, d)
    t = 1
    g = O.bf16_round(np.float32(math.fsum(float(a) * float(b) for a, b in zip(x[t], Wg[5]))))
    assert g == O.linear_bf16(x, Wg)[t, 5]


def test_combine_closed_form():
    y = O.bf16_round(np.array([[[1.0, 2.0], [3.0, -4.0]]], np.float32))
    w = np.array([[0.5, 0.25]], np.float32)
    shared = np.array([[0.125, 1.0]], np.float32)
    out = O.combine(y, w, shared)
    np.testing.assert_array_equal(out, [[0.5 + 0.75 + 0.125, 1.0 - 1.0 + 1.0]])


def test_moe_layer_runs_end_to_end_small():
    rng = np.random.default_rng(11)
    T, d, E, k, I = 4, 64, 8, 2, 32
    bank = _tiny_bank(rng, E, d, I)
    x = O.bf16_round(rng.normal(0, 1, (T, d)).astype(np.float32))
    W = rng.normal(0, 0.02, (E, d)).astype(np.float32)
    shared = tuple(O.bf16_round(rng.normal(0, 0.02, s).astype(np.float32))
                   for s in [(I, d), (I, d), (d, I)])
    out, inter = O.moe_layer(x, W, np.zeros(E, np.float32), bank, shared, top_k=k, n_group=1,
                             topk_group=1, norm_topk_prob=True, routed_scaling_factor=2.5,
                             swiglu_limit=10.0, return_intermediates=True)
    assert out.shape == (T, d) and out.dtype == np.float32
    manual = O.combine(inter["route_outputs"], inter["weights"], inter["shared"])
    np.testing.assert_array_equal(out, manual)
    np.testing.assert_allclose(inter["weights"].sum(axis=1), 2.5, rtol=1e-6)


# --------------------------------------------------------------------------- golden vectors


def _golden():
    import importlib.util
    import os
    here = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    spec = importlib.util.spec_from_file_location("make_fixtures",
                                                  os.path.join(here, "make_fixtures.py"))
    mf = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mf)
    return mf, np.load(os.path.join(here, "moe_small.npz"))


def test_oracle_reproduces_committed_golden_layer():
    # the committed vectors pin the oracle against drift: inputs are regenerated
    # from the seed and every expected array must match bit for bit
    mf, z = _golden()
    layer = mf.small_layer()
    for key, value in layer.items():
        assert np.array_equal(value, z[key]), key
    for key, value in mf.expected(layer).items():
        assert value.dtype == z[key].dtype and np.array_equal(value.view(np.uint8),
                                                              z[key].view(np.uint8)), key


# --------------------------------------------------------------------------- C restatement


@pytest.fixture(scope="module")
def cpu_twin():
    import os
    from oracle import build, cpu
    if not os.path.exists(cpu.LIB):
        build.build()
    cpu.load()
    return cpu


@pytest.mark.parametrize("n_group,topk_group,shared", [(1, 1, True), (4, 2, True), (2, 1, False)])
def test_c_restatement_matches_numpy_layer(cpu_twin, n_group, topk_group, shared):
    # the C twin (bench.py's CPU baseline) against the numpy oracle on one layer
    from livglm_amd.workloads import MoEShape
    rng = np.random.default_rng(90 + n_group)
    shape = MoEShape("tiny", T=6, d=128, E=16, k=4, I=64, I_shared=64 if shared else 0,
                     n_group=n_group, topk_group=topk_group)
    bank = _tiny_bank(rng, shape.E, shape.d, shape.I)
    x = O.f32_to_bf16_bits(rng.normal(0, 1, (shape.T, shape.d)).astype(np.float32))
    W = rng.normal(0, 0.02, (shape.E, shape.d)).astype(np.float32)
    b = rng.normal(0, 0.1, shape.E).astype(np.float32)
    sw = [O.f32_to_bf16_bits(rng.normal(0, 0.02, s).astype(np.float32))
          for s in [(64, shape.d), (64, shape.d), (shape.d, 64)]]
    layer = {"x": x, "router_weight": W, "router_bias": b,
             "shared.gate": sw[0], "shared.up": sw[1], "shared.down": sw[2]}
    layer.update(zip(("gate_proj.weight_packed", "gate_proj.weight_scale", "up_proj.weight_packed",
                      "up_proj.weight_scale", "down_proj.weight_packed", "down_proj.weight_scale"),
                     (bank.gate_w, bank.gate_s, bank.up_w, bank.up_s, bank.down_w,
                      bank.down_s)))
    out, w, idx = cpu_twin.moe_layer(layer, shape, shared=shared)
    want, inter = O.moe_layer(O.bf16_bits_to_f32(x), W, b, bank,
                              tuple(O.bf16_bits_to_f32(s) for s in sw) if shared else None,
                              top_k=shape.k, n_group=n_group, topk_group=topk_group,
                              norm_topk_prob=True, routed_scaling_factor=2.5, swiglu_limit=10.0,
                              return_intermediates=True)
    assert np.array_equal(idx, inter["indices"])
    np.testing.assert_allclose(w, inter["weights"], rtol=1e-6)
    assert O.rel_l2(out, want) < 1e-5  # f32 lane sums vs exact products: last-bit differences


def test_c_restatement_router_nan_choice(cpu_twin):
    # a NaN router row: the C twin ranks the NaN choice as -inf, as the numpy
    # oracle and the kernels do
    from livglm_amd.workloads import MoEShape
    rng = np.random.default_rng(33)
    shape = MoEShape("tiny", T=4, d=128, E=16, k=4, I=64, I_shared=0, n_group=4, topk_group=2)
    bank = _tiny_bank(rng, shape.E, shape.d, shape.I)
    x = O.f32_to_bf16_bits(rng.normal(0, 1, (shape.T, shape.d)).astype(np.float32))
    W = rng.normal(0, 0.02, (shape.E, shape.d)).astype(np.float32)
    W[6, 0] = np.nan
    b = np.zeros(shape.E, np.float32)
    b[6] = 5.0
    layer = {"x": x, "router_weight": W, "router_bias": b}
    layer.update(zip(("gate_proj.weight_packed", "gate_proj.weight_scale", "up_proj.weight_packed",
                      "up_proj.weight_scale", "down_proj.weight_packed", "down_proj.weight_scale"),
                     (bank.gate_w, bank.gate_s, bank.up_w, bank.up_s, bank.down_w,
                      bank.down_s)))
    _, _, idx = cpu_twin.moe_layer(layer, shape, shared=False)
    _, _, want, _ = O.router(O.bf16_bits_to_f32(x), W, b, top_k=shape.k, n_group=4, topk_group=2,
                             norm_topk_prob=True, routed_scaling_factor=2.5)
    assert not (want == 6).any()
    np.testing.assert_array_equal(idx, want)


def test_c_restatement_nan_gate_scale(cpu_twin):
    # one routed expert's gate row with a NaN scale byte (E8M0 255): its gate
    # value is NaN while its up value is finite; the NaN passes the SwiGLU
    # clamp (as through mx.minimum) and every output of the tokens routed to
    # that expert is NaN, in the C twin as in the numpy oracle
    from livglm_amd.workloads import MoEShape
    rng = np.random.default_rng(35)
    shape = MoEShape("tiny", T=6, d=128, E=16, k=4, I=64, I_shared=0)
    bank = _tiny_bank(rng, shape.E, shape.d, shape.I)
    x = O.f32_to_bf16_bits(rng.normal(0, 1, (shape.T, shape.d)).astype(np.float32))
    W = rng.normal(0, 0.02, (shape.E, shape.d)).astype(np.float32)
    b = np.zeros(shape.E, np.float32)
    _, _, idx0, _ = O.router(O.bf16_bits_to_f32(x), W, b, top_k=shape.k, n_group=1,
                             topk_group=1, norm_topk_prob=True, routed_scaling_factor=2.5)
    e = int(idx0[0, 0])
    bank.gate_s[e, 3, 0] = 255
    layer = {"x": x, "router_weight": W, "router_bias": b}
    layer.update(zip(("gate_proj.weight_packed", "gate_proj.weight_scale", "up_proj.weight_packed",
                      "up_proj.weight_scale", "down_proj.weight_packed", "down_proj.weight_scale"),
                     (bank.gate_w, bank.gate_s, bank.up_w, bank.up_s, bank.down_w,
                      bank.down_s)))
    out, _, idx = cpu_twin.moe_layer(layer, shape, shared=False)
    want = O.moe_layer(O.bf16_bits_to_f32(x), W, b, bank, None, top_k=shape.k, n_group=1,
                       topk_group=1, norm_topk_prob=True, routed_scaling_factor=2.5,
                       swiglu_limit=10.0)
    hit = (idx0 == e).any(axis=1)
    assert hit.any() and not hit.all()
    assert np.array_equal(np.isnan(want), np.repeat(hit[:, None], shape.d, axis=1))
    assert np.array_equal(np.isnan(out), np.isnan(want))
    assert O.rel_l2(out[~hit], want[~hit]) < 1e-5


def test_c_restatement_mxfp8_linear(cpu_twin):
    rng = np.random.default_rng(5308)
    w = O.f32_to_bf16_bits(rng.normal(0, 0.05, (96, 256)).astype(np.float32))
    x = O.f32_to_bf16_bits(rng.normal(0, 1, (3, 256)).astype(np.float32))
    codes, scales = O.quantize_mx(w, 8, O.MX_RULE_NEAREST)
    got = O.bf16_bits_to_f32(cpu_twin.linear_mxfp8(x, codes, scales))
    want = O.linear_bf16(O.bf16_bits_to_f32(x), O.dequant_mxfp8(codes, scales))
    assert O.rel_l2(got, want) < 1e-5
    assert np.mean(got == want) > 0.95
    with pytest.raises(ValueError):
        cpu_twin.linear_mxfp8(x[:, :128], codes, scales)


def test_three_way_bf16_split_of_f32_is_exact():
    # the many-token router GEMM multiplies x by w0, w1 and w2 with
    # w0 = bf16(w), w1 = bf16(w - w0), w2 = bf16(w - w0 - w1) (round to nearest
    # even) and adds the products in f32; that equals x . w up to f32
    # summation order when w0 + w1 + w2 == w.  Exact for 2^-100 <= |w| <
    # 2^127 (the remainders stay normal bf16 numbers); below, the error is
    # under 2^-133, far under any f32 logit's resolution.
    rng = np.random.default_rng(91)
    w = np.concatenate([rng.normal(0, 0.02, 200000), rng.normal(0, 1, 50000),
                        rng.uniform(-1e30, 1e30, 1000),
                        np.ldexp(rng.uniform(1, 2, 2000), rng.integers(-100, 127, 2000)),
                        [0.0, -0.0, 1.0, -1.0]]).astype(np.float32)
    tiny = np.ldexp(rng.uniform(-1, 1, 2000), rng.integers(-149, -100, 2000)).astype(np.float32)

    def split(v):
        w0 = O.bf16_round(v)
        r1 = (v - w0).astype(np.float32)
        w1 = O.bf16_round(r1)
        w2 = O.bf16_round((r1 - w1).astype(np.float32))
        return w0.astype(np.float64) + w1.astype(np.float64) + w2.astype(np.float64)

    assert np.array_equal(split(w), w.astype(np.float64))
    assert np.max(np.abs(split(tiny) - tiny.astype(np.float64))) < 2.0 ** -133
