"""CPU checks that pin the numpy model of the grouped GEMMs' activation
formats (``tests/act_formats.py``): the E2M3 value table against the OCP MX
v1.0 element definition, the encoders' rounding (round trip, ties to the even
code, saturation), the scale rule at its boundaries, the splits' error bounds
and the byte layout against independent unpacking."""

from __future__ import annotations

import numpy as np

import act_formats as A
from oracle import moe_oracle as O


def test_e2m3_table_is_the_ocp_element():
    # OCP MX v1.0, FP6 E2M3: bias 1, no inf/NaN; subnormals m/8, min normal 1,
    # max normal 7.5
    mags = A.e2m3_magnitudes()
    assert mags.shape == (32,)
    assert np.all(np.diff(mags) > 0)
    assert list(mags[:8]) == [m / 8 for m in range(8)]
    assert mags[8] == 1.0 and mags[16] == 2.0 and mags[24] == 4.0 and mags[31] == 7.5
    assert mags[15] == 1.875 and mags[23] == 3.75


def test_encoders_round_trip_ties_to_even_and_saturate():
    for enc, dec, n, sign in [(A.e2m3_encode, A.e2m3_decode, 32, 0x20),
                              (O.e2m1_encode, A.e2m1_decode, 8, 0x8)]:
        codes = np.arange(n)
        vals = dec(codes)
        assert np.array_equal(enc(vals.astype(np.float32)), codes)
        assert np.array_equal(enc((-vals).astype(np.float32)), codes | sign)
        mid = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
        got = enc(mid)
        want = np.where(codes[:-1] % 2 == 0, codes[:-1], codes[1:])
        assert np.array_equal(got, want)
        assert enc(np.float32(vals[-1] * 4)) == n - 1
        assert enc(np.float32(-0.0)) == sign


def test_scale_byte_boundaries():
    for elem, top in [("e4m3", 448.0), ("e2m3", 7.5), ("e2m1", 6.0)]:
        for j in (-20, 0, 13):
            exact = np.ldexp(top, j)
            assert A.scale_byte(exact, elem) == 127 + j
            assert A.scale_byte(np.nextafter(exact, np.inf), elem) == 128 + j
        assert A.scale_byte(0.0, elem) == 127


def _groups(rng, rows, K):
    x = rng.normal(0, 1, (rows, K // 32, 32)) * np.ldexp(1.0, rng.integers(-8, 8, (rows, K // 32, 1)))
    return O.f32_to_bf16_bits(x.reshape(rows, K).astype(np.float32))


def test_split_error_bounds():
    rng = np.random.default_rng(5)
    rows, K = 64, 512
    xb = _groups(rng, rows, K)
    x = O.bf16_bits_to_f32(xb).astype(np.float64)
    amax = np.abs(x.reshape(rows, -1, 32)).max(axis=2)
    for fmt, bound in [(A.FP8X2, 2.0 ** -22), (A.FP6X2, 2.0 ** -6), (A.FP4, 2.0 ** -2),
                       (A.FP8FP6, 1.0 / 840)]:
        err = np.abs(A.dequant(A.split(xb, K, fmt), K, fmt) - x).reshape(rows, -1, 32).max(axis=2)
        assert np.all(err <= bound * amax), (A.NAMES[fmt], float((err / amax).max()))
    # one term cannot do better than its element's half quantum at the top
    e1 = np.abs(A.dequant(A.split(xb, K, A.FP4), K, A.FP4) - x).reshape(rows, -1, 32).max(axis=2)
    assert np.mean(e1 > 2.0 ** -6 * amax) > 0.9


def test_fp8fp6_exact_near_the_group_maximum():
    # hi E4M3 keeps 4 significant bits, lo E2M3 the next 4 wherever the lo
    # scale reaches: every element at most two binades below its group
    # maximum's comes back exactly (a bf16 element has 8 bits); below that
    # lo's two-bit exponent runs out and the error stays under max / 840
    rng = np.random.default_rng(6)
    rows, K = 128, 512
    xb = _groups(rng, rows, K)
    x = O.bf16_bits_to_f32(xb).astype(np.float64).reshape(rows, -1, 32)
    d = A.dequant(A.split(xb, K, A.FP8FP6), K, A.FP8FP6).reshape(rows, -1, 32)
    amax = np.abs(x).max(axis=2, keepdims=True)
    _, emax = np.frexp(amax)
    _, e = np.frexp(np.where(x != 0, np.abs(x), amax))
    near = (emax - e <= 2) & (x != 0)
    assert near.mean() > 0.5 and np.array_equal(d[near], x[near])
    # the hi term alone is the FP8X2 split's hi term, byte for byte
    hi8, hi86 = A.split(xb, K, A.FP8X2)[0], A.split(xb, K, A.FP8FP6)[0]
    assert np.array_equal(hi8[0], hi86[0]) and np.array_equal(hi8[1], hi86[1])


def test_fp6_packing_against_bit_unpacking():
    rng = np.random.default_rng(8)
    rows, K = 3, 256
    codes = rng.integers(0, 64, (rows, K)).astype(np.uint8)
    scales = rng.integers(100, 140, (rows, K // 32)).astype(np.uint8)
    buf = A.pack([(codes, scales), (codes[::-1].copy(), scales[::-1].copy())], rows, K, A.FP6X2)
    hi = buf[:rows * K].reshape(rows, K // 128, 128)
    for row in range(rows):
        for c in range(K // 128):
            for g in range(4):
                b = np.concatenate([hi[row, c, 16 * g:16 * g + 16], hi[row, c, 64 + 16 * g:72 + 16 * g]])
                assert not hi[row, c, 72 + 16 * g:80 + 16 * g].any()
                bits = np.unpackbits(b, bitorder="little")
                for s in range(32):
                    v = int(np.packbits(bits[6 * s:6 * s + 6], bitorder="little")[0])
                    assert v == codes[row, 128 * c + 32 * g + s]
    cb = (rows * K + 255) // 256 * 256
    sb = (rows * K // 32 + 255) // 256 * 256
    assert np.array_equal(buf[2 * cb:2 * cb + rows * K // 32].reshape(rows, -1), scales)
    assert np.array_equal(buf[2 * cb + sb:2 * cb + sb + rows * K // 32].reshape(rows, -1),
                          scales[::-1])


def test_fp4_packing_is_the_mxfp4_weight_layout():
    rng = np.random.default_rng(9)
    rows, K = 5, 128
    codes = rng.integers(0, 16, (rows, K)).astype(np.uint8)
    scales = rng.integers(100, 140, (rows, K // 32)).astype(np.uint8)
    buf = A.pack([(codes, scales)], rows, K, A.FP4)
    packed = buf[:rows * K // 2].reshape(rows, K // 2)
    assert np.array_equal(O.unpack_e2m1_codes(packed), codes)
    assert A.split_bytes(rows, K, A.FP4) == 512 + 256  # codes 320 B, scales 20 B, 256-aligned
