"""numpy model of the activation formats of the block-scaled grouped GEMMs.

The grouped prefill GEMMs take MXFP4 weights as stored and the bf16
activations in one of three block-scaled forms (32-element groups, E8M0
scales, round to nearest even):

* ``FP8X2``: two E4M3FN terms, hi + lo (exact for normal-range groups);
* ``FP6X2``: two E2M3 terms, hi + lo;
* ``FP4``:   one E2M1 term;
* ``FP8FP6``: hi E4M3FN + lo E2M3 (exact for elements at most two binades
  below their group maximum's, the lo MFMA at the FP6 rate).

Each term's scale is the smallest power of two that keeps the group's largest
magnitude within the element format's maximum (448, 7.5, 6); lo encodes the
exact f32 residual x - hi under its own scale.  The byte layout of a split
buffer is modelled too (``pack``), so the GPU split kernels can be checked bit
for bit.  Test infrastructure only.
"""

from __future__ import annotations

import numpy as np

from oracle import moe_oracle as O

FP8X2, FP6X2, FP4, FP8FP6 = 0, 1, 2, 3
NAMES = {FP8X2: "fp8x2", FP6X2: "fp6x2", FP4: "fp4", FP8FP6: "fp8fp6"}
TERMS = {FP8X2: 2, FP6X2: 2, FP4: 1, FP8FP6: 2}


def e2m3_magnitudes() -> np.ndarray:
    """The 32 non-negative E2M3 values in code order: exponent bits [4:3]
    (bias 1), mantissa bits [2:0]; exponent 0 is subnormal (m / 8)."""
    c = np.arange(32)
    e, m = c >> 3, c & 7
    return np.where(e == 0, m / 8.0, (1.0 + m / 8.0) * np.ldexp(1.0, e - 1))


def _nearest_even_code(values, mags: np.ndarray, sign_bit: int) -> np.ndarray:
    """Code of the magnitude nearest to |v| (saturating at the largest), ties
    to the even code; the sign bit is set for every v with its sign bit set
    (-0 included)."""
    v = np.asarray(values, dtype=np.float64)
    a = np.minimum(np.abs(v), mags[-1])
    diff = np.abs(a[..., None] - mags)
    best = np.argmin(diff, axis=-1)
    dmin = np.take_along_axis(diff, best[..., None], axis=-1)[..., 0]
    tie = np.sum(diff == dmin[..., None], axis=-1) > 1
    best = np.where(tie & (best % 2 == 1), best + 1, best)
    return (best | np.where(np.signbit(v), sign_bit, 0)).astype(np.uint8)


def e2m3_encode(values) -> np.ndarray:
    return _nearest_even_code(values, e2m3_magnitudes(), 0x20)


def e2m3_decode(codes) -> np.ndarray:
    c = np.asarray(codes).astype(np.int64)
    return np.where(c & 0x20, -1.0, 1.0) * e2m3_magnitudes()[c & 0x1F]


def e2m1_decode(codes) -> np.ndarray:
    c = np.asarray(codes).astype(np.int64)
    return np.where(c & 0x8, -1.0, 1.0) * np.asarray(O.E2M1_MAGNITUDES)[c & 0x7]


def e4m3_decode(codes) -> np.ndarray:
    return O.e4m3fn_table().astype(np.float64)[np.asarray(codes)]


# (format max as m * 2**3 with m in [0.5, 1), encoder, decoder) per element format
_ELEM = {
    "e4m3": (448.0 / 512.0, 9, O.e4m3fn_encode, e4m3_decode),
    "e2m3": (7.5 / 8.0, 3, e2m3_encode, e2m3_decode),
    "e2m1": (6.0 / 8.0, 3, O.e2m1_encode, e2m1_decode),
}
# element format of each term
_TERM_ELEM = {FP8X2: ("e4m3", "e4m3"), FP6X2: ("e2m3", "e2m3"), FP4: ("e2m1",),
              FP8FP6: ("e4m3", "e2m3")}


def scale_byte(amax, elem: str) -> np.ndarray:
    """Smallest E8M0 byte b with amax * 2**(127 - b) <= the format maximum
    (127 for an all-zero group), clamped to [0, 254]."""
    mmax, emax, _, _ = _ELEM[elem]
    m, e = np.frexp(np.asarray(amax, dtype=np.float64))
    k = np.where(m <= mmax, e - emax, e - emax + 1)
    return np.where(np.asarray(amax) > 0, np.clip(k + 127, 0, 254), 127).astype(np.int64)


def split(xb, K: int, fmt: int):
    """bf16 bit patterns [rows, K] -> list of (codes [rows, K] u8, scales
    [rows, K / 32] u8), one per term."""
    x = O.bf16_bits_to_f32(xb).astype(np.float32).reshape(-1, K // 32, 32)
    terms = []
    r = x
    for elem in _TERM_ELEM[fmt]:
        _, _, enc, dec = _ELEM[elem]
        b = scale_byte(np.abs(r).max(axis=2), elem)
        codes = enc(np.ldexp(r.astype(np.float64), (127 - b)[..., None]).astype(np.float32))
        back = dec(codes) * np.ldexp(1.0, b - 127)[..., None]
        terms.append((codes.reshape(-1, K), b.astype(np.uint8).reshape(-1, K // 32)))
        r = (r.astype(np.float64) - back).astype(np.float32)  # exact in f32
    return terms


def dequant(terms, K: int, fmt: int) -> np.ndarray:
    """Sum of the terms' values, float64 [rows, K]."""
    out = 0.0
    for elem, (codes, scales) in zip(_TERM_ELEM[fmt], terms):
        v = _ELEM[elem][3](codes).reshape(-1, K // 32, 32) * np.ldexp(
            1.0, scales.astype(np.int64) - 127)[..., None]
        out = out + v.reshape(-1, K)
    return out


def _round256(n: int) -> int:
    return (n + 255) // 256 * 256


def code_row_bytes(K: int, fmt: int) -> int:
    return K // 2 if fmt == FP4 else K


def split_bytes(rows: int, K: int, fmt: int) -> int:
    return TERMS[fmt] * (_round256(rows * code_row_bytes(K, fmt)) + _round256(rows * K // 32))


def _pack_codes(codes, K: int, elem: str) -> np.ndarray:
    """One term's codes [rows, K] -> its stored rows [rows, code_row_bytes].

    E4M3: one byte per element.  E2M1: two codes per byte, low nibble first
    (the MXFP4 weight layout).  E2M3: per 128-element chunk 128 bytes; the
    32 codes of group g are packed 6 bits each, low bits first, into 24 bytes,
    bytes 0-15 at 16 g and bytes 16-23 at 64 + 16 g (the other 8 bytes zero)."""
    rows = codes.shape[0]
    if elem == "e4m3":
        return codes.astype(np.uint8)
    if elem == "e2m1":
        c = codes.reshape(rows, K // 2, 2).astype(np.uint8)
        return (c[..., 0] | (c[..., 1] << 4)).astype(np.uint8)
    g = codes.reshape(rows, K // 32, 32).astype(np.uint64)
    bits = np.zeros((rows, K // 32, 24), dtype=np.uint8)
    for s in range(32):
        for b in range(6):
            pos = 6 * s + b
            bits[:, :, pos // 8] |= (((g[:, :, s] >> np.uint64(b)) & np.uint64(1)).astype(np.uint8)
                                     << np.uint8(pos % 8))
    out = np.zeros((rows, K // 128, 128), dtype=np.uint8)
    grp = bits.reshape(rows, K // 128, 4, 24)
    for q in range(4):
        out[:, :, 16 * q:16 * q + 16] = grp[:, :, q, :16]
        out[:, :, 64 + 16 * q:64 + 16 * q + 8] = grp[:, :, q, 16:]
    return out.reshape(rows, K)


def pack(terms, rows: int, K: int, fmt: int) -> np.ndarray:
    """The split buffer: each term's code rows, then each term's scale rows,
    every region 256-byte aligned (hi codes, lo codes, hi scales, lo scales)."""
    cb, sb = _round256(rows * code_row_bytes(K, fmt)), _round256(rows * K // 32)
    out = np.zeros(split_bytes(rows, K, fmt), dtype=np.uint8)
    nt = len(terms)
    for i, (elem, (codes, scales)) in enumerate(zip(_TERM_ELEM[fmt], terms)):
        out[i * cb:i * cb + rows * code_row_bytes(K, fmt)] = _pack_codes(codes, K, elem).ravel()
        o = nt * cb + i * sb
        out[o:o + rows * K // 32] = scales.ravel()
    return out
