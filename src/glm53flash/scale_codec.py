"""ScaleX Mode-A/B: lossless coding of one expert's E8M0 scale bytes.

The reference's format (``scale_codec.py``), byte for byte: a 24-byte header
``<4sB4B3xIII`` (magic ``LSA1``, codec, four palette bytes, raw size, primary
size, exception count), then the primary stream -- one bit per scale over the
two most frequent values, two bits over the four most frequent, or the raw
bytes -- then the exception positions (u32 little-endian, ascending) and their
values (u8).  The encoder keeps the smallest of the three forms
(``scale_codec.py:35-91``).  Mode B appends a u16 directory of the first
exception of every 512-scale tile (``scale_codec.py:117-152``).

On MI355X the decoding runs once, on the GPU, when a ScaleX shard is loaded
into the HBM bank (``glm_scalex_decode``); this module is the host side: the
encoder (used to write ScaleX shards), header inspection and validation, and a
numpy decoder.
"""

from __future__ import annotations

from dataclasses import dataclass
import struct

import numpy as np

MODE_A_MAGIC = b"LSA1"
MODE_A_HEADER = struct.Struct("<4sB4B3xIII")
A_RAW = 0
A_ONE_BIT = 1
A_TWO_BIT = 2
MODE_B_TILE_SCALES = 512
CODEC_NAMES = {A_RAW: "raw", A_ONE_BIT: "one_bit", A_TWO_BIT: "two_bit"}


class ScaleCodecError(ValueError):
    """A ScaleX record is malformed (``scale_codec.py:21-22``)."""


@dataclass(frozen=True)
class ModeAInfo:
    raw_bytes: int
    encoded_bytes: int
    codec: str
    palette: tuple[int, int, int, int]
    primary_bytes: int
    exceptions: int


def _pack_codes(codes: np.ndarray, bits: int) -> bytes:
    if bits == 1:
        return np.packbits(codes, bitorder="little").tobytes()
    pad = (-codes.size) % 4
    c = np.pad(codes, (0, pad)).reshape(-1, 4).astype(np.uint8)
    return (c[:, 0] | (c[:, 1] << 2) | (c[:, 2] << 4) | (c[:, 3] << 6)).astype(np.uint8).tobytes()


def encode_mode_a(source: bytes) -> bytes:
    """Encodes the scale bytes of one expert without changing any value."""
    values = np.frombuffer(source, dtype=np.uint8)
    counts = np.bincount(values, minlength=256)
    # most frequent first, ties to the smaller byte value
    palette = np.lexsort((np.arange(256), -counts))[:4].astype(np.uint8)
    forms = []
    for codec, bits, width in ((A_ONE_BIT, 1, 2), (A_TWO_BIT, 2, 4)):
        codes = np.zeros(values.size, dtype=np.uint8)
        represented = np.zeros(values.size, dtype=bool)
        for code, value in enumerate(palette[:width]):
            hit = values == value
            codes[hit] = code
            represented |= hit
        primary = _pack_codes(codes, bits)
        positions = np.flatnonzero(~represented).astype("<u4")
        forms.append((len(primary) + 5 * positions.size, codec, primary, positions,
                      values[~represented]))
    forms.append((len(source), A_RAW, bytes(source), np.zeros(0, "<u4"), np.zeros(0, np.uint8)))
    # the smallest form; on equal sizes the earlier one (one bit, two bits, raw)
    best = min(forms, key=lambda form: form[0])
    _, codec, primary, positions, exc_values = best
    header = MODE_A_HEADER.pack(MODE_A_MAGIC, codec, *(int(v) for v in palette), len(source),
                                len(primary), positions.size)
    return header + primary + positions.astype("<u4").tobytes() + exc_values.tobytes()


def inspect_mode_a(encoded) -> ModeAInfo:
    """Header fields of a record, checked against its length (``scale_codec.py:94-114``)."""
    if len(encoded) < MODE_A_HEADER.size:
        raise ScaleCodecError(f"record of {len(encoded)} B is truncated: a Mode-A header takes "
                              f"{MODE_A_HEADER.size}")
    magic, codec, p0, p1, p2, p3, raw, primary, exceptions = MODE_A_HEADER.unpack_from(encoded)
    if magic != MODE_A_MAGIC or codec not in CODEC_NAMES:
        raise ScaleCodecError(f"not a Mode-A record (magic {magic!r}, codec {codec})")
    if MODE_A_HEADER.size + primary + 5 * exceptions != len(encoded):
        raise ScaleCodecError(f"record is {len(encoded)} B; its header describes "
                              f"{MODE_A_HEADER.size + primary + 5 * exceptions} B")
    return ModeAInfo(raw_bytes=raw, encoded_bytes=len(encoded), codec=CODEC_NAMES[codec],
                     palette=(p0, p1, p2, p3), primary_bytes=primary, exceptions=exceptions)


def validate_mode_a(encoded) -> ModeAInfo:
    """Everything a decoder relies on: the header, the primary length of the
    codec, and exception positions ascending and inside the raw size
    (``scale_codec.py:170-201``)."""
    info = inspect_mode_a(encoded)
    if info.codec == "raw":
        if info.primary_bytes != info.raw_bytes or info.exceptions:
            raise ScaleCodecError("a raw record must carry exactly its scale bytes and no "
                                  "exceptions")
        return info
    bits = 1 if info.codec == "one_bit" else 2
    if info.primary_bytes != (info.raw_bytes * bits + 7) // 8:
        raise ScaleCodecError(f"{info.codec} stream of {info.primary_bytes} B cannot code "
                              f"{info.raw_bytes} scales")
    positions = np.frombuffer(encoded, dtype="<u4", count=info.exceptions,
                              offset=MODE_A_HEADER.size + info.primary_bytes)
    if info.exceptions and (positions[-1] >= info.raw_bytes or np.any(positions[1:] <= positions[:-1])):
        raise ScaleCodecError("exception positions must ascend and stay below the scale "
                              "count")
    return info


def decode_mode_a(encoded) -> bytes:
    """The raw scale bytes of a record (numpy)."""
    info = validate_mode_a(encoded)
    start = MODE_A_HEADER.size
    primary = np.frombuffer(encoded, dtype=np.uint8, count=info.primary_bytes, offset=start)
    if info.codec == "raw":
        return primary.tobytes()
    if info.codec == "one_bit":
        codes = np.unpackbits(primary, bitorder="little")[: info.raw_bytes]
        palette = np.array(info.palette[:2], np.uint8)
    else:
        codes = np.stack([(primary >> s) & 3 for s in (0, 2, 4, 6)], axis=1).reshape(-1)
        codes = codes[: info.raw_bytes]
        palette = np.array(info.palette, np.uint8)
    out = palette[codes]
    if info.exceptions:
        pos_at = start + info.primary_bytes
        positions = np.frombuffer(encoded, dtype="<u4", count=info.exceptions, offset=pos_at)
        vals = np.frombuffer(encoded, dtype=np.uint8, count=info.exceptions,
                             offset=pos_at + 4 * info.exceptions)
        out[positions] = vals
    return out.tobytes()


def mode_b_tile_prefix(encoded) -> bytes:
    """u16 index of the first exception at or after each 512-scale tile start
    (``scale_codec.py:117-141``)."""
    info = validate_mode_a(encoded)
    if info.exceptions > np.iinfo(np.uint16).max:
        raise ScaleCodecError(f"{info.exceptions} exceptions overflow the u16 tile directory")
    positions = np.frombuffer(encoded, dtype="<u4", count=info.exceptions,
                              offset=MODE_A_HEADER.size + info.primary_bytes)
    tiles = (info.raw_bytes + MODE_B_TILE_SCALES - 1) // MODE_B_TILE_SCALES
    bounds = np.minimum(np.arange(tiles + 1, dtype=np.uint64) * MODE_B_TILE_SCALES, info.raw_bytes)
    return np.searchsorted(positions, bounds, side="left").astype("<u2").tobytes()


def mode_b_indexed_nbytes(encoded_bytes: int, raw_bytes: int) -> int:
    """``scale_codec.py:144-148``."""
    if encoded_bytes < MODE_A_HEADER.size or raw_bytes < 1:
        raise ScaleCodecError(f"no Mode-B row for {encoded_bytes} coded / {raw_bytes} raw bytes")
    tiles = (raw_bytes + MODE_B_TILE_SCALES - 1) // MODE_B_TILE_SCALES
    return encoded_bytes + (encoded_bytes & 1) + 2 * (tiles + 1)


def encode_mode_b_row(encoded: bytes) -> bytes:
    """A Mode-A record padded to even length plus its tile directory."""
    return bytes(encoded) + b"\0" * (len(encoded) & 1) + mode_b_tile_prefix(encoded)


def mode_b_dir_bytes(raw_bytes: int) -> int:
    """Bytes of the tile directory at the front of a resident row (u16 per
    512-scale tile boundary, zero-padded to a multiple of 16)."""
    tiles = (raw_bytes + MODE_B_TILE_SCALES - 1) // MODE_B_TILE_SCALES
    return (2 * (tiles + 1) + 15) // 16 * 16


def mode_b_slot(encoded) -> bytes:
    """The resident form of a Mode-B row for ``glm_moe_forward_scalex``: the
    same directory and record as ``encode_mode_b_row``, with the directory in
    front (zero-padded to 16 bytes) so that the kernels find it and the
    record's header at fixed offsets."""
    info = validate_mode_a(encoded)
    directory = mode_b_tile_prefix(encoded)
    pad = mode_b_dir_bytes(info.raw_bytes) - len(directory)
    return directory + b"\0" * pad + bytes(encoded)


def mode_b_record(slot, raw_bytes: int) -> bytes:
    """The Mode-A record inside a resident row (``mode_b_slot``, possibly
    padded further): after the directory, its length from the header."""
    start = mode_b_dir_bytes(raw_bytes)
    head = bytes(slot[start:start + MODE_A_HEADER.size])
    if len(head) < MODE_A_HEADER.size:
        raise ScaleCodecError("a resident row shorter than its directory and a Mode-A header")
    _, _, _, _, _, _, _, primary, exceptions = MODE_A_HEADER.unpack(head)
    return bytes(slot[start:start + MODE_A_HEADER.size + primary + 5 * exceptions])


def mode_b_bank(gate_scales, down_scales, up_scales, *, align: int = 256):
    """The HBM form of a layer's coded scales for ``glm_moe_forward_scalex``:
    expert e's resident Mode-B row (``mode_b_slot`` of the Mode-A record of
    its gate | down | up scale bytes, the reference's record order) at
    ``rows[e]``, every row padded to one stride, a multiple of ``align``.
    Returns ``(rows uint8 [E, stride], stride, coded_bytes)`` where
    ``coded_bytes`` sums the experts' own row lengths."""
    g, dn, u = (np.ascontiguousarray(a, dtype=np.uint8) for a in (gate_scales, down_scales, up_scales))
    if not (g.shape[0] == dn.shape[0] == u.shape[0]):
        raise ScaleCodecError("gate, down and up scales disagree on the expert count")
    E = g.shape[0]
    rows = []
    for e in range(E):
        raw = g[e].tobytes() + dn[e].tobytes() + u[e].tobytes()
        rows.append(mode_b_slot(encode_mode_a(raw)))
    stride = max(len(r) for r in rows)
    stride = (stride + align - 1) // align * align
    out = np.zeros((E, stride), dtype=np.uint8)
    for e, r in enumerate(rows):
        out[e, :len(r)] = np.frombuffer(r, dtype=np.uint8)
    return out, stride, sum(len(r) for r in rows)

