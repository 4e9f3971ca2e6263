"""ScaleX layer containers: one layer's expert shard with every expert's scale
tensors coded by ScaleX Mode A.

The reference's format (``scalex_container.py:24-352``): a prefix ``<8sIIQ``
(magic ``LVGLMSX1``, version 1, metadata length, stored length), JSON metadata
(format ``livglm_scalex_layer_v1``, layer, experts, original file length and
SHA-256, original safetensors prefix length and SHA-256, one record entry per
expert), then the stored data: the original safetensors prefix (the virtual
header every tensor name resolves against), followed per expert by
``encoded gate+down+up scales | gate weight | down weight | up weight``.

Here: the reader with the reference's checks, ``read_scalex_tensor``, a writer
(``compress_scalex_layer``) and ``verify_scalex_layer`` (the original file
rebuilt and hashed).  The reference's in-place conversion and its free-space
and fsync transaction handling (``scalex_container.py:471-711``) belong to its
checkpoint tooling and are not mirrored.
"""

from __future__ import annotations

from dataclasses import dataclass
import hashlib
import json
import os
from pathlib import Path
import re
import struct
from typing import Any, Iterator

from .scale_codec import (decode_mode_a, encode_mode_a, inspect_mode_a, mode_b_indexed_nbytes,
                          mode_b_tile_prefix)

SCALEX_FORMAT = "livglm_scalex_layer_v1"
SCALEX_MAGIC = b"LVGLMSX1"
SCALEX_VERSION = 1
SCALEX_PREFIX = struct.Struct("<8sIIQ")
SCALE_COMPONENTS = ("gate_proj", "down_proj", "up_proj")  # record order of scales and weights
_EXPERT_RE = re.compile(
    r"^model\.language_model\.layers\.(\d+)\.mlp\.experts\.(\d+)\."
    r"(down_proj|gate_proj|up_proj)\.(weight_packed|weight_scale)$")


class ScaleXContainerError(RuntimeError):
    """A ScaleX shard is malformed (``scalex_container.py:39-40``)."""


def _name(layer: int, expert: int, component: str, part: str) -> str:
    return f"model.language_model.layers.{layer}.mlp.experts.{expert}.{component}.{part}"


@dataclass(frozen=True)
class ScaleXRecord:
    """One expert's stored record (``scalex_container.py:43-61``)."""

    expert: int
    absolute_offset: int
    encoded_bytes: int
    decoded_bytes: int
    scale_names: tuple[str, str, str]
    scale_nbytes: tuple[int, int, int]
    weight_names: tuple[str, str, str]
    weight_nbytes: tuple[int, int, int]
    codec: str

    @property
    def physical_bytes(self) -> int:
        return self.encoded_bytes + sum(self.weight_nbytes)

    @property
    def mode_b_row_bytes(self) -> int:
        return mode_b_indexed_nbytes(self.encoded_bytes, self.decoded_bytes)


@dataclass(frozen=True)
class ScaleXLayout:
    """``scalex_container.py:64-104``."""

    path: Path
    metadata: dict[str, Any]
    data_base: int
    original_prefix: bytes
    virtual_header: dict[str, Any]
    records: tuple[ScaleXRecord, ...]

    @property
    def layer(self) -> int:
        return int(self.metadata["layer"])

    @property
    def experts(self) -> int:
        return len(self.records)

    @property
    def original_bytes(self) -> int:
        return int(self.metadata["original_bytes"])

    @property
    def virtual_data_base(self) -> int:
        return len(self.original_prefix)

    def record(self, expert: int) -> ScaleXRecord:
        if not 0 <= expert < len(self.records):
            raise ScaleXContainerError(f"ScaleX expert is out of range: {expert}")
        rec = self.records[expert]
        if rec.expert != expert:
            raise ScaleXContainerError("ScaleX record ordering changed")
        return rec


def is_scalex_layer(path) -> bool:
    try:
        with open(path, "rb") as f:
            return f.read(len(SCALEX_MAGIC)) == SCALEX_MAGIC
    except FileNotFoundError:
        return False


def _tensor_range(header: dict[str, Any], name: str, base: int) -> tuple[int, int]:
    entry = header.get(name)
    if not isinstance(entry, dict):
        raise ScaleXContainerError(f"missing tensor in expert shard: {name}")
    try:
        start, end = (int(v) for v in entry["data_offsets"])
    except (KeyError, TypeError, ValueError) as exc:
        raise ScaleXContainerError(f"invalid tensor offsets: {name}") from exc
    if start < 0 or end <= start:
        raise ScaleXContainerError(f"invalid tensor range: {name}")
    return base + start, end - start


def _original_order(header: dict[str, Any], prefix_bytes: int, original_bytes: int):
    """Tensor names in file order; the payload must be gap-free and end at the
    original file length (``scalex_container.py:399-420``)."""
    spans = []
    for name, entry in header.items():
        if name == "__metadata__":
            continue
        start, length = _tensor_range(header, name, 0)
        spans.append((start, start + length, name))
    cursor, order = 0, []
    for start, end, name in sorted(spans):
        if start != cursor:
            raise ScaleXContainerError(f"embedded payload has a gap before {name}")
        cursor = end
        order.append(name)
    if prefix_bytes + cursor != original_bytes:
        raise ScaleXContainerError("embedded payload length differs from original file")
    return tuple(order)


def read_scalex_layout(path) -> ScaleXLayout:
    """Parses and checks a ScaleX layer (``scalex_container.py:220-350``)."""
    source = Path(path).expanduser().resolve()
    with source.open("rb") as f:
        prefix = f.read(SCALEX_PREFIX.size)
        if len(prefix) != SCALEX_PREFIX.size:
            raise ScaleXContainerError(f"truncated ScaleX prefix: {source}")
        magic, version, meta_bytes, stored = SCALEX_PREFIX.unpack(prefix)
        if magic != SCALEX_MAGIC or version != SCALEX_VERSION:
            raise ScaleXContainerError(f"unsupported ScaleX container: {source}")
        if not 2 <= meta_bytes <= 64 << 20:
            raise ScaleXContainerError("invalid ScaleX metadata length")
        raw_meta = f.read(meta_bytes)
        if len(raw_meta) != meta_bytes:
            raise ScaleXContainerError("truncated ScaleX metadata")
        try:
            meta = json.loads(raw_meta)
        except (json.JSONDecodeError, UnicodeDecodeError) as exc:
            raise ScaleXContainerError("invalid ScaleX metadata") from exc
        if (not isinstance(meta, dict) or meta.get("format") != SCALEX_FORMAT
                or int(meta.get("version", -1)) != SCALEX_VERSION):
            raise ScaleXContainerError("unexpected ScaleX metadata format")
        data_base = SCALEX_PREFIX.size + meta_bytes
        if data_base + int(stored) != source.stat().st_size:
            raise ScaleXContainerError("ScaleX stored length differs from file size")
        prefix_bytes = int(meta.get("original_prefix_bytes", -1))
        if prefix_bytes < 10 or prefix_bytes > stored:
            raise ScaleXContainerError("invalid embedded safetensors prefix length")
        original_prefix = f.read(prefix_bytes)
    if len(original_prefix) != prefix_bytes:
        raise ScaleXContainerError("truncated embedded safetensors prefix")
    if hashlib.sha256(original_prefix).hexdigest() != meta.get("original_prefix_sha256"):
        raise ScaleXContainerError("embedded safetensors prefix hash changed")
    (hlen,) = struct.unpack("<Q", original_prefix[:8])
    if hlen + 8 != len(original_prefix):
        raise ScaleXContainerError("embedded safetensors prefix geometry changed")
    try:
        header = json.loads(original_prefix[8:])
    except (json.JSONDecodeError, UnicodeDecodeError) as exc:
        raise ScaleXContainerError("invalid embedded safetensors header") from exc
    if not isinstance(header, dict):
        raise ScaleXContainerError("embedded safetensors header is not an object")
    raw_records = meta.get("records")
    experts = int(meta.get("experts", -1))
    if not isinstance(raw_records, list) or experts < 1 or len(raw_records) != experts:
        raise ScaleXContainerError("ScaleX record inventory changed")
    layer = int(meta["layer"])
    records, cursor = [], prefix_bytes
    for expert, raw in enumerate(raw_records):
        if not isinstance(raw, dict) or int(raw.get("expert", -1)) != expert:
            raise ScaleXContainerError("ScaleX expert ordering changed")
        lists = [raw.get(k) for k in ("scale_names", "scale_nbytes", "weight_names",
                                      "weight_nbytes")]
        if (int(raw.get("stored_offset", -1)) != cursor or int(raw.get("encoded_bytes", -1)) < 24
                or int(raw.get("decoded_bytes", -1)) < 1
                or not all(isinstance(v, list) and len(v) == 3 for v in lists)):
            raise ScaleXContainerError("invalid ScaleX expert record")
        rec = ScaleXRecord(expert=expert, absolute_offset=data_base + cursor,
                           encoded_bytes=int(raw["encoded_bytes"]),
                           decoded_bytes=int(raw["decoded_bytes"]),
                           scale_names=tuple(str(v) for v in lists[0]),
                           scale_nbytes=tuple(int(v) for v in lists[1]),
                           weight_names=tuple(str(v) for v in lists[2]),
                           weight_nbytes=tuple(int(v) for v in lists[3]),
                           codec=str(raw.get("codec")))
        if sum(rec.scale_nbytes) != rec.decoded_bytes or min(
                (*rec.scale_nbytes, *rec.weight_nbytes)) <= 0:
            raise ScaleXContainerError("invalid ScaleX tensor byte geometry")
        if (rec.scale_names != tuple(_name(layer, expert, c, "weight_scale")
                                     for c in SCALE_COMPONENTS)
                or rec.weight_names != tuple(_name(layer, expert, c, "weight_packed")
                                             for c in SCALE_COMPONENTS)):
            raise ScaleXContainerError("ScaleX tensor ordering changed")
        if rec.codec not in {"raw", "one_bit", "two_bit"}:
            raise ScaleXContainerError("invalid ScaleX codec name")
        for name, nbytes in zip((*rec.scale_names, *rec.weight_names),
                                (*rec.scale_nbytes, *rec.weight_nbytes)):
            entry = header.get(name)
            if not isinstance(entry, dict) or entry.get("dtype") != "U8":
                raise ScaleXContainerError(f"invalid embedded ScaleX tensor: {name}")
            if _tensor_range(header, name, 0)[1] != nbytes:
                raise ScaleXContainerError(f"ScaleX tensor length changed: {name}")
        cursor += rec.physical_bytes
        records.append(rec)
    if cursor != int(stored):
        raise ScaleXContainerError("ScaleX records do not cover stored data")
    if int(meta.get("original_bytes", -1)) <= len(original_prefix):
        raise ScaleXContainerError("invalid original ScaleX file length")
    layout = ScaleXLayout(path=source, metadata=meta, data_base=data_base,
                          original_prefix=original_prefix, virtual_header=header,
                          records=tuple(records))
    _original_order(header, len(original_prefix), layout.original_bytes)
    return layout


def _record_tensors(layout: ScaleXLayout, f, expert: int) -> dict[str, bytes]:
    rec = layout.record(expert)
    f.seek(rec.absolute_offset)
    blob = f.read(rec.physical_bytes)
    if len(blob) != rec.physical_bytes:
        raise ScaleXContainerError(f"short read of ScaleX expert {expert}")
    encoded = blob[:rec.encoded_bytes]
    info = inspect_mode_a(encoded)
    if info.raw_bytes != rec.decoded_bytes or info.codec != rec.codec:
        raise ScaleXContainerError(f"ScaleX record metadata changed for expert {expert}")
    scales = decode_mode_a(encoded)
    out, at = {}, 0
    for name, n in zip(rec.scale_names, rec.scale_nbytes):
        out[name] = scales[at:at + n]
        at += n
    at = rec.encoded_bytes
    for name, n in zip(rec.weight_names, rec.weight_nbytes):
        out[name] = blob[at:at + n]
        at += n
    return out


def read_scalex_tensor(layout: ScaleXLayout, name: str) -> bytes:
    """One virtual safetensors tensor of a ScaleX layer (``scalex_container.py:384-396``)."""
    m = _EXPERT_RE.fullmatch(name)
    if m is None or int(m.group(1)) != layout.layer:
        raise ScaleXContainerError(f"tensor is not part of ScaleX layer {layout.layer}: {name}")
    with layout.path.open("rb") as f:
        tensors = _record_tensors(layout, f, int(m.group(2)))
    if name not in tensors:
        raise ScaleXContainerError(f"ScaleX record does not contain tensor: {name}")
    return tensors[name]


def reconstructed_blocks(layout: ScaleXLayout) -> Iterator[bytes]:
    """The original safetensors file, block by block (``scalex_container.py:423-439``)."""
    yield layout.original_prefix
    current, tensors = -1, {}
    with layout.path.open("rb") as f:
        for name in _original_order(layout.virtual_header, len(layout.original_prefix),
                                    layout.original_bytes):
            m = _EXPERT_RE.fullmatch(name)
            if m is None or int(m.group(1)) != layout.layer:
                raise ScaleXContainerError(f"unexpected embedded tensor: {name}")
            if int(m.group(2)) != current:
                current = int(m.group(2))
                tensors = _record_tensors(layout, f, current)
            yield tensors[name]


def verify_scalex_layer(path) -> str:
    """Rebuilds the original file and checks its SHA-256; returns the digest."""
    layout = read_scalex_layout(path)
    digest = hashlib.sha256()
    for block in reconstructed_blocks(layout):
        digest.update(block)
    if digest.hexdigest() != layout.metadata.get("original_sha256"):
        raise ScaleXContainerError("reconstructed ScaleX layer differs from the original")
    return digest.hexdigest()


def compress_scalex_layer(source, destination, *, layer: int, experts: int) -> ScaleXLayout:
    """Writes the ScaleX container of a native expert shard that holds exactly
    the routed-expert tensors of ``layer`` (``scalex_container.py:490-620``)."""
    src, dst = Path(source), Path(destination)
    if is_scalex_layer(src):
        raise ScaleXContainerError("source is already a ScaleX layer")
    if dst.exists():
        raise ScaleXContainerError(f"destination already exists: {dst}")
    with src.open("rb") as f:
        raw_len = f.read(8)
        (hlen,) = struct.unpack("<Q", raw_len)
        raw_header = f.read(hlen)
        original_prefix = raw_len + raw_header
        header = json.loads(raw_header)
        base = len(original_prefix)
        want = {_name(layer, e, c, p) for e in range(experts) for c in SCALE_COMPONENTS
                for p in ("weight_packed", "weight_scale")}
        if set(header) - {"__metadata__"} != want:
            raise ScaleXContainerError("expert shard inventory changed")
        _original_order(header, base, src.stat().st_size)
        records, blobs, cursor = [], [], base
        for e in range(experts):
            scale_names = [_name(layer, e, c, "weight_scale") for c in SCALE_COMPONENTS]
            weight_names = [_name(layer, e, c, "weight_packed") for c in SCALE_COMPONENTS]
            scale_parts = []
            for n in scale_names:
                off, ln = _tensor_range(header, n, base)
                f.seek(off)
                scale_parts.append(f.read(ln))
            raw_scales = b"".join(scale_parts)
            encoded = encode_mode_a(raw_scales)
            if decode_mode_a(encoded) != raw_scales:
                raise ScaleXContainerError(f"ScaleX round trip failed for expert {e}")
            mode_b_tile_prefix(encoded)
            weights = []
            for n in weight_names:
                off, ln = _tensor_range(header, n, base)
                f.seek(off)
                weights.append(f.read(ln))
            records.append({"expert": e, "stored_offset": cursor, "encoded_bytes": len(encoded),
                            "decoded_bytes": len(raw_scales),
                            "codec": inspect_mode_a(encoded).codec, "scale_names": scale_names,
                            "scale_nbytes": [len(p) for p in scale_parts],
                            "weight_names": weight_names, "weight_nbytes": [len(w) for w in weights]})
            blobs.append(encoded + b"".join(weights))
            cursor += len(blobs[-1])
    digest = hashlib.sha256()
    with src.open("rb") as f:
        for block in iter(lambda: f.read(16 << 20), b""):
            digest.update(block)
    meta = {"format": SCALEX_FORMAT, "version": SCALEX_VERSION, "layer": int(layer),
            "experts": int(experts), "scale_order": list(SCALE_COMPONENTS),
            "weight_order": list(SCALE_COMPONENTS), "original_bytes": src.stat().st_size,
            "original_sha256": digest.hexdigest(), "original_prefix_bytes": base,
            "original_prefix_sha256": hashlib.sha256(original_prefix).hexdigest(),
            "records": records}
    raw_meta = json.dumps(meta, sort_keys=True, separators=(",", ":")).encode()
    with dst.open("xb") as out:
        out.write(SCALEX_PREFIX.pack(SCALEX_MAGIC, SCALEX_VERSION, len(raw_meta), cursor))
        out.write(raw_meta)
        out.write(original_prefix)
        for blob in blobs:
            out.write(blob)
    os.chmod(dst, src.stat().st_mode)
    verify_scalex_layer(dst)
    return read_scalex_layout(dst)
