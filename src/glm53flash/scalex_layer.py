"""ScaleX layer containers: one layer's routed-expert shard with each expert's
three scale tensors stored coded (``scale_codec`` Mode A) and its weights as
they were.

File format (the reference's ``livglm_scalex_layer_v1``, kept byte for byte so
that containers written by either side read on the other):

  prefix    ``<8sIIQ``: magic ``LVGLMSX1``, version 1, metadata length m,
            stored length s
  metadata  m bytes of JSON: ``format``, ``version``, ``layer``, ``experts``,
            ``scale_order`` = ``weight_order`` = gate, down, up,
            ``original_bytes`` / ``original_sha256`` (the safetensors file it
            was made from), ``original_prefix_bytes`` /
            ``original_prefix_sha256``, and ``records``: per expert
            ``expert``, ``stored_offset``, ``encoded_bytes``,
            ``decoded_bytes``, ``codec``, ``scale_names`` / ``scale_nbytes``,
            ``weight_names`` / ``weight_nbytes``
  stored    s bytes: the original file's prefix (length + JSON header, so
            every tensor name still resolves against the original layout),
            then per expert in id order: coded scales | gate | down | up
            weights

The original file can be rebuilt exactly (``ScaleXLayer.verify`` hashes the
rebuild against ``original_sha256``).  The HBM bank loader reads one record
per expert: the coded scales and the three weights in one range.
"""

from __future__ import annotations

from dataclasses import dataclass
import hashlib
import json
import math
from pathlib import Path
import re
import struct
from typing import Any, Iterator

from .checkpoint import ELEMENT_BYTES, read_safetensors_header
from .contract import ContractError
from .scale_codec import MODE_A_HEADER, decode_mode_a, inspect_mode_a

FORMAT = "livglm_scalex_layer_v1"
MAGIC = b"LVGLMSX1"
VERSION = 1
PREFIX = struct.Struct("<8sIIQ")
RECORD_ORDER = ("gate_proj", "down_proj", "up_proj")  # scales, then weights, in this order
CODECS = ("raw", "one_bit", "two_bit")

_TENSOR = re.compile(r"^model\.language_model\.layers\.(\d+)\.mlp\.experts\.(\d+)\."
                     r"(down_proj|gate_proj|up_proj)\.(weight_packed|weight_scale)$")


class ScaleXError(ContractError):
    """A ScaleX container is malformed or does not match what it claims."""


def tensor_name(layer: int, expert: int, component: str, part: str) -> str:
    return f"model.language_model.layers.{layer}.mlp.experts.{expert}.{component}.{part}"


def is_scalex_file(path) -> bool:
    try:
        with open(path, "rb") as fh:
            return fh.read(len(MAGIC)) == MAGIC
    except OSError:
        return False


@dataclass(frozen=True)
class CodedExpert:
    """One expert's record: ``coded_bytes`` of Mode-A scales, then the gate,
    down and up weights, starting at file offset ``offset``."""

    expert: int
    offset: int
    coded_bytes: int
    codec: str
    scale_bytes: tuple[int, int, int]   # decoded gate, down, up scale sizes
    weight_bytes: tuple[int, int, int]  # gate, down, up packed weights

    @property
    def nbytes(self) -> int:
        return self.coded_bytes + sum(self.weight_bytes)

    @property
    def decoded_bytes(self) -> int:
        return sum(self.scale_bytes)

    def weight_offset(self, i: int) -> int:
        """Offset of weight ``i`` (gate 0, down 1, up 2) inside the record."""
        return self.coded_bytes + sum(self.weight_bytes[:i])


# metadata fields: name -> check of its value
def _is_count(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool) and v >= 0


def _is_digest(v) -> bool:
    return isinstance(v, str) and re.fullmatch(r"[0-9a-f]{64}", v) is not None


_META_FIELDS = {
    "format": lambda v: v == FORMAT,
    "version": lambda v: v == VERSION,
    "layer": _is_count,
    "experts": lambda v: _is_count(v) and v >= 1,
    "scale_order": lambda v: v == list(RECORD_ORDER),
    "weight_order": lambda v: v == list(RECORD_ORDER),
    "original_bytes": _is_count,
    "original_sha256": _is_digest,
    "original_prefix_bytes": lambda v: _is_count(v) and v > PREFIX.size,
    "original_prefix_sha256": _is_digest,
    "records": lambda v: isinstance(v, list),
}

_RECORD_FIELDS = {
    "expert": _is_count,
    "stored_offset": _is_count,
    "encoded_bytes": lambda v: _is_count(v) and v >= MODE_A_HEADER.size,
    "decoded_bytes": lambda v: _is_count(v) and v >= 1,
    "codec": lambda v: v in CODECS,
    "scale_names": lambda v: isinstance(v, list) and len(v) == 3,
    "scale_nbytes": lambda v: isinstance(v, list) and len(v) == 3 and all(
        _is_count(x) and x > 0 for x in v),
    "weight_names": lambda v: isinstance(v, list) and len(v) == 3,
    "weight_nbytes": lambda v: isinstance(v, list) and len(v) == 3 and all(
        _is_count(x) and x > 0 for x in v),
}


def _check_fields(obj: Any, fields: dict, what: str) -> None:
    if not isinstance(obj, dict):
        raise ScaleXError(f"{what} is not a JSON object")
    for key, ok in fields.items():
        if key not in obj:
            raise ScaleXError(f"{what} lacks {key!r}")
        if not ok(obj[key]):
            raise ScaleXError(f"{what} has an unusable {key!r}: {obj[key]!r}")


def _header_size(header: dict[str, Any], name: str) -> int:
    """Bytes of tensor ``name`` in the embedded header (U8 required)."""
    entry = header.get(name)
    if not isinstance(entry, dict) or entry.get("dtype") != "U8":
        raise ScaleXError(f"the embedded header has no U8 tensor {name}")
    begin, end = entry.get("data_offsets", (0, -1))
    if end - begin != math.prod(entry.get("shape", ())) * ELEMENT_BYTES["U8"] or begin < 0:
        raise ScaleXError(f"{name}: embedded byte range does not match its shape")
    return end - begin


def _payload_order(header: dict[str, Any]) -> list[tuple[int, int, str]]:
    """(begin, end, name) of every tensor, in file order, tiling the data area
    from byte 0 with no gap (the original file can then be rebuilt)."""
    spans = sorted((int(e["data_offsets"][0]), int(e["data_offsets"][1]), n)
                   for n, e in header.items() if n != "__metadata__")
    at = 0
    for begin, end, n in spans:
        if begin != at:
            raise ScaleXError(f"the original data area is not contiguous at {n}")
        at = end
    return spans


@dataclass(frozen=True)
class ScaleXLayer:
    path: Path
    layer: int
    records: tuple[CodedExpert, ...]
    original_bytes: int
    original_sha256: str
    original_prefix: bytes
    original_header: dict[str, Any]

    @property
    def original_data_base(self) -> int:
        """Where the original file's data area started (its tensors' offsets
        count from there)."""
        return len(self.original_prefix)

    @property
    def experts(self) -> int:
        return len(self.records)

    def record(self, expert: int) -> CodedExpert:
        if not 0 <= expert < len(self.records):
            raise ScaleXError(f"{self.path}: no expert {expert} (layer holds {self.experts})")
        return self.records[expert]

    # ------------------------------------------------------------ reading
    @classmethod
    def read(cls, path) -> "ScaleXLayer":
        path = Path(path).expanduser().resolve()
        size = path.stat().st_size
        with path.open("rb") as fh:
            head = fh.read(PREFIX.size)
            if len(head) != PREFIX.size:
                raise ScaleXError(f"{path}: shorter than the ScaleX prefix")
            magic, version, meta_len, stored = PREFIX.unpack(head)
            if magic != MAGIC or version != VERSION:
                raise ScaleXError(f"{path}: magic {magic!r} version {version} is not ScaleX v1")
            if PREFIX.size + meta_len + stored != size:
                raise ScaleXError(f"{path}: prefix promises {PREFIX.size + meta_len + stored} "
                                  f"bytes, the file has {size}")
            try:
                meta = json.loads(fh.read(meta_len))
            except (UnicodeDecodeError, json.JSONDecodeError) as exc:
                raise ScaleXError(f"{path}: metadata is not JSON ({exc})") from exc
            _check_fields(meta, _META_FIELDS, f"{path} metadata")
            n_prefix = meta["original_prefix_bytes"]
            if n_prefix > stored:
                raise ScaleXError(f"{path}: original prefix ({n_prefix} B) exceeds stored data")
            prefix = fh.read(n_prefix)
        if hashlib.sha256(prefix).hexdigest() != meta["original_prefix_sha256"]:
            raise ScaleXError(f"{path}: the embedded original prefix fails its SHA-256")
        (hlen,) = struct.unpack_from("<Q", prefix)
        if 8 + hlen != n_prefix:
            raise ScaleXError(f"{path}: embedded prefix length {n_prefix} != 8 + {hlen}")
        try:
            header = json.loads(prefix[8:])
        except (UnicodeDecodeError, json.JSONDecodeError) as exc:
            raise ScaleXError(f"{path}: embedded header is not JSON ({exc})") from exc
        if not isinstance(header, dict):
            raise ScaleXError(f"{path}: embedded header is not an object")
        spans = _payload_order(header)
        if n_prefix + (spans[-1][1] if spans else 0) != meta["original_bytes"]:
            raise ScaleXError(f"{path}: the original tensors do not add up to "
                              f"original_bytes = {meta['original_bytes']}")
        layer, n_exp = meta["layer"], meta["experts"]
        raw = meta["records"]
        if len(raw) != n_exp:
            raise ScaleXError(f"{path}: {len(raw)} records for {n_exp} experts")
        base = PREFIX.size + meta_len
        cursor = n_prefix  # stored offset of the next record
        records = []
        for e, r in enumerate(raw):
            what = f"{path} record {e}"
            _check_fields(r, _RECORD_FIELDS, what)
            if r["expert"] != e or r["stored_offset"] != cursor:
                raise ScaleXError(f"{what}: expert {r['expert']} at {r['stored_offset']}, "
                                  f"expected expert {e} at {cursor}")
            want_s = [tensor_name(layer, e, c, "weight_scale") for c in RECORD_ORDER]
            want_w = [tensor_name(layer, e, c, "weight_packed") for c in RECORD_ORDER]
            if r["scale_names"] != want_s or r["weight_names"] != want_w:
                raise ScaleXError(f"{what}: tensor names are not layer {layer} expert {e}'s "
                                  "gate, down, up")
            if sum(r["scale_nbytes"]) != r["decoded_bytes"]:
                raise ScaleXError(f"{what}: scale sizes do not sum to decoded_bytes")
            for n, nb in zip(want_s + want_w, r["scale_nbytes"] + r["weight_nbytes"]):
                if _header_size(header, n) != nb:
                    raise ScaleXError(f"{what}: {n} is {nb} bytes here, "
                                      f"{_header_size(header, n)} in the embedded header")
            rec = CodedExpert(expert=e, offset=base + cursor, coded_bytes=r["encoded_bytes"],
                              codec=r["codec"], scale_bytes=tuple(r["scale_nbytes"]),
                              weight_bytes=tuple(r["weight_nbytes"]))
            records.append(rec)
            cursor += rec.nbytes
        if cursor != stored:
            raise ScaleXError(f"{path}: records end at {cursor}, stored data at {stored}")
        return cls(path=path, layer=layer, records=tuple(records),
                   original_bytes=meta["original_bytes"], original_sha256=meta["original_sha256"],
                   original_prefix=prefix, original_header=header)

    def _expert_tensors(self, fh, expert: int) -> dict[str, bytes]:
        """All six tensors of one expert, scales decoded."""
        rec = self.record(expert)
        fh.seek(rec.offset)
        blob = fh.read(rec.nbytes)
        if len(blob) != rec.nbytes:
            raise ScaleXError(f"{self.path}: record {expert} cut short")
        coded = blob[:rec.coded_bytes]
        info = inspect_mode_a(coded)
        if info.codec != rec.codec or info.raw_bytes != rec.decoded_bytes:
            raise ScaleXError(f"{self.path}: record {expert} is coded as {info.codec} of "
                              f"{info.raw_bytes} B, metadata says {rec.codec} of "
                              f"{rec.decoded_bytes} B")
        scales = decode_mode_a(coded)
        out: dict[str, bytes] = {}
        s_at = 0
        for i, comp in enumerate(RECORD_ORDER):
            n = rec.scale_bytes[i]
            out[tensor_name(self.layer, expert, comp, "weight_scale")] = scales[s_at:s_at + n]
            s_at += n
            w_at = rec.weight_offset(i)
            out[tensor_name(self.layer, expert, comp, "weight_packed")] = \
                blob[w_at:w_at + rec.weight_bytes[i]]
        return out

    def tensor_bytes(self, name: str) -> bytes:
        """The bytes tensor ``name`` had in the original file."""
        m = _TENSOR.fullmatch(name)
        if m is None or int(m.group(1)) != self.layer:
            raise ScaleXError(f"{self.path}: {name} is not a routed tensor of layer {self.layer}")
        with self.path.open("rb") as fh:
            return self._expert_tensors(fh, int(m.group(2)))[name]

    def original_blocks(self) -> Iterator[bytes]:
        """The original safetensors file, piece by piece."""
        yield self.original_prefix
        cache: tuple[int, dict[str, bytes]] = (-1, {})
        with self.path.open("rb") as fh:
            for _, _, n in _payload_order(self.original_header):
                m = _TENSOR.fullmatch(n)
                if m is None or int(m.group(1)) != self.layer:
                    raise ScaleXError(f"{self.path}: embedded tensor {n} is not this layer's")
                e = int(m.group(2))
                if cache[0] != e:
                    cache = (e, self._expert_tensors(fh, e))
                yield cache[1][n]

    def verify(self) -> str:
        """Rebuilds the original file and checks its SHA-256; returns it."""
        h = hashlib.sha256()
        for block in self.original_blocks():
            h.update(block)
        if h.hexdigest() != self.original_sha256:
            raise ScaleXError(f"{self.path}: rebuilt original does not match original_sha256")
        return self.original_sha256
