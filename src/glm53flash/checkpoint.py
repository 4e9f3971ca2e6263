"""Read-only view of a safetensors checkpoint directory, as far as the expert
bank loader needs it: which shard holds a tensor and at which file bytes.

A checkpoint directory holds ``model.safetensors.index.json`` (its
``weight_map`` maps every tensor name to a shard file) and the shards.  A
safetensors shard is an 8-byte little-endian length ``n``, an ``n``-byte JSON
header ``{name: {"dtype", "shape", "data_offsets": [begin, end]}}`` and the data
area, which starts right after the header; offsets are relative to it.  A
shard may also be a ScaleX layer container (``scalex_layer``), whose embedded
original prefix answers the same questions about the original file.

Shard headers are read lazily, once each, and every tensor entry is checked
before it is handed out: a known dtype, non-negative dimensions, a byte range
of exactly dtype size x element count, inside the (original) file.
"""

from __future__ import annotations

from dataclasses import dataclass
import json
import math
from pathlib import Path
import struct
from typing import Any

from .contract import ContractError

INDEX_FILE = "model.safetensors.index.json"

# bytes per element of the safetensors dtype names
ELEMENT_BYTES = {
    "BOOL": 1, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E5M2": 1, "F8_E8M0": 1,
    "U16": 2, "I16": 2, "F16": 2, "BF16": 2,
    "U32": 4, "I32": 4, "F32": 4,
    "U64": 8, "I64": 8, "F64": 8,
}

_LEN = struct.Struct("<Q")
_MAX_HEADER = 256 << 20


@dataclass(frozen=True)
class TensorRange:
    """A tensor's bytes: ``nbytes`` at ``offset`` of ``shard`` (an offset into
    the original file for a ScaleX shard)."""

    name: str
    shard: str
    offset: int
    nbytes: int
    dtype: str
    shape: tuple[int, ...]

    @property
    def end(self) -> int:
        return self.offset + self.nbytes


def read_safetensors_header(path) -> tuple[int, dict[str, Any]]:
    """(file offset of the data area, the JSON header) of a safetensors file."""
    with open(path, "rb") as fh:
        head = fh.read(_LEN.size)
        if len(head) < _LEN.size:
            raise ContractError(f"{path}: shorter than a safetensors length field")
        (n,) = _LEN.unpack(head)
        if n > _MAX_HEADER:
            raise ContractError(f"{path}: header length {n} is implausible")
        raw = fh.read(n)
    if len(raw) != n:
        raise ContractError(f"{path}: header cut short ({len(raw)} of {n} bytes)")
    try:
        header = json.loads(raw)
    except (UnicodeDecodeError, json.JSONDecodeError) as exc:
        raise ContractError(f"{path}: header is not JSON ({exc})") from exc
    if not isinstance(header, dict):
        raise ContractError(f"{path}: header is a {type(header).__name__}, not an object")
    return _LEN.size + n, header


def _entry_range(name: str, entry: Any) -> tuple[str, tuple[int, ...], int, int]:
    """dtype, shape and (begin, end) of one header entry, checked for shape."""
    if not isinstance(entry, dict):
        raise ContractError(f"{name}: header entry is not an object")
    dtype = entry.get("dtype")
    shape = entry.get("shape")
    offsets = entry.get("data_offsets")
    if not isinstance(dtype, str) or dtype not in ELEMENT_BYTES:
        raise ContractError(f"{name}: dtype {dtype!r} is not a safetensors dtype")
    if (not isinstance(shape, list) or not all(isinstance(v, int) and v >= 0 for v in shape)):
        raise ContractError(f"{name}: shape {shape!r} is not a list of sizes")
    if (not isinstance(offsets, list) or len(offsets) != 2
            or not all(isinstance(v, int) for v in offsets)):
        raise ContractError(f"{name}: data_offsets {offsets!r} are not a [begin, end] pair")
    begin, end = offsets
    want = ELEMENT_BYTES[dtype] * math.prod(shape)
    if begin < 0 or end - begin != want:
        raise ContractError(f"{name}: data_offsets {offsets} hold {end - begin} bytes; "
                            f"{dtype} {shape} needs {want}")
    return dtype, tuple(shape), begin, end


class ShardIndex:
    """The checkpoint at ``root``: tensor name -> shard, shard headers on demand."""

    def __init__(self, root, weight_map: dict[str, str], config: dict[str, Any] | None = None):
        self.root = Path(root)
        if not isinstance(weight_map, dict) or not weight_map:
            raise ContractError(f"{self.root}: the index maps no tensors")
        for key, shard in weight_map.items():
            if not isinstance(key, str) or not isinstance(shard, str) or not shard:
                raise ContractError(f"{self.root}: index entry {key!r} -> {shard!r} is malformed")
        self.weight_map = dict(weight_map)
        self.config = config or {}
        self._shards: dict[str, tuple[int, dict[str, Any], int, Any]] = {}

    @classmethod
    def open(cls, root) -> "ShardIndex":
        root = Path(root).expanduser().resolve()
        index_path = root / INDEX_FILE
        if not index_path.is_file():
            raise ContractError(f"{root}: no {INDEX_FILE}")
        try:
            index = json.loads(index_path.read_text(encoding="utf-8"))
        except (OSError, UnicodeDecodeError, json.JSONDecodeError) as exc:
            raise ContractError(f"{index_path}: unreadable ({exc})") from exc
        if not isinstance(index, dict):
            raise ContractError(f"{index_path}: not a JSON object")
        config = None
        config_path = root / "config.json"
        if config_path.is_file():
            try:
                config = json.loads(config_path.read_text(encoding="utf-8"))
            except (OSError, UnicodeDecodeError, json.JSONDecodeError) as exc:
                raise ContractError(f"{config_path}: unreadable ({exc})") from exc
        return cls(root, index.get("weight_map"), config if isinstance(config, dict) else None)

    def shard_path(self, shard: str) -> Path:
        return self.root / shard

    def _shard(self, shard: str):
        """(data base, header, file size as the header sees it, ScaleX layer or None)."""
        got = self._shards.get(shard)
        if got is None:
            from .scalex_layer import ScaleXError, ScaleXLayer, is_scalex_file
            path = self.shard_path(shard)
            if not path.is_file():
                raise ContractError(f"{path}: shard named by the index does not exist")
            if is_scalex_file(path):
                try:
                    layer = ScaleXLayer.read(path)
                except ScaleXError as exc:
                    raise ContractError(f"{path}: {exc}") from exc
                got = (layer.original_data_base, layer.original_header, layer.original_bytes,
                       layer)
            else:
                base, header = read_safetensors_header(path)
                got = (base, header, path.stat().st_size, None)
            self._shards[shard] = got
        return got

    def scalex(self, shard: str):
        """The shard's ScaleX layer, or None for a plain safetensors shard."""
        return self._shard(shard)[3]

    def locate(self, name: str) -> TensorRange:
        """Where tensor ``name`` lies."""
        shard = self.weight_map.get(name)
        if shard is None:
            raise ContractError(f"{name}: not in the checkpoint index")
        base, header, size, _ = self._shard(shard)
        if name not in header:
            raise ContractError(f"{name}: the index names {shard}, whose header lacks it")
        dtype, shape, begin, end = _entry_range(name, header[name])
        if base + end > size:
            raise ContractError(f"{name}: bytes [{base + begin}, {base + end}) run past the "
                                f"{size}-byte shard {shard}")
        return TensorRange(name, shard, base + begin, end - begin, dtype, shape)
