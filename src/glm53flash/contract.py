"""Checkpoint contract: errors, the routed-expert tensor names, and a
metadata-only view of a safetensors checkpoint (index + shard headers).

Mirrors the parts of the reference's ``contract.py`` that locate routed-expert
bytes on disk: ``ContractError`` (``contract.py:54-55``), the expert naming
and component order (``contract.py:20-26,47-51``), ``tensor_payload_bytes``
(``contract.py:58-70``), ``TensorSource`` (``contract.py:73-83``) and
``ModelContract`` with ``partition`` / ``_header`` / ``tensor`` (``contract.py:112-364``), plus the
local header reader ``local_safetensors_header`` (``hf_range.py:123-132``).
The reference's provenance checks of its composite checkpoint
(``VALIDATION.json`` and ``livseek-composite.json``, ``contract.py:139-196``)
and its whole-model inventory counts (``contract.py:198-250,273-291``) belong to the
checkpoint builder and are not part of this layer's loader.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass
import json
import os
import re
import struct
from pathlib import Path
from typing import Any, Iterable

FIRST_MOE_LAYER = 3
LAST_MAIN_LAYER = 44
MTP_LAYER = 45
EXPERTS_PER_LAYER = 288
TOP_K = 8
EXPERT_COMPONENTS = ("down_proj", "gate_proj", "up_proj")
EXPERT_PARTS = ("weight_packed", "weight_scale")

DTYPE_BYTES = {
    "BOOL": 1, "U8": 1, "I8": 1, "F8_E4M3": 1, "F8_E5M2": 1, "F8_E8M0": 1,
    "U16": 2, "I16": 2, "F16": 2, "BF16": 2,
    "U32": 4, "I32": 4, "F32": 4,
    "U64": 8, "I64": 8, "F64": 8,
}

ROUTED_EXPERT_RE = re.compile(
    r"^model\.language_model\.layers\.(\d+)\.mlp\.experts\.(\d+)\."
    r"(down_proj|gate_proj|up_proj)\.(weight_packed|weight_scale)$"
)
LANGUAGE_LAYER_RE = re.compile(r"^model\.language_model\.layers\.(\d+)\.")


class ContractError(ValueError):
    """The inputs do not satisfy the supported native contract."""


def expert_tensor_name(layer: int, expert: int, component: str, part: str) -> str:
    """Checkpoint name of one routed-expert tensor (``expert_source.py:281-284``)."""
    return f"model.language_model.layers.{layer}.mlp.experts.{expert}.{component}.{part}"


def tensor_payload_bytes(dtype: str, shape: Iterable[int]) -> int:
    """``contract.py:58-70``."""
    try:
        element_bytes = DTYPE_BYTES[dtype]
    except KeyError as exc:
        raise ContractError(f"unsupported safetensors dtype: {dtype}") from exc
    elements = 1
    for raw in shape:
        dim = int(raw)
        if dim < 0:
            raise ContractError(f"negative tensor dimension: {dim}")
        elements *= dim
    return elements * element_bytes


def local_safetensors_header(path: str | os.PathLike) -> tuple[int, dict[str, Any]]:
    """(absolute offset of the data area, parsed JSON header) of a local
    safetensors file: an 8-byte little-endian header length, the JSON header,
    then the data (``hf_range.py:123-132``)."""
    with open(path, "rb") as handle:
        raw = handle.read(8)
        if len(raw) != 8:
            raise ValueError(f"truncated safetensors file: {path}")
        (length,) = struct.unpack("<Q", raw)
        header = handle.read(length)
        if len(header) != length:
            raise ValueError(f"truncated safetensors header: {path}")
    value = json.loads(header)
    if not isinstance(value, dict):
        raise ValueError(f"safetensors header is not an object: {path}")
    return 8 + length, value


@dataclass(frozen=True)
class TensorSource:
    """Where one tensor's bytes sit in its shard (``contract.py:73-83``)."""

    name: str
    shard_name: str
    absolute_offset: int
    byte_length: int
    dtype: str
    shape: tuple[int, ...]

    def as_dict(self) -> dict[str, Any]:
        return asdict(self)


class ModelContract:
    """Metadata-only view of a checkpoint directory: ``config.json`` and
    ``model.safetensors.index.json`` (``weight_map``: tensor name -> shard),
    with each shard's header read on first use (``contract.py:112-169,293-310``)."""

    def __init__(self, model_dir: str | os.PathLike, config: dict[str, Any],
                 index: dict[str, Any]):
        self.model_dir = Path(model_dir)
        self.config = config
        self.index = index
        weight_map = index.get("weight_map")
        if not isinstance(weight_map, dict) or not weight_map:
            raise ContractError("model index has no weight_map")
        if any(not isinstance(n, str) or not isinstance(s, str) for n, s in weight_map.items()):
            raise ContractError("model index weight_map must contain string names and shards")
        self.weight_map: dict[str, str] = dict(weight_map)
        self._headers: dict[str, tuple[int, dict[str, Any]]] = {}
        self._sources: dict[str, TensorSource] = {}
        self._scalex: dict[str, Any] = {}

    @classmethod
    def from_model_dir(cls, model_dir: str | os.PathLike) -> "ModelContract":
        root = Path(model_dir).expanduser().resolve()
        required = {"config": root / "config.json", "index": root / "model.safetensors.index.json"}
        missing = [str(p) for p in required.values() if not p.is_file()]
        if missing:
            raise ContractError(f"checkpoint metadata is incomplete: {missing}")

        def read(path: Path) -> dict[str, Any]:
            try:
                value = json.loads(path.read_text(encoding="utf-8"))
            except (OSError, json.JSONDecodeError) as exc:
                raise ContractError(f"cannot read JSON metadata: {path}") from exc
            if not isinstance(value, dict):
                raise ContractError(f"JSON metadata must be an object: {path}")
            return value

        return cls(root, read(required["config"]), read(required["index"]))

    @property
    def tensor_names(self) -> tuple[str, ...]:
        return tuple(self.weight_map)

    @staticmethod
    def partition(name: str) -> str:
        """``contract.py:252-268``."""
        if name.startswith("model.visual."):
            return "vision"
        expert = ROUTED_EXPERT_RE.fullmatch(name)
        if expert is not None:
            layer = int(expert.group(1))
            if FIRST_MOE_LAYER <= layer <= LAST_MAIN_LAYER:
                return "routed"
            if layer == MTP_LAYER:
                return "mtp"
            return "unknown"
        match = LANGUAGE_LAYER_RE.match(name)
        if match is not None and int(match.group(1)) == MTP_LAYER:
            return "mtp"
        if name.startswith("model.language_model.") or name == "lm_head.weight":
            return "resident"
        return "unknown"

    def names_for(self, partition: str) -> tuple[str, ...]:
        return tuple(n for n in self.weight_map if self.partition(n) == partition)

    def shard_path(self, shard_name: str) -> Path:
        return self.model_dir / shard_name

    def scalex_layout(self, shard_name: str):
        """The ScaleX layout of a shard, or None for a native safetensors shard
        (``contract.py:312-320``)."""
        if shard_name not in self._scalex:
            from .scalex_container import ScaleXContainerError, is_scalex_layer, read_scalex_layout
            path = self.shard_path(shard_name)
            try:
                self._scalex[shard_name] = (read_scalex_layout(path) if is_scalex_layer(path)
                                            else None)
            except ScaleXContainerError as exc:
                raise ContractError(str(exc)) from exc
        return self._scalex[shard_name]

    def _header(self, shard_name: str) -> tuple[int, dict[str, Any]]:
        """(data base, header) of a shard; for a ScaleX shard the embedded
        original header, whose offsets address the original file
        (``contract.py:293-310``)."""
        cached = self._headers.get(shard_name)
        if cached is not None:
            return cached
        path = self.shard_path(shard_name)
        if not path.is_file():
            raise ContractError(f"indexed shard is missing: {path}")
        layout = self.scalex_layout(shard_name)
        try:
            cached = (local_safetensors_header(path) if layout is None
                      else (layout.virtual_data_base, layout.virtual_header))
        except (OSError, ValueError) as exc:
            raise ContractError(f"cannot read safetensors header: {path}") from exc
        self._headers[shard_name] = cached
        return cached

    def tensor(self, name: str) -> TensorSource:
        """Resolves ``name`` to its shard byte range, checking that the header
        entry is well formed, that its byte length matches dtype x shape and
        that it lies inside the shard (``contract.py:322-364``)."""
        cached = self._sources.get(name)
        if cached is not None:
            return cached
        try:
            shard_name = self.weight_map[name]
        except KeyError as exc:
            raise ContractError(f"tensor is absent from model index: {name}") from exc
        data_base, header = self._header(shard_name)
        entry = header.get(name)
        if not isinstance(entry, dict):
            raise ContractError(f"indexed tensor is absent from {shard_name}: {name}")
        try:
            dtype = str(entry["dtype"])
            shape = tuple(int(v) for v in entry["shape"])
            start, end = (int(v) for v in entry["data_offsets"])
        except (KeyError, TypeError, ValueError) as exc:
            raise ContractError(f"invalid safetensors metadata for {name}") from exc
        byte_length = end - start
        expected = tensor_payload_bytes(dtype, shape)
        if start < 0 or byte_length != expected:
            raise ContractError(f"invalid tensor byte range for {name}: {byte_length} != {expected}")
        absolute_offset = data_base + start
        layout = self.scalex_layout(shard_name)
        size = (layout.original_bytes if layout is not None
                else self.shard_path(shard_name).stat().st_size)
        if absolute_offset + byte_length > size:
            raise ContractError(f"tensor exceeds shard size: {name}")
        source = TensorSource(name=name, shard_name=shard_name, absolute_offset=absolute_offset,
                              byte_length=byte_length, dtype=dtype, shape=shape)
        self._sources[name] = source
        return source


def routed_expert_parts(name: str) -> tuple[int, int, str, str]:
    """(layer, expert, component, part) of a routed-expert tensor name
    (``contract.py:383-392``)."""
    match = ROUTED_EXPERT_RE.fullmatch(name)
    if match is None:
        raise ContractError(f"not a native routed-expert tensor: {name}")
    return int(match.group(1)), int(match.group(2)), match.group(3), match.group(4)
