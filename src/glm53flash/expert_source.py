"""Where each routed expert's MXFP4 tensors sit in the checkpoint shards.

Mirrors the reference's native-safetensors source plan (``expert_source.py``):
per (layer, expert) the six U8 tensors in canonical order -- components
``down_proj, gate_proj, up_proj`` x parts ``weight_packed, weight_scale``
(``contract.py:25-26``) -- with their shard byte ranges, their shape checks,
and the expert's coalesced read ranges.  A checkpoint at the real geometry
stores each expert as one contiguous 13,369,344-byte record, so one read
covers it (``expert_source.py:365-381``).  In a ScaleX layer shard an expert is
one physical record too -- its coded scales then its gate, down and up weights
(``expert_source.py:306-337``) -- read as one range.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

from .contract import (
    EXPERT_COMPONENTS,
    EXPERT_PARTS,
    EXPERTS_PER_LAYER,
    FIRST_MOE_LAYER,
    LAST_MAIN_LAYER,
    ContractError,
    ModelContract,
    TensorSource,
    expert_tensor_name,
)
from .model_config import GLMTextConfig

REAL_EXPERT_RECORD_BYTES = 13_369_344


@dataclass(frozen=True)
class ExpertTensorSource:
    """One expert tensor: its checkpoint name and byte range, and the name,
    dtype and shape the reference gives its slot array (U32 view of the packed
    codes, U8 scales; ``expert_source.py:22-32,207-229``)."""

    source_name: str
    destination_name: str
    shard_name: str
    absolute_offset: int
    byte_length: int
    source_shape: tuple[int, ...]
    mlx_dtype: str
    mlx_shape: tuple[int, ...]

    @property
    def bank_name(self) -> str:
        """Key of the stacked bank tensor this tensor fills
        (``<component>.weight_packed`` / ``<component>.weight_scale``)."""
        return ".".join(self.source_name.rsplit(".", 2)[-2:])


@dataclass(frozen=True)
class ExpertReadRange:
    """A run of adjacent tensors in one shard, read as one range
    (``expert_source.py:34-43``)."""

    shard_name: str
    absolute_offset: int
    byte_length: int
    tensors: tuple[ExpertTensorSource, ...]

    def relative_offset(self, tensor: ExpertTensorSource) -> int:
        return tensor.absolute_offset - self.absolute_offset


@dataclass(frozen=True)
class NativeExpertSource:
    """``expert_source.py:45-60``."""

    layer: int
    expert: int
    tensors: tuple[ExpertTensorSource, ...]
    read_ranges: tuple[ExpertReadRange, ...]
    scalex_record: object = None  # a ScaleXRecord for a ScaleX shard

    @property
    def payload_bytes(self) -> int:
        return sum(t.byte_length for t in self.tensors)

    @property
    def read_bytes(self) -> int:
        return sum(r.byte_length for r in self.read_ranges)


@dataclass(frozen=True)
class NativeExpertSourcePlan:
    """Every routed expert of layers ``first_layer..last_layer`` in canonical
    (layer, expert) order (``expert_source.py:62-186``)."""

    model_dir: str
    first_layer: int
    last_layer: int
    experts_per_layer: int
    packs: tuple[NativeExpertSource, ...]

    @property
    def layer_count(self) -> int:
        return self.last_layer - self.first_layer + 1

    @property
    def expert_count(self) -> int:
        return len(self.packs)

    @property
    def tensor_count(self) -> int:
        return sum(len(p.tensors) for p in self.packs)

    @property
    def payload_bytes(self) -> int:
        return sum(p.payload_bytes for p in self.packs)

    @property
    def read_bytes(self) -> int:
        return sum(p.read_bytes for p in self.packs)

    @property
    def source_shard_count(self) -> int:
        return len({r.shard_name for p in self.packs for r in p.read_ranges})

    @property
    def uniform_pack_bytes(self) -> int | None:
        values = {p.payload_bytes for p in self.packs}
        return next(iter(values)) if len(values) == 1 else None

    @property
    def uniform_read_count(self) -> int | None:
        values = {len(p.read_ranges) for p in self.packs}
        return next(iter(values)) if len(values) == 1 else None

    @property
    def scalex_mode_b(self) -> bool:
        return bool(self.packs) and self.packs[0].scalex_record is not None

    @property
    def source_format(self) -> str:
        return "livglm_scalex_mode_b" if self.scalex_mode_b else "native_mxfp4"

    def slot_bytes(self, layer: int) -> int:
        """Bytes of one slot row as the reference sizes it (``expert_source.py:112-130``):
        weights plus the largest Mode-B row for ScaleX layers.  The HBM bank
        itself always holds decoded scales (``payload_bytes``)."""
        sources = self.layer_sources(layer)
        if self.scalex_mode_b:
            if any(s.scalex_record is None for s in sources):
                raise ContractError(f"layer {layer} mixes ScaleX and native experts")
            weights = sum(t.byte_length for t in sources[0].tensors
                          if t.destination_name.endswith(".weight"))
            return weights + max(s.scalex_record.mode_b_row_bytes for s in sources)
        sizes = {s.payload_bytes for s in sources}
        if len(sizes) != 1:
            raise ContractError(f"layer {layer} expert row sizes are not uniform")
        return next(iter(sizes))

    @property
    def slot_bytes_by_layer(self) -> tuple[int, ...]:
        return tuple(self.slot_bytes(layer) for layer in range(self.first_layer, self.last_layer + 1))

    def expert(self, layer: int, expert: int) -> NativeExpertSource:
        if not self.first_layer <= layer <= self.last_layer:
            raise ContractError(f"expert layer is out of range: {layer}")
        if not 0 <= expert < self.experts_per_layer:
            raise ContractError(f"expert id is out of range: {expert}")
        pack = self.packs[(layer - self.first_layer) * self.experts_per_layer + expert]
        if (pack.layer, pack.expert) != (layer, expert):
            raise ContractError("native expert source plan lost canonical ordering")
        return pack

    def layer_sources(self, layer: int) -> tuple[NativeExpertSource, ...]:
        return tuple(self.expert(layer, e) for e in range(self.experts_per_layer))

    def as_dict(self) -> dict[str, Any]:
        layers = []
        for layer in range(self.first_layer, self.last_layer + 1):
            sources = self.layer_sources(layer)
            layers.append({
                "layer": layer,
                "expert_count": self.experts_per_layer,
                "payload_bytes": sum(s.payload_bytes for s in sources),
                "source_shards": sorted({r.shard_name for s in sources for r in s.read_ranges}),
            })
        return {
            "source_kind": "livseek_glm_native_safetensors",
            "model_dir": self.model_dir,
            "first_layer": self.first_layer,
            "last_layer": self.last_layer,
            "layer_count": self.layer_count,
            "experts_per_layer": self.experts_per_layer,
            "expert_count": self.expert_count,
            "tensor_count": self.tensor_count,
            "payload_bytes": self.payload_bytes,
            "read_bytes": self.read_bytes,
            "source_shard_count": self.source_shard_count,
            "uniform_pack_bytes": self.uniform_pack_bytes,
            "uniform_read_count": self.uniform_read_count,
            "source_format": self.source_format,
            "scalex_mode_b": self.scalex_mode_b,
            "slot_bytes_by_layer": list(self.slot_bytes_by_layer),
            "layers": layers,
        }


def expected_shape(component: str, part: str, *, hidden_size: int,
                   intermediate_size: int) -> tuple[int, int]:
    """[rows, bytes per row] of a routed-expert tensor: gate/up have
    ``intermediate`` rows of ``hidden`` inputs, down the transpose; packed codes
    hold two inputs per byte, scales one byte per 32 (``expert_source.py:189-204``)."""
    rows, cols = ((hidden_size, intermediate_size) if component == "down_proj"
                  else (intermediate_size, hidden_size))
    divisor = 2 if part == "weight_packed" else 32
    if cols % divisor:
        raise ContractError(f"expert width is not divisible by {divisor}")
    return rows, cols // divisor


def _destination(source: TensorSource, component: str, part: str) -> ExpertTensorSource:
    """``expert_source.py:207-229``."""
    if source.dtype != "U8":
        raise ContractError(f"native MXFP4 tensor must use U8 storage: {source.name}")
    if part == "weight_packed":
        if source.shape[-1] % 4:
            raise ContractError(f"packed expert width is not U32-viewable: {source.name}")
        dtype, shape, dest = "U32", (*source.shape[:-1], source.shape[-1] // 4), f"{component}.weight"
    else:
        dtype, shape, dest = "U8", source.shape, f"{component}.scales"
    return ExpertTensorSource(source_name=source.name, destination_name=dest,
                              shard_name=source.shard_name, absolute_offset=source.absolute_offset,
                              byte_length=source.byte_length, source_shape=source.shape,
                              mlx_dtype=dtype, mlx_shape=shape)


def coalesce(tensors: tuple[ExpertTensorSource, ...]) -> tuple[ExpertReadRange, ...]:
    """Groups tensors that follow each other byte for byte in one shard into
    single read ranges, in (shard, offset) order (``expert_source.py:232-267``)."""
    ranges: list[ExpertReadRange] = []
    run: list[ExpertTensorSource] = []

    def flush() -> None:
        if run:
            start = run[0].absolute_offset
            end = run[-1].absolute_offset + run[-1].byte_length
            ranges.append(ExpertReadRange(run[0].shard_name, start, end - start, tuple(run)))

    for t in sorted(tensors, key=lambda t: (t.shard_name, t.absolute_offset)):
        if run and not (run[-1].shard_name == t.shard_name
                        and run[-1].absolute_offset + run[-1].byte_length == t.absolute_offset):
            flush()
            run = []
        run.append(t)
    flush()
    return tuple(ranges)


def build_native_expert_source_plan(contract: ModelContract, config: GLMTextConfig, *,
                                    first_layer: int = FIRST_MOE_LAYER,
                                    last_layer: int = LAST_MAIN_LAYER) -> NativeExpertSourcePlan:
    """Plans every routed expert of ``first_layer..last_layer``
    (``expert_source.py:270-381``): each tensor must exist, be U8 and have the
    shape the config implies; an expert's six tensors must share one shard."""
    if last_layer < first_layer:
        raise ContractError(f"empty layer range {first_layer}..{last_layer}")
    packs: list[NativeExpertSource] = []
    for layer in range(first_layer, last_layer + 1):
        for expert in range(config.n_routed_experts):
            tensors = []
            for component in EXPERT_COMPONENTS:
                for part in EXPERT_PARTS:
                    name = expert_tensor_name(layer, expert, component, part)
                    source = contract.tensor(name)
                    want = expected_shape(component, part, hidden_size=config.hidden_size,
                                          intermediate_size=config.moe_intermediate_size)
                    if source.shape != want:
                        raise ContractError(
                            f"native MXFP4 shape mismatch for {name}: {source.shape} != {want}")
                    tensors.append(_destination(source, component, part))
            tensor_tuple = tuple(tensors)
            shards = {t.shard_name for t in tensor_tuple}
            if len(shards) != 1:
                raise ContractError(f"expert {layer}/{expert} spans multiple shards")
            shard = shards.pop()
            layout = contract.scalex_layout(shard)
            record = None
            if layout is None:
                ranges = coalesce(tensor_tuple)
            else:
                if layout.layer != layer:
                    raise ContractError(f"ScaleX layer identity changed: {layout.layer} != {layer}")
                try:
                    record = layout.record(expert)
                except Exception as exc:  # ScaleXContainerError
                    raise ContractError(str(exc)) from exc
                by_name = {t.source_name: t for t in tensor_tuple}
                ranges = (ExpertReadRange(shard, record.absolute_offset, record.physical_bytes,
                                          tuple(by_name[n] for n in record.weight_names)),)
            packs.append(NativeExpertSource(layer=layer, expert=expert, tensors=tensor_tuple,
                                            read_ranges=ranges, scalex_record=record))
    plan = NativeExpertSourcePlan(model_dir=str(contract.model_dir), first_layer=first_layer,
                                  last_layer=last_layer,
                                  experts_per_layer=config.n_routed_experts, packs=tuple(packs))
    expected = (last_layer - first_layer + 1) * config.n_routed_experts
    if plan.expert_count != expected or plan.tensor_count != expected * 6:
        raise ContractError("native expert source inventory is incomplete")
    if len({p.scalex_record is not None for p in plan.packs}) != 1:
        raise ContractError("routed layers mix ScaleX and native MXFP4 shards")
    if (first_layer == FIRST_MOE_LAYER and last_layer == LAST_MAIN_LAYER
            and config.n_routed_experts == EXPERTS_PER_LAYER):
        if plan.uniform_pack_bytes != REAL_EXPERT_RECORD_BYTES:
            raise ContractError(f"native expert record size changed: {plan.uniform_pack_bytes}")
        if plan.uniform_read_count != 1:
            raise ContractError("native GLM experts are no longer exact one-range records")
        if plan.scalex_mode_b:
            if plan.read_bytes >= plan.payload_bytes:
                raise ContractError("ScaleX expert payload did not shrink")
        elif plan.read_bytes != plan.payload_bytes:
            raise ContractError("native GLM expert read bytes changed")
    return plan
